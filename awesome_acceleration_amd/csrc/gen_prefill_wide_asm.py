#!/usr/bin/env python3
"""Generate prefill_wide_asm.inc: the per-item body of the wide prefill kernel
(prefill_wide.hip) as one gfx950 inline-assembly template.

    python gen_prefill_wide_asm.py        # rewrites prefill_wide_asm.inc

Why assembly.  One wave per SIMD owns two 32-query columns and must keep the
matrix pipe fed from its own instruction stream.  A hand-ordered slot of
16 32x32x16 MFMAs + 2 row-sum MFMAs with the other column's 16 FMA, 16 exp,
8 cvt, the row max and 24 LDS reads measured 597 cycles against 545 for the
MFMAs alone on MI355X; the compiler's schedule of the same C++ took ~1100
(register copies, waits and a clustered score chain).  Inline assembly cannot
name single registers of a compiler-allocated tuple, so the values the
softmax touches element by element live in fixed registers that the
statement clobbers; Q, the addressing and the loop bounds are operands.

Register map (fixed, clobbered):
  v152-v167 S0, v168-v183 S1     scores of column 0 / 1 (32 keys x 32 queries)
  v184-v191 P0, v192-v199 P1     bf16 probabilities, two 16-key steps each
  v200-v203 L0, v204-v207 L1     row sums (16x16x32 selector MFMA layout)
  v208-v215 KA                   K read addresses (one per 16-dim step), tile t+1
  v216-v219 VA, v220-v223 VB     V read addresses (one per 32-dim block), tiles t, t+1
  v224-v227 ZERO                 zeros (MFMA operands for zero-init)
  v228 M0 v229 M1                reference max (raw score units)
  v230 MX0 v231 MX1              row max of the newest scores of each column
  v232 THR0 v233 THR1            M + kRescale / scale_log2
  v234 NB0 v235 NB1              -M * scale_log2
  v236-v239 T0-T3, v240 NEGINF, v242-v249 scratch (tuples start at even registers)
  a0-a127   O  (column c, dim block db at a[64c+16db : +15])
  a128-a159 K fragments (8 x 4), a160-a191 V fragments of even sub-tiles,
  a192-a223 V fragments of odd sub-tiles

Hazards (gfx950), each satisfied by construction below:
  * MFMA result -> VALU read: >= 19 wait states.  Scores are read two or more
    MFMAs after the chain's last MFMA; O and row sums only after three s_nop 7.
  * VALU write -> MFMA read: 2 wait states.  Probabilities are converted at
    least two instructions before the row-sum MFMA that reads them, and a
    slot earlier than the P*V MFMAs.
  * Transcendental -> VALU read: 1 wait state (exp results are converted
    three or more instructions later).
  * An LDS load into a fragment register is issued one MFMA after the last
    MFMA that reads the register.
  * s_mov m0 -> LDS-DMA load: s_nop 0; VALU write -> v_permlane32_swap: s_nop 1.
"""
from __future__ import annotations

import sys
from pathlib import Path

OPITCH_BYTES = 136 * 2  # output staging row pitch (bytes), as prefill_common.h OPITCH


def v(n):
    return f"v{n}"


def vr(b, n):
    return f"v[{b}:{b + n - 1}]"


def ar(b, n):
    return f"a[{b}:{b + n - 1}]"


S = [152, 168]
P = [184, 192]
L = [200, 204]
KA, VA, VB, ZERO = 208, 216, 220, 224
M, MX, THR, NB = [228, 229], [230, 231], [232, 233], [234, 235]
T0, T1, T2, T3, NEGINF, SCR = 236, 237, 238, 239, 240, 242
O_A, KF_A, VF_A = 0, 128, 160


def S_t(c):
    return vr(S[c], 16)


def S_e(c, i):
    return v(S[c] + i)


def P_t(c, tt):
    return vr(P[c] + 4 * tt, 4)


def P_e(c, w):
    return v(P[c] + w)


def L_t(c):
    return vr(L[c], 4)


def O_t(c, db):
    return ar(O_A + 64 * c + 16 * db, 16)


def KF(t):
    return ar(KF_A + 4 * t, 4)


def VF(par, f):  # V fragment f = 2*db + tt of a sub-tile of parity par
    return ar(VF_A + 32 * par + 4 * f, 4)


def VF_half(par, f, h):
    return ar(VF_A + 32 * par + 4 * f + 2 * h, 2)


MFMA = "v_mfma_f32_32x32x16_bf16"
SELM = "v_mfma_f32_16x16x32_bf16"


class Emitter:
    def __init__(self):
        self.lines: list[str] = []
        self.n_label = 0

    def __call__(self, s: str):
        self.lines.append(s)

    def label(self, base: str) -> str:
        self.n_label += 1
        return f"{base}_{self.n_label}_%="

    def text(self) -> str:
        return "\n".join(self.lines)


def row_max_tail(e, c):
    """MX[c] = max over both lane halves of T0 (the lane-partial max)."""
    e(f"v_mov_b32 {v(T1)}, {v(T0)}")
    e("s_nop 1")
    e(f"v_permlane32_swap_b32 {v(T0)}, {v(T1)}")
    e(f"v_maximum3_f32 {v(MX[c])}, {v(T0)}, {v(T1)}, {v(T1)}")


def row_max_ops(c):
    """The lane-partial max of S[c] as 8 instructions (T0)."""
    ops = [f"v_maximum3_f32 {v(T0)}, {S_e(c, 0)}, {S_e(c, 1)}, {S_e(c, 2)}"]
    for i in range(3, 15, 2):
        ops.append(f"v_maximum3_f32 {v(T0)}, {v(T0)}, {S_e(c, i)}, {S_e(c, i + 1)}")
    ops.append(f"v_maximum3_f32 {v(T0)}, {v(T0)}, {S_e(c, 15)}, {S_e(c, 15)}")
    return ops


def softmax_ops(x):
    """Per-step VALU of the softmax of S[x] in place -> P[x]: entries 0-15 go
    beside MFMA steps 0-15, entry 16 (the last exp) and entry 17 (the last
    convert) after them, with at least one instruction between the two."""
    steps = [[] for _ in range(18)]
    for i in range(16):
        steps[i].append(f"v_fma_f32 {S_e(x, i)}, {S_e(x, i)}, %[cs], {v(NB[x])}")
    for i in range(16):
        steps[i + 1].append(f"v_exp_f32 {S_e(x, i)}, {S_e(x, i)}")
    for w in range(8):
        at = 2 * w + 3 if w < 7 else 17
        steps[at].append(f"v_cvt_pk_bf16_f32 {P_e(x, w)}, {S_e(x, 2 * w)}, {S_e(x, 2 * w + 1)}")
    return steps


def selector(x, tt):
    return f"{SELM} {L_t(x)}, %[sel], {P_t(x, tt)}, {L_t(x)}"


def check(e, x):
    """Rescale column x when some row max exceeds its threshold (rare)."""
    ok = e.label("Lok")
    e(f"v_cmp_gt_f32 vcc, {v(MX[x])}, {v(THR[x])}")
    e(f"s_cbranch_vccz {ok}")
    e(f"s_call_b64 %[ret], Lresc{x}_%=")
    e(f"{ok}:")


def mask(e, x, jj_expr_sgpr):
    """Scores of S[x] for keys at or past this lane's limit -> -inf; then the
    row max MX[x] again.  jj_expr_sgpr holds 32 * (sub-tile index)."""
    e(f"v_subrev_u32 {v(T2)}, {jj_expr_sgpr}, %[mylim]")
    e(f"v_sub_u32 {v(T2)}, {v(T2)}, %[hl4]")
    for i in range(16):
        ci = 8 * (i >> 2) + (i & 3)
        e(f"v_cmp_lt_i32 vcc, {ci}, {v(T2)}")
        e(f"v_cndmask_b32 {S_e(x, i)}, {v(NEGINF)}, {S_e(x, i)}, vcc")
    for op in row_max_ops(x):
        e(op)
    row_max_tail(e, x)


def slot(e, c, par, kind):
    """One slot.  c: MFMA column; x = 1 - c: softmax column.
    kind 'A': no LDS reads; 'B': reload K(j+2) and V(j+1) (par = parity of j).
    MFMA steps 0-7: S[c] = K Q_c^T; 8-15: O[c] += V^T P[c]."""
    x = 1 - c
    sm = softmax_ops(x)
    mx = row_max_ops(c)
    reads = [[] for _ in range(17)]
    if kind == "B":
        # K(j+2): tile t+1, half par; register t free once MFMA t issued
        for t in range(8):
            reads[t + 1].append(f"ds_read_b128 {KF(t)}, {v(KA + t)} offset:{8192 * par}")
        # V(j+1) into the other parity's registers: par 0 -> tile t half 1 (VA),
        # par 1 -> tile t+1 half 0 (VB)
        base, off0 = (VA, 8192) if par == 0 else (VB, 0)
        vr_list = []
        for db in range(4):
            for tt in range(2):
                f = 2 * db + tt
                for h in range(2):
                    vr_list.append(f"ds_read_b64_tr_b16 {VF_half(1 - par, f, h)}, {v(base + db)} "
                                   f"offset:{off0 + 4096 * tt + 2048 * h}")
        # 16 V reads over steps 2-15 (two at steps 2 and 3)
        at = [2, 2, 3, 3] + list(range(4, 16))
        for r, s in zip(vr_list, at):
            reads[s].append(r)
    for i in range(16):
        if kind == "A" and i == 0:
            e("s_waitcnt lgkmcnt(9)")   # K fragments of this slot landed
        if kind == "A" and i == 8:
            e("s_waitcnt lgkmcnt(0)")   # V fragments landed
        if i < 8:
            e(f"{MFMA} {S_t(c)}, {KF(i)}, %[q{c}{i}], {'0' if i == 0 else S_t(c)}")
        else:
            tt, db = (i - 8) // 4, (i - 8) % 4
            e(f"{MFMA} {O_t(c, db)}, {VF(par, 2 * db + tt)}, {P_t(c, tt)}, {O_t(c, db)}")
        for op in sm[i]:
            e(op)
        for op in reads[i]:
            e(op)
        if i >= 9:
            e(mx[i - 9])
        if i == 11:
            e(selector(x, 0))
    for op in sm[16]:
        e(op)
    e(mx[7])
    for op in sm[17]:
        e(op)
    row_max_tail(e, c)
    e(selector(x, 1))


def last(e, par):
    """Last sub-tile of the wave: softmax of S1 -> P1, then O0 += V P0 and O1 += V P1."""
    sm = softmax_ops(1)
    e("s_waitcnt lgkmcnt(0)")
    for i in range(8):
        tt, db = i // 4, i % 4
        e(f"{MFMA} {O_t(0, db)}, {VF(par, 2 * db + tt)}, {P_t(0, tt)}, {O_t(0, db)}")
        for op in sm[i]:
            e(op)
    for i in range(8, 17):
        for op in sm[i]:
            e(op)
    e("s_nop 0")
    for op in sm[17]:
        e(op)
    e("s_nop 1")
    e(selector(1, 0))
    e(selector(1, 1))
    for i in range(8):
        tt, db = i // 4, i % 4
        e(f"{MFMA} {O_t(1, db)}, {VF(par, 2 * db + tt)}, {P_t(1, tt)}, {O_t(1, db)}")


def rescale_sub(e, x):
    """Subroutine: new reference max for column x, O[x] and L[x] scaled by
    alpha = exp2((M - max(M, MX)) * scale_log2)."""
    e(f"Lresc{x}_%=:")
    e("s_nop 7")
    e("s_nop 7")
    e("s_nop 7")
    e(f"v_max_f32 {v(T0)}, {v(M[x])}, {v(MX[x])}")
    e(f"v_sub_f32 {v(T1)}, {v(M[x])}, {v(T0)}")
    e(f"v_mul_f32 {v(T1)}, %[cs], {v(T1)}")
    e(f"v_exp_f32 {v(T1)}, {v(T1)}")
    e(f"v_mov_b32 {v(M[x])}, {v(T0)}")
    e(f"v_add_f32 {v(THR[x])}, %[kthr], {v(T0)}")
    e(f"v_mul_f32 {v(NB[x])}, %[ncs], {v(T0)}")
    e("s_nop 1")
    base = O_A + 64 * x
    for g in range(0, 64, 8):
        for i in range(8):
            e(f"v_accvgpr_read_b32 {v(SCR + i)}, a{base + g + i}")
        for i in range(8):
            e(f"v_mul_f32 {v(SCR + i)}, {v(SCR + i)}, {v(T1)}")
        for i in range(8):
            e(f"v_accvgpr_write_b32 a{base + g + i}, {v(SCR + i)}")
    # L[x][0] of lane n < 16 is query n; L[x][1] is query 16 + n, whose alpha
    # sits in lane (n & 15) + 16
    e(f"ds_bpermute_b32 {v(T2)}, %[bpahi], {v(T1)}")
    e("s_waitcnt lgkmcnt(0)")
    e(f"v_mul_f32 {v(L[x])}, {v(L[x])}, {v(T1)}")
    e(f"v_mul_f32 {v(L[x] + 1)}, {v(L[x] + 1)}, {v(T2)}")
    e("s_nop 2")
    e("s_setpc_b64 %[ret]")


def set_ref(e, x):
    e(f"v_max_f32 {v(M[x])}, 0xf149f2ca, {v(MX[x])}")  # max(mx, -1e30)
    e(f"v_add_f32 {v(THR[x])}, %[kthr], {v(M[x])}")
    e(f"v_mul_f32 {v(NB[x])}, %[ncs], {v(M[x])}")


def softmax_block(e, x):
    """The softmax of S[x] with no MFMA beside it (prologue)."""
    sm = softmax_ops(x)
    for i in range(17):
        for op in sm[i]:
            e(op)
    e("s_nop 0")
    for op in sm[17]:
        e(op)
    e("s_nop 1")
    e(selector(x, 0))
    e(selector(x, 1))


def generate() -> str:
    e = Emitter()
    # ---------------------------------------------------------------- entry
    e("s_waitcnt lgkmcnt(0)")
    for i in range(4):
        e(f"v_mov_b32 {v(ZERO + i)}, 0")
    for i in range(8):
        e(f"v_mov_b32 {v(L[0] + i)}, 0")
    e(f"v_mov_b32 {v(NEGINF)}, 0xff800000")
    e("s_nop 1")
    for c in range(2):
        for db in range(4):
            e(f"{MFMA} {O_t(c, db)}, {vr(ZERO, 4)}, {vr(ZERO, 4)}, 0")
    # ------------------------------------------------------------- prologue
    e("s_cmp_eq_u32 %[nsub], 0")
    e("s_cbranch_scc1 Lpro_end_%=")
    for t in range(8):
        e(f"v_add_u32 {v(KA + t)}, %[lds0], %[ko{t}]")
    for t in range(8):
        e(f"ds_read_b128 {KF(t)}, {v(KA + t)}")
    e("s_waitcnt lgkmcnt(0)")
    for t in range(8):
        e(f"{MFMA} {S_t(0)}, {KF(t)}, %[q0{t}], {'0' if t == 0 else S_t(0)}")
        e(f"{MFMA} {S_t(1)}, {KF(t)}, %[q1{t}], {'0' if t == 0 else S_t(1)}")
        if t >= 1:
            e(f"ds_read_b128 {KF(t - 1)}, {v(KA + t - 1)} offset:8192")
    e(f"ds_read_b128 {KF(7)}, {v(KA + 7)} offset:8192")
    e("s_add_u32 %[s2], %[lds0], 0x4000")
    for db in range(4):
        e(f"v_add_u32 {v(VA + db)}, %[s2], %[vo{db}]")
    for db in range(4):
        for tt in range(2):
            for h in range(2):
                e(f"ds_read_b64_tr_b16 {VF_half(0, 2 * db + tt, h)}, {v(VA + db)} offset:{4096 * tt + 2048 * h}")
    e("s_nop 7")
    e("s_nop 7")
    e("s_nop 7")
    e("s_cmp_lt_u32 %[wfull], 32")
    e("s_cbranch_scc0 Lpro_nomask_%=")
    e("s_mov_b32 %[s6], 0")
    mask(e, 0, "%[s6]")
    mask(e, 1, "%[s6]")
    e("s_branch Lpro_ref_%=")
    e("Lpro_nomask_%=:")
    for c in range(2):
        for op in row_max_ops(c):
            e(op)
        row_max_tail(e, c)
    e("Lpro_ref_%=:")
    set_ref(e, 0)
    set_ref(e, 1)
    softmax_block(e, 0)
    e("Lpro_end_%=:")
    # ------------------------------------------------------------ tile loop
    e("s_mov_b32 %[t], 0")
    e("Ltile_%=:")
    e("s_cmp_ge_u32 %[t], %[nt]")
    e("s_cbranch_scc1 Ltdone_%=")
    e("s_and_b32 %[s0], %[t], 3")
    e("s_lshl_b32 %[s0], %[s0], 15")
    e("s_add_u32 %[s0], %[s0], %[lds0]")          # stage base of tile t
    e("s_add_u32 %[s1], %[t], 1")
    e("s_and_b32 %[s1], %[s1], 3")
    e("s_lshl_b32 %[s1], %[s1], 15")
    e("s_add_u32 %[s1], %[s1], %[lds0]")          # stage base of tile t+1
    for t in range(8):
        e(f"v_add_u32 {v(KA + t)}, %[s1], %[ko{t}]")
    e("s_add_u32 %[s2], %[s0], 0x4000")
    for db in range(4):
        e(f"v_add_u32 {v(VA + db)}, %[s2], %[vo{db}]")
    e("s_add_u32 %[s2], %[s1], 0x4000")
    for db in range(4):
        e(f"v_add_u32 {v(VB + db)}, %[s2], %[vo{db}]")
    for sub in range(2):
        # j = 2t + sub;  s5 = j + 1
        e("s_lshl_b32 %[j], %[t], 1")
        if sub:
            e("s_add_u32 %[j], %[j], 1")
        e("s_add_u32 %[s5], %[j], 1")
        e("s_lshl_b32 %[s6], %[j], 5")              # 32 j
        e("s_cmp_lt_u32 %[s5], %[nsub]")
        e(f"s_cbranch_scc0 Lnofull{sub}_%=")
        # ---- full sub-tile: slot A(j)
        e("s_add_u32 %[s3], %[s6], 32")
        e("s_cmp_gt_u32 %[s3], %[wfull]")
        e(f"s_cbranch_scc0 LmA{sub}_%=")
        mask(e, 1, "%[s6]")
        e(f"LmA{sub}_%=:")
        check(e, 1)
        slot(e, 0, sub, "A")
        if sub == 0:
            e(f"s_branch Lsync_%=")
        else:
            e(f"s_branch LB{sub}_%=")
        # ---- last sub-tile of the wave
        e(f"Lnofull{sub}_%=:")
        e("s_cmp_eq_u32 %[s5], %[nsub]")
        e(f"s_cbranch_scc0 Lskip{sub}_%=")
        e("s_add_u32 %[s3], %[s6], 32")
        e("s_cmp_gt_u32 %[s3], %[wfull]")
        e(f"s_cbranch_scc0 LmL{sub}_%=")
        mask(e, 1, "%[s6]")
        e(f"LmL{sub}_%=:")
        check(e, 1)
        last(e, sub)
        e(f"Lskip{sub}_%=:")
        if sub == 0:
            # ---- sync point of the tile: tile t+1 landed everywhere; the
            # stage of tile t-1 is free for tile t+3
            e("Lsync_%=:")
            e("s_waitcnt vmcnt(8)")
            e("s_barrier")
            e("s_add_u32 %[s2], %[t], 3")
            e("s_and_b32 %[s3], %[s2], 3")
            e("s_lshl_b32 %[s3], %[s3], 15")
            e("s_add_u32 %[s3], %[s3], %[ldsw]")
            e("s_mul_i32 %[s4], %[s2], %[ks64]")
            e("s_mul_i32 %[s2], %[s2], %[vs64]")
            for i in range(4):
                e("s_mov_b32 m0, %[s3]")
                e("s_nop 0")
                e("buffer_load_dwordx4 %[ldk], %[rsk], %[s4] offen lds")
                e("s_add_u32 %[s4], %[s4], %[ks16]")
                e("s_add_u32 %[s3], %[s3], 0x1000")
            for i in range(4):
                e("s_mov_b32 m0, %[s3]")
                e("s_nop 0")
                e("buffer_load_dwordx4 %[ldv], %[rsv], %[s2] offen lds")
                e("s_add_u32 %[s2], %[s2], %[vs16]")
                e("s_add_u32 %[s3], %[s3], 0x1000")
            # slot B(2t) when 2t is a full sub-tile
            e("s_lshl_b32 %[j], %[t], 1")
            e("s_add_u32 %[s5], %[j], 1")
            e("s_cmp_lt_u32 %[s5], %[nsub]")
            e(f"s_cbranch_scc0 LBend{sub}_%=")
        else:
            e(f"s_branch LBend{sub}_%=")
        e(f"LB{sub}_%=:")
        # ---- slot B(j): mask S0 (sub-tile j+1) when needed
        e("s_lshl_b32 %[s6], %[j], 5")
        e("s_add_u32 %[s3], %[s6], 64")
        e("s_cmp_gt_u32 %[s3], %[wfull]")
        e(f"s_cbranch_scc0 LmB{sub}_%=")
        e("s_add_u32 %[s3], %[s6], 32")
        mask(e, 0, "%[s3]")
        e(f"LmB{sub}_%=:")
        check(e, 0)
        slot(e, 1, sub, "B")
        e(f"LBend{sub}_%=:")
    e("s_add_u32 %[t], %[t], 1")
    e("s_branch Ltile_%=")
    e("Ltdone_%=:")
    # ------------------------------------------------------------- epilogue
    # every wave is done with the ring and no tile load is still writing it
    e("s_waitcnt vmcnt(0) lgkmcnt(0)")
    e("s_barrier")
    e("s_nop 7")
    e("s_nop 7")
    e("s_nop 7")
    for x in range(2):
        e(f"ds_bpermute_b32 {v(T0)}, %[bpa], {v(L[x])}")
        e(f"ds_bpermute_b32 {v(T1)}, %[bpa], {v(L[x] + 1)}")
        e("s_waitcnt lgkmcnt(0)")
        e(f"v_cmp_ne_u32 vcc, 0, %[hi16]")
        e(f"v_cndmask_b32 {v(T0)}, {v(T0)}, {v(T1)}, vcc")        # row sum of this lane's query
        e(f"v_rcp_f32 {v(T1)}, {v(T0)}")
        e(f"v_cmp_lt_f32 vcc, 0, {v(T0)}")
        e(f"v_cndmask_b32 {v(T1)}, 0, {v(T1)}, vcc")              # 1/l, 0 for an empty row
        e("s_nop 1")
        base = O_A + 64 * x
        for db in range(4):
            for r in range(4):
                a0 = base + 16 * db + 4 * r
                for i in range(4):
                    e(f"v_accvgpr_read_b32 {v(SCR + i)}, a{a0 + i}")
                for i in range(4):
                    e(f"v_mul_f32 {v(SCR + i)}, {v(SCR + i)}, {v(T1)}")
                e(f"v_cvt_pk_bf16_f32 {v(SCR + 4)}, {v(SCR)}, {v(SCR + 1)}")
                e(f"v_cvt_pk_bf16_f32 {v(SCR + 5)}, {v(SCR + 2)}, {v(SCR + 3)}")
                off = x * 32 * OPITCH_BYTES + (32 * db + 8 * r) * 2
                e(f"ds_write_b64 %[obase], {vr(SCR + 4, 2)} offset:{off}")
    e("s_waitcnt lgkmcnt(0)")
    e("s_branch Lend_%=")
    # ---------------------------------------------------------- subroutines
    rescale_sub(e, 0)
    rescale_sub(e, 1)
    e("Lend_%=:")
    return e.text()


HEADER = """// Generated by gen_prefill_wide_asm.py -- do not edit by hand.
// The per-item body of prefill_wide_kernel (zero-init, scores of sub-tile 0,
// the tile loop with its slots, masks, rescales and LDS staging, and the
// normalised output written to the LDS staging area) as one gfx950
// inline-assembly template; register map and hazard rules in the generator.
#pragma once
"""


def main() -> int:
    body = generate()
    lit = "\n".join('  "' + ln.replace('"', '\\"') + '\\n"' for ln in body.split("\n"))
    n = sum(1 for ln in body.split("\n") if ln and not ln.endswith(":"))
    out = HEADER + f"// {n} instructions.\n#define AAC_PW_ITEM_ASM \\\n" + " \\\n".join(
        lit.split("\n")) + "\n"
    path = Path(__file__).resolve().parent / "prefill_wide_asm.inc"
    if len(sys.argv) > 1 and sys.argv[1] == "--check":
        return 0 if path.read_text() == out else 1
    path.write_text(out)
    print(f"wrote {path} ({n} instructions)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
