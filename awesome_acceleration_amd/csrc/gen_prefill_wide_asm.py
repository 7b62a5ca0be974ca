#!/usr/bin/env python3
"""Generate prefill_wide_asm.inc: the per-item body of the wide prefill kernel
(prefill_wide.hip) as one gfx950 inline-assembly template.

    python gen_prefill_wide_asm.py           # rewrites prefill_wide_asm.inc
    python gen_prefill_wide_asm.py --check   # exit 1 if the file is stale

Why assembly.  One wave per SIMD owns two 32-query columns and must keep the
matrix pipe fed from its own instruction stream.  A hand-ordered slot of
16 32x32x16 MFMAs + 2 row-sum MFMAs with the other column's 16 FMA, 16 exp,
8 cvt, the row max and 24 LDS reads measured 597 cycles against 545 for the
MFMAs alone on MI355X; the compiler's schedule of the same C++ took ~1100
(register copies, waits and a clustered score chain).  Inline assembly cannot
name single registers of a compiler-allocated tuple, so the values the
softmax touches element by element live in fixed registers that the
statement clobbers; Q, the addressing and the loop bounds are operands.

Schedule.  Sub-tile j (32 keys) runs two slots; slot A(j) issues the MFMAs
of column 0 and the softmax of column 1, slot B(j) the reverse:
  A(j): S_0(j+1) = K(j+1) Q_0^T, O_0 += V(j)^T P_0(j) | softmax S_1(j) -> P_1(j)
        LDS: K(j+2) into K set j%2 (8 x 1 KiB)
  B(j): S_1(j+1) = K(j+1) Q_1^T, O_1 += V(j)^T P_1(j) | softmax S_0(j+1) -> P_0(j+1)
        LDS: V(j+1) into V set (j+1)%2 (16 x 512 B)
so each slot reads 8 KiB from LDS, and with K and V double-buffered no read
waits on the other column.  Each slot ends with the row max of the scores
its MFMAs produced and the compare against the rescale threshold; the next
slot branches on it (not taken unless a row max grew by more than kRescale)
after its first MFMA, so the compare's latency is hidden.  Tile t (64 keys)
is iteration t of the loop: a barrier at its start (tile t+1 has landed for
every wave; no wave still reads tile t-1) and then, when both sub-tiles are
full and need no causal mask, four slots in straight-line code with the
eight loads of tile t+3 into the freed stage spread two per slot; otherwise
a general path with the masks, the wave's last sub-tile and the loads issued
together.

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
  a128-a159 K set 0, a224-a255 K set 1 (8 x 4 each: one fragment per 16-dim step)
  a160-a191 V set 0, a192-a223 V set 1 (8 fragments f = 2 db + tt of 4)

Hazards (gfx950), each satisfied by construction below:
  * MFMA result -> VALU read: >= 19 wait states.  Scores are read two or more
    MFMAs after the chain's last MFMA; O and row sums only after three s_nop 7.
  * VALU write -> MFMA read: 2 wait states.  Probabilities are converted at
    least two instructions before the row-sum MFMA that reads them, and a
    slot earlier than the P*V MFMAs.
  * Transcendental -> VALU read: 1 wait state (exp results are converted
    three or more instructions later).
  * An LDS load into a fragment register is issued a slot or more after the
    last MFMA that reads the register; every MFMA that reads a fragment is
    preceded by an s_waitcnt lgkmcnt that the read tracker below computes.
  * s_mov m0 -> LDS-DMA load: s_nop 0; VALU write -> v_permlane32_swap: s_nop 1.
  * VCC holds the compare for the next slot's branch from the end of a slot:
    nothing between writes VCC except a mask, which compares again.
"""
from __future__ import annotations

import sys
from pathlib import Path



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
O_A, VF_A = 0, 160
# Buffer resources built in fixed SGPRs (the statement clobbers them): the
# active K / V sources of the tile loads (this item's, then the next item's
# from the position where its tiles start), the next item's, and at the end
# the output rows of this wave.
RK, RV, RKN, RVN = "s[88:91]", "s[92:95]", "s[80:83]", "s[84:87]"
SGPR_CLOBBER = range(80, 96)
KF_SET = [128, 224]
N_OUT_STORES = 16   # output stores the body issues after the next item's Q loads
N_OWN_STORES = 16   # and KV-cache stores (when it stores)
VGPR_CLOBBER = range(152, 250)
AGPR_CLOBBER = range(0, 256)


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


def KF(kset, t):  # K fragment of 16-dim step t in set kset
    return ar(KF_SET[kset] + 4 * t, 4)


def VF(vset, f):  # V fragment f = 2*db + tt in set vset
    return ar(VF_A + 32 * vset + 4 * f, 4)


def VF_half(vset, f, h):
    return ar(VF_A + 32 * vset + 4 * f + 2 * h, 2)


# Schedule options (kept switchable so the slot can be timed in isolation):
# LAYOUT places the softmax ops over the MFMA steps ("base": op i of each
# kind at step i / i+1, the last exp and convert after step 15; "early2": two
# elements at step 0 and one ahead after, all done by step 15).  PARTIAL
# compares the lane-partial row max with the threshold (any lane over it
# rescales; only the rescale needs the cross-half max).
LAYOUT = "early2"
PARTIAL = True

MFMA = "v_mfma_f32_32x32x16_bf16"
SELM = "v_mfma_f32_16x16x32_bf16"


class Emitter:
    def __init__(self):
        self.lines: list[str] = []
        self.n_label = 0
        self.stubs: list[str] = []  # out-of-line code, emitted after the body

    def __call__(self, s: str):
        self.lines.append(s)

    def label(self, base: str) -> str:
        self.n_label += 1
        return f"{base}_{self.n_label}_%="

    def text(self) -> str:
        return "\n".join(self.lines)


class Lgkm:
    """In-order LDS read tracker: `pending` lists the tags of the reads in
    flight, oldest first; need(tag) emits the s_waitcnt that guarantees every
    read carrying that tag has returned (lgkmcnt counts at most 15)."""

    def __init__(self, pending):
        self.pending = list(pending)

    def issue(self, tag):
        self.pending.append(tag)

    def need(self, e, tag):
        idx = max((i for i, t in enumerate(self.pending) if t == tag), default=-1)
        if idx < 0:
            return
        after = len(self.pending) - idx - 1
        n = min(after, 15)
        e(f"s_waitcnt lgkmcnt({n})")
        self.pending = self.pending[len(self.pending) - n:]


# LDS reads of the two slot kinds, in issue order, with the MFMA step each
# goes after.  A(j): K(j+2), one per even step.  B(j): V(j+1), one half per
# step, in the order the P*V MFMAs of the next A consume them
# (step 8 + 4 tt + db uses fragment 2 db + tt).
K_READ_STEPS = [2 * t for t in range(8)]
V_READ_STEPS = list(range(16))
V_ORDER = [(2 * db + tt, h) for tt in range(2) for db in range(4) for h in range(2)]


def pv_frag(i):
    """Fragment (2 db + tt) and accumulator block db of P*V MFMA step i (8-15)."""
    tt, db = (i - 8) // 4, (i - 8) % 4
    return 2 * db + tt, db, tt


def b_reads_pending():
    """Pending tags at the start of an A slot: slot B's 16 V halves."""
    return [("V", f) for f, _ in V_ORDER]


def row_max_tail(e, c):
    """MX[c] = max over both lane halves of T0 (the lane-partial max)."""
    e(f"v_mov_b32 {v(T1)}, {v(T0)}")
    e("s_nop 1")
    e(f"v_permlane32_swap_b32 {v(T0)}, {v(T1)}")
    e(f"v_maximum3_f32 {v(MX[c])}, {v(T0)}, {v(T1)}, {v(T1)}")


def compare(e, c):
    """VCC = lanes whose row max passed the rescale threshold of column c."""
    e(f"v_cmp_gt_f32 vcc, {v(MX[c])}, {v(THR[c])}")


def compare_partial(e, c):
    """VCC = lanes whose partial row max (T0) passed the threshold of column c."""
    e(f"v_cmp_gt_f32 vcc, {v(T0)}, {v(THR[c])}")


def row_max_ops(c):
    """The lane-partial max of S[c] as 8 instructions (T0)."""
    ops = [f"v_maximum3_f32 {v(T0)}, {S_e(c, 0)}, {S_e(c, 1)}, {S_e(c, 2)}"]
    for i in range(3, 15, 2):
        ops.append(f"v_maximum3_f32 {v(T0)}, {v(T0)}, {S_e(c, i)}, {S_e(c, i + 1)}")
    ops.append(f"v_maximum3_f32 {v(T0)}, {v(T0)}, {S_e(c, 15)}, {S_e(c, 15)}")
    return ops


def softmax_ops(x):
    """Per-step VALU of the softmax of S[x] in place -> P[x]: entries 0-15 go
    beside MFMA steps 0-15, entries 16 and 17 after them.  A convert reads
    exp results of an earlier entry (one instruction at least between a
    transcendental and its reader)."""
    steps = [[] for _ in range(18)]
    fma = lambda i: f"v_fma_f32 {S_e(x, i)}, {S_e(x, i)}, %[cs], {v(NB[x])}"
    ex = lambda i: f"v_exp_f32 {S_e(x, i)}, {S_e(x, i)}"
    cvt = lambda w: f"v_cvt_pk_bf16_f32 {P_e(x, w)}, {S_e(x, 2 * w)}, {S_e(x, 2 * w + 1)}"
    if LAYOUT == "base":
        for i in range(16):
            steps[i].append(fma(i))
        for i in range(16):
            steps[i + 1].append(ex(i))
        for w in range(8):
            steps[2 * w + 3 if w < 7 else 17].append(cvt(w))
    elif LAYOUT == "early2":
        steps[0] += [fma(0), fma(1), ex(0), ex(1)]
        for st in range(1, 15):
            steps[st].append(fma(st + 1))
            if st % 2 == 1:
                steps[st].append(cvt((st - 1) // 2))
            steps[st].append(ex(st + 1))
        steps[15].append(cvt(7))
    else:
        raise ValueError(LAYOUT)
    return steps


def sel0_step():
    """Step after whose MFMA the first row-sum MFMA goes (two instructions or
    more after the convert of the last word of P[x](0))."""
    return 11 if LAYOUT == "base" else 9


def selector(x, tt):
    return f"{SELM} {L_t(x)}, %[sel], {P_t(x, tt)}, {L_t(x)}"


def check_branch(e, x):
    """Rescale column x when the compare left in VCC found a row max past its
    threshold (rare): a not-taken branch to an out-of-line call."""
    stub = e.label("Lfix")
    back = e.label("Lback")
    e(f"s_cbranch_vccnz {stub}")
    e(f"{back}:")
    e.stubs += [f"{stub}:", f"s_call_b64 %[ret], Lresc{x}_%=", f"s_branch {back}"]


def mask(e, x, jj_expr_sgpr, full=False):
    """Scores of S[x] for keys at or past this lane's limit -> -inf; then the
    row max and its compare again (with PARTIAL the lane-partial max in T0,
    the full max MX[x] only when `full`: the prologue's reference max needs
    it).  jj_expr_sgpr holds 32 * (sub-tile index)."""
    e(f"v_subrev_u32 {v(T2)}, {jj_expr_sgpr}, %[mylim]")
    e(f"v_sub_u32 {v(T2)}, {v(T2)}, %[hl4]")
    for i in range(16):
        ci = 8 * (i >> 2) + (i & 3)
        e(f"v_cmp_lt_i32 vcc, {ci}, {v(T2)}")
        e(f"v_cndmask_b32 {S_e(x, i)}, {v(NEGINF)}, {S_e(x, i)}, vcc")
    for op in row_max_ops(x):
        e(op)
    if PARTIAL and not full:
        compare_partial(e, x)
    else:
        row_max_tail(e, x)
        compare(e, x)


def k_read(kset, t, par):
    """K fragment t of sub-tile j+2 into set kset; tile t+1, half par."""
    return f"ds_read_b128 {KF(kset, t)}, {v(KA + t)} offset:{8192 * par}"


def v_read(vset, f, h, par):
    """Half h of V fragment f of sub-tile j+1 into set vset: for par 0 tile t
    half 1 (VA), for par 1 tile t+1 half 0 (VB)."""
    base, off0 = (VA, 8192) if par == 0 else (VB, 0)
    db, tt = f // 2, f % 2
    return f"ds_read_b64_tr_b16 {VF_half(vset, f, h)}, {v(base + db)} offset:{off0 + 4096 * tt + 2048 * h}"


def slot(e, c, par, extra=None):
    """One slot of sub-tile j (par = j % 2).  c = 0: slot A (MFMA column 0,
    softmax column 1, reads K(j+2)); c = 1: slot B (MFMA column 1, softmax
    column 0, reads V(j+1)).  extra: step -> instructions to place after that
    step's MFMA (the spread tile loads)."""
    x = 1 - c
    kuse, kset_new = 1 - par, par          # K(j+1) in set (j+1)%2; K(j+2) into set j%2
    vuse, vset_new = par, 1 - par          # V(j) in set j%2; V(j+1) into set (j+1)%2
    sm = softmax_ops(x)
    mx = row_max_ops(c)
    reads = [[] for _ in range(16)]
    lg = None
    if c == 0:
        lg = Lgkm(b_reads_pending())
        for t, st in enumerate(K_READ_STEPS):
            reads[st].append((("K", t), k_read(kset_new, t, par)))
    else:
        for st, (f, h) in zip(V_READ_STEPS, V_ORDER):
            reads[st].append((("V", f), v_read(vset_new, f, h, par)))
    for i in range(16):
        if i < 8:
            if lg is not None and i == 0:
                # K(j+1) was read in the previous A: pending as the oldest reads
                lg.pending = [("Kold", 0)] * 8 + lg.pending
                lg.need(e, ("Kold", 0))
            e(f"{MFMA} {S_t(c)}, {KF(kuse, i)}, %[q{c}{i}], {'0' if i == 0 else S_t(c)}")
        else:
            f, db, tt = pv_frag(i)
            if lg is not None:
                lg.need(e, ("V", f))
            e(f"{MFMA} {O_t(c, db)}, {VF(vuse, f)}, {P_t(c, tt)}, {O_t(c, db)}")
        if i == 0:
            check_branch(e, x)
        for op in sm[i]:
            e(op)
        for tag, op in reads[i]:
            e(op)
            if lg is not None:
                lg.issue(tag)
        if extra and i in extra:
            for op in extra[i]:
                e(op)
        if i >= 9:
            e(mx[i - 9])
        if i == sel0_step():
            e(selector(x, 0))
    for op in sm[16]:
        e(op)
    e(mx[7])
    for op in sm[17]:
        e(op)
    if PARTIAL:
        compare_partial(e, c)
        e("s_nop 0")
        e(selector(x, 1))
    else:
        row_max_tail(e, c)
        e(selector(x, 1))
        compare(e, c)


def q_load(c, t):
    """One fragment of the next item's Q (column c, 16-dim step t)."""
    return f"global_load_dwordx4 %[q{c}{t}], %[qn], off offset:{256 * c + 32 * t}"


def last(e, par):
    """Last sub-tile j of the wave (par = j % 2): softmax of S1(j) -> P1(j),
    then O0 += V(j) P0(j) and O1 += V(j) P1(j).  No score MFMA reads Q any
    more, so the next item's Q loads go out here, one beside each MFMA (each
    spans 32 query rows: issued in a burst they hold the wave for ~2000
    cycles); %[qd] records that they did."""
    sm = softmax_ops(1)
    e("s_waitcnt lgkmcnt(0)")
    for i in range(8):
        f, db, tt = pv_frag(8 + i)
        e(f"{MFMA} {O_t(0, db)}, {VF(par, f)}, {P_t(0, tt)}, {O_t(0, db)}")
        if i == 0:
            check_branch(e, 1)
        for op in sm[i]:
            e(op)
        e(q_load(0, i))
    for i in range(8, 18):
        e("s_nop 0")
        for op in sm[i]:
            e(op)
    e("s_nop 1")
    e(selector(1, 0))
    e(selector(1, 1))
    for i in range(8):
        f, db, tt = pv_frag(8 + i)
        e(f"{MFMA} {O_t(1, db)}, {VF(par, f)}, {P_t(1, tt)}, {O_t(1, db)}")
        e(q_load(1, i))
    e("s_mov_b32 %[qd], 1")


def rescale_sub(e, x):
    """Subroutine: new reference max for column x, O[x] and L[x] scaled by
    alpha = exp2((M - max(M, MX)) * scale_log2)."""
    e(f"Lresc{x}_%=:")
    e("s_nop 7")
    e("s_nop 7")
    e("s_nop 7")
    if PARTIAL:
        row_max_tail(e, x)
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
    for i in range(18):
        if i:
            e("s_nop 0")
        for op in sm[i]:
            e(op)
    e("s_nop 1")
    e(selector(x, 0))
    e(selector(x, 1))


def dma_setup(e):
    """Scalar state of the loads of stream position p = t+3 into its ring
    stage ((g0 + p) % 4): %[dm] the LDS address of this wave's first 1 KiB,
    %[dk] / %[dv] the byte offsets of the K / V rows.  Positions from nt on
    are the next item's tiles p - nt (its resources replace this item's)."""
    e("s_add_u32 %[s2], %[t], 3")
    e("s_sub_u32 %[s3], %[s2], %[nt]")
    e("s_cmp_ge_u32 %[s2], %[nt]")
    e("s_cselect_b32 %[s3], %[s3], %[s2]")
    e("s_cselect_b64 s[88:89], s[80:81], s[88:89]")
    e("s_cselect_b64 s[90:91], s[82:83], s[90:91]")
    e("s_cselect_b64 s[92:93], s[84:85], s[92:93]")
    e("s_cselect_b64 s[94:95], s[86:87], s[94:95]")
    e("s_mul_i32 %[dk], %[s3], %[ks64]")
    e("s_mul_i32 %[dv], %[s3], %[vs64]")
    stage_addr(e, "%[dm]", "%[s2]", "%[ldsw]")


def stage_addr(e, dst, pos, base):
    """dst = base + 32 KiB * ((g0 + pos) % 4)."""
    e(f"s_add_u32 {dst}, {pos}, %[g0]")
    e(f"s_and_b32 {dst}, {dst}, 3")
    e(f"s_lshl_b32 {dst}, {dst}, 15")
    e(f"s_add_u32 {dst}, {dst}, {base}")


def dma_load(kind, rk=RK, rv=RV):
    """One 1 KiB load (16 rows of K or V) straight into LDS."""
    if kind == "K":
        return ["s_mov_b32 m0, %[dm]", "s_nop 0", f"buffer_load_dwordx4 %[ldk], {rk}, %[dk] offen lds",
                "s_add_u32 %[dk], %[dk], %[ks16]", "s_add_u32 %[dm], %[dm], 0x1000"]
    return ["s_mov_b32 m0, %[dm]", "s_nop 0", f"buffer_load_dwordx4 %[ldv], {rv}, %[dv] offen lds",
            "s_add_u32 %[dv], %[dv], %[vs16]", "s_add_u32 %[dm], %[dm], 0x1000"]


def build_rsrc(e, fixed_lo, base, rng):
    """Fixed SGPRs fixed_lo..+3 = raw buffer resource {base, rng bytes}."""
    e(f"s_mov_b64 s[{fixed_lo}:{fixed_lo + 1}], {base}")
    e(f"s_mov_b32 s{fixed_lo + 2}, {rng}")
    e(f"s_mov_b32 s{fixed_lo + 3}, 0x20000")


def generate() -> str:
    e = Emitter()
    # ---------------------------------------------------------------- entry
    # This item's Q and first tiles were loaded before the previous item's
    # output (and KV-cache) stores, the youngest memory operations of its
    # body: once no more than those are in flight they have landed; the
    # barrier makes that true for every wave.
    e("s_cmp_eq_u32 %[dostore], 0")
    e("s_cbranch_scc1 Lwait_out_%=")
    e(f"s_waitcnt vmcnt({N_OUT_STORES + N_OWN_STORES})")
    e("s_branch Lwaited_%=")
    e("Lwait_out_%=:")
    e(f"s_waitcnt vmcnt({N_OUT_STORES})")
    e("Lwaited_%=:")
    e("s_waitcnt lgkmcnt(0)")
    build_rsrc(e, 88, "%[kb]", "%[kr]")
    build_rsrc(e, 92, "%[vb]", "%[vr]")
    build_rsrc(e, 80, "%[knb]", "%[knr]")
    build_rsrc(e, 84, "%[vnb]", "%[vnr]")
    e("s_mov_b32 %[qd], 0")
    e("s_barrier")
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
    # S(0) of both columns from K(0) (set 0); then K(1) into set 1 and V(0)
    # into V set 0 in the order of slot A's and slot B's reads, so the first
    # A finds the reads in flight that every later A finds.
    e("s_cmp_eq_u32 %[nsub], 0")
    e("s_cbranch_scc1 Lpro_end_%=")
    e("s_mov_b32 %[s2], 0")
    stage_addr(e, "%[s0]", "%[s2]", "%[lds0]")    # stage of tile 0
    for t in range(8):
        e(f"v_add_u32 {v(KA + t)}, %[s0], %[ko{t}]")
    for t in range(8):
        e(f"ds_read_b128 {KF(0, t)}, {v(KA + t)}")
    e("s_add_u32 %[s2], %[s0], 0x4000")
    for db in range(4):
        e(f"v_add_u32 {v(VA + db)}, %[s2], %[vo{db}]")
    e("s_waitcnt lgkmcnt(0)")
    for t in range(8):
        e(f"{MFMA} {S_t(0)}, {KF(0, t)}, %[q0{t}], {'0' if t == 0 else S_t(0)}")
        e(f"{MFMA} {S_t(1)}, {KF(0, t)}, %[q1{t}], {'0' if t == 0 else S_t(1)}")
        e(f"ds_read_b128 {KF(1, t)}, {v(KA + t)} offset:8192")
    for f, h in V_ORDER:
        db, tt = f // 2, f % 2
        e(f"ds_read_b64_tr_b16 {VF_half(0, f, h)}, {v(VA + db)} offset:{4096 * tt + 2048 * h}")
    e("s_nop 7")
    e("s_nop 7")
    e("s_nop 7")
    e("s_cmp_lt_u32 %[wfull], 32")
    e("s_cbranch_scc0 Lpro_nomask_%=")
    e("s_mov_b32 %[s6], 0")
    mask(e, 0, "%[s6]", full=True)
    mask(e, 1, "%[s6]", full=True)
    e("s_branch Lpro_ref_%=")
    e("Lpro_nomask_%=:")
    for c in range(2):
        for op in row_max_ops(c):
            e(op)
        row_max_tail(e, c)
    e("Lpro_ref_%=:")
    set_ref(e, 0)
    set_ref(e, 1)
    compare(e, 1)   # false: the reference max of column 1 is its row max
    softmax_block(e, 0)
    e("Lpro_end_%=:")
    # ------------------------------------------------------------ tile loop
    # Read addresses at the start of iteration t: KA of tile t+1 (K(2t+2),
    # K(2t+3) in the A slots), VA of tile t (V(2t+1) in B(2t)), VB of tile t+1
    # (V(2t+2) in B(2t+1)), each refreshed in a slot that does not read it:
    # VB in A(2t), VA <- VB in A(2t+1), KA in B(2t+1).  %[s0] holds the V base
    # of tile t+1 and %[s1] the stage of tile t+2 for those updates.
    e("s_mov_b32 %[s2], 1")
    stage_addr(e, "%[s1]", "%[s2]", "%[lds0]")
    for t in range(8):
        e(f"v_add_u32 {v(KA + t)}, %[s1], %[ko{t}]")
    e("s_mov_b32 %[s2], 0")
    stage_addr(e, "%[s0]", "%[s2]", "%[lds0]")
    e("s_add_u32 %[s0], %[s0], 0x4000")
    for db in range(4):
        e(f"v_add_u32 {v(VA + db)}, %[s0], %[vo{db}]")
    e("s_mov_b32 %[t], 0")
    e("s_cmp_eq_u32 %[nt], 0")
    e("s_cbranch_scc1 Ltdone_%=")
    e("Ltile_%=:")
    e("s_add_u32 %[s2], %[t], 1")
    stage_addr(e, "%[s0]", "%[s2]", "%[lds0]")
    e("s_add_u32 %[s0], %[s0], 0x4000")          # V base of tile t+1
    e("s_add_u32 %[s2], %[t], 2")
    stage_addr(e, "%[s1]", "%[s2]", "%[lds0]")    # stage of tile t+2
    dma_setup(e)
    # sync: tile t+1 has landed for every wave, and every wave is done with
    # tile t-1, whose stage the loads of position t+3 refill (at t = 0 the
    # entry's wait and barrier did both)
    e("s_cmp_eq_u32 %[t], 0")
    e("s_cbranch_scc1 Lsynced_%=")
    e("s_waitcnt vmcnt(8)")
    e("s_barrier")
    e("Lsynced_%=:")
    # straight-line iteration when sub-tiles 2t, 2t+1 are full and unmasked
    # (64 t + 96 <= w_full implies 2t + 2 < nsub)
    e("s_lshl_b32 %[s5], %[t], 6")
    e("s_add_u32 %[s5], %[s5], 96")
    e("s_cmp_le_u32 %[s5], %[wfull]")
    e("s_cbranch_scc0 Lgen_%=")
    loads = [dma_load("K"), dma_load("K"), dma_load("K"), dma_load("K"),
             dma_load("V"), dma_load("V"), dma_load("V"), dma_load("V")]
    vb_upd = [f"v_add_u32 {v(VB + db)}, %[s0], %[vo{db}]" for db in range(4)]
    va_upd = [f"v_mov_b32 {v(VA + db)}, {v(VB + db)}" for db in range(4)]
    ka_upd = [f"v_add_u32 {v(KA + t)}, %[s1], %[ko{t}]" for t in range(8)]

    def extras(ld0, ld1, addr, steps):
        x = {3: list(ld0), 11: list(ld1)}
        for st, op in zip(steps, addr):
            x.setdefault(st, []).append(op)
        return x

    slot(e, 0, 0, extra=extras(loads[0], loads[1], vb_upd, [1, 5, 9, 13]))
    slot(e, 1, 0, extra=extras(loads[2], loads[3], [], []))
    slot(e, 0, 1, extra=extras(loads[4], loads[5], va_upd, [1, 5, 9, 13]))
    slot(e, 1, 1, extra=extras(loads[6], loads[7], ka_upd, [0, 2, 4, 6, 8, 10, 12, 14]))
    e("s_add_u32 %[t], %[t], 1")
    e("s_cmp_lt_u32 %[t], %[nt]")
    e("s_cbranch_scc1 Ltile_%=")
    e("s_branch Ltdone_%=")
    # ---- general iteration: the loads together, then per sub-tile j the
    # masks, the slots, or the wave's last sub-tile
    e("Lgen_%=:")
    for ld in loads:
        for op in ld:
            e(op)
    for op in vb_upd:
        e(op)
    for sub in range(2):
        e("s_lshl_b32 %[j], %[t], 1")
        if sub:
            e("s_add_u32 %[j], %[j], 1")
        e("s_add_u32 %[s5], %[j], 1")
        e("s_lshl_b32 %[s6], %[j], 5")              # 32 j
        e("s_cmp_lt_u32 %[s5], %[nsub]")
        e(f"s_cbranch_scc0 Lnofull{sub}_%=")
        # ---- full sub-tile j: A(j), B(j)
        e("s_add_u32 %[s3], %[s6], 32")
        e("s_cmp_gt_u32 %[s3], %[wfull]")
        e(f"s_cbranch_scc0 LmA{sub}_%=")
        mask(e, 1, "%[s6]")
        e(f"LmA{sub}_%=:")
        slot(e, 0, sub)
        e("s_add_u32 %[s3], %[s6], 64")
        e("s_cmp_gt_u32 %[s3], %[wfull]")
        e(f"s_cbranch_scc0 LmB{sub}_%=")
        e("s_add_u32 %[s3], %[s6], 32")
        mask(e, 0, "%[s3]")
        e(f"LmB{sub}_%=:")
        slot(e, 1, sub)
        e(f"s_branch Lsub{sub}_%=")
        # ---- last sub-tile of the wave
        e(f"Lnofull{sub}_%=:")
        e("s_cmp_eq_u32 %[s5], %[nsub]")
        e(f"s_cbranch_scc0 Lsub{sub}_%=")
        e("s_add_u32 %[s3], %[s6], 32")
        e("s_cmp_gt_u32 %[s3], %[wfull]")
        e(f"s_cbranch_scc0 LmL{sub}_%=")
        mask(e, 1, "%[s6]")
        e(f"LmL{sub}_%=:")
        last(e, sub)
        e(f"Lsub{sub}_%=:")
    for op in va_upd + ka_upd:
        e(op)
    e("s_add_u32 %[t], %[t], 1")
    e("s_cmp_lt_u32 %[t], %[nt]")
    e("s_cbranch_scc1 Ltile_%=")
    e("Ltdone_%=:")
    # ------------------------------------------------------------- epilogue
    # (1) Items of fewer than three tiles: the next item's tiles at stream
    # positions nt..2 (its tiles 0..2-nt) go into the stages of this item's
    # phantom tiles once every wave is done with the ring.
    e("s_cmp_lt_u32 %[nt], 3")
    e("s_cbranch_scc0 Lnomiss_%=")
    e("s_waitcnt lgkmcnt(0)")
    e("s_barrier")
    e("s_mov_b32 %[s2], %[nt]")
    e("Lmiss_%=:")
    e("s_sub_u32 %[s3], %[s2], %[nt]")
    e("s_mul_i32 %[dk], %[s3], %[ks64]")
    e("s_mul_i32 %[dv], %[s3], %[vs64]")
    stage_addr(e, "%[dm]", "%[s2]", "%[ldsw]")
    for kind in "KKKKVVVV":
        for op in dma_load(kind, RKN, RVN):
            e(op)
    e("s_add_u32 %[s2], %[s2], 1")
    e("s_cmp_lt_u32 %[s2], 3")
    e("s_cbranch_scc1 Lmiss_%=")
    e("Lnomiss_%=:")
    # (2) KV-cache store (when %[dostore]): this wave's own rows of the item
    # (rows %[lrow] + 4 i of its share, 16 bytes at chunk l % 16) and their
    # slots, loaded now from L2 (the tiles staged them moments ago) into the
    # fragment AGPRs, dead after the loop; stored after the output.
    e("s_cmp_eq_u32 %[dostore], 0")
    e("s_cbranch_scc1 Lnoload_%=")
    build_rsrc(e, 80, "%[okb]", "%[okr]")   # from the wave's first own row (not clamped to max_seqlen_k)
    build_rsrc(e, 84, "%[ovb]", "%[ovr]")
    build_rsrc(e, 88, "%[sb]", "%[srng]")
    e("s_lshr_b32 %[s5], %[ks16], 2")     # 4 K rows
    e("s_lshr_b32 %[s6], %[vs16], 2")     # 4 V rows
    e("s_mov_b32 %[s2], 0")
    e("s_mov_b32 %[s3], 0")
    for i in range(8):
        e(f"buffer_load_dwordx4 {ar(KF_SET[0] + 4 * i, 4)}, %[rvk], s[80:83], %[s2] offen")
        e(f"buffer_load_dwordx4 {ar(VF_A + 4 * i, 4)}, %[rvv], s[84:87], %[s3] offen")
        e(f"buffer_load_dwordx2 {ar(VF_A + 32 + 2 * i, 2)}, %[slv], s[88:91], 0 offen offset:{32 * i}")
        if i < 7:
            e("s_add_u32 %[s2], %[s2], %[s5]")
            e("s_add_u32 %[s3], %[s3], %[s6]")
    e("Lnoload_%=:")
    # (3) Q of the next item into the Q operands, unless the wave's last
    # sub-tile loaded it (a wave without queries has none)
    e("s_cmp_eq_u32 %[qd], 0")
    e("s_cbranch_scc0 Lqdone_%=")
    for c in range(2):
        for t in range(8):
            e(q_load(c, t))
    e("Lqdone_%=:")
    # (4) O / l rounded to bf16, through this wave's LDS staging rows (beside
    # the ring: 32 rows x 128 bytes at a 136-byte pitch, one half of a column
    # at a time) to whole 128-byte row segments in global memory.  Lane l
    # holds query l % 32, dims 32 db + 8 i + 4 (l / 32) + 0..3 of register
    # group i; rows past the segment fall outside the output resource.  A
    # wave's LDS operations execute in order, so a half's reads follow its
    # writes and the next half's writes follow those reads with no wait; only
    # the global stores wait for the read data.  The address registers (dead
    # after the loop) take 16 accumulators at a time, the score registers the
    # read-back rows.  The stores are non-temporal: nothing reads the output
    # back in this launch, and streamed past the L2 it leaves the K/V rows
    # there (8 x 1024 at 16/8 heads: 41.2-41.8 against 42.1-42.8 us).
    build_rsrc(e, 88, "%[ob]", "%[orng]")
    e("s_nop 7")
    e("s_nop 7")
    e("s_nop 7")
    e(f"ds_bpermute_b32 {v(T0)}, %[bpa], {v(L[0])}")
    e(f"ds_bpermute_b32 {v(T1)}, %[bpa], {v(L[0] + 1)}")
    e(f"ds_bpermute_b32 {v(T2)}, %[bpa], {v(L[1])}")
    e(f"ds_bpermute_b32 {v(T3)}, %[bpa], {v(L[1] + 1)}")
    e("s_waitcnt lgkmcnt(0)")
    e(f"v_cmp_ne_u32 vcc, 0, %[hi16]")
    e(f"v_cndmask_b32 {v(T0)}, {v(T0)}, {v(T1)}, vcc")        # row sum of this lane's query, column 0
    e(f"v_cndmask_b32 {v(T2)}, {v(T2)}, {v(T3)}, vcc")        # column 1
    e(f"v_rcp_f32 {v(T1)}, {v(T0)}")
    e(f"v_rcp_f32 {v(T3)}, {v(T2)}")
    e(f"v_cmp_lt_f32 vcc, 0, {v(T0)}")
    e(f"v_cndmask_b32 {v(T1)}, 0, {v(T1)}, vcc")              # 1/l, 0 for an empty row
    e(f"v_cmp_lt_f32 vcc, 0, {v(T2)}")
    e(f"v_cndmask_b32 {v(T3)}, 0, {v(T3)}, vcc")
    n_out = 0
    for x in range(2):
        inv = v(T1) if x == 0 else v(T3)
        base = O_A + 64 * x
        for hh in range(2):
            for db in (2 * hh, 2 * hh + 1):
                for i in range(16):
                    e(f"v_accvgpr_read_b32 {v(KA + i)}, a{base + 16 * db + i}")
                for i in range(16):
                    e(f"v_mul_f32 {v(KA + i)}, {v(KA + i)}, {inv}")
                pb = P[db % 2]
                for r in range(4):
                    e(f"v_cvt_pk_bf16_f32 {v(pb + 2 * r)}, {v(KA + 4 * r)}, {v(KA + 4 * r + 1)}")
                    e(f"v_cvt_pk_bf16_f32 {v(pb + 2 * r + 1)}, {v(KA + 4 * r + 2)}, {v(KA + 4 * r + 3)}")
                for r in range(4):
                    e(f"ds_write_b64 %[stw], {vr(pb + 2 * r, 2)} offset:{64 * (db % 2) + 16 * r}")
            # rows 8 i + l / 8, bytes 16 (l % 8) of the half
            for i in range(4):
                e(f"ds_read_b128 {vr(S[hh] + 4 * i, 4)}, %[str] offset:{1088 * i}")
        e("s_waitcnt lgkmcnt(0)")
        for hh in range(2):
            e("s_mov_b32 %[s2], 0")
            for i in range(4):
                e(f"buffer_store_dwordx4 {vr(S[hh] + 4 * i, 4)}, %[osv], {RK}, %[s2] offen offset:{256 * x + 128 * hh} nt")
                n_out += 1
                if i < 3:
                    e("s_add_u32 %[s2], %[s2], %[ost8]")
    assert n_out == N_OUT_STORES, n_out
    # (5) the own rows into the KV caches: row valid when within the wave's
    # share and its slot in [0, num_rows); an invalid row's offset falls
    # outside the cache resource.  The rows' loads are older than the output
    # stores (and younger than the Q loads, unless the epilogue issued those).
    e("s_cmp_eq_u32 %[dostore], 0")
    e("s_cbranch_scc1 Lnostore_%=")
    e(f"s_waitcnt vmcnt({N_OUT_STORES})")
    build_rsrc(e, 88, "%[kcb]", "%[crng]")
    build_rsrc(e, 92, "%[vcb]", "%[crng]")
    e("s_mov_b32 s80, %[nrows]")
    e("s_mov_b32 s81, 0")
    for i in range(8):
        e(f"v_accvgpr_read_b32 {v(T0)}, a{VF_A + 32 + 2 * i}")
        e(f"v_accvgpr_read_b32 {v(T1)}, a{VF_A + 33 + 2 * i}")
        e(f"s_sub_u32 %[s2], %[nvalid], {4 * i}")
        e(f"v_cmp_gt_i32 %[ret], %[s2], %[lrow]")                # row within the share
        e(f"v_cmp_gt_u64 vcc, s[80:81], {vr(T0, 2)}")            # slot in [0, num_rows)
        e("s_and_b64 vcc, vcc, %[ret]")
        e(f"v_mul_lo_u32 {v(T2)}, {v(T0)}, %[cstride]")
        e(f"v_add_u32 {v(T2)}, {v(T2)}, %[chunk16]")
        e(f"v_cndmask_b32 {v(T2)}, -1, {v(T2)}, vcc")
        e(f"buffer_store_dwordx4 {ar(KF_SET[0] + 4 * i, 4)}, {v(T2)}, s[88:91], 0 offen")
        e(f"buffer_store_dwordx4 {ar(VF_A + 4 * i, 4)}, {v(T2)}, s[92:95], 0 offen")
    assert 2 * 8 == N_OWN_STORES
    e("Lnostore_%=:")
    e("s_branch Lend_%=")
    # ------------------------------------------------- out-of-line code
    for ln in e.stubs:
        e(ln)
    rescale_sub(e, 0)
    rescale_sub(e, 1)
    e("Lend_%=:")
    return e.text()


HEADER = """// Generated by gen_prefill_wide_asm.py -- do not edit by hand.
// The per-item body of prefill_wide_kernel (zero-init, scores of sub-tile 0,
// the tile loop with its slots, masks, rescales and LDS staging, and the
// normalised output written to the LDS staging area) as one gfx950
// inline-assembly template, and the registers it clobbers; register map,
// schedule and hazard rules in the generator.
#pragma once
"""


def render() -> str:
    body = generate()
    lit = "\n".join('  "' + ln.replace('"', '\\"') + '\\n"' for ln in body.split("\n"))
    n = sum(1 for ln in body.split("\n") if ln and not ln.endswith(":"))
    clob = ", ".join([f'"v{i}"' for i in VGPR_CLOBBER] + [f'"a{i}"' for i in AGPR_CLOBBER] +
                     [f'"s{i}"' for i in SGPR_CLOBBER] + ['"vcc"', '"m0"', '"scc"', '"memory"'])
    return (HEADER + f"// {n} instructions.\n#define AAC_PW_ITEM_ASM \\\n" + " \\\n".join(lit.split("\n")) +
            "\n\n#define AAC_PW_CLOBBERS " + clob + "\n")


def main() -> int:
    out = render()
    path = Path(__file__).resolve().parent / "prefill_wide_asm.inc"
    if len(sys.argv) > 1 and sys.argv[1] == "--check":
        return 0 if path.read_text() == out else 1
    path.write_text(out)
    print(f"wrote {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
