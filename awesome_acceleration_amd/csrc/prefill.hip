// Varlen causal GQA prefill attention (gfx950, bf16/fp16 MFMA) -- the
// reference's flash_attn_varlen_func(q, k, v, cu, cu, max, max, causal=True)
// call (llm.py:178-184), and with the store folded in, llm.py:171-184.
//
// Tiling (FlashAttention-2 style, Dao 2023, re-derived for CDNA4 MFMA):
//   * A workgroup (8 wavefronts, 2 per SIMD) owns one KV head h of one
//     segment and a block of BQ queries for all G = Hq/Hkv query heads that
//     read h.  Wave w serves 32 queries of one head; with G = 2 the eight
//     waves cover 128 queries x 2 heads, so every K/V tile staged in LDS feeds
//     2 heads x 128 queries (the KV head is shared across its query heads).
//     Two waves per SIMD let one wave's MFMAs overlap the other's softmax.
//   * Scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_32x32x16_{bf16,f16}: A = 32 keys x 16 dims read from LDS,
//     B = 16 dims x 32 queries held in registers for the whole kernel.  The
//     32x32 accumulator gives lane l the column of query l%32 and 16 of the 32
//     keys (rows 8*(i/4) + 4*(l/32) + i%4), so the softmax of one query lives
//     in one lane and its partner l^32: a row max costs one cross-lane swap,
//     the row sum stays lane-partial until the end.
//   * The probabilities, rounded to bf16, are already laid out as the B operand
//     of O^T += V^T P^T (B[k][n] sits in lane n + 32*(k/8)); V^T comes from an
//     LDS tile that is written transposed ([dim][key]) when it is staged.
//   * Online softmax in fp32 in the log2 domain (exp via v_exp_f32) with
//     lazy rescaling (the running max used for the exponent only moves when a
//     row max exceeds it by more than 2^8, as in FlashAttention-3), so the
//     accumulators are rarely touched by VALU work.
//   * Causal masking is bottom-right aligned (query i sees keys
//     j <= i + Lk - Lq); key tiles beyond a wave's last visible key are
//     skipped, and only tiles that cross the diagonal evaluate the mask.
//   * Persistent grid, one workgroup per CU: the work items (KV head,
//     segment, q-block) are taken heaviest causal q-blocks first in a zigzag
//     that pairs heavy with light items, and each workgroup issues the next
//     item's Q and first K/V tile before the current item's epilogue.
//   * Store in the same kernel (llm.py:171-174, the causal self-attention
//     call): each item writes its own q-block's K/V rows into the cache
//     through slot_mapping after its output, while the next item's loads are
//     in flight -- one launch instead of a store kernel and an attention
//     kernel (8 x 1024 Qwen3-0.6B layer: 60.9 -> 53.1 us).
//
// FLOPs per launch (the MFMA roofline): 4 * Hq * D * sum over segments of the
// visible (query, key) pairs, i.e. 4*Hq*D*L(L+1)/2 per causal segment.

#include <algorithm>
#include <atomic>

#include "prefill_common.h"
#include "prefill_wide.h"

namespace aac {

namespace pf {

constexpr int kWaves = 8;        // wavefronts per workgroup (2 per SIMD)
constexpr int kThreads = 64 * kWaves;

template <int G, bool CAUSAL, bool F16, bool STORE, bool SPLIT>
__global__ __launch_bounds__(kThreads, 1) void prefill_kernel(Args a) {
  constexpr int WH = G;                // head slots per workgroup (one head per wave)
  constexpr int WQ = kWaves / WH;      // 32-query slots per workgroup
  constexpr int BQ = 32 * WQ;
  static_assert(WH * WQ == kWaves, "eight waves per workgroup");
  typedef Mfma<F16> M;

  // LDS: the K / V^T ring, reused after each item to stage the output tile
  constexpr int kRingElems = STAGES * (BKV * KPITCH + D * BKV);
  static_assert(kWaves * 32 * OPITCH <= kRingElems, "output staging fits in the ring");
  __shared__ __attribute__((aligned(16))) u16 lds[kRingElems];
  __shared__ int split_last;  // SPLIT: this workgroup's piece was its item's last
  auto Ks = [&](int st) { return lds + st * (BKV * KPITCH); };
  auto Vt = [&](int st) { return lds + STAGES * BKV * KPITCH + st * (D * BKV); };

  const int tid = threadIdx.x, lane = tid & 63;
  // The wave index made explicitly wave-uniform: the staging role, buffer
  // resource, row stride and scalar offsets then live in SGPRs (a per-lane
  // resource would turn every buffer load into a readfirstlane loop).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Column slot (head wh, 32-query slot wq) of this wave.  Waves w and w+4 of
  // a workgroup share a SIMD (measured), so wave w >= 4 takes slot 11 - w:
  // on the causal diagonal each SIMD then pairs a wave with few visible keys
  // with one that has many, instead of two heavy (or two light) waves.
  const int cslot = wave < 4 ? wave : 11 - wave;
  const int wq = cslot % WQ, wh = cslot / WQ;
  const int hl = lane >> 5;  // lane half
  const int col = lane & 31;

  // ---- staging.  Waves 0-3 stage K (thread: rows (tid>>4) + 16*i), waves
  // 4-7 stage V (thread: rows 4*(tid>>4) + i, transposed into V^T), 16 B at
  // dim (tid&15)*8.  Buffer loads return zeros for rows >= kv_end (the
  // resource covers exactly the visible rows), so tails need no clamping.
  const bool k_role = wave < 4;
  const int st_r = (tid & 255) >> 4, st_c = (tid & 15) * 8;
  const int row_bytes = (int)((k_role ? a.k_stride : a.v_stride) * 2);
  // per-thread staging offsets: global (bytes, one VGPR; the row step goes
  // into the scalar offset) and LDS (elements)
  const int st_voff = (k_role ? st_r : st_r * 4) * row_bytes + st_c * 2;
  const int st_rstep = k_role ? 16 * row_bytes : row_bytes;
  const int k_woff = st_r * KPITCH + st_c;
  u32x4 sp[4];

  // per-lane LDS read offsets (elements).  For V^T row 32c + col the octet
  // swizzle term is sw0 ^ 4*(c & 1), so the octet of key group g is
  // (hl ^ sw0) ^ 4*(c&1) ^ 2*g: four distinct offsets cover every (c, g).
  const int k_rd = col * KPITCH + hl * 8;
  const int v_base = col * BKV;
  int v_oct[4];
  {
    const int x0 = hl ^ ((col ^ (col >> 3)) & 7);
#pragma unroll
    for (int k = 0; k < 4; ++k) v_oct[k] = (x0 ^ (2 * k)) << 3;
  }

  // ---- work items (q-block rank z, segment s, KV head h), numbered
  // rank-major so that the heaviest causal q-blocks come first.  The grid is
  // persistent (one workgroup per CU): workgroup w of P takes item k*P + w in
  // even rounds k and (k+1)*P - 1 - w in odd rounds, a zigzag that pairs
  // heavy with light items, and skips the ranks a short segment lacks.
  struct Item {
    int h, s, qb, q_beg, Lq, k_beg, Lk;
    int t0, t1;         // key tiles [t0, t1) of this piece (the whole range without SPLIT)
    int id, piece, np;  // SPLIT: item number, piece, pieces of the item
  };
  const int n_hs = a.hkv * a.n_seqs;
  const int n_split = SPLIT ? a.n_split : 1;
  const int per_rank = n_hs * n_split;  // work units of one q-block rank
  const int n_items = per_rank * a.n_qblocks;
  const int P = gridDim.x, w = blockIdx.x;
  auto item_index = [&](int k) { return (k & 1) ? (k + 1) * P - 1 - w : k * P + w; };
  auto seg_of = [&](int i) { return ((i % per_rank) % n_hs) / a.hkv; };
  // keys visible to the whole workgroup (bottom-right causal alignment)
  auto kv_end_of = [&](const Item& it) {
    const int wg_qmax = min(it.qb * BQ + BQ, it.Lq) - 1;
    return CAUSAL ? max(0, min(it.Lk, wg_qmax + 1 + it.Lk - it.Lq)) : it.Lk;
  };
  // item i from its segment's bounds; false for a rank the segment lacks
  auto decode = [&](int i, int q0, int q1, int k0, int k1, Item& it) -> bool {
    const int z = i / per_rank;
    const int r = i - z * per_rank;
    const int pc = SPLIT ? r / n_hs : 0;
    const int hs = r - pc * n_hs;
    it.s = hs / a.hkv;
    it.h = hs - it.s * a.hkv;
    it.q_beg = q0;
    it.Lq = q1 - q0;
    it.k_beg = k0;
    // clamped to max_seqlen_k, which the host checked against the 32-bit
    // staging offsets (a caller that understates it gets truncated
    // attention, never an out-of-range read)
    it.Lk = min(k1 - k0, a.max_k);
    const int nqb = (it.Lq + BQ - 1) / BQ;
    it.qb = CAUSAL ? nqb - 1 - z : z;
    if (z >= nqb) return false;
    if constexpr (SPLIT) {
      const int nt = (kv_end_of(it) + BKV - 1) / BKV;
      it.id = z * n_hs + hs;
      it.piece = pc;
      it.np = min(n_split, max(nt, 1));
      if (pc >= it.np) return false;  // a short item has fewer pieces
      it.t0 = pc * nt / it.np;
      it.t1 = (pc + 1) * nt / it.np;
    }
    return true;
  };
  // key tiles [t_first, t_end) of an item's piece (all of them without SPLIT)
  auto t_first = [&](const Item& it) { return SPLIT ? it.t0 : 0; };
  auto t_end = [&](const Item& it, int kv_end) { return SPLIT ? it.t1 : (kv_end + BKV - 1) / BKV; };
  // first valid item of round k or later (k is left at its round)
  auto next_item = [&](int& k, Item& it) -> bool {
    for (; k * P < n_items; ++k) {
      const int i = item_index(k);
      if (i >= n_items) continue;
      const int sg = seg_of(i);
      if (decode(i, a.cu_q[sg], a.cu_q[sg + 1], a.cu_k[sg], a.cu_k[sg + 1], it)) return true;
    }
    return false;
  };
  auto rsrc_of = [&](const Item& it, int kv_end) {
    const u16* base = (k_role ? a.k + (int64_t)it.k_beg * a.k_stride
                              : a.v + (int64_t)it.k_beg * a.v_stride) + it.h * D;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<u16*>(base), 0,
                                             kv_end > 0 ? (kv_end - 1) * row_bytes + D * 2 : 0,
                                             0x00020000);
  };
  // Q fragments: B operand of S^T = K Q^T, lane = query column, 8 dims; rows
  // past the segment are clamped (and never stored).
  u32x4 qf[8];
  f32x16 o[4];  // O^T accumulators (dims 32c..32c+31 x the wave's 32 queries)
  auto load_q = [&](const Item& it) {
    const int qi = it.qb * BQ + wq * 32 + col;
    const int qrow = it.q_beg + min(qi, max(it.Lq - 1, 0));
    const u16* qp = a.q + (int64_t)qrow * a.q_stride + (it.h * G + wh) * D + hl * 8;
#pragma unroll
    for (int t = 0; t < 8; ++t) qf[t] = *reinterpret_cast<const u32x4*>(qp + 16 * t);
  };

  // ---- the KV-cache store (STORE).  Each item stores the K/V rows of its own
  // q-block (its queries' rows taken as keys, since cu_q == cu_k) for its KV
  // head: loaded right after its tile loop (they were staged moments before,
  // so they come from L2), ahead of the next item's loads so that waiting
  // for them never waits for those, and written after the output.  The item
  // of rank 0 of a segment also stores the q-blocks no item owns (a
  // max_seqlen_q below the segment's length), and workgroup 0 the tokens
  // before cu[0] and from cu[n] on.  Every token's rows are thus written at
  // least once; a row written twice gets the same bytes both times.  The
  // store's arguments are read from the kernel-argument segment where they
  // are used, so they hold no SGPRs through the tile loop.
  auto sargs = [&]() { return kernel_args(); };
  auto copy_span = [&](int64_t t0, int64_t t1, int h0, int h1) {  // the rare paths
    store_kv_span<kThreads>(a, tid, t0, t1, h0, h1);
  };
  // own rows of an item: thread rows (tid >> 4) + 32 i, 16 B at dim 8 (tid & 15);
  // rows past the q-block repeat its last row (same bytes to the same slot)
  constexpr int NI = BQ / 32 < 4 ? BQ / 32 : 4;  // passes issued early (G = 1 has 8)
  int64_t csl[NI];
  u32x4 ck[NI], cv[NI];
  auto own_load = [&](KArgs* sa, const Item& it, int pass, int64_t& sl, u32x4& kx, u32x4& vx) {
    const int r0 = it.qb * BQ;
    const int nr = min(BQ, it.Lq - r0);  // >= 1 for an existing item
    const int rr = min((tid >> 4) + 32 * pass, nr - 1);
    const int64_t t = (int64_t)it.k_beg + r0 + rr;
    const int64_t tok = min(t, (int64_t)sa->n_tok - 1);
    sl = t < sa->n_tok ? sa->slots[tok] : -1;
    kx = *reinterpret_cast<const u32x4*>(a.k + tok * a.k_stride + it.h * D + (tid & 15) * 8);
    vx = *reinterpret_cast<const u32x4*>(a.v + tok * a.v_stride + it.h * D + (tid & 15) * 8);
  };
  auto own_store = [&](KArgs* sa, const Item& it, int64_t sl, const u32x4& kx, const u32x4& vx) {
    if ((uint64_t)sl < (uint64_t)sa->num_rows) {
      const int64_t dst = (sl * a.hkv + it.h) * D + (tid & 15) * 8;
      *reinterpret_cast<u32x4*>(sa->kc + dst) = kx;
      *reinterpret_cast<u32x4*>(sa->vc + dst) = vx;
    }
  };
  auto store_rest = [&](const Item& it) {  // after the early passes' stores
    KArgs* sa = sargs();
#pragma unroll
    for (int i = NI; i < BQ / 32; ++i) {
      int64_t sl;
      u32x4 kx, vx;
      own_load(sa, it, i, sl, kx, vx);
      own_store(sa, it, sl, kx, vx);
    }
    const int nqb = (it.Lq + BQ - 1) / BQ;
    if (nqb - 1 - it.qb == 0 && nqb > a.n_qblocks) {  // rank 0 (causal numbering)
      const int lo = nqb - a.n_qblocks;               // q-blocks [lo, nqb) have items
      copy_span(it.k_beg, it.k_beg + (int64_t)lo * BQ, it.h, it.h + 1);
    }
  };
  // workgroup 0: tokens outside [cu[0], cu[n]) (lanes 0 / 1 load the bounds now)
  const int edge_cu = STORE && blockIdx.x == 0 ? a.cu_q[(lane & 1) ? a.n_seqs : 0] : 0;
  auto store_edges = [&]() {
    if (STORE && blockIdx.x == 0) {
      const int c0 = __builtin_amdgcn_readlane(edge_cu, 0), cn = __builtin_amdgcn_readlane(edge_cu, 1);
      copy_span(0, c0, 0, a.hkv);
      copy_span(cn, sargs()->n_tok, 0, a.hkv);
    }
  };

  int k = 0;
  Item cur;
  if (!next_item(k, cur)) {
    store_edges();
    return;
  }
  int kv_end = kv_end_of(cur);
  __amdgpu_buffer_rsrc_t rs = rsrc_of(cur, kv_end);

  auto prefetch = [&](int t) {
    const int soff = t * BKV * row_bytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) sp[i] = buf_load16(rs, st_voff, soff + i * st_rstep);
  };
  auto stage_write = [&](int t) {
    if (k_role) {
      u16* ks = Ks(t % STAGES) + k_woff;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(ks + 16 * i * KPITCH) = sp[i];
    } else {
      u16* vt = Vt(t % STAGES);
#pragma unroll
      for (int jw = 0; jw < 4; ++jw) {  // dims st_c+2jw (lo halves) and st_c+2jw+1 (hi halves)
        u32x2 lo, hi;
        lo[0] = __builtin_amdgcn_perm(sp[1][jw], sp[0][jw], kSelLo);
        lo[1] = __builtin_amdgcn_perm(sp[3][jw], sp[2][jw], kSelLo);
        hi[0] = __builtin_amdgcn_perm(sp[1][jw], sp[0][jw], kSelHi);
        hi[1] = __builtin_amdgcn_perm(sp[3][jw], sp[2][jw], kSelHi);
        *reinterpret_cast<u32x2*>(vt + vt_quad_off(st_c + 2 * jw, st_r)) = lo;
        *reinterpret_cast<u32x2*>(vt + vt_quad_off(st_c + 2 * jw + 1, st_r)) = hi;
      }
    }
  };
  // S^T (scores of sub-tile j: keys 32j..32j+31) for this wave's head
  auto scores = [&](int j) {
    const u16* kr = Ks((j >> 1) % STAGES) + (j & 1) * 32 * KPITCH + k_rd;
    f32x16 st;
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) st = M::run(*reinterpret_cast<const u32x4*>(kr + 16 * t), qf[t], st);
    return st;
  };

  auto pv_step = [&](int jp, const u32x4* pb) {  // O += V(jp) P(jp)
    const u16* vt = Vt((jp >> 1) % STAGES) + v_base;
    const int g0 = 2 * (jp & 1);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int k = (2 * (c & 1)) ^ (g0 + tt);  // (4*(c&1) ^ 2*g) / 2
        const u32x4 va = *reinterpret_cast<const u32x4*>(vt + 32 * c * BKV + v_oct[k]);
        o[c] = M::run(va, pb[tt], o[c]);
      }
  };

  // Item prologue (Q and tile 0 in flight): tile 0 in LDS, tile 1 in
  // flight, S of sub-tile 0.  It is placed before the item loop and at the
  // end of each iteration, so that each copy waits for exactly its own loads
  // (one copy at the loop top would merge the wait counts of the first item
  // with those of later items, which also have the previous item's output
  // stores outstanding).
  auto prologue = [&](int t0, int t1) {
    f32x16 s0;
    if (t1 > t0) {
      stage_write(t0);
      if (t1 > t0 + 1) prefetch(t0 + 1);
      __syncthreads();
      s0 = scores(2 * t0);
    } else {
      // Q must be complete on this path too: Q left pending on any path into
      // the tile loop would make every tile wait for all vector loads,
      // including the prefetch two tiles ahead.  (gfx9 encoding: vmcnt 0,
      // expcnt and lgkmcnt unconstrained.)
      __builtin_amdgcn_s_waitcnt(0x0F70);
#pragma unroll
      for (int i = 0; i < 16; ++i) s0[i] = 0.f;
    }
    return s0;
  };

  load_q(cur);
  prefetch(t_first(cur));  // an empty resource (kv_end == 0) reads zeros
  f32x16 sc = prologue(t_first(cur), t_end(cur, kv_end));

  for (;;) {
    // Segment bounds of the next round's item, loaded now so that they have
    // arrived when this item ends (a dependent load there would cost a
    // memory round trip per item).  Lane 0 loads the start and lane 1 the
    // end: a lane-varying load stays in VGPRs until it is used, where a
    // uniform one would be moved to SGPRs (and waited for) right away.
    // The loads are issued on every path (segment 0 when there is no
    // candidate) so that the outstanding-load count the waits below rely on
    // does not depend on the branch.
    const int kc = k + 1, ic = item_index(kc);
    const bool cand = kc * P < n_items && ic < n_items;
    const int c_sg = (cand ? seg_of(ic) : 0) + (lane & 1);
    const int c_q = a.cu_q[c_sg];
    const int c_k = a.cu_k[c_sg];

    const int qi = cur.qb * BQ + wq * 32 + col;  // query index in the segment
    const int shift = cur.Lk - cur.Lq;  // bottom-right causal alignment
    // keys visible to this wave / this lane
    const int w_qmin = cur.qb * BQ + wq * 32;
    const int w_qmax = min(w_qmin + 31, cur.Lq - 1);
    const int w_end = w_qmin >= cur.Lq ? 0 : (CAUSAL ? max(0, min(cur.Lk, w_qmax + 1 + shift)) : cur.Lk);
    const int w_full = CAUSAL ? min(cur.Lk, w_qmin + 1 + shift) : cur.Lk;  // keys < w_full need no mask
    const int my_lim = CAUSAL ? min(cur.Lk, qi + 1 + shift) : cur.Lk;
    const int t0 = t_first(cur), nt = t_end(cur, kv_end);  // LDS tiles [t0, nt) (workgroup-uniform)
    const int nsub = (w_end + 31) / 32;  // 32-key sub-tiles this wave computes (of all keys)

#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[c][i] = 0.f;
    float m = -1e30f, l = 0.f;  // m: reference max of the raw scores (scale applied in exp2)


    // Ring schedule: iteration t writes tile t+1 (prefetched one tile
    // earlier) into stage (t+1)%3, issues the loads of tile t+2, computes
    // sub-tile 2t, then a barrier, then sub-tile 2t+1.  The stage's last
    // reader, tile t-2, finished before the mid-tile barrier of iteration t-1,
    // which every wave has passed; the mid-tile barrier of iteration t makes
    // tile t+1 visible before the look-ahead of sub-tile 2t+1 reads it.  The
    // LDS writes thus overlap sub-tile 2t instead of preceding a barrier.
    for (int t = t0; t < nt; ++t) {
      if (t + 1 < nt) stage_write(t + 1);
      if (t + 2 < nt) prefetch(t + 2);
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        if (sub == 1) __syncthreads();
        const int j = 2 * t + sub;
        if (j < nsub) {  // wave-uniform
          // ---- causal mask (only sub-tiles that cross this wave's diagonal)
          const int kb = 32 * j;
          if (kb + 32 > w_full) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int key = kb + 8 * (i >> 2) + 4 * hl + (i & 3);
              sc[i] = key < my_lim ? sc[i] : -INFINITY;
            }
          }
          // ---- row max (the partner lane l^32 holds the other 16 keys)
          float mx = vmax3(sc[0], sc[1], sc[2]);
#pragma unroll
          for (int i = 3; i < 15; i += 2) mx = vmax3(mx, sc[i], sc[i + 1]);
          mx = vmax(mx, sc[15]);
          {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                             false, false);
            mx = vmax(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
          }
          // Lazy rescaling: the reference max m only moves when some row max
          // exceeds it by more than kRescale (log2 units), so p <= 2^kRescale
          // and the accumulators (normalised exactly at the end) are rescaled
          // rarely; on the first sub-tile they are still zero.
          if (j == 2 * t0) {
            m = vmax(mx, -1e30f);
          } else if (__any((mx - m) * a.scale_log2 > kRescale)) {
            const float mn = vmax(m, mx);
            const float alpha = fast_exp2((m - mn) * a.scale_log2);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
              for (int i = 0; i < 16; ++i) o[c][i] *= alpha;
          }
          // ---- look-ahead scores of sub-tile j+1 (MFMA) beside the
          // exponentials of sub-tile j (VALU).  Past the wave's last sub-tile
          // the look-ahead reads a stale stage and its result is discarded.
          const float nb = -m * a.scale_log2;
          const f32x16 sn = scores(j + 1);
          float p[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sc[i], a.scale_log2, nb));
          u32x4 pb[2];
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int w = 0; w < 4; ++w) pb[tt][w] = M::pack(p[8 * tt + 2 * w], p[8 * tt + 2 * w + 1]);
          // row sum of the rounded probabilities the PV product uses
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int w = 0; w < 4; ++w) l = M::dot2_ones(pb[tt][w], l);
          pv_step(j, pb);
          sc = sn;
        }
      }
    }

    if (STORE) {
      KArgs* sa = sargs();
#pragma unroll
      for (int i = 0; i < NI; ++i) own_load(sa, cur, i, csl[i], ck[i], cv[i]);
    }

    // The next item's Q and first K/V tile go out before this item's
    // epilogue, so their latency overlaps the normalisation and stores.
    Item nxt;
    int kn = kc;
    bool more;
    if (cand && decode(ic, __builtin_amdgcn_readlane(c_q, 0), __builtin_amdgcn_readlane(c_q, 1),
                       __builtin_amdgcn_readlane(c_k, 0), __builtin_amdgcn_readlane(c_k, 1), nxt)) {
      more = true;
    } else {  // a hole or a missing rank: search the later rounds
      kn = kc + 1;
      more = kc * P < n_items && next_item(kn, nxt);
    }
    if (more) {
      kv_end = kv_end_of(nxt);
      rs = rsrc_of(nxt, kv_end);
      load_q(nxt);
      prefetch(t_first(nxt));
    }

    // ---- split keys: every piece of an item leaves its accumulators and
    // (m, l) in the workspace, and the last piece of the item to finish
    // merges the pieces in piece order -- the result does not depend on which
    // piece finishes last -- and stores the output; the others store nothing.
    // The workspace is written and read with agent-scope relaxed atomic
    // accesses (coherent across XCDs without flushing the L2, which a fence
    // would do), every piece waits for its writes to complete before it
    // counts itself finished, and the merging piece resets the count to zero
    // for the next call.  Nothing waits on another workgroup.
    bool emit = true;
    if (SPLIT && cur.np > 1) {
      typedef unsigned long long u64;
      const int64_t slot0 = (int64_t)cur.id * n_split;
      // one buffer resource over this wave's accumulator blocks of every
      // piece of the item: piece pc at pc * kPieceStride bytes, block (c, r)
      // at (c*4 + r) * 1 KiB, lane at 16 B; accessed with the sc1 policy
      // (coherent across XCDs, as the compiler's agent-scope atomics are)
      constexpr int kPieceStride = kWaves * 16 * 64 * 16;
      constexpr int kSc1 = 16;
      const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<char*>(a.ws_o) + (slot0 * kWaves + wave) * (16 * 64 * 16), 0,
          (n_split - 1) * kPieceStride + 16 * 64 * 16, 0x00020000);
      auto pml = [&](int pc) {
        return reinterpret_cast<u64*>(a.ws_ml + ((slot0 + pc) * kWaves + wave) * 64 + lane);
      };
      auto pack2 = [](float x, float y) {
        return (u64)__float_as_uint(x) | ((u64)__float_as_uint(y) << 32);
      };
      {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = o[c][4 * r + i];
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs,
                                                   lane * 16 + (c * 4 + r) * 1024,
                                                   cur.piece * kPieceStride, kSc1);
          }
        __hip_atomic_store(pml(cur.piece), pack2(m, l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this lane's writes have completed
      __syncthreads();
      if (tid == 0)
        split_last = __hip_atomic_fetch_add(a.ws_cnt + cur.id, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) == cur.np - 1;
      __syncthreads();
      emit = split_last != 0;
      if (emit) {
        if (tid == 0) __hip_atomic_store(a.ws_cnt + cur.id, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float2 ml[4];
        float mx = -1e30f;
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {
          ml[pc] = make_float2(-1e30f, 0.f);
          if (pc < cur.np) {
            if (pc == cur.piece) {
              ml[pc] = make_float2(m, l);
            } else {
              const u64 b = __hip_atomic_load(pml(pc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              ml[pc] = make_float2(__uint_as_float((u32)b), __uint_as_float((u32)(b >> 32)));
            }
          }
          mx = vmax(mx, ml[pc].x);
        }
        float wt[4];
        l = 0.f;
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {
          wt[pc] = fast_exp2((ml[pc].x - mx) * a.scale_log2);
          if (pc < cur.np) l = fmaf(ml[pc].y, wt[pc], l);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          f32x16 acc;
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
          for (int pc = 0; pc < 4; ++pc) {
            if (pc >= cur.np) continue;
            if (pc == cur.piece) {
#pragma unroll
              for (int i = 0; i < 16; ++i) acc[i] = fmaf(o[c][i], wt[pc], acc[i]);
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const f32x4 v = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, lane * 16 + (c * 4 + r) * 1024,
                                                                 pc * kPieceStride, kSc1));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[4 * r + i] = fmaf(v[i], wt[pc], acc[4 * r + i]);
              }
            }
          }
          o[c] = acc;
        }
        m = mx;
      }
    }

    // ---- epilogue: full row sum (partner lane holds the other 16 keys of
    // each 32-key sub-tile), normalise, store.  The tile goes through LDS so
    // that each store instruction writes four whole 256-byte head rows (the
    // accumulator layout would scatter 8-byte pieces over 32 rows per store).
    float lt;
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
      lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;
    __syncthreads();  // every wave is done with the ring (including the discarded look-ahead)
    u16* ob = lds + wave * (32 * OPITCH);  // this wave's 32 rows x 128 dims
    if (emit) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x2 wv;
        wv[0] = M::pack(o[c][4 * r] * inv, o[c][4 * r + 1] * inv);
        wv[1] = M::pack(o[c][4 * r + 2] * inv, o[c][4 * r + 3] * inv);
        *reinterpret_cast<u32x2*>(ob + col * OPITCH + 32 * c + 8 * r + 4 * hl) = wv;
      }
    {
      // All eight rows are read back before any store, and the stores go
      // through a buffer resource that ends after the segment's last valid
      // row, so rows past it are dropped without a branch per row.  They are
      // non-temporal (cache policy nt): 1-2% faster at 8 x 1024 than plain
      // stores, measured on MI355X.
      constexpr int kNt = 2;
      const int row0 = cur.qb * BQ + wq * 32;  // the wave's first query
      const int nrow = min(32, cur.Lq - row0);
      u16* og = a.out + (int64_t)(cur.q_beg + row0) * a.o_stride + (cur.h * G + wh) * D;
      const int ostep = (int)(a.o_stride * 2);
      const __amdgpu_buffer_rsrc_t ors =
          __builtin_amdgcn_make_buffer_rsrc(og, 0, nrow > 0 ? nrow * ostep : 0, 0x00020000);
      u32x4 val[8];
#pragma unroll
      for (int it = 0; it < 8; ++it)
        val[it] = *reinterpret_cast<const u32x4*>(ob + (4 * it + (lane >> 4)) * OPITCH + (lane & 15) * 8);
      const int voff = (lane >> 4) * ostep + (lane & 15) * 16;
#pragma unroll
      for (int it = 0; it < 8; ++it)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, val[it]), ors, voff, 4 * it * ostep, kNt);
    }
    }  // emit
    if (STORE) {
      KArgs* sa = sargs();
#pragma unroll
      for (int i = 0; i < NI; ++i) own_store(sa, cur, csl[i], ck[i], cv[i]);
      store_rest(cur);
    }
    if (!more) break;
    // Every wave has read its output rows back before the next item's tile 0
    // overwrites them.
    __syncthreads();
    cur = nxt;
    k = kn;
    sc = prologue(t_first(cur), t_end(cur, kv_end));
  }
  store_edges();
}

template <int G, bool CAUSAL, bool F16, bool STORE, bool SPLIT>
static void launch_t(Args a, int max_q, int n_cu, hipStream_t st) {
  constexpr int BQ = 32 * (kWaves / G);
  a.n_qblocks = (int)cdiv(max_q, BQ);
  const int64_t n_items = (int64_t)a.hkv * a.n_seqs * a.n_qblocks * (SPLIT ? a.n_split : 1);
  const int grid = (int)std::min<int64_t>(n_items, n_cu);  // persistent: one workgroup per CU
  hipLaunchKernelGGL((prefill_kernel<G, CAUSAL, F16, STORE, SPLIT>), dim3(grid), dim3(kThreads), 0, st,
                     a);
}

template <bool CAUSAL, bool F16, bool STORE = false, bool SPLIT = false>
static int launch_g(const Args& a, int g, int max_q, int n_cu, hipStream_t st) {
  switch (g) {
    case 1: launch_t<1, CAUSAL, F16, STORE, SPLIT>(a, max_q, n_cu, st); break;
    case 2: launch_t<2, CAUSAL, F16, STORE, SPLIT>(a, max_q, n_cu, st); break;
    case 4: launch_t<4, CAUSAL, F16, STORE, SPLIT>(a, max_q, n_cu, st); break;
    case 8: launch_t<8, CAUSAL, F16, STORE, SPLIT>(a, max_q, n_cu, st); break;
    default: return AAC_ERR_UNSUPPORTED;
  }
  return AAC_OK;
}

// ------------------------------------------------------------------ split plan
// Two pieces per item when the items are too few for the CUs and long enough
// that halving the heaviest one outweighs writing and merging the partial
// results (128 KiB per piece).  Measured on MI355X (256 CUs, bf16, causal;
// unsplit -> split, us): one 1024-token request 32.0 -> 27.4 (16/8 heads)
// and 33.0 -> 28.2 (32/8), 2 x 1024 32.6 -> 28.8, 1 x 2048 58.5 -> 43.2,
// 1 x 4096 111.9 -> 92.0; not split because it measured slower: 256 items
// of at most 16 tiles (8 x 1024 at 8/4 heads 34.8 -> 43.0, 4 x 1024 at 16/8
// 34.0 -> 43.3), items under 16 tiles (1 x 512 19.0 -> 19.4, 2 x 256
// 12.3 -> 15.9); four pieces never beat two by more than noise.
struct SplitPlan {
  int32_t n_split;
  int64_t n_items;  // items (without pieces): counters in the workspace
  size_t ws_bytes;
};
constexpr int kMaxSplit = 2;
constexpr size_t kPieceBytes = (size_t)kWaves * 64 * (64 * 4 + 8);  // accumulators + (m, l) per lane
// The item counters sit in a region of fixed size at the start of every
// workspace, so that no call's partial results ever land where a later call
// (with more items) keeps its counters; calls with more items do not split.
constexpr int64_t kMaxSplitItems = 4096;
constexpr size_t kCntBytes = kMaxSplitItems * 4;

static SplitPlan plan_split(int32_t n_seqs, int32_t max_q, int32_t max_k, int32_t hq, int32_t hkv,
                            bool causal, int n_cu) {
  SplitPlan p = {1, 0, 0};
  if (n_seqs <= 0 || max_q <= 0 || max_k <= 0 || hkv <= 0 || hq % hkv || n_cu <= 0) return p;
  const int g = hq / hkv;
  if (g != 1 && g != 2 && g != 4 && g != 8) return p;
  const int64_t BQ = 32 * (kWaves / g);
  const int64_t nqb = cdiv(max_q, BQ);
  const int64_t n_hs = (int64_t)hkv * n_seqs;
  p.n_items = n_hs * nqb;
  // plenty of items: nothing to gain (and the counters hold kMaxSplitItems)
  if (p.n_items >= 4 * (int64_t)n_cu || p.n_items > kMaxSplitItems) return p;
  auto tiles = [&](int64_t z) -> int64_t {  // key tiles of the q-block of rank z
    if (!causal) return cdiv(max_k, BKV);
    const int64_t qb = nqb - 1 - z;
    const int64_t qmax = std::min<int64_t>((qb + 1) * BQ, max_q) - 1;
    const int64_t ke = std::max<int64_t>(0, std::min<int64_t>(max_k, qmax + 1 + max_k - max_q));
    return cdiv(ke, BKV);
  };
  const int64_t heavy = tiles(0);
  const bool split = heavy >= 16 && (2 * p.n_items <= n_cu || (p.n_items <= n_cu && heavy >= 48));
  if (!split) return p;
  const int s = kMaxSplit;
  p.n_split = s;
  p.ws_bytes = kCntBytes + (size_t)p.n_items * s * kPieceBytes;
  return p;
}

}  // namespace pf

static int prefill_common(const void* q, const void* k, const void* v, int64_t q_tok_stride,
                          int64_t k_tok_stride, int64_t v_tok_stride, const int32_t* cu_seqlens_q,
                          const int32_t* cu_seqlens_k, int32_t n_seqs, int32_t max_seqlen_q,
                          int32_t max_seqlen_k, int32_t n_q_heads, int32_t n_kv_heads,
                          int32_t head_dim, float scale, int32_t causal, void* out,
                          int64_t out_tok_stride, int32_t dtype, hipStream_t stream,
                          bool launch, void* k_cache = nullptr, void* v_cache = nullptr,
                          int64_t num_cache_rows = 0, const int64_t* slot_mapping = nullptr,
                          int32_t n_store = 0, void* workspace = nullptr,
                          size_t workspace_bytes = 0) {
  if (dtype != AAC_DTYPE_BF16 && dtype != AAC_DTYPE_FP16) return AAC_ERR_UNSUPPORTED;
  if (head_dim != pf::D) return AAC_ERR_UNSUPPORTED;
  if (n_seqs < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || max_seqlen_q < 0 || max_seqlen_k < 0 ||
      q_tok_stride < 0 || k_tok_stride < 0 || v_tok_stride < 0 || out_tok_stride < 0)
    return AAC_ERR_INVALID_ARGUMENT;
  if (n_q_heads % n_kv_heads) return AAC_ERR_SHAPE;
  const int g = n_q_heads / n_kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8) return AAC_ERR_UNSUPPORTED;
  if (n_seqs == 0 || max_seqlen_q == 0) return AAC_OK;
  if (!q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k) return AAC_ERR_INVALID_ARGUMENT;
  if (q_tok_stride < (int64_t)n_q_heads * head_dim || out_tok_stride < (int64_t)n_q_heads * head_dim ||
      k_tok_stride < (int64_t)n_kv_heads * head_dim || v_tok_stride < (int64_t)n_kv_heads * head_dim)
    return AAC_ERR_SHAPE;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 || q_tok_stride % 8 ||
      k_tok_stride % 8 || v_tok_stride % 8 || out_tok_stride % 8)
    return AAC_ERR_MISALIGNED;
  // staging uses 32-bit byte offsets within one segment's K/V rows
  if ((int64_t)max_seqlen_k * std::max(k_tok_stride, v_tok_stride) * 2 >= (int64_t(1) << 31))
    return AAC_ERR_UNSUPPORTED;
  // the output stores use 32-bit byte offsets over a wave's 32 rows
  if (out_tok_stride * 2 * 32 >= (int64_t(1) << 31)) return AAC_ERR_UNSUPPORTED;
  // work items (KV head, segment, 32-query block at most) are numbered in int32
  if ((int64_t)n_kv_heads * n_seqs * cdiv(max_seqlen_q, 32) >= (int64_t(1) << 30))
    return AAC_ERR_UNSUPPORTED;
  if (!launch) return AAC_OK;
  pf::Args a;
  a.q = (const u16*)q;
  a.k = (const u16*)k;
  a.v = (const u16*)v;
  a.q_stride = q_tok_stride;
  a.k_stride = k_tok_stride;
  a.v_stride = v_tok_stride;
  a.o_stride = out_tok_stride;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.n_seqs = n_seqs;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.out = (u16*)out;
  a.max_k = max_seqlen_k;
  a.kc = (u16*)k_cache;
  a.vc = (u16*)v_cache;
  a.slots = slot_mapping;
  a.num_rows = num_cache_rows;
  a.n_tok = n_store;
  a.n_split = 1;
  a.ws_o = nullptr;
  a.ws_ml = nullptr;
  a.ws_cnt = nullptr;
  const bool f16 = dtype == AAC_DTYPE_FP16;
  int n_cu = 0;
  int rc = device_cu_count(&n_cu);
  if (rc != AAC_OK) return rc;
  // split keys when a workspace is given, the plan asks for it and the
  // workspace holds it (otherwise the call runs unsplit)
  pf::SplitPlan sp = {1, 0, 0};
  if (n_store == 0 && workspace && (uintptr_t)workspace % 256 == 0)
    sp = pf::plan_split(n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads, causal != 0, n_cu);
  if (sp.n_split > 1 && workspace_bytes >= sp.ws_bytes) {
    a.n_split = sp.n_split;
    a.ws_cnt = reinterpret_cast<int32_t*>(workspace);
    a.ws_o = reinterpret_cast<float*>((char*)workspace + pf::kCntBytes);
    a.ws_ml = reinterpret_cast<float2*>(a.ws_o + (size_t)sp.n_items * sp.n_split * pf::kWaves * 64 * 64);
    rc = causal ? (f16 ? pf::launch_g<true, true, false, true>(a, g, max_seqlen_q, n_cu, stream)
                       : pf::launch_g<true, false, false, true>(a, g, max_seqlen_q, n_cu, stream))
                : (f16 ? pf::launch_g<false, true, false, true>(a, g, max_seqlen_q, n_cu, stream)
                       : pf::launch_g<false, false, false, true>(a, g, max_seqlen_q, n_cu, stream));
  } else if (prefill_wide_supports(g, scale, f16) &&
             (n_store == 0 || num_cache_rows * n_kv_heads * head_dim * 2 < (int64_t(1) << 32)))
    // the wide kernel's cache store addresses a head's rows with 32-bit offsets
    rc = prefill_wide_launch(a, g, causal != 0, n_store > 0, max_seqlen_q, n_cu, stream);
  else if (n_store > 0)  // the store variant exists for causal attention only
    rc = f16 ? pf::launch_g<true, true, true>(a, g, max_seqlen_q, n_cu, stream)
             : pf::launch_g<true, false, true>(a, g, max_seqlen_q, n_cu, stream);
  else if (causal)
    rc = f16 ? pf::launch_g<true, true>(a, g, max_seqlen_q, n_cu, stream)
             : pf::launch_g<true, false>(a, g, max_seqlen_q, n_cu, stream);
  else
    rc = f16 ? pf::launch_g<false, true>(a, g, max_seqlen_q, n_cu, stream)
             : pf::launch_g<false, false>(a, g, max_seqlen_q, n_cu, stream);
  if (rc != AAC_OK) return rc;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}

}  // namespace aac

using namespace aac;

extern "C" size_t aac_prefill_workspace_bytes(int32_t n_seqs, int32_t max_seqlen_q,
                                              int32_t max_seqlen_k, int32_t n_q_heads,
                                              int32_t n_kv_heads, int32_t head_dim,
                                              int32_t causal) {
  if (head_dim != pf::D) return 0;
  int n_cu = 0;
  if (device_cu_count(&n_cu) != AAC_OK) return 0;
  return pf::plan_split(n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads, causal != 0, n_cu)
      .ws_bytes;
}

extern "C" int aac_prefill_varlen(const void* q, const void* k, const void* v, int64_t q_tok_stride,
                                  int64_t k_tok_stride, int64_t v_tok_stride,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int32_t n_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                  int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                  float scale, int32_t causal, void* out, int64_t out_tok_stride,
                                  void* workspace, size_t workspace_bytes, int32_t dtype,
                                  void* stream) {
  return prefill_common(q, k, v, q_tok_stride, k_tok_stride, v_tok_stride, cu_seqlens_q,
                        cu_seqlens_k, n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads,
                        head_dim, scale, causal, out, out_tok_stride, dtype, (hipStream_t)stream,
                        true, nullptr, nullptr, 0, nullptr, 0, workspace, workspace_bytes);
}

extern "C" int aac_kv_store(const void* k, const void* v, int64_t k_tok_stride,
                            int64_t v_tok_stride, void* k_cache, void* v_cache,
                            int64_t num_cache_rows, const int64_t* slot_mapping, int64_t n_tokens,
                            int32_t n_kv_heads, int32_t head_dim, int32_t dtype, void* stream);

extern "C" int aac_prefill_varlen_store(const void* q, const void* k, const void* v,
                                        int64_t q_tok_stride, int64_t k_tok_stride,
                                        int64_t v_tok_stride, const int32_t* cu_seqlens_q,
                                        const int32_t* cu_seqlens_k, int32_t n_seqs,
                                        int32_t max_seqlen_q, int32_t max_seqlen_k,
                                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                        float scale, int32_t causal, void* out,
                                        int64_t out_tok_stride, void* k_cache, void* v_cache,
                                        int64_t num_cache_rows, const int64_t* slot_mapping,
                                        int64_t n_kv_tokens, int32_t dtype, void* stream) {
  // validate the attention arguments before anything is enqueued
  int rc = prefill_common(q, k, v, q_tok_stride, k_tok_stride, v_tok_stride, cu_seqlens_q,
                          cu_seqlens_k, n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads,
                          head_dim, scale, causal, out, out_tok_stride, dtype, (hipStream_t)stream,
                          false);
  if (rc != AAC_OK) return rc;
  if (n_kv_tokens < 0 || num_cache_rows < 0) return AAC_ERR_INVALID_ARGUMENT;
  if (n_kv_tokens > 0 && (!k_cache || !v_cache || !slot_mapping)) return AAC_ERR_INVALID_ARGUMENT;
  // Causal self-attention (one cu_seqlens array for queries and keys) stores
  // inside the attention kernel; anything else stores first, then attends.
  if (causal && cu_seqlens_q == cu_seqlens_k && max_seqlen_q == max_seqlen_k && n_seqs > 0 &&
      max_seqlen_q > 0 && n_kv_tokens > 0 && n_kv_tokens < (int64_t(1) << 31) &&
      ((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0)
    return prefill_common(q, k, v, q_tok_stride, k_tok_stride, v_tok_stride, cu_seqlens_q,
                          cu_seqlens_k, n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads,
                          head_dim, scale, causal, out, out_tok_stride, dtype,
                          (hipStream_t)stream, true, k_cache, v_cache, num_cache_rows, slot_mapping,
                          (int32_t)n_kv_tokens);
  rc = aac_kv_store(k, v, k_tok_stride, v_tok_stride, k_cache, v_cache, num_cache_rows, slot_mapping,
                    n_kv_tokens, n_kv_heads, head_dim, dtype, stream);
  if (rc != AAC_OK) return rc;
  return prefill_common(q, k, v, q_tok_stride, k_tok_stride, v_tok_stride, cu_seqlens_q,
                        cu_seqlens_k, n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads,
                        head_dim, scale, causal, out, out_tok_stride, dtype, (hipStream_t)stream,
                        true);
}
