// Varlen causal GQA prefill, "wide" form (gfx950, bf16/fp16 MFMA): the same
// call as prefill.hip (flash_attn_varlen_func(q, k, v, cu, cu, max, max,
// causal), llm.py:178-184) for GQA groups of 2, 4 and 8.
//
// Why a second kernel.  With one 32-query column per wave (prefill.hip) every
// MFMA reads its K or V^T fragment from LDS for that column alone, and the
// softmax of a wave runs beside MFMAs only when the other wave of its SIMD
// happens to be in its MFMA phase.  Here a workgroup is four waves, one per
// SIMD, and each wave owns TWO columns: the same 32 queries for two query
// heads of one KV head.  Two consequences:
//   * every K / V fragment read from LDS feeds two MFMAs (one per column),
//     halving the LDS reads per MFMA;
//   * the two columns run half a sub-tile apart inside the wave's own
//     instruction stream (an in-wave ping-pong): while the MFMAs of column c
//     compute the next scores S_c(j+1) and the product O_c += V(j) P_c(j), the
//     VALU and transcendental units run the softmax of the other column on
//     scores already computed.  Neither half waits for the other, so the
//     MFMA pipe is fed from one wave without another wave's help.
// With 512 registers per lane at one wave per SIMD the O accumulators of both
// columns (128 registers) sit beside Q (64), the shared fragments (64) and the
// scores and probabilities of both columns.
//
// Sub-tile j = 32 keys; per j the wave runs two slots:
//   slot A(j): MFMA  S_0(j+1) = K(j+1) Q_0^T,  O_0 += V(j)^T P_0(j)
//              VALU  softmax of S_1(j) -> P_1(j)
//   slot B(j): MFMA  S_1(j+1) = K(j+1) Q_1^T,  O_1 += V(j)^T P_1(j)
//              VALU  softmax of S_0(j+1) -> P_0(j+1)
// The K(j+1) and V(j) fragments are read once, used in both slots, and each
// register is refilled for sub-tiles j+2 / j+1 right after its last use in
// slot B.  Row sums of the rounded probabilities come from a 16x16x32 MFMA
// with a constant selector operand (two per column and sub-tile) instead of
// VALU or v_dot2 work.
//
// Staging: K and V tiles (64 keys) go from global memory straight into LDS
// (buffer_load_dwordx4 ... lds: 1 KiB per wave instruction, no registers,
// no VALU), four stages deep.  K rows are stored with their 16-byte chunks
// XOR-swizzled by the row (chunk c of row r at c ^ (r & 15)), so the score
// MFMA's fragment reads (32 rows, one chunk) spread over all banks.  V rows
// are stored row-major (chunk c of row r at c ^ 4 (r & 3)) and read with the
// transposing LDS load ds_read_b64_tr_b16, which hands every lane four keys
// of one dimension -- exactly the V^T operand of the P*V MFMA -- so V needs
// no transpose on the way in.
//
// Everything else follows prefill.hip: scores transposed (S^T = K Q^T,
// v_mfma_f32_32x32x16) so a lane holds one query column, the probabilities
// already in the B-operand layout of O^T += V^T P^T, online softmax in the
// log2 domain with lazy rescaling, bottom-right causal alignment, buffer
// resources that zero-fill past the visible keys, and the persistent
// heavy-first zigzag grid.
//
// FLOPs per launch (the MFMA roofline): 4 * Hq * D * (visible query/key pairs).

#include <algorithm>

#include "prefill_common.h"
#include "prefill_wide.h"
#include "prefill_wide_asm.inc"

namespace aac {
namespace pw {

using pf::Args;
using pf::BKV;
using pf::D;
using pf::kRescale;

constexpr int kWaves = 4;  // one per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kRing = 4;                   // LDS stages
constexpr int kTileBytes = BKV * D * 2;    // 16 KiB: one K or V tile
constexpr int kStageBytes = 2 * kTileBytes;
constexpr int kLdsBytes = kRing * kStageBytes;  // 128 KiB
constexpr int kOutPitch = 136;             // output staging row pitch (bytes): 128 + 8
constexpr int kOutBytes = 32 * kOutPitch;  // one wave's staging rows (half a column)
constexpr int kLoadsPerTile = 8;           // direct loads per thread per tile (4 K + 4 V)

typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef short v4s __attribute__((ext_vector_type(4)));

// 16 bytes from global memory (buffer resource, 32-bit offsets) straight into
// LDS at m0 + 16 * lane.  The load is issued from inline assembly: the
// compiler then does not count it, so the waits for it are explicit (see the
// tile loop); m0 is set right before it and used by nothing else here.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, int voff, int soff, u32 lds_dst) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(r), "s"(soff), "s"(lds_dst)
               : "memory", "m0");
#pragma clang diagnostic pop
}

template <int G, bool CAUSAL, bool STORE, bool F16>
__global__ __launch_bounds__(kThreads, 1) void prefill_wide_kernel(Args a) {
  static_assert(G == 2 || G == 4 || G == 8, "two heads of one KV head per wave");
  static_assert(CAUSAL || !STORE, "the store variant is causal self-attention");
  constexpr int WP = G / 2;          // head pairs per workgroup
  constexpr int WQ = kWaves / WP;    // 32-query slots per workgroup
  constexpr int BQ = 32 * WQ;
  static_assert(!F16, "the item body is written for bf16");

  // LDS: kRing stages of [K tile | V tile], filled in stream order: the
  // tiles of consecutive items of this workgroup follow each other around the
  // ring (item tile T at stage (g0 + T) % kRing).
  __shared__ __attribute__((aligned(1024))) unsigned char lds[kLdsBytes + kWaves * kOutBytes];
  const u32 lds0 = (u32)(uintptr_t)(lds_u8*)lds;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wq = wave % WQ, wp = wave / WQ;  // query slot, head pair
  const int hl = lane >> 5;
  const int col = lane & 31;

  // ---- direct loads: instruction i of wave w fills LDS rows 16 i + 4 w +
  // lane/16 (1 KiB), lane%16 = the LDS chunk slot of its row, read from the
  // global chunk that the row's swizzle puts there.
  const int k_row_bytes = (int)(a.k_stride * 2), v_row_bytes = (int)(a.v_stride * 2);
  const int r4 = 4 * wave + (lane >> 4);
  const int ld_voff_k = r4 * k_row_bytes + 16 * ((lane & 15) ^ (r4 & 15));
  const int ld_voff_v = r4 * v_row_bytes + 16 * ((lane & 15) ^ (4 * (lane >> 4)));

  // ---- per-lane LDS read offsets (bytes within a stage's tile).
  // K (A operand of S^T = K Q^T): row col (+32 for the second sub-tile of a
  // tile), dims 16 t + 8 hl .. +7, i.e. logical chunk 2 t + hl.
  int koff[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) koff[t] = col * 256 + 16 * ((2 * t + hl) ^ (col & 15));
  // V (A operand of O^T = V^T P^T through ds_read_b64_tr_b16): in each
  // 16-lane group g, lane i supplies row 4 (g>>1) + (i>>2) (keys; +8 for the
  // second read of a fragment, +16 per 16-key step), dims 32 db + 16 (g&1) +
  // 4 (i&3) .. +3; the read then gives lane j of the group the four keys
  // 4 (g>>1) + 0..3 of dim 32 db + 16 (g&1) + j -- the B-operand key order of
  // the probabilities (keys 4 hl + 0..3, then 8 + 4 hl + 0..3).
  int voff[4];
  {
    const int g = lane >> 4, i = lane & 15;
    const int l0 = (4 * (g >> 1) + (i >> 2)) * 256 + 32 * (g & 1) + 8 * (i & 3);
#pragma unroll
    for (int db = 0; db < 4; ++db) voff[db] = l0 + 64 * (db ^ (i >> 2));
  }
  // selector of the row-sum MFMA (16x16x32, A = selector, B = probabilities
  // of one 16-key step): A[0][k] = 1 for k in [0,8) u [16,24) (the
  // probabilities of queries 0-15), A[1][k] = 1 for k in [8,16) u [24,32)
  // (queries 16-31); lane l holds A[l%16][8 (l/16) ..+7]
  u32x4 sel;
  {
    const bool one = lane == 0 || lane == 32 || lane == 17 || lane == 49;
#pragma unroll
    for (int i = 0; i < 4; ++i) sel[i] = one ? 0x3f803f80u : 0u;  // bf16 ones
  }

  // ---- work items (q-block rank z, segment s, KV head h), rank-major inside
  // each chunk of segments (below) so a chunk's heaviest causal q-blocks come
  // first.  Persistent grid: workgroup w of P takes item k P + w in even
  // rounds and, in odd rounds, the mirror image taken in groups of eight
  // (item (k+1) P - 8 - 8 (w/8) + w%8 when P is a multiple of 8): heavy items
  // pair with light ones, and item i mod 8 stays equal to w mod 8, so with
  // eight KV heads each head's K/V rows are read by one XCD's workgroups
  // (workgroups are dealt to the 8 XCDs round-robin).
  struct Item {
    int h, s, qb, q_beg, Lq, k_beg, Lk;
  };
  const int n_hs = a.hkv * a.n_seqs;
  const int n_items = n_hs * a.n_qblocks;
  const int P = gridDim.x, w = blockIdx.x;
  auto item_index = [&](int k) {
    if (!(k & 1)) return k * P + w;
    return (P & 7) == 0 ? (k + 1) * P - 8 - (w & ~7) + (w & 7) : (k + 1) * P - 1 - w;
  };
  // Items are numbered chunk by chunk: a chunk is chunk_segs consecutive
  // segments (the last may be shorter), numbered rank-major inside (rank z,
  // segment, KV head).  A chunk's K/V rows per head are sized to about half
  // an XCD's L2, so the workgroups of one XCD (one KV head with eight KV
  // heads) stream a few segments at a time and re-read their tiles from L2.
  const int per_chunk = a.chunk_segs * a.n_qblocks * a.hkv;  // items in a full chunk
  struct Place {
    int z, s, h;
  };
  auto place_of = [&](int i) {
    const int c = i / per_chunk;
    const int r = i - c * per_chunk;
    const int cs = min(a.chunk_segs, a.n_seqs - c * a.chunk_segs);  // segments in chunk c
    const int z = r / (cs * a.hkv);
    const int rem = r - z * cs * a.hkv;
    const int sl = rem / a.hkv;
    return Place{z, c * a.chunk_segs + sl, rem - sl * a.hkv};
  };
  auto kv_end_of = [&](const Item& it) {
    const int wg_qmax = min(it.qb * BQ + BQ, it.Lq) - 1;
    return CAUSAL ? max(0, min(it.Lk, wg_qmax + 1 + it.Lk - it.Lq)) : it.Lk;
  };
  auto decode = [&](const Place& pl, int q0, int q1, int k0, int k1, Item& it) -> bool {
    const int z = pl.z;
    it.s = pl.s;
    it.h = pl.h;
    it.q_beg = q0;
    it.Lq = q1 - q0;
    it.k_beg = k0;
    it.Lk = min(k1 - k0, a.max_k);
    const int nqb = (it.Lq + BQ - 1) / BQ;
    it.qb = CAUSAL ? nqb - 1 - z : z;
    return z < nqb;
  };
  // segment bounds through scalar loads (the arrays are read-only here), so
  // no vector-memory wait between items covers the body's loads in flight
  typedef const int32_t __attribute__((address_space(4))) cint;
  const cint* cuq = (const cint*)(uintptr_t)a.cu_q;
  const cint* cuk = (const cint*)(uintptr_t)a.cu_k;
  auto next_item = [&](int& k, Item& it) -> bool {
    for (; k * P < n_items; ++k) {
      const int i = item_index(k);
      if (i >= n_items) continue;
      const Place pl = place_of(i);
      const int sg = pl.s;
      if (decode(pl, cuq[sg], cuq[sg + 1], cuk[sg], cuk[sg + 1], it)) return true;
    }
    return false;
  };
  auto rsrc_of = [&](const u16* base, int row_bytes, int kv_end) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<u16*>(base), 0,
                                             kv_end > 0 ? (kv_end - 1) * row_bytes + D * 2 : 0,
                                             0x00020000);
  };

  // Q fragments of both columns (B operand of S^T = K Q^T; lane = query):
  // this lane's address; the item body loads the next item's Q into qf at its
  // end, the first item's come from load_q.  The loads are issued from inline
  // assembly: the compiler does not track them and inserts no wait for them.
  u32x4 qf[2][8];
  auto q_addr = [&](const Item& it) {
    const int qi = it.qb * BQ + wq * 32 + col;
    const int qrow = it.q_beg + min(qi, max(it.Lq - 1, 0));
    return a.q + (int64_t)qrow * a.q_stride + (it.h * G + 2 * wp) * D + hl * 8;
  };
  auto load_q = [&](const Item& it) {
    const u16* qp = q_addr(it);
    asm volatile(
        "global_load_dwordx4 %0, %16, off\n\tglobal_load_dwordx4 %1, %16, off offset:32\n\t"
        "global_load_dwordx4 %2, %16, off offset:64\n\tglobal_load_dwordx4 %3, %16, off offset:96\n\t"
        "global_load_dwordx4 %4, %16, off offset:128\n\tglobal_load_dwordx4 %5, %16, off offset:160\n\t"
        "global_load_dwordx4 %6, %16, off offset:192\n\tglobal_load_dwordx4 %7, %16, off offset:224\n\t"
        "global_load_dwordx4 %8, %16, off offset:256\n\tglobal_load_dwordx4 %9, %16, off offset:288\n\t"
        "global_load_dwordx4 %10, %16, off offset:320\n\tglobal_load_dwordx4 %11, %16, off offset:352\n\t"
        "global_load_dwordx4 %12, %16, off offset:384\n\tglobal_load_dwordx4 %13, %16, off offset:416\n\t"
        "global_load_dwordx4 %14, %16, off offset:448\n\tglobal_load_dwordx4 %15, %16, off offset:480"
        : "=&v"(qf[0][0]), "=&v"(qf[0][1]), "=&v"(qf[0][2]), "=&v"(qf[0][3]), "=&v"(qf[0][4]),
          "=&v"(qf[0][5]), "=&v"(qf[0][6]), "=&v"(qf[0][7]), "=&v"(qf[1][0]), "=&v"(qf[1][1]),
          "=&v"(qf[1][2]), "=&v"(qf[1][3]), "=&v"(qf[1][4]), "=&v"(qf[1][5]), "=&v"(qf[1][6]),
          "=&v"(qf[1][7])
        : "v"(qp)
        : "memory");
  };

  // ---- the KV-cache store (STORE).  Each item stores the K/V rows of its own
  // q-block (its queries' rows taken as keys, since cu_q == cu_k) for its KV
  // head: the item body loads them from L2 (the tiles staged them moments
  // before) right after its tile loop and writes them to the caches after the
  // output, each wave its share of 64 / G rows.  The item of rank 0 of a
  // segment also stores the q-blocks no item owns (a max_seqlen_q below the
  // segment's length), and workgroup 0 the tokens before cu[0] and from cu[n]
  // on.  Every token's rows are thus written at least once; a row written
  // twice gets the same bytes both times.
  constexpr int kShare = 64 / G;               // own rows per wave
  const int share0 = wq * 32 + wp * kShare;    // the wave's first own row in a q-block
  auto store_unowned = [&](const Item& it) {
    const int nqb = (it.Lq + BQ - 1) / BQ;
    if (nqb - 1 - it.qb == 0 && nqb > a.n_qblocks) {  // rank 0 (causal numbering)
      const int lo = nqb - a.n_qblocks;               // q-blocks [lo, nqb) have items
      pf::store_kv_span<kThreads>(a, tid, it.k_beg, it.k_beg + (int64_t)lo * BQ, it.h, it.h + 1);
      // the next item body's first wait counts only its predecessor's stores
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  };
  // workgroup 0: tokens outside [cu[0], cu[n])
  auto store_edges = [&]() {
    if (STORE && blockIdx.x == 0) {
      pf::store_kv_span<kThreads>(a, tid, 0, a.cu_q[0], 0, a.hkv);
      pf::store_kv_span<kThreads>(a, tid, a.cu_q[a.n_seqs], pf::kernel_args()->n_tok, 0, a.hkv);
    }
  };

  int k = 0;
  Item cur;
  if (!next_item(k, cur)) {
    store_edges();
    return;
  }
  int kv_end = kv_end_of(cur);

  const float cs = a.scale_log2;
  const float ncs = -cs;
  const float kthr = kRescale / cs;
  // per-lane constants of the item body: 4 hl (key offset of the lane half),
  // bpermute addresses of lanes (lane & 15) and (lane & 15) + 16, the lane's
  // bit 4, and the byte offset of this lane's output (row col, dims 4 hl ..)
  const int hl4 = 4 * hl;
  const int bpa = (lane & 15) * 4, bpahi = ((lane & 15) + 16) * 4, hi16 = lane & 16;
  // output: staging write / read addresses of this lane (wave's rows beside
  // the ring), the global byte offset of its read-back row (8 rows of 128
  // bytes per store) and the offset of eight rows
  const int ostep = (int)(a.o_stride * 2);
  const u32 stg = lds0 + (u32)(kLdsBytes + wave * kOutBytes);
  const int stw = (int)stg + col * kOutPitch + 8 * hl;
  const int str = (int)stg + (lane >> 3) * kOutPitch + 16 * (lane & 7);
  const int osv = (lane >> 3) * ostep + 16 * (lane & 7);
  const int ost8 = 8 * ostep;
  // KV-cache store: lane's row within a group of 4 and byte chunk within a
  // row, slot offset of that row, cache head-row stride and the caches' byte
  // range from the head's first row (the host keeps it below 4 GiB)
  const int lrow = lane >> 4, chunk16 = 16 * (lane & 15), slv = 8 * lrow;
  const int rvk = lrow * k_row_bytes + chunk16, rvv = lrow * v_row_bytes + chunk16;
  int cstride = 0, crng = 0, nrows = 0;
  if constexpr (STORE) {
    pf::KArgs* sa = pf::kernel_args();
    cstride = a.hkv * D * 2;
    nrows = (int)sa->num_rows;
    // from a head's base: rows 0..num_rows-1 (a slot past them is refused per row)
    crng = sa->num_rows > 0 ? (int)((sa->num_rows - 1) * cstride + D * 2) : 0;
  }
  const u32 ldsw = lds0 + (u32)(wave * 1024);
  const int ks16 = 16 * k_row_bytes, vs16 = 16 * v_row_bytes;
  const int ks64 = 64 * k_row_bytes, vs64 = 64 * v_row_bytes;

  // First item: Q and tiles 0-2 (stream positions 0-2, stages 0-2; past its
  // last tile the resource range check reads zeros).  Every later item finds
  // its Q and first tiles loaded by the body of the item before it.
  {
    const __amdgpu_buffer_rsrc_t rsk =
        rsrc_of(a.k + (int64_t)cur.k_beg * a.k_stride + cur.h * D, k_row_bytes, kv_end);
    const __amdgpu_buffer_rsrc_t rsv =
        rsrc_of(a.v + (int64_t)cur.k_beg * a.v_stride + cur.h * D, v_row_bytes, kv_end);
    load_q(cur);
    for (int T = 0; T < 3; ++T) {
      const u32 st = lds0 + (u32)(T * kStageBytes) + (u32)(wave * 1024);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        load_lds16(rsk, ld_voff_k, T * ks64 + i * ks16, st + i * 4096);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        load_lds16(rsv, ld_voff_v, T * vs64 + i * vs16, st + kTileBytes + i * 4096);
    }
    // The body reads tiles 0 and 1 before its first barrier; tile 2 (the
    // youngest 8 loads) is waited for at the start of its second tile
    // iteration.  An item of fewer than three tiles has no such iteration
    // and refills tile 2's stage in its epilogue, so it waits for all.
    if (kv_end > 2 * BKV)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  int g0 = 0;  // ring stage of the current item's tile 0

  for (;;) {
    Item nxt;
    int kn = k + 1;
    const bool more = next_item(kn, nxt);
    const int kv_end_n = more ? kv_end_of(nxt) : 0;

    const int qi = cur.qb * BQ + wq * 32 + col;
    const int shift = cur.Lk - cur.Lq;
    const int w_qmin = cur.qb * BQ + wq * 32;
    const int w_qmax = min(w_qmin + 31, cur.Lq - 1);
    const int w_end = w_qmin >= cur.Lq ? 0 : (CAUSAL ? max(0, min(cur.Lk, w_qmax + 1 + shift)) : cur.Lk);
    // keys < w_full need no mask (at most w_end: a wave without queries has none)
    const int w_full = min(w_end, CAUSAL ? max(0, min(cur.Lk, w_qmin + 1 + shift)) : cur.Lk);
    const int my_lim = CAUSAL ? min(cur.Lk, qi + 1 + shift) : cur.Lk;
    const int nt = (kv_end + BKV - 1) / BKV;  // LDS tiles (workgroup-uniform)
    const int nsub = (w_end + 31) / 32;       // 32-key sub-tiles of this wave
    // buffer ranges: this item's and the next item's K/V rows, this wave's
    // output rows (none past the segment)
    auto range = [&](int n, int row_bytes) {
      return __builtin_amdgcn_readfirstlane(n > 0 ? (n - 1) * row_bytes + D * 2 : 0);
    };
    const u16* kb = a.k + (int64_t)cur.k_beg * a.k_stride + cur.h * D;
    const u16* vb = a.v + (int64_t)cur.k_beg * a.v_stride + cur.h * D;
    const u16* knb = more ? a.k + (int64_t)nxt.k_beg * a.k_stride + nxt.h * D : a.k;
    const u16* vnb = more ? a.v + (int64_t)nxt.k_beg * a.v_stride + nxt.h * D : a.v;
    const int kr = range(kv_end, k_row_bytes), vr = range(kv_end, v_row_bytes);
    const int knr = range(kv_end_n, k_row_bytes), vnr = range(kv_end_n, v_row_bytes);
    const int row0 = cur.qb * BQ + wq * 32;
    const int orng = __builtin_amdgcn_readfirstlane(max(0, min(32, cur.Lq - row0)) * ostep);
    const u16* ob = a.out + (int64_t)(cur.q_beg + row0) * a.o_stride + (cur.h * G + 2 * wp) * D;
    const u16* qn = q_addr(more ? nxt : cur);  // the last item reloads its own Q (unused)
    // KV-cache store of the wave's own rows (STORE; inert operands otherwise)
    int nvalid = 0, srng = 0, okr = 0, ovr = 0;
    const int64_t* sb = a.slots;
    const u16 *kcb = a.k, *vcb = a.v, *okb = a.k, *ovb = a.v;
    if constexpr (STORE) {
      pf::KArgs* sa = pf::kernel_args();
      const int r0 = cur.qb * BQ + share0;              // first own row (in the segment)
      const int64_t t0 = (int64_t)cur.k_beg + r0;       // its token
      const int64_t tok_left = max((int64_t)0, (int64_t)sa->n_tok - t0);
      nvalid = __builtin_amdgcn_readfirstlane((int)min((int64_t)max(0, min(kShare, cur.Lq - r0)), tok_left));
      srng = __builtin_amdgcn_readfirstlane((int)min(tok_left, (int64_t)32) * 8);
      sb = sa->slots + t0;
      kcb = sa->kc + cur.h * D;
      vcb = sa->vc + cur.h * D;
      okb = a.k + t0 * a.k_stride + cur.h * D;
      ovb = a.v + t0 * a.v_stride + cur.h * D;
      okr = range(nvalid, k_row_bytes);
      ovr = range(nvalid, v_row_bytes);
    }

    // The item: O = softmax(Q K^T) V for both columns, normalised and stored;
    // the next item's Q and first tiles loaded (see gen_prefill_wide_asm.py).
    {
      int r_t, r_j, r0, r1, r2, r3, r5, r6, r_dm, r_dk, r_dv, r_qd;
      unsigned long long r_ret;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile(AAC_PW_ITEM_ASM
                   : [t] "=&s"(r_t), [j] "=&s"(r_j), [s0] "=&s"(r0), [s1] "=&s"(r1), [s2] "=&s"(r2),
                     [s3] "=&s"(r3), [s5] "=&s"(r5), [s6] "=&s"(r6), [dm] "=&s"(r_dm), [dk] "=&s"(r_dk),
                     [dv] "=&s"(r_dv), [qd] "=&s"(r_qd), [ret] "=&s"(r_ret),
                     [q00] "+v"(qf[0][0]), [q01] "+v"(qf[0][1]), [q02] "+v"(qf[0][2]), [q03] "+v"(qf[0][3]),
                     [q04] "+v"(qf[0][4]), [q05] "+v"(qf[0][5]), [q06] "+v"(qf[0][6]), [q07] "+v"(qf[0][7]),
                     [q10] "+v"(qf[1][0]), [q11] "+v"(qf[1][1]), [q12] "+v"(qf[1][2]), [q13] "+v"(qf[1][3]),
                     [q14] "+v"(qf[1][4]), [q15] "+v"(qf[1][5]), [q16] "+v"(qf[1][6]), [q17] "+v"(qf[1][7])
                   : [ko0] "v"(koff[0]), [ko1] "v"(koff[1]), [ko2] "v"(koff[2]), [ko3] "v"(koff[3]),
                     [ko4] "v"(koff[4]), [ko5] "v"(koff[5]), [ko6] "v"(koff[6]), [ko7] "v"(koff[7]),
                     [vo0] "v"(voff[0]), [vo1] "v"(voff[1]), [vo2] "v"(voff[2]), [vo3] "v"(voff[3]),
                     [sel] "v"(sel), [cs] "s"(cs), [ncs] "s"(ncs), [kthr] "s"(kthr), [mylim] "v"(my_lim),
                     [hl4] "v"(hl4), [bpa] "v"(bpa), [bpahi] "v"(bpahi), [hi16] "v"(hi16),
                     [lds0] "s"(lds0), [ldsw] "s"(ldsw), [ldk] "v"(ld_voff_k), [ldv] "v"(ld_voff_v),
                     [ks16] "s"(ks16), [vs16] "s"(vs16), [ks64] "s"(ks64), [vs64] "s"(vs64),
                     [nsub] "s"(nsub), [wfull] "s"(w_full), [nt] "s"(nt), [g0] "s"(g0),
                     [kb] "s"(kb), [kr] "s"(kr), [vb] "s"(vb), [vr] "s"(vr),
                     [knb] "s"(knb), [knr] "s"(knr), [vnb] "s"(vnb), [vnr] "s"(vnr),
                     [ob] "s"(ob), [orng] "s"(orng), [stw] "v"(stw), [str] "v"(str), [osv] "v"(osv),
                     [ost8] "s"(ost8), [qn] "v"(qn), [dostore] "s"((int)STORE), [sb] "s"(sb), [okb] "s"(okb), [okr] "s"(okr), [ovb] "s"(ovb), [ovr] "s"(ovr),
                     [srng] "s"(srng), [kcb] "s"(kcb), [vcb] "s"(vcb), [crng] "s"(crng),
                     [cstride] "s"(cstride), [nrows] "s"(nrows), [nvalid] "s"(nvalid), [rvk] "v"(rvk),
                     [rvv] "v"(rvv), [slv] "v"(slv), [lrow] "v"(lrow), [chunk16] "v"(chunk16)
                   : AAC_PW_CLOBBERS);
#pragma clang diagnostic pop
    }
    if constexpr (STORE) store_unowned(cur);
    if (!more) break;
    g0 = (g0 + nt) & 3;
    cur = nxt;
    k = kn;
    kv_end = kv_end_n;
  }
  // no load may still be writing LDS or registers when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  store_edges();
}

template <int G, bool CAUSAL, bool STORE, bool F16>
static void launch_t(const Args& a0, int max_q, int n_cu, hipStream_t st) {
  Args a = a0;
  constexpr int BQ = 32 * (kWaves / (G / 2));
  a.n_qblocks = (int)cdiv(max_q, BQ);
  // segments per item chunk: K/V rows of a chunk's segments for one head
  // about 2 MiB (half an XCD's L2), at least one segment
  const int64_t kv_head_bytes = (int64_t)std::max(a.max_k, 1) * D * 2 * 2;
  a.chunk_segs = (int)std::max<int64_t>(1, std::min<int64_t>(a.n_seqs, (int64_t(2) << 20) / kv_head_bytes));
  const int64_t n_items = (int64_t)a.hkv * a.n_seqs * a.n_qblocks;
  const int grid = (int)std::min<int64_t>(n_items, n_cu);
  hipLaunchKernelGGL((prefill_wide_kernel<G, CAUSAL, STORE, F16>), dim3(grid), dim3(kThreads), 0, st, a);
}

template <bool CAUSAL, bool STORE, bool F16>
static int launch_g(const Args& a, int g, int max_q, int n_cu, hipStream_t st) {
  switch (g) {
    case 2: launch_t<2, CAUSAL, STORE, F16>(a, max_q, n_cu, st); break;
    case 4: launch_t<4, CAUSAL, STORE, F16>(a, max_q, n_cu, st); break;
    case 8: launch_t<8, CAUSAL, STORE, F16>(a, max_q, n_cu, st); break;
    default: return AAC_ERR_UNSUPPORTED;
  }
  return AAC_OK;
}

}  // namespace pw

bool prefill_wide_supports(int g, float scale, bool f16) {
  return (g == 2 || g == 4 || g == 8) && scale > 0.f && !f16;
}

int prefill_wide_launch(const pf::Args& a, int g, bool causal, bool store, int max_q, int n_cu,
                        hipStream_t st) {
  if (store)  // causal self-attention with the KV-cache store
    return causal ? pw::launch_g<true, true, false>(a, g, max_q, n_cu, st) : AAC_ERR_UNSUPPORTED;
  return causal ? pw::launch_g<true, false, false>(a, g, max_q, n_cu, st)
                : pw::launch_g<false, false, false>(a, g, max_q, n_cu, st);
}

}  // namespace aac
