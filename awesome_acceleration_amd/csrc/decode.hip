// Paged decode attention (gfx950): one query token per sequence against a
// paged KV cache -- the attend half of the reference's
// flash_attn_with_kvcache call (model/model.py:233-240).
//
// Work decomposition
//   grid = (kv_head, partition, sequence), 256 threads (4 wavefronts); the KV
//   heads of one token range are adjacent in dispatch order, so the 256-byte
//   head slices of each 2 KiB cache row are fetched at about the same time.
//   A workgroup owns one KV head of one sequence over a partition of
//   `part_tokens` consecutive context tokens and serves all G = Hq/Hkv query
//   heads that share that KV head, so each K/V byte is read from HBM once.
//   Without a split (up to 1024 sequences), blockIdx.z is a rank in
//   descending context-length order, which every workgroup maps to its
//   sequence: the dispatcher, which hands out workgroups in index order as
//   slots free up, then starts long sequences first and fills the end of the
//   launch with short ones instead of leaving a few long ones running alone
//   (256 sequences of 1024..2047 tokens: 264 -> 254 us).
//   Inside the workgroup every 16-lane DPP row owns one token row at a time:
//   lane li holds head dims [8*li, 8*li+8) and loads them with one 16-byte
//   global load (two for fp32), so a wavefront reads 4 token rows (4 x 256 B
//   in bf16) per load instruction and U=8 rows per DPP row (4 for G=8) are in
//   flight before the first use: the block-table entries of an iteration are
//   loaded one iteration ahead and all K/V loads are issued before any math
//   (with in-order load counters, a block-table load waited for in between
//   would also wait for every earlier K/V load).  The 16 rows of a workgroup
//   walk the partition in lock step (row slot r takes tokens t0 + r,
//   t0 + r + 16, ...); slots past the partition end re-read token t0's row
//   (finite, probability 0) so the loads never branch.  K/V are read with
//   non-temporal loads: each byte is used once per step, so it should not
//   displace anything from L2/MALL (measured +10% bandwidth).  Power-of-two
//   block sizes use shift/mask for the block-table lookup.
//
// Softmax
//   Each DPP row keeps its own online-softmax state (running max m, running
//   sum l, fp32 accumulator for its 8 dims x G heads; Milakov & Gimelshein
//   2018), in the log2 domain (exponentiated with v_exp_f32).  bf16/fp16: q.k
//   is v_dot2 on the packed rows, the probabilities are rounded to the input
//   type and P.V is v_dot2 over V words paired across two tokens (v_perm);
//   fp32: unpacked fp32 FMAs with q pre-scaled.  The 16 row states of a workgroup are
//   merged at the end (cross-row shuffles inside a wave, LDS across waves).
//   A sequence whose context spans one partition writes the final output
//   directly; longer contexts write a normalised partial output and its
//   log-sum-exp to the workspace, and a second kernel combines the
//   partitions (the FlashDecoding split-K method).
//
// Bytes per launch (the HBM roofline): every context token's K and V row of
// each KV head is read exactly once, 2 * Hkv * D * elem_bytes per token, plus
// q and out; the reduction adds 2 * B * Hq * P * (D + 1) * 4 bytes when split.

#include <algorithm>
#include <climits>
#include <mutex>

#include "aac_common.h"

namespace aac {

constexpr int kHeadDim = 128;
constexpr int kRowLanes = 16;  // lanes per token row: 128 dims / 8 per lane

struct DecodeArgs {
  const void* q;
  int64_t q_seq_stride;  // elements
  const void* k_cache;
  const void* v_cache;
  int64_t num_blocks;
  int32_t block_size;
  const int32_t* block_tables;
  int32_t max_blocks;
  const int32_t* lens;  // context length of sequence b = lens[b] + lens_add
  int32_t lens_add;
  int32_t n_seqs;
  int32_t hq;
  int32_t hkv;
  float scale_log2;  // softmax scale * log2(e)
  void* out;
  int64_t out_seq_stride;  // elements
  float* ws_o;             // [B][Hq][P][D] normalised partial outputs
  float* ws_lse;           // [B][Hq][P]    log2-sum-exp of each partition
  int32_t n_parts;
  int32_t part_tokens;
  int32_t bs_shift;  // log2(block_size) when it is a power of two
  // otherwise t / block_size = (t * bs_magic) >> bs_mshift for 0 <= t < 2^31
  // (Granlund & Montgomery 1994, Thm 4.2: bs_magic = floor(2^(31+l) / d) + 1
  // with l = ceil(log2 d), bs_mshift = 31 + l)
  uint64_t bs_magic;
  int32_t bs_mshift;
  int32_t lpt;       // 1: blockIdx.z is a rank in descending context order
  int32_t lpt_max;   // context bound the length classes are scaled to
};

// Raw storage for the 8 elements one lane owns in one token row.
template <Dt DT> struct Raw8 {
  static constexpr int kWords = Elem<DT>::kBytes * 8 / 16;  // u32x4 words
  u32x4 w[kWords];
  __device__ inline void load(const char* p) {
#pragma unroll
    for (int i = 0; i < kWords; ++i)
      w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 16 * i));
  }
  __device__ inline void zero() {
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = u32x4{0, 0, 0, 0};
  }
  __device__ inline void unpack(float* f) const {
    if constexpr (DT == Dt::FP32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[i] = __uint_as_float(w[0][i]);
        f[4 + i] = __uint_as_float(w[1][i]);
      }
    } else {
      Elem<DT>::unpack8(w[0], f);
    }
  }
};

__device__ __forceinline__ int context_len(const DecodeArgs& a, int b) {
  int ctx = a.lens[b] + a.lens_add;
  const int cap = a.max_blocks * a.block_size;
  ctx = ctx < 0 ? 0 : ctx;
  return ctx > cap ? cap : ctx;
}

__device__ __forceinline__ int parts_of(const DecodeArgs& a, int ctx) {
  int n = (int)cdiv(ctx, a.part_tokens);
  return n > a.n_parts ? a.n_parts : n;
}

// Sequence of rank `rank` in descending context-length order, by length
// class: class c = ctx * 64 / (lpt_max + 1) (64 classes, longest first),
// index order inside a class.  Counts, prefix sums and ballots do not depend
// on timing, so every workgroup derives the same bijection rank -> sequence:
//   1. histogram of the classes (LDS atomics; the counts are exact),
//   2. one wavefront scans the 64 counts and finds the class and position of
//      `rank`,
//   3. per 64-sequence chunk a ballot of "in that class" and its popcounts
//      give each sequence its position inside the class.
constexpr int kLptMaxSeqs = 1024;
constexpr int kLptClasses = 64;
__device__ __forceinline__ int seq_of_rank(const DecodeArgs& a, int rank, int tid) {
  __shared__ int s_cnt[kLptClasses];
  __shared__ int s_wcnt[kLptMaxSeqs / 64];
  __shared__ int s_sel[2];
  __shared__ int s_pick;
  const int n = a.n_seqs, lane = tid & 63, wave = tid >> 6;
  if (tid < kLptClasses) s_cnt[tid] = 0;
  __syncthreads();
  int cls[kLptMaxSeqs / 256];  // descending class index of sequences tid + 256k (-1: none)
#pragma unroll
  for (int k = 0; k < kLptMaxSeqs / 256; ++k) {
    const int i = tid + 256 * k;
    cls[k] = -1;
    if (i < n) {
      const int64_t c = (int64_t)context_len(a, i) * kLptClasses / ((int64_t)a.lpt_max + 1);
      cls[k] = kLptClasses - 1 - (int)(c < kLptClasses - 1 ? c : kLptClasses - 1);
      atomicAdd(&s_cnt[cls[k]], 1);
    }
  }
  __syncthreads();
  if (wave == 0) {
    const int v = s_cnt[lane];
    int incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    if (rank >= incl - v && rank < incl) {
      s_sel[0] = lane;
      s_sel[1] = rank - (incl - v);
    }
  }
  __syncthreads();
  const int csel = s_sel[0], psel = s_sel[1];
  unsigned long long bal[kLptMaxSeqs / 256];
#pragma unroll
  for (int k = 0; k < kLptMaxSeqs / 256; ++k) {
    bal[k] = __ballot(cls[k] == csel);
    if (lane == 0) s_wcnt[4 * k + wave] = __popcll(bal[k]);
  }
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int k = 0; k < kLptMaxSeqs / 256; ++k) {
    const int chunk = 4 * k + wave;  // 64-sequence chunks in index order
    int before = base;
    for (int m = 4 * k; m < chunk; ++m) before += s_wcnt[m];
    const int pos = before + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal[k] >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((unsigned)bal[k], 0u));
    if (cls[k] == csel && pos == psel) s_pick = tid + 256 * k;
    for (int m = 4 * k; m < 4 * k + 4; ++m) base += s_wcnt[m];
  }
  __syncthreads();
  return s_pick;
}

template <Dt DT>
__device__ __forceinline__ void store_out2(void* out, int64_t idx, float x0, float x1) {
  if constexpr (DT == Dt::FP32) {
    *reinterpret_cast<float2*>(reinterpret_cast<float*>(out) + idx) = make_float2(x0, x1);
  } else {
    *reinterpret_cast<u32*>(reinterpret_cast<u16*>(out) + idx) = Elem<DT>::pack2(x0, x1);
  }
}

template <Dt DT, int G, int U, bool POW2>
// Occupancy: with G <= 2 the kernel fits 128 VGPRs, i.e. four workgroups per
// CU (16 wavefronts); larger groups hold more accumulators.
__global__ __launch_bounds__(256, G <= 2 ? 4 : 2) void decode_paged_kernel(DecodeArgs a) {
  constexpr int ES = Elem<DT>::kBytes;
  // The KV heads of one token range are dispatched together.  Workgroups go
  // to the 8 XCDs round-robin, so with an even head count workgroup x runs
  // on an XCD of x's parity; it attends head x ^ 1, on the XCD of the other
  // parity: measured on MI355X over all eight rotations of heads to XCDs,
  // the odd ones (256 seqs x 1-2k, 16/8 heads: 246.4-247.0 us) beat the even
  // ones (253.2-253.3 us), and likewise at 8/4 heads (129.4-129.7 against
  // 132.8-133.0 us).
  const int h = (a.hkv & 1) ? (int)blockIdx.x : (int)(blockIdx.x ^ 1u);
  const int part = blockIdx.y;
  const int tid = threadIdx.x;
  // Longest contexts first: the dispatcher hands out workgroups in index
  // order as slots free up, so the short sequences fill the tail instead of
  // a few long ones running alone at the end.
  const int b = a.lpt ? __builtin_amdgcn_readfirstlane(seq_of_rank(a, blockIdx.z, tid))
                     : (int)blockIdx.z;  // wave-uniform (SGPR) either way
  const int ctx = context_len(a, b);
  const int np = parts_of(a, ctx);

  if (part >= np) {
    if (part == 0) {  // empty context: zeros (FA2 convention)
      for (int i = tid; i < G * (kHeadDim / 2); i += 256) {
        const int g = i / (kHeadDim / 2), d2 = (i % (kHeadDim / 2)) * 2;
        store_out2<DT>(a.out, (int64_t)b * a.out_seq_stride + (int64_t)(h * G + g) * kHeadDim + d2,
                       0.f, 0.f);
      }
    }
    return;
  }
  const int t0 = part * a.part_tokens;
  const int t1 = (part == np - 1) ? ctx : t0 + a.part_tokens;

  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, grp = lane >> 4;
  const int rslot = wave * 4 + grp;  // 0..15

  // q for the G heads of this KV head.  fp32: unpacked and pre-scaled into
  // the log2 domain.  bf16/fp16 (PK): kept packed and exact for v_dot2; the
  // scale is applied to the scores instead.
  constexpr bool PK = DT != Dt::FP32;
  float qf[PK ? 1 : G][8];
  u32 qp[PK ? G : 1][4];
  {
    const char* qb = reinterpret_cast<const char*>(a.q) +
                     ((int64_t)b * a.q_seq_stride + (int64_t)h * G * kHeadDim + li * 8) * ES;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      Raw8<DT> r;
      r.load(qb + (int64_t)g * kHeadDim * ES);
      if constexpr (PK) {
#pragma unroll
        for (int w = 0; w < 4; ++w) qp[g][w] = r.w[0][w];
      } else {
        r.unpack(qf[g]);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[g][i] *= a.scale_log2;
      }
    }
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -1e30f;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }

  const int64_t tok_bytes = (int64_t)a.hkv * kHeadDim * ES;  // cache row stride
  const char* kbase = reinterpret_cast<const char*>(a.k_cache) + ((int64_t)h * kHeadDim + li * 8) * ES;
  const char* vbase = reinterpret_cast<const char*>(a.v_cache) + ((int64_t)h * kHeadDim + li * 8) * ES;
  const int32_t* bt = a.block_tables + (int64_t)b * a.max_blocks;
  const uint32_t nb32 = a.num_blocks < 0x7fffffff ? (uint32_t)a.num_blocks : 0x7fffffffu;

  // Token t of this partition, or t0 (a valid token whose row is finite and
  // whose probability is set to 0) past its end, so loads never branch.
  auto token = [&](int t) { return t < t1 ? t : t0; };
  auto block_index = [&](int t) {
    return POW2 ? t >> a.bs_shift : (int)(((uint64_t)(uint32_t)t * a.bs_magic) >> a.bs_mshift);
  };
  // The block numbers of an iteration's U tokens are loaded one iteration
  // ahead: a block-table load waited for right before the K/V loads would,
  // with in-order load counters, also wait for every K/V load issued before
  // it and leave one token per wave in flight.
  int blk[U];
#pragma unroll
  for (int u = 0; u < U; ++u) blk[u] = bt[block_index(token(t0 + rslot + 16 * u))];

  for (int tb = t0 + rslot; tb < t1; tb += 16 * U) {
    Raw8<DT> kr[U], vr[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      valid[u] = tb + 16 * u < t1;
      const int t = token(tb + 16 * u);
      const int bi = block_index(t);
      const int off = POW2 ? t & (a.block_size - 1) : t - bi * a.block_size;
      const uint32_t bk = (uint32_t)blk[u] < nb32 ? (uint32_t)blk[u] : 0u;  // bad entries read block 0
      const int64_t row = (int64_t)bk * a.block_size + off;
      kr[u].load(kbase + row * tok_bytes);
      vr[u].load(vbase + row * tok_bytes);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) blk[u] = bt[block_index(token(tb + 16 * U + 16 * u))];
    // Every load above is issued before any arithmetic below (the scheduler
    // would otherwise pull each token's math up behind its load and wait).
    __builtin_amdgcn_sched_barrier(0);
    float s[U][G];
    if constexpr (PK) {
      // Packed bf16/fp16: q.k with v_dot2 on the packed rows (no unpacking),
      // raw scores; the probabilities are rounded to the input type (as the
      // MFMA prefill and FA2 do for the PV product) and packed per token pair,
      // so that P V is v_dot2 too, over V words paired across two tokens by
      // v_perm.  The row sum l adds the same rounded probabilities.
      typedef Elem<DT> E;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float d = 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w) d = E::dot2(kr[u].w[0][w], qp[g][w], d);
          d = row16_sum(d);
          s[u][g] = valid[u] ? d : -INFINITY;
        }
      u32 pp[U / 2][G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mr = s[0][g];
#pragma unroll
        for (int u = 1; u + 1 < U; u += 2) mr = vmax3(mr, s[u][g], s[u + 1][g]);
        mr = vmax(mr, s[U - 1][g]);
        const float mx = vmax(m[g], mr * a.scale_log2);
        const float alpha = fast_exp2(m[g] - mx);
        m[g] = mx;
        l[g] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
#pragma unroll
        for (int v = 0; v < U / 2; ++v) {
          const float p0 = fast_exp2(fmaf(s[2 * v][g], a.scale_log2, -mx));
          const float p1 = fast_exp2(fmaf(s[2 * v + 1][g], a.scale_log2, -mx));
          pp[v][g] = E::pack2_hw(p0, p1);
          l[g] = E::dot2(pp[v][g], E::kOnes, l[g]);
        }
      }
#pragma unroll
      for (int v = 0; v < U / 2; ++v)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          // (token 2v, token 2v+1) of dims 2w and 2w+1
          const u32 lo = __builtin_amdgcn_perm(vr[2 * v + 1].w[0][w], vr[2 * v].w[0][w], kSelLo);
          const u32 hi = __builtin_amdgcn_perm(vr[2 * v + 1].w[0][w], vr[2 * v].w[0][w], kSelHi);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            acc[g][2 * w] = E::dot2(lo, pp[v][g], acc[g][2 * w]);
            acc[g][2 * w + 1] = E::dot2(hi, pp[v][g], acc[g][2 * w + 1]);
          }
        }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float kf[8];
        kr[u].unpack(kf);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) d = fmaf(qf[g][i], kf[i], d);
          d = row16_sum(d);
          s[u][g] = valid[u] ? d : -INFINITY;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = m[g];
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u][g]);
        const float alpha = fast_exp2(m[g] - mx);
        m[g] = mx;
        l[g] *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) s[u][g] = fast_exp2(s[u][g] - mx);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float vf[8];
        vr[u].unpack(vf);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          l[g] += s[u][g];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] = fmaf(s[u][g], vf[i], acc[g][i]);
        }
      }
    }
  }

  // Merge the 4 DPP rows of this wave (lanes li, li+16, li+32, li+48 hold the
  // same dims).
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = fmaxf(m[g], __shfl_xor(m[g], 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float f = fast_exp2(m[g] - mx);
    m[g] = mx;
    l[g] *= f;
    l[g] += __shfl_xor(l[g], 16);
    l[g] += __shfl_xor(l[g], 32);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float x = acc[g][i] * f;
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      acc[g][i] = x;
    }
  }

  __shared__ float sm_m[4][G], sm_l[4][G];
  __shared__ float sm_acc[4][G][kHeadDim];
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sm_acc[wave][g][li * 8 + i] = acc[g][i];
      if (li == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  for (int i = tid; i < G * (kHeadDim / 2); i += 256) {
    const int g = i / (kHeadDim / 2), d2 = (i % (kHeadDim / 2)) * 2;
    float mx = sm_m[0][g];
#pragma unroll
    for (int w = 1; w < 4; ++w) mx = fmaxf(mx, sm_m[w][g]);
    float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = fast_exp2(sm_m[w][g] - mx);
      L += sm_l[w][g] * f;
      o0 += sm_acc[w][g][d2] * f;
      o1 += sm_acc[w][g][d2 + 1] * f;
    }
    const float inv = 1.f / L;
    const int hq = h * G + g;
    if (np == 1) {
      store_out2<DT>(a.out, (int64_t)b * a.out_seq_stride + (int64_t)hq * kHeadDim + d2, o0 * inv,
                     o1 * inv);
    } else {
      const int64_t slot = ((int64_t)b * a.hq + hq) * a.n_parts + part;
      *reinterpret_cast<float2*>(a.ws_o + slot * kHeadDim + d2) = make_float2(o0 * inv, o1 * inv);
      if (d2 == 0) a.ws_lse[slot] = mx + __log2f(L);
    }
  }
}

// Combine the partitions of every (sequence, query head) whose context was
// split: out = sum_p 2^(lse_p - LSE) o_p with LSE = log2 sum_p 2^lse_p.
template <Dt DT>
__global__ __launch_bounds__(64) void decode_reduce_kernel(DecodeArgs a) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int np = parts_of(a, context_len(a, b));
  if (np <= 1) return;
  const int lane = threadIdx.x;
  const int64_t slot0 = ((int64_t)b * a.hq + hq) * a.n_parts;
  float mx = -INFINITY;
  for (int p = 0; p < np; ++p) mx = fmaxf(mx, a.ws_lse[slot0 + p]);
  float W = 0.f, o0 = 0.f, o1 = 0.f;
  for (int p = 0; p < np; ++p) {
    const float w = fast_exp2(a.ws_lse[slot0 + p] - mx);
    const float2 o = *reinterpret_cast<const float2*>(a.ws_o + (slot0 + p) * kHeadDim + 2 * lane);
    W += w;
    o0 = fmaf(w, o.x, o0);
    o1 = fmaf(w, o.y, o1);
  }
  const float inv = 1.f / W;
  store_out2<DT>(a.out, (int64_t)b * a.out_seq_stride + (int64_t)hq * kHeadDim + 2 * lane, o0 * inv,
                 o1 * inv);
}

// ------------------------------------------------------------------ planning
struct DecodePlan {
  int32_t part_tokens;
  int32_t n_parts;
  size_t ws_bytes;
};

static DecodePlan plan_decode(int32_t n_seqs, int32_t hq, int32_t hkv, int32_t block_size,
                              int32_t max_blocks, int32_t max_context_len, int32_t part_tokens) {
  DecodePlan p;
  int64_t cap = (int64_t)max_blocks * block_size;
  if (max_context_len > 0 && max_context_len < cap) cap = max_context_len;
  if (cap < 1) cap = 1;
  int64_t part = part_tokens;
  if (part <= 0) {
    // Measured on MI355X (bf16, block 256): with >= 1024 (sequence, KV head)
    // items and contexts up to 4096 tokens one workgroup per item streams at
    // the HBM ceiling and needs no reduction; otherwise 3072-token partitions
    // (64 x 16k-32k GQA-4 over four context draws: 75.4% of HBM peak against
    // 73.8% for 2048, 75.1% for 2560, 74.3% for 3584 and 72.5% for 4096),
    // halved until there are >= 2048 workgroups for 256 CUs.
    const int64_t items = (int64_t)n_seqs * hkv;
    if (items >= 1024 && cap <= 4096) {
      part = cap;
    } else {
      part = 3072;
      while (part > 256 && items * cdiv(cap, part) < 2048) part /= 2;
    }
  }
  if (part > cap) part = cap;
  p.part_tokens = (int32_t)part;
  p.n_parts = (int32_t)cdiv(cap, part);
  p.ws_bytes = p.n_parts > 1 ? (size_t)n_seqs * hq * p.n_parts * (kHeadDim + 1) * sizeof(float) : 0;
  return p;
}

template <Dt DT, int G>
static void launch_decode_t(const DecodeArgs& a, hipStream_t s) {
  // Token rows in flight per DPP row: eight for bf16/fp16, four for fp32,
  // whose rows take twice the registers (at eight, the fp32 instances of
  // groups 1 and 2 spill under the 128-VGPR bound of four workgroups per
  // CU).  At bf16 group 8, eight rows (233 VGPRs, 2 workgroups per CU) beat
  // four (181) by 3% on 256 seqs x 1-2k at 64/8 heads (318.0 against
  // 328.2 us).
  constexpr int U = DT == Dt::FP32 ? 4 : 8;
  dim3 grid(a.hkv, a.n_parts, a.n_seqs);
  if (a.bs_shift >= 0)
    hipLaunchKernelGGL((decode_paged_kernel<DT, G, U, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((decode_paged_kernel<DT, G, U, false>), grid, dim3(256), 0, s, a);
  if (a.n_parts > 1)
    hipLaunchKernelGGL((decode_reduce_kernel<DT>), dim3(a.hq, a.n_seqs), dim3(64), 0, s, a);
}

template <Dt DT>
static int launch_decode_g(const DecodeArgs& a, int g, hipStream_t s) {
  switch (g) {
    case 1: launch_decode_t<DT, 1>(a, s); break;
    case 2: launch_decode_t<DT, 2>(a, s); break;
    case 4: launch_decode_t<DT, 4>(a, s); break;
    case 8: launch_decode_t<DT, 8>(a, s); break;
    default: return AAC_ERR_UNSUPPORTED;
  }
  return AAC_OK;
}

}  // namespace aac

using namespace aac;

extern "C" size_t aac_decode_workspace_bytes(int32_t n_seqs, int32_t n_q_heads, int32_t n_kv_heads,
                                             int32_t head_dim, int32_t block_size,
                                             int32_t max_blocks_per_seq, int32_t max_context_len,
                                             int32_t partition_tokens) {
  (void)head_dim;
  if (n_seqs <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || block_size <= 0 || max_blocks_per_seq <= 0)
    return 0;
  return plan_decode(n_seqs, n_q_heads, n_kv_heads, block_size, max_blocks_per_seq, max_context_len,
                     partition_tokens)
      .ws_bytes;
}

static int decode_common(const void* q, int64_t q_seq_stride, const void* k_cache,
                         const void* v_cache, int64_t num_blocks, int32_t block_size,
                         const int32_t* block_tables, int32_t max_blocks_per_seq,
                         const int32_t* lens, int32_t lens_add, int32_t n_seqs,
                         int32_t max_context_len, int32_t n_q_heads, int32_t n_kv_heads,
                         int32_t head_dim, float scale, void* out, int64_t out_seq_stride,
                         void* workspace, size_t workspace_bytes, int32_t partition_tokens,
                         int32_t dtype, hipStream_t stream) {
  if (n_seqs < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || num_blocks <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0 || q_seq_stride < 0 || out_seq_stride < 0)
    return AAC_ERR_INVALID_ARGUMENT;
  if (head_dim != kHeadDim) return AAC_ERR_UNSUPPORTED;
  if (n_q_heads % n_kv_heads) return AAC_ERR_SHAPE;
  if (n_seqs == 0) return AAC_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !lens || !out) return AAC_ERR_INVALID_ARGUMENT;
  if (q_seq_stride < (int64_t)n_q_heads * head_dim || out_seq_stride < (int64_t)n_q_heads * head_dim)
    return AAC_ERR_SHAPE;
  int es;
  Dt dt;
  switch (dtype) {
    case AAC_DTYPE_BF16: es = 2; dt = Dt::BF16; break;
    case AAC_DTYPE_FP16: es = 2; dt = Dt::FP16; break;
    case AAC_DTYPE_FP32: es = 4; dt = Dt::FP32; break;
    default: return AAC_ERR_UNSUPPORTED;
  }
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 ||
      (q_seq_stride * es) % 16 || (uintptr_t)out % 8 || (out_seq_stride * es) % 8)
    return AAC_ERR_MISALIGNED;
  const DecodePlan plan = plan_decode(n_seqs, n_q_heads, n_kv_heads, block_size,
                                      max_blocks_per_seq, max_context_len, partition_tokens);
  if (plan.ws_bytes) {
    if (!workspace || workspace_bytes < plan.ws_bytes) return AAC_ERR_WORKSPACE;
    if ((uintptr_t)workspace % 16) return AAC_ERR_MISALIGNED;
  }
  DecodeArgs a = {};
  a.q = q;
  a.q_seq_stride = q_seq_stride;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks_per_seq;
  a.lens = lens;
  a.lens_add = lens_add;
  a.n_seqs = n_seqs;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.out = out;
  a.out_seq_stride = out_seq_stride;
  a.n_parts = plan.n_parts;
  a.part_tokens = plan.part_tokens;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  if (a.bs_shift < 0) {  // block_size >= 3 here
    const int l = 32 - __builtin_clz((unsigned)(block_size - 1));
    a.bs_magic = (uint64_t(1) << (31 + l)) / (uint64_t)block_size + 1;
    a.bs_mshift = 31 + l;
  } else {
    a.bs_magic = 0;
    a.bs_mshift = 0;
  }
  // length order only without a split: split partitions are already
  // uniform work units, and the ordering costs every workgroup a few barriers
  a.lpt = plan.n_parts == 1 && n_seqs >= 2 && n_seqs <= kLptMaxSeqs;
  a.lpt_max = max_context_len > 0
                  ? max_context_len
                  : (int32_t)std::min<int64_t>((int64_t)max_blocks_per_seq * block_size, INT32_MAX);
  if (plan.ws_bytes) {
    a.ws_o = reinterpret_cast<float*>(workspace);
    a.ws_lse = a.ws_o + (size_t)n_seqs * n_q_heads * plan.n_parts * kHeadDim;
  }
  const int g = n_q_heads / n_kv_heads;
  int rc;
  switch (dt) {
    case Dt::BF16: rc = launch_decode_g<Dt::BF16>(a, g, stream); break;
    case Dt::FP16: rc = launch_decode_g<Dt::FP16>(a, g, stream); break;
    default: rc = launch_decode_g<Dt::FP32>(a, g, stream); break;
  }
  if (rc != AAC_OK) return rc;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}

extern "C" int aac_decode_paged(const void* q, int64_t q_seq_stride, const void* k_cache,
                                const void* v_cache, int64_t num_blocks, int32_t block_size,
                                const int32_t* block_tables, int32_t max_blocks_per_seq,
                                const int32_t* context_lens, int32_t n_seqs,
                                int32_t max_context_len, int32_t n_q_heads, int32_t n_kv_heads,
                                int32_t head_dim, float scale, void* out, int64_t out_seq_stride,
                                void* workspace, size_t workspace_bytes, int32_t partition_tokens,
                                int32_t dtype, void* stream) {
  return decode_common(q, q_seq_stride, k_cache, v_cache, num_blocks, block_size, block_tables,
                       max_blocks_per_seq, context_lens, 0, n_seqs, max_context_len, n_q_heads,
                       n_kv_heads, head_dim, scale, out, out_seq_stride, workspace,
                       workspace_bytes, partition_tokens, dtype, (hipStream_t)stream);
}

// ------------------------------------------------------------------ static scratch
// Split-K scratch of aac_decode_paged_noalloc: one array per GPU, held until
// the process ends.  In host code `scratch` names a host-side stand-in, not
// device memory; the array's device address on each GPU comes from
// hipGetSymbolAddress (looked up once per device, with that device current)
// and only that address is handed to the kernels.
static __device__ __align__(256) unsigned char scratch[AAC_DECODE_SCRATCH_BYTES];

static int scratch_address(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return AAC_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return AAC_ERR_SCRATCH;
    addr[dev] = p;
  }
  *out = addr[dev];
  return AAC_OK;
}

extern "C" int aac_decode_paged_noalloc(const void* q, int64_t q_seq_stride, const void* k_cache,
                                        const void* v_cache, int64_t num_blocks, int32_t block_size,
                                        const int32_t* block_tables, int32_t max_blocks_per_seq,
                                        const int32_t* context_lens, int32_t n_seqs,
                                        int32_t max_context_len, int32_t n_q_heads,
                                        int32_t n_kv_heads, int32_t head_dim, float scale,
                                        void* out, int64_t out_seq_stride,
                                        int32_t partition_tokens, int32_t dtype, void* stream) {
  // the plan is host arithmetic: a call it does not fit is rejected before
  // the device is touched
  const size_t need = aac_decode_workspace_bytes(n_seqs, n_q_heads, n_kv_heads, head_dim,
                                                 block_size, max_blocks_per_seq, max_context_len,
                                                 partition_tokens);
  if (need > AAC_DECODE_SCRATCH_BYTES) return AAC_ERR_SCRATCH;
  void* ws = nullptr;
  if (need) {
    const int rc = scratch_address(&ws);
    if (rc != AAC_OK) return rc;
  }
  return decode_common(q, q_seq_stride, k_cache, v_cache, num_blocks, block_size, block_tables,
                       max_blocks_per_seq, context_lens, 0, n_seqs, max_context_len, n_q_heads,
                       n_kv_heads, head_dim, scale, out, out_seq_stride, ws,
                       need ? (size_t)AAC_DECODE_SCRATCH_BYTES : 0, partition_tokens, dtype,
                       (hipStream_t)stream);
}

extern "C" int aac_decode_append_paged(const void* q, int64_t q_seq_stride, const void* k,
                                       const void* v, int64_t k_tok_stride, int64_t v_tok_stride,
                                       void* k_cache, void* v_cache, int64_t num_blocks,
                                       int32_t block_size, const int32_t* block_tables,
                                       int32_t max_blocks_per_seq, const int32_t* cache_seqlens,
                                       int32_t n_seqs, int32_t max_context_len, int32_t n_q_heads,
                                       int32_t n_kv_heads, int32_t head_dim, float scale, void* out,
                                       int64_t out_seq_stride, void* workspace,
                                       size_t workspace_bytes, int32_t partition_tokens,
                                       int32_t dtype, void* stream) {
  if (head_dim != kHeadDim) return AAC_ERR_UNSUPPORTED;
  const int rc = aac_kv_append_paged(k, v, k_tok_stride, v_tok_stride, k_cache, v_cache, num_blocks,
                                     block_size, block_tables, max_blocks_per_seq, cache_seqlens,
                                     n_seqs, n_kv_heads, head_dim, dtype, stream);
  if (rc != AAC_OK) return rc;
  return decode_common(q, q_seq_stride, k_cache, v_cache, num_blocks, block_size, block_tables,
                       max_blocks_per_seq, cache_seqlens, 1, n_seqs, max_context_len, n_q_heads,
                       n_kv_heads, head_dim, scale, out, out_seq_stride, workspace,
                       workspace_bytes, partition_tokens, dtype, (hipStream_t)stream);
}
