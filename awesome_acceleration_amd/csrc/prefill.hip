// Varlen causal GQA prefill attention (gfx950, bf16/fp16 MFMA) -- the
// reference's flash_attn_varlen_func(q, k, v, cu, cu, max, max, causal=True)
// call (llm.py:178-184), and with the store folded in, llm.py:171-184.
//
// Tiling (FlashAttention-2 style, Dao 2023, re-derived for CDNA4 MFMA):
//   * A workgroup (4 wavefronts) owns one KV head h of one segment and a block
//     of BQ queries for all G = Hq/Hkv query heads that read h.  Wave w serves
//     32 queries x HPW (<= 2) heads; with G = 2 the four waves cover 128
//     queries x 2 heads, so every K/V tile staged in LDS feeds 2 heads x 128
//     queries (the KV head is shared across its query heads).
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
//   * Online softmax in fp32 in the log2 domain (exp via v_exp_f32).
//   * Causal masking is bottom-right aligned (query i sees keys
//     j <= i + Lk - Lq); key tiles beyond a wave's last visible key are
//     skipped, and only tiles that cross the diagonal evaluate the mask.
//   * Grid = (kv head, segment, q-block rank) with the last (heaviest) causal
//     q-blocks dispatched first.
//
// FLOPs per launch (the MFMA roofline): 4 * Hq * D * sum over segments of the
// visible (query, key) pairs, i.e. 4*Hq*D*L(L+1)/2 per causal segment.

#include "aac_common.h"

namespace aac {

namespace pf {

constexpr int D = 128;
constexpr int BKV = 64;         // keys per LDS tile
constexpr int KPITCH = D + 8;   // K tile row pitch (elements)
constexpr int VPITCH = BKV + 8; // V^T tile row pitch (elements)

struct Args {
  const u16* q;
  const u16* k;
  const u16* v;
  int64_t q_stride, k_stride, v_stride, o_stride;  // token strides (elements)
  const int32_t* cu_q;
  const int32_t* cu_k;
  int32_t n_seqs;
  int32_t hq, hkv;
  float scale_log2;
  u16* out;
};

template <bool F16> struct Mfma;
template <> struct Mfma<false> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline u32 pack(float a, float b) { return pack_bf16x2(a, b); }
};
template <> struct Mfma<true> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline u32 pack(float a, float b) { return pack_f16x2(a, b); }
};

// byte-select masks for v_perm_b32(hi_src, lo_src, sel)
constexpr u32 kSelLo = 0x05040100u;  // (lo16 of lo_src, lo16 of hi_src)
constexpr u32 kSelHi = 0x07060302u;  // (hi16 of lo_src, hi16 of hi_src)

template <int G, bool CAUSAL, bool F16>
__global__ __launch_bounds__(256) void prefill_kernel(Args a) {
  constexpr int HPW = G >= 2 ? 2 : 1;  // query heads per wave
  constexpr int WH = G / HPW;          // head slots per workgroup
  constexpr int WQ = 4 / WH;           // 32-query slots per workgroup
  constexpr int BQ = 32 * WQ;
  static_assert(WH * WQ == 4, "four waves per workgroup");
  typedef Mfma<F16> M;

  __shared__ __attribute__((aligned(16))) u16 Ks[BKV * KPITCH];
  __shared__ __attribute__((aligned(16))) u16 Vt[D * VPITCH];

  const int h = blockIdx.x;
  const int s = blockIdx.y;
  const int q_beg = a.cu_q[s], Lq = a.cu_q[s + 1] - q_beg;
  const int k_beg = a.cu_k[s], Lk = a.cu_k[s + 1] - k_beg;
  const int nqb = (Lq + BQ - 1) / BQ;
  const int rank = blockIdx.z;
  if (rank >= nqb) return;
  const int qb = CAUSAL ? nqb - 1 - rank : rank;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wq = wave % WQ, wh = wave / WQ;
  const int hl = lane >> 5;  // lane half
  const int col = lane & 31;
  const int qi = qb * BQ + wq * 32 + col;  // query index in the segment
  const bool q_ok = qi < Lq;
  const int shift = Lk - Lq;  // bottom-right causal alignment

  // keys visible to the whole workgroup / this wave / this lane
  const int wg_qmax = min(qb * BQ + BQ, Lq) - 1;
  const int kv_end = CAUSAL ? max(0, min(Lk, wg_qmax + 1 + shift)) : Lk;
  const int w_qmin = qb * BQ + wq * 32;
  const int w_qmax = min(w_qmin + 31, Lq - 1);
  const int w_end = CAUSAL ? max(0, min(Lk, w_qmax + 1 + shift)) : Lk;
  const int w_full = CAUSAL ? min(Lk, w_qmin + 1 + shift) : Lk;  // keys < w_full need no mask
  const int my_lim = CAUSAL ? min(Lk, qi + 1 + shift) : Lk;

  // Q fragments: B operand of S^T = K Q^T, lane = query column, 8 dims.
  u32x4 qf[HPW][8];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const int hq = h * G + wh * HPW + j;
    const u16* qp = a.q + (int64_t)(q_beg + qi) * a.q_stride + hq * D + hl * 8;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      qf[j][t] = q_ok ? *reinterpret_cast<const u32x4*>(qp + 16 * t) : u32x4{0, 0, 0, 0};
  }

  f32x16 o[HPW][4];
  float m[HPW], l[HPW];
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    m[j] = -1e30f;
    l[j] = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[j][c][i] = 0.f;
  }

  const u16* kg = a.k + (int64_t)k_beg * a.k_stride + h * D;
  const u16* vg = a.v + (int64_t)k_beg * a.v_stride + h * D;

  for (int kt = 0; kt < kv_end; kt += BKV) {
    __syncthreads();
    // ---- stage K tile [BKV][D] (row pitch KPITCH)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int chunk = tid + 256 * i;
      const int r = chunk >> 4, c8 = (chunk & 15) * 8;
      u32x4 val = {0, 0, 0, 0};
      if (kt + r < kv_end) val = *reinterpret_cast<const u32x4*>(kg + (int64_t)(kt + r) * a.k_stride + c8);
      *reinterpret_cast<u32x4*>(Ks + r * KPITCH + c8) = val;
    }
    // ---- stage V^T tile [D][BKV]: thread = 4 keys x 8 dims, transposed in registers
    {
      const int kq = tid >> 4;       // key quad 0..15
      const int d0 = (tid & 15) * 8;  // first dim
      u32x4 r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt + kq * 4 + i;
        r[i] = key < kv_end ? *reinterpret_cast<const u32x4*>(vg + (int64_t)key * a.v_stride + d0)
                            : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int jw = 0; jw < 4; ++jw) {  // dims d0+2jw (lo) and d0+2jw+1 (hi)
        u32x2 lo, hi;
        lo[0] = __builtin_amdgcn_perm(r[1][jw], r[0][jw], kSelLo);
        lo[1] = __builtin_amdgcn_perm(r[3][jw], r[2][jw], kSelLo);
        hi[0] = __builtin_amdgcn_perm(r[1][jw], r[0][jw], kSelHi);
        hi[1] = __builtin_amdgcn_perm(r[3][jw], r[2][jw], kSelHi);
        *reinterpret_cast<u32x2*>(Vt + (d0 + 2 * jw) * VPITCH + kq * 4) = lo;
        *reinterpret_cast<u32x2*>(Vt + (d0 + 2 * jw + 1) * VPITCH + kq * 4) = hi;
      }
    }
    __syncthreads();

#pragma unroll
    for (int sub = 0; sub < BKV / 32; ++sub) {
      const int kb = kt + sub * 32;
      if (kb >= w_end) break;  // wave-uniform
      // ---- S^T = K Q^T for HPW heads
      f32x16 st[HPW];
#pragma unroll
      for (int j = 0; j < HPW; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) st[j][i] = 0.f;
      const u16* kr = Ks + (sub * 32 + col) * KPITCH + hl * 8;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(kr + 16 * t);
#pragma unroll
        for (int j = 0; j < HPW; ++j) st[j] = M::run(ka, qf[j][t], st[j]);
      }
      const bool need_mask = kb + 32 > w_full;  // wave-uniform
      // ---- online softmax (log2 domain); P^T packed as the PV B operand
      u32x4 pb[HPW][2];
#pragma unroll
      for (int j = 0; j < HPW; ++j) {
        float sv[16];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float x = st[j][i] * a.scale_log2;
          if (need_mask) {
            const int key = kb + 8 * (i >> 2) + 4 * hl + (i & 3);
            x = key < my_lim ? x : -INFINITY;
          }
          sv[i] = x;
          mx = fmaxf(mx, x);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m[j], mx);
        const float alpha = fast_exp2(m[j] - mn);
        m[j] = mn;
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          sv[i] = fast_exp2(sv[i] - mn);
          ps += sv[i];
        }
        l[j] = l[j] * alpha + ps;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[j][c][i] *= alpha;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int w = 0; w < 4; ++w) pb[j][t][w] = M::pack(sv[8 * t + 2 * w], sv[8 * t + 2 * w + 1]);
      }
      // ---- O^T += V^T P^T  (A = V^T rows: dims; k: keys in the lane-half order)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u16* vr = Vt + (32 * c + col) * VPITCH + sub * 32 + 4 * hl;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const u32x2 v0 = *reinterpret_cast<const u32x2*>(vr + 16 * t);
          const u32x2 v1 = *reinterpret_cast<const u32x2*>(vr + 16 * t + 8);
          const u32x4 va = {v0[0], v0[1], v1[0], v1[1]};
#pragma unroll
          for (int j = 0; j < HPW; ++j) o[j][c] = M::run(va, pb[j][t], o[j][c]);
        }
      }
    }
  }

  // ---- epilogue: full row sum (partner lane holds the other 16 keys of each
  // 32-key sub-tile), normalise, store.
  if (!q_ok) return;
#pragma unroll
  for (int j = 0; j < HPW; ++j) {
    const float lt = l[j] + __shfl_xor(l[j], 32);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int hq = h * G + wh * HPW + j;
    u16* op = a.out + (int64_t)(q_beg + qi) * a.o_stride + hq * D + 4 * hl;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x2 w;
        w[0] = M::pack(o[j][c][4 * r] * inv, o[j][c][4 * r + 1] * inv);
        w[1] = M::pack(o[j][c][4 * r + 2] * inv, o[j][c][4 * r + 3] * inv);
        *reinterpret_cast<u32x2*>(op + 32 * c + 8 * r) = w;
      }
  }
}

template <int G, bool CAUSAL, bool F16>
static void launch_t(const Args& a, int max_q, hipStream_t st) {
  constexpr int HPW = G >= 2 ? 2 : 1;
  constexpr int BQ = 32 * (4 / (G / HPW));
  dim3 grid(a.hkv, a.n_seqs, (unsigned)cdiv(max_q, BQ));
  hipLaunchKernelGGL((prefill_kernel<G, CAUSAL, F16>), grid, dim3(256), 0, st, a);
}

template <bool CAUSAL, bool F16>
static int launch_g(const Args& a, int g, int max_q, hipStream_t st) {
  switch (g) {
    case 1: launch_t<1, CAUSAL, F16>(a, max_q, st); break;
    case 2: launch_t<2, CAUSAL, F16>(a, max_q, st); break;
    case 4: launch_t<4, CAUSAL, F16>(a, max_q, st); break;
    case 8: launch_t<8, CAUSAL, F16>(a, max_q, st); break;
    default: return AAC_ERR_UNSUPPORTED;
  }
  return AAC_OK;
}

}  // namespace pf

static int prefill_common(const void* q, const void* k, const void* v, int64_t q_tok_stride,
                          int64_t k_tok_stride, int64_t v_tok_stride, const int32_t* cu_seqlens_q,
                          const int32_t* cu_seqlens_k, int32_t n_seqs, int32_t max_seqlen_q,
                          int32_t max_seqlen_k, int32_t n_q_heads, int32_t n_kv_heads,
                          int32_t head_dim, float scale, int32_t causal, void* out,
                          int64_t out_tok_stride, int32_t dtype, hipStream_t stream,
                          bool launch) {
  (void)max_seqlen_k;
  if (dtype != AAC_DTYPE_BF16 && dtype != AAC_DTYPE_FP16) return AAC_ERR_UNSUPPORTED;
  if (head_dim != pf::D) return AAC_ERR_UNSUPPORTED;
  if (n_seqs < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || max_seqlen_q < 0 || q_tok_stride < 0 ||
      k_tok_stride < 0 || v_tok_stride < 0 || out_tok_stride < 0)
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
  const bool f16 = dtype == AAC_DTYPE_FP16;
  int rc;
  if (causal)
    rc = f16 ? pf::launch_g<true, true>(a, g, max_seqlen_q, stream)
             : pf::launch_g<true, false>(a, g, max_seqlen_q, stream);
  else
    rc = f16 ? pf::launch_g<false, true>(a, g, max_seqlen_q, stream)
             : pf::launch_g<false, false>(a, g, max_seqlen_q, stream);
  if (rc != AAC_OK) return rc;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}

}  // namespace aac

using namespace aac;

extern "C" int aac_prefill_varlen(const void* q, const void* k, const void* v, int64_t q_tok_stride,
                                  int64_t k_tok_stride, int64_t v_tok_stride,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int32_t n_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                  int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                  float scale, int32_t causal, void* out, int64_t out_tok_stride,
                                  int32_t dtype, void* stream) {
  return prefill_common(q, k, v, q_tok_stride, k_tok_stride, v_tok_stride, cu_seqlens_q,
                        cu_seqlens_k, n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads,
                        head_dim, scale, causal, out, out_tok_stride, dtype, (hipStream_t)stream,
                        true);
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
  rc = aac_kv_store(k, v, k_tok_stride, v_tok_stride, k_cache, v_cache, num_cache_rows, slot_mapping,
                    n_kv_tokens, n_kv_heads, head_dim, dtype, stream);
  if (rc != AAC_OK) return rc;
  return prefill_common(q, k, v, q_tok_stride, k_tok_stride, v_tok_stride, cu_seqlens_q,
                        cu_seqlens_k, n_seqs, max_seqlen_q, max_seqlen_k, n_q_heads, n_kv_heads,
                        head_dim, scale, causal, out, out_tok_stride, dtype, (hipStream_t)stream,
                        true);
}
