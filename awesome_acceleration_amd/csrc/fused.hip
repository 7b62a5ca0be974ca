// Fused elementwise kernels around the attention call site (gfx950).
//
// The reference runs these as chains of small torch kernels per layer:
//   RMSNorm                  model/model.py:47-52   (fp32 statistics, result
//                            cast to the activation dtype, times the weight)
//   residual add             model/model.py:259, :265 / llm.py:188, :194
//   q/k RMSNorm + RoPE       model/model.py:225-228 (rotation in the
//                            activation dtype, model/model.py:86-99)
//   KV store / append        llm.py:171-174, model/model.py:233-240
//   SiLU(gate) * up          model/model.py:188
// Here each chain is one launch.  Every value is rounded to the activation
// dtype at the same points as the torch expression it replaces, so the fused
// results equal the unfused ones up to fp32 summation order inside the norm.
//
// All three kernels are HBM-bound streaming passes (one read and one write of
// each tensor).

#include <type_traits>

#include "qk_head.h"

namespace aac {

// token count from which q/k norm + RoPE runs one wavefront per token
// (measured: 32% faster at 262,144 tokens, 85% slower at 256)
constexpr int64_t kQkTokenKernelMin = 4096;

namespace fz {

__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// ---------------------------------------------------------------- RMSNorm
// One wavefront per row; lane owns 8 consecutive elements per 512-element
// chunk.  With a residual: h = x + residual (rounded), residual_out = h.
template <Dt DT, bool RESID, int MAXC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const u16* x, int64_t x_stride,
                                                      const u16* res, u16* res_out,
                                                      const u16* w, u16* out, int64_t rows,
                                                      int hidden, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nc = hidden / 512;  // full 512-element chunks
  float v[MAXC][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    if (c < nc) {
      const int e = c * 512 + lane * 8;
      unpack8<DT>(*reinterpret_cast<const u32x4*>(x + row * x_stride + e), v[c]);
      if (RESID) {
        float r[8];
        unpack8<DT>(*reinterpret_cast<const u32x4*>(res + row * hidden + e), r);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] = Cvt<DT>::round(v[c][i] + r[i]);
        *reinterpret_cast<u32x4*>(res_out + row * hidden + e) = pack8<DT>(v[c]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[c][i], v[c][i], ss);
    }
  }
  ss = wave_sum(ss);
  const float rs = __frsqrt_rn(ss / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    if (c < nc) {
      const int e = c * 512 + lane * 8;
      float wf[8], o[8];
      unpack8<DT>(*reinterpret_cast<const u32x4*>(w + e), wf);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = wf[i] * Cvt<DT>::round(v[c][i] * rs);
      *reinterpret_cast<u32x4*>(out + row * hidden + e) = pack8<DT>(o);
    }
  }
}


// Few tokens (a decode step): one 16-lane DPP row per (token, head), the
// most parallel mapping.  Heads 0..hq-1 are query heads, hq..hq+hkv-1 key
// heads, then value heads.
template <Dt DT>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QkArgs a) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int heads = a.hq + 2 * a.hkv;
  const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // (token, head)
  const int64_t t = item / heads;
  const int hh = (int)(item - t * heads);
  if (t >= a.n_tokens) return;  // the whole 16-lane row
  const u32x4 xr = *reinterpret_cast<const u32x4*>(a.qkv + t * a.qkv_stride +
                                                   (int64_t)hh * kHeadDimFused + li * 8);
  const int64_t crow = cache_row(a, t);
  float wf[8], cf[8], sf[8];
  const int p = clamp_pos(a, a.positions[t]);
  if (hh < a.hq + a.hkv) {
    unpack8<DT>(*reinterpret_cast<const u32x4*>((hh < a.hq ? a.qw : a.kw) + li * 8), wf);
    unpack8<DT>(*reinterpret_cast<const u32x4*>(a.cos + (int64_t)p * kHeadDimFused + li * 8), cf);
    unpack8<DT>(*reinterpret_cast<const u32x4*>(a.sin + (int64_t)p * kHeadDimFused + li * 8), sf);
  }
  norm_rope_head<DT>(a, t, hh, li, xr, crow, wf, cf, sf);
}

// Many tokens (a prefill chunk): one wavefront per token; its four DPP rows
// take the heads in turn (row r: heads r, r + 4, ...), so the token's
// position, cos/sin vectors, norm weights and cache row are fetched once,
// and a row loads a group of its heads before it processes the first.
template <Dt DT>
__global__ __launch_bounds__(256) void qk_norm_rope_tok_kernel(QkArgs a) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, r = lane >> 4;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.n_tokens) return;  // the whole wavefront
  const int heads = a.hq + 2 * a.hkv;
  const u16* src = a.qkv + t * a.qkv_stride + li * 8;
  const int64_t crow = cache_row(a, t);
  const int p = clamp_pos(a, a.positions[t]);
  float cf[8], sf[8], qwf[8], kwf[8];
  unpack8<DT>(*reinterpret_cast<const u32x4*>(a.qw + li * 8), qwf);
  unpack8<DT>(*reinterpret_cast<const u32x4*>(a.kw + li * 8), kwf);
  unpack8<DT>(*reinterpret_cast<const u32x4*>(a.cos + (int64_t)p * kHeadDimFused + li * 8), cf);
  unpack8<DT>(*reinterpret_cast<const u32x4*>(a.sin + (int64_t)p * kHeadDimFused + li * 8), sf);
  constexpr int U = 4;  // heads per row per group
  for (int h0 = 0; h0 < heads; h0 += 4 * U) {
    u32x4 xr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int hh = h0 + 4 * u + r;
      if (hh < heads) xr[u] = *reinterpret_cast<const u32x4*>(src + (int64_t)hh * kHeadDimFused);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int hh = h0 + 4 * u + r;  // uniform across the 16-lane row
      if (hh < heads) norm_rope_head<DT>(a, t, hh, li, xr[u], crow, hh < a.hq ? qwf : kwf, cf, sf);
    }
  }
}

// ---------------------------------------------------------------- SiLU * up
template <Dt DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const u16* gu, u16* out, int64_t rows,
                                                       int inter) {
  const int64_t per_row = inter / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * per_row) return;
  const int64_t r = i / per_row, c = (i - r * per_row) * 8;
  float g[8], u[8], o[8];
  unpack8<DT>(*reinterpret_cast<const u32x4*>(gu + r * 2 * inter + c), g);
  unpack8<DT>(*reinterpret_cast<const u32x4*>(gu + r * 2 * inter + inter + c), u);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float s = Cvt<DT>::round(g[k] / (1.f + __expf(-g[k])));  // F.silu, rounded
    o[k] = s * u[k];
  }
  *reinterpret_cast<u32x4*>(out + r * inter + c) = pack8<DT>(o);
}

// ---------------------------------------------------------------- argmax
// Greedy sampling (llm.py:215-219, temperature 0): the index of the largest
// logit of each row, the first one among equal maxima, a NaN counting as
// larger than every number -- torch.argmax's result.  One workgroup per row;
// each thread scans 16-byte chunks t, t + 1024, ... (coalesced), keeping
// its first best, then the workgroup reduces the (value, index) pairs.
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <Dt DT>
__global__ __launch_bounds__(1024) void argmax_kernel(const void* x, int64_t stride, int cols,
                                                      int64_t* out) {
  typedef typename std::conditional<DT == Dt::FP32, float, u16>::type T;
  constexpr int E = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  const int tid = threadIdx.x;
  const T* p = reinterpret_cast<const T*>(x) + blockIdx.x * stride;
  auto value = [&](const T* q) {
    if constexpr (DT == Dt::FP32) return *q;
    else return Cvt<DT>::lo(*q);
  };
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  // elements before the row's first 16-byte boundary, whole chunks, the rest
  const int head = min(cols, (int)(((16 - ((uintptr_t)p & 15)) & 15) / sizeof(T)));
  const int nch = (cols - head) / E;
  for (int i = tid; i < head; i += 1024)
    if (am_better(value(p + i), i, bv, bi)) { bv = value(p + i); bi = i; }
  for (int c = tid; c < nch; c += 1024) {
    const int i0 = head + c * E;
    float v[8];
    const u32x4 w = *reinterpret_cast<const u32x4*>(p + i0);
    if constexpr (DT == Dt::FP32) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e]);
    } else {
      unpack8<DT>(w, v);
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (am_better(v[e], i0 + e, bv, bi)) { bv = v[e]; bi = i0 + e; }
  }
  for (int i = head + nch * E + tid; i < cols; i += 1024)
    if (am_better(value(p + i), i, bv, bi)) { bv = value(p + i); bi = i; }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid < 64) {
    bv = tid < 16 ? sv[tid] : -INFINITY;
    bi = tid < 16 ? si[tid] : 0x7fffffff;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (tid == 0) out[blockIdx.x] = bi;
  }
}

}  // namespace fz
}  // namespace aac

using namespace aac;

static bool fz_dtype(int32_t dtype, Dt* dt) {
  if (dtype == AAC_DTYPE_BF16) { *dt = Dt::BF16; return true; }
  if (dtype == AAC_DTYPE_FP16) { *dt = Dt::FP16; return true; }
  return false;
}

static int fz_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}

extern "C" int aac_rmsnorm(const void* x, int64_t x_row_stride, const void* residual,
                           void* residual_out, const void* weight, void* out, int64_t n_rows,
                           int32_t hidden, float eps, int32_t dtype, void* stream) {
  Dt dt;
  if (!fz_dtype(dtype, &dt)) return AAC_ERR_UNSUPPORTED;
  if (n_rows < 0 || hidden <= 0 || x_row_stride < hidden) return AAC_ERR_INVALID_ARGUMENT;
  if (hidden % 512 || hidden > 4096) return AAC_ERR_UNSUPPORTED;
  if (n_rows == 0) return AAC_OK;
  if (!x || !weight || !out || ((residual == nullptr) != (residual_out == nullptr)))
    return AAC_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)residual |
       (uintptr_t)residual_out) % 16 || x_row_stride % 8)
    return AAC_ERR_MISALIGNED;
  const dim3 grid((unsigned)cdiv(n_rows, 4));
  auto* xs = (const u16*)x;
  auto* rs = (const u16*)residual;
  auto* ro = (u16*)residual_out;
  auto* w = (const u16*)weight;
  auto* o = (u16*)out;
  hipStream_t s = (hipStream_t)stream;
#define AAC_RMS(DTV, R)                                                                         \
  hipLaunchKernelGGL((fz::rmsnorm_kernel<DTV, R, 8>), grid, dim3(256), 0, s, xs, x_row_stride, rs, \
                     ro, w, o, n_rows, hidden, eps)
  if (dt == Dt::BF16) {
    if (residual) AAC_RMS(Dt::BF16, true); else AAC_RMS(Dt::BF16, false);
  } else {
    if (residual) AAC_RMS(Dt::FP16, true); else AAC_RMS(Dt::FP16, false);
  }
#undef AAC_RMS
  return fz_status();
}

extern "C" int aac_qk_norm_rope_store(
    const void* qkv, int64_t qkv_tok_stride, int64_t n_tokens, int32_t n_q_heads,
    int32_t n_kv_heads, int32_t head_dim, const void* q_norm_weight, const void* k_norm_weight,
    float eps, const void* cos_table, const void* sin_table, int32_t max_position,
    const int32_t* positions, void* q_out, void* k_out, void* k_cache, void* v_cache,
    int64_t num_cache_rows, const int64_t* slot_mapping, const int32_t* block_tables,
    int32_t max_blocks_per_seq, const int32_t* cache_seqlens, int32_t block_size, int32_t dtype,
    void* stream) {
  Dt dt;
  if (!fz_dtype(dtype, &dt)) return AAC_ERR_UNSUPPORTED;
  if (head_dim != kHeadDimFused) return AAC_ERR_UNSUPPORTED;
  if (n_tokens < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || max_position <= 0)
    return AAC_ERR_INVALID_ARGUMENT;
  if (qkv_tok_stride < (int64_t)(n_q_heads + 2 * n_kv_heads) * head_dim) return AAC_ERR_SHAPE;
  if (n_tokens == 0) return AAC_OK;
  if (!qkv || !q_norm_weight || !k_norm_weight || !cos_table || !sin_table || !positions || !q_out)
    return AAC_ERR_INVALID_ARGUMENT;
  const bool store = v_cache != nullptr;
  if (store) {
    if (!k_cache) return AAC_ERR_INVALID_ARGUMENT;
    if (!slot_mapping) {
      if (!block_tables || !cache_seqlens || block_size <= 0 || max_blocks_per_seq <= 0)
        return AAC_ERR_INVALID_ARGUMENT;
    }
  }
  if (((uintptr_t)qkv | (uintptr_t)q_out | (uintptr_t)k_out | (uintptr_t)k_cache |
       (uintptr_t)v_cache | (uintptr_t)cos_table | (uintptr_t)sin_table) % 16 ||
      qkv_tok_stride % 8)
    return AAC_ERR_MISALIGNED;
  fz::QkArgs a;
  a.qkv = (const u16*)qkv;
  a.qkv_stride = qkv_tok_stride;
  a.n_tokens = n_tokens;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.qw = (const u16*)q_norm_weight;
  a.kw = (const u16*)k_norm_weight;
  a.eps = eps;
  a.cos = (const u16*)cos_table;
  a.sin = (const u16*)sin_table;
  a.positions = positions;
  a.max_pos = max_position;
  a.q_out = (u16*)q_out;
  a.k_out = (u16*)k_out;
  a.k_cache = (u16*)k_cache;
  a.v_cache = (u16*)v_cache;
  a.slot_mapping = slot_mapping;
  a.num_rows = num_cache_rows;
  a.block_tables = block_tables;
  a.max_blocks = max_blocks_per_seq;
  a.cache_seqlens = cache_seqlens;
  a.block_size = block_size;
  a.num_blocks = block_size > 0 ? num_cache_rows / block_size : 0;
  hipStream_t s = (hipStream_t)stream;
  if (n_tokens >= kQkTokenKernelMin) {  // one wavefront per token
    const dim3 grid((unsigned)cdiv(n_tokens, 4));
    if (dt == Dt::BF16)
      hipLaunchKernelGGL((fz::qk_norm_rope_tok_kernel<Dt::BF16>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((fz::qk_norm_rope_tok_kernel<Dt::FP16>), grid, dim3(256), 0, s, a);
  } else {  // one 16-lane row per (token, head)
    const int64_t items = n_tokens * (n_q_heads + 2 * n_kv_heads);
    const dim3 grid((unsigned)cdiv(items * 16, 256));
    if (dt == Dt::BF16)
      hipLaunchKernelGGL((fz::qk_norm_rope_kernel<Dt::BF16>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((fz::qk_norm_rope_kernel<Dt::FP16>), grid, dim3(256), 0, s, a);
  }
  return fz_status();
}

extern "C" int aac_silu_mul(const void* gate_up, void* out, int64_t n_rows, int32_t intermediate,
                            int32_t dtype, void* stream) {
  Dt dt;
  if (!fz_dtype(dtype, &dt)) return AAC_ERR_UNSUPPORTED;
  if (n_rows < 0 || intermediate <= 0) return AAC_ERR_INVALID_ARGUMENT;
  if (intermediate % 8) return AAC_ERR_UNSUPPORTED;
  if (n_rows == 0) return AAC_OK;
  if (!gate_up || !out) return AAC_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)gate_up | (uintptr_t)out) % 16) return AAC_ERR_MISALIGNED;
  const dim3 grid((unsigned)cdiv(n_rows * (intermediate / 8), 256));
  hipStream_t s = (hipStream_t)stream;
  if (dt == Dt::BF16)
    hipLaunchKernelGGL((fz::silu_mul_kernel<Dt::BF16>), grid, dim3(256), 0, s,
                       (const u16*)gate_up, (u16*)out, n_rows, intermediate);
  else
    hipLaunchKernelGGL((fz::silu_mul_kernel<Dt::FP16>), grid, dim3(256), 0, s,
                       (const u16*)gate_up, (u16*)out, n_rows, intermediate);
  return fz_status();
}

extern "C" int aac_argmax_rows(const void* x, int64_t row_stride, int64_t n_rows, int64_t n_cols,
                               int64_t* out, int32_t dtype, void* stream) {
  if (dtype != AAC_DTYPE_BF16 && dtype != AAC_DTYPE_FP16 && dtype != AAC_DTYPE_FP32)
    return AAC_ERR_UNSUPPORTED;
  if (n_rows < 0 || n_cols <= 0 || row_stride < n_cols) return AAC_ERR_INVALID_ARGUMENT;
  if (n_cols >= 0x7fffffff || n_rows >= 0x7fffffff) return AAC_ERR_UNSUPPORTED;
  if (n_rows == 0) return AAC_OK;
  if (!x || !out) return AAC_ERR_INVALID_ARGUMENT;
  if ((uintptr_t)x % (dtype == AAC_DTYPE_FP32 ? 4 : 2)) return AAC_ERR_MISALIGNED;
  const dim3 grid((unsigned)n_rows);
  hipStream_t s = (hipStream_t)stream;
  const int cols = (int)n_cols;
  if (dtype == AAC_DTYPE_BF16)
    hipLaunchKernelGGL((fz::argmax_kernel<Dt::BF16>), grid, dim3(1024), 0, s, x, row_stride, cols, out);
  else if (dtype == AAC_DTYPE_FP16)
    hipLaunchKernelGGL((fz::argmax_kernel<Dt::FP16>), grid, dim3(1024), 0, s, x, row_stride, cols, out);
  else
    hipLaunchKernelGGL((fz::argmax_kernel<Dt::FP32>), grid, dim3(1024), 0, s, x, row_stride, cols, out);
  return fz_status();
}
