// Per-head q/k RMSNorm + RoPE + KV store of one token, shared by the fused
// call-site kernels (csrc/fused.hip) and the QKV projection's epilogue
// (csrc/gemm.hip): the arithmetic of model/model.py:47-52 and :86-99 with
// the reference's rounding points, and the K/V destination row of the
// llm.py:171-174 store or the model/model.py:233-240 decode append.
#pragma once

#include "aac_common.h"

namespace aac {

constexpr int kHeadDimFused = 128;

namespace fz {

template <Dt DT> struct Cvt;
template <> struct Cvt<Dt::BF16> {
  __device__ static inline float lo(u32 w) { return bf16lo(w); }
  __device__ static inline float hi(u32 w) { return bf16hi(w); }
  __device__ static inline u32 pack(float a, float b) { return pack_bf16x2(a, b); }
  __device__ static inline float round(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }
};
template <> struct Cvt<Dt::FP16> {
  __device__ static inline float lo(u32 w) { return f16lo(w); }
  __device__ static inline float hi(u32 w) { return f16hi(w); }
  __device__ static inline u32 pack(float a, float b) { return pack_f16x2(a, b); }
  __device__ static inline float round(float x) { return (float)(_Float16)x; }
};

template <Dt DT>
__device__ __forceinline__ void unpack8(const u32x4& w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = Cvt<DT>::lo(w[i]);
    f[2 * i + 1] = Cvt<DT>::hi(w[i]);
  }
}
template <Dt DT>
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = Cvt<DT>::pack(f[2 * i], f[2 * i + 1]);
  return w;
}

// ------------------------------------------------- q/k RMSNorm + RoPE + store
struct QkArgs {
  const u16* qkv;
  int64_t qkv_stride;  // elements between tokens
  int64_t n_tokens;
  int32_t hq, hkv;
  const u16* qw;  // q_norm weight [128]
  const u16* kw;  // k_norm weight [128]
  float eps;
  const u16* cos;  // [max_pos, 128]
  const u16* sin;
  const int32_t* positions;  // [T]
  int32_t max_pos;
  u16* q_out;  // [T, hq, 128]
  u16* k_out;  // [T, hkv, 128] or null
  u16* k_cache;
  u16* v_cache;  // rows [*, hkv, 128]; null: no store
  const int64_t* slot_mapping;  // explicit rows, or null: paged append
  int64_t num_rows;
  const int32_t* block_tables;
  int32_t max_blocks;
  const int32_t* cache_seqlens;  // append position of token t (= sequence t)
  int32_t block_size;
  int64_t num_blocks;
};

// Destination cache row of token t for the K/V store, or -1 (none or out of range).
__device__ __forceinline__ int64_t cache_row(const QkArgs& a, int64_t t) {
  int64_t crow = -1;
  if (a.v_cache == nullptr) return crow;
  if (a.slot_mapping != nullptr) {
    crow = a.slot_mapping[t];
    if (crow >= a.num_rows) crow = -1;
  } else {
    const int p = a.cache_seqlens[t];
    if (p >= 0 && (int64_t)p < (int64_t)a.max_blocks * a.block_size) {
      const int blk = a.block_tables[t * a.max_blocks + p / a.block_size];
      if (blk >= 0 && blk < a.num_blocks) crow = (int64_t)blk * a.block_size + p % a.block_size;
    }
  }
  return crow;
}

// One head row of token t, held by the 16 lanes of a DPP row (lane li owns
// dims [8li, 8li+8)): a value head is copied into the cache; a query or key
// head gets RMSNorm over the head (model/model.py:47-52) and RoPE, out =
// x*cos + rotate_half(x)*sin with each product and the sum rounded
// (model/model.py:90-99); rotate_half pairs dim d with d +- 64, i.e. lane li
// with lane li ^ 8 (DPP row_ror:8).  The caller keeps the row's 16 lanes
// together on every branch.
template <Dt DT>
__device__ __forceinline__ void norm_rope_head(const QkArgs& a, int64_t t, int hh, int li,
                                               const u32x4& xr, int64_t crow, const float* wf,
                                               const float* cf, const float* sf) {
  // Each product and the sum are rounded separately; for fp16 those rounds
  // become half-precision operations, which contraction would merge into one
  // fused multiply-add (a single rounding, unlike the torch expression).
#pragma clang fp contract(off)
  if (hh >= a.hq + a.hkv) {  // value head
    if (crow >= 0)
      *reinterpret_cast<u32x4*>(a.v_cache + (crow * a.hkv + (hh - a.hq - a.hkv)) * kHeadDimFused +
                                li * 8) = xr;
    return;
  }
  float x[8];
  unpack8<DT>(xr, x);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
  ss = row16_sum(ss);
  const float rs = __frsqrt_rn(ss / (float)kHeadDimFused + a.eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = Cvt<DT>::round(wf[i] * Cvt<DT>::round(x[i] * rs));
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float partner = __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(x[i]), 0x128, 0xF, 0xF, false));
    const float rot = li < 8 ? -partner : partner;
    o[i] = Cvt<DT>::round(Cvt<DT>::round(x[i] * cf[i]) + Cvt<DT>::round(rot * sf[i]));
  }
  const u32x4 packed = pack8<DT>(o);
  if (hh < a.hq) {
    *reinterpret_cast<u32x4*>(a.q_out + (t * a.hq + hh) * kHeadDimFused + li * 8) = packed;
  } else {
    const int kh = hh - a.hq;
    if (a.k_out != nullptr)
      *reinterpret_cast<u32x4*>(a.k_out + (t * a.hkv + kh) * kHeadDimFused + li * 8) = packed;
    if (crow >= 0)
      *reinterpret_cast<u32x4*>(a.k_cache + (crow * a.hkv + kh) * kHeadDimFused + li * 8) = packed;
  }
}

__device__ __forceinline__ int clamp_pos(const QkArgs& a, int p) {
  return p < 0 ? 0 : (p >= a.max_pos ? a.max_pos - 1 : p);
}

}  // namespace fz
}  // namespace aac
