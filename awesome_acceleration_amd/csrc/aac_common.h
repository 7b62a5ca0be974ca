// Device helpers shared by the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/aac_attn.h"

namespace aac {

typedef unsigned int u32;
typedef unsigned short u16;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- bf16 / fp16
__device__ __forceinline__ float bf16lo(u32 w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(u32 w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ u32 f32_to_bf16_bits(float f) {
  u32 u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ u32 pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ float f16lo(u32 w) {
  return (float)__builtin_bit_cast(f16x2, w)[0];
}
__device__ __forceinline__ float f16hi(u32 w) {
  return (float)__builtin_bit_cast(f16x2, w)[1];
}
__device__ __forceinline__ u32 pack_f16x2(float lo, float hi) {
  f16x2 h;
  h[0] = (_Float16)lo;
  h[1] = (_Float16)hi;
  return __builtin_bit_cast(u32, h);
}

// Element-type traits: how 8 consecutive elements are loaded, unpacked to
// fp32 and how fp32 values are packed back.
enum class Dt { BF16, FP16, FP32 };

template <Dt D> struct Elem;
template <> struct Elem<Dt::BF16> {
  static constexpr int kBytes = 2;
  __device__ static inline void unpack8(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16lo(w[i]);
      f[2 * i + 1] = bf16hi(w[i]);
    }
  }
  __device__ static inline u32 pack2(float a, float b) { return pack_bf16x2(a, b); }
  // hardware round-to-nearest-even pack (v_cvt_pk_bf16_f32)
  __device__ static inline u32 pack2_hw(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) float f2;
    return __builtin_bit_cast(u32, __builtin_convertvector((f2){a, b}, bf16x2));
  }
  // acc + x.lo * y.lo + x.hi * y.hi in fp32 (v_dot2_f32_bf16)
  __device__ static inline float dot2(u32 x, u32 y, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, y),
                                           acc, false);
  }
  static constexpr u32 kOnes = 0x3f803f80u;  // (1.0, 1.0)
};
template <> struct Elem<Dt::FP16> {
  static constexpr int kBytes = 2;
  __device__ static inline void unpack8(const u32x4& w, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = f16lo(w[i]);
      f[2 * i + 1] = f16hi(w[i]);
    }
  }
  __device__ static inline u32 pack2(float a, float b) { return pack_f16x2(a, b); }
  __device__ static inline u32 pack2_hw(float a, float b) { return pack_f16x2(a, b); }
  // acc + x.lo * y.lo + x.hi * y.hi in fp32 (v_dot2_f32_f16)
  __device__ static inline float dot2(u32 x, u32 y, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, y), acc,
                                  false);
  }
  static constexpr u32 kOnes = 0x3c003c00u;  // (1.0, 1.0)
};
template <> struct Elem<Dt::FP32> {
  static constexpr int kBytes = 4;
};

// byte-select masks for v_perm_b32(hi_src, lo_src, sel) on 16-bit pairs
constexpr u32 kSelLo = 0x05040100u;  // (lo16 of lo_src, lo16 of hi_src)
constexpr u32 kSelHi = 0x07060302u;  // (hi16 of lo_src, hi16 of hi_src)

// ---------------------------------------------------------------- DPP
// dpp_ctrl encodings (GCN/CDNA DPP16)
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of 16 lanes (a DPP "row"); every lane of the
// row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<kDppQuadXor1>(x);
  x += dpp_f<kDppQuadXor2>(x);
  x += dpp_f<kDppRowHalfMirror>(x);
  x += dpp_f<kDppRowMirror>(x);
  return x;
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_f<kDppQuadXor1>(x));
  x = fmaxf(x, dpp_f<kDppQuadXor2>(x));
  x = fmaxf(x, dpp_f<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp_f<kDppRowMirror>(x));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// IEEE 754-2019 maximum (NaN-propagating).  Unlike fmaxf it needs no
// canonicalisation of its inputs, and chains of two fold into one
// v_maximum3_f32 on gfx950.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmax3(float a, float b, float c) { return vmax(vmax(a, b), c); }

__host__ __device__ constexpr inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- host
// Compute units of the current device (the persistent grid size), cached per
// device; a racing first query stores the same value twice.
inline int device_cu_count(int* n_cu) {
  static std::atomic<int> cache[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *n_cu = c;
      return AAC_OK;
    }
  }
  int n = 0;
  e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return (int)e;
  if (n <= 0) return AAC_ERR_UNSUPPORTED;
  if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  *n_cu = n;
  return AAC_OK;
}


}  // namespace aac
