// Definitions shared by the two varlen prefill kernels (prefill.hip: eight
// waves of one 32-query column each; prefill_wide.hip: four waves of two
// columns each): tile geometry, kernel arguments, the MFMA wrappers and the
// V^T tile layout.
#pragma once

#include "aac_common.h"

namespace aac {
namespace pf {

constexpr int D = 128;
constexpr int BKV = 64;        // keys per LDS tile (two 32-key sub-tiles)
constexpr int KPITCH = D + 8;  // K tile row pitch (elements): 8 consecutive rows hit 8 disjoint bank quads
constexpr int OPITCH = D + 8;  // output staging row pitch (elements)
constexpr int STAGES = 3;      // LDS ring: one barrier per tile (see the hazard note in the kernel)
constexpr float kRescale = 8.f;  // lazy-rescale threshold (log2 units): p <= 256

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
  int32_t n_qblocks;  // q-blocks of the longest segment
  int32_t chunk_segs; // segments per item chunk (wide kernel: items are numbered chunk by chunk)
  int32_t max_k;      // max_seqlen_k: bounds every segment's key count
  // KV-cache store in the same kernel (self-attention, cu_q == cu_k): token
  // t's K/V rows go to cache row slots[t] of the [num_rows, hkv, D] caches
  u16* kc;
  u16* vc;
  const int64_t* slots;
  int64_t num_rows;
  int32_t n_tok;  // k/v tokens the store covers
  // Split keys (SPLIT): every item's key tiles are cut into up to n_split
  // pieces, worked on by different workgroups; each piece leaves its
  // unnormalised accumulators and (m, l) per lane in the workspace, and the
  // last piece of an item to finish merges them (ws_cnt counts finished
  // pieces and is reset to zero by the merging piece).
  int32_t n_split;
  float* ws_o;     // [item][piece][wave][16 float4][64 lanes]
  float2* ws_ml;   // [item][piece][wave][64 lanes]: reference max, lane-partial sum
  int32_t* ws_cnt; // [item]
};

template <bool F16> struct Mfma;
template <> struct Mfma<false> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline u32 pack(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) float f2;
    return __builtin_bit_cast(u32, __builtin_convertvector((f2){a, b}, bf16x2));
  }
  __device__ static inline float dot2_ones(u32 x, float acc) {  // acc + x.lo + x.hi
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x),
                                           __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
  }
};
template <> struct Mfma<true> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline u32 pack(float a, float b) { return pack_f16x2(a, b); }
  __device__ static inline float dot2_ones(u32 x, float acc) {  // acc + x.lo + x.hi
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, 0x3c003c00u),
                                  acc, false);
  }
};


// V^T tile layout: 128 rows (dims) x 64 keys, no padding.  Keys are handled
// in quads (4 keys = 8 bytes).  Inside each 16-key group the quad order is
// (0,2,1,3) so that the 8 keys one lane half feeds to an MFMA (keys
// 4h..4h+3 and 8+4h..8+4h+3 of the group) are one contiguous 16-byte octet;
// the 8 octets of a row are XOR-swizzled by (row ^ row>>3) & 7 so that both
// the b128 reads (8 consecutive rows, same octet) and the b64 writes (rows
// 8*i + c, same quad) spread over the banks.
__device__ __forceinline__ int vt_quad_off(int row, int quad) {
  const int g = quad >> 2, qq = quad & 3;
  const int pq = (g << 2) | ((qq & 1) << 1) | (qq >> 1);
  const int oct = (pq >> 1) ^ ((row ^ (row >> 3)) & 7);
  return row * BKV + oct * 8 + (pq & 1) * 4;
}
// element offset of the octet holding keys {16*g + 4*hl + 0..3, 16*g + 8 + 4*hl + 0..3}
__device__ __forceinline__ int vt_octet_off(int row, int g, int hl) {
  return row * BKV + (((2 * g + hl) ^ ((row ^ (row >> 3)) & 7)) * 8);
}


__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// The kernel's arguments read from the kernel-argument segment where they are
// used: the empty asm hides the pointer's origin, so the compiler keeps none
// of the fields in SGPRs through the tile loop (the store's fields are needed
// only after it).
typedef const Args __attribute__((address_space(4))) KArgs;
__device__ __forceinline__ KArgs* kernel_args() {
  KArgs* p = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return p;
}

// KV-cache store of tokens [t0, t1) (clamped to the n_tok stored tokens) for
// KV heads [h0, h1): token t's K and V rows to cache row slots[t] (rows with a
// slot outside [0, num_rows) are skipped).  16 threads per 256-byte row, NT
// threads of the workgroup take NT / 16 rows per pass.
template <int NT>
__device__ __forceinline__ void store_kv_span(const Args& a, int tid, int64_t t0, int64_t t1, int h0,
                                              int h1) {
  KArgs* sa = kernel_args();
  t0 = max(t0, (int64_t)0);
  t1 = min(t1, (int64_t)sa->n_tok);
  const int nh = h1 - h0;
  const int64_t n = t1 > t0 ? (t1 - t0) * nh : 0;
  for (int64_t r = tid >> 4; r < n; r += NT / 16) {
    // the lane's dims, opaque here so that no address is hoisted out of this
    // rare loop into registers held through the whole kernel
    int dim = (tid & 15) * 8;
    asm volatile("" : "+v"(dim));
    const int64_t tok = t0 + r / nh;
    const int hh = h0 + (int)(r % nh);
    const int64_t sl = sa->slots[tok];
    const u32x4 kx = *reinterpret_cast<const u32x4*>(a.k + tok * a.k_stride + hh * D + dim);
    const u32x4 vx = *reinterpret_cast<const u32x4*>(a.v + tok * a.v_stride + hh * D + dim);
    if ((uint64_t)sl < (uint64_t)sa->num_rows) {
      const int64_t dst = (sl * a.hkv + hh) * D + dim;
      *reinterpret_cast<u32x4*>(sa->kc + dst) = kx;
      *reinterpret_cast<u32x4*>(sa->vc + dst) = vx;
    }
  }
}

}  // namespace pf
}  // namespace aac
