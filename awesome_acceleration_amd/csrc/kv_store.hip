// KV-cache store kernels (gfx950).
//
// Prefill store: a row scatter of k/v token rows into the flat cache rows
// named by slot_mapping -- the reference's
//   kv_flat.index_copy_(0, scatter_indices, k); v_flat.index_copy_(...)
// (llm.py:171-174).  Decode append: the same copy with the destination row
// computed from (block_tables, cache_seqlens), the k=/v= half of
// flash_attn_with_kvcache (model/model.py:233-240).
//
// The copy is pure data movement (bit-exact).  One wavefront moves one token:
// its K row and V row (n_kv_heads * head_dim elements each, 2 KiB for the
// Qwen3 shape in bf16) with VEC-byte vector loads, all loads of a row issued
// before the first store so a wave keeps 4 KiB in flight.  A row is
// contiguous in the source (head stride == head_dim) even when the token
// stride is not (v is a view of the fused qkv buffer).

#include "aac_common.h"

namespace aac {

template <int VEC> struct VecT;
template <> struct VecT<16> { typedef u32x4 T; };
template <> struct VecT<8> { typedef u32x2 T; };
template <> struct VecT<4> { typedef u32 T; };
template <> struct VecT<2> { typedef u16 T; };

struct StoreArgs {
  const char* k;
  const char* v;
  int64_t k_stride;  // bytes between source tokens
  int64_t v_stride;
  char* kc;
  char* vc;
  int64_t row_bytes;  // n_kv_heads * head_dim * elem_bytes
  int64_t n_tokens;
  // explicit slots
  const int64_t* slot_mapping;
  int64_t num_rows;
  // paged append
  const int32_t* block_tables;
  const int32_t* seqlens;
  int64_t num_blocks;
  int32_t block_size;
  int32_t max_blocks;
};

template <int VEC, bool PAGED>
__global__ __launch_bounds__(256) void kv_store_kernel(StoreArgs a) {
  typedef typename VecT<VEC>::T V;
  constexpr int kMaxIt = 4;  // rows up to 4 * 64 * VEC bytes keep all loads in flight
  const int lane = threadIdx.x & 63;
  const int64_t wstride = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < a.n_tokens; t += wstride) {
    int64_t row;
    if (PAGED) {
      const int p = a.seqlens[t];
      if (p < 0 || (int64_t)p >= (int64_t)a.max_blocks * a.block_size) continue;
      const int blk = a.block_tables[t * a.max_blocks + p / a.block_size];
      if (blk < 0 || blk >= a.num_blocks) continue;
      row = (int64_t)blk * a.block_size + p % a.block_size;
    } else {
      row = a.slot_mapping[t];
      if (row < 0 || row >= a.num_rows) continue;
    }
    const char* ks = a.k + t * a.k_stride;
    const char* vs = a.v + t * a.v_stride;
    char* kd = a.kc + row * a.row_bytes;
    char* vd = a.vc + row * a.row_bytes;
    for (int64_t base = 0; base < a.row_bytes; base += (int64_t)kMaxIt * 64 * VEC) {
      V kr[kMaxIt], vr[kMaxIt];
#pragma unroll
      for (int i = 0; i < kMaxIt; ++i) {
        const int64_t off = base + ((int64_t)i * 64 + lane) * VEC;
        if (off < a.row_bytes) {
          kr[i] = *reinterpret_cast<const V*>(ks + off);
          vr[i] = *reinterpret_cast<const V*>(vs + off);
        }
      }
#pragma unroll
      for (int i = 0; i < kMaxIt; ++i) {
        const int64_t off = base + ((int64_t)i * 64 + lane) * VEC;
        if (off < a.row_bytes) {
          *reinterpret_cast<V*>(kd + off) = kr[i];
          *reinterpret_cast<V*>(vd + off) = vr[i];
        }
      }
    }
  }
}

static int elem_bytes(int32_t dtype) {
  switch (dtype) {
    case AAC_DTYPE_BF16:
    case AAC_DTYPE_FP16:
      return 2;
    case AAC_DTYPE_FP32:
      return 4;
    default:
      return 0;
  }
}

template <bool PAGED>
static int launch_store(const StoreArgs& a, hipStream_t stream) {
  if (a.n_tokens == 0) return AAC_OK;
  auto al = [&](int v) {
    return ((uintptr_t)a.k % v) == 0 && ((uintptr_t)a.v % v) == 0 && ((uintptr_t)a.kc % v) == 0 &&
           ((uintptr_t)a.vc % v) == 0 && (a.k_stride % v) == 0 && (a.v_stride % v) == 0 &&
           (a.row_bytes % v) == 0;
  };
  int64_t blocks = cdiv(a.n_tokens, 4);
  if (blocks > 65536) blocks = 65536;
  dim3 grid((unsigned)blocks), block(256);
  if (al(16))
    hipLaunchKernelGGL((kv_store_kernel<16, PAGED>), grid, block, 0, stream, a);
  else if (al(8))
    hipLaunchKernelGGL((kv_store_kernel<8, PAGED>), grid, block, 0, stream, a);
  else if (al(4))
    hipLaunchKernelGGL((kv_store_kernel<4, PAGED>), grid, block, 0, stream, a);
  else if (al(2))
    hipLaunchKernelGGL((kv_store_kernel<2, PAGED>), grid, block, 0, stream, a);
  else
    return AAC_ERR_MISALIGNED;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}

}  // namespace aac

using namespace aac;

extern "C" int aac_kv_store(const void* k, const void* v, int64_t k_tok_stride,
                            int64_t v_tok_stride, void* k_cache, void* v_cache,
                            int64_t num_cache_rows, const int64_t* slot_mapping, int64_t n_tokens,
                            int32_t n_kv_heads, int32_t head_dim, int32_t dtype, void* stream) {
  const int es = elem_bytes(dtype);
  if (!es) return AAC_ERR_UNSUPPORTED;
  if (n_tokens < 0 || n_kv_heads <= 0 || head_dim <= 0 || num_cache_rows < 0 ||
      k_tok_stride < 0 || v_tok_stride < 0)
    return AAC_ERR_INVALID_ARGUMENT;
  if (n_tokens == 0) return AAC_OK;
  if (!k || !v || !k_cache || !v_cache || !slot_mapping) return AAC_ERR_INVALID_ARGUMENT;
  if (k_tok_stride < (int64_t)n_kv_heads * head_dim || v_tok_stride < (int64_t)n_kv_heads * head_dim)
    return AAC_ERR_SHAPE;
  StoreArgs a = {};
  a.k = (const char*)k;
  a.v = (const char*)v;
  a.k_stride = k_tok_stride * es;
  a.v_stride = v_tok_stride * es;
  a.kc = (char*)k_cache;
  a.vc = (char*)v_cache;
  a.row_bytes = (int64_t)n_kv_heads * head_dim * es;
  a.n_tokens = n_tokens;
  a.slot_mapping = slot_mapping;
  a.num_rows = num_cache_rows;
  return launch_store<false>(a, (hipStream_t)stream);
}

extern "C" int aac_kv_append_paged(const void* k, const void* v, int64_t k_tok_stride,
                                   int64_t v_tok_stride, void* k_cache, void* v_cache,
                                   int64_t num_blocks, int32_t block_size,
                                   const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int32_t* cache_seqlens, int32_t n_seqs,
                                   int32_t n_kv_heads, int32_t head_dim, int32_t dtype,
                                   void* stream) {
  const int es = elem_bytes(dtype);
  if (!es) return AAC_ERR_UNSUPPORTED;
  if (n_seqs < 0 || n_kv_heads <= 0 || head_dim <= 0 || num_blocks < 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0 || k_tok_stride < 0 || v_tok_stride < 0)
    return AAC_ERR_INVALID_ARGUMENT;
  if (n_seqs == 0) return AAC_OK;
  if (!k || !v || !k_cache || !v_cache || !block_tables || !cache_seqlens)
    return AAC_ERR_INVALID_ARGUMENT;
  if (k_tok_stride < (int64_t)n_kv_heads * head_dim || v_tok_stride < (int64_t)n_kv_heads * head_dim)
    return AAC_ERR_SHAPE;
  StoreArgs a = {};
  a.k = (const char*)k;
  a.v = (const char*)v;
  a.k_stride = k_tok_stride * es;
  a.v_stride = v_tok_stride * es;
  a.kc = (char*)k_cache;
  a.vc = (char*)v_cache;
  a.row_bytes = (int64_t)n_kv_heads * head_dim * es;
  a.n_tokens = n_seqs;
  a.block_tables = block_tables;
  a.seqlens = cache_seqlens;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.max_blocks = max_blocks_per_seq;
  return launch_store<true>(a, (hipStream_t)stream);
}
