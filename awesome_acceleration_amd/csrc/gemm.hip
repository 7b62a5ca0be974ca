// Decode-batch projection GEMM (gfx950, bf16/fp16 MFMA): Y = X W^T with X the
// [M, K] activations of one decode step (M = running sequences, at most a few
// hundred) and W a torch Linear weight [N, K] -- the QKV, o_proj, gate_up and
// down projections of the Qwen3 layer (model/model.py:132-154, :258, :178-188).
// With `silu_intermediate` = I the weight is the fused [gate | up] projection
// [2I, K] and the epilogue writes silu(gate) * up [M, I] (model/model.py:188),
// rounded where the unfused torch expression rounds.
//
// Why a hand-written kernel: at M = 256 these GEMMs are weight-streaming
// bound (QKV: 8 MiB of weights against 2.1 GFLOP), and the library's tiles for
// this shape leave most CUs idle while a few stream long K ranges.  Here the
// output is cut into tiles so that every CU gets one (or a few), and the K
// range of a tile can be split over the workgroup's waves (reduced through
// LDS at the end).
//
// Tiling: a workgroup is 4 or 8 waves; wave (wm, wn, ks) owns the 32 x 32
// output block (rows 32 wm, columns 32 wn) for the K slice ks of every staged
// stage.  MW x NW x KS = 4 or 8.  One stage holds KT = 64 KF KS columns of K
// (each wave takes 64 KF of them: 4 KF MFMA steps) for the workgroup's 32 MW
// X rows and 32 NW (x2 with the gate/up pairing) W rows.  The MFMA computes
// D = W_blk X_blk^T (v_mfma_f32_32x32x16: A = 32 W rows x 16 k, B = 16 k x 32
// X rows), so a lane ends with one token (column of D) and 4 runs of 4
// consecutive output features: 8-byte stores.
//
// Staging: global memory goes straight into LDS (global_load_lds_dwordx4,
// 1 KiB per wave instruction, no registers and no ds_write), three stages
// deep.  Each stage buffer holds unpadded rows whose 16-byte chunks are
// XOR-swizzled by the row (chunk c of row r at c ^ (r & 15)): a load
// instruction fills 1 KiB of consecutive positions, and the MFMA fragment
// reads (32 rows, one chunk) still spread over all banks.  Measured against
// the same tiles staged through registers and ds_write: 9-17% faster.
//
// Tiles are numbered so that the M-tiles of one N-tile are consecutive and
// land on one XCD (workgroups are dealt round-robin over the 8 XCDs), so a
// W tile is fetched from HBM once per XCD and re-read from that XCD's L2.

#include "qk_head.h"

namespace aac {
namespace gm {

struct Args {
  const u16* x;
  const u16* w;
  u16* y;
  int64_t x_stride, w_stride, y_stride;  // row strides (elements)
  int32_t m, k;
  int32_t n_tiles;   // tiles along the output columns
  int32_t silu_off;  // gate/up pairing: W row of up column 0 (= I)
  fz::QkArgs qk;     // QKV epilogue: q/k norm + RoPE, q out, K/V to the cache
};

template <bool F16> struct Mma;
template <> struct Mma<false> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline float round(float f) { return bf16lo(f32_to_bf16_bits(f)); }
  __device__ static inline u32 pack(float a, float b) { return pack_bf16x2(a, b); }
};
template <> struct Mma<true> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline float round(float f) { return (float)(_Float16)f; }
  __device__ static inline u32 pack(float a, float b) { return pack_f16x2(a, b); }
};

template <int MW, int NW, int KS, int KF, bool SILU, bool F16, bool QK = false>
__global__ __launch_bounds__(64 * MW * NW * KS) void gemm_kernel(Args a) {
  constexpr int NB = SILU ? 2 : 1;        // accumulators per wave (gate, up)
  constexpr int MT = 32 * MW;             // X rows per tile
  constexpr int WT = 32 * NW * NB;        // W rows per tile
  constexpr int R = MT + WT;              // staged rows
  constexpr int KW = 64 * KF;             // K per wave per stage (4 KF MFMA steps)
  constexpr int KT = KW * KS;             // K per stage
  constexpr int C = KT / 8;               // 16-byte chunks per staged row
  static_assert(MW * NW * KS == 4 || MW * NW * KS == 8, "four or eight waves");
  static_assert((KS - 1) * MW * NW * NB * 16 * 64 * 4 <= R * KT * 2, "reduction fits");
  typedef Mma<F16> M;

  // direct-to-LDS staging: three stage buffers (separate LDS objects, so the
  // compiler can tell which loads fill which buffer), rows unpadded, the
  // 16-byte chunk c of row r at position c ^ (r & 15)
  constexpr int SB = R * KT;
  __shared__ __attribute__((aligned(16))) u16 sb0[SB];
  __shared__ __attribute__((aligned(16))) u16 sb1[SB];
  __shared__ __attribute__((aligned(16))) u16 sb2[SB];
  u16* const lds = sb0;  // the epilogue's scratch

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % MW, wn = (wave / MW) % NW, ks = wave / (MW * NW);

  const int n_mt = (a.m + MT - 1) / MT;
  const int T = n_mt * a.n_tiles;
  int t = blockIdx.x;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  const int mt = t % n_mt, nt = t / n_mt;
  const int m0 = mt * MT, n0 = nt * 32 * NW;  // first token / output column

  constexpr int NWV = MW * NW * KS;
  constexpr int IPW = R * C / (64 * NWV);  // 1 KiB loads per wave per stage
  static_assert(R * C % (64 * NWV) == 0 && C >= 16, "whole 1 KiB loads, 16-chunk swizzle");
  // load i of this wave fills positions (wave IPW + i) * 64 + lane of the
  // stage: row g / C, position g % C, i.e. chunk (g % C) ^ (row & 15)
  const u16* dsrc[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int g = (wave * IPW + i) * 64 + lane;
    const int r = g / C, ch = (g % C) ^ (r & 15);
    if (r < MT) {
      dsrc[i] = a.x + (int64_t)min(m0 + r, a.m - 1) * a.x_stride + ch * 8;
    } else {
      const int wr = r - MT;
      const int row = SILU && wr >= 32 * NW ? a.silu_off + n0 + wr - 32 * NW : n0 + wr;
      dsrc[i] = a.w + (int64_t)row * a.w_stride + ch * 8;
    }
  }
  const int nk = a.k / KT;
  // The 16-byte-per-lane LDS load is issued as inline assembly: the
  // compiler then neither counts it nor guards later LDS reads with waits
  // for it (it cannot tell which buffer it fills); the waits are explicit.
  // M0 (the LDS destination) is a reserved register the compiler does not
  // track through a clobber; nothing else in these kernels uses it (no LDS
  // builtins, readlane-by-M0, movrel or messages), so each load sets it.
  typedef __attribute__((address_space(3))) u16 lds_u16;
  auto issue = [&](u16* buf, int stage) {
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const u32 dst = (u32)(uintptr_t)(lds_u16*)(buf + (wave * IPW + i) * 512);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                   :
                   : "v"(dsrc[i] + stage * KT), "s"(dst)
                   : "memory", "m0");
#pragma clang diagnostic pop
    }
  };

  f32x16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[nb][i] = 0.f;

  // fragment reads: lane = (row l%32, 8 k at 8*(l/32)); rows are multiples
  // of 16 apart from l%32, so the swizzle term is l & 15
  const int l15 = lane & 15;
  const int fx = (32 * wm + (lane & 31)) * KT;
  const int fw = (MT + 32 * wn + (lane & 31)) * KT;
  const int c0 = KW * ks / 8 + (lane >> 5);
  auto compute = [&](const u16* buf) {
#pragma unroll
    for (int s = 0; s < 4 * KF; ++s) {
      const int off = ((c0 + 2 * s) ^ l15) << 3;
      const u32x4 bx = *reinterpret_cast<const u32x4*>(buf + fx + off);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const u32x4 aw = *reinterpret_cast<const u32x4*>(buf + fw + nb * 32 * NW * KT + off);
        acc[nb] = M::run(aw, bx, acc[nb]);
      }
    }
  };
  // Stage s sits in buffer s % 3.  Before the barrier of stage s every wave
  // waits for its own loads of s (those of s + 1 may still be in flight);
  // after it the loads of s + 2 go into the buffer of s - 1, whose readers
  // all passed the barrier.  The barrier is the bare instruction between
  // compiler-only fences: the full __syncthreads fence would also wait for
  // the loads of s + 1.
  auto step = [&](u16* cur, u16* nxt, int s) {
    if (s + 1 < nk) {
      constexpr int n = IPW;
      __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (s + 2 < nk) issue(nxt, s + 2);
    compute(cur);
  };
  issue(sb0, 0);
  if (nk > 1) issue(sb1, 1);
  int kk = 0;
  for (; kk + 3 <= nk; kk += 3) {
    step(sb0, sb2, kk);
    step(sb1, sb0, kk + 1);
    step(sb2, sb1, kk + 2);
  }
  if (kk < nk) step(sb0, sb2, kk);
  if (kk + 1 < nk) step(sb1, sb0, kk + 1);

  // K-split waves hand their partial sums to the ks = 0 wave of their block
  if (KS > 1) {
    float* red = reinterpret_cast<float*>(lds);
    const int slot = wm + MW * wn;
    __syncthreads();  // every wave is done with the stage buffers
    if (ks > 0) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          red[((((ks - 1) * MW * NW + slot) * NB + nb) * 16 + i) * 64 + lane] = acc[nb][i];
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int j = 0; j < KS - 1; ++j)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            acc[nb][i] += red[(((j * MW * NW + slot) * NB + nb) * 16 + i) * 64 + lane];
    } else if (!QK) {
      return;
    }
  }

  if constexpr (QK) {
    // The tile is one head (128 columns) of 32 tokens: the ks = 0 waves write
    // it, rounded, to LDS (after the reduction's floats), then each of the
    // 32 DPP rows of the 8 waves takes one token and runs the per-head q/k
    // RMSNorm + RoPE + store of the fused call-site kernel on it.
    static_assert(MW == 1 && NW == 4 && KS == 2 && !SILU, "one head of 32 tokens on 8 waves");
    constexpr int TP = 128 + 8;  // tile row pitch (elements)
    constexpr int kRedElems = 2 * (KS - 1) * MW * NW * 16 * 64;  // the floats, in u16 units
    static_assert(kRedElems + 32 * TP <= SB, "tile fits");
    u16* tile = lds + kRedElems;
    if (ks == 0) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 o;
        o[0] = M::pack(acc[0][4 * g], acc[0][4 * g + 1]);
        o[1] = M::pack(acc[0][4 * g + 2], acc[0][4 * g + 3]);
        *reinterpret_cast<u32x2*>(tile + (lane & 31) * TP + 32 * wn + 8 * g + 4 * (lane >> 5)) = o;
      }
    }
    __syncthreads();
    constexpr Dt DT = F16 ? Dt::FP16 : Dt::BF16;
    const fz::QkArgs& q = a.qk;
    const int r = wave * 4 + (lane >> 4), li = lane & 15;  // token row, 8 dims at 8 li
    const int64_t t = m0 + r;
    if (t >= a.m) return;  // the whole 16-lane row
    const u32x4 xr = *reinterpret_cast<const u32x4*>(tile + r * TP + li * 8);
    const int hh = nt;  // head of this tile: q heads, then k heads, then v heads
    const int64_t crow = fz::cache_row(q, t);
    float wf[8], cf[8], sf[8];
    if (hh < q.hq + q.hkv) {
      const int p = fz::clamp_pos(q, q.positions[t]);
      fz::unpack8<DT>(*reinterpret_cast<const u32x4*>((hh < q.hq ? q.qw : q.kw) + li * 8), wf);
      fz::unpack8<DT>(*reinterpret_cast<const u32x4*>(q.cos + (int64_t)p * kHeadDimFused + li * 8), cf);
      fz::unpack8<DT>(*reinterpret_cast<const u32x4*>(q.sin + (int64_t)p * kHeadDimFused + li * 8), sf);
    }
    fz::norm_rope_head<DT>(q, t, hh, li, xr, crow, wf, cf, sf);
    return;
  }

  const int m = m0 + 32 * wm + (lane & 31);
  if (m >= a.m) return;
  u16* yr = a.y + (int64_t)m * a.y_stride + n0 + 32 * wn + 4 * (lane >> 5);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (SILU) {
        // torch rounds the gate_up product, then F.silu, then the product
        const float gt = M::round(acc[0][4 * g + j]);
        const float up = M::round(acc[NB - 1][4 * g + j]);
        const float s = M::round(gt / (1.f + __expf(-gt)));
        v[j] = s * up;
      } else {
        v[j] = acc[0][4 * g + j];
      }
    }
    u32x2 o;
    o[0] = M::pack(v[0], v[1]);
    o[1] = M::pack(v[2], v[3]);
    *reinterpret_cast<u32x2*>(yr + 8 * g) = o;
  }
}

template <int MW, int NW, int KS, int KF, bool SILU, bool F16>
static int launch_t(Args a, int n_out, hipStream_t st) {
  constexpr int lds_bytes = 3 * (32 * MW + 32 * NW * (SILU ? 2 : 1)) * (64 * KF * KS) * 2;
  if constexpr (lds_bytes > 160 * 1024) {
    return AAC_ERR_UNSUPPORTED;  // the gate/up pairing does not fit LDS at this stage size
  } else {
    a.n_tiles = n_out / (32 * NW);
    const int grid = (int)cdiv(a.m, 32 * MW) * a.n_tiles;
    hipLaunchKernelGGL((gemm_kernel<MW, NW, KS, KF, SILU, F16>), dim3(grid),
                       dim3(64 * MW * NW * KS), 0, st, a);
    return AAC_OK;
  }
}

// The QKV projection with the q/k norm + RoPE + store epilogue: 32 tokens x
// one head per workgroup, K split over two of its 8 waves (the summation
// order of tiling 6, so q, k and v are those of the plain projection).
template <bool F16>
static void launch_qk(Args a, int heads, hipStream_t st) {
  a.n_tiles = heads;
  const int grid = (int)cdiv(a.m, 32) * heads;
  hipLaunchKernelGGL((gemm_kernel<1, 4, 2, 1, false, F16, true>), dim3(grid), dim3(512), 0, st, a);
}

template <bool SILU, bool F16>
static int launch_c(const Args& a, int cfg, int n_out, hipStream_t st) {
  switch (cfg) {
    case 1: return launch_t<2, 2, 1, 2, SILU, F16>(a, n_out, st);
    case 2: return launch_t<1, 1, 4, 1, SILU, F16>(a, n_out, st);
    case 3: return launch_t<2, 1, 2, 1, SILU, F16>(a, n_out, st);
    case 4: return launch_t<1, 2, 2, 1, SILU, F16>(a, n_out, st);
    case 5: return launch_t<2, 1, 4, 1, SILU, F16>(a, n_out, st);
    case 6: return launch_t<2, 2, 2, 1, SILU, F16>(a, n_out, st);
    default: return AAC_ERR_INVALID_ARGUMENT;
  }
}

// (MW, NW, K per stage) of each configuration id
static const int kCfg[7][3] = {{0, 0, 0},    {2, 2, 128}, {1, 1, 256}, {2, 1, 128},
                               {1, 2, 128}, {2, 1, 256}, {2, 2, 128}};

// The configuration for a shape.  Measured at m = 256 (the Qwen3-0.6B decode
// projections, HIP-graph replay, cold weights): 64 x 64 tiles on 8 waves
// (K split over two, config 6) are the fastest tiling once there are 128 or
// more of them (QKV 6.1 us, gate/up + SiLU 11.6 us); with fewer, 32 x 32
// tiles with K split over 4 waves (config 2: o_proj 6.0 us, down 7.2 us).
// Otherwise: the fewest K splits whose tile count fills the GPU (>= 256
// tiles), else the tiling with the most tiles.
static int pick_config(int m, int n_out, int k) {
  if (n_out % 64 == 0 && k % 128 == 0 && cdiv(m, 64) * (n_out / 64) >= 128) return 6;
  if (n_out % 32 == 0 && k % 256 == 0 && cdiv(m, 32) * (n_out / 32) >= 256) return 2;
  const int order[4] = {1, 3, 4, 2};
  int best = 0;
  int64_t best_tiles = -1;
  for (int c : order) {
    const int tc = 32 * kCfg[c][1];
    if (n_out % tc || k % kCfg[c][2]) continue;
    const int64_t tiles = cdiv(m, 32 * kCfg[c][0]) * (n_out / tc);
    if (tiles >= 256) return c;
    if (tiles > best_tiles) {
      best_tiles = tiles;
      best = c;
    }
  }
  return best;
}

}  // namespace gm
}  // namespace aac

using namespace aac;

extern "C" int aac_gemm_nt(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                           void* y, int64_t y_row_stride, int32_t m, int32_t n, int32_t k,
                           int32_t silu_intermediate, int32_t config, int32_t dtype, void* stream) {
  if (dtype != AAC_DTYPE_BF16 && dtype != AAC_DTYPE_FP16) return AAC_ERR_UNSUPPORTED;
  if (m < 0 || n <= 0 || k <= 0 || silu_intermediate < 0 || config < 0 || config > 6)
    return AAC_ERR_INVALID_ARGUMENT;
  const bool silu = silu_intermediate > 0;
  if (silu && silu_intermediate != n) return AAC_ERR_SHAPE;  // n = I output columns
  if (x_row_stride < k || w_row_stride < k || y_row_stride < n) return AAC_ERR_SHAPE;
  if (m == 0) return AAC_OK;
  if (!x || !w || !y) return AAC_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x | (uintptr_t)w) % 16 || (uintptr_t)y % 8 || x_row_stride % 8 ||
      w_row_stride % 8 || y_row_stride % 4)
    return AAC_ERR_MISALIGNED;
  const int cfg = config ? config : gm::pick_config(m, n, k);
  if (cfg == 0) return AAC_ERR_UNSUPPORTED;
  const int tc = 32 * gm::kCfg[cfg][1];
  if (n % tc || k % gm::kCfg[cfg][2]) return AAC_ERR_UNSUPPORTED;
  if (cdiv(m, 32 * gm::kCfg[cfg][0]) * (n / tc) >= (int64_t(1) << 31)) return AAC_ERR_UNSUPPORTED;
  gm::Args a{};
  a.x = (const u16*)x;
  a.w = (const u16*)w;
  a.y = (u16*)y;
  a.x_stride = x_row_stride;
  a.w_stride = w_row_stride;
  a.y_stride = y_row_stride;
  a.m = m;
  a.k = k;
  a.silu_off = silu_intermediate;
  a.n_tiles = 0;
  const hipStream_t st = (hipStream_t)stream;
  int rc;
  if (dtype == AAC_DTYPE_FP16)
    rc = silu ? gm::launch_c<true, true>(a, cfg, n, st) : gm::launch_c<false, true>(a, cfg, n, st);
  else
    rc = silu ? gm::launch_c<true, false>(a, cfg, n, st) : gm::launch_c<false, false>(a, cfg, n, st);
  if (rc != AAC_OK) return rc;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}

extern "C" int aac_qkv_norm_rope_store(
    const void* x, int64_t x_row_stride, const void* w_qkv, int64_t w_row_stride, int64_t n_tokens,
    int32_t hidden, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const void* cos_table,
    const void* sin_table, int32_t max_position, const int32_t* positions, void* q_out, void* k_out,
    void* k_cache, void* v_cache, int64_t num_cache_rows, const int64_t* slot_mapping,
    const int32_t* block_tables, int32_t max_blocks_per_seq, const int32_t* cache_seqlens,
    int32_t block_size, int32_t dtype, void* stream) {
  if (dtype != AAC_DTYPE_BF16 && dtype != AAC_DTYPE_FP16) return AAC_ERR_UNSUPPORTED;
  if (head_dim != kHeadDimFused) return AAC_ERR_UNSUPPORTED;
  if (n_tokens < 0 || hidden <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || max_position <= 0)
    return AAC_ERR_INVALID_ARGUMENT;
  if (hidden % 128) return AAC_ERR_UNSUPPORTED;  // whole 128-column K stages
  if (x_row_stride < hidden || w_row_stride < hidden) return AAC_ERR_SHAPE;
  if (n_tokens == 0) return AAC_OK;
  if (n_tokens >= (int64_t(1) << 31) / 32) return AAC_ERR_UNSUPPORTED;
  if (!x || !w_qkv || !q_norm_weight || !k_norm_weight || !cos_table || !sin_table || !positions ||
      !q_out)
    return AAC_ERR_INVALID_ARGUMENT;
  if (v_cache) {
    if (!k_cache) return AAC_ERR_INVALID_ARGUMENT;
    if (!slot_mapping && (!block_tables || !cache_seqlens || block_size <= 0 || max_blocks_per_seq <= 0))
      return AAC_ERR_INVALID_ARGUMENT;
  }
  if (((uintptr_t)x | (uintptr_t)w_qkv | (uintptr_t)q_out | (uintptr_t)k_out | (uintptr_t)k_cache |
       (uintptr_t)v_cache | (uintptr_t)cos_table | (uintptr_t)sin_table | (uintptr_t)q_norm_weight |
       (uintptr_t)k_norm_weight) % 16 ||
      x_row_stride % 8 || w_row_stride % 8)
    return AAC_ERR_MISALIGNED;
  gm::Args a{};
  a.x = (const u16*)x;
  a.w = (const u16*)w_qkv;
  a.y = nullptr;
  a.x_stride = x_row_stride;
  a.w_stride = w_row_stride;
  a.y_stride = 0;
  a.m = (int32_t)n_tokens;
  a.k = hidden;
  a.silu_off = 0;
  a.n_tiles = 0;
  fz::QkArgs& q = a.qk;
  q.qkv = nullptr;
  q.qkv_stride = 0;
  q.n_tokens = n_tokens;
  q.hq = n_q_heads;
  q.hkv = n_kv_heads;
  q.qw = (const u16*)q_norm_weight;
  q.kw = (const u16*)k_norm_weight;
  q.eps = eps;
  q.cos = (const u16*)cos_table;
  q.sin = (const u16*)sin_table;
  q.positions = positions;
  q.max_pos = max_position;
  q.q_out = (u16*)q_out;
  q.k_out = (u16*)k_out;
  q.k_cache = (u16*)k_cache;
  q.v_cache = (u16*)v_cache;
  q.slot_mapping = slot_mapping;
  q.num_rows = num_cache_rows;
  q.block_tables = block_tables;
  q.max_blocks = max_blocks_per_seq;
  q.cache_seqlens = cache_seqlens;
  q.block_size = block_size;
  q.num_blocks = block_size > 0 ? num_cache_rows / block_size : 0;
  const hipStream_t st = (hipStream_t)stream;
  const int heads = n_q_heads + 2 * n_kv_heads;
  if (dtype == AAC_DTYPE_FP16)
    gm::launch_qk<true>(a, heads, st);
  else
    gm::launch_qk<false>(a, heads, st);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? AAC_OK : (int)e;
}
