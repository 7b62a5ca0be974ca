/*
 * aac_attn.h -- C ABI of libaac_attn.so, the MI355X (gfx950) attention hot
 * path of the Qwen3 serving engine: the slot_mapping KV-cache store, varlen
 * causal GQA prefill and paged decode.
 *
 * Conventions shared by every entry point
 *   - All tensor pointers are device pointers; every buffer is owned by the
 *     caller.  The library allocates no device memory (aac_decode_paged_noalloc
 *     uses one static device array instead of a workspace argument).
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is enqueued asynchronously; no entry point synchronises the host.
 *   - Strides are in ELEMENTS.  Within one token the [heads, head_dim] block
 *     must be contiguous (head stride == head_dim, dim stride == 1); only the
 *     token (or sequence) stride is free.  This admits the reference's v,
 *     a strided view of the fused qkv buffer with token stride
 *     (Hq + 2*Hkv) * head_dim (llm.py:156, model/model.py:222).
 *   - Caches are [num_blocks, block_size, n_kv_heads, head_dim], token-major
 *     ("NHD").  The reference's slot cache [num_slots, max_seq_len, Hkv, D]
 *     (model/model.py:324-336) is the case block_size = max_seq_len with one
 *     block per sequence (block_tables[b] = {slot_b}).
 *   - Return value: 0 on success, a negative AAC_ERR_* code for a rejected
 *     argument, or a positive hipError_t when a launch failed.  Nothing is
 *     thrown across the ABI; aac_strerror() gives the message.
 *   - Calls are stateless and reentrant, except aac_decode_paged_noalloc,
 *     whose calls share one scratch array per GPU.
 *
 * Reference interfaces replaced (reference paths are relative to the
 * yijichar/AWesome_ACceleration tree):
 *   aac_kv_store             kv_flat.index_copy_(0, scatter_indices, k)/(v)
 *                            llm.py:171-174
 *   aac_kv_append_paged      the k=/v= append half of flash_attn_with_kvcache
 *                            model/model.py:233-240
 *   aac_prefill_varlen       flash_attn_varlen_func(..., causal=True)
 *                            llm.py:178-184 (also flash_attn_func,
 *                            model/model.py:253-254, with uniform cu_seqlens)
 *   aac_prefill_varlen_store llm.py:171-184 (store + attend in one call)
 *   aac_decode_paged         the attend half of flash_attn_with_kvcache
 *                            model/model.py:233-240
 *   aac_decode_append_paged  all of flash_attn_with_kvcache(k=, v=)
 *                            model/model.py:233-240
 */
#ifndef AAC_ATTN_H
#define AAC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AAC_ABI_VERSION 2

/* element types */
enum {
  AAC_DTYPE_BF16 = 0,
  AAC_DTYPE_FP16 = 1,
  AAC_DTYPE_FP32 = 2
};

/* status codes (positive values are hipError_t) */
enum {
  AAC_OK = 0,
  AAC_ERR_INVALID_ARGUMENT = -1, /* null pointer, negative or zero size  */
  AAC_ERR_UNSUPPORTED = -2,      /* dtype / head_dim / GQA group not built */
  AAC_ERR_MISALIGNED = -3,       /* pointer or stride breaks 16-B access  */
  AAC_ERR_WORKSPACE = -4,        /* split-K workspace too small           */
  AAC_ERR_SHAPE = -5,            /* inconsistent shape arguments          */
  AAC_ERR_SCRATCH = -6           /* plan exceeds the static decode scratch */
};

/* ABI revision of the loaded library (AAC_ABI_VERSION it was built with). */
int aac_abi_version(void);

/* Message for a status code returned by any entry point (never NULL). */
const char* aac_strerror(int code);

/*
 * KV store: for t in [0, n_tokens):
 *   if slot_mapping[t] >= 0:
 *     k_cache_rows[slot_mapping[t]] = k[t];  v_cache_rows[slot_mapping[t]] = v[t]
 * where *_cache_rows views the cache as [num_cache_rows, n_kv_heads, head_dim].
 * Byte copy: the cache contents are bit-exact.  A negative slot is padding and
 * is skipped; a slot >= num_cache_rows is skipped too (never written), which the
 * reference would reject with an IndexError -- validate on the host if that
 * matters.  Duplicate slots leave an unspecified one of the rows.
 * Replaces llm.py:171-174.
 */
int aac_kv_store(const void* k, const void* v, int64_t k_tok_stride, int64_t v_tok_stride,
                 void* k_cache, void* v_cache, int64_t num_cache_rows,
                 const int64_t* slot_mapping, int64_t n_tokens, int32_t n_kv_heads,
                 int32_t head_dim, int32_t dtype, void* stream);

/*
 * Decode append: the new token of sequence b (k[b], v[b]) is written at
 * position p = cache_seqlens[b], i.e. cache row
 *   block_tables[b * max_blocks_per_seq + p / block_size] * block_size + p % block_size.
 * cache_seqlens is NOT modified (the reference's caller increments it,
 * model/model.py:241).  Positions beyond the table capacity and block ids
 * outside [0, num_blocks) are skipped.
 * Replaces the k=/v= half of flash_attn_with_kvcache (model/model.py:233-240).
 */
int aac_kv_append_paged(const void* k, const void* v, int64_t k_tok_stride, int64_t v_tok_stride,
                        void* k_cache, void* v_cache, int64_t num_blocks, int32_t block_size,
                        const int32_t* block_tables, int32_t max_blocks_per_seq,
                        const int32_t* cache_seqlens, int32_t n_seqs, int32_t n_kv_heads,
                        int32_t head_dim, int32_t dtype, void* stream);

/*
 * Varlen attention over packed segments.  Segment s owns query rows
 * [cu_seqlens_q[s], cu_seqlens_q[s+1]) and key rows
 * [cu_seqlens_k[s], cu_seqlens_k[s+1]).  Query head h reads KV head
 * h / (n_q_heads / n_kv_heads).  With causal != 0 the mask is bottom-right
 * aligned (query i sees keys j <= i + Lk - Lq); a query row that sees no key
 * gets zeros.  Softmax in fp32, output rounded to dtype.
 *   q   [Nq, n_q_heads, head_dim]  token stride q_tok_stride
 *   k,v [Nk, n_kv_heads, head_dim] token strides k_tok_stride / v_tok_stride
 *   out [Nq, n_q_heads, head_dim]  token stride out_tok_stride
 * max_seqlen_q / max_seqlen_k bound the segment lengths (as in FA2; they size
 * the launch grid).  A caller that understates them gets what FA2 gives:
 * a segment longer than max_seqlen_q has rows the grid does not cover, left
 * unwritten (here the segment's first rows, since causal q-blocks are
 * numbered from its end), and only its first max_seqlen_k keys are
 * attended; no access leaves the segment's rows.  Built for dtype
 * BF16/FP16, head_dim 128, group 1/2/4/8.  With too few work items for the
 * GPU -- one or a few long requests -- the key range of each item is split
 * over two workgroups whose partial results are merged by a log-sum-exp
 * combine (in a fixed order: results are the same on every run).  The split needs `workspace` of
 * aac_prefill_workspace_bytes(...) bytes, 256-byte aligned, ZERO-FILLED
 * ONCE when it is allocated: its first 16 KiB are per-item counters that
 * every call leaves at zero again, the rest partial results (do not share
 * it with other data or with calls that overlap on another stream).
 * workspace NULL, too small or misaligned: the call runs without a split.
 * Replaces flash_attn_varlen_func (llm.py:178-184).
 */
int aac_prefill_varlen(const void* q, const void* k, const void* v, int64_t q_tok_stride,
                       int64_t k_tok_stride, int64_t v_tok_stride, const int32_t* cu_seqlens_q,
                       const int32_t* cu_seqlens_k, int32_t n_seqs, int32_t max_seqlen_q,
                       int32_t max_seqlen_k, int32_t n_q_heads, int32_t n_kv_heads,
                       int32_t head_dim, float scale, int32_t causal, void* out,
                       int64_t out_tok_stride, void* workspace, size_t workspace_bytes,
                       int32_t dtype, void* stream);

/*
 * Workspace bytes aac_prefill_varlen would use to split this shape's key
 * ranges on the current device (0: the plan does not split).
 */
size_t aac_prefill_workspace_bytes(int32_t n_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                   int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                   int32_t causal);

/*
 * The result of aac_kv_store(k, v -> caches via slot_mapping) followed by
 * aac_prefill_varlen on the same stream: the whole per-layer attention block
 * of the reference's prefill (llm.py:171-184).  slot_mapping has n_kv_tokens
 * entries, one per packed key token (n_kv_tokens = cu_seqlens_k[n_seqs]);
 * every one of them is stored, also tokens outside all segments.  Causal
 * self-attention (cu_seqlens_q == cu_seqlens_k as pointers, equal max_seqlen)
 * runs as one kernel that stores each q-block's K/V rows after attending to
 * them; other calls launch the store, then the attention.  This call never
 * splits key ranges (no workspace).
 */
int aac_prefill_varlen_store(const void* q, const void* k, const void* v, int64_t q_tok_stride,
                             int64_t k_tok_stride, int64_t v_tok_stride,
                             const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                             int32_t n_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                             int32_t causal, void* out, int64_t out_tok_stride, void* k_cache,
                             void* v_cache, int64_t num_cache_rows, const int64_t* slot_mapping,
                             int64_t n_kv_tokens, int32_t dtype, void* stream);

/*
 * Bytes of split-K workspace aac_decode_paged needs for this shape.
 * max_context_len <= 0 means "table capacity" (max_blocks_per_seq *
 * block_size), partition_tokens <= 0 means "library's choice".  Returns 0
 * when the chosen plan needs no workspace.
 */
size_t aac_decode_workspace_bytes(int32_t n_seqs, int32_t n_q_heads, int32_t n_kv_heads,
                                  int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                                  int32_t max_context_len, int32_t partition_tokens);

/*
 * Paged decode attention: one query token per sequence,
 *   out[b, h] = softmax(scale * q[b, h] . K_b^T) V_b
 * over the first context_lens[b] tokens of sequence b, located through
 * block_tables[b * max_blocks_per_seq + i] (physical block of tokens
 * [i*block_size, (i+1)*block_size)).  context_lens[b] == 0 gives zeros; a
 * context longer than the table capacity is clamped to it.  Block ids outside
 * [0, num_blocks) are read as block 0 (output undefined, memory safe).
 *   q   [n_seqs, n_q_heads, head_dim]  seq stride q_seq_stride
 *   out [n_seqs, n_q_heads, head_dim]  seq stride out_seq_stride
 * Long contexts are split into partitions of partition_tokens (<= 0: auto)
 * that are combined with a log-sum-exp reduction in `workspace`
 * (aac_decode_workspace_bytes).  max_context_len (<= 0: table capacity) is
 * an upper bound on context_lens used to size the grid.
 * Built for dtype BF16/FP16/FP32, head_dim 128, group 1/2/4/8.
 * Replaces the attend half of flash_attn_with_kvcache (model/model.py:233-240).
 */
int aac_decode_paged(const void* q, int64_t q_seq_stride, const void* k_cache, const void* v_cache,
                     int64_t num_blocks, int32_t block_size, const int32_t* block_tables,
                     int32_t max_blocks_per_seq, const int32_t* context_lens, int32_t n_seqs,
                     int32_t max_context_len, int32_t n_q_heads, int32_t n_kv_heads,
                     int32_t head_dim, float scale, void* out, int64_t out_seq_stride,
                     void* workspace, size_t workspace_bytes, int32_t partition_tokens,
                     int32_t dtype, void* stream);

/* Bytes of the static split-K scratch aac_decode_paged_noalloc uses. */
#define AAC_DECODE_SCRATCH_BYTES (64u << 20)

/*
 * aac_decode_paged without a workspace: the same kernels, plan and results,
 * with the split-K partials in a static device array of
 * AAC_DECODE_SCRATCH_BYTES that the library holds on each GPU it runs on
 * until the process ends.  Allocates nothing (no hipMalloc, no library
 * allocation): for callers that cannot allocate device memory -- code under
 * HIP graph capture, tight serving loops, harnesses that forbid it.  A plan
 * whose workspace (aac_decode_workspace_bytes) exceeds the scratch returns
 * AAC_ERR_SCRATCH before anything is enqueued.  Every call on a GPU shares
 * that GPU's array (the device current on the calling thread), so calls
 * that overlap on one GPU -- other streams or threads -- race and must be
 * serialised by the caller; each call writes every scratch slot it reads, so
 * nothing carries over between calls.
 * No counterpart in the reference: an extra for callers that cannot
 * allocate.
 */
int aac_decode_paged_noalloc(const void* q, int64_t q_seq_stride, const void* k_cache,
                             const void* v_cache, int64_t num_blocks, int32_t block_size,
                             const int32_t* block_tables, int32_t max_blocks_per_seq,
                             const int32_t* context_lens, int32_t n_seqs,
                             int32_t max_context_len, int32_t n_q_heads, int32_t n_kv_heads,
                             int32_t head_dim, float scale, void* out, int64_t out_seq_stride,
                             int32_t partition_tokens, int32_t dtype, void* stream);

/*
 * flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, cache_seqlens,
 * block_table, softmax_scale, causal=False): append k/v at position
 * cache_seqlens[b] (aac_kv_append_paged), then attend over
 * cache_seqlens[b] + 1 tokens.  cache_seqlens is not modified.
 * max_context_len bounds cache_seqlens[b] + 1 (<= 0: table capacity).
 * Replaces model/model.py:233-240.
 */
int aac_decode_append_paged(const void* q, int64_t q_seq_stride, const void* k, const void* v,
                            int64_t k_tok_stride, int64_t v_tok_stride, void* k_cache,
                            void* v_cache, int64_t num_blocks, int32_t block_size,
                            const int32_t* block_tables, int32_t max_blocks_per_seq,
                            const int32_t* cache_seqlens, int32_t n_seqs, int32_t max_context_len,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                            void* out, int64_t out_seq_stride, void* workspace,
                            size_t workspace_bytes, int32_t partition_tokens, int32_t dtype,
                            void* stream);

/* ------------------------------------------------------------------------
 * Fused kernels of the attention call site.  Each replaces a chain of small
 * torch kernels of the reference layer with one launch and rounds to the
 * activation dtype at the same points.  dtype: BF16 or FP16.
 * ---------------------------------------------------------------------- */

/*
 * out = weight * dtype(h * rsqrt(mean(h^2) + eps)), statistics in fp32, where
 * h = x, or h = dtype(x + residual) with residual_out = h when residual is
 * given (residual and residual_out together or neither).  x rows have stride
 * x_row_stride; residual, residual_out and out are contiguous [n_rows, hidden].
 * hidden must be a multiple of 512, at most 4096.
 * Replaces RMSNorm (model/model.py:47-52) and the residual add before it
 * (model/model.py:259, :265; llm.py:188, :194).
 */
int aac_rmsnorm(const void* x, int64_t x_row_stride, const void* residual, void* residual_out,
                const void* weight, void* out, int64_t n_rows, int32_t hidden, float eps,
                int32_t dtype, void* stream);

/*
 * Per token of the fused QKV projection qkv [n_tokens, (Hq + 2*Hkv) * 128]
 * (row stride qkv_tok_stride): RMSNorm of every q and k head with
 * q_norm_weight / k_norm_weight, then RoPE with the cos/sin tables
 * [max_position, 128] at positions[t] (x*cos + rotate_half(x)*sin, each term
 * rounded), writing q_out [n_tokens, Hq, 128] and, if k_out is given,
 * k_out [n_tokens, Hkv, 128].  If v_cache is given the rotated k and the raw v
 * of token t are stored in the caches (rows [*, Hkv, 128]): at row
 * slot_mapping[t] (negative or >= num_cache_rows: skipped), or, when
 * slot_mapping is NULL, appended at position cache_seqlens[t] of block table
 * row t (decode: token t is sequence t).
 * Replaces model/model.py:219-228 plus the KV store llm.py:171-174 /
 * the k=/v= append of flash_attn_with_kvcache (model/model.py:233-240).
 */
int aac_qk_norm_rope_store(const void* qkv, int64_t qkv_tok_stride, int64_t n_tokens,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           const void* q_norm_weight, const void* k_norm_weight, float eps,
                           const void* cos_table, const void* sin_table, int32_t max_position,
                           const int32_t* positions, void* q_out, void* k_out, void* k_cache,
                           void* v_cache, int64_t num_cache_rows, const int64_t* slot_mapping,
                           const int32_t* block_tables, int32_t max_blocks_per_seq,
                           const int32_t* cache_seqlens, int32_t block_size, int32_t dtype,
                           void* stream);

/*
 * out[r, i] = dtype(silu(gate_up[r, i])) * gate_up[r, intermediate + i] for the
 * fused [gate | up] projection gate_up [n_rows, 2*intermediate].
 * Replaces act_fn(gate_proj(x)) * up_proj(x) (model/model.py:188).
 */
int aac_silu_mul(const void* gate_up, void* out, int64_t n_rows, int32_t intermediate,
                 int32_t dtype, void* stream);

/*
 * Decode-batch projection: y[m, n] = sum_k x[m, k] * w[n, k] (torch's
 * F.linear(x, w), fp32 accumulation, rounded to dtype) for x [m, k] and a
 * Linear weight w [n, k], rows strided by *_row_stride elements.  With
 * silu_intermediate = I (> 0) the weight is the fused [gate | up] projection
 * [2I, k], n must equal I, and y[m, i] = dtype(silu(dtype(gate))) *
 * dtype(up), the rounding of act_fn(gate_proj(x)) * up_proj(x)
 * (model/model.py:188) -- the product of aac_silu_mul without the [m, 2I]
 * intermediate.  Built for shapes where n is a multiple of 32 and k of 64
 * (of 128 / 256 for some tilings); config 0 lets the library pick the tiling,
 * 1..6 force one (tuning; a tiling whose stages do not fit LDS with the
 * gate/up pairing returns AAC_ERR_UNSUPPORTED).  Meant for the small m of a decode step (tens to
 * hundreds of rows): every output tile is one workgroup.
 * Replaces the q/k/v, o_proj, gate/up and down nn.Linear calls of the
 * decoder layer (model/model.py:132-154, :258, :178-188) on decode steps.
 */
int aac_gemm_nt(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, void* y,
                int64_t y_row_stride, int32_t m, int32_t n, int32_t k, int32_t silu_intermediate,
                int32_t config, int32_t dtype, void* stream);

/*
 * The fused QKV projection of a decode step followed by aac_qk_norm_rope_store
 * in one launch: qkv = x w_qkv^T (x [n_tokens, hidden], w_qkv the fused
 * [(Hq + 2*Hkv) * 128, hidden] weight, fp32 accumulation rounded to dtype
 * exactly as aac_gemm_nt's tiling 6 rounds it), then per token the q/k
 * RMSNorm + RoPE of every q and k head and the K/V store or decode append,
 * with the arguments and results of aac_qk_norm_rope_store (the [n_tokens,
 * Hq+2Hkv, 128] qkv intermediate is never written).  hidden must be a
 * multiple of 128.  Replaces the QKV projection and model/model.py:219-228
 * plus the k=/v= append of flash_attn_with_kvcache (model/model.py:233-240).
 */
int aac_qkv_norm_rope_store(const void* x, int64_t x_row_stride, const void* w_qkv,
                            int64_t w_row_stride, int64_t n_tokens, int32_t hidden,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                            const void* q_norm_weight, const void* k_norm_weight, float eps,
                            const void* cos_table, const void* sin_table, int32_t max_position,
                            const int32_t* positions, void* q_out, void* k_out, void* k_cache,
                            void* v_cache, int64_t num_cache_rows, const int64_t* slot_mapping,
                            const int32_t* block_tables, int32_t max_blocks_per_seq,
                            const int32_t* cache_seqlens, int32_t block_size, int32_t dtype,
                            void* stream);

/*
 * Greedy sampling: out[r] = the index of the largest element of row r of x
 * [n_rows, n_cols] (row stride row_stride elements; BF16, FP16 or FP32), the
 * first one among equal maxima, a NaN counting as the largest -- the result
 * of torch.argmax(dim=-1).  Replaces logits.argmax(dim=-1) of the sampler
 * (llm.py:215-219, temperature 0).
 */
int aac_argmax_rows(const void* x, int64_t row_stride, int64_t n_rows, int64_t n_cols,
                    int64_t* out, int32_t dtype, void* stream);

/*
 * KV export: gather the first `length` tokens of one sequence from a paged
 * cache into a contiguous buffer out[n_layers][2][length][Hkv][D] (index 0 =
 * K, 1 = V).  Layer l's K cache starts at kv_cache + l * layer_stride and its
 * V cache kv_stride elements after that (both [num_blocks, block_size, Hkv,
 * D]); token t lives in block block_table[t / block_size] (table width
 * max_blocks; length <= max_blocks * block_size).  Entries outside
 * [0, num_blocks) export zeros.  Replaces the per-layer slices
 * k_cache[slot, :length] / v_cache[slot, :length] of export_kv and
 * export_request_kv (model/model.py:156-165, :386-390); the slot layout is
 * block_table = [slot], block_size = max_seq_len.
 */
int aac_kv_export_paged(const void* kv_cache, int64_t layer_stride, int64_t kv_stride,
                        int32_t n_layers, int64_t num_blocks, int32_t block_size,
                        int32_t n_kv_heads, int32_t head_dim, const int32_t* block_table,
                        int32_t max_blocks, int32_t length, void* out, int32_t dtype,
                        void* stream);

/*
 * KV import: scatter src[n_layers][2][length][Hkv][D] into the paged cache
 * through block_table (same layout and arguments as aac_kv_export_paged);
 * entries outside [0, num_blocks) are skipped.  Replaces the per-layer
 * copy_ of import_kv and import_request_kv (model/model.py:167-177, :392-401);
 * cache_seqlens stays with the caller, as the reference sets it separately.
 */
int aac_kv_import_paged(const void* src, void* kv_cache, int64_t layer_stride, int64_t kv_stride,
                        int32_t n_layers, int64_t num_blocks, int32_t block_size,
                        int32_t n_kv_heads, int32_t head_dim, const int32_t* block_table,
                        int32_t max_blocks, int32_t length, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AAC_ATTN_H */
