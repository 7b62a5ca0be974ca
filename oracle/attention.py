"""CPU restatement of the reference's attention hot path (numpy, float64 math).

TEST INFRASTRUCTURE ONLY -- this module is the oracle the HIP kernels are
checked against.  It is never imported by the product package.

The reference delegates all attention arithmetic to the third-party
``flash_attn`` package (Dao-AILab FlashAttention-2 Python API; not vendored,
no pinned version in the reference, needs a 2.x release that accepts
``cache_batch_idx``).  The semantics restated here are the published FA2
API semantics at the reference's call sites:

* ``flash_attn_varlen_func(q, k, v, cu, cu, max_L, max_L, causal=True,
  softmax_scale)``                                     -- llm.py:178-184
* ``flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v,
  cache_seqlens, cache_batch_idx, softmax_scale, causal=False)`` followed by
  ``_cache_seqlens[slot_indices] += 1``                 -- model/model.py:233-241
* the prefill KV store ``cache.view(-1, Hkv, D).index_copy_(0, idx, x)``
                                                        -- llm.py:171-174

and the reference's own index construction (llm.py:127-140).

Causal masking follows FA2 >= 2.1 (bottom-right aligned): query row ``i`` of
a segment with ``Lq`` queries and ``Lk`` keys sees keys ``j <= i + Lk - Lq``.
At every reference call site ``Lq == Lk`` so this is the ordinary lower
triangle.  A query row that sees no key returns zeros (FA2 behaviour).

GQA: query head ``h`` reads KV head ``h // (Hq // Hkv)``
(model/model.py:110 ``num_kv_groups``; FA2's head mapping).

How each function is pinned (tests/test_oracle_pins.py):

* ``kv_store``: bit-exact against ``torch.Tensor.index_copy_`` on CPU -- the
  very op the reference calls -- with sentinel-filled caches so untouched rows
  are compared too.
* ``prefill_metadata``: against torch's ``cumsum``/``repeat_interleave``
  evaluation of llm.py:132-140 and closed forms (ranges, monotonicity).
* ``paged_slot_mapping`` / ``decode_slot_mapping``: the slot layout special
  case (one block of size ``max_seq_len`` per sequence) must reproduce
  llm.py:140 exactly; a permutation of physical block ids must map
  bijectively.
* ``varlen_attention``: against ``torch.nn.functional.scaled_dot_product_attention``
  (float64, ``is_causal``) per segment with KV heads repeat-interleaved;
  closed forms -- q = 0 gives the causal prefix mean of V per KV head (catches
  a mask off-by-one or a wrong GQA map), single-token segments return v,
  a large-scale one-hot query returns the selected key's value row.
* ``paged_decode``: equals the last row of a causal prefill over the gathered
  context; invariant under permutation of physical block ids; context 1
  returns v0; against SDPA.
* ``kv_export`` / ``kv_import``: in the slot layout (``block_size =
  max_seq_len``, ``block_table = [slot]``) the export is exactly the
  reference's ``k_cache[slot, :length]`` / ``v_cache[slot, :length]`` per
  layer (model/model.py:156-165), the import exactly its
  ``k_cache[slot, :length].copy_(k[:length])`` (:167-177), with every other
  cache byte untouched; over a permuted pool, import-then-export returns the
  payload and a block relabelling commutes with both.
* bf16 helpers: bit-exact against ``torch.Tensor.to(torch.bfloat16)``
  (round-to-nearest-even) including ties, subnormals, inf and NaN.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "f32_to_bf16_bits",
    "bf16_bits_to_f32",
    "bf16_round",
    "kv_store",
    "kv_export",
    "kv_import",
    "prefill_metadata",
    "paged_slot_mapping",
    "decode_slot_mapping",
    "gather_paged",
    "varlen_attention",
    "paged_decode",
    "decode_append_attend",
]


# ----------------------------------------------------------------------------
# bf16 bit helpers (the reference keeps activations and caches in bf16:
# llm.py:47 dtype=torch.bfloat16, model/model.py:328-335)
# ----------------------------------------------------------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round-to-nearest-even, NaN kept quiet."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    bias = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    r = ((u + bias) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint64(16)).astype(np.uint16)) | np.uint16(0x0040)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    """bf16 bit pattern (uint16) -> float32 (exact)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16-representable float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ----------------------------------------------------------------------------
# KV store -- llm.py:171-174
# ----------------------------------------------------------------------------
def kv_store(cache: np.ndarray, x: np.ndarray, slot_mapping) -> None:
    """In-place row scatter ``cache.view(-1, Hkv, D)[slot_mapping[t]] = x[t]``.

    Restates ``kv_flat.index_copy_(0, scatter_indices, k)`` (llm.py:171-174).
    ``cache`` is any contiguous array whose trailing dims are ``x.shape[1:]``
    (the reference's ``[S, Lmax, Hkv, D]`` slot cache or a paged
    ``[num_blocks, block_size, Hkv, D]`` cache); the copy is a byte copy, so
    any dtype (float32, or uint16 bf16 bit patterns) is stored bit-exactly.

    A negative slot means "padding, skip" (vLLM/FA convention used by the
    HIP kernel); an index at or beyond the row count raises ``IndexError``
    like ``index_copy_`` does.  Duplicate slots are undefined (as for
    ``index_copy_``) and callers must not pass them.
    """
    if not cache.flags.c_contiguous:
        raise ValueError("cache must be contiguous")
    rows = cache.reshape((-1,) + tuple(x.shape[1:]))
    if not np.shares_memory(rows, cache):
        raise ValueError("cache reshape did not produce a view")
    sm = np.asarray(slot_mapping, dtype=np.int64).reshape(-1)
    if sm.shape[0] != x.shape[0]:
        raise ValueError("slot_mapping length must equal the token count")
    if (sm >= rows.shape[0]).any():
        raise IndexError("slot_mapping entry out of range")
    keep = sm >= 0
    rows[sm[keep]] = x[keep]


# ----------------------------------------------------------------------------
# Metadata -- llm.py:127-140 and its paged generalisation
# ----------------------------------------------------------------------------
def prefill_metadata(seq_lens, slot_indices, max_seq_len: int):
    """Return ``(cu_seqlens int32[n+1], positions int64[N], scatter int64[N])``.

    Restates llm.py:129-140: ``cu_seqlens[1:] = cumsum(seq_lens)``,
    ``positions = cat(arange(L_i))`` and
    ``scatter = repeat_interleave(slot * max_seq_len, L) + positions``.
    """
    seq_lens = [int(s) for s in seq_lens]
    cu = np.zeros(len(seq_lens) + 1, dtype=np.int32)
    pos_parts, sc_parts = [], []
    acc = 0
    for i, (L, s) in enumerate(zip(seq_lens, slot_indices)):
        acc += L
        cu[i + 1] = acc
        p = np.arange(L, dtype=np.int64)
        pos_parts.append(p)
        sc_parts.append(np.int64(s) * np.int64(max_seq_len) + p)
    positions = np.concatenate(pos_parts) if pos_parts else np.zeros(0, np.int64)
    scatter = np.concatenate(sc_parts) if sc_parts else np.zeros(0, np.int64)
    return cu, positions, scatter


def paged_slot_mapping(block_tables, seq_lens, block_size: int, start_positions=None):
    """Flat cache row for every packed token of a prefill over a paged cache.

    Token at position ``p`` of sequence ``b`` lands in row
    ``block_tables[b][p // block_size] * block_size + p % block_size``.  With
    one block of size ``max_seq_len`` per sequence
    (``block_tables[b] = [slot_b]``) this is exactly llm.py:140.
    ``start_positions[b]`` offsets the first position (0 for a fresh prompt).
    """
    bt = np.asarray(block_tables, dtype=np.int64)
    out = []
    for b, L in enumerate(seq_lens):
        p0 = 0 if start_positions is None else int(start_positions[b])
        p = np.arange(p0, p0 + int(L), dtype=np.int64)
        out.append(bt[b, p // block_size] * block_size + p % block_size)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def decode_slot_mapping(block_tables, cache_seqlens, block_size: int):
    """Row of the appended token for each decode sequence.

    ``flash_attn_with_kvcache(k=, v=)`` writes the new token of batch row
    ``b`` at position ``cache_seqlens[b]`` of that sequence
    (model/model.py:233-240); in paged form that is
    ``block_tables[b][p // bs] * bs + p % bs`` with ``p = cache_seqlens[b]``.
    """
    bt = np.asarray(block_tables, dtype=np.int64)
    p = np.asarray(cache_seqlens, dtype=np.int64)
    b = np.arange(p.shape[0])
    return bt[b, p // block_size] * block_size + p % block_size


def gather_paged(cache: np.ndarray, block_table_row, n_tokens: int, block_size: int) -> np.ndarray:
    """Gather the first ``n_tokens`` token rows of one sequence from a paged cache."""
    bt = np.asarray(block_table_row, dtype=np.int64)
    rows = cache.reshape((-1,) + tuple(cache.shape[2:]))
    p = np.arange(int(n_tokens), dtype=np.int64)
    return rows[bt[p // block_size] * block_size + p % block_size]


def kv_export(storage: np.ndarray, block_table_row, length: int) -> np.ndarray:
    """Export of one sequence (model/model.py:156-165, :386-390, paged form):
    ``storage`` [L, 2, num_blocks, block_size, Hkv, D] -> [L, 2, length, Hkv, D]
    with layer l, index c (0 = K, 1 = V) the first ``length`` token rows of
    that cache.  Tokens whose block id is outside [0, num_blocks) read zeros."""
    L, _, nb, bs = storage.shape[:4]
    bt = np.asarray(block_table_row, dtype=np.int64)
    p = np.arange(int(length), dtype=np.int64)
    blk = bt[p // bs]
    ok = (blk >= 0) & (blk < nb)
    rows = storage.reshape((L, 2, nb * bs) + tuple(storage.shape[4:]))
    out = np.zeros((L, 2, int(length)) + tuple(storage.shape[4:]), dtype=storage.dtype)
    out[:, :, ok] = rows[:, :, (blk * bs + p % bs)[ok]]
    return out


def kv_import(src: np.ndarray, storage: np.ndarray, block_table_row, length: int) -> np.ndarray:
    """Import (model/model.py:167-177, :392-401, paged form): writes src[:, :,
    :length] into the sequence's token rows of ``storage`` in place (entries
    outside [0, num_blocks) are skipped); returns ``storage``."""
    L, _, nb, bs = storage.shape[:4]
    bt = np.asarray(block_table_row, dtype=np.int64)
    p = np.arange(int(length), dtype=np.int64)
    blk = bt[p // bs]
    ok = (blk >= 0) & (blk < nb)
    rows = storage.reshape((L, 2, nb * bs) + tuple(storage.shape[4:]))
    rows[:, :, (blk * bs + p % bs)[ok]] = src[:, :, :int(length)][:, :, ok]
    return storage


# ----------------------------------------------------------------------------
# Attention math (float64)
# ----------------------------------------------------------------------------
def _as_f64(x):
    x = np.asarray(x)
    if x.dtype == np.uint16:  # bf16 bit patterns
        return bf16_bits_to_f32(x).astype(np.float64)
    return x.astype(np.float64)


def _attend(qs, ks, vs, scale, causal, want_lse=False):
    """One segment.  qs [Lq,Hq,D], ks/vs [Lk,Hkv,D] float64 -> [Lq,Hq,D] (+ lse [Lq,Hq])."""
    Lq, Hq, D = qs.shape
    Lk, Hkv, _ = ks.shape
    g = Hq // Hkv
    out = np.zeros((Lq, Hq, D), dtype=np.float64)
    lse = np.full((Lq, Hq), -np.inf, dtype=np.float64)
    if Lq == 0 or Lk == 0:
        return (out, lse) if want_lse else out
    q4 = qs.transpose(1, 0, 2).reshape(Hkv, g, Lq, D)        # [Hkv,g,Lq,D]
    kt = ks.transpose(1, 2, 0)                                # [Hkv,D,Lk]
    vt = vs.transpose(1, 0, 2)                                # [Hkv,Lk,D]
    s = np.matmul(q4, kt[:, None]) * scale                    # [Hkv,g,Lq,Lk]
    if causal:
        i = np.arange(Lq)[:, None]
        j = np.arange(Lk)[None, :]
        allowed = j <= i + (Lk - Lq)
        s = np.where(allowed[None, None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    has = np.isfinite(m)
    m_safe = np.where(has, m, 0.0)
    p = np.exp(s - m_safe)
    l = p.sum(axis=-1, keepdims=True)
    o = np.matmul(p, vt[:, None]) / np.where(l > 0, l, 1.0)   # [Hkv,g,Lq,D]
    o = np.where(has, o, 0.0)
    out[:] = o.reshape(Hq, Lq, D).transpose(1, 0, 2)
    if want_lse:
        ls = np.where(has, m_safe + np.log(np.where(l > 0, l, 1.0)), -np.inf)
        lse[:] = ls.reshape(Hq, Lq).T
        return out, lse
    return out


def varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k=None, scale=None, causal=True):
    """Packed varlen attention, ``flash_attn_varlen_func`` semantics (llm.py:178-184).

    q ``[Nq, Hq, D]``, k/v ``[Nk, Hkv, D]`` (float32/float64 or uint16 bf16
    bits); segment ``s`` covers rows ``cu[s]:cu[s+1]``.  Returns float64
    ``[Nq, Hq, D]``.
    """
    qf, kf, vf = _as_f64(q), _as_f64(k), _as_f64(v)
    Hq, D = qf.shape[1], qf.shape[2]
    Hkv = kf.shape[1]
    if Hq % Hkv:
        raise ValueError("Hq must be a multiple of Hkv")
    if scale is None:
        scale = D ** -0.5
    cq = np.asarray(cu_seqlens_q, dtype=np.int64)
    ck = cq if cu_seqlens_k is None else np.asarray(cu_seqlens_k, dtype=np.int64)
    out = np.zeros(qf.shape, dtype=np.float64)
    for s in range(cq.shape[0] - 1):
        q0, q1, k0, k1 = cq[s], cq[s + 1], ck[s], ck[s + 1]
        out[q0:q1] = _attend(qf[q0:q1], kf[k0:k1], vf[k0:k1], scale, causal)
    return out


def paged_decode(q, k_cache, v_cache, block_tables, context_lens, block_size=None,
                 scale=None, return_lse=False):
    """Single-query attention over a paged cache (attend half of model/model.py:233-240).

    q ``[B, Hq, D]``; caches ``[num_blocks, block_size, Hkv, D]``; sequence
    ``b`` attends its first ``context_lens[b]`` tokens, found through
    ``block_tables[b]``.  ``context_lens[b] == 0`` yields zeros.  Returns
    float64 ``[B, Hq, D]`` (and the per-head log-sum-exp when asked).
    """
    qf = _as_f64(q)
    B, Hq, D = qf.shape
    if block_size is None:
        block_size = k_cache.shape[1]
    if scale is None:
        scale = D ** -0.5
    out = np.zeros((B, Hq, D), dtype=np.float64)
    lse = np.full((B, Hq), -np.inf, dtype=np.float64)
    for b in range(B):
        n = int(context_lens[b])
        ks = _as_f64(gather_paged(k_cache, block_tables[b], n, block_size))
        vs = _as_f64(gather_paged(v_cache, block_tables[b], n, block_size))
        o, l = _attend(qf[b:b + 1], ks, vs, scale, causal=False, want_lse=True)
        out[b] = o[0]
        lse[b] = l[0]
    return (out, lse) if return_lse else out


def decode_append_attend(q, k_cache, v_cache, k_new, v_new, block_tables, cache_seqlens,
                         block_size=None, scale=None):
    """``flash_attn_with_kvcache(q, kc, vc, k=k_new, v=v_new, cache_seqlens, ...)``
    followed by ``cache_seqlens += 1`` (model/model.py:233-241), paged form.

    Mutates ``k_cache``/``v_cache`` in place (row ``cache_seqlens[b]`` of
    sequence ``b`` receives ``k_new[b]``/``v_new[b]``), then attends over
    ``cache_seqlens[b] + 1`` keys.  Returns ``(out float64 [B,Hq,D],
    new_seqlens int32 [B])``.  The reference's slot layout is the special case
    ``block_tables[b] = [cache_batch_idx[b]]``, ``block_size = max_seq_len``.
    """
    if block_size is None:
        block_size = k_cache.shape[1]
    sm = decode_slot_mapping(block_tables, cache_seqlens, block_size)
    kv_store(k_cache, np.asarray(k_new).reshape((-1,) + k_cache.shape[2:]), sm)
    kv_store(v_cache, np.asarray(v_new).reshape((-1,) + v_cache.shape[2:]), sm)
    ctx = np.asarray(cache_seqlens, dtype=np.int64) + 1
    out = paged_decode(q, k_cache, v_cache, block_tables, ctx, block_size, scale)
    return out, ctx.astype(np.int32)
