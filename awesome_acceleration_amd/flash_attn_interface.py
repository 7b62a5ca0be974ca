"""FlashAttention-2-compatible Python surface over libaac_attn.so.

The reference engine calls three functions of the third-party ``flash_attn``
package; this module provides drop-in replacements with the same names,
argument meanings, return values and error behaviour (``RuntimeError`` for a
rejected input), backed by the gfx950 kernels:

* ``flash_attn_varlen_func``  -- llm.py:178-184 (packed causal prefill)
* ``flash_attn_with_kvcache`` -- model/model.py:233-240 (append + decode)
* ``flash_attn_func``         -- model/model.py:253-254 (padded prefill)

plus the KV store the reference does with ``index_copy_`` (llm.py:171-174):

* ``kv_store``                -- slot_mapping row scatter
* ``varlen_prefill_with_kvcache`` -- store + varlen attention in one call

Only the features the reference uses are accepted (no dropout, no sliding
window, no ALiBi, no softcap, no rotary inside the call); anything else
raises ``NotImplementedError`` instead of silently computing something else.
Every op runs on ``torch.cuda.current_stream()`` and never synchronises.
Outputs are allocated here (FA2 returns a new tensor); caches are updated in
place; ``cache_seqlens`` is never modified (the reference increments it
itself, model/model.py:241).
"""
from __future__ import annotations

import math
import os
import threading
from typing import Optional

import torch

from . import _lib

__all__ = [
    "kv_store",
    "flash_attn_varlen_func",
    "varlen_prefill_with_kvcache",
    "flash_attn_with_kvcache",
    "flash_attn_func",
    "decode_paged",
]

_CHECK = os.environ.get("AAC_CHECK", "0") not in ("", "0")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _dtype_code(t: torch.Tensor) -> int:
    code = _lib.AAC_DTYPE.get(t.dtype)
    _require(code is not None, f"unsupported dtype {t.dtype}")
    return code


def _on_gpu(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        _require(t.is_cuda, "all tensors must be on a GPU (no CPU path exists)")
        if dev is None:
            dev = t.device
        _require(t.device == dev, "all tensors must be on the same GPU")
    return dev


def _token_rows(t: torch.Tensor, name: str) -> int:
    """Token stride (elements) of a [N, H, D] tensor whose [H, D] block is contiguous."""
    _require(t.dim() == 3, f"{name} must be [tokens, heads, head_dim]")
    _require(t.stride(2) == 1 and t.stride(1) == t.shape[2],
             f"{name}: heads and head_dim must be contiguous within a token")
    return t.stride(0) if t.shape[0] > 1 else t.shape[1] * t.shape[2]


# ---------------------------------------------------------------- workspace
_ws_lock = threading.Lock()
_ws: dict[tuple[int, int], torch.Tensor] = {}
_pf_ws: dict[tuple[int, int], torch.Tensor] = {}
_ws_retired: list[torch.Tensor] = []


def _stream_key(device: torch.device) -> tuple[int, int]:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return idx, torch.cuda.current_stream(idx).cuda_stream


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch for split-K decode partials, one per (device, stream), grown on
    demand: calls on different streams never share partials.  A buffer that
    is outgrown is kept alive rather than freed: a captured HIP graph may hold
    its address."""
    key = _stream_key(device)
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                _ws_retired.append(buf)
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _ws[key] = buf
        return buf


def _prefill_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Workspace of the split-key prefill, one per (device, stream): zero-filled
    (by a fill kernel) when it is allocated, since its leading per-item
    counters must start at zero and every call leaves them at zero; grown on
    demand, never shared with the decode workspace, and outgrown buffers stay
    alive (a captured graph may hold them).  Per stream, so prefills that
    overlap on two streams never count into each other's counters."""
    key = _stream_key(device)
    with _ws_lock:
        buf = _pf_ws.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                # under graph capture the fill would be recorded, not run, so
                # the counters of a new buffer would not start at zero: the
                # call runs unsplit instead
                return None
            if buf is not None:
                _ws_retired.append(buf)
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _pf_ws[key] = buf
        return buf


_PF_COUNTER_BYTES = 16 << 10  # the split prefill's per-item counters at the workspace start


def _check_prefill_counters(ws: torch.Tensor) -> None:
    """With ``AAC_CHECK``: the split prefill leaves its per-item counters at
    zero; anything else means a workspace that was not zero-filled or was
    shared by overlapping calls, and rows may have been left unwritten."""
    if int(ws[:_PF_COUNTER_BYTES].count_nonzero()):
        raise RuntimeError("split-prefill workspace counters are not zero after the call: the "
                           "workspace was not zero-filled or is shared by overlapping calls")


# ---------------------------------------------------------------- KV store
def check_mode() -> bool:
    """Whether ``AAC_CHECK`` is set: the stores then validate slot_mapping as
    ``index_copy_`` does (one device sync per call)."""
    return _CHECK


def _check_slots(slot_mapping: torch.Tensor, rows: int) -> None:
    """With ``AAC_CHECK``: ``IndexError`` for any slot outside ``[0, rows)``,
    negative ones included -- the contract of the reference's ``index_copy_``
    (llm.py:171-174).  Without it the kernels skip such slots (a negative slot
    is the padding convention of paged engines), and the engine validates its
    own slot mappings on the host (``paged.check_slots``)."""
    if _CHECK and slot_mapping.numel():
        lo, hi = torch.aminmax(slot_mapping)
        lo, hi = int(lo), int(hi)
        if lo < 0 or hi >= rows:
            bad = lo if lo < 0 else hi
            raise IndexError(f"index {bad} is out of bounds for dimension 0 with size {rows}")


def kv_store(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             slot_mapping: torch.Tensor) -> None:
    """``k_cache.view(-1,Hkv,D).index_copy_(0, slot_mapping, k)`` and the same for v.

    Replaces llm.py:171-174.  ``k``/``v`` are ``[N, Hkv, D]`` (any token
    stride, e.g. v as a view of the fused qkv buffer); the caches are
    contiguous ``[..., Hkv, D]``; ``slot_mapping`` is int64 ``[N]`` on the
    device.  Negative and out-of-range slots are skipped.  With ``AAC_CHECK=1``
    any slot outside ``[0, rows)`` raises ``IndexError`` like ``index_copy_``
    (this synchronises).
    """
    _on_gpu(k, v, k_cache, v_cache, slot_mapping)
    ks, vs = _token_rows(k, "k"), _token_rows(v, "v")
    _require(k.shape == v.shape, "k and v must have the same shape")
    _require(k.dtype == v.dtype == k_cache.dtype == v_cache.dtype, "dtype mismatch")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    _require(k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape")
    _require(tuple(k_cache.shape[-2:]) == tuple(k.shape[1:]), "cache row shape != [Hkv, D]")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.dim() == 1
             and slot_mapping.shape[0] == k.shape[0], "slot_mapping must be int64 [N]")
    _require(slot_mapping.is_contiguous(), "slot_mapping must be contiguous")
    rows = k_cache.numel() // (k.shape[1] * k.shape[2])
    _check_slots(slot_mapping, rows)
    rc = _lib.lib().aac_kv_store(
        k.data_ptr(), v.data_ptr(), ks, vs, k_cache.data_ptr(), v_cache.data_ptr(), rows,
        slot_mapping.data_ptr(), k.shape[0], k.shape[1], k.shape[2], _dtype_code(k), _stream(k))
    _lib.check(rc, "aac_kv_store")


# ---------------------------------------------------------------- prefill
def _unsupported(dropout_p, window_size, softcap, alibi_slopes, return_attn_probs):
    if dropout_p:
        raise NotImplementedError("dropout is not supported (inference-only kernels)")
    if tuple(window_size) != (-1, -1):
        raise NotImplementedError("sliding-window attention is not supported")
    if softcap:
        raise NotImplementedError("softcap is not supported")
    if alibi_slopes is not None:
        raise NotImplementedError("ALiBi is not supported")
    if return_attn_probs:
        raise NotImplementedError("return_attn_probs is not supported")


def _prefill_checks(q, k, v, cu_seqlens_q, cu_seqlens_k):
    _on_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k)
    qs, ks, vs = _token_rows(q, "q"), _token_rows(k, "k"), _token_rows(v, "v")
    _require(q.dtype in (torch.bfloat16, torch.float16), "prefill supports fp16 and bf16 only")
    _require(q.dtype == k.dtype == v.dtype, "q, k, v must share a dtype")
    _require(k.shape == v.shape, "k and v must have the same shape")
    _require(q.shape[2] == k.shape[2], "head_dim mismatch")
    _require(q.shape[1] % k.shape[1] == 0, "number of query heads must be a multiple of KV heads")
    for c in (cu_seqlens_q, cu_seqlens_k):
        _require(c.dtype == torch.int32 and c.dim() == 1 and c.is_contiguous(),
                 "cu_seqlens must be contiguous int32 [batch+1]")
    _require(cu_seqlens_q.shape == cu_seqlens_k.shape, "cu_seqlens_q / cu_seqlens_k length mismatch")
    return qs, ks, vs


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1),
                           softcap=0.0, alibi_slopes=None, deterministic=False,
                           return_attn_probs=False, block_table=None):
    """Packed variable-length attention (llm.py:178-184).

    q ``[Nq, Hq, D]``, k/v ``[Nk, Hkv, D]``, ``cu_seqlens_*`` int32
    ``[batch+1]``.  Returns a new ``[Nq, Hq, D]`` tensor.  ``causal`` masks
    bottom-right aligned, as FA2 >= 2.1 does.
    """
    _unsupported(dropout_p, window_size, softcap, alibi_slopes, return_attn_probs)
    if block_table is not None:
        raise NotImplementedError("paged K/V for varlen prefill is not supported")
    qs, ks, vs = _prefill_checks(q, k, v, cu_seqlens_q, cu_seqlens_k)
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if q.shape[0] == 0:
        return out
    if k.shape[0] == 0:  # no key anywhere: every row sees none
        return out.zero_()
    L = _lib.lib()
    n_seqs = cu_seqlens_q.shape[0] - 1
    ws_bytes = L.aac_prefill_workspace_bytes(n_seqs, int(max_seqlen_q), int(max_seqlen_k),
                                             q.shape[1], k.shape[1], q.shape[2],
                                             int(bool(causal)))
    ws = _prefill_workspace(ws_bytes, q.device) if ws_bytes else None
    rc = L.aac_prefill_varlen(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), qs, ks, vs, cu_seqlens_q.data_ptr(),
        cu_seqlens_k.data_ptr(), n_seqs, int(max_seqlen_q), int(max_seqlen_k),
        q.shape[1], k.shape[1], q.shape[2], scale, int(bool(causal)), out.data_ptr(),
        out.stride(0), ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _dtype_code(q), _stream(q))
    _lib.check(rc, "aac_prefill_varlen")
    if _CHECK and ws is not None:
        _check_prefill_counters(ws)
    return out


def varlen_prefill_with_kvcache(q, k, v, cu_seqlens, max_seqlen, k_cache, v_cache, slot_mapping,
                                softmax_scale=None, causal=True):
    """Store k/v into the cache through ``slot_mapping`` and run causal varlen
    attention, in one call (the per-layer block llm.py:171-184)."""
    qs, ks, vs = _prefill_checks(q, k, v, cu_seqlens, cu_seqlens)
    _on_gpu(q, k_cache, v_cache, slot_mapping)
    _require(k_cache.dtype == v_cache.dtype == q.dtype, "cache dtype mismatch")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    _require(k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape")
    _require(tuple(k_cache.shape[-2:]) == tuple(k.shape[1:]), "cache row shape != [Hkv, D]")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.dim() == 1
             and slot_mapping.shape[0] == k.shape[0] and slot_mapping.is_contiguous(),
             "slot_mapping must be contiguous int64 [N]")
    rows = k_cache.numel() // (k.shape[1] * k.shape[2])
    _check_slots(slot_mapping, rows)
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else float(softmax_scale)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    rc = _lib.lib().aac_prefill_varlen_store(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), qs, ks, vs, cu_seqlens.data_ptr(),
        cu_seqlens.data_ptr(), cu_seqlens.shape[0] - 1, int(max_seqlen), int(max_seqlen),
        q.shape[1], k.shape[1], q.shape[2], scale, int(bool(causal)), out.data_ptr(),
        out.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), rows, slot_mapping.data_ptr(),
        k.shape[0], _dtype_code(q), _stream(q))
    _lib.check(rc, "aac_prefill_varlen_store")
    return out


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                    window_size=(-1, -1), softcap=0.0, alibi_slopes=None, deterministic=False,
                    return_attn_probs=False):
    """Padded-batch attention ``[B, T, H, D]`` (model/model.py:253-254), run as
    varlen attention with uniform ``cu_seqlens``."""
    _unsupported(dropout_p, window_size, softcap, alibi_slopes, return_attn_probs)
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k, v must be [B, T, H, D]")
    B, Tq, Hq, D = q.shape
    Tk = k.shape[1]
    _require(k.shape[0] == B and v.shape[0] == B, "batch mismatch")
    qf = q.reshape(B * Tq, Hq, D)
    kf = k.reshape(B * Tk, k.shape[2], D)
    vf = v.reshape(B * Tk, v.shape[2], D)
    steps = torch.arange(B + 1, dtype=torch.int32, device=q.device)
    cu_q, cu_k = steps * Tq, steps * Tk  # (valid for empty sequences too)
    out = flash_attn_varlen_func(qf, kf, vf, cu_q, cu_k, Tq, Tk, softmax_scale=softmax_scale,
                                 causal=causal)
    return out.view(B, Tq, Hq, D)


# ---------------------------------------------------------------- decode
def decode_paged(q, k_cache, v_cache, block_tables, context_lens, softmax_scale=None,
                 max_context_len=None, partition_tokens=0, out=None):
    """Attend-only paged decode: ``q [B, Hq, D]`` against the first
    ``context_lens[b]`` tokens of each sequence (block_tables int32
    ``[B, max_blocks]``, caches ``[num_blocks, block_size, Hkv, D]``)."""
    _on_gpu(q, k_cache, v_cache, block_tables, context_lens)
    _require(q.dim() == 3, "q must be [B, Hq, D]")
    B, Hq, D = q.shape
    _require(q.stride(2) == 1 and q.stride(1) == D, "q heads/head_dim must be contiguous")
    _check_cache(q, k_cache, v_cache)
    _require(block_tables.dtype == torch.int32 and block_tables.dim() == 2
             and block_tables.shape[0] == B and block_tables.is_contiguous(),
             "block_tables must be contiguous int32 [B, max_blocks]")
    _require(context_lens.dtype == torch.int32 and context_lens.shape == (B,)
             and context_lens.is_contiguous(), "context_lens must be contiguous int32 [B]")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    nblk, bs, hkv = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    mb = block_tables.shape[1]
    mcl = int(max_context_len or 0)
    L = _lib.lib()
    ws_bytes = L.aac_decode_workspace_bytes(B, Hq, hkv, D, bs, mb, mcl, int(partition_tokens))
    ws = _workspace(ws_bytes, q.device) if ws_bytes else None
    rc = L.aac_decode_paged(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), nblk, bs,
        block_tables.data_ptr(), mb, context_lens.data_ptr(), B, mcl, Hq, hkv, D,
        _scale(softmax_scale, D), out.data_ptr(), out.stride(0),
        ws.data_ptr() if ws is not None else None, ws_bytes, int(partition_tokens),
        _dtype_code(q), _stream(q))
    _lib.check(rc, "aac_decode_paged")
    return out


def _scale(softmax_scale, D):
    return D ** -0.5 if softmax_scale is None else float(softmax_scale)


def _check_cache(q, k_cache, v_cache):
    _require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape,
             "caches must be [num_blocks, block_size, Hkv, D] with equal shapes")
    _require(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    _require(k_cache.dtype == v_cache.dtype == q.dtype, "q and caches must share a dtype")
    _require(k_cache.shape[3] == q.shape[-1], "head_dim mismatch")
    _require(q.shape[-2] % k_cache.shape[2] == 0, "query heads must be a multiple of KV heads")


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None,
                            block_table=None, softmax_scale=None, causal=False,
                            window_size=(-1, -1), softcap=0.0, rotary_interleaved=True,
                            alibi_slopes=None, num_splits=0, return_softmax_lse=False,
                            *, max_context_len=None):
    """Decode with KV cache (model/model.py:233-240).

    q ``[B, 1, Hq, D]``.  Without ``block_table`` the caches are the
    reference's slot caches ``[num_slots, max_seq_len, Hkv, D]`` and batch
    row ``b`` uses slot ``cache_batch_idx[b]`` (default ``b``); with
    ``block_table`` (int32 ``[B, max_blocks]``) they are paged caches
    ``[num_blocks, block_size, Hkv, D]``.  When ``k``/``v`` (``[B, 1, Hkv,
    D]``) are given they are written at position ``cache_seqlens[b]`` first
    and the call attends over ``cache_seqlens[b] + 1`` tokens, otherwise over
    ``cache_seqlens[b]``.  ``cache_seqlens`` is not modified.  Returns a new
    ``[B, 1, Hq, D]`` tensor.
    """
    _unsupported(0.0, window_size, softcap, alibi_slopes, False)
    if rotary_cos is not None or rotary_sin is not None:
        raise NotImplementedError("rotary inside the kernel is not supported; apply RoPE first")
    if cache_leftpad is not None:
        raise NotImplementedError("cache_leftpad is not supported")
    if return_softmax_lse:
        raise NotImplementedError("return_softmax_lse is not supported")
    _require(q.dim() == 4, "q must be [B, S, Hq, D]")
    B, S, Hq, D = q.shape
    if S != 1:
        raise NotImplementedError("only one query token per sequence (decode) is supported")
    _require((k is None) == (v is None), "k and v must be given together")
    _on_gpu(q, k_cache, v_cache, k, v, cache_batch_idx, block_table)
    _check_cache(q, k_cache, v_cache)
    dev = q.device
    if block_table is None:
        if cache_batch_idx is None:
            tables = torch.arange(B, dtype=torch.int32, device=dev).view(B, 1)
        else:
            tables = cache_batch_idx.to(torch.int32).reshape(B, 1).contiguous()
    else:
        _require(cache_batch_idx is None, "cache_batch_idx cannot be combined with block_table")
        _require(block_table.dtype == torch.int32 and block_table.dim() == 2
                 and block_table.shape[0] == B, "block_table must be int32 [B, max_blocks]")
        tables = block_table.contiguous()
    if cache_seqlens is None:
        raise RuntimeError("cache_seqlens is required")
    if isinstance(cache_seqlens, int):
        seqlens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=dev)
    else:
        _on_gpu(q, cache_seqlens)
        seqlens = cache_seqlens.to(torch.int32).contiguous()
        _require(seqlens.shape == (B,), "cache_seqlens must be [B]")
    nblk, bs, hkv = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    mb = tables.shape[1]
    q3 = q.view(B, Hq, D) if q.is_contiguous() else q.reshape(B, Hq, D)
    _require(q3.stride(2) == 1 and q3.stride(1) == D, "q heads/head_dim must be contiguous")
    out = torch.empty((B, 1, Hq, D), dtype=q.dtype, device=dev)
    mcl = int(max_context_len or 0)
    part = 0
    if num_splits and num_splits > 0:
        cap = min(mcl, mb * bs) if mcl > 0 else mb * bs
        part = max(1, math.ceil(cap / int(num_splits)))
    L = _lib.lib()
    ws_bytes = L.aac_decode_workspace_bytes(B, Hq, hkv, D, bs, mb, mcl, part)
    ws = _workspace(ws_bytes, dev) if ws_bytes else None
    wsp = ws.data_ptr() if ws is not None else None
    if k is None:
        rc = L.aac_decode_paged(
            q3.data_ptr(), q3.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), nblk, bs,
            tables.data_ptr(), mb, seqlens.data_ptr(), B, mcl, Hq, hkv, D, _scale(softmax_scale, D),
            out.data_ptr(), Hq * D, wsp, ws_bytes, part, _dtype_code(q), _stream(q))
        _lib.check(rc, "aac_decode_paged")
        return out
    _require(k.shape == v.shape and k.shape[0] == B and k.shape[1] == 1,
             "k/v must be [B, 1, Hkv, D]")
    _require(k.dtype == q.dtype and v.dtype == q.dtype, "k/v dtype mismatch")
    k3 = k.reshape(B, k.shape[2], D) if not (k.stride(3) == 1 and k.stride(2) == D) else \
        k.as_strided((B, k.shape[2], D), (k.stride(0), D, 1))
    v3 = v.reshape(B, v.shape[2], D) if not (v.stride(3) == 1 and v.stride(2) == D) else \
        v.as_strided((B, v.shape[2], D), (v.stride(0), D, 1))
    _require(tuple(k3.shape[1:]) == (hkv, D), "k/v head shape must match the cache")
    ks, vs = _token_rows(k3, "k"), _token_rows(v3, "v")
    rc = L.aac_decode_append_paged(
        q3.data_ptr(), q3.stride(0), k3.data_ptr(), v3.data_ptr(), ks, vs, k_cache.data_ptr(),
        v_cache.data_ptr(), nblk, bs, tables.data_ptr(), mb, seqlens.data_ptr(), B, mcl, Hq, hkv,
        D, _scale(softmax_scale, D), out.data_ptr(), Hq * D, wsp, ws_bytes, part,
        _dtype_code(q), _stream(q))
    _lib.check(rc, "aac_decode_append_paged")
    return out
