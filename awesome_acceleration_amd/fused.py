"""Python surface of the fused call-site kernels (RMSNorm + residual, q/k
RMSNorm + RoPE + KV store, SiLU * up).  Device tensors only; every op runs on
the current stream and fails loudly without the HIP library."""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib

__all__ = ["rmsnorm", "qk_norm_rope_store", "qkv_norm_rope_store", "silu_mul", "linear",
           "linear_supported", "rmsnorm_supported", "argmax"]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _req(cond: bool, msg: str):
    if not cond:
        raise RuntimeError(msg)


def _code(t: torch.Tensor) -> int:
    _req(t.dtype in (torch.bfloat16, torch.float16), f"unsupported dtype {t.dtype}")
    return _lib.AAC_DTYPE[t.dtype]


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: Optional[torch.Tensor] = None):
    """RMSNorm of ``x`` [rows, hidden] (model/model.py:47-52).  With
    ``residual``: returns ``(norm(x + residual), x + residual)``."""
    _req(x.is_cuda and x.dim() == 2 and x.stride(1) == 1, "x must be a [rows, hidden] GPU tensor")
    rows, hidden = x.shape
    out = torch.empty((rows, hidden), dtype=x.dtype, device=x.device)
    res_out = None
    if residual is not None:
        _req(residual.shape == x.shape and residual.is_contiguous(), "residual shape")
        res_out = torch.empty_like(residual)
    rc = _lib.lib().aac_rmsnorm(
        x.data_ptr(), x.stride(0), residual.data_ptr() if residual is not None else None,
        res_out.data_ptr() if res_out is not None else None, weight.data_ptr(), out.data_ptr(),
        rows, hidden, float(eps), _code(x), _stream(x))
    _lib.check(rc, "aac_rmsnorm")
    return out if residual is None else (out, res_out)


def _cache_args(T, n_kv_heads, k_cache, v_cache, slot_mapping, block_tables, cache_seqlens):
    """(rows, block_size, table width) of the K/V store arguments, checked."""
    rows = bs = mb = 0
    if v_cache is not None:
        _req(k_cache is not None and k_cache.shape == v_cache.shape and k_cache.is_contiguous()
             and v_cache.is_contiguous(), "caches must be contiguous and alike")
        rows = k_cache.numel() // (n_kv_heads * 128)
        if slot_mapping is None:
            _req(block_tables is not None and cache_seqlens is not None,
                 "append needs block_tables and cache_seqlens")
            _req(block_tables.dtype == torch.int32 and block_tables.is_contiguous()
                 and block_tables.shape[0] == T, "block_tables must be int32 [T, W]")
            _req(cache_seqlens.dtype == torch.int32 and cache_seqlens.shape == (T,),
                 "cache_seqlens must be int32 [T]")
            bs = k_cache.shape[1]
            mb = block_tables.shape[1]
        else:
            _req(slot_mapping.dtype == torch.int64 and slot_mapping.shape == (T,),
                 "slot_mapping must be int64 [T]")
    return rows, bs, mb


def qk_norm_rope_store(qkv: torch.Tensor, n_q_heads: int, n_kv_heads: int,
                       q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                       cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                       k_cache: Optional[torch.Tensor] = None,
                       v_cache: Optional[torch.Tensor] = None,
                       slot_mapping: Optional[torch.Tensor] = None,
                       block_tables: Optional[torch.Tensor] = None,
                       cache_seqlens: Optional[torch.Tensor] = None, want_k: bool = True):
    """q/k RMSNorm + RoPE of the fused projection ``qkv`` [T, (Hq+2Hkv)*128]
    (model/model.py:219-228) and, with caches, the K/V store through
    ``slot_mapping`` (llm.py:171-174) or the decode append at
    ``cache_seqlens`` of ``block_tables`` (model/model.py:233-240).
    Returns ``(q [T,Hq,128], k [T,Hkv,128] or None)``."""
    _req(qkv.is_cuda and qkv.dim() == 2 and qkv.stride(1) == 1, "qkv must be [T, width]")
    T = qkv.shape[0]
    D = 128
    _req(qkv.shape[1] == (n_q_heads + 2 * n_kv_heads) * D, "qkv width")
    _req(positions.dtype == torch.int32 and positions.shape == (T,), "positions must be int32 [T]")
    q = torch.empty((T, n_q_heads, D), dtype=qkv.dtype, device=qkv.device)
    k = torch.empty((T, n_kv_heads, D), dtype=qkv.dtype, device=qkv.device) if want_k else None
    rows, bs, mb = _cache_args(T, n_kv_heads, k_cache, v_cache, slot_mapping, block_tables,
                               cache_seqlens)
    rc = _lib.lib().aac_qk_norm_rope_store(
        qkv.data_ptr(), qkv.stride(0), T, n_q_heads, n_kv_heads, D, q_norm_weight.data_ptr(),
        k_norm_weight.data_ptr(), float(eps), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        positions.data_ptr(), q.data_ptr(), k.data_ptr() if k is not None else None,
        k_cache.data_ptr() if v_cache is not None else None,
        v_cache.data_ptr() if v_cache is not None else None, rows,
        slot_mapping.data_ptr() if slot_mapping is not None else None,
        block_tables.data_ptr() if (v_cache is not None and slot_mapping is None) else None, mb,
        cache_seqlens.data_ptr() if (v_cache is not None and slot_mapping is None) else None, bs,
        _code(qkv), _stream(qkv))
    _lib.check(rc, "aac_qk_norm_rope_store")
    return q, k


def qkv_norm_rope_store(x: torch.Tensor, w_qkv: torch.Tensor, n_q_heads: int, n_kv_heads: int,
                        q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                        cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                        k_cache: Optional[torch.Tensor] = None,
                        v_cache: Optional[torch.Tensor] = None,
                        slot_mapping: Optional[torch.Tensor] = None,
                        block_tables: Optional[torch.Tensor] = None,
                        cache_seqlens: Optional[torch.Tensor] = None, want_k: bool = True):
    """``qk_norm_rope_store(linear(x, w_qkv), ...)`` in one launch for a decode
    step's few tokens: the fused QKV projection (model/model.py:132-154), q/k
    RMSNorm + RoPE (model/model.py:219-228) and the K/V store or append,
    without the qkv intermediate.  Returns ``(q [T,Hq,128], k [T,Hkv,128] or None)``."""
    _req(x.is_cuda and x.dim() == 2 and x.stride(1) == 1, "x must be a [T, hidden] GPU tensor")
    T, hidden = x.shape
    D = 128
    _req(w_qkv.dim() == 2 and w_qkv.stride(1) == 1 and w_qkv.dtype == x.dtype
         and w_qkv.shape == ((n_q_heads + 2 * n_kv_heads) * D, hidden), "w_qkv shape")
    _req(positions.dtype == torch.int32 and positions.shape == (T,), "positions must be int32 [T]")
    q = torch.empty((T, n_q_heads, D), dtype=x.dtype, device=x.device)
    k = torch.empty((T, n_kv_heads, D), dtype=x.dtype, device=x.device) if want_k else None
    rows, bs, mb = _cache_args(T, n_kv_heads, k_cache, v_cache, slot_mapping, block_tables,
                               cache_seqlens)
    rc = _lib.lib().aac_qkv_norm_rope_store(
        x.data_ptr(), x.stride(0), w_qkv.data_ptr(), w_qkv.stride(0), T, hidden, n_q_heads,
        n_kv_heads, D, q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(eps),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0], positions.data_ptr(), q.data_ptr(),
        k.data_ptr() if k is not None else None,
        k_cache.data_ptr() if v_cache is not None else None,
        v_cache.data_ptr() if v_cache is not None else None, rows,
        slot_mapping.data_ptr() if slot_mapping is not None else None,
        block_tables.data_ptr() if (v_cache is not None and slot_mapping is None) else None, mb,
        cache_seqlens.data_ptr() if (v_cache is not None and slot_mapping is None) else None, bs,
        _code(x), _stream(x))
    _lib.check(rc, "aac_qkv_norm_rope_store")
    return q, k


def linear(x: torch.Tensor, weight: torch.Tensor, silu: bool = False,
           config: int = 0) -> torch.Tensor:
    """``F.linear(x, weight)`` for a decode step's small ``x`` [m, k]; with
    ``silu`` the weight is the fused [gate | up] projection [2I, k] and the
    result is ``silu(gate) * up`` [m, I] (model/model.py:188)."""
    _req(x.is_cuda and x.dim() == 2 and x.stride(1) == 1, "x must be a [m, k] GPU tensor")
    _req(weight.dim() == 2 and weight.stride(1) == 1 and weight.dtype == x.dtype,
         "weight must be [n, k] with contiguous rows, same dtype as x")
    m, k = x.shape
    _req(weight.shape[1] == k, "inner dimensions differ")
    n = weight.shape[0] // 2 if silu else weight.shape[0]
    _req(not silu or weight.shape[0] == 2 * n, "gate/up weight must have an even row count")
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    rc = _lib.lib().aac_gemm_nt(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                y.data_ptr(), y.stride(0), m, n, k, n if silu else 0, config,
                                _code(x), _stream(x))
    _lib.check(rc, "aac_gemm_nt")
    return y


def linear_supported(m: int, n: int, k: int) -> bool:
    """Whether aac_gemm_nt's own tiling choice (config 0) has a tiling for this
    shape: every tiling it picks from needs n % 32 == 0 and k % 128 == 0
    (whole 32-column output tiles, whole 128-element K stages)."""
    return m > 0 and n % 32 == 0 and k % 128 == 0


def rmsnorm_supported(hidden: int) -> bool:
    """Whether aac_rmsnorm handles rows of ``hidden`` elements (one wavefront
    per row, 8 elements per lane per pass: a multiple of 512, at most 4096)."""
    return hidden > 0 and hidden % 512 == 0 and hidden <= 4096


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` of the fused [gate | up] projection (model/model.py:188)."""
    _req(gate_up.is_cuda and gate_up.dim() == 2 and gate_up.is_contiguous(), "gate_up [rows, 2I]")
    rows, two_i = gate_up.shape
    out = torch.empty((rows, two_i // 2), dtype=gate_up.dtype, device=gate_up.device)
    rc = _lib.lib().aac_silu_mul(gate_up.data_ptr(), out.data_ptr(), rows, two_i // 2,
                                 _code(gate_up), _stream(gate_up))
    _lib.check(rc, "aac_silu_mul")
    return out


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """``logits.argmax(dim=-1)`` of a [rows, cols] GPU tensor (int64), the
    greedy sampler of llm.py:215-219: the first index of each row's maximum."""
    _req(logits.is_cuda and logits.dim() == 2 and logits.stride(1) == 1, "logits must be [rows, cols]")
    _req(logits.dtype in _lib.AAC_DTYPE, f"unsupported dtype {logits.dtype}")
    out = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    rc = _lib.lib().aac_argmax_rows(logits.data_ptr(), logits.stride(0), logits.shape[0],
                                    logits.shape[1], out.data_ptr(), _lib.AAC_DTYPE[logits.dtype],
                                    _stream(logits))
    _lib.check(rc, "aac_argmax_rows")
    return out
