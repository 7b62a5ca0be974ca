"""fp32 torch restatement of the attention hot path on the host.

TEST INFRASTRUCTURE ONLY -- bench.py's CPU baseline (configs 1-4 timed on
the host cores) and a cross-check of the numpy oracle; never the product.

The reference's CPU-runnable semantics, in fp32 on (bf16- or fp32-valued)
inputs:

* the store is the reference's own op, ``cache.view(-1, Hkv, D).index_copy_(
  0, slot_mapping, k)`` (llm.py:171-174);
* prefill attention is causal softmax attention per segment with query head
  ``h`` reading KV head ``h // g`` (flash_attn_varlen_func, llm.py:178-184),
  computed by torch's own ``scaled_dot_product_attention`` on the host;
* decode stores each new K/V at ``cache_seqlens[b]`` through the block table
  and attends over ``cache_seqlens[b] + 1`` tokens (flash_attn_with_kvcache
  with k=/v=, model/model.py:233-241).

Checked against the float64 oracle (oracle/attention.py) in
tests/test_oracle_pins.py: stores bit-exact, attention within fp32 rounding.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["prefill_store_attend", "decode_store_attend", "cpu_threads"]


def _store(cache: torch.Tensor, rows: torch.Tensor, x: torch.Tensor) -> None:
    hkv, d = x.shape[-2], x.shape[-1]
    cache.view(-1, hkv, d).index_copy_(0, rows, x.to(cache.dtype))


def prefill_store_attend(q, k, v, cu_seqlens, k_cache, v_cache, slot_mapping, scale,
                         causal: bool = True) -> torch.Tensor:
    """q ``[N, Hq, D]``, k/v ``[N, Hkv, D]``, ``cu_seqlens`` int ``[n+1]``
    (host list or tensor), caches ``[..., Hkv, D]``, ``slot_mapping`` int64
    ``[N]``.  Stores k/v, returns the fp32 attention output ``[N, Hq, D]``."""
    _store(k_cache, slot_mapping, k)
    _store(v_cache, slot_mapping, v)
    cu = [int(c) for c in cu_seqlens]
    out = torch.empty(q.shape, dtype=torch.float32)
    for a, b in zip(cu[:-1], cu[1:]):
        if b == a:
            continue
        qs = q[a:b].float().transpose(0, 1)  # [Hq, L, D]
        ks = k[a:b].float().transpose(0, 1)  # [Hkv, L, D]
        vs = v[a:b].float().transpose(0, 1)
        o = F.scaled_dot_product_attention(qs, ks, vs, is_causal=causal, scale=scale,
                                           enable_gqa=True)
        out[a:b] = o.transpose(0, 1)
    return out


def decode_store_attend(q, k_new, v_new, k_cache, v_cache, block_tables, cache_seqlens,
                        scale) -> torch.Tensor:
    """q ``[B, Hq, D]``, k_new/v_new ``[B, Hkv, D]``, paged caches
    ``[num_blocks, block_size, Hkv, D]``, ``block_tables`` int ``[B, W]``,
    ``cache_seqlens`` ``[B]`` (before the append).  Stores the new tokens,
    returns the fp32 attention output ``[B, Hq, D]`` over ``cache_seqlens+1``
    tokens of each sequence."""
    bs, hkv, d = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    lens = [int(x) for x in cache_seqlens]
    bt = torch.as_tensor(block_tables, dtype=torch.int64)
    pos = torch.tensor(lens, dtype=torch.int64)
    rows = bt[torch.arange(len(lens)), pos // bs] * bs + pos % bs
    _store(k_cache, rows, k_new)
    _store(v_cache, rows, v_new)
    out = torch.empty(q.shape, dtype=torch.float32)
    for b, n in enumerate(lens):
        ctx = n + 1
        nb = -(-ctx // bs)
        kb = k_cache[bt[b, :nb]].reshape(-1, hkv, d)[:ctx].float().transpose(0, 1)
        vb = v_cache[bt[b, :nb]].reshape(-1, hkv, d)[:ctx].float().transpose(0, 1)
        qb = q[b].float()[:, None, :]  # [Hq, 1, D]
        out[b] = F.scaled_dot_product_attention(qb, kb, vb, scale=scale,
                                                enable_gqa=True)[:, 0, :]
    return out


def cpu_threads() -> int:
    """Host threads for a CPU baseline: every core this process may run on,
    capped by OMP_NUM_THREADS when the job sets it (its CPU share)."""
    import os
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n
