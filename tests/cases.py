"""Seeded input generators shared by the CPU and GPU tests and the fixture script.

Inputs come from ``np.random.RandomState(seed)`` -- numpy's frozen legacy
MT19937 stream -- so the same arrays are regenerated bit-identically on any
machine; committed fixtures only need to hold outputs and input digests.
"""
from __future__ import annotations

import hashlib

import numpy as np

import oracle


def sha256(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return oracle.f32_to_bf16_bits(x.astype(np.float32))


def ragged_block_tables(ctx, block_size, perm, width=None, fill=-1):
    """Blocks for each sequence taken in order from ``perm`` (unused entries = fill)."""
    need = [int(np.ceil(c / block_size)) for c in ctx]
    width = width or max(need)
    bt = np.full((len(ctx), width), fill, dtype=np.int32)
    k = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k:k + n]
        k += n
    return bt


# --------------------------------------------------------------------------
# Single-layer Qwen3-0.6B paged decode, fp32, seed 0: batch 4, 16 query
# heads, 8 KV heads, head_dim 128, post-store context lengths
# {17, 64, 200, 511}, KV block 256, blocks taken in order from a random
# permutation of a 16-block pool.  Each step stores the new token, then
# attends.
# --------------------------------------------------------------------------
CFG1 = dict(B=4, HQ=16, HKV=8, D=128, BS=256, POOL=16, CTX=(17, 64, 200, 511))


def config1_inputs():
    c = CFG1
    rs = np.random.RandomState(0)
    perm = rs.permutation(c["POOL"]).astype(np.int32)
    q = rs.standard_normal((c["B"], c["HQ"], c["D"])).astype(np.float32)
    k_new = rs.standard_normal((c["B"], c["HKV"], c["D"])).astype(np.float32)
    v_new = rs.standard_normal((c["B"], c["HKV"], c["D"])).astype(np.float32)
    k_cache = rs.standard_normal((c["POOL"], c["BS"], c["HKV"], c["D"])).astype(np.float32)
    v_cache = rs.standard_normal((c["POOL"], c["BS"], c["HKV"], c["D"])).astype(np.float32)
    ctx = np.asarray(c["CTX"], dtype=np.int32)
    bt = ragged_block_tables(ctx, c["BS"], perm)
    cache_seqlens = (ctx - 1).astype(np.int32)
    return dict(q=q, k_new=k_new, v_new=v_new, k_cache=k_cache, v_cache=v_cache,
                block_tables=bt, cache_seqlens=cache_seqlens, context_lens=ctx,
                block_size=c["BS"], scale=c["D"] ** -0.5)


# --------------------------------------------------------------------------
# Tiny bf16 cases whose inputs are stored whole in the fixtures.
# --------------------------------------------------------------------------
def tiny_prefill_inputs():
    rs = np.random.RandomState(1)
    lens = [1, 5, 12, 3]
    n = sum(lens)
    hq, hkv, d = 4, 2, 128
    q = to_bf16_bits(rs.standard_normal((n, hq, d)))
    k = to_bf16_bits(rs.standard_normal((n, hkv, d)))
    v = to_bf16_bits(rs.standard_normal((n, hkv, d)))
    cu = np.zeros(len(lens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(lens)
    return dict(q=q, k=k, v=v, cu_seqlens=cu, scale=d ** -0.5)


def tiny_decode_inputs():
    rs = np.random.RandomState(2)
    B, hq, hkv, d, bs, pool = 3, 8, 2, 128, 16, 10
    ctx = np.asarray([1, 16, 37], dtype=np.int32)
    perm = rs.permutation(pool).astype(np.int32)
    q = to_bf16_bits(rs.standard_normal((B, hq, d)))
    k_new = to_bf16_bits(rs.standard_normal((B, hkv, d)))
    v_new = to_bf16_bits(rs.standard_normal((B, hkv, d)))
    k_cache = to_bf16_bits(rs.standard_normal((pool, bs, hkv, d)))
    v_cache = to_bf16_bits(rs.standard_normal((pool, bs, hkv, d)))
    bt = ragged_block_tables(ctx, bs, perm)
    return dict(q=q, k_new=k_new, v_new=v_new, k_cache=k_cache, v_cache=v_cache,
                block_tables=bt, cache_seqlens=(ctx - 1).astype(np.int32), context_lens=ctx,
                block_size=bs, scale=d ** -0.5)
