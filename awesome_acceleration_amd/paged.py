"""Host-side paged-KV bookkeeping: block allocation and per-step metadata.

The reference keeps one contiguous slot of ``max_seq_len`` tokens per
sequence and hands out slot ids lowest-first from a sorted free list
(engine/cache_manager.py:5-30, inlined in llm.py:318/354/377/436).  The
paged cache generalises a slot to a list of fixed-size blocks; the slot
layout is the special case ``block_size = max_seq_len`` with one block per
sequence, which ``slot_block_tables`` builds so the reference's caches work
unchanged.

Metadata produced here mirrors llm.py:127-140 (``cu_seqlens``, positions and
the flat scatter index, called ``slot_mapping``), generalised to block
tables, and is shipped to the device with a single host-to-device copy per
tensor.
"""
from __future__ import annotations

import bisect
import math
from typing import Iterable, Sequence

import numpy as np
import torch

__all__ = [
    "SlotCacheManager",
    "BlockAllocator",
    "slot_block_tables",
    "blocks_needed",
    "prefill_slot_mapping",
    "decode_slot_mapping",
    "build_prefill_metadata",
    "pad_block_tables",
    "check_slots",
    "padded_prefill_slot_mapping",
    "KV_SKEW_BYTES",
    "alloc_kv_storage",
    "alloc_kv_cache",
]


class SlotCacheManager:
    """Lowest-free-first slot allocator with the reference's interface
    (engine/cache_manager.py:5-30)."""

    def __init__(self, max_num_seqs: int):
        self.max_num_seqs = max_num_seqs
        self.free_slots = list(range(max_num_seqs))
        self.used_slots: set[int] = set()

    def allocate_slot(self) -> int:
        if not self.free_slots:
            raise RuntimeError("No free slots available")
        slot = self.free_slots.pop(0)
        self.used_slots.add(slot)
        return slot

    def free_slot(self, slot: int) -> None:
        if slot in self.used_slots:
            self.used_slots.remove(slot)
            bisect.insort(self.free_slots, slot)

    def reset(self) -> None:
        self.free_slots = list(range(self.max_num_seqs))
        self.used_slots.clear()


class BlockAllocator:
    """Fixed-size KV block pool, lowest-free-first like the slot allocator.

    ``allocate(n)`` returns ``n`` block ids or raises ``RuntimeError`` when
    the pool cannot supply them (the pool is left unchanged).  ``free``
    returns ids to the pool; freeing an id that is not allocated is ignored,
    as ``SlotCacheManager.free_slot`` ignores unknown slots.
    """

    def __init__(self, num_blocks: int):
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        self.num_blocks = num_blocks
        self._free = list(range(num_blocks))
        self._used: set[int] = set()

    @property
    def num_free(self) -> int:
        return len(self._free)

    def allocate(self, n: int) -> list[int]:
        if n < 0:
            raise ValueError("n must be >= 0")
        if n > len(self._free):
            raise RuntimeError(f"No free blocks available (need {n}, have {len(self._free)})")
        out, self._free = self._free[:n], self._free[n:]
        self._used.update(out)
        return out

    def free(self, blocks: Iterable[int]) -> None:
        for b in blocks:
            if b in self._used:
                self._used.remove(b)
                bisect.insort(self._free, b)

    def reset(self) -> None:
        self._free = list(range(self.num_blocks))
        self._used.clear()


# Distance of each layer's V cache from its K cache, modulo 1 KiB.  The decode
# kernel reads token t's K and V rows of one KV head together; when the two
# caches start at the same address modulo 1 KiB (as two separate large
# allocations do, being 2 MiB-aligned) those reads share address bits 8-9,
# and on MI355X decode attention then runs 2-4% slower than with the V cache
# 512 bytes further on (256 seqs x 1-2k at 16/8 heads: 248.5 against 238.0 us;
# 64 x 16k-32k at 32/8: 1062 against 1037-1040 us; 8/4 heads: 129.7 against
# 124.0 us; offsets of 1, 2, 4, 8 KiB and more measured like 0, 256 and 768
# bytes in between).
KV_SKEW_BYTES = 512


def alloc_kv_storage(n_layers: int, num_blocks: int, block_size: int, n_kv_heads: int,
                     head_dim: int, *, dtype: torch.dtype, device) -> torch.Tensor:
    """Zero-filled K/V caches of ``n_layers`` layers as one strided tensor
    ``[n_layers, 2, num_blocks, block_size, Hkv, D]`` (``[layer, 0]`` the K
    cache, ``[layer, 1]`` the V cache, each contiguous), with every V cache
    ``KV_SKEW_BYTES`` past a 1 KiB multiple from its K cache.  The layout the
    reference allocates (model/model.py:324-335, one zero tensor per cache) is
    the same per cache; only the caches' relative placement differs."""
    es = torch.empty((), dtype=dtype).element_size()
    if KV_SKEW_BYTES % es or 1024 % es:
        raise ValueError(f"element size {es} does not divide the 512-byte skew")
    part = num_blocks * block_size * n_kv_heads * head_dim  # elements of one cache
    unit = 1024 // es
    dist = -(-part // unit) * unit + KV_SKEW_BYTES // es     # K -> V distance, elements
    flat = torch.zeros(n_layers * 2 * dist, dtype=dtype, device=device)
    return flat.as_strided((n_layers, 2, num_blocks, block_size, n_kv_heads, head_dim),
                           (2 * dist, dist, block_size * n_kv_heads * head_dim,
                            n_kv_heads * head_dim, head_dim, 1))


def alloc_kv_cache(num_blocks: int, block_size: int, n_kv_heads: int, head_dim: int, *,
                   dtype: torch.dtype, device) -> tuple[torch.Tensor, torch.Tensor]:
    """One layer's zero-filled ``(k_cache, v_cache)``, each a contiguous
    ``[num_blocks, block_size, Hkv, D]`` tensor, placed as ``alloc_kv_storage``
    places them (the drop-in for model/model.py:328-335's two ``torch.zeros``)."""
    s = alloc_kv_storage(1, num_blocks, block_size, n_kv_heads, head_dim, dtype=dtype, device=device)
    return s[0, 0], s[0, 1]


def blocks_needed(n_tokens: int, block_size: int) -> int:
    return max(0, math.ceil(n_tokens / block_size))


def slot_block_tables(slot_indices: Sequence[int]) -> np.ndarray:
    """Block tables of the reference's slot layout: one block (= slot) per sequence."""
    return np.asarray(slot_indices, dtype=np.int32).reshape(-1, 1)


def pad_block_tables(tables: Sequence[Sequence[int]], width: int | None = None,
                     fill: int = 0) -> np.ndarray:
    """Rectangular int32 ``[B, width]`` array from ragged block lists."""
    width = width if width is not None else max((len(t) for t in tables), default=1)
    out = np.full((len(tables), max(width, 1)), fill, dtype=np.int32)
    for i, t in enumerate(tables):
        if len(t) > width:
            raise ValueError("block list longer than the table width")
        out[i, :len(t)] = t
    return out


def check_slots(slots: np.ndarray, num_cache_rows: int) -> None:
    """Raise ``IndexError`` unless every slot is a row of the cache, as the
    reference's ``index_copy_`` into ``[num_cache_rows, Hkv, D]`` rejects an
    index outside ``[0, num_cache_rows)`` (llm.py:171-174).  Host-side: the
    engine builds its slot mappings here, so the check costs no device sync."""
    s = np.asarray(slots)
    if s.size and (int(s.min()) < 0 or int(s.max()) >= num_cache_rows):
        bad = int(s.min()) if int(s.min()) < 0 else int(s.max())
        raise IndexError(f"index {bad} is out of bounds for dimension 0 with size {num_cache_rows}")


def _table_rows(bt: np.ndarray, rows: np.ndarray, p: np.ndarray, block_size: int) -> np.ndarray:
    """Cache rows of positions ``p`` of sequences ``rows`` through the tables;
    a position past a table's width raises ``IndexError``."""
    blk = p // block_size
    if blk.size and (int(blk.min()) < 0 or int(blk.max()) >= bt.shape[1]):
        raise IndexError(f"position {int(p.max())} is past the block table "
                         f"({bt.shape[1]} blocks of {block_size})")
    return bt[rows, blk] * block_size + p % block_size


def prefill_slot_mapping(block_tables: np.ndarray, seq_lens: Sequence[int], block_size: int,
                         start_positions: Sequence[int] | None = None,
                         num_cache_rows: int | None = None) -> np.ndarray:
    """Flat cache row of every packed prefill token (paged form of llm.py:139-140).

    With ``num_cache_rows`` every row is checked against the cache
    (``IndexError`` as ``index_copy_`` raises)."""
    bt = np.asarray(block_tables, dtype=np.int64)
    parts = []
    for b, L in enumerate(seq_lens):
        p0 = 0 if start_positions is None else int(start_positions[b])
        p = np.arange(p0, p0 + int(L), dtype=np.int64)
        parts.append(_table_rows(bt, np.full(p.shape, b), p, block_size))
    out = np.concatenate(parts) if parts else np.zeros(0, dtype=np.int64)
    if num_cache_rows is not None:
        check_slots(out, num_cache_rows)
    return out


def decode_slot_mapping(block_tables: np.ndarray, positions: Sequence[int],
                        block_size: int, num_cache_rows: int | None = None) -> np.ndarray:
    """Flat cache row of the token each decode sequence appends at ``positions[b]``
    (checked against the cache with ``num_cache_rows``, as above)."""
    bt = np.asarray(block_tables, dtype=np.int64)
    p = np.asarray(positions, dtype=np.int64)
    out = _table_rows(bt, np.arange(p.shape[0]), p, block_size)
    if num_cache_rows is not None:
        check_slots(out, num_cache_rows)
    return out


def padded_prefill_slot_mapping(slot_indices: Sequence[int], seq_lens: Sequence[int],
                                padded_len: int, max_seq_len: int) -> np.ndarray:
    """Slot mapping that turns the padded prefill branch's per-slot stores
    ``k_cache[slot_i, :L_i] = k[i, :L_i]`` (model/model.py:244-250, over
    ``k [B, T, Hkv, D]`` flattened to ``[B*T, Hkv, D]``) into one ``kv_store``
    call: token ``t`` of row ``i`` goes to cache row ``slot_i * max_seq_len + t``
    for ``t < L_i``; padding tokens get -1, which the store skips."""
    B, T = len(slot_indices), int(padded_len)
    if len(seq_lens) != B:
        raise ValueError("one sequence length per slot")
    out = np.full((B, T), -1, dtype=np.int64)
    t = np.arange(T, dtype=np.int64)
    for i, (slot, L) in enumerate(zip(slot_indices, seq_lens)):
        if not 0 <= int(L) <= min(T, max_seq_len):
            raise ValueError(f"sequence length {L} outside [0, min(padded_len, max_seq_len)]")
        out[i, :L] = int(slot) * max_seq_len + t[:L]
    return out.reshape(-1)


def build_prefill_metadata(seq_lens: Sequence[int], block_tables: np.ndarray, block_size: int,
                           device: torch.device | str, num_cache_rows: int | None = None):
    """``(cu_seqlens int32 [n+1], positions int64 [N], slot_mapping int64 [N])`` on ``device``.

    Same values as llm.py:129-140 for the slot layout; each tensor is built on
    the host and copied once (the reference issues one small copy per list
    and a device-side ``repeat_interleave``).  With ``num_cache_rows`` a slot
    outside the cache raises ``IndexError`` before anything is copied, the
    error the reference's ``index_copy_`` store raises (llm.py:171-174).
    """
    lens = np.asarray(seq_lens, dtype=np.int64)
    cu = np.zeros(lens.shape[0] + 1, dtype=np.int32)
    np.cumsum(lens, out=cu[1:])
    positions = (np.concatenate([np.arange(L, dtype=np.int64) for L in lens])
                 if lens.size else np.zeros(0, dtype=np.int64))
    slots = prefill_slot_mapping(block_tables, lens, block_size, num_cache_rows=num_cache_rows)
    to = lambda a: torch.from_numpy(a).to(device, non_blocking=False)  # noqa: E731
    return to(cu), to(positions), to(slots)
