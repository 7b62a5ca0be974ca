"""KV export / import of one sequence over the paged cache (the PD payload).

The reference moves a finished prefill's KV cache to the decode side as
``{"layers": [{"k": Tensor[length, Hkv, D], "v": ..., "seqlen": int}, ...]}``
with CPU tensors (``export_kv`` / ``import_kv``, model/model.py:156-177;
``export_request_kv`` / ``import_request_kv``, model/model.py:386-401;
shipped by pd/kv_connector_shm.py:97-151), slicing and copying each layer
separately.  Here one HIP launch gathers every layer's K and V rows of a
sequence through its block table into a contiguous device buffer
``[n_layers, 2, length, Hkv, D]`` (``aac_kv_export_paged``) and one copy
moves it to pinned host memory; the payload tensors are views of that host
buffer.  Import is the reverse: one host-to-device copy and one scatter
launch (``aac_kv_import_paged``) into the blocks the receiving side chose.

The cache is the engine's single tensor ``[n_layers, 2, num_blocks,
block_size, Hkv, D]`` (``qwen3.PagedKVCache.storage``); the reference's slot
cache is the special case ``block_size = max_seq_len``, ``block_table =
[slot]``.  Block-table entries outside ``[0, num_blocks)`` export zeros and
are skipped on import.  ``seqlen`` travels with the payload and, as in the
reference, is the caller's to apply.
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _lib
from .flash_attn_interface import _dtype_code, _require, _stream

__all__ = ["kv_export", "kv_import", "export_request_kv", "import_request_kv"]


def _check_storage(storage: torch.Tensor) -> None:
    _require(storage.is_cuda, "the KV cache must be on a GPU (no CPU path exists)")
    _require(storage.dim() == 6 and storage.shape[1] == 2,
             "KV storage must be [n_layers, 2, num_blocks, block_size, Hkv, D]")
    _, _, nb, bs, hkv, d = storage.shape
    _require(storage.stride()[2:] == (bs * hkv * d, hkv * d, d, 1),
             "each layer's K and V cache in the KV storage must be contiguous")
    _require(storage.stride(1) >= nb * bs * hkv * d and storage.stride(0) >= 2 * storage.stride(1),
             "the KV storage's layer and K/V strides must not overlap its caches")


def _table(block_table, device) -> torch.Tensor:
    if isinstance(block_table, torch.Tensor):
        t = block_table.to(device=device, dtype=torch.int32).reshape(-1).contiguous()
    else:
        t = torch.tensor(list(block_table), dtype=torch.int32, device=device)
    return t


def kv_export(storage: torch.Tensor, block_table, length: int,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """Gather the first ``length`` tokens of one sequence (all layers, K and V)
    into ``out`` = ``[n_layers, 2, length, Hkv, D]`` on the cache's device."""
    _check_storage(storage)
    L, _, nb, bs, hkv, d = storage.shape
    bt = _table(block_table, storage.device)
    if out is None:
        out = torch.empty((L, 2, length, hkv, d), dtype=storage.dtype, device=storage.device)
    _require(out.shape == (L, 2, length, hkv, d) and out.dtype == storage.dtype
             and out.is_contiguous() and out.device == storage.device,
             "out must be a contiguous [n_layers, 2, length, Hkv, D] tensor like the cache")
    per_layer = storage.stride(0)
    _lib.check(_lib.lib().aac_kv_export_paged(
        storage.data_ptr(), per_layer, storage.stride(1), L, nb, bs, hkv, d, bt.data_ptr(),
        bt.numel(), length, out.data_ptr(), _dtype_code(storage), _stream(storage)), "kv_export")
    return out


def kv_import(src: torch.Tensor, storage: torch.Tensor, block_table, length: int) -> None:
    """Scatter ``src`` = ``[n_layers, 2, >= length, Hkv, D]`` (device) into the
    paged cache through ``block_table``."""
    _check_storage(storage)
    L, _, nb, bs, hkv, d = storage.shape
    _require(src.is_cuda and src.device == storage.device and src.dtype == storage.dtype,
             "src must be on the cache's device with the cache's dtype")
    _require(src.dim() == 5 and src.shape[0] == L and src.shape[1] == 2 and src.shape[2] >= length
             and tuple(src.shape[3:]) == (hkv, d), "src must be [n_layers, 2, length, Hkv, D]")
    if src.shape[2] != length or not src.is_contiguous():
        src = src[:, :, :length].contiguous()
    bt = _table(block_table, storage.device)
    _lib.check(_lib.lib().aac_kv_import_paged(
        src.data_ptr(), storage.data_ptr(), storage.stride(0), storage.stride(1), L, nb, bs, hkv,
        d, bt.data_ptr(), bt.numel(), length, _dtype_code(storage), _stream(storage)), "kv_import")


def export_request_kv(storage: torch.Tensor, block_table, length: int, seqlen: int) -> dict:
    """The reference's ``export_request_kv`` payload for one sequence:
    ``{"layers": [{"k": [length, Hkv, D] CPU, "v": ..., "seqlen": seqlen}]}``.
    Synchronises the current stream (the payload is host data)."""
    dev_buf = kv_export(storage, block_table, length)
    host = torch.empty(dev_buf.shape, dtype=dev_buf.dtype, pin_memory=True)
    host.copy_(dev_buf, non_blocking=True)
    torch.cuda.current_stream(storage.device).synchronize()
    return {"layers": [{"k": host[i, 0], "v": host[i, 1], "seqlen": int(seqlen)}
                       for i in range(host.shape[0])]}


def import_request_kv(storage: torch.Tensor, block_table, payload: dict, length: int) -> int:
    """The reference's ``import_request_kv``: write the payload's first
    ``length`` tokens of every layer into the sequence's blocks; returns the
    payload's ``seqlen`` (for the caller's cache length bookkeeping)."""
    _check_storage(storage)
    layers: Sequence[dict] = payload["layers"]
    L, _, _, _, hkv, d = storage.shape
    if len(layers) != L:
        raise ValueError(f"Layer count mismatch: payload has {len(layers)}, model has {L}")
    host = torch.empty((L, 2, length, hkv, d), dtype=storage.dtype, pin_memory=True)
    for i, lp in enumerate(layers):
        host[i, 0].copy_(lp["k"][:length].to(dtype=storage.dtype).reshape(length, hkv, d))
        host[i, 1].copy_(lp["v"][:length].to(dtype=storage.dtype).reshape(length, hkv, d))
    dev_buf = host.to(storage.device, non_blocking=True)
    kv_import(dev_buf, storage, block_table, length)
    seqlens = {int(lp["seqlen"]) for lp in layers}
    _require(len(seqlens) == 1, "payload layers disagree on seqlen")
    return seqlens.pop()
