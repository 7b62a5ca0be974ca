"""Qwen3 decoder whose attention runs on the gfx950 kernels.

Mirrors the reference's single-GPU model (model/model.py): fused QKV
projection (model/model.py:132-154), per-head q/k RMSNorm
(model/model.py:40-52, :225-226), RoPE applied in the activation dtype
(model/model.py:55-99, :228), and the attention call site
(TransformerBlock.forward, model/model.py:202-267).  Differences, all on the
hot path:

* The KV cache is paged: per layer one K and one V tensor of shape
  ``[num_blocks, block_size, Hkv, D]`` (model/model.py:324-336 keeps one
  ``max_seq_len`` slot per sequence -- the special case of one block per
  sequence).
* Prefill stores K/V through ``slot_mapping`` and runs causal varlen
  attention in one library call (llm.py:171-184); decode appends the new K/V
  at ``cache_seqlens`` and attends (model/model.py:233-240).  The caller keeps
  ``cache_seqlens`` (model/model.py:241 increments it after the call).
* RoPE cos/sin come from a table precomputed for ``max_position`` tokens, so
  no per-layer ``position_ids.max().item()`` host sync (model/model.py:82).

Weights are random-initialised (no checkpoint is available offline);
``init_weights`` draws them from N(0, 0.02) with RMSNorm weights at 1, which
keeps activations finite through all layers.
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import flash_attn_interface as fai
from . import fused as fz
from . import kv_transfer
from . import paged

__all__ = ["Qwen3Config", "Qwen3ForCausalLM", "PagedKVCache", "StepMeta"]


@dataclass
class Qwen3Config:
    """Same fields and defaults as the reference's Qwen3Config (model/model.py:13-37)."""
    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    max_position_embeddings: int = 40960
    rope_theta: float = 1000000.0
    rms_norm_eps: float = 1e-6
    hidden_act: str = "silu"
    tie_word_embeddings: bool = True
    bos_token_id: int = 151643
    eos_token_id: int = 151645

    @classmethod
    def from_json(cls, path: str):
        with open(path) as f:
            data = json.load(f)
        return cls(**{k: v for k, v in data.items() if k in cls.__annotations__})


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm with the reference's numerics (model/model.py:47-52): statistics
    in fp32, normalised value cast back to the input dtype, then scaled."""
    dt = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(dt)


class Rope:
    """cos/sin tables in the activation dtype (model/model.py:64-78), indexed
    by position on the device."""

    def __init__(self, head_dim: int, max_pos: int, theta: float, device, dtype):
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        t = torch.arange(max_pos, dtype=torch.float32)
        freqs = torch.outer(t, inv)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos = emb.cos().to(device=device, dtype=dtype)
        self.sin = emb.sin().to(device=device, dtype=dtype)
        self.half = head_dim // 2

    def apply(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """x [T, H, D], positions [T] -> x*cos + rotate_half(x)*sin (model/model.py:86-99)."""
        cos = self.cos[positions].unsqueeze(1)
        sin = self.sin[positions].unsqueeze(1)
        x1, x2 = x[..., :self.half], x[..., self.half:]
        rot = torch.cat((-x2, x1), dim=-1)
        return x * cos + rot * sin


class PagedKVCache:
    """Per-layer paged K/V caches ``[num_blocks, block_size, Hkv, D]``,
    zero-initialised like model/model.py:328-335, in one strided storage
    ``[n_layers, 2, ...]`` whose V caches sit 512 bytes (modulo 1 KiB) from
    their K caches (``paged.alloc_kv_storage``)."""

    def __init__(self, cfg: Qwen3Config, num_blocks: int, block_size: int, device, dtype):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.storage = paged.alloc_kv_storage(cfg.num_hidden_layers, num_blocks, block_size,
                                              cfg.num_key_value_heads, cfg.head_dim,
                                              dtype=dtype, device=device)

    def k(self, layer: int) -> torch.Tensor:
        return self.storage[layer, 0]

    def v(self, layer: int) -> torch.Tensor:
        return self.storage[layer, 1]

    @property
    def nbytes(self) -> int:
        return self.storage.untyped_storage().nbytes()

    def export_request_kv(self, block_table, length: int, seqlen: int) -> dict:
        """The reference's export_request_kv (model/model.py:386-390) for the
        sequence whose blocks are ``block_table``."""
        return kv_transfer.export_request_kv(self.storage, block_table, length, seqlen)

    def import_request_kv(self, block_table, payload: dict, length: int) -> int:
        """The reference's import_request_kv (model/model.py:392-401) into the
        blocks ``block_table``; returns the payload's seqlen."""
        return kv_transfer.import_request_kv(self.storage, block_table, payload, length)


@dataclass
class StepMeta:
    """Device-side metadata of one forward pass.

    prefill: ``cu_seqlens`` int32 [n+1], ``positions`` int64 [N],
             ``slot_mapping`` int64 [N], ``max_seqlen``, ``last_idx`` int64 [n]
    decode:  ``positions`` int32 [B], ``block_tables`` int32 [B, W],
             ``cache_seqlens`` int32 [B] (length before this step's append),
             ``context_lens`` int32 [B] (= cache_seqlens + 1),
             ``max_context_len`` (upper bound on cache_seqlens + 1)
    """
    positions: torch.Tensor
    cu_seqlens: torch.Tensor | None = None
    slot_mapping: torch.Tensor | None = None
    max_seqlen: int = 0
    last_idx: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    cache_seqlens: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    max_context_len: int = 0


class Qwen3ForCausalLM:
    """Random-initialised Qwen3 with tied embeddings (model/model.py:289-322)."""

    def __init__(self, cfg: Qwen3Config, device, dtype=torch.bfloat16, seed: int = 0,
                 fused: bool = True):
        self.cfg = cfg
        # the fused call-site kernels need head_dim 128 and a hidden size the
        # RMSNorm kernel covers; other shapes run the unfused torch layer
        self.fused = (fused and cfg.head_dim == 128
                      and fz.rmsnorm_supported(cfg.hidden_size))
        self.device = torch.device(device)
        self.dtype = dtype
        self.hq, self.hkv, self.d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.q_size = self.hq * self.d
        self.kv_size = self.hkv * self.d
        self.scale = self.d ** -0.5
        # decode steps up to this many sequences use the decode-batch GEMM
        # (its tiles assume a few hundred rows at most)
        self.small_gemm_rows = 512
        self.init_weights(seed)
        H, I = cfg.hidden_size, cfg.intermediate_size
        if self.d != 128 or H % 128 or not all(fz.linear_supported(1, n, k) for n, k in (
                (self.q_size + 2 * self.kv_size, H), (H, self.q_size), (I, H), (H, I))):
            self.small_gemm_rows = 0  # a shape the decode-batch GEMM has no tiling for
        self.rope = Rope(self.d, cfg.max_position_embeddings, cfg.rope_theta, self.device, dtype)

    @torch.no_grad()
    def init_weights(self, seed: int, std: float = 0.02):
        cfg, dev, dt = self.cfg, self.device, self.dtype
        g = torch.Generator(device=dev).manual_seed(seed)

        def rnd(*shape):
            return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std).to(dt)

        H, I = cfg.hidden_size, cfg.intermediate_size
        self.embed = rnd(cfg.vocab_size, H)
        self.layers = []
        for _ in range(cfg.num_hidden_layers):
            self.layers.append(dict(
                ln1=torch.ones(H, device=dev, dtype=dt),
                ln2=torch.ones(H, device=dev, dtype=dt),
                q_norm=torch.ones(self.d, device=dev, dtype=dt),
                k_norm=torch.ones(self.d, device=dev, dtype=dt),
                qkv=rnd(self.q_size + 2 * self.kv_size, H),   # fused [Q | K | V]
                o=rnd(H, self.q_size),
                gate_up=rnd(2 * I, H),                         # fused [gate | up]
                down=rnd(H, I),
            ))
        self.norm = torch.ones(H, device=dev, dtype=dt)

    # ---------------------------------------------------------------- layers
    def _qkv(self, L, h, positions):
        """Fused QKV, q/k RMSNorm, RoPE.  Returns q [T,Hq,D], k [T,Hkv,D] (new
        tensors) and v [T,Hkv,D] (a strided view of the qkv buffer, as at
        llm.py:156)."""
        T = h.shape[0]
        eps = self.cfg.rms_norm_eps
        qkv = F.linear(h, L["qkv"])
        q = qkv[:, :self.q_size].view(T, self.hq, self.d)
        k = qkv[:, self.q_size:self.q_size + self.kv_size].view(T, self.hkv, self.d)
        v = qkv[:, self.q_size + self.kv_size:].view(T, self.hkv, self.d)
        q = rms_norm(q, L["q_norm"], eps)
        k = rms_norm(k, L["k_norm"], eps)
        q = self.rope.apply(q, positions)
        k = self.rope.apply(k, positions)
        return q, k, v

    def _mlp(self, L, h):
        gu = F.linear(h, L["gate_up"])
        I = self.cfg.intermediate_size
        return F.linear(F.silu(gu[:, :I]) * gu[:, I:], L["down"])

    def _layer(self, li, h, meta: StepMeta, cache: PagedKVCache, prefill: bool):
        L = self.layers[li]
        eps = self.cfg.rms_norm_eps
        res = h
        x = rms_norm(h, L["ln1"], eps)
        q, k, v = self._qkv(L, x, meta.positions)
        if prefill:
            # store K/V through slot_mapping and attend (llm.py:171-184)
            attn = fai.varlen_prefill_with_kvcache(
                q, k, v, meta.cu_seqlens, meta.max_seqlen, cache.k(li), cache.v(li),
                meta.slot_mapping, softmax_scale=self.scale, causal=True)
        else:
            # append at cache_seqlens and attend (model/model.py:233-240)
            B = q.shape[0]
            attn = fai.flash_attn_with_kvcache(
                q.view(B, 1, self.hq, self.d), cache.k(li), cache.v(li),
                k=k.view(B, 1, self.hkv, self.d), v=v.view(B, 1, self.hkv, self.d),
                cache_seqlens=meta.cache_seqlens, block_table=meta.block_tables,
                softmax_scale=self.scale, causal=False, max_context_len=meta.max_context_len)
        h = res + F.linear(attn.reshape(q.shape[0], -1), L["o"])
        res = h
        h = res + self._mlp(L, rms_norm(h, L["ln2"], eps))
        return h

    def _forward_fused(self, input_ids, meta: StepMeta, cache: PagedKVCache, prefill: bool):
        """The same layer with the fused call-site kernels: residual add +
        RMSNorm, q/k RMSNorm + RoPE + KV store/append, SiLU * up are one launch
        each, and the residual add of each block is folded into the next norm.
        A decode step's projections (one row per sequence) run on the
        decode-batch GEMM, QKV with the q/k norm + RoPE + KV append and
        gate/up with SiLU * up in their epilogues; prefill steps (many rows)
        keep the library GEMMs."""
        eps = self.cfg.rms_norm_eps
        I = self.cfg.intermediate_size
        h = F.embedding(input_ids, self.embed)
        res, delta = h, None
        T = h.shape[0]
        pos = meta.positions if meta.positions.dtype == torch.int32 else meta.positions.int()
        small = not prefill and T <= self.small_gemm_rows
        lin = fz.linear if small else F.linear
        for li, L in enumerate(self.layers):
            if delta is None:
                x = fz.rmsnorm(res, L["ln1"], eps)
            else:
                x, res = fz.rmsnorm(delta, L["ln1"], eps, residual=res)
            if small:  # projection, q/k norm + RoPE and the KV append in one launch
                q, _ = fz.qkv_norm_rope_store(
                    x, L["qkv"], self.hq, self.hkv, L["q_norm"], L["k_norm"], eps, self.rope.cos,
                    self.rope.sin, pos, cache.k(li), cache.v(li), block_tables=meta.block_tables,
                    cache_seqlens=meta.cache_seqlens, want_k=False)
            else:
                qkv = F.linear(x, L["qkv"])
                if prefill:
                    q, k = fz.qk_norm_rope_store(
                        qkv, self.hq, self.hkv, L["q_norm"], L["k_norm"], eps, self.rope.cos,
                        self.rope.sin, pos, cache.k(li), cache.v(li), slot_mapping=meta.slot_mapping)
                    v = qkv[:, self.q_size + self.kv_size:].view(T, self.hkv, self.d)
                    attn = fai.flash_attn_varlen_func(q, k, v, meta.cu_seqlens, meta.cu_seqlens,
                                                      meta.max_seqlen, meta.max_seqlen,
                                                      softmax_scale=self.scale, causal=True)
                else:
                    q, _ = fz.qk_norm_rope_store(
                        qkv, self.hq, self.hkv, L["q_norm"], L["k_norm"], eps, self.rope.cos,
                        self.rope.sin, pos, cache.k(li), cache.v(li),
                        block_tables=meta.block_tables, cache_seqlens=meta.cache_seqlens,
                        want_k=False)
            if not prefill:
                attn = fai.decode_paged(q, cache.k(li), cache.v(li), meta.block_tables,
                                        meta.context_lens, softmax_scale=self.scale,
                                        max_context_len=meta.max_context_len)
            o = lin(attn.reshape(T, -1), L["o"])
            x, res = fz.rmsnorm(o, L["ln2"], eps, residual=res)
            if small:
                delta = fz.linear(fz.linear(x, L["gate_up"], silu=True), L["down"])
            else:
                delta = F.linear(fz.silu_mul(F.linear(x, L["gate_up"])), L["down"])
        if prefill:
            delta, res = delta[meta.last_idx], res[meta.last_idx]
        h, _ = fz.rmsnorm(delta, self.norm, eps, residual=res)
        return F.linear(h, self.embed)  # tied embeddings

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, meta: StepMeta, cache: PagedKVCache,
                prefill: bool) -> torch.Tensor:
        """Logits for the last token of every sequence: prefill takes packed
        tokens (llm.py:116-208), decode one token per sequence
        (model/model.py:302-322)."""
        if self.fused:
            return self._forward_fused(input_ids, meta, cache, prefill)
        h = F.embedding(input_ids, self.embed)
        for li in range(self.cfg.num_hidden_layers):
            h = self._layer(li, h, meta, cache, prefill)
        if prefill:
            h = h[meta.last_idx]
        h = rms_norm(h, self.norm, self.cfg.rms_norm_eps)
        return F.linear(h, self.embed)  # tied embeddings

    def kv_bytes_per_token(self) -> int:
        return 2 * self.hkv * self.d * 2 * self.cfg.num_hidden_layers
