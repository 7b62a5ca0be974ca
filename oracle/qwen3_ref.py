"""fp32 torch restatement of the reference's Qwen3 model and engine loop.

TEST INFRASTRUCTURE ONLY -- a checker and the host-side baseline, never the
product.  Plain fp32 torch on whatever device the caller picks (the host for
bench.py's CPU baseline, the GPU for the engine tests' teacher forcing).

Restated from the reference:

* RMSNorm (model/model.py:40-52): ``w * x * rsqrt(mean(x^2) + eps)``.
* RoPE, theta 1e6 (model/model.py:55-99): ``inv = 1 / theta^(2i/D)``,
  ``emb = cat(pos * inv, pos * inv)``, ``x * cos + rotate_half(x) * sin``
  with ``rotate_half(x) = cat(-x2, x1)``.
* The decoder layer (model/model.py:202-267): fused QKV, q/k RMSNorm per
  head, RoPE, attention (GQA: query head ``h`` reads KV head ``h // g``),
  o_proj, residual, RMSNorm, SiLU-gated MLP (model/model.py:178-188),
  residual; tied lm_head (model/model.py:289-322).
* The engine (llm.py:116-219, :315-446) with the reference's slot caches
  ``[num_slots, max_seq_len, Hkv, D]`` (model/model.py:324-336): a packed
  varlen prefill that stores K/V with ``index_copy_`` at
  ``slot * max_seq_len + position`` (llm.py:127-175) and attends causally per
  segment (llm.py:178-184); batched decode steps that store the new K/V at
  ``cache_seqlens`` and attend over ``cache_seqlens + 1`` tokens, then
  increment ``cache_seqlens`` (model/model.py:233-241); greedy sampling
  (llm.py:215-219) and the finish rule ``len(tokens) >= max_tokens`` (the
  count includes the prefill token), ``position >= max_seq_len``, or EOS
  unless ``ignore_eos`` (llm.py:366-383, :413-443).

Everything is fp32 (the reference runs bf16 weights; this restatement keeps
the same weights upcast, so it is the exact-arithmetic target the bf16
engine approximates).

Pinned against transformers' own Qwen3 (transformers/models/qwen3/
modeling_qwen3.py: Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb,
eager attention with repeat_kv), an implementation written independently of
both the reference and this file: with the same weights, the full-sequence
logits agree to fp32 rounding and the slot-cache engine's greedy tokens equal
transformers' greedy continuation for every prompt
(tests/test_oracle_pins.py).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["Qwen3Ref", "rms_norm", "rope_tables", "apply_rope"]


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """model/model.py:47-52 in fp32."""
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float):
    """cos, sin ``[T, head_dim]`` for integer positions (model/model.py:64-78)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32,
                                        device=positions.device) / head_dim))
    freqs = positions.to(torch.float32)[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x ``[T, H, D]`` -> ``x * cos + rotate_half(x) * sin`` (model/model.py:86-99)."""
    h = x.shape[-1] // 2
    c, s = cos[:, None, :], sin[:, None, :]
    return x * c + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * s


def _attend(q, k, v, causal: bool, scale: float):
    """q ``[Tq, Hq, D]``, k/v ``[Tk, Hkv, D]`` -> ``[Tq, Hq, D]``: softmax
    attention with KV heads repeated to the query heads (bottom-right causal
    alignment, as FA2; at every reference call site Tq == Tk or Tq == 1)."""
    g = q.shape[1] // k.shape[1]
    qh = q.transpose(0, 1)                                  # [Hq, Tq, D]
    kh = k.transpose(0, 1).repeat_interleave(g, 0)          # [Hq, Tk, D]
    vh = v.transpose(0, 1).repeat_interleave(g, 0)
    s = torch.matmul(qh, kh.transpose(1, 2).contiguous()) * scale
    if causal:
        tq, tk = q.shape[0], k.shape[0]
        i = torch.arange(tq, device=q.device)[:, None]
        j = torch.arange(tk, device=q.device)[None, :]
        s = s.masked_fill(j > i + (tk - tq), float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vh).transpose(0, 1)


class Qwen3Ref:
    """fp32 Qwen3 with the reference's slot-cache engine loop.

    ``weights``: ``embed [V, H]``, ``norm [H]`` and per layer ``ln1``, ``ln2``,
    ``q_norm``, ``k_norm``, ``qkv [(Hq+2Hkv)D, H]`` (fused [Q | K | V]), ``o``,
    ``gate_up [2I, H]`` (fused [gate | up]), ``down`` -- the layout
    model/model.py:132-154 builds and the product model uses.
    """

    def __init__(self, cfg, weights: dict, device="cpu"):
        self.cfg = cfg
        self.device = torch.device(device)
        f = lambda t: t.detach().to(device=self.device, dtype=torch.float32)  # noqa: E731
        self.embed = f(weights["embed"])
        self.norm = f(weights["norm"])
        self.layers = [{k: f(v) for k, v in L.items()} for L in weights["layers"]]
        self.hq, self.hkv, self.d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.scale = self.d ** -0.5

    @classmethod
    def from_model(cls, model, device=None):
        """The same weights as a product ``Qwen3ForCausalLM``, upcast to fp32."""
        w = dict(embed=model.embed, norm=model.norm, layers=model.layers)
        return cls(model.cfg, w, device if device is not None else model.device)

    @classmethod
    def random(cls, cfg, seed: int = 0, device="cpu", std: float = 0.02, tiled: bool = False):
        """Random weights drawn as the product draws them (N(0, std), norms at 1).
        ``tiled`` fills every matrix from one 4 Mi-value draw at random offsets
        (seconds instead of a minute for 0.6B parameters; for timing runs)."""
        g = torch.Generator(device="cpu").manual_seed(seed)
        H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads
        if tiled:
            base = torch.randn(1 << 22, generator=g) * std

            def rnd(*s):
                n = 1
                for x in s:
                    n *= x
                off = int(torch.randint(0, base.numel(), (1,), generator=g))
                reps = -(-(n + off) // base.numel())
                return base.repeat(reps)[off:off + n].view(*s).clone()
        else:
            rnd = lambda *s: torch.randn(*s, generator=g) * std  # noqa: E731
        layers = [dict(ln1=torch.ones(H), ln2=torch.ones(H), q_norm=torch.ones(D),
                       k_norm=torch.ones(D), qkv=rnd((hq + 2 * hkv) * D, H), o=rnd(H, hq * D),
                       gate_up=rnd(2 * I, H), down=rnd(H, I))
                  for _ in range(cfg.num_hidden_layers)]
        return cls(cfg, dict(embed=rnd(cfg.vocab_size, H), norm=torch.ones(H), layers=layers),
                   device)

    # ------------------------------------------------------------ the layer
    def _qkv(self, L, x, positions):
        eps, T = self.cfg.rms_norm_eps, x.shape[0]
        qkv = F.linear(rms_norm(x, L["ln1"], eps), L["qkv"])
        qs, ks = self.hq * self.d, self.hkv * self.d
        q = rms_norm(qkv[:, :qs].reshape(T, self.hq, self.d), L["q_norm"], eps)
        k = rms_norm(qkv[:, qs:qs + ks].reshape(T, self.hkv, self.d), L["k_norm"], eps)
        v = qkv[:, qs + ks:].reshape(T, self.hkv, self.d)
        cos, sin = rope_tables(positions, self.d, self.cfg.rope_theta)
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v

    def _finish_layer(self, L, h, attn):
        eps, I = self.cfg.rms_norm_eps, self.cfg.intermediate_size
        h = h + F.linear(attn.reshape(h.shape[0], -1), L["o"])
        gu = F.linear(rms_norm(h, L["ln2"], eps), L["gate_up"])
        return h + F.linear(F.silu(gu[:, :I]) * gu[:, I:], L["down"])

    def _head(self, h):
        return F.linear(rms_norm(h, self.norm, self.cfg.rms_norm_eps), self.embed)

    @torch.no_grad()
    def logits(self, ids) -> torch.Tensor:
        """Teacher-forced logits ``[T, vocab]`` of one sequence (positions 0..T-1)."""
        ids = torch.as_tensor(ids, dtype=torch.int64, device=self.device)
        pos = torch.arange(ids.shape[0], device=self.device)
        h = self.embed[ids]
        for L in self.layers:
            q, k, v = self._qkv(L, h, pos)
            h = self._finish_layer(L, h, _attend(q, k, v, True, self.scale))
        return self._head(h)

    # ------------------------------------------------------------ the engine
    def _caches(self, num_slots: int, max_seq_len: int):
        shape = (num_slots, max_seq_len, self.hkv, self.d)
        self.k_cache = [torch.zeros(shape, device=self.device) for _ in self.layers]
        self.v_cache = [torch.zeros(shape, device=self.device) for _ in self.layers]
        self.cache_seqlens = torch.zeros(num_slots, dtype=torch.int32, device=self.device)
        self.max_seq_len = max_seq_len

    @torch.no_grad()
    def prefill(self, prompts, slots) -> torch.Tensor:
        """Packed varlen prefill (llm.py:116-208): logits of each prompt's last token."""
        dev, lmax = self.device, self.max_seq_len
        lens = [len(p) for p in prompts]
        cu = [0]
        for n in lens:
            cu.append(cu[-1] + n)
        ids = torch.tensor([t for p in prompts for t in p], dtype=torch.int64, device=dev)
        pos = torch.cat([torch.arange(n, device=dev) for n in lens])
        scatter = torch.repeat_interleave(torch.tensor(slots, device=dev) * lmax,
                                          torch.tensor(lens, device=dev)) + pos
        h = self.embed[ids]
        for li, L in enumerate(self.layers):
            q, k, v = self._qkv(L, h, pos)
            self.k_cache[li].view(-1, self.hkv, self.d).index_copy_(0, scatter, k)
            self.v_cache[li].view(-1, self.hkv, self.d).index_copy_(0, scatter, v)
            attn = torch.cat([_attend(q[a:b], k[a:b], v[a:b], True, self.scale)
                              for a, b in zip(cu[:-1], cu[1:])])
            h = self._finish_layer(L, h, attn)
        self.cache_seqlens[torch.tensor(slots, device=dev)] = torch.tensor(
            lens, dtype=torch.int32, device=dev)
        return self._head(h[torch.tensor(cu[1:], device=dev) - 1])

    @torch.no_grad()
    def decode(self, tokens, slots) -> torch.Tensor:
        """One decode step of a batch (model/model.py:202-267, seq_len 1):
        store at ``cache_seqlens``, attend over ``cache_seqlens + 1`` tokens,
        then ``cache_seqlens += 1``."""
        dev = self.device
        sl = torch.tensor(slots, dtype=torch.int64, device=dev)
        lens = self.cache_seqlens[sl].to(torch.int64)
        h = self.embed[torch.tensor(tokens, dtype=torch.int64, device=dev)]
        lens_host = lens.tolist()
        for li, L in enumerate(self.layers):
            q, k, v = self._qkv(L, h, lens)
            self.k_cache[li][sl, lens] = k
            self.v_cache[li][sl, lens] = v
            attn = torch.cat([
                _attend(q[b:b + 1], self.k_cache[li][s, :n + 1], self.v_cache[li][s, :n + 1],
                        False, self.scale)
                for b, (s, n) in enumerate(zip(slots, lens_host))])
            h = self._finish_layer(L, h, attn)
        self.cache_seqlens[sl] += 1
        return self._head(h)

    @torch.no_grad()
    def generate(self, prompts, max_tokens: int, max_seq_len: int, ignore_eos: bool = True):
        """Greedy generation of every prompt with all of them admitted at once
        (one slot each): the packed prefill, then batched decode steps until
        each sequence meets the finish rule.  Returns the token lists."""
        n = len(prompts)
        self._caches(n, max_seq_len)
        out = [[int(t)] for t in self.prefill(prompts, list(range(n))).argmax(-1).tolist()]
        pos = [len(p) for p in prompts]
        eos = self.cfg.eos_token_id

        def done(i):
            t = out[i]
            return (len(t) >= max_tokens or pos[i] >= max_seq_len
                    or (not ignore_eos and t[-1] == eos))

        live = [i for i in range(n) if not done(i)]
        while live:
            nxt = self.decode([out[i][-1] for i in live], live).argmax(-1).tolist()
            for i, t in zip(live, nxt):
                out[i].append(int(t))
                pos[i] += 1
            live = [i for i in live if not done(i)]
        return out

    def num_params(self) -> int:
        per = sum(t.numel() for t in self.layers[0].values())
        return per * len(self.layers) + self.embed.numel() + self.norm.numel()
