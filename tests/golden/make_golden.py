"""Write the committed golden fixtures under tests/golden/.

The reference ships no golden vectors or tests for this path (its attention
arithmetic lives in the absent third-party flash_attn package), so the
fixtures are produced from the oracle AFTER it has been cross-checked here
against torch's scaled_dot_product_attention (float64, causal) and torch's
index_copy_ -- the library routines closest to the reference's calls.  The
fixtures then pin the oracle (and through it the GPU kernels) against drift.

Run: ``python tests/golden/make_golden.py`` from the repository root.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(HERE.parent))

import oracle  # noqa: E402
from cases import (config1_inputs, sha256, tiny_decode_inputs,  # noqa: E402
                   tiny_prefill_inputs)


def as_torch(a):
    """numpy array -> torch tensor; uint16 arrays are bf16 bit patterns."""
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(a)


def sdpa_decode(q, ks, vs, scale):
    """torch SDPA, float64, one query per head, KV heads repeat-interleaved."""
    g = q.shape[0] // ks.shape[1]
    qt = torch.from_numpy(q).double()[:, None, :]                        # [Hq,1,D]
    kt = torch.from_numpy(ks).double().permute(1, 0, 2).repeat_interleave(g, 0)
    vt = torch.from_numpy(vs).double().permute(1, 0, 2).repeat_interleave(g, 0)
    return torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale)[:, 0].numpy()


def sdpa_prefill(q, k, v, cu, scale):
    out = np.zeros(q.shape, dtype=np.float64)
    g = q.shape[1] // k.shape[1]
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        qt = torch.from_numpy(q[a:b]).double().permute(1, 0, 2)
        kt = torch.from_numpy(k[a:b]).double().permute(1, 0, 2).repeat_interleave(g, 0)
        vt = torch.from_numpy(v[a:b]).double().permute(1, 0, 2).repeat_interleave(g, 0)
        o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True, scale=scale)
        out[a:b] = o.permute(1, 0, 2).numpy()
    return out


def decode_fixture(inp, f32):
    kc, vc = inp["k_cache"].copy(), inp["v_cache"].copy()
    digest_in = sha256(inp["q"], inp["k_new"], inp["v_new"], inp["k_cache"], inp["v_cache"],
                       inp["block_tables"], inp["cache_seqlens"])
    # store through the oracle and through torch index_copy_ (the reference op)
    sm = oracle.decode_slot_mapping(inp["block_tables"], inp["cache_seqlens"], inp["block_size"])
    out, new_lens = oracle.decode_append_attend(
        inp["q"], kc, vc, inp["k_new"], inp["v_new"], inp["block_tables"], inp["cache_seqlens"],
        inp["block_size"], inp["scale"])
    tk = as_torch(inp["k_cache"].copy())
    tk.view(-1, *tk.shape[2:]).index_copy_(0, torch.from_numpy(sm), as_torch(inp["k_new"]))
    assert np.array_equal(tk.view(torch.uint8).numpy(), kc.view(np.uint8)), "store != index_copy_"
    # attention vs SDPA
    for b in range(out.shape[0]):
        n = int(inp["context_lens"][b])
        ks = oracle.gather_paged(kc, inp["block_tables"][b], n, inp["block_size"])
        vs = oracle.gather_paged(vc, inp["block_tables"][b], n, inp["block_size"])
        if not f32:
            ks, vs = oracle.bf16_bits_to_f32(ks), oracle.bf16_bits_to_f32(vs)
            qb = oracle.bf16_bits_to_f32(inp["q"][b])
        else:
            qb = inp["q"][b]
        ref = sdpa_decode(qb, ks, vs, inp["scale"])
        assert np.abs(ref - out[b]).max() < 1e-12, "oracle decode != SDPA"
    return dict(out=out, new_lens=new_lens, slot_mapping=sm,
                digest_inputs=digest_in, digest_k_cache_after=sha256(kc),
                digest_v_cache_after=sha256(vc))


def main():
    manifest = {}
    # config 1 (fp32; inputs regenerated from RandomState(0), only outputs stored)
    inp = config1_inputs()
    fx = decode_fixture(inp, f32=True)
    np.savez(HERE / "config1_decode_fp32.npz", out=fx["out"], new_lens=fx["new_lens"],
             slot_mapping=fx["slot_mapping"])
    manifest["config1_decode_fp32"] = {k: fx[k] for k in
                                       ("digest_inputs", "digest_k_cache_after",
                                        "digest_v_cache_after")}
    # tiny decode (bf16 bits; inputs stored whole)
    inp = tiny_decode_inputs()
    fx = decode_fixture(inp, f32=False)
    np.savez(HERE / "tiny_decode_bf16.npz", out=fx["out"], new_lens=fx["new_lens"],
             slot_mapping=fx["slot_mapping"],
             **{k: inp[k] for k in ("q", "k_new", "v_new", "k_cache", "v_cache", "block_tables",
                                    "cache_seqlens", "context_lens")})
    manifest["tiny_decode_bf16"] = {k: fx[k] for k in ("digest_inputs", "digest_k_cache_after",
                                                       "digest_v_cache_after")}
    # tiny prefill (bf16 bits; inputs stored whole)
    inp = tiny_prefill_inputs()
    out = oracle.varlen_attention(inp["q"], inp["k"], inp["v"], inp["cu_seqlens"],
                                  scale=inp["scale"])
    f = oracle.bf16_bits_to_f32
    ref = sdpa_prefill(f(inp["q"]), f(inp["k"]), f(inp["v"]), inp["cu_seqlens"], inp["scale"])
    assert np.abs(ref - out).max() < 1e-12, "oracle prefill != SDPA"
    np.savez(HERE / "tiny_prefill_bf16.npz", out=out, **inp)
    manifest["tiny_prefill_bf16"] = {"digest_inputs": sha256(inp["q"], inp["k"], inp["v"],
                                                             inp["cu_seqlens"])}
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
