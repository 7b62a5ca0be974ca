"""Fused call-site kernels against the reference's own torch expressions:
RMSNorm (model/model.py:47-52) with the residual add before it, q/k RMSNorm +
RoPE (model/model.py:86-99, :225-228) with the KV store (llm.py:171-174) or
decode append, and SiLU * up (model/model.py:188), and the QKV projection with
the q/k norm + RoPE + store in its epilogue.  The fused kernels round at
the same points, so results match to one unit in the last place where fp32
summation order differs, and the cache stores are bit-exact."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from awesome_acceleration_amd import fused as fz
from awesome_acceleration_amd.qwen3 import Rope, rms_norm

pytestmark = pytest.mark.gpu


def ulp_close(a: torch.Tensor, b: torch.Tensor, what: str, max_frac: float = 2e-2,
              scale: torch.Tensor | None = None):
    """Equal except for at most ``max_frac`` of the elements, each within a
    few units in the last place.  A one-ulp difference in the normalised value
    (fp32 summation order, correctly rounded vs. library rsqrt) can move a
    later rounded product or sum (x weight, x cos, + rotated term) by up to
    two ulps of the result; the bound allows four, relative to the larger
    magnitude (or to ``scale``, the magnitude of the rounded terms a result
    was summed from, where they can cancel), plus the subnormal spacing."""
    mant = 8 if a.dtype == torch.bfloat16 else 11  # significand bits
    tiny = 2.0 ** -133 if a.dtype == torch.bfloat16 else 2.0 ** -24
    a, b = a.float(), b.float()
    assert torch.isfinite(a).all(), what
    mag = torch.maximum(a.abs(), b.abs())
    if scale is not None:
        mag = torch.maximum(mag, scale.float())
    tol = mag * 2.0 ** -(mant - 3) + 4 * tiny
    diff = (a - b).abs()
    assert (diff <= tol).all(), f"{what}: max diff {float(diff.max()):.3e}"
    frac = float((diff > 0).float().mean())
    assert frac <= max_frac, f"{what}: {frac:.4%} elements differ"


def rope_terms(rope: Rope, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """|x cos| + |rotate_half(x) sin|: the magnitude of the two rounded terms
    each RoPE output is the sum of (they cancel where the output is small)."""
    cos = rope.cos[positions].unsqueeze(1).float()
    sin = rope.sin[positions].unsqueeze(1).float()
    x = x.float()
    x1, x2 = x[..., :rope.half], x[..., rope.half:]
    return (x * cos).abs() + (torch.cat((-x2, x1), dim=-1) * sin).abs()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden", [1024, 4096])
def test_rmsnorm_with_and_without_residual(gpu, dtype, hidden):
    print(f"case: rmsnorm {dtype} {hidden}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(0)
    rows = 300
    x = torch.randn((rows, hidden), generator=g, device=gpu).to(dtype)
    r = torch.randn((rows, hidden), generator=g, device=gpu).to(dtype)
    w = (1 + 0.3 * torch.randn(hidden, generator=g, device=gpu)).to(dtype)
    out = fz.rmsnorm(x, w, 1e-6)
    ulp_close(out, rms_norm(x, w, 1e-6), "rmsnorm")
    out2, h = fz.rmsnorm(x, w, 1e-6, residual=r)
    assert torch.equal(h, r + x)  # the residual add, rounded like torch
    ulp_close(out2, rms_norm(r + x, w, 1e-6), "add+rmsnorm")
    # strided rows (a view into a wider buffer)
    wide = torch.randn((rows, hidden + 64), generator=g, device=gpu).to(dtype)
    ulp_close(fz.rmsnorm(wide[:, :hidden], w, 1e-6), rms_norm(wide[:, :hidden], w, 1e-6), "strided")


@pytest.mark.parametrize("hq,hkv,T", [(16, 8, 777), (32, 8, 777), (8, 8, 777), (16, 8, 5000),
                                      (32, 8, 4097)])
def test_qk_norm_rope_prefill_store(gpu, hq, hkv, T):
    # T >= 4096 takes the one-wavefront-per-token kernel, smaller T the
    # one-row-per-(token, head) kernel
    print(f"case: qk norm rope store {hq}/{hkv} T={T}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(1)
    D, bs = 128, 64
    pool = -(-T // bs) + 8
    qkv = torch.randn((T, (hq + 2 * hkv) * D), generator=g, device=gpu).to(torch.bfloat16)
    qw = (1 + 0.3 * torch.randn(D, generator=g, device=gpu)).to(torch.bfloat16)
    kw = (1 + 0.3 * torch.randn(D, generator=g, device=gpu)).to(torch.bfloat16)
    rope = Rope(D, 4096, 1e6, gpu, torch.bfloat16)
    pos = torch.randint(0, 4096, (T,), generator=g, device=gpu, dtype=torch.int32)
    kc = torch.randn((pool, bs, hkv, D), generator=g, device=gpu).to(torch.bfloat16)
    vc = torch.randn((pool, bs, hkv, D), generator=g, device=gpu).to(torch.bfloat16)
    kc0, vc0 = kc.clone(), vc.clone()
    slots = torch.randperm(pool * bs, generator=g, device=gpu)[:T].to(torch.int64)
    slots[5] = -1  # padding token: not stored
    q, k = fz.qk_norm_rope_store(qkv, hq, hkv, qw, kw, 1e-6, rope.cos, rope.sin, pos, kc, vc,
                                 slot_mapping=slots)
    torch.cuda.synchronize()
    qn = rms_norm(qkv[:, :hq * D].view(T, hq, D), qw, 1e-6)
    kn = rms_norm(qkv[:, hq * D:(hq + hkv) * D].view(T, hkv, D), kw, 1e-6)
    ulp_close(q, rope.apply(qn, pos), "q", scale=rope_terms(rope, qn, pos))
    ulp_close(k, rope.apply(kn, pos), "k", scale=rope_terms(rope, kn, pos))
    v = qkv[:, (hq + hkv) * D:].view(T, hkv, D)
    keep = slots >= 0
    ek, ev = kc0.view(-1, hkv, D).clone(), vc0.view(-1, hkv, D).clone()
    ek[slots[keep]] = k[keep]
    ev[slots[keep]] = v[keep]
    assert torch.equal(kc.view(-1, hkv, D), ek)  # stored bits are the returned k, untouched rows kept
    assert torch.equal(vc.view(-1, hkv, D), ev)


def test_qk_norm_rope_decode_append(gpu):
    print("case: qk norm rope append", flush=True)
    g = torch.Generator(device=gpu).manual_seed(2)
    B, hq, hkv, D, bs, W = 9, 16, 8, 128, 16, 4
    qkv = torch.randn((B, (hq + 2 * hkv) * D), generator=g, device=gpu).to(torch.bfloat16)
    w1 = torch.ones(D, device=gpu, dtype=torch.bfloat16)
    rope = Rope(D, 1024, 1e6, gpu, torch.bfloat16)
    pool = B * W
    bt = torch.randperm(pool, generator=g, device=gpu).view(B, W).to(torch.int32)
    seqlens = torch.randint(0, W * bs, (B,), generator=g, device=gpu, dtype=torch.int32)
    kc = torch.zeros((pool, bs, hkv, D), device=gpu, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    q, none = fz.qk_norm_rope_store(qkv, hq, hkv, w1, w1, 1e-6, rope.cos, rope.sin, seqlens, kc,
                                    vc, block_tables=bt, cache_seqlens=seqlens, want_k=False)
    torch.cuda.synchronize()
    assert none is None
    kn = rms_norm(qkv[:, hq * D:(hq + hkv) * D].view(B, hkv, D), w1, 1e-6)
    kr = rope.apply(kn, seqlens)
    v = qkv[:, (hq + hkv) * D:].view(B, hkv, D)
    btn, sl = bt.cpu().numpy(), seqlens.cpu().numpy()
    rows = torch.tensor([int(btn[b, sl[b] // bs]) * bs + int(sl[b]) % bs for b in range(B)],
                        device=gpu)
    ulp_close(kc.view(-1, hkv, D)[rows], kr, "appended k", scale=rope_terms(rope, kn, seqlens))
    assert torch.equal(vc.view(-1, hkv, D)[rows], v)
    assert int((kc.view(-1, hkv, D).abs().sum((1, 2)) > 0).sum()) == B  # nothing else written


def test_silu_mul(gpu):
    print("case: silu mul", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    gu = torch.randn((513, 2 * 3072), generator=g, device=gpu).to(torch.bfloat16)
    ref = F.silu(gu[:, :3072]) * gu[:, 3072:]
    ulp_close(fz.silu_mul(gu), ref, "silu*up")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,hq,hkv,append", [(256, 16, 8, True), (1, 16, 8, True), (37, 16, 8, True),
                                             (300, 32, 8, True), (100, 16, 8, False),
                                             (512, 16, 8, True)])
def test_qkv_projection_fused_with_norm_rope_store(gpu, dtype, T, hq, hkv, append):
    """The QKV projection with q/k norm + RoPE + store in its epilogue equals,
    bit for bit, the decode-batch GEMM with the same K split (tiling 6)
    followed by the q/k norm + RoPE + store kernel: q, k and both caches."""
    print(f"case: qkv projection + norm rope store {dtype} T={T} {hq}/{hkv} append={append}",
          flush=True)
    g = torch.Generator(device=gpu).manual_seed(4)
    D, H, bs = 128, 1024, 16
    x = torch.randn((T, H), generator=g, device=gpu).to(dtype)
    w = (torch.randn(((hq + 2 * hkv) * D, H), generator=g, device=gpu) * 0.05).to(dtype)
    qw = (1 + 0.3 * torch.randn(D, generator=g, device=gpu)).to(dtype)
    kw = (1 + 0.3 * torch.randn(D, generator=g, device=gpu)).to(dtype)
    rope = Rope(D, 2048, 1e6, gpu, dtype)
    W = 8
    pool = T * W + 1
    kc = torch.randn((pool, bs, hkv, D), generator=g, device=gpu).to(dtype)
    vc = torch.randn_like(kc)
    kc2, vc2 = kc.clone(), vc.clone()
    if append:
        bt = (1 + torch.randperm(pool - 1, generator=g, device=gpu)[:T * W]).view(T, W).to(torch.int32)
        seqlens = torch.randint(0, W * bs, (T,), generator=g, device=gpu, dtype=torch.int32)
        kwargs = dict(block_tables=bt, cache_seqlens=seqlens)
        pos = seqlens
    else:
        slots = torch.randperm(pool * bs, generator=g, device=gpu)[:T].to(torch.int64)
        slots[3] = -1  # padding token: not stored
        kwargs = dict(slot_mapping=slots)
        pos = torch.randint(0, 2048, (T,), generator=g, device=gpu, dtype=torch.int32)
    qkv = fz.linear(x, w, config=6)
    q1, k1 = fz.qk_norm_rope_store(qkv, hq, hkv, qw, kw, 1e-6, rope.cos, rope.sin, pos, kc, vc,
                                   **kwargs)
    q2, k2 = fz.qkv_norm_rope_store(x, w, hq, hkv, qw, kw, 1e-6, rope.cos, rope.sin, pos, kc2, vc2,
                                    **kwargs)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2)
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    # and the fused path's q is the reference expression of the projection
    qn = rms_norm(qkv[:, :hq * D].view(T, hq, D), qw, 1e-6)
    ulp_close(q2, rope.apply(qn, pos), "q", scale=rope_terms(rope, qn, pos))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,cols,pad", [(256, 151936, 0), (7, 1001, 24), (1, 5, 3), (3, 2048, 0)])
def test_argmax_matches_torch(gpu, dtype, rows, cols, pad):
    """Row argmax (the greedy sampler) equals torch.argmax(dim=-1): random
    rows, rows with repeated maxima (first index wins), all -inf rows, NaNs
    (a NaN counts as the maximum), strided rows, odd widths."""
    print(f"case: argmax {dtype} {rows}x{cols} pad {pad}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(6)
    base = torch.randn((rows, cols + pad), generator=g, device=gpu).to(dtype)
    x = base[:, :cols]
    if rows >= 3 and cols >= 5:
        x[0, :] = x[0, 0]                   # all equal: index 0
        x[1, :] = -float("inf")             # all -inf: index 0
        x[2, cols // 3] = float("nan")      # NaN wins
        x[2, cols - 1] = float("nan")       # ... the first NaN
    if rows >= 5:
        m = x[4].max()
        x[4, cols - 1] = m                  # a tie with an earlier maximum
    got = fz.argmax(x)
    ref = torch.argmax(x, dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (got[:8].tolist(), ref[:8].tolist())
