"""Decode-batch projection GEMM (aac_gemm_nt) against an fp32 reference.

y = x w^T (torch's F.linear for the q/k/v, o_proj, gate/up and down
projections, model/model.py:132-154, :258, :178-188) is checked against the same
product in fp32 on the bf16 inputs: the kernel accumulates in fp32 in its own
order and rounds once, so every element is within one rounding of the exact
value (2^-8 relative, with margin for the fp32 summation).  The gate/up
variant is checked against the reference expression evaluated from the fp32
products rounded to the activation dtype, act_fn(gate) * up
(model/model.py:188): elements whose rounded gate or up differ from the
kernel's by the fp32 summation order may move by a few ulps."""
import pytest
import torch
import torch.nn.functional as F

from awesome_acceleration_amd import fused as fz

pytestmark = pytest.mark.gpu


def _inputs(gpu, m, n_rows, k, dtype, seed, x_pad=0, w_pad=0):
    g = torch.Generator(device=gpu).manual_seed(seed)
    x = torch.randn((m, k + x_pad), generator=g, device=gpu).to(dtype)[:, :k]
    w = (torch.randn((n_rows, k + w_pad), generator=g, device=gpu) * 0.05).to(dtype)[:, :k]
    return x, w


def _ref(x, w):
    return x.float() @ w.float().t()


def _check_linear(y, x, w, what):
    ref = _ref(x, w)
    mag = x.float().abs() @ w.float().abs().t()  # scale of the summed terms
    mant = 8 if y.dtype == torch.bfloat16 else 11
    tol = ref.abs() * 2.0 ** -(mant - 1) + mag * 2.0 ** -20 + 1e-30
    err = (y.float() - ref).abs()
    assert torch.isfinite(y.float()).all(), what
    assert (err <= tol).all(), f"{what}: worst excess {float((err - tol).max()):.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [
    (256, 4096, 1024),   # q/k/v projection, Qwen3-0.6B decode step of 256 sequences
    (256, 1024, 2048),   # o_proj
    (256, 1024, 3072),   # down
    (1, 4096, 1024), (7, 1024, 2048), (100, 4096, 1024), (300, 1024, 3072), (64, 192, 256),
    (512, 4096, 1024), (512, 1024, 3072),  # the largest decode batch the model sends here
])
def test_linear_matches_fp32_reference(gpu, m, n, k, dtype):
    x, w = _inputs(gpu, m, n, k, dtype, seed=m + n + k)
    y = fz.linear(x, w)
    torch.cuda.synchronize()
    _check_linear(y, x, w, f"{m}x{n}x{k} {dtype}")


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5, 6])
def test_every_tiling(gpu, config):
    """Each forced tiling on a shape all of them support, with strided rows."""
    m, n, k = 200, 512, 1024
    x, w = _inputs(gpu, m, n, k, torch.bfloat16, seed=config, x_pad=24, w_pad=8)
    y = fz.linear(x, w, config=config)
    torch.cuda.synchronize()
    _check_linear(y, x, w, f"config {config}")


def _silu_ref(x, w):
    """act_fn(gate_proj(x)) * up_proj(x) with the products rounded to the
    activation dtype first (torch's bf16 linear), then F.silu and the product
    rounded as torch rounds them."""
    I = w.shape[0] // 2
    gu = _ref(x, w).to(x.dtype)
    return F.silu(gu[:, :I]) * gu[:, I:], gu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,i,k,config", [
    (256, 3072, 1024, 0),  # gate/up of a Qwen3-0.6B decode step
    (256, 3072, 1024, 1), (256, 3072, 1024, 2), (256, 3072, 1024, 4),
    (200, 3072, 1024, 3), (37, 3072, 1024, 0), (100, 3072, 1024, 6),
    (5, 3072, 1024, 0), (130, 256, 512, 0), (512, 3072, 1024, 0),
])
def test_silu_gate_up_matches_reference(gpu, m, i, k, config, dtype):
    x, w = _inputs(gpu, m, 2 * i, k, dtype, seed=7 * m + i)
    y = fz.linear(x, w, silu=True, config=config)
    ref, gu = _silu_ref(x, w)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    mant = 8 if dtype == torch.bfloat16 else 11
    # one ulp of gate or up moves silu(g) * u by about one ulp of the product
    g, u = gu[:, :i].float().abs(), gu[:, i:].float().abs()
    scale = (g + 1) * u
    # fp32 summation order moves gate and up by up to ~2^-20 of the summed
    # magnitudes (large relative to a cancelled sum); |silu'| <= 1.1
    mag = x.float().abs() @ w.float().abs().t()
    acc = (g * mag[:, i:] + 1.1 * u * mag[:, :i]) * 2.0 ** -20
    tol = (ref.float().abs() + scale) * 2.0 ** -(mant - 2) + acc + 1e-6
    err = (y.float() - ref.float()).abs()
    assert (err <= tol).all(), f"worst excess {float((err - tol).max()):.3e}"
    # and most elements are identical (the products round the same way)
    frac = float((err > 0).float().mean())
    assert frac < 0.05, f"{frac:.2%} of the elements differ"


def test_gate_up_tiling_that_does_not_fit_lds_is_rejected(gpu):
    """Tiling 5 stages 128 rows x 256 K with the gate/up pairing: three stages
    exceed LDS, so the call fails with an error instead of launching."""
    x = torch.zeros((64, 1024), device=gpu, dtype=torch.bfloat16)
    w = torch.zeros((2 * 3072, 1024), device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        fz.linear(x, w, silu=True, config=5)


def test_rejects_bad_arguments(gpu):
    x = torch.zeros((4, 1024), device=gpu, dtype=torch.bfloat16)
    w = torch.zeros((96, 1024), device=gpu, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):  # tiling 1 needs n % 64 == 0
        fz.linear(x, w, config=1)
    with pytest.raises(RuntimeError):
        fz.linear(x, torch.zeros((64, 1000), device=gpu, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError):
        fz.linear(x.float(), w.float())
