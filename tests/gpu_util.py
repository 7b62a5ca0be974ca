"""Helpers for the GPU parity tests (tensor <-> numpy and tolerance checks)."""
from __future__ import annotations

import numpy as np
import torch

import oracle

# The parity bar for bf16/fp16 attention outputs: max |out - oracle| <= 2e-2
# against the float64 oracle evaluated on the same (bf16-rounded) inputs.
ATOL_BF16 = 2e-2


def np_of(t: torch.Tensor) -> np.ndarray:
    """bf16 -> uint16 bit patterns, fp16/fp32 -> float arrays (host copy)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def t_of(a: np.ndarray, device, dtype=None) -> torch.Tensor:
    """uint16 arrays are bf16 bit patterns."""
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(device)
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(device=device, dtype=dtype) if dtype is not None else t.to(device)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float64).cpu().numpy()


def bytes_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def check_attention(out: torch.Tensor, ref: np.ndarray, atol: float = ATOL_BF16, what: str = "",
                    absv: np.ndarray | None = None):
    """Parity check: max-abs within ``atol`` and, more strictly, every element
    within a bound derived from the arithmetic.

    * Output rounding: at most 2^-9 |ref| for a bf16 result.
    * ``absv`` (optional) is the same attention evaluated with |V|, i.e.
      sum_j p_j |v_j|.  When the kernel rounds the probabilities to bf16 before
      the PV product (as the MFMA prefill and the bf16/fp16 decode do, like FA2), each term carries at
      most 2^-9 relative error, so the sum moves by at most 2^-9 * absv.
    Both bounds get a factor 2 of margin for fp32 accumulation and exp2
    approximation error, plus a small absolute floor.
    """
    o = f64(out).reshape(ref.shape)
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    err = np.abs(o - ref)
    mx = float(err.max()) if err.size else 0.0
    assert mx <= atol, f"{what}: max-abs error {mx:.3e} > {atol}"
    if out.dtype in (torch.bfloat16, torch.float16):
        lim = 2.0 ** -8 * np.abs(ref) + 1e-3
        if absv is not None:
            lim = lim + 2.0 ** -8 * np.abs(absv).reshape(ref.shape)
    else:
        lim = 1e-5 * np.abs(ref) + 1e-5
    bad = err > lim
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond the rounding bound " \
                          f"(worst excess {float((err - lim).max()):.3e})"
    return mx


def bf16_np_to_f64(a: np.ndarray) -> np.ndarray:
    return oracle.bf16_bits_to_f32(a).astype(np.float64)
