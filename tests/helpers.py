"""Comparison helpers for the parity tests."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _ordered16(t: torch.Tensor) -> torch.Tensor:
    """Monotone integer image of 16-bit float bit patterns (sign-magnitude -> two's complement)."""
    u = t.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    return torch.where(u < 0x8000, u, 0x8000 - u)


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between two bf16/fp16 tensors of equal dtype."""
    assert a.dtype == b.dtype and a.dtype in (torch.bfloat16, torch.float16), (a.dtype, b.dtype)
    return (_ordered16(a.cpu()) - _ordered16(b.cpu())).abs()


def max_ulp(a: torch.Tensor, b: torch.Tensor) -> int:
    d = ulp_diff(a, b)
    return int(d.max()) if d.numel() else 0


def round_to(t: np.ndarray | torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """float64 reference values rounded to `dtype` (the best any kernel can return)."""
    if isinstance(t, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(t))
    return t.to(torch.float64).to(dtype)


def assert_ulp(actual: torch.Tensor, expected: torch.Tensor, max_ulps: int = 1,
               tiny: float = 0.0, what: str = "") -> None:
    """|actual - expected| <= max_ulps bf16/fp16 ulps, or <= tiny in absolute terms."""
    a, e = actual.detach().cpu(), expected.detach().cpu()
    assert a.shape == e.shape, (what, a.shape, e.shape)
    if a.dtype == torch.float32:
        rel = (a - e).abs() / e.abs().clamp(min=1e-30)
        bad = (rel > max_ulps * 2.0 ** -23) & ((a - e).abs() > tiny)
    else:
        d = ulp_diff(a, e.to(a.dtype))
        bad = (d > max_ulps) & ((a.float() - e.float()).abs() > tiny)
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(
            f"{what}: {int(bad.sum())} elements beyond {max_ulps} ulp; first at {idx}: "
            f"actual={a[tuple(idx)].item()!r} expected={e[tuple(idx)].item()!r}")
