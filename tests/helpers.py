"""Comparison helpers for the parity tests."""
from __future__ import annotations

import ctypes
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


# ---------------------------------------------------------------------------
# Guard bands (tests/test_gpu_guard.py): tensors inside larger buffers whose
# other elements hold a NaN bit pattern
# ---------------------------------------------------------------------------
BF, F16, F32 = torch.bfloat16, torch.float16, torch.float32
G = 2048  # elements in each guard band
GUARD_BITS = {BF: (torch.int16, 0x7FC1), F16: (torch.int16, 0x7E01),
              F32: (torch.int32, 0x7FC00001), torch.uint8: (torch.uint8, 0xA5)}


class Guarded:
    """A [rows, cols] tensor `t` with row stride ld (>= cols) inside a buffer whose
    other elements, and its own before it is written, hold the dtype's NaN pattern."""

    def __init__(self, rows, cols, ld, dtype, dev, values=None):
        self.rows, self.cols, self.ld, self.dtype = rows, cols, ld, dtype
        n = rows * ld
        self.buf = torch.empty(2 * G + n, dtype=dtype, device=dev)
        iv, bits = GUARD_BITS[dtype]
        self.buf.view(iv).fill_(bits)
        self.t = self.buf[G:G + n].view(rows, ld)[:, :cols]
        if values is not None:
            self.t.copy_(values.reshape(rows, cols))

    @property
    def p(self):
        return ctypes.c_void_p(self.t.data_ptr())

    def intact(self):
        """Whether every element outside the tensor still holds the pattern."""
        iv, bits = GUARD_BITS[self.dtype]
        keep = torch.ones(self.buf.numel(), dtype=torch.bool, device=self.buf.device)
        keep[G:G + self.rows * self.ld].view(self.rows, self.ld)[:, :self.cols] = False
        return bool((self.buf.view(iv)[keep] == bits).all())


def flat(n, dtype, dev, values=None):
    return Guarded(1, n, n, dtype, dev, values)


def same(a, b):
    """Bit-identical (NaN payloads included)."""
    if a.dtype in (BF, F16):
        return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))
    if a.dtype == F32:
        return torch.equal(a.contiguous().view(torch.int32), b.contiguous().view(torch.int32))
    return torch.equal(a, b)
