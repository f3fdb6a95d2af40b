"""Drop-in counterparts of TrainScale's ``kernels/layernorm_kernels.py`` RMSNorm ops.

Reference (``data_pipeline/trainer/``):

* ``RMSLayerNormFunction`` (kernels/layernorm_kernels.py:676-807):
  forward(X, weight, eps, compute_weight_grad) -> Y; backward -> (dX, dW, None, None).
  Its forward rounds x * rstd to the weight dtype before the weight product
  (y = x_norm.to(w.dtype) * w, :189-194): with a 16-bit weight that is a
  second rounding, which the ROUND_TWICE kernel mode reproduces; with an fp32
  weight the product is formed in fp32 and rounded once into the data dtype.
* ``rms_layernorm`` and its alias ``fast_rms_layernorm`` (:1054-1070, :1141).
* ``RMSNorm`` module (:1150-1189).
* ``FusedAddRMSLayerNormFunction`` (:949-1047), ``fused_add_rms_layernorm``
  (:1094-1121) and the ``FusedRMSNorm`` module (:1241-1269): h = X + residual
  in fp32, Y = RMSNorm(h) with the same round-twice numerics, and h rounded to
  the data dtype as ``residual_out``. As in the reference, backward returns
  the same dX for X and residual, computed from dY and the rounded h; the
  gradient arriving at ``residual_out`` is not added and the weight gets no
  gradient (the reference's backward returns None for it).

LayerNorm/Welford and dropout+RMS are not part of this layer.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from .. import ops

DEFAULT_EPS_RMS = 1e-6

__all__ = [
    "RMSLayerNormFunction",
    "rms_layernorm",
    "fast_rms_layernorm",
    "RMSNorm",
    "FusedAddRMSLayerNormFunction",
    "fused_add_rms_layernorm",
    "FusedRMSNorm",
    "DEFAULT_EPS_RMS",
]


class RMSLayerNormFunction(torch.autograd.Function):
    """RMSNorm with the reference's rounding: y = round(round(x*rstd) * w) for 16-bit w."""

    @staticmethod
    def forward(ctx, X: Tensor, weight: Tensor, eps: float = DEFAULT_EPS_RMS,
                compute_weight_grad: bool = True) -> Tensor:
        orig_shape = X.shape
        x2d, ldx = ops.as_rows(X)
        y, rstd = ops.rmsnorm_forward(x2d, ldx, weight, eps, ops.ROUND_TWICE)
        ctx.save_for_backward(x2d, weight, rstd)
        ctx.ldx = ldx
        ctx.orig_shape = orig_shape
        ctx.compute_weight_grad = compute_weight_grad
        return y.view(orig_shape)

    @staticmethod
    def backward(ctx, dY: Tensor) -> Tuple[Optional[Tensor], ...]:
        x2d, weight, rstd = ctx.saved_tensors
        dy2d, lddy = ops.as_rows(dY)
        need_dw = bool(ctx.compute_weight_grad and weight is not None and weight.requires_grad)
        dx, dw = ops.rmsnorm_backward(dy2d, lddy, x2d, ctx.ldx, weight, rstd, need_dw=need_dw)
        return dx.view(ctx.orig_shape), dw, None, None


def rms_layernorm(X: Tensor, weight: Tensor, eps: float = DEFAULT_EPS_RMS) -> Tensor:
    """RMSNorm (reference: kernels/layernorm_kernels.py:1054-1070)."""
    return RMSLayerNormFunction.apply(X, weight, eps, True)


fast_rms_layernorm = rms_layernorm


class _RMSNormNoWeight(torch.autograd.Function):
    @staticmethod
    def forward(ctx, X: Tensor, eps: float) -> Tensor:
        orig_shape = X.shape
        x2d, ldx = ops.as_rows(X)
        y, rstd = ops.rmsnorm_forward(x2d, ldx, None, eps, ops.ROUND_ONCE)
        ctx.save_for_backward(x2d, rstd)
        ctx.ldx = ldx
        ctx.orig_shape = orig_shape
        return y.view(orig_shape)

    @staticmethod
    def backward(ctx, dY: Tensor):
        x2d, rstd = ctx.saved_tensors
        dy2d, lddy = ops.as_rows(dY)
        dx, _ = ops.rmsnorm_backward(dy2d, lddy, x2d, ctx.ldx, None, rstd, need_dw=False)
        return dx.view(ctx.orig_shape), None


class RMSNorm(nn.Module):
    """RMSNorm module (reference: kernels/layernorm_kernels.py:1150-1189)."""

    def __init__(self, hidden_size: int, eps: float = DEFAULT_EPS_RMS,
                 elementwise_affine: bool = True, device: Optional[torch.device] = None,
                 dtype: torch.dtype = torch.float32):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
        else:
            self.register_parameter("weight", None)

    def forward(self, X: Tensor) -> Tensor:
        if self.elementwise_affine:
            return rms_layernorm(X, self.weight, self.eps)
        return _RMSNormNoWeight.apply(X, self.eps)

    def extra_repr(self) -> str:
        return f"{self.hidden_size}, eps={self.eps}, elementwise_affine={self.elementwise_affine}"


class FusedAddRMSLayerNormFunction(torch.autograd.Function):
    """Residual add + RMSNorm in one pass (reference: kernels/layernorm_kernels.py:949-1047).

    forward(X, residual, weight, eps, store_residual) -> (Y, residual_out or None).
    One kernel reads X and residual once and writes Y and h = X + residual
    (rounded); h is also kept for backward when a gradient is needed and
    store_residual is False (the reference then recomputes X + residual).
    """

    @staticmethod
    def forward(ctx, X: Tensor, residual: Tensor, weight: Tensor, eps: float = DEFAULT_EPS_RMS,
                store_residual: bool = True) -> Tuple[Tensor, Optional[Tensor]]:
        orig_shape = X.shape
        if residual.shape != X.shape:
            raise ValueError(f"fused_add_rms_layernorm: residual {tuple(residual.shape)} != "
                             f"X {tuple(X.shape)}")
        x2d, ldx = ops.as_rows(X)
        r2d, ldr = ops.as_rows(residual)
        need_h = store_residual or any(ctx.needs_input_grad[:2])
        y, h, rstd = ops.add_rmsnorm_forward(x2d, ldx, r2d, ldr, weight, eps, ops.ROUND_TWICE,
                                             store_h=need_h)
        ctx.save_for_backward(h, weight, rstd)
        ctx.orig_shape = orig_shape
        return y.view(orig_shape), (h.view(orig_shape) if store_residual else None)

    @staticmethod
    def backward(ctx, dY: Tensor, _unused: Optional[Tensor]):
        h, weight, rstd = ctx.saved_tensors
        dy2d, lddy = ops.as_rows(dY)
        dx, _ = ops.rmsnorm_backward(dy2d, lddy, h, h.shape[1], weight, rstd, need_dw=False)
        dx = dx.view(ctx.orig_shape)
        return dx, dx, None, None, None


def fused_add_rms_layernorm(X: Tensor, residual: Tensor, weight: Tensor,
                            eps: float = DEFAULT_EPS_RMS, return_residual: bool = False):
    """Y = RMSNorm(X + residual) * weight (reference: kernels/layernorm_kernels.py:1094-1121);
    with return_residual also returns X + residual."""
    Y, residual_out = FusedAddRMSLayerNormFunction.apply(X, residual, weight, eps,
                                                         return_residual)
    if return_residual:
        return Y, residual_out
    return Y


class FusedRMSNorm(nn.Module):
    """Residual add + RMSNorm module (reference: kernels/layernorm_kernels.py:1241-1269)."""

    def __init__(self, hidden_size: int, eps: float = DEFAULT_EPS_RMS,
                 device: Optional[torch.device] = None, dtype: torch.dtype = torch.float32):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, X: Tensor, residual: Tensor, return_residual: bool = False):
        return fused_add_rms_layernorm(X, residual, self.weight, self.eps, return_residual)

    def extra_repr(self) -> str:
        return f"{self.hidden_size}, eps={self.eps}"
