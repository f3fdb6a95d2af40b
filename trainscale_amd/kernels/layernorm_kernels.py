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

LayerNorm/Welford, dropout+RMS and fused residual-add are not part of this
layer.
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
