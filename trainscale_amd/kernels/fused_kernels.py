"""Drop-in counterparts of TrainScale's ``kernels/triton_kernels.py`` hot-path ops.

Same class and function names, argument meanings and return values as the
reference (paths relative to ``data_pipeline/trainer/``):

* ``Fast_RMS_LayerNorm`` / ``fast_rms_layernorm`` / ``TritonRMSNorm``
  (kernels/triton_kernels.py:602-703, :1397-1406): y = x * rstd * w computed in
  fp32 and rounded once; backward returns (dX, dW, None).
* ``Fast_RoPE`` / ``apply_rope`` / ``precompute_freqs_cis``
  (kernels/triton_kernels.py:893-1032): out-of-place rotation of Q and K from
  cos/sin tables indexed by sequence position.
* ``Fast_CrossEntropyLoss`` / ``fast_cross_entropy_loss``
  (kernels/triton_kernels.py:309-467): per-row losses with optional logit
  scaling and softcapping; the backward writes the gradient into the saved
  logits buffer and returns it, as the reference does.
* ``Fast_SwiGLU`` / ``swiglu_forward`` (kernels/triton_kernels.py:1105-1148):
  out = silu(gate).to(up.dtype) * up; backward returns (dgate, dup) in fp32
  arithmetic rounded once.

Every op runs the gfx950 kernels of ``libtrainscale_amd.so``. Unlike the
reference there is no eager fallback: CPU tensors raise.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from .. import ops

__all__ = [
    "Fast_RMS_LayerNorm",
    "fast_rms_layernorm",
    "HipRMSNorm",
    "TritonRMSNorm",
    "Fast_RoPE",
    "apply_rope",
    "precompute_freqs_cis",
    "Fast_CrossEntropyLoss",
    "fast_cross_entropy_loss",
    "Fast_SwiGLU",
    "swiglu_forward",
]


# ---------------------------------------------------------------------------
# RMSNorm (kernels/triton_kernels.py:602-703)
# ---------------------------------------------------------------------------

class Fast_RMS_LayerNorm(torch.autograd.Function):
    """RMSNorm whose forward rounds y = x * rstd * w to the input dtype once."""

    @staticmethod
    def forward(ctx, X: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
        original_shape = X.shape
        x2d, ldx = ops.as_rows(X)
        y, rstd = ops.rmsnorm_forward(x2d, ldx, weight, eps, ops.ROUND_ONCE)
        ctx.save_for_backward(x2d, weight, rstd)
        ctx.ldx = ldx
        ctx.original_shape = original_shape
        return y.view(original_shape)

    @staticmethod
    def backward(ctx, dY: Tensor) -> Tuple[Optional[Tensor], Optional[Tensor], None]:
        x2d, weight, rstd = ctx.saved_tensors
        dy2d, lddy = ops.as_rows(dY)
        dx, dw = ops.rmsnorm_backward(dy2d, lddy, x2d, ctx.ldx, weight, rstd,
                                      need_dw=ctx.needs_input_grad[1])
        return dx.view(ctx.original_shape), dw, None


def fast_rms_layernorm(X: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    """RMSNorm over the last dimension (reference: kernels/triton_kernels.py:687-703)."""
    return Fast_RMS_LayerNorm.apply(X, weight, eps)


class HipRMSNorm(nn.Module):
    """RMSNorm layer on the gfx950 kernels (reference: TritonRMSNorm, triton_kernels.py:1397)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: Tensor) -> Tensor:
        return fast_rms_layernorm(x, self.weight, self.eps)


# The reference's class name, kept so callers need no change.
TritonRMSNorm = HipRMSNorm


# ---------------------------------------------------------------------------
# RoPE (kernels/triton_kernels.py:893-1032)
# ---------------------------------------------------------------------------

class Fast_RoPE(torch.autograd.Function):
    """Out-of-place RoPE of Q [B,S,Hq,D] and K [B,S,Hk,D] at positions 0..S-1.

    cos/sin are [max_seq_len, D/2] tables; the rotation is evaluated in fp32 and
    rounded once to the input dtype. Backward applies the transpose rotation.
    """

    @staticmethod
    def forward(ctx, q: Tensor, k: Tensor, cos: Tensor, sin: Tensor,
                interleaved: bool = False) -> Tuple[Tensor, Tensor]:
        q = ops._bshd(q, "Fast_RoPE q")
        k = ops._bshd(k, "Fast_RoPE k")
        q_out = torch.empty_like(q)
        k_out = torch.empty_like(k)
        ops.rope_apply(q, q_out, k, k_out, cos=cos, sin=sin, interleaved=interleaved)
        ctx.save_for_backward(cos, sin)
        ctx.interleaved = interleaved
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq: Optional[Tensor], dk: Optional[Tensor]):
        cos, sin = ctx.saved_tensors
        dq_out = dk_out = None
        if dq is not None:
            dq = ops._bshd(dq, "Fast_RoPE dq")
            dq_out = torch.empty_like(dq)
        if dk is not None:
            dk = ops._bshd(dk, "Fast_RoPE dk")
            dk_out = torch.empty_like(dk)
        ops.rope_apply(dq, dq_out, dk, dk_out, cos=cos, sin=sin,
                       interleaved=ctx.interleaved, backward=True)
        return dq_out, dk_out, None, None, None


def apply_rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor,
               interleaved: bool = False) -> Tuple[Tensor, Tensor]:
    """RoPE of Q and K (reference: kernels/triton_kernels.py:984-1004)."""
    return Fast_RoPE.apply(q, k, cos, sin, interleaved)


def precompute_freqs_cis(dim: int, max_seq_len: int, theta: float = 10000.0,
                         device: Optional[torch.device] = None,
                         dtype: torch.dtype = torch.float32,
                         scaling_factor: float = 1.0) -> Tuple[Tensor, Tensor]:
    """cos/sin tables [max_seq_len, dim//2] (reference: kernels/triton_kernels.py:1007-1032).

    inv_freq = 1 / theta**(arange(0, dim, 2)/dim) and the angle
    outer(arange(max_seq_len)/scaling_factor, inv_freq), all in fp32.
    """
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, device=device, dtype=torch.float32) / dim))
    t = torch.arange(max_seq_len, device=device, dtype=torch.float32) / scaling_factor
    angles = torch.outer(t, freqs)
    return torch.cos(angles).to(dtype), torch.sin(angles).to(dtype)


# ---------------------------------------------------------------------------
# Cross-entropy (kernels/triton_kernels.py:309-467)
# ---------------------------------------------------------------------------

class Fast_CrossEntropyLoss(torch.autograd.Function):
    """Per-row cross-entropy over logits [N, V] with ignore_index -100.

    forward -> fp32 losses [N] (0 for ignored rows). backward writes
    dloss * (softmax - onehot) (with the scaling/softcap chain rule) into the
    logits buffer saved by forward and returns that buffer, like the reference.
    """

    @staticmethod
    def forward(ctx, logits: Tensor, labels: Tensor, logit_softcapping: float = 0.0,
                logit_scaling: float = 0.0) -> Tensor:
        if logits.dim() != 2:
            raise ValueError(f"Fast_CrossEntropyLoss: logits must be [N, V], got {tuple(logits.shape)}")
        l2d, ld = ops.as_rows(logits)
        losses, lse = ops.ce_forward(l2d, ld, labels, -100, logit_scaling, logit_softcapping)
        ctx.save_for_backward(l2d, lse, labels)
        ctx.ld = ld
        ctx.logit_softcapping = logit_softcapping
        ctx.logit_scaling = logit_scaling
        return losses

    @staticmethod
    def backward(ctx, dlosses: Tensor):
        l2d, lse, labels = ctx.saved_tensors
        ops.ce_backward(l2d, ctx.ld, labels, lse, dlosses, l2d, ctx.ld,
                        ignore_index=-100, logit_scale=ctx.logit_scaling,
                        softcap=ctx.logit_softcapping)
        return l2d, None, None, None


def fast_cross_entropy_loss(logits: Tensor, labels: Tensor, logit_softcapping: float = 0.0,
                            logit_scaling: float = 0.0, n_items: Optional[int] = None,
                            reduction: str = "mean") -> Tensor:
    """Cross-entropy with mean/sum/none reduction (reference: triton_kernels.py:427-467)."""
    original_shape = logits.shape
    if logits.dim() == 3:
        batch, seq_len, vocab = logits.shape
        logits = logits.view(batch * seq_len, vocab)
        labels = labels.view(-1)
    loss = Fast_CrossEntropyLoss.apply(logits, labels, logit_softcapping, logit_scaling)
    if reduction == "none":
        return loss.view(original_shape[:-1]) if len(original_shape) == 3 else loss
    if reduction == "sum":
        return loss.sum()
    if n_items is None:
        n_items = (labels != -100).sum()
    return loss.sum() / n_items


class Fast_SwiGLU(torch.autograd.Function):
    """SwiGLU (reference: kernels/triton_kernels.py:1105-1143): forward(gate, up) -> out."""

    @staticmethod
    def forward(ctx, gate: Tensor, up: Tensor) -> Tensor:
        out = ops.swiglu_forward(gate, up)
        ctx.save_for_backward(gate.contiguous(), up.contiguous())
        return out

    @staticmethod
    def backward(ctx, dout: Tensor) -> Tuple[Tensor, Tensor]:
        gate, up = ctx.saved_tensors
        return ops.swiglu_backward(dout, gate, up)


def swiglu_forward(gate: Tensor, up: Tensor) -> Tensor:
    """silu(gate) * up (reference: kernels/triton_kernels.py:1146-1148)."""
    return Fast_SwiGLU.apply(gate, up)
