"""Drop-in counterparts of the cross-entropy classes of TrainScale's ``loss/sota_losses.py``.

Reference (``data_pipeline/trainer/``):

* ``FusedCrossEntropyFunction`` (loss/sota_losses.py:437-532):
  apply(logits, labels, ignore_index, label_smoothing, reduction) -> reduced loss;
* ``FusedCrossEntropyLoss`` (:539-617);
* ``ChunkedCrossEntropyLoss`` (:620-744) — the trainer's configured loss on
  ROCm (trainers/sota_trainer.py:1876-1883).

All three compute the same quantity: per-row
loss = (1-a)*(lse - x[label]) + a*(lse - mean(x)), zero on ignore_index rows,
reduced by mean (over non-ignored rows, at least 1), sum, batchmean (over all
rows) or none. Here every one runs the gfx950 kernels directly on the logits
in their own dtype with fp32 arithmetic: with a reduction, one pass reads each
valid row once and writes its gradient (the forward forms it); without one,
one read in forward, one read plus one write in backward. The reference's ChunkedCrossEntropyLoss builds an
fp32 copy of the logits and differentiates through torch ops; its eval mode
accumulates in the logits dtype, where this version stays in fp32.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from .. import ops

__all__ = [
    "CrossEntropyRowsFunction",
    "UpstreamGradHint",
    "FusedCrossEntropyFunction",
    "FusedCrossEntropyLoss",
    "ChunkedCrossEntropyLoss",
    "reduce_rows",
]

_REDUCTIONS = ("mean", "sum", "batchmean", "none")


class CrossEntropyRowsFunction(torch.autograd.Function):
    """Per-row cross-entropy losses (fp32 [N]) of logits [N, V] with autograd.

    backward returns a new gradient tensor in the logits dtype.
    """

    @staticmethod
    def forward(ctx, logits: Tensor, labels: Tensor, ignore_index: int = -100,
                label_smoothing: float = 0.0, logit_scale: float = 0.0,
                softcap: float = 0.0) -> Tensor:
        l2d, ld = ops.as_rows(logits)
        loss, lse = ops.ce_forward(l2d, ld, labels, ignore_index, logit_scale, softcap,
                                   label_smoothing)
        ctx.save_for_backward(l2d, labels, lse)
        ctx.ld = ld
        ctx.cfg = (ignore_index, label_smoothing, logit_scale, softcap)
        ctx.shape = logits.shape
        return loss

    @staticmethod
    def backward(ctx, dloss: Tensor):
        l2d, labels, lse = ctx.saved_tensors
        ignore_index, label_smoothing, logit_scale, softcap = ctx.cfg
        grad = torch.empty(l2d.shape, dtype=l2d.dtype, device=l2d.device)
        ops.ce_backward(l2d, ctx.ld, labels, lse, dloss, grad, l2d.shape[1],
                        ignore_index=ignore_index, logit_scale=logit_scale, softcap=softcap,
                        label_smoothing=label_smoothing)
        return grad.view(ctx.shape), None, None, None, None, None


def reduce_rows(loss: Tensor, labels: Tensor, ignore_index: int, reduction: str) -> Tensor:
    """Reduction of per-row losses as the reference's loss classes do it."""
    if reduction == "mean":
        valid = (labels.reshape(-1) != ignore_index).sum()
        return loss.sum() / valid.clamp(min=1)
    if reduction == "sum":
        return loss.sum()
    if reduction == "batchmean":
        return loss.sum() / loss.shape[0] if loss.shape[0] > 0 else loss.sum()
    return loss


def _flatten(logits: Tensor, labels: Tensor) -> Tuple[Tensor, Tensor]:
    if logits.dim() == 3:
        logits = logits.reshape(-1, logits.size(-1))
        labels = labels.reshape(-1)
    return logits, labels


def _row_weight(labels: Tensor, ignore_index: int, reduction: str, n: int) -> Tensor:
    """d(reduced loss)/d(row loss) as a one-element fp32 device tensor (no host sync)."""
    if reduction == "mean":
        valid = (labels != ignore_index).sum().clamp(min=1)
        return valid.to(torch.float32).reciprocal().reshape(1)
    if reduction == "batchmean":
        return torch.full((1,), 1.0 / max(n, 1), dtype=torch.float32, device=labels.device)
    return torch.ones((1,), dtype=torch.float32, device=labels.device)


SECOND_BACKWARD_MSG = (
    "backward was called a second time through a loss whose gradient is formed in the "
    "forward pass and scaled in place by the first backward (retain_graph=True); run the "
    "forward again, or use reduction='none' (two-pass schedule, which supports it)")


class UpstreamGradHint:
    """Prediction of a loss's upstream gradient, one fp32 device scalar per device.

    A trainer scales the loss the same way every step (the reference divides it
    by gradient_accumulation_steps, trainers/sota_trainer.py:2190, which is 4 in
    its ROCm configs), so the upstream gradient of step t predicts that of step
    t+1. The forward pass forms the gradient for the prediction; backward
    corrects it by now/predicted, which is exactly 1 (nothing written) once the
    prediction holds, and records the new value. All on the device, no sync.
    """

    def __init__(self) -> None:
        self._per_device = {}

    def get(self, device: torch.device) -> Tensor:
        t = self._per_device.get(device)
        if t is None:
            t = torch.ones((1,), dtype=torch.float32, device=device)
            self._per_device[device] = t
        return t


class FusedCrossEntropyFunction(torch.autograd.Function):
    """Reduced cross-entropy in one autograd node (reference: loss/sota_losses.py:437-532).

    For mean, sum and batchmean the gradient is formed in the forward pass in
    the same read of the logits that yields the loss (ts_ce_fwd_bwd: one read
    of each valid row, one write of each gradient row), for a predicted
    upstream gradient (``hint``, an UpstreamGradHint, else 1); backward
    rescales it in place by actual/predicted, on the device and only when the
    ratio is not 1. Without a gradient to compute (no_grad, eval) only the
    forward kernel runs. reduction="none" keeps the two-pass schedule, since
    per-row upstream gradients are unknown until backward.
    """

    @staticmethod
    def forward(ctx, logits: Tensor, labels: Tensor, ignore_index: int, label_smoothing: float,
                reduction: str, hint: Optional[UpstreamGradHint] = None) -> Tensor:
        if reduction not in _REDUCTIONS:
            raise ValueError(f"Invalid reduction: {reduction}")
        l2d, ld = ops.as_rows(logits)
        flat = labels.reshape(-1)
        ctx.shape = logits.shape
        ctx.cfg = (ignore_index, label_smoothing, reduction)
        if reduction != "none" and ctx.needs_input_grad[0]:
            w = _row_weight(flat, ignore_index, reduction, l2d.shape[0])
            if hint is not None:
                ctx.hint = hint.get(l2d.device)
                used = ctx.hint.clone()
                w = w * used
            else:
                ctx.hint = None
                used = None
            loss, _, grad = ops.ce_forward_backward(l2d, ld, flat, w, 1.0, ignore_index, 0.0, 0.0,
                                                    label_smoothing)
            ctx.fused = True
            ctx.save_for_backward(grad, used)
            return reduce_rows(loss, flat, ignore_index, reduction)
        loss, lse = ops.ce_forward(l2d, ld, flat, ignore_index, 0.0, 0.0, label_smoothing)
        ctx.fused = False
        ctx.save_for_backward(l2d, flat, lse)
        ctx.ld = ld
        return reduce_rows(loss, flat, ignore_index, reduction)

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        ignore_index, label_smoothing, reduction = ctx.cfg
        if ctx.fused:
            # The gradient was formed in the forward and is scaled here in place; a
            # second backward through the same graph (retain_graph=True) would scale
            # it again, so it is refused rather than returning a wrong gradient.
            if getattr(ctx, "backward_done", False):
                raise RuntimeError(SECOND_BACKWARD_MSG)
            ctx.backward_done = True
            grad, used = ctx.saved_tensors
            if used is None:
                ops.scale_(grad, grad_output)
            else:
                ops.rescale_(grad, grad_output, used, ctx.hint)
            return grad.view(ctx.shape), None, None, None, None, None
        l2d, labels, lse = ctx.saved_tensors
        n = l2d.shape[0]
        if reduction == "none":
            dloss = grad_output.float().reshape(-1)
        else:
            dloss = grad_output.float() * _row_weight(labels, ignore_index, reduction, n)
        grad = torch.empty(l2d.shape, dtype=l2d.dtype, device=l2d.device)
        ops.ce_backward(l2d, ctx.ld, labels, lse, dloss, grad, l2d.shape[1],
                        ignore_index=ignore_index, label_smoothing=label_smoothing)
        return grad.view(ctx.shape), None, None, None, None, None


class FusedCrossEntropyLoss(nn.Module):
    """Cross-entropy module (reference: loss/sota_losses.py:539-617).

    The reference casts the logits to fp32 before its kernel; the gfx950
    kernel reads them in their own dtype and accumulates in fp32.
    """

    __constants__ = ["ignore_index", "label_smoothing", "reduction"]

    def __init__(self, ignore_index: int = -100, label_smoothing: float = 0.0,
                 reduction: str = "mean") -> None:
        super().__init__()
        if reduction not in _REDUCTIONS:
            raise ValueError(f"Invalid reduction: {reduction}")
        self.ignore_index = ignore_index
        self.label_smoothing = label_smoothing
        self.reduction = reduction
        self.grad_hint = UpstreamGradHint()

    def forward(self, logits: Tensor, labels: Tensor) -> Tensor:
        logits, labels = _flatten(logits, labels)
        return FusedCrossEntropyFunction.apply(logits, labels, self.ignore_index,
                                               self.label_smoothing, self.reduction,
                                               self.grad_hint)

    def extra_repr(self) -> str:
        return (f"ignore_index={self.ignore_index}, label_smoothing={self.label_smoothing}, "
                f"reduction='{self.reduction}'")


class ChunkedCrossEntropyLoss(nn.Module):
    """Cross-entropy over large vocabularies (reference: loss/sota_losses.py:620-744).

    ``chunk_size`` is kept for signature compatibility; the gfx950 kernel walks
    the whole vocabulary row with an online max/sum and never materialises an
    fp32 copy, so no chunking is needed. With a reduction, the gradient is
    formed in the forward pass (see FusedCrossEntropyFunction).
    """

    __constants__ = ["ignore_index", "label_smoothing", "reduction", "chunk_size"]

    def __init__(self, ignore_index: int = -100, label_smoothing: float = 0.0,
                 reduction: str = "mean", chunk_size: int = 32768) -> None:
        super().__init__()
        if reduction not in _REDUCTIONS:
            raise ValueError(f"Invalid reduction: {reduction}")
        self.ignore_index = ignore_index
        self.label_smoothing = label_smoothing
        self.reduction = reduction
        self.chunk_size = chunk_size
        self.grad_hint = UpstreamGradHint()

    def forward(self, logits: Tensor, labels: Tensor) -> Tensor:
        logits, labels = _flatten(logits, labels)
        if self.reduction == "none":
            return CrossEntropyRowsFunction.apply(logits, labels, self.ignore_index,
                                                  self.label_smoothing)
        return FusedCrossEntropyFunction.apply(logits, labels, self.ignore_index,
                                               self.label_smoothing, self.reduction,
                                               self.grad_hint)
