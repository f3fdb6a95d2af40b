"""Cross-entropy losses with TrainScale's loss API on the gfx950 kernels.

``CrossEntropyLoss`` mirrors loss/__init__.py:130-279 of TrainScale
(data_pipeline/trainer/): ignore_index, label_smoothing in [0, 1),
reduction mean/sum/none. The reference's Triton forward returned losses
without a gradient; this one is differentiable.
"""
from __future__ import annotations

import torch.nn as nn
from torch import Tensor

from .linear_ce import (FusedLinearCrossEntropyFunction, LinearCrossEntropyFunction,
                        SelectiveLogSoftmaxFunction, chunked_log_softmax,
                        fused_linear_cross_entropy, selective_log_softmax)
from .sota_losses import (
    ChunkedCrossEntropyLoss,
    CrossEntropyRowsFunction,
    FusedCrossEntropyFunction,
    FusedCrossEntropyLoss,
    UpstreamGradHint,
    reduce_rows,
)

__all__ = [
    "CrossEntropyLoss",
    "ChunkedCrossEntropyLoss",
    "FusedCrossEntropyLoss",
    "FusedCrossEntropyFunction",
    "CrossEntropyRowsFunction",
    "UpstreamGradHint",
    "LinearCrossEntropyFunction",
    "FusedLinearCrossEntropyFunction",
    "fused_linear_cross_entropy",
    "chunked_log_softmax",
    "selective_log_softmax",
    "SelectiveLogSoftmaxFunction",
]


class CrossEntropyLoss(nn.Module):
    """Cross-entropy with label smoothing (reference: loss/__init__.py:130-279)."""

    def __init__(self, ignore_index: int = -100, label_smoothing: float = 0.0,
                 reduction: str = "mean", *, use_triton: bool = True):
        super().__init__()
        if not 0.0 <= label_smoothing < 1.0:
            raise ValueError(f"label_smoothing must be in [0, 1), got {label_smoothing}")
        if reduction not in ("mean", "sum", "none"):
            raise ValueError(f"Invalid reduction: {reduction}")
        self.ignore_index = ignore_index
        self.label_smoothing = label_smoothing
        self.reduction = reduction
        # Accepted for signature compatibility; every path runs the gfx950 kernels.
        self.use_triton = use_triton
        self.grad_hint = UpstreamGradHint()

    def forward(self, logits: Tensor, labels: Tensor) -> Tensor:
        if logits.dim() == 3:
            logits = logits.reshape(-1, logits.shape[-1])
            labels = labels.reshape(-1)
        if self.reduction == "none":
            return CrossEntropyRowsFunction.apply(logits, labels, self.ignore_index,
                                                  self.label_smoothing)
        return FusedCrossEntropyFunction.apply(logits, labels, self.ignore_index,
                                               self.label_smoothing, self.reduction,
                                               self.grad_hint)
