"""Fused linear cross-entropy: loss of (hidden @ weight.T) without materialising the logits.

TrainScale has no such op; its nearest relative is
``chunked_log_softmax(hidden, lm_head[V, H], input_ids)`` (rl_training.py:138-191),
whose weight layout and softcap/scale keywords this API follows.
"""
from __future__ import annotations

import torch
from torch import Tensor

__all__ = ["LinearCrossEntropyFunction", "fused_linear_cross_entropy"]


class LinearCrossEntropyFunction(torch.autograd.Function):
    """Placeholder until the MFMA kernel lands; raises instead of falling back."""

    @staticmethod
    def forward(ctx, hidden: Tensor, weight: Tensor, labels: Tensor, ignore_index: int = -100,
                reduction: str = "mean") -> Tensor:
        raise NotImplementedError("fused linear cross-entropy kernel is not built yet")

    @staticmethod
    def backward(ctx, grad_output: Tensor):  # pragma: no cover
        raise NotImplementedError


def fused_linear_cross_entropy(hidden: Tensor, weight: Tensor, labels: Tensor,
                               ignore_index: int = -100, reduction: str = "mean",
                               logit_softcapping: float = 0.0,
                               logit_scaling: float = 0.0) -> Tensor:
    if logit_softcapping != 0.0 or logit_scaling != 0.0:
        raise NotImplementedError("softcap/scale are not supported by fused linear CE yet")
    return LinearCrossEntropyFunction.apply(hidden, weight, labels, ignore_index, reduction)
