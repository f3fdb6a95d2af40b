"""Vocabulary-parallel cross entropy with TrainScale's API on the gfx950 kernels.

Mirrors ``VocabParallelCrossEntropyLoss`` and ``vocab_parallel_cross_entropy``
of distributed/tensor_parallel.py:1479-1666 (data_pipeline/trainer/): logits
are this rank's vocabulary shard [..., Vp], the loss is the mean over every
row (no ignore_index), label smoothing uses the rank's own shard mean, and the
backward is the reference's ((1 - a) * (softmax - onehot) - a / Vp) / (B * S).

The reference makes three all-reduces per step (row max, sum of exp, target
logit). Here each rank reads its shard once into one 16-byte partial per row
(``ops.ce_vocab_shard_stats``); one exchange of those partials between the
ranks (an all-gather of [N, 4] fp32) gives every rank all P partials, which it
merges itself (``ops.ce_vocab_merge``). The exchange is a hook,
``VocabShardExchange.gather``: the default is the single-rank identity; a
tensor-parallel caller installs one that all-gathers over its group, e.g.

    def gather(stats):
        out = stats.new_empty((world, *stats.shape))
        torch.distributed.all_gather_into_tensor(out, stats, group=tp_group)
        return out
    set_vocab_exchange(VocabShardExchange(gather, rank, world))
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Tuple

import torch
from torch import Tensor

from .. import ops
from ..loss.linear_ce import linear_ce_vocab_phase1, linear_ce_vocab_phase2
from ..loss.sota_losses import SECOND_BACKWARD_MSG


def _local_gather(stats: Tensor) -> Tensor:
    return stats.unsqueeze(0)


def _identity(t: Tensor) -> Tensor:
    return t


@dataclass
class VocabShardExchange:
    """How this rank obtains every rank's partials.

    gather(stats [N, 4]) returns [world_size, N, 4], rank-major, with this rank's
    own partials at index ``rank``. reduce_sum(t) returns the sum of t over the
    ranks (the vocabulary-parallel linear CE's grad_hidden partials).
    """
    gather: Callable[[Tensor], Tensor] = _local_gather
    rank: int = 0
    world_size: int = 1
    reduce_sum: Callable[[Tensor], Tensor] = _identity


_exchange = VocabShardExchange()


def set_vocab_exchange(exchange: Optional[VocabShardExchange]) -> None:
    """Installs the partials exchange (None restores the single-rank identity)."""
    global _exchange
    _exchange = exchange if exchange is not None else VocabShardExchange()


def get_vocab_exchange() -> VocabShardExchange:
    return _exchange


def get_tensor_parallel_world_size() -> int:
    return _exchange.world_size


def get_tensor_parallel_rank() -> int:
    return _exchange.rank


class VocabParallelCrossEntropyLoss(torch.autograd.Function):
    """Cross entropy over a vocabulary split across ranks
    (reference: distributed/tensor_parallel.py:1479-1634)."""

    @staticmethod
    def forward(ctx, logits: Tensor, targets: Tensor, vocab_start: int, vocab_end: int,
                label_smoothing: float = 0.0) -> Tensor:
        vp = logits.shape[-1]
        if vocab_end - vocab_start != vp:
            raise ValueError(f"vocab_parallel_cross_entropy: shard [{vocab_start}, {vocab_end}) "
                             f"does not match logits width {vp}")
        x2d, ld = ops.as_rows(logits)
        t = targets.reshape(-1)
        if t.shape[0] != x2d.shape[0]:
            raise ValueError(f"vocab_parallel_cross_entropy: {t.shape[0]} targets for "
                             f"{x2d.shape[0]} rows")
        ex = _exchange
        stats = ops.ce_vocab_shard_stats(x2d, ld, t, vocab_start)
        stats_all = ex.gather(stats) if ex.world_size > 1 else stats.unsqueeze(0)
        if stats_all.shape[0] != ex.world_size or stats_all.shape[1:] != stats.shape:
            raise ValueError(f"vocab_parallel_cross_entropy: exchange returned "
                             f"{tuple(stats_all.shape)} for {ex.world_size} ranks x "
                             f"{tuple(stats.shape)}")
        lse, loss = ops.ce_vocab_merge(stats_all, ex.rank if ex.world_size > 1 else 0, vp,
                                       label_smoothing)
        ctx.save_for_backward(x2d, t, lse)
        ctx.ld = ld
        ctx.vocab_start = int(vocab_start)
        ctx.label_smoothing = float(label_smoothing)
        ctx.shape = logits.shape
        return loss.mean()

    @staticmethod
    def backward(ctx, grad_output: Tensor) -> Tuple[Optional[Tensor], None, None, None, None]:
        x2d, t, lse = ctx.saved_tensors
        n = x2d.shape[0]
        grad = ops.ce_vocab_shard_backward(x2d, ctx.ld, t, lse, grad_output,
                                           1.0 / max(n, 1), ctx.vocab_start,
                                           ctx.label_smoothing)
        return grad.view(ctx.shape), None, None, None, None


def vocab_parallel_cross_entropy(logits: Tensor, targets: Tensor,
                                 label_smoothing: float = 0.0) -> Tensor:
    """Loss over this rank's shard, columns rank * Vp .. (rank + 1) * Vp - 1
    (reference: distributed/tensor_parallel.py:1637-1666)."""
    vp = logits.size(-1)
    vocab_start = get_tensor_parallel_rank() * vp
    return VocabParallelCrossEntropyLoss.apply(logits, targets, vocab_start, vocab_start + vp,
                                               label_smoothing)


class VocabParallelLinearCrossEntropyFunction(torch.autograd.Function):
    """CE of hidden @ weight_shard.T over a vocabulary split across ranks, each rank
    holding the LM head rows vocab_start .. vocab_start + Vp - 1, with the
    gradients formed in the forward (upstream gradient 1) and scaled in the
    backward. The ranks exchange one 16-byte partial per row and sum their
    grad_hidden partials (the exchange hooks); grad_weight stays local."""

    @staticmethod
    def forward(ctx, hidden: Tensor, weight_shard: Tensor, labels: Tensor, vocab_start: int,
                ignore_index: int = -100, reduction: str = "mean") -> Tensor:
        shape = hidden.shape
        ex = _exchange
        stats, state = linear_ce_vocab_phase1(hidden.reshape(-1, shape[-1]), weight_shard,
                                              labels, vocab_start, ignore_index)
        stats_all = ex.gather(stats) if ex.world_size > 1 else stats.unsqueeze(0)
        loss, _, _, gh, gw = linear_ce_vocab_phase2(
            state, stats_all, ignore_index, reduction,
            need_grad_hidden=ctx.needs_input_grad[0], need_grad_weight=ctx.needs_input_grad[1])
        if gh is not None and ex.world_size > 1:
            gh = ex.reduce_sum(gh)
        ctx.hidden_shape = shape
        ctx.save_for_backward(gh, gw)
        return loss

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        if getattr(ctx, "backward_done", False):
            raise RuntimeError(SECOND_BACKWARD_MSG)
        ctx.backward_done = True
        gh, gw = ctx.saved_tensors
        scale = grad_output.detach().float().reshape(1).contiguous()
        if gh is not None:
            ops.scale_(gh, scale)
        if gw is not None:
            ops.scale_(gw, scale)
        gh = gh.view(ctx.hidden_shape) if gh is not None else None
        return gh, gw, None, None, None, None


def vocab_parallel_linear_cross_entropy(hidden: Tensor, weight_shard: Tensor, labels: Tensor,
                                        ignore_index: int = -100,
                                        reduction: str = "mean") -> Tensor:
    """Mean (or sum) CE of hidden @ lm_head.T with this rank's LM head rows
    weight_shard [Vp, H] (vocabulary columns rank * Vp .. (rank + 1) * Vp - 1)."""
    vocab_start = get_tensor_parallel_rank() * weight_shard.shape[0]
    return VocabParallelLinearCrossEntropyFunction.apply(hidden, weight_shard, labels,
                                                         vocab_start, ignore_index, reduction)
