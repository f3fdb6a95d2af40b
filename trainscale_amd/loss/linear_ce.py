"""Fused linear cross-entropy: loss of (hidden @ weight.T) without materialising the logits.

TrainScale has no such op; its nearest relative is
``chunked_log_softmax(hidden, lm_head[V, H], input_ids)`` (rl_training.py:138-191),
whose weight layout and logit transforms (softcapping, then scaling, then
temperature, rl_training.py:114-122) this API follows, with the keywords of
``fast_cross_entropy_loss`` (kernels/triton_kernels.py:427-467).

Two schedules run on the gfx950 kernels:

* ``"two_pass"`` (any reduction, any upstream gradient, backward twice): the
  forward (``ts_flce_forward``) runs the logits GEMM once and keeps only
  per-row softmax statistics and the label's logit; no logits are stored. The
  backward (``ts_flce_backward``) recomputes the logits one vocabulary chunk
  at a time (about V/8 columns), forms the chunk's dlogits in the GEMM's
  epilogue and runs the two gradient GEMMs on them: grad_hidden accumulates
  over the chunks in fp32, grad_weight's rows of the chunk are written
  directly. Scratch: N x chunk bf16 dlogits plus N x H fp32.
* ``"fused"`` (mean/sum, no transforms): one call (``ts_flce_fwd_bwd``) forms
  the loss and both gradients for an upstream gradient of 1, token chunk by
  token chunk: half the tokens by default, whose bf16 logits are the only
  [rows, V] scratch (half the [N, V] logits), with grad_weight summed over the
  chunks in its bf16 output (one bf16 rounding of the partial sum between the
  chunks; fp32 accumulation is opt-in); the backward scales the gradients in
  place. Three GEMMs instead of four.
* ``"stored_logits"`` (opt-in; any reduction and transform): the two-pass
  forward also keeps the bf16 logits ([N, V], N * V * 2 bytes, as the
  reference's chunked_log_softmax keeps each chunk's logits for autograd);
  the backward forms dlogits over them in place and runs the two gradient
  GEMMs, three GEMMs in all instead of four. The kept logits are consumed: a
  second backward recomputes, as "two_pass" does.
* ``"auto"`` (the default): "fused" when gradients are needed for mean/sum
  without transforms, "two_pass" otherwise (forward only, reduction "none",
  transforms).

Numerics follow the reference's bf16 path: logits are rounded to bf16 as a
bf16 matmul rounds them, softmax statistics and the loss are fp32, dlogits are
bf16, and the gradient GEMMs accumulate in fp32.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from .. import _lib, ops
from .._lib import check, ptr
from .sota_losses import SECOND_BACKWARD_MSG

__all__ = ["LinearCrossEntropyFunction", "FusedLinearCrossEntropyFunction",
           "fused_linear_cross_entropy", "chunked_log_softmax", "selective_log_softmax",
           "SelectiveLogSoftmaxFunction", "DEFAULT_TOKEN_CHUNKS",
           "linear_ce_forward", "linear_ce_backward", "linear_ce_forward_backward",
           "VocabShardState", "linear_ce_vocab_phase1", "linear_ce_vocab_phase2"]

# The one-call schedule's token chunk with chunk_tokens=None: half the tokens
# (rounded up to 256 rows), so its bf16 logits scratch stays within half of the
# [N, V] logits; batches of up to 256 tokens run as one chunk. Measured on MI355X
# at C5 (N = 8192): 21.5 ms with two chunks of 4096 tokens, 22.5 ms with four of
# 2048 (two more bf16 read-modify-write passes over grad_weight), 21.4 ms with all
# the logits in one chunk.
DEFAULT_TOKEN_CHUNKS = 2

_REDUCTIONS = {"mean": 0, "sum": 1}
TS_FLCE_GRADS, TS_FLCE_ACCUM_BF16 = 1, 2  # include/trainscale_amd.h
_REDUCTIONS_2P = {"mean": 0, "sum": 1, "none": 2}


def _chunk_rows(N: int, V: int, chunk_tokens: Optional[int]) -> int:
    """Token chunk of the one-call schedule (0: one chunk)."""
    if chunk_tokens is not None:
        return int(chunk_tokens)
    rows = -(-N // DEFAULT_TOKEN_CHUNKS)
    rows = -(-rows // 256) * 256
    return 0 if rows >= N else rows


def _pad_h(hidden: Tensor, weight: Tensor):
    """The kernels take H in whole 16-byte vectors (8 bf16): for other H, hidden and
    weight are copied into zero-padded [.., round_up(H, 8)] tensors. The zero columns
    leave the logits unchanged and receive zero gradients, which the callers slice
    off. Returns (hidden, weight, H of the caller)."""
    H = hidden.shape[1]
    if H % 8 == 0:
        return hidden, weight, H
    pad = 8 - H % 8
    return (torch.nn.functional.pad(hidden, (0, pad)), torch.nn.functional.pad(weight, (0, pad)),
            H)


def _unpad(g: Optional[Tensor], H: int) -> Optional[Tensor]:
    return g if g is None or g.shape[1] == H else g[:, :H].contiguous()


def _logits_ld(V: int) -> int:
    """Row stride of the bf16 logits the kernels keep: whole 16-byte vectors."""
    return -(-V // 8) * 8


def _operands(what: str, hidden: Tensor, weight: Tensor, labels: Tensor):
    dev = _lib.require_gpu(what, hidden, weight, labels)
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError(f"{what}: hidden and weight must be bfloat16 (got {hidden.dtype}, "
                        f"{weight.dtype})")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"{what}: hidden {tuple(hidden.shape)} and weight "
                         f"{tuple(weight.shape)} must be [N, H] and [V, H]")
    hidden, weight, _ = _pad_h(hidden, weight)
    hidden, weight = _rows_operand(hidden), _rows_operand(weight)
    labels = labels.reshape(-1)
    if labels.shape[0] != hidden.shape[0]:
        raise ValueError(f"{what}: {labels.shape[0]} labels for {hidden.shape[0]} rows")
    labels = labels.to(torch.int64).contiguous()
    return dev, hidden, weight, labels


def _ld(t: Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def linear_ce_forward(hidden: Tensor, weight: Tensor, labels: Tensor, ignore_index: int = -100,
                      reduction: str = "mean", logit_softcapping: float = 0.0,
                      logit_scaling: float = 0.0, temperature: float = 1.0,
                      keep_logits: bool = False):
    """ts_flce_forward: returns (loss fp32 0-d or None for reduction "none",
    loss_rows fp32 [N], lse fp32 [N]). lse is that of the transformed logits and
    is what linear_ce_backward needs. With keep_logits (ts_flce_forward_keep) a
    fourth value, the bf16 logits [N, V] (a view of rows padded to whole 16-byte
    vectors, row stride round_up(V, 8)), for linear_ce_backward(logits=...)."""
    if reduction not in _REDUCTIONS_2P:
        raise ValueError(f"fused_linear_cross_entropy: reduction must be 'mean', 'sum' or "
                         f"'none', got {reduction!r}")
    dev, hidden, weight, labels = _operands("fused_linear_cross_entropy", hidden, weight, labels)
    N, H = hidden.shape
    V = weight.shape[0]
    loss = (torch.empty((), dtype=torch.float32, device=dev) if reduction != "none" else None)
    rows = torch.empty((N,), dtype=torch.float32, device=dev)
    lse = torch.empty((N,), dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws_bytes = int(lib.ts_flce_forward_workspace_size(N, V))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    args = (ptr(hidden), _ld(hidden), ptr(weight), _ld(weight), ptr(labels), N, H, V,
            int(ignore_index), _REDUCTIONS_2P[reduction], float(logit_softcapping),
            float(logit_scaling), float(temperature), ptr(loss), ptr(rows), ptr(lse))
    if not keep_logits:
        with _lib.on_device(dev):
            check(lib.ts_flce_forward(*args, ptr(ws), ws_bytes, _lib.stream_handle(dev)),
                  "ts_flce_forward")
        return loss, rows, lse
    logits = torch.empty((N, _logits_ld(V)), dtype=torch.bfloat16, device=dev)
    with _lib.on_device(dev):
        check(lib.ts_flce_forward_keep(*args, ptr(logits), ptr(ws), ws_bytes,
                                       _lib.stream_handle(dev)), "ts_flce_forward_keep")
    return loss, rows, lse, logits[:, :V]


def linear_ce_backward(hidden: Tensor, weight: Tensor, labels: Tensor, lse: Tensor,
                       dloss: Tensor, ignore_index: int = -100, reduction: str = "mean",
                       logit_softcapping: float = 0.0, logit_scaling: float = 0.0,
                       temperature: float = 1.0, need_grad_hidden: bool = True,
                       need_grad_weight: bool = True, vocab_chunk: Optional[int] = None,
                       logits: Optional[Tensor] = None):
    """ts_flce_backward: (grad_hidden [N, H] or None, grad_weight [V, H] or None) for the
    upstream gradient dloss (one value for mean/sum, or [N] per-row values for "none";
    a single value broadcasts). vocab_chunk: columns per recomputed chunk (default
    about V/8). With `logits`, the [N, V] bf16 logits linear_ce_forward kept
    (keep_logits), ts_flce_backward_kept forms the gradients from them instead of
    recomputing, and overwrites them."""
    if reduction not in _REDUCTIONS_2P:
        raise ValueError(f"fused_linear_cross_entropy: bad reduction {reduction!r}")
    H0 = hidden.shape[-1]
    dev, hidden, weight, labels = _operands("fused_linear_cross_entropy", hidden, weight, labels)
    N, H = hidden.shape
    V = weight.shape[0]
    dloss = dloss.detach().to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if dloss.numel() not in (1, N):
        raise ValueError(f"fused_linear_cross_entropy: {dloss.numel()} upstream values for "
                         f"{N} rows")
    stride = 1 if dloss.numel() == N and N > 1 else 0
    lse = lse.detach().to(torch.float32).reshape(-1).contiguous()
    gh = torch.empty((N, H), dtype=torch.bfloat16, device=dev) if need_grad_hidden else None
    gw = torch.empty((V, H), dtype=torch.bfloat16, device=dev) if need_grad_weight else None
    lib = _lib.load()
    if logits is not None:
        if (logits.shape != (N, V) or logits.dtype != torch.bfloat16 or logits.device != dev or
                (N > 0 and (logits.stride(1) != 1 or logits.stride(0) != _logits_ld(V)))):
            raise ValueError(f"fused_linear_cross_entropy: kept logits must be bf16 [{N}, {V}] "
                             f"on {dev} with row stride {_logits_ld(V)} (as linear_ce_forward "
                             f"returns them)")
        ws_bytes = int(lib.ts_flce_backward_kept_workspace_size(N))
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        with _lib.on_device(dev):
            check(lib.ts_flce_backward_kept(
                ptr(hidden), _ld(hidden), ptr(weight), _ld(weight), ptr(labels), N, H, V,
                int(ignore_index), _REDUCTIONS_2P[reduction], float(logit_softcapping),
                float(logit_scaling), float(temperature), ptr(lse), ptr(dloss), stride,
                ptr(logits), ptr(gh), ptr(gw), ptr(ws), ws_bytes, _lib.stream_handle(dev)),
                "ts_flce_backward_kept")
        return _unpad(gh, H0), _unpad(gw, H0)
    chunk = int(vocab_chunk) if vocab_chunk else 0
    ws_bytes = int(lib.ts_flce_backward_workspace_size(N, H, V, chunk))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    with _lib.on_device(dev):
        check(lib.ts_flce_backward(
            ptr(hidden), _ld(hidden), ptr(weight), _ld(weight), ptr(labels), N, H, V,
            int(ignore_index), _REDUCTIONS_2P[reduction], float(logit_softcapping),
            float(logit_scaling), float(temperature), ptr(lse), ptr(dloss), stride, ptr(gh),
            ptr(gw), chunk, ptr(ws), ws_bytes, _lib.stream_handle(dev)), "ts_flce_backward")
    return _unpad(gh, H0), _unpad(gw, H0)


def linear_ce_forward_backward(hidden: Tensor, weight: Tensor, labels: Tensor,
                               ignore_index: int = -100, reduction: str = "mean",
                               need_grad_hidden: bool = True, need_grad_weight: bool = True,
                               chunk_tokens: Optional[int] = None,
                               grad_weight_accum: str = "fp32"):
    """Runs ts_flce_fwd_bwd; returns (loss fp32 0-d, loss_rows [N], lse [N],
    grad_hidden or None, grad_weight or None) for an upstream gradient of 1.
    chunk_tokens: rows per token chunk (None: half the tokens, 0: one chunk);
    grad_weight_accum: "fp32" (a V x H fp32 workspace, rounded once) or "bf16" (summed
    in the bf16 output, rounded after each chunk)."""
    if grad_weight_accum not in ("fp32", "bf16"):
        raise ValueError(f"fused_linear_cross_entropy: grad_weight_accum must be 'fp32' or "
                         f"'bf16', got {grad_weight_accum!r}")
    dev = _lib.require_gpu("fused_linear_cross_entropy", hidden, weight, labels)
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("fused_linear_cross_entropy: hidden and weight must be bfloat16")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"fused_linear_cross_entropy: hidden {tuple(hidden.shape)} and weight "
                         f"{tuple(weight.shape)} must be [N, H] and [V, H]")
    if reduction not in _REDUCTIONS:
        raise ValueError(f"fused_linear_cross_entropy: reduction must be 'mean' or 'sum', "
                         f"got {reduction!r}")
    if hidden.shape[1] % 8 != 0:
        H0 = hidden.shape[1]
        hp, wp, _ = _pad_h(hidden, weight)
        loss, rows, lse, gh, gw = linear_ce_forward_backward(
            hp, wp, labels, ignore_index, reduction, need_grad_hidden, need_grad_weight,
            chunk_tokens, grad_weight_accum)
        return loss, rows, lse, _unpad(gh, H0), _unpad(gw, H0)
    if hidden.stride(1) != 1 or (hidden.shape[0] > 1 and hidden.stride(0) % 8 != 0):
        hidden = hidden.contiguous()
    if weight.stride(1) != 1 or (weight.shape[0] > 1 and weight.stride(0) % 8 != 0):
        weight = weight.contiguous()
    N, H = hidden.shape
    V = weight.shape[0]
    labels = labels.reshape(-1)
    if labels.shape[0] != N:
        raise ValueError(f"fused_linear_cross_entropy: {labels.shape[0]} labels for {N} rows")
    labels = labels.to(torch.int64).contiguous()
    if N % 8 != 0:
        # the one-call kernel takes whole groups of 8 rows: pad with ignored rows, which
        # change neither the loss nor grad_weight, and drop their grad_hidden rows
        pad = 8 - N % 8
        hidden = torch.cat([hidden, hidden.new_zeros((pad, H))])
        labels = torch.cat([labels, labels.new_full((pad,), int(ignore_index))])
        out = linear_ce_forward_backward(hidden, weight, labels, ignore_index, reduction,
                                         need_grad_hidden, need_grad_weight, chunk_tokens,
                                         grad_weight_accum)
        loss, rows, lse, gh, gw = out
        return loss, rows[:N], lse[:N], gh[:N] if gh is not None else None, gw
    ldh = hidden.stride(0) if N > 1 else H
    ldw = weight.stride(0) if V > 1 else H
    loss = torch.empty((), dtype=torch.float32, device=dev)
    loss_rows = torch.empty((N,), dtype=torch.float32, device=dev)
    lse = torch.empty((N,), dtype=torch.float32, device=dev)
    gh = torch.empty((N, H), dtype=torch.bfloat16, device=dev) if need_grad_hidden else None
    gw = torch.empty((V, H), dtype=torch.bfloat16, device=dev) if need_grad_weight else None
    chunk = _chunk_rows(N, V, chunk_tokens)
    lib = _lib.load()
    grads = gh is not None or gw is not None
    flags = TS_FLCE_ACCUM_BF16 if grad_weight_accum == "bf16" else 0
    ws_bytes = int(lib.ts_flce_workspace_size(N, H, V, chunk,
                                              (TS_FLCE_GRADS if grads else 0) | flags))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    with _lib.on_device(dev):
        check(lib.ts_flce_fwd_bwd(
            ptr(hidden), ldh, ptr(weight), ldw, ptr(labels), N, H, V, int(ignore_index),
            _REDUCTIONS[reduction], ptr(loss), ptr(loss_rows), ptr(lse), ptr(gh), ptr(gw),
            chunk, flags, ptr(ws), ws_bytes, _lib.stream_handle(dev)), "ts_flce_fwd_bwd")
    return loss, loss_rows, lse, gh, gw


class VocabShardState:
    """What phase 2 of the vocabulary-parallel linear CE needs from phase 1: the
    rank's operands (padded to whole groups of 8 rows and 8 columns: the kernels'
    shape), the caller's N and H, and the workspace that holds its shard's logits."""

    def __init__(self, hidden, weight, labels, vocab_start, ws, ws_bytes, dev, n0, h0):
        self.hidden, self.weight, self.labels = hidden, weight, labels
        self.vocab_start, self.ws, self.ws_bytes, self.dev = vocab_start, ws, ws_bytes, dev
        self.N, self.H = hidden.shape
        self.N0, self.H0 = n0, h0
        self.Vp = weight.shape[0]
        self.ldh = hidden.stride(0) if self.N > 1 else self.H
        self.ldw = weight.stride(0) if self.Vp > 1 else self.H


def _rows_operand(t: Tensor) -> Tensor:
    if t.stride(1) != 1 or (t.shape[0] > 1 and t.stride(0) % 8 != 0):
        t = t.contiguous()
    return t


def linear_ce_vocab_phase1(hidden: Tensor, weight_shard: Tensor, labels: Tensor,
                           vocab_start: int, ignore_index: int = -100):
    """ts_flce_vocab_fwd: this rank's logits over its shard of the LM head (kept in the
    workspace) and its per-row partials [N, 4] fp32, the tensor the ranks exchange.
    Returns (partials, state). Any N, H and shard width Vp: the kernels take N and H in
    groups of 8, so other shapes run on copies padded with rows labelled ignore_index
    (which phase 2 must then be given) and zero columns."""
    dev = _lib.require_gpu("vocab_parallel_linear_cross_entropy", hidden, weight_shard, labels)
    if hidden.dtype != torch.bfloat16 or weight_shard.dtype != torch.bfloat16:
        raise TypeError("vocab_parallel_linear_cross_entropy: hidden and weight must be bfloat16")
    if hidden.dim() != 2 or weight_shard.dim() != 2 or hidden.shape[1] != weight_shard.shape[1]:
        raise ValueError(f"vocab_parallel_linear_cross_entropy: hidden {tuple(hidden.shape)} and "
                         f"weight {tuple(weight_shard.shape)} must be [N, H] and [Vp, H]")
    n0, h0 = hidden.shape
    labels = labels.reshape(-1)
    if labels.shape[0] != n0:
        raise ValueError(f"vocab_parallel_linear_cross_entropy: {labels.shape[0]} labels for "
                         f"{n0} rows")
    labels = labels.to(torch.int64).contiguous()
    hidden, weight_shard, _ = _pad_h(hidden, weight_shard)
    if n0 % 8 != 0:
        pad = 8 - n0 % 8
        hidden = torch.cat([hidden, hidden.new_zeros((pad, hidden.shape[1]))])
        labels = torch.cat([labels, labels.new_full((pad,), int(ignore_index))])
    hidden, weight_shard = _rows_operand(hidden), _rows_operand(weight_shard)
    N = hidden.shape[0]
    if N == 0:  # no rows: nothing to launch; phase 2 returns the empty results
        state = VocabShardState(hidden, weight_shard, labels, int(vocab_start), None, 0, dev,
                                n0, h0)
        return torch.empty((0, 4), dtype=torch.float32, device=dev), state
    lib = _lib.load()
    ws_bytes = int(lib.ts_flce_vocab_workspace_size(N, weight_shard.shape[0]))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    state = VocabShardState(hidden, weight_shard, labels, int(vocab_start), ws, ws_bytes, dev,
                            n0, h0)
    stats = torch.empty((N, 4), dtype=torch.float32, device=dev)
    with _lib.on_device(dev):
        check(lib.ts_flce_vocab_fwd(ptr(hidden), state.ldh, ptr(weight_shard), state.ldw,
                                    ptr(labels), N, state.H, state.Vp, state.vocab_start,
                                    ptr(stats), ptr(ws), ws_bytes, _lib.stream_handle(dev)),
              "ts_flce_vocab_fwd")
    return stats[:n0], state


def linear_ce_vocab_phase2(state: VocabShardState, stats_all: Tensor, ignore_index: int = -100,
                           reduction: str = "mean", need_grad_hidden: bool = True,
                           need_grad_weight: bool = True):
    """ts_flce_vocab_bwd from every rank's partials [P, N, 4]: returns (loss, loss_rows,
    lse, grad_hidden_partial [N, H] or None, grad_weight_shard [Vp, H] or None) for an
    upstream gradient of 1; grad_hidden_partial is this rank's term of the sum over ranks.
    ignore_index must be the one phase 1 was given."""
    if reduction not in _REDUCTIONS:
        raise ValueError(f"vocab_parallel_linear_cross_entropy: reduction must be 'mean' or "
                         f"'sum', got {reduction!r}")
    if (stats_all.dim() != 3 or stats_all.shape[1] != state.N0 or stats_all.shape[2] != 4 or
            stats_all.dtype != torch.float32):
        raise ValueError(f"vocab_parallel_linear_cross_entropy: partials must be fp32 "
                         f"[P, {state.N0}, 4], got {stats_all.dtype} {tuple(stats_all.shape)}")
    if state.N == 0:  # no rows: loss 0 (the mean over no valid rows, as the one-GPU kernel)
        dev = state.dev
        gh = (torch.empty((0, state.H0), dtype=torch.bfloat16, device=dev)
              if need_grad_hidden else None)
        gw = (torch.zeros((state.Vp, state.H0), dtype=torch.bfloat16, device=dev)
              if need_grad_weight else None)
        empty = torch.empty((0,), dtype=torch.float32, device=dev)
        return torch.zeros((), dtype=torch.float32, device=dev), empty, empty.clone(), gh, gw
    if state.N != state.N0:  # the padded rows are ignored: their partials take no part
        stats_all = torch.cat([stats_all, stats_all.new_zeros(
            (stats_all.shape[0], state.N - state.N0, 4))], dim=1)
    stats_all = stats_all.contiguous()
    dev = state.dev
    loss = torch.empty((), dtype=torch.float32, device=dev)
    loss_rows = torch.empty((state.N,), dtype=torch.float32, device=dev)
    lse = torch.empty((state.N,), dtype=torch.float32, device=dev)
    gh = (torch.empty((state.N, state.H), dtype=torch.bfloat16, device=dev)
          if need_grad_hidden else None)
    gw = (torch.empty((state.Vp, state.H), dtype=torch.bfloat16, device=dev)
          if need_grad_weight else None)
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_flce_vocab_bwd(ptr(state.hidden), state.ldh, ptr(state.weight), state.ldw,
                                    ptr(state.labels), state.N, state.H, state.Vp,
                                    state.vocab_start, ptr(stats_all), stats_all.shape[0],
                                    int(ignore_index), _REDUCTIONS[reduction], ptr(loss),
                                    ptr(loss_rows), ptr(lse), ptr(gh), ptr(gw), ptr(state.ws),
                                    state.ws_bytes, _lib.stream_handle(dev)),
              "ts_flce_vocab_bwd")
    n0 = state.N0
    gh = _unpad(gh[:n0], state.H0) if gh is not None else None
    return loss, loss_rows[:n0], lse[:n0], gh, _unpad(gw, state.H0)


def _scale_(t: Optional[Tensor], scale: Tensor) -> None:
    if t is not None:
        ops.scale_(t, scale)


class LinearCrossEntropyFunction(torch.autograd.Function):
    """loss = CE(t(hidden @ weight.T), labels), two-pass schedule: the forward keeps
    per-row statistics only, the backward recomputes the logits by vocabulary chunk.
    With keep_logits the forward also keeps the bf16 logits and the first backward
    forms the gradients from them (consuming them). Returns the reduced loss, or the
    per-row losses [N] for reduction "none" (0 on ignore_index rows). Calling
    backward again (retain_graph) recomputes."""

    @staticmethod
    def forward(ctx, hidden: Tensor, weight: Tensor, labels: Tensor, ignore_index: int = -100,
                reduction: str = "mean", logit_softcapping: float = 0.0,
                logit_scaling: float = 0.0, temperature: float = 1.0,
                vocab_chunk: Optional[int] = None, keep_logits: bool = False) -> Tensor:
        shape = hidden.shape
        h2 = hidden.reshape(-1, shape[-1])
        # kept only when a backward can consume them (forward runs without grad mode,
        # so needs_input_grad says whether this call is recorded for one)
        keep = keep_logits and (ctx.needs_input_grad[0] or ctx.needs_input_grad[1])
        out = linear_ce_forward(h2, weight, labels, ignore_index, reduction, logit_softcapping,
                                logit_scaling, temperature, keep_logits=keep)
        loss, rows, lse = out[:3]
        # the kept logits are not a saved tensor: the first backward overwrites them
        ctx.logits = out[3] if keep else None
        ctx.cfg = (ignore_index, reduction, logit_softcapping, logit_scaling, temperature,
                   vocab_chunk)
        ctx.hidden_shape = shape
        ctx.save_for_backward(h2, weight, labels, lse)
        return loss if reduction != "none" else rows

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        h2, weight, labels, lse = ctx.saved_tensors
        ignore_index, reduction, cap, sc, temp, chunk = ctx.cfg
        logits, ctx.logits = ctx.logits, None
        gh, gw = linear_ce_backward(h2, weight, labels, lse, grad_output, ignore_index, reduction,
                                    cap, sc, temp, need_grad_hidden=ctx.needs_input_grad[0],
                                    need_grad_weight=ctx.needs_input_grad[1], vocab_chunk=chunk,
                                    logits=logits)
        gh = gh.view(ctx.hidden_shape) if gh is not None else None
        return gh, gw, None, None, None, None, None, None, None, None


class FusedLinearCrossEntropyFunction(torch.autograd.Function):
    """loss = CE(hidden @ weight.T, labels) with the gradients formed in the forward
    (schedule "fused": mean or sum, no logit transforms)."""

    @staticmethod
    def forward(ctx, hidden: Tensor, weight: Tensor, labels: Tensor, ignore_index: int = -100,
                reduction: str = "mean", chunk_tokens: Optional[int] = None,
                grad_weight_accum: str = "bf16") -> Tensor:
        shape = hidden.shape
        h2 = hidden.reshape(-1, shape[-1])
        loss, _, _, gh, gw = linear_ce_forward_backward(
            h2, weight, labels, ignore_index, reduction,
            need_grad_hidden=ctx.needs_input_grad[0], need_grad_weight=ctx.needs_input_grad[1],
            chunk_tokens=chunk_tokens, grad_weight_accum=grad_weight_accum)
        ctx.hidden_shape = shape
        ctx.save_for_backward(gh, gw)
        return loss

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        # the saved gradients are scaled in place: a second backward would scale them again
        if getattr(ctx, "backward_done", False):
            raise RuntimeError(SECOND_BACKWARD_MSG)
        ctx.backward_done = True
        gh, gw = ctx.saved_tensors
        scale = grad_output.detach().float().reshape(1).contiguous()
        _scale_(gh, scale)
        _scale_(gw, scale)
        gh = gh.view(ctx.hidden_shape) if gh is not None else None
        return gh, gw, None, None, None, None, None


def fused_linear_cross_entropy(hidden: Tensor, weight: Tensor, labels: Tensor,
                               ignore_index: int = -100, reduction: str = "mean",
                               logit_softcapping: float = 0.0,
                               logit_scaling: float = 0.0,
                               temperature: float = 1.0,
                               schedule: str = "auto",
                               vocab_chunk: Optional[int] = None,
                               chunk_tokens: Optional[int] = None,
                               grad_weight_accum: str = "bf16") -> Tensor:
    """Cross-entropy of hidden @ weight.T against labels, without all logits in memory.

    hidden [..., H] and weight [V, H] in bfloat16 (the lm_head layout of
    rl_training.py:156-162); labels [...] int64, ignore_index rows skipped.
    The logits z are transformed as selective_log_softmax does
    (rl_training.py:114-122): t = softcap * tanh(z / softcap) when
    logit_softcapping > 0, then t * logit_scaling when logit_scaling > 0, then
    t / temperature. reduction "mean" (over non-ignored rows), "sum", or "none"
    (per-row losses, shaped like labels).

    schedule: "auto" (default), "fused", "two_pass" or "stored_logits" (module
    docstring). "fused": chunk_tokens rows per token chunk (None: half of
    the tokens, 0: one chunk, i.e. all [N, V] logits), grad_weight_accum "bf16"
    (summed in the bf16 output) or "fp32" (a V x H fp32 workspace); a second
    backward through its graph raises. "two_pass": vocab_chunk columns per
    recomputed chunk (None: about V/8). "stored_logits": the two-pass schedule
    with the bf16 logits kept from the forward to the backward (N * V * 2 bytes).
    """
    if schedule == "auto":
        grads = torch.is_grad_enabled() and (hidden.requires_grad or weight.requires_grad)
        plain = logit_softcapping == 0.0 and logit_scaling == 0.0 and temperature == 1.0
        schedule = "fused" if grads and plain and reduction in _REDUCTIONS else "two_pass"
    if schedule == "fused":
        if reduction not in _REDUCTIONS:
            raise ValueError("fused_linear_cross_entropy: schedule 'fused' takes reduction "
                             "'mean' or 'sum'")
        if logit_softcapping != 0.0 or logit_scaling != 0.0 or temperature != 1.0:
            raise ValueError("fused_linear_cross_entropy: schedule 'fused' takes no logit "
                             "transforms; use schedule 'two_pass'")
        return FusedLinearCrossEntropyFunction.apply(hidden, weight, labels, ignore_index,
                                                     reduction, chunk_tokens, grad_weight_accum)
    if schedule not in ("two_pass", "stored_logits"):
        raise ValueError(f"fused_linear_cross_entropy: unknown schedule {schedule!r}")
    out = LinearCrossEntropyFunction.apply(hidden, weight, labels, ignore_index, reduction,
                                           float(logit_softcapping), float(logit_scaling),
                                           float(temperature), vocab_chunk,
                                           schedule == "stored_logits")
    if reduction == "none":
        out = out.view(labels.shape)
    return out


# A label value no token id takes: every position of the RL drop-ins counts (the
# reference gathers at every position, rl_training.py:131-134).
_NO_IGNORE = -(1 << 62)


def chunked_log_softmax(hidden_states: Tensor, lm_head: Tensor, input_ids: Tensor,
                        num_chunks: int = 4, temperature: float = 1.0,
                        logit_softcapping: float = 0.0, logit_scale: float = 0.0,
                        store_logits: bool = False,
                        out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """Drop-in for chunked_log_softmax (rl_training.py:138-191): log-probabilities
    [B, L] of input_ids under the transformed logits of hidden_states [B, L, H] @
    lm_head[V, H].T, differentiable in hidden_states and lm_head.

    The reference splits the sequence into num_chunks and materialises each
    chunk's [B, chunk, V] logits, which autograd keeps for the backward. Here
    the logits are never stored (the two-pass schedule), so num_chunks is
    accepted for the signature and unused; store_logits=True keeps one bf16
    copy of them ([B * L, V]) so the backward skips their recompute.

    The log-probs come back in the logits' dtype, as the reference's do (its
    selective_log_softmax computes in the dtype of hidden_states @ lm_head.T):
    formed in fp32 and rounded once. out_dtype=torch.float32 keeps them unrounded.
    """
    del num_chunks
    rows = fused_linear_cross_entropy(hidden_states, lm_head, input_ids, ignore_index=_NO_IGNORE,
                                      reduction="none", logit_softcapping=logit_softcapping,
                                      logit_scaling=logit_scale, temperature=temperature,
                                      schedule="stored_logits" if store_logits else "two_pass")
    return (-rows).to(out_dtype or hidden_states.dtype)


def _rl_as_ce_xform(temperature: float, logit_softcapping: float, logit_scale: float):
    """selective_log_softmax's transform t = (c tanh(z / c) or z) * (s or 1) / T
    (rl_training.py:114-122) as the CE kernels' scale-then-softcap form
    t = c' tanh(s' z / c') (or s' z): with m = (s or 1) / T, s' = m and c' = c m give
    c m tanh(m z / (c m)) = c m tanh(z / c). Returns (logit_scale, softcap) for the
    CE kernels, 0 meaning off."""
    if not temperature > 0 or not math.isfinite(temperature):
        raise ValueError(f"selective_log_softmax: temperature must be > 0, got {temperature}")
    if logit_softcapping < 0 or logit_scale < 0:
        raise ValueError("selective_log_softmax: logit_softcapping and logit_scale must be >= 0")
    m = (logit_scale if logit_scale > 0 else 1.0) / temperature
    return (m if m != 1.0 else 0.0), (logit_softcapping * m if logit_softcapping > 0 else 0.0)


class SelectiveLogSoftmaxFunction(torch.autograd.Function):
    """log_softmax(t(logits))[input_ids] over explicit logits [..., V] on the CE kernels
    (ts_ce_fwd, ts_ce_bwd): forward returns the log-probs shaped like input_ids; the
    backward writes the gradient of the logits into a new tensor."""

    @staticmethod
    def forward(ctx, logits: Tensor, input_ids: Tensor, temperature: float,
                logit_softcapping: float, logit_scale: float,
                out_dtype: Optional[torch.dtype]) -> Tensor:
        if logits.shape[:-1] != input_ids.shape:
            raise ValueError(f"selective_log_softmax: logits {tuple(logits.shape)} and input_ids "
                             f"{tuple(input_ids.shape)} do not match")
        scale, cap = _rl_as_ce_xform(temperature, logit_softcapping, logit_scale)
        l2d, ld = ops.as_rows(logits)
        ids = input_ids.reshape(-1)
        rows, lse = ops.ce_forward(l2d, ld, ids, _NO_IGNORE, scale, cap)
        ctx.save_for_backward(l2d, ids, lse)
        ctx.cfg = (ld, scale, cap, logits.shape)
        return (-rows).to(out_dtype or logits.dtype).view(input_ids.shape)

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        l2d, ids, lse = ctx.saved_tensors
        ld, scale, cap, shape = ctx.cfg
        grad = torch.empty((l2d.shape[0], l2d.shape[1]), dtype=l2d.dtype, device=l2d.device)
        # d(log-prob)/d(row loss) = -1
        dl = -grad_out.detach().float().reshape(-1)
        ops.ce_backward(l2d, ld, ids, lse, dl, grad, grad.shape[1], 1.0, _NO_IGNORE, scale, cap)
        return grad.view(shape), None, None, None, None, None


def selective_log_softmax(logits: Tensor, input_ids: Tensor, temperature: float = 1.0,
                          logit_softcapping: float = 0.0, logit_scale: float = 0.0,
                          out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """Drop-in for selective_log_softmax (rl_training.py:95-135): the log-probability
    of input_ids [...] under logits [..., V] after softcapping, then scaling, then
    temperature, without a [..., V] log-softmax in memory; differentiable in logits.
    Returns the logits' dtype as the reference does (formed in fp32, rounded once;
    out_dtype=torch.float32 keeps them unrounded). temperature must be > 0."""
    return SelectiveLogSoftmaxFunction.apply(logits, input_ids, float(temperature),
                                             float(logit_softcapping), float(logit_scale),
                                             out_dtype)
