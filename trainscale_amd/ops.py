"""Tensor-level entry points over the C ABI.

These functions take torch tensors that already live on a ROCm GPU, derive
pointers, sizes and strides, allocate outputs and workspaces with torch's
caching allocator, and launch on torch's current stream. The autograd
wrappers with the reference's signatures (``trainscale_amd.kernels``,
``trainscale_amd.loss``) are built on them.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib
from ._lib import check, ptr

# round modes of ts_rmsnorm_fwd
ROUND_ONCE = 0
ROUND_TWICE = 1


def as_rows(t: Tensor) -> Tuple[Tensor, int]:
    """[..., C] -> (2-D view or copy with unit column stride, row stride)."""
    c = t.shape[-1]
    t2 = t.reshape(-1, c)
    if c > 1 and t2.stride(1) != 1:
        t2 = t2.contiguous()
    ld = t2.stride(0) if t2.shape[0] > 1 else c
    if ld < c:  # overlapping rows (e.g. an expanded tensor)
        t2 = t2.contiguous()
        ld = c
    return t2, ld


def _norm_stride(t: Tensor, dim: int) -> int:
    """Stride of `dim`, or 0 when the dimension has a single element."""
    return 0 if t.shape[dim] == 1 else t.stride(dim)


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def rmsnorm_forward(x2d: Tensor, ldx: int, weight: Optional[Tensor], eps: float,
                    round_mode: int = ROUND_ONCE) -> Tuple[Tensor, Tensor]:
    """y = x * rstd * w over the rows of x2d; returns (y [rows, cols] contiguous, rstd fp32)."""
    dev = _lib.require_gpu("rmsnorm_forward", x2d, weight)
    rows, cols = x2d.shape
    y = torch.empty((rows, cols), dtype=x2d.dtype, device=dev)
    rstd = torch.empty((rows,), dtype=torch.float32, device=dev)
    if rows == 0:
        return y, rstd
    if weight is not None:
        if weight.dim() != 1 or weight.shape[0] != cols:
            raise ValueError(f"rmsnorm: weight shape {tuple(weight.shape)} != ({cols},)")
        weight = weight.contiguous()
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_rmsnorm_fwd(
            ptr(x2d), ldx, _lib.dtype_code(x2d, "rmsnorm"),
            ptr(weight), _lib.dtype_code(weight, "rmsnorm weight") if weight is not None else 0,
            ptr(y), cols, ptr(rstd), rows, cols, float(eps), round_mode,
            _lib.stream_handle(dev)), "ts_rmsnorm_fwd")
    return y, rstd


def add_rmsnorm_forward(x2d: Tensor, ldx: int, r2d: Tensor, ldr: int, weight: Optional[Tensor],
                        eps: float, round_mode: int = ROUND_TWICE, store_h: bool = True
                        ) -> Tuple[Tensor, Optional[Tensor], Tensor]:
    """h = x + r, y = h * rstd * w over the rows; returns (y, h rounded to the data dtype
    or None, rstd fp32), y and h contiguous [rows, cols]."""
    dev = _lib.require_gpu("add_rmsnorm_forward", x2d, r2d, weight)
    rows, cols = x2d.shape
    if r2d.shape != x2d.shape:
        raise ValueError(f"add_rmsnorm: residual {tuple(r2d.shape)} != x {tuple(x2d.shape)}")
    if r2d.dtype != x2d.dtype:
        raise TypeError(f"add_rmsnorm: residual dtype {r2d.dtype} != x dtype {x2d.dtype}")
    y = torch.empty((rows, cols), dtype=x2d.dtype, device=dev)
    h = torch.empty((rows, cols), dtype=x2d.dtype, device=dev) if store_h else None
    rstd = torch.empty((rows,), dtype=torch.float32, device=dev)
    if rows == 0:
        return y, h, rstd
    if weight is not None:
        if weight.dim() != 1 or weight.shape[0] != cols:
            raise ValueError(f"add_rmsnorm: weight shape {tuple(weight.shape)} != ({cols},)")
        weight = weight.contiguous()
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_add_rmsnorm_fwd(
            ptr(x2d), ldx, ptr(r2d), ldr, _lib.dtype_code(x2d, "add_rmsnorm"),
            ptr(weight), _lib.dtype_code(weight, "add_rmsnorm weight") if weight is not None else 0,
            ptr(y), cols, ptr(h), cols, ptr(rstd), rows, cols, float(eps), round_mode,
            _lib.stream_handle(dev)), "ts_add_rmsnorm_fwd")
    return y, h, rstd


def rmsnorm_backward(dy2d: Tensor, lddy: int, x2d: Tensor, ldx: int, weight: Optional[Tensor],
                     rstd: Tensor, need_dw: bool) -> Tuple[Tensor, Optional[Tensor]]:
    """Returns (dx [rows, cols] contiguous, dw in the weight dtype or None)."""
    dev = _lib.require_gpu("rmsnorm_backward", dy2d, x2d, weight, rstd)
    rows, cols = x2d.shape
    if dy2d.dtype != x2d.dtype:
        dy2d = dy2d.to(x2d.dtype)
        dy2d, lddy = as_rows(dy2d)
    dx = torch.empty((rows, cols), dtype=x2d.dtype, device=dev)
    dw = None
    if need_dw and weight is not None:
        dw = torch.empty_like(weight, memory_format=torch.contiguous_format)
        weight = weight.contiguous()
    lib = _lib.load()
    ws = None
    ws_bytes = 0
    if dw is not None and rows > 0:
        ws_bytes = int(lib.ts_rmsnorm_bwd_workspace_size(rows, cols))
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    w_code = _lib.dtype_code(weight, "rmsnorm weight") if weight is not None else 0
    with _lib.on_device(dev):
        check(lib.ts_rmsnorm_bwd(
            ptr(dy2d), lddy, ptr(x2d), ldx, _lib.dtype_code(x2d, "rmsnorm"),
            ptr(weight), w_code, ptr(rstd.contiguous()), ptr(dx), cols, ptr(dw),
            ptr(ws), ws_bytes, rows, cols, _lib.stream_handle(dev)), "ts_rmsnorm_bwd")
    return dx, dw


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def _bshd(t: Tensor, what: str) -> Tensor:
    if t.dim() != 4:
        raise ValueError(f"{what}: expected [batch, seq, heads, head_dim], got {tuple(t.shape)}")
    if t.shape[3] > 1 and t.stride(3) != 1:
        t = t.contiguous()
    return t


def rope_apply(q_in: Optional[Tensor], q_out: Optional[Tensor],
               k_in: Optional[Tensor], k_out: Optional[Tensor], *,
               cos: Optional[Tensor] = None, sin: Optional[Tensor] = None,
               inv_freq: Optional[Tensor] = None, pos_div: float = 1.0,
               angle_scale: float = 1.0,
               position_ids: Optional[Tensor] = None, position_offset: int = 0,
               interleaved: bool = False, backward: bool = False) -> None:
    """Rotates q_in -> q_out and k_in -> k_out (either pair may be None; in == out is in place).

    All tensors are [B, S, H, D] with a unit last stride. Angles come from the
    cos/sin tables ([rows, D/2], gathered at the position) or, when both are
    None, from `inv_freq` (D/2 fp32 values, CPU) evaluated on the GPU.
    """
    ref = q_in if q_in is not None else k_in
    if ref is None:
        return
    dev = _lib.require_gpu("rope", q_in, q_out, k_in, k_out, cos, sin, position_ids)
    B, S, _, D = ref.shape
    for name, t in (("q_in", q_in), ("q_out", q_out), ("k_in", k_in), ("k_out", k_out)):
        if t is not None:
            if t.dim() != 4 or t.shape[0] != B or t.shape[1] != S or t.shape[3] != D:
                raise ValueError(f"rope: {name} shape {tuple(t.shape)} does not match "
                                 f"[{B}, {S}, H, {D}]")
            if t.numel() > 0 and t.shape[3] > 1 and t.stride(3) != 1:
                raise ValueError(f"rope: {name} needs a contiguous head dimension")
            if t.dtype != ref.dtype:
                raise TypeError(f"rope: {name} dtype {t.dtype} != {ref.dtype}")
    if q_in is not None and q_out.shape != q_in.shape:
        raise ValueError("rope: q_out shape differs from q_in")
    if k_in is not None and k_out.shape != k_in.shape:
        raise ValueError("rope: k_out shape differs from k_in")
    Hq = q_in.shape[2] if q_in is not None else 0
    Hk = k_in.shape[2] if k_in is not None else 0

    tab_code, tab_ld, tab_rows = 0, 0, 0
    inv_ptr = None
    inv_host = None
    if cos is not None or sin is not None:
        if cos is None or sin is None:
            raise ValueError("rope: cos and sin must both be given")
        cos = cos.reshape(-1, cos.shape[-1]) if cos.dim() != 2 else cos
        sin = sin.reshape(-1, sin.shape[-1]) if sin.dim() != 2 else sin
        if cos.shape != sin.shape:
            raise ValueError(f"rope: cos {tuple(cos.shape)} and sin {tuple(sin.shape)} differ")
        if cos.shape[1] < D // 2:
            raise ValueError(f"rope: tables have {cos.shape[1]} columns, need {D // 2}")
        if cos.dtype != sin.dtype:
            sin = sin.to(cos.dtype)
        if cos.stride(1) != 1 or sin.stride(1) != 1 or cos.stride(0) != sin.stride(0):
            cos, sin = cos.contiguous(), sin.contiguous()
        tab_code = _lib.dtype_code(cos, "rope table")
        tab_ld = cos.stride(0) if cos.shape[0] > 1 else cos.shape[1]
        tab_rows = cos.shape[0]
    else:
        if inv_freq is None:
            raise ValueError("rope: need cos/sin tables or inv_freq")
        inv_host = inv_freq.detach().to("cpu", torch.float32).contiguous()
        if inv_host.numel() != D // 2:
            raise ValueError(f"rope: inv_freq has {inv_host.numel()} values, need {D // 2}")
        inv_ptr = ptr(inv_host)

    pos_sb = pos_ss = 0
    if position_ids is not None:
        if position_ids.dtype != torch.int64:
            position_ids = position_ids.to(torch.int64)
        if position_ids.dim() == 1:
            if position_ids.shape[0] != S:
                raise ValueError(f"rope: position_ids has {position_ids.shape[0]} entries, need {S}")
            pos_ss = _norm_stride(position_ids, 0)
        elif position_ids.dim() == 2:
            if position_ids.shape[1] != S or position_ids.shape[0] not in (1, B):
                raise ValueError(f"rope: position_ids shape {tuple(position_ids.shape)} does not "
                                 f"match [{B}, {S}]")
            pos_sb = _norm_stride(position_ids, 0)
            pos_ss = _norm_stride(position_ids, 1)
        else:
            raise ValueError("rope: position_ids must be [S] or [B, S]")

    def strides(t):
        if t is None:
            return (0, 0, 0)
        return (_norm_stride(t, 0), _norm_stride(t, 1), _norm_stride(t, 2))

    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_rope_apply(
            ptr(q_in), ptr(q_out), *strides(q_in), *strides(q_out), Hq,
            ptr(k_in), ptr(k_out), *strides(k_in), *strides(k_out), Hk,
            _lib.dtype_code(ref, "rope"), B, S, D,
            ptr(cos), ptr(sin), tab_code, tab_ld, tab_rows,
            inv_ptr, float(pos_div), float(angle_scale),
            ptr(position_ids), pos_sb, pos_ss, int(position_offset),
            int(bool(interleaved)), int(bool(backward)), _lib.stream_handle(dev)),
            "ts_rope_apply")
    # keep host/device temporaries alive until the launch is enqueued
    del inv_host


# ---------------------------------------------------------------------------
# Cross-entropy
# ---------------------------------------------------------------------------

def _labels(labels: Tensor, n: int) -> Tensor:
    labels = labels.reshape(-1)
    if labels.shape[0] != n:
        raise ValueError(f"cross_entropy: {labels.shape[0]} labels for {n} rows")
    if labels.dtype != torch.int64:
        labels = labels.to(torch.int64)
    return labels.contiguous()


def ce_forward(logits2d: Tensor, ld: int, labels: Tensor, ignore_index: int = -100,
               logit_scale: float = 0.0, softcap: float = 0.0,
               label_smoothing: float = 0.0) -> Tuple[Tensor, Tensor]:
    """Per-row (loss, lse), both fp32 [N]. Ignored rows: loss 0, lse 0."""
    dev = _lib.require_gpu("cross_entropy", logits2d, labels)
    n, v = logits2d.shape
    labels = _labels(labels, n)
    loss = torch.empty((n,), dtype=torch.float32, device=dev)
    lse = torch.empty((n,), dtype=torch.float32, device=dev)
    if n == 0:
        return loss, lse
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_ce_fwd(ptr(logits2d), ld, _lib.dtype_code(logits2d, "cross_entropy"),
                            ptr(labels), n, v, int(ignore_index), float(logit_scale),
                            float(softcap), float(label_smoothing), ptr(loss), ptr(lse),
                            _lib.stream_handle(dev)), "ts_ce_fwd")
    return loss, lse


def ce_backward(logits2d: Tensor, ld: int, labels: Tensor, lse: Tensor, dloss: Tensor,
                grad: Tensor, ld_grad: int, dloss_scale: float = 1.0, ignore_index: int = -100,
                logit_scale: float = 0.0, softcap: float = 0.0,
                label_smoothing: float = 0.0) -> Tensor:
    """Writes dL/dlogits into `grad` (may be logits2d itself) and returns it.

    dloss is fp32 with one value per row, or a single value (0-d / one element)
    broadcast to every row.
    """
    dev = _lib.require_gpu("cross_entropy_backward", logits2d, labels, lse, dloss, grad)
    n, v = logits2d.shape
    labels = _labels(labels, n)
    if dloss.dtype != torch.float32:
        dloss = dloss.float()
    if dloss.numel() == 1:
        dloss = dloss.reshape(1)
        dstride = 0
    else:
        dloss = dloss.reshape(-1)
        if dloss.shape[0] != n:
            raise ValueError(f"cross_entropy_backward: {dloss.shape[0]} upstream grads for {n} rows")
        dstride = dloss.stride(0)
    if n == 0:
        return grad
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_ce_bwd(ptr(logits2d), ld, _lib.dtype_code(logits2d, "cross_entropy"),
                            ptr(labels), ptr(lse.contiguous()), ptr(dloss), dstride,
                            float(dloss_scale), ptr(grad), ld_grad,
                            _lib.dtype_code(grad, "cross_entropy grad"), n, v,
                            int(ignore_index), float(logit_scale), float(softcap),
                            float(label_smoothing), _lib.stream_handle(dev)), "ts_ce_bwd")
    return grad


def ce_forward_backward(logits2d: Tensor, ld: int, labels: Tensor, dloss: Tensor,
                        dloss_scale: float = 1.0, ignore_index: int = -100,
                        logit_scale: float = 0.0, softcap: float = 0.0,
                        label_smoothing: float = 0.0,
                        grad_dtype: Optional[torch.dtype] = None,
                        grad: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Per-row (loss, lse) and dL/dlogits for the upstream gradient `dloss` (fp32,
    one value per row or a single value for every row) in one pass over the logits.
    Returns (loss [N] fp32, lse [N] fp32, grad [N, V] in grad_dtype or the logits dtype);
    `grad`, if given, is a contiguous [N, V] tensor to write into."""
    dev = _lib.require_gpu("cross_entropy", logits2d, labels, dloss)
    n, v = logits2d.shape
    labels = _labels(labels, n)
    if dloss.dtype != torch.float32:
        dloss = dloss.float()
    if dloss.numel() == 1:
        dloss = dloss.reshape(1)
        dstride = 0
    else:
        dloss = dloss.reshape(-1)
        if dloss.shape[0] != n:
            raise ValueError(f"cross_entropy: {dloss.shape[0]} upstream grads for {n} rows")
        dstride = dloss.stride(0)
    loss = torch.empty((n,), dtype=torch.float32, device=dev)
    lse = torch.empty((n,), dtype=torch.float32, device=dev)
    if grad is None:
        grad = torch.empty((n, v), dtype=grad_dtype or logits2d.dtype, device=dev)
    elif grad.shape != (n, v) or not grad.is_contiguous():
        raise ValueError("cross_entropy: grad must be a contiguous [N, V] tensor")
    if n == 0:
        return loss, lse, grad
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_ce_fwd_bwd(ptr(logits2d), ld, _lib.dtype_code(logits2d, "cross_entropy"),
                                ptr(labels), n, v, int(ignore_index), float(logit_scale),
                                float(softcap), float(label_smoothing), ptr(dloss), dstride,
                                float(dloss_scale), ptr(loss), ptr(lse), ptr(grad), v,
                                _lib.dtype_code(grad, "cross_entropy grad"),
                                _lib.stream_handle(dev)), "ts_ce_fwd_bwd")
    return loss, lse, grad


# ---------------------------------------------------------------------------
# Vocabulary-parallel cross entropy (the kernels of one rank)
# ---------------------------------------------------------------------------

def ce_vocab_shard_stats(logits2d: Tensor, ld: int, targets: Tensor, vocab_start: int) -> Tensor:
    """Per-row partials [N, 4] fp32 of this rank's shard: (lse over the shard,
    target logit if the target is in the shard else 0, sum of the shard's
    logits, 0). The tensor an all-gather exchanges between the ranks."""
    dev = _lib.require_gpu("vocab_parallel_cross_entropy", logits2d, targets)
    n, vp = logits2d.shape
    targets = _labels(targets, n)
    stats = torch.empty((n, 4), dtype=torch.float32, device=dev)
    if n == 0:
        return stats
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_ce_vocab_shard_stats(ptr(logits2d), ld,
                                          _lib.dtype_code(logits2d, "vocab_parallel_cross_entropy"),
                                          ptr(targets), n, vp, int(vocab_start), ptr(stats),
                                          _lib.stream_handle(dev)), "ts_ce_vocab_shard_stats")
    return stats


def ce_vocab_merge(stats_all: Tensor, self_index: int, vp: int,
                   label_smoothing: float = 0.0) -> Tuple[Tensor, Tensor]:
    """(lse [N], loss [N]) of rank `self_index` from every rank's partials [P, N, 4]."""
    dev = _lib.require_gpu("vocab_parallel_cross_entropy", stats_all)
    if stats_all.dim() != 3 or stats_all.shape[2] != 4 or stats_all.dtype != torch.float32:
        raise ValueError(f"vocab_parallel_cross_entropy: partials must be fp32 [P, N, 4], "
                         f"got {stats_all.dtype} {tuple(stats_all.shape)}")
    stats_all = stats_all.contiguous()
    p, n = stats_all.shape[0], stats_all.shape[1]
    lse = torch.empty((n,), dtype=torch.float32, device=dev)
    loss = torch.empty((n,), dtype=torch.float32, device=dev)
    if n == 0:
        return lse, loss
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_ce_vocab_merge(ptr(stats_all), p, int(self_index), n, int(vp),
                                    float(label_smoothing), ptr(lse), ptr(loss),
                                    _lib.stream_handle(dev)), "ts_ce_vocab_merge")
    return lse, loss


def ce_vocab_shard_backward(logits2d: Tensor, ld: int, targets: Tensor, lse: Tensor,
                            grad_output: Tensor, dloss_scale: float, vocab_start: int,
                            label_smoothing: float = 0.0,
                            grad_dtype: Optional[torch.dtype] = None) -> Tensor:
    """Gradient [N, Vp] of this rank's shard (a new tensor, the logits dtype or fp32)."""
    dev = _lib.require_gpu("vocab_parallel_cross_entropy_backward", logits2d, targets, lse,
                           grad_output)
    n, vp = logits2d.shape
    targets = _labels(targets, n)
    grad = torch.empty((n, vp), dtype=grad_dtype or logits2d.dtype, device=dev)
    if n == 0:
        return grad
    go = grad_output.detach().reshape(-1)[:1].float().contiguous()
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_ce_vocab_shard_bwd(ptr(logits2d), ld,
                                        _lib.dtype_code(logits2d, "vocab_parallel_cross_entropy"),
                                        ptr(targets), ptr(lse.contiguous()), ptr(go),
                                        float(dloss_scale), n, vp, int(vocab_start),
                                        float(label_smoothing), ptr(grad), vp,
                                        _lib.dtype_code(grad, "vocab_parallel grad"),
                                        _lib.stream_handle(dev)), "ts_ce_vocab_shard_bwd")
    return grad


def scale_(t: Tensor, scale: Tensor) -> Tensor:
    """t *= scale in place (scale: a one-element fp32 device tensor); a no-op on the
    device when scale == 1, without synchronising."""
    if t.numel() == 0:
        return t
    dev = _lib.require_gpu("scale_", t, scale)
    if not t.is_contiguous():
        raise ValueError("scale_: tensor must be contiguous")
    scale = scale.detach().to(torch.float32).reshape(1).contiguous()
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_scale_inplace(ptr(t), t.numel(), _lib.dtype_code(t, "scale_"), ptr(scale),
                                   _lib.stream_handle(dev)), "ts_scale_inplace")
    return t


def rescale_(t: Tensor, now: Tensor, used: Tensor, hint_out: Optional[Tensor] = None) -> Tensor:
    """t *= now / used in place (one-element fp32 device tensors); a no-op on the device
    when the ratio is exactly 1. hint_out (one-element fp32, distinct from now and used)
    receives now when finite and non-zero, else 1."""
    dev = _lib.require_gpu("rescale_", t, now, used)
    if not t.is_contiguous():
        raise ValueError("rescale_: tensor must be contiguous")
    now = now.detach().to(torch.float32).reshape(1).contiguous()
    used = used.detach().to(torch.float32).reshape(1).contiguous()
    if hint_out is not None and (hint_out.dtype != torch.float32 or hint_out.numel() != 1
                                 or hint_out.device != t.device):
        raise ValueError("rescale_: hint_out must be a one-element fp32 tensor on the device")
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_rescale_inplace(ptr(t), t.numel(), _lib.dtype_code(t, "rescale_"),
                                     ptr(now), ptr(used), ptr(hint_out),
                                     _lib.stream_handle(dev)), "ts_rescale_inplace")
    return t


def _flat(t: Tensor, name: str) -> Tensor:
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    return t


def swiglu_forward(gate: Tensor, up: Tensor) -> Tensor:
    """out = round(round(silu(gate)) * up) elementwise; a new tensor shaped like gate."""
    dev = _lib.require_gpu("swiglu_forward", gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError(f"swiglu: gate {tuple(gate.shape)} {gate.dtype} and up "
                         f"{tuple(up.shape)} {up.dtype} must match")
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_swiglu_fwd(ptr(gate), ptr(up), ptr(out), gate.numel(),
                                _lib.dtype_code(gate, "swiglu"), _lib.stream_handle(dev)),
              "ts_swiglu_fwd")
    return out


def swiglu_backward(dout: Tensor, gate: Tensor, up: Tensor) -> Tuple[Tensor, Tensor]:
    """(dgate, dup) of out = silu(gate) * up for the upstream gradient dout."""
    dev = _lib.require_gpu("swiglu_backward", dout, gate, up)
    gate, up = _flat(gate, "swiglu"), _flat(up, "swiglu")
    dout = dout.to(gate.dtype).contiguous()
    if dout.shape != gate.shape:
        raise ValueError(f"swiglu: dout {tuple(dout.shape)} != gate {tuple(gate.shape)}")
    dgate, dup = torch.empty_like(gate), torch.empty_like(up)
    lib = _lib.load()
    with _lib.on_device(dev):
        check(lib.ts_swiglu_bwd(ptr(dout), ptr(gate), ptr(up), ptr(dgate), ptr(dup),
                                gate.numel(), _lib.dtype_code(gate, "swiglu"),
                                _lib.stream_handle(dev)), "ts_swiglu_bwd")
    return dgate, dup
