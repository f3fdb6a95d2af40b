"""Oracle restatements (torch CPU, fp32 arithmetic). TEST INFRASTRUCTURE ONLY.

Each function cites the reference lines it restates (paths relative to
data_pipeline/trainer/ of generalaimodels/TrainScale). Inputs may be bf16/fp16
CPU tensors; arithmetic is fp32 and the result is rounded once to the output
dtype, as the reference's GPU kernels do (they upcast every load to fp32).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

__all__ = [
    "rms_norm_fwd",
    "add_rms_norm_fwd",
    "rms_norm_bwd",
    "rope_inv_freq",
    "rope_tables",
    "rope_apply",
    "rope_positions",
    "ce_fwd",
    "ce_bwd",
    "linear_ce",
    "rl_logit_xform",
    "selective_log_softmax",
    "vocab_parallel_ce",
    "swiglu_fwd",
    "swiglu_bwd",
]


def _cpu(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.detach().cpu()


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def rms_norm_fwd(x: Tensor, w: Optional[Tensor], eps: float = 1e-6,
                 round_twice: bool = False) -> Tuple[Tensor, Tensor]:
    """y = x * rstd * w, rstd = rsqrt(mean(x^2) + eps), fp32, rounded once to x.dtype.

    Restates _rms_layernorm_forward_kernel (kernels/triton_kernels.py:501-514;
    eager form :612-616). With round_twice and a weight of x's 16-bit dtype it
    restates layernorm_kernels.py:189-194 instead: y = round(round(x*rstd) * w).
    Returns (y [..., C] in x.dtype, rstd fp32 [rows]).
    """
    x = _cpu(x)
    w = _cpu(w)
    c = x.shape[-1]
    x32 = x.reshape(-1, c).float()
    mean_sq = (x32 * x32).sum(-1) / c
    rstd = 1.0 / torch.sqrt(mean_sq + eps)
    xn = x32 * rstd[:, None]
    if w is not None:
        if round_twice and w.dtype == x.dtype and x.dtype != torch.float32:
            y = xn.to(x.dtype).float() * w.float()
        else:
            y = xn * w.float()
    else:
        y = xn
    return y.to(x.dtype).reshape(x.shape), rstd


def add_rms_norm_fwd(x: Tensor, r: Tensor, w: Optional[Tensor], eps: float = 1e-6,
                     round_twice: bool = True) -> Tuple[Tensor, Tensor, Tensor]:
    """Residual add + RMSNorm: h = x + r in fp32, rstd from the unrounded h,
    y = h * rstd * w (round_twice: y = round(round(h*rstd) * w) for a 16-bit w of
    x's dtype), and h rounded once to x.dtype.

    Restates _fused_add_rms_layernorm_kernel (kernels/layernorm_kernels.py:528-552)
    as FusedAddRMSLayerNormFunction.forward launches it (:957-1009). Returns
    (y, h, rstd fp32 [rows]); the backward is rms_norm_bwd on the rounded h
    (:1011-1045).
    """
    x, r, w = _cpu(x), _cpu(r), _cpu(w)
    c = x.shape[-1]
    h32 = x.reshape(-1, c).float() + r.reshape(-1, c).float()
    rstd = 1.0 / torch.sqrt((h32 * h32).sum(-1) / c + eps)
    hn = h32 * rstd[:, None]
    if w is not None:
        if round_twice and w.dtype == x.dtype and x.dtype != torch.float32:
            y = hn.to(x.dtype).float() * w.float()
        else:
            y = hn * w.float()
    else:
        y = hn
    return y.to(x.dtype).reshape(x.shape), h32.to(x.dtype).reshape(x.shape), rstd


def rms_norm_bwd(dy: Tensor, x: Tensor, w: Optional[Tensor],
                 rstd: Tensor) -> Tuple[Tensor, Optional[Tensor]]:
    """dx = rstd*(dy*w - xhat*mean(dy*w*xhat)), dw = sum_rows(dy*xhat), fp32.

    Restates _rms_layernorm_backward_kernel and _rms_layernorm_backward_dw_kernel
    (kernels/triton_kernels.py:557-562, :596-597; eager form
    kernels/layernorm_kernels.py:777-781, :804-805). dx in x.dtype, dw in w.dtype.
    """
    dy, x, w, rstd = _cpu(dy), _cpu(x), _cpu(w), _cpu(rstd)
    c = x.shape[-1]
    x32 = x.reshape(-1, c).float()
    dy32 = dy.reshape(-1, c).float()
    r = rstd.float()[:, None]
    xhat = x32 * r
    dyw = dy32 * (w.float() if w is not None else 1.0)
    c1 = (dyw * xhat).sum(-1, keepdim=True) / c
    dx = r * (dyw - xhat * c1)
    dw = None
    if w is not None:
        dw = (dy32 * xhat).sum(0).to(w.dtype)
    return dx.to(x.dtype).reshape(x.shape), dw


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def rope_inv_freq(dim: int, theta: float) -> Tensor:
    """inv_freq_i = 1/theta**(2i/dim) in fp32 (kernels/rope_kernels.py:203-207)."""
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))


def rope_tables(dim: int, n_pos: int, theta: float, pos_div: float = 1.0,
                dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor]:
    """cos/sin [n_pos, dim/2]: fp32 angle outer(arange/pos_div, inv_freq).

    Restates compute_rope_frequencies / precompute_freqs_cis
    (kernels/rope_kernels.py:172-195; kernels/triton_kernels.py:1029-1032).
    """
    t = torch.arange(n_pos, dtype=torch.float32) / pos_div
    ang = torch.outer(t, rope_inv_freq(dim, theta))
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


def rope_positions(B: int, S: int, position_ids: Optional[Tensor] = None,
                   position_offset: int = 0) -> Tensor:
    """int64 [B, S] positions: position_ids broadcast over the batch, else s + offset."""
    if position_ids is None:
        return (torch.arange(S, dtype=torch.int64) + position_offset).expand(B, S)
    p = _cpu(position_ids).to(torch.int64)
    if p.dim() == 1:
        p = p[None, :]
    return p.expand(B, S)


def rope_apply(x: Tensor, cos: Tensor, sin: Tensor, positions: Tensor,
               interleaved: bool = False, backward: bool = False) -> Tensor:
    """Rotation of x [B,S,H,D] by the table rows at positions [B,S], fp32, rounded once.

    NeoX: o1 = x1*c - x2*s, o2 = x2*c + x1*s on halves [0, D/2) / [D/2, D);
    interleaved: the same on (x[2i], x[2i+1]). Backward negates sin.
    Restates _rope_forward_kernel / _rope_backward_kernel
    (kernels/triton_kernels.py:764-806, :848-890) and the eager form with the
    BSHD broadcast of triton_kernels.py:908-925 and the position_ids gather of
    kernels/rope_kernels.py:965-993 (cos[position_ids] -> [B, S, 1, D/2]).
    """
    x, cos, sin, positions = _cpu(x), _cpu(cos), _cpu(sin), _cpu(positions)
    D = x.shape[-1]
    h = D // 2
    c = cos.float()[positions][:, :, None, :h]
    s = sin.float()[positions][:, :, None, :h]
    if backward:
        s = -s
    x32 = x.float()
    if interleaved:
        x1, x2 = x32[..., 0::2], x32[..., 1::2]
    else:
        x1, x2 = x32[..., :h], x32[..., h:]
    o1 = x1 * c - x2 * s
    o2 = x2 * c + x1 * s
    if interleaved:
        out = torch.stack([o1, o2], dim=-1).flatten(-2)
    else:
        out = torch.cat([o1, o2], dim=-1)
    return out.to(x.dtype)


# ---------------------------------------------------------------------------
# Cross-entropy
# ---------------------------------------------------------------------------

def _xform(x32: Tensor, logit_scale: float, softcap: float) -> Tensor:
    # scale then softcap, kernels/triton_kernels.py:331-334
    if logit_scale != 0.0:
        x32 = logit_scale * x32
    if softcap != 0.0:
        x32 = softcap * torch.tanh(x32 / softcap)
    return x32


def ce_fwd(logits: Tensor, labels: Tensor, ignore_index: int = -100,
           logit_scale: float = 0.0, softcap: float = 0.0,
           label_smoothing: float = 0.0) -> Tuple[Tensor, Tensor]:
    """Per-row (loss, lse) in fp32; loss 0 on ignore_index rows.

    loss = (1-a)*(lse - z[label]) + a*(lse - mean(z)), z the transformed logits.
    Restates Fast_CrossEntropyLoss's eager path (kernels/triton_kernels.py:
    328-337: F.cross_entropy(logits.float(), reduction='none') after scaling and
    softcapping) and ChunkedCrossEntropyLoss's training path
    (loss/sota_losses.py:695-744, incl. label smoothing :726-731).
    """
    logits, labels = _cpu(logits), _cpu(labels).reshape(-1).to(torch.int64)
    z = _xform(logits.reshape(-1, logits.shape[-1]).float(), logit_scale, softcap)
    lse = torch.logsumexp(z, dim=-1)
    valid = labels != ignore_index
    tgt = torch.gather(z, 1, labels.clamp(min=0)[:, None]).squeeze(1)
    loss = lse - tgt
    if label_smoothing > 0:
        loss = (1 - label_smoothing) * loss + label_smoothing * (lse - z.mean(dim=-1))
    loss = torch.where(valid, loss, torch.zeros_like(loss))
    return loss, lse


def ce_bwd(logits: Tensor, labels: Tensor, dloss: Tensor, ignore_index: int = -100,
           logit_scale: float = 0.0, softcap: float = 0.0, label_smoothing: float = 0.0,
           out_dtype: Optional[torch.dtype] = None) -> Tensor:
    """dL/dlogits = dloss * dz/dx * (softmax(z) - (1-a)*onehot - a/V), 0 on ignored rows.

    Restates _cross_entropy_backward_kernel (kernels/triton_kernels.py:271-306)
    and _fused_cross_entropy_bwd_kernel (loss/sota_losses.py:262-289).
    dloss: fp32 [N] or a scalar. Returns the gradient in out_dtype (default logits.dtype).
    """
    logits, labels, dloss = _cpu(logits), _cpu(labels).reshape(-1).to(torch.int64), _cpu(dloss)
    n, v = logits.shape[0], logits.shape[-1]
    x32 = logits.reshape(n, v).float()
    z = _xform(x32, logit_scale, softcap)
    p = torch.softmax(z, dim=-1)
    onehot = torch.zeros_like(p)
    valid = labels != ignore_index
    onehot[torch.arange(n)[valid], labels[valid]] = 1.0
    g = (1 - label_smoothing) * (p - onehot) + label_smoothing * (p - 1.0 / v)
    if softcap != 0.0:
        t = torch.tanh((logit_scale * x32 if logit_scale != 0.0 else x32) / softcap)
        g = g * (1 - t * t)
    if logit_scale != 0.0:
        g = g * logit_scale
    d = dloss.float().reshape(-1)
    d = d.expand(n) if d.numel() == 1 else d
    g = g * torch.where(valid, d, torch.zeros_like(d))[:, None]
    return g.to(out_dtype or logits.dtype).reshape(logits.shape)


def vocab_parallel_ce(shards, targets: Tensor, label_smoothing: float = 0.0):
    """Every rank's (loss, grad) of VocabParallelCrossEntropyLoss over P = len(shards)
    vocabulary shards (rank p holds shards[p], columns p*Vp .. (p+1)*Vp - 1), for an
    upstream gradient of 1.

    Restates distributed/tensor_parallel.py:1497-1632 with its all-reduces taken
    over the list of shards: the row max (:1522-1531, MAX), the sum of exp
    (:1537-1545, SUM), the masked target logit (:1553-1573, SUM), the loss
    -target + max + log(sum) (:1576), label smoothing with the rank's own shard
    mean (:1587-1588), loss.mean() (:1597); backward: exp(z - max) / sum
    (:1607), minus the target mask at the clamped local target (:1623), then
    (1 - a) * g - a / Vp with smoothing (:1628-1629), times 1 / (B * S) (:1632).
    No ignore_index: every row counts, as there. The reference computes in the
    logits' dtype; this restatement computes in fp32 (the north star's fp32
    accumulation bar) and returns grads in fp32. Like the reference it multiplies
    the gathered logit by the 0/1 mask (:1569), which is NaN when a shard without
    the target holds -inf at the clamped index (the kernels take 0 there).
    """
    xs = [_cpu(x).reshape(-1, x.shape[-1]).float() for x in shards]
    t = _cpu(targets).reshape(-1).to(torch.int64)
    n, vp = xs[0].shape
    rows = torch.arange(n)
    m = torch.stack([x.max(dim=-1).values for x in xs]).max(dim=0).values
    norm = [x - m[:, None] for x in xs]
    sum_exp = torch.stack([z.exp().sum(dim=-1) for z in norm]).sum(dim=0)
    lse_d = sum_exp.log()
    tgt = torch.zeros(n)
    masks, locals_ = [], []
    for p, x in enumerate(xs):
        v0 = p * vp
        mask = (t >= v0) & (t < v0 + vp)
        local = (t - v0).clamp(min=0, max=vp - 1)
        tgt = tgt + x.gather(1, local[:, None]).squeeze(1) * mask.float()
        masks.append(mask)
        locals_.append(local)
    nll = -tgt + m + lse_d
    out = []
    for p, z in enumerate(norm):
        loss = nll
        if label_smoothing > 0:
            smooth = -z.mean(dim=-1) + lse_d
            loss = (1 - label_smoothing) * loss + label_smoothing * smooth
        g = z.exp() / sum_exp[:, None]
        g[rows, locals_[p]] -= masks[p].float()
        if label_smoothing > 0:
            g = (1 - label_smoothing) * g - label_smoothing / vp
        out.append((loss.mean(), g / n))
    return out


def rl_logit_xform(z32: Tensor, logit_softcapping: float = 0.0, logit_scale: float = 0.0,
                   temperature: float = 1.0) -> Tuple[Tensor, Tensor]:
    """(t, dt/dz) of selective_log_softmax's logit transforms (rl_training.py:114-122):
    softcapping t = c * tanh(z / c) when c > 0, then scaling t * s when s > 0, then
    t / temperature when temperature != 1. fp32 arithmetic (the reference computes
    in the logits' dtype)."""
    t = z32
    d = torch.ones_like(z32)
    if logit_softcapping > 0:
        th = torch.tanh(z32 / logit_softcapping)
        t = logit_softcapping * th
        d = 1 - th * th
    if logit_scale > 0:
        t = t * logit_scale
        d = d * logit_scale
    if temperature != 1.0:
        t = t / temperature
        d = d / temperature
    return t, d


def selective_log_softmax(logits: Tensor, input_ids: Tensor, temperature: float = 1.0,
                          logit_softcapping: float = 0.0, logit_scale: float = 0.0) -> Tensor:
    """fp32 log-probabilities of input_ids [...] under logits [..., V].

    Restates selective_log_softmax (rl_training.py:95-135): softcapping, then
    scaling, then temperature (:114-122), a max-shifted log-softmax (:127-130) and
    a gather at input_ids (:133-134). The reference computes in the logits'
    dtype; this restatement computes in fp32.
    """
    logits, ids = _cpu(logits), _cpu(input_ids).to(torch.int64)
    t, _ = rl_logit_xform(logits.float(), logit_softcapping, logit_scale, temperature)
    m = t.max(dim=-1, keepdim=True).values
    shifted = t - m
    lp = shifted - torch.log(torch.exp(shifted).sum(dim=-1, keepdim=True))
    return torch.gather(lp, -1, ids.unsqueeze(-1)).squeeze(-1)


def linear_ce(hidden: Tensor, weight: Tensor, labels: Tensor, ignore_index: int = -100,
              reduction: str = "mean", bf16_logits: bool = False,
              return_rows: bool = False, logit_softcapping: float = 0.0,
              logit_scaling: float = 0.0, temperature: float = 1.0,
              dloss: Optional[Tensor] = None):
    """Fused linear cross-entropy as its composition: logits = hidden @ weight.T -> CE.

    hidden [N, H], weight [V, H] (the lm_head layout of rl_training.py:156-177),
    fp32 products. With bf16_logits the logits are rounded to bf16 as the
    reference's bf16 matmul rounds them (rl_training.py:177, bf16 operands), the
    loss is the fp32 CE of those bf16 logits (kernels/triton_kernels.py:328-337),
    and dlogits are rounded to bf16 as autograd hands them to the bf16 matmul's
    backward. The logits pass through rl_logit_xform (softcap, scale,
    temperature, in rl_training.py:114-122's order) before the CE; the per-row
    loss is -selective_log_softmax (rl_training.py:123-134).

    reduction "mean" (over non-ignored rows), "sum" or "none" (per-row losses).
    dloss: the upstream gradient (a scalar for mean/sum, [N] or a scalar for
    none; default 1). Returns (loss fp32 scalar or [N] rows, grad_hidden,
    grad_weight) in the input dtypes; with return_rows also (loss_rows, lse).
    """
    hidden, weight, labels = _cpu(hidden), _cpu(weight), _cpu(labels).reshape(-1)
    h32, w32 = hidden.float(), weight.float()
    logits = h32 @ w32.t()
    if bf16_logits:
        logits = logits.to(torch.bfloat16).float()
    t, dtdz = rl_logit_xform(logits, logit_softcapping, logit_scaling, temperature)
    loss_rows, lse = ce_fwd(t, labels, ignore_index)
    n_valid = max(int((labels != ignore_index).sum()), 1)
    up = torch.ones(()) if dloss is None else _cpu(dloss).float().reshape(-1)
    if reduction == "none":
        loss = loss_rows
        d = up
    else:
        scale = 1.0 / n_valid if reduction == "mean" else 1.0
        loss = loss_rows.sum() * scale
        d = up.reshape(()) * scale
    g = ce_bwd(t, labels, d, ignore_index, out_dtype=torch.float32) * dtdz
    if bf16_logits:
        g = g.to(torch.bfloat16).float()
    grad_h = (g @ w32).to(hidden.dtype)
    grad_w = (g.t() @ h32).to(weight.dtype)
    if return_rows:
        return loss, grad_h, grad_w, loss_rows, lse
    return loss, grad_h, grad_w


def swiglu_fwd(gate: Tensor, up: Tensor) -> Tensor:
    """out = (silu(g) rounded to up.dtype) * up, silu(g) = g * sigmoid(g) in fp32.

    Restates _swiglu_forward_kernel (kernels/triton_kernels.py:1058-1066):
    silu.to(up.dtype) * up, the product of two values of up's dtype formed in
    fp32 and rounded once more.
    """
    gate, up = _cpu(gate), _cpu(up)
    g = gate.float()
    silu = g * torch.sigmoid(g)
    return (silu.to(up.dtype).float() * up.float()).to(up.dtype)


def swiglu_bwd(dout: Tensor, gate: Tensor, up: Tensor) -> Tuple[Tensor, Tensor]:
    """dgate = dout*up*s*(1 + g*(1 - s)), dup = dout*g*s, s = sigmoid(g), fp32, rounded once.

    Restates _swiglu_backward_kernel (kernels/triton_kernels.py:1089-1101).
    """
    dout, gate, up = _cpu(dout), _cpu(gate), _cpu(up)
    d, g, u = dout.float(), gate.float(), up.float()
    s = torch.sigmoid(g)
    dg = d * u * (s * (1.0 + g * (1.0 - s)))
    du = d * (g * s)
    return dg.to(gate.dtype), du.to(up.dtype)
