"""The reference's eager PyTorch op sequences for configs C1-C5, run on the CPU.

TEST AND BENCHMARK INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times these
on the GPU box's host cores; nothing in the product imports them. Each function
runs a forward and a backward pass op for op as the reference's CPU path does
it (paths relative to data_pipeline/trainer/), on bf16 inputs:

* rmsnorm: Fast_RMS_LayerNorm's fallback forward (kernels/triton_kernels.py:
  612-616) and RMSLayerNormFunction's fallback backward
  (kernels/layernorm_kernels.py:777-781 for dX, :804-805 for dW).
* rope: Fast_RoPE's fallback (kernels/triton_kernels.py:908-925); the backward
  is the same rotation with sin negated (kernels/rope_kernels.py:1099-1104).
  With position_ids the tables are gathered per token first, as
  _apply_rope_pytorch does (rope_kernels.py:975-976, with the BSHD broadcast).
* ce_chunked: ChunkedCrossEntropyLoss's training path (loss/sota_losses.py:
  695-744: fp32 copy, detached max, exp-sum over 32768-column chunks, gather
  from the bf16 logits, masked mean), backward by autograd.
* ce_float: Fast_CrossEntropyLoss's fallback (kernels/triton_kernels.py:328-337:
  F.cross_entropy(logits.float(), reduction='none')) reduced as
  fast_cross_entropy_loss does (:459-467, sum / n_items), backward by autograd.
* linear_ce: logits = hidden @ lm_head.t() in bf16 (rl_training.py:177)
  followed by ce_float, backward by autograd.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

__all__ = ["rmsnorm", "rope", "ce_chunked", "ce_float", "linear_ce"]


def rmsnorm(x: Tensor, w: Tensor, dy: Tensor, eps: float = 1e-6):
    variance = x.float().pow(2).mean(-1, keepdim=True)
    x_norm = x * torch.rsqrt(variance + eps)
    y = (w * x_norm).to(x.dtype)
    rstd = torch.rsqrt(variance + eps).squeeze(-1)
    # backward
    xn = x * rstd[:, None]
    dy_w = dy * w
    mean_term = (dy_w * xn).mean(dim=-1, keepdim=True)
    dx = rstd[:, None] * (dy_w - xn * mean_term)
    dw = (dy * xn).sum(dim=0)
    return y, dx.to(x.dtype), dw.to(w.dtype)


def _rotate(t: Tensor, cos_e: Tensor, sin_e: Tensor) -> Tensor:
    half = t.shape[-1] // 2
    t1, t2 = t[..., :half], t[..., half:]
    return torch.cat([t1 * cos_e - t2 * sin_e, t1 * sin_e + t2 * cos_e], dim=-1)


def rope(q: Tensor, k: Tensor, dq: Tensor, dk: Tensor, cos: Tensor, sin: Tensor,
         position_ids: Optional[Tensor] = None):
    """q, k [B, S, H, D] bf16; cos, sin [max_pos, D/2] in q's dtype."""
    S = q.shape[1]
    if position_ids is None:
        cos_e = cos[:S].unsqueeze(0).unsqueeze(2)
        sin_e = sin[:S].unsqueeze(0).unsqueeze(2)
    else:
        cos_e = cos[position_ids].unsqueeze(2)
        sin_e = sin[position_ids].unsqueeze(2)
    qo, ko = _rotate(q, cos_e, sin_e), _rotate(k, cos_e, sin_e)
    dqo, dko = _rotate(dq, cos_e, -sin_e), _rotate(dk, cos_e, -sin_e)
    return qo, ko, dqo, dko


def ce_chunked(logits: Tensor, labels: Tensor, ignore_index: int = -100,
               chunk_size: int = 32768):
    x = logits.detach().clone().requires_grad_()
    N, V = x.shape
    logits_fp32 = x.float()
    max_val = logits_fp32.max(dim=-1, keepdim=True).values.detach()
    parts = []
    for start in range(0, V, chunk_size):
        end = min(start + chunk_size, V)
        parts.append(torch.exp(logits_fp32[:, start:end] - max_val).sum(dim=-1, keepdim=True))
    total = sum(parts)
    lse = max_val.squeeze(-1) + torch.log(total.squeeze(-1))
    valid = labels != ignore_index
    tgt = torch.gather(x, dim=1, index=labels.clamp(min=0).unsqueeze(-1)).squeeze(-1)
    loss = -tgt + lse
    loss = torch.where(valid, loss, torch.zeros_like(loss))
    loss = loss.sum() / valid.sum().clamp(min=1)
    loss.backward()
    return loss.detach(), x.grad


def ce_float(logits: Tensor, labels: Tensor):
    x = logits.detach().clone().requires_grad_()
    rows = F.cross_entropy(x.float(), labels, ignore_index=-100, reduction="none")
    n_items = (labels != -100).sum()
    loss = rows.sum() / n_items
    loss.backward()
    return loss.detach(), x.grad


def linear_ce(hidden: Tensor, weight: Tensor, labels: Tensor):
    h = hidden.detach().clone().requires_grad_()
    w = weight.detach().clone().requires_grad_()
    logits = h @ w.t()
    rows = F.cross_entropy(logits.float(), labels, ignore_index=-100, reduction="none")
    loss = rows.sum() / (labels != -100).sum()
    loss.backward()
    return loss.detach(), h.grad, w.grad
