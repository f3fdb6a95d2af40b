"""Empty inputs through every op (GPU): zero rows, zero tokens, zero elements.

Each op returns outputs of the right (empty) shape without launching anything
that reads or writes out of range, and reductions follow the reference's
definitions: a mean over zero rows is 0 / 0 (NaN) where the reference divides
by the count (fast_cross_entropy_loss, triton_kernels.py:464-467; the
vocab-parallel loss.mean(), tensor_parallel.py:1597), and 0 where the loss
classes define the mean of no valid rows as 0.
"""
import math

import pytest
import torch

from trainscale_amd import ops
from trainscale_amd.distributed import vocab_parallel_cross_entropy
from trainscale_amd.kernels import (Fast_CrossEntropyLoss, Fast_RoPE, Fast_SwiGLU,
                                    apply_rope, apply_rope_theta, fast_cross_entropy_loss)
from trainscale_amd.kernels.layernorm_kernels import fused_add_rms_layernorm
from trainscale_amd.loss import (ChunkedCrossEntropyLoss, fused_linear_cross_entropy,
                                 selective_log_softmax)

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.mark.parametrize("shape", [(2, 0, 4, 64), (0, 5, 4, 64)])
def test_rope_empty(gpu, shape):
    q = torch.randn(shape, device=gpu).to(BF).requires_grad_()
    k = torch.randn(shape[:2] + (2, 64), device=gpu).to(BF).requires_grad_()
    cos = torch.ones(8, 32, device=gpu)
    sin = torch.zeros(8, 32, device=gpu)
    qo, ko = Fast_RoPE.apply(q, k, cos, sin, False)
    assert qo.shape == q.shape and ko.shape == k.shape
    (qo.float().sum() + ko.float().sum()).backward()
    assert q.grad.shape == q.shape and k.grad.shape == k.shape
    x = torch.randn(shape, device=gpu).to(BF)
    assert apply_rope(x, cos, sin, inplace=False).shape == shape
    assert apply_rope_theta(x, 10000.0, inplace=False).shape == shape


def test_cross_entropy_empty(gpu):
    V = 1024
    logits = torch.randn(0, V, device=gpu).to(BF).requires_grad_()
    labels = torch.zeros(0, dtype=torch.int64, device=gpu)
    rows = Fast_CrossEntropyLoss.apply(logits.clone(), labels)
    assert rows.shape == (0,)
    loss = fast_cross_entropy_loss(logits, labels)
    assert math.isnan(loss.item())  # 0 / 0, as the reference's sum / n_items
    loss = ChunkedCrossEntropyLoss()(logits, labels)
    assert loss.item() == 0.0
    loss.backward()
    assert logits.grad.shape == (0, V)
    l, lse, g = ops.ce_forward_backward(logits.detach(), V, labels,
                                        torch.ones(1, device=gpu))
    assert l.shape == (0,) and lse.shape == (0,) and g.shape == (0, V)


def test_swiglu_empty(gpu):
    gate = torch.randn(0, 4096, device=gpu).to(BF).requires_grad_()
    up = torch.randn(0, 4096, device=gpu).to(BF).requires_grad_()
    out = Fast_SwiGLU.apply(gate, up)
    assert out.shape == (0, 4096)
    out.float().sum().backward()
    assert gate.grad.shape == gate.shape and up.grad.shape == up.shape


def test_add_rmsnorm_empty(gpu):
    x = torch.randn(0, 4096, device=gpu).to(BF)
    r = torch.randn(0, 4096, device=gpu).to(BF)
    w = torch.ones(4096, device=gpu).to(BF)
    y, h = fused_add_rms_layernorm(x, r, w, 1e-6, return_residual=True)
    assert y.shape == (0, 4096) and h.shape == (0, 4096)


@pytest.mark.parametrize("schedule", ["auto", "fused", "two_pass"])
def test_linear_ce_empty(gpu, schedule):
    H, V = 128, 1000
    hidden = torch.randn(0, H, device=gpu).to(BF).requires_grad_()
    weight = (0.02 * torch.randn(V, H, device=gpu)).to(BF)
    weight.fill_(1.0)  # grad_weight must come back zero, not a leftover
    weight.requires_grad_()
    labels = torch.zeros(0, dtype=torch.int64, device=gpu)
    loss = fused_linear_cross_entropy(hidden, weight, labels, schedule=schedule)
    assert loss.item() == 0.0
    loss.backward()
    assert hidden.grad.shape == (0, H)
    assert torch.count_nonzero(weight.grad) == 0
    rows = fused_linear_cross_entropy(hidden, weight, labels, reduction="none")
    assert rows.shape == (0,)


def test_vocab_parallel_empty(gpu):
    x = torch.randn(2, 0, 512, device=gpu).to(BF).requires_grad_()
    t = torch.zeros(2, 0, dtype=torch.int64, device=gpu)
    loss = vocab_parallel_cross_entropy(x, t)
    assert math.isnan(loss.item())  # loss.mean() over no rows, as the reference
    loss.backward()
    assert x.grad.shape == x.shape


def test_vocab_parallel_linear_ce_empty(gpu):
    from trainscale_amd.distributed import vocab_parallel_linear_cross_entropy
    hidden = torch.randn(0, 100, device=gpu).to(BF).requires_grad_()
    weight = torch.ones(777, 100, device=gpu).to(BF).requires_grad_()
    labels = torch.zeros(0, dtype=torch.int64, device=gpu)
    loss = vocab_parallel_linear_cross_entropy(hidden, weight, labels)
    assert loss.item() == 0.0  # as fused_linear_cross_entropy over no rows
    loss.backward()
    assert hidden.grad.shape == (0, 100)
    assert weight.grad.shape == weight.shape and torch.count_nonzero(weight.grad) == 0


def test_selective_log_softmax_empty(gpu):
    logits = torch.randn(2, 0, 1000, device=gpu).to(BF).requires_grad_()
    ids = torch.zeros(2, 0, dtype=torch.int64, device=gpu)
    out = selective_log_softmax(logits, ids, temperature=0.7)
    assert out.shape == (2, 0) and out.dtype == BF
    out.float().sum().backward()
    assert logits.grad.shape == logits.shape
