"""Seeded random shapes through every op against the oracle (GPU).

Each op's hand-picked tests cover the shapes its plans and paths distinguish; here a
fixed-seed generator draws further shapes (row lengths on and off the 16-byte vector,
dtypes, layouts, position modes, transforms, token chunks) and holds them to
the same bars through the same checks as the op's own suite:
* RMSNorm: test_gpu_rmsnorm.check_against_oracle (1 ulp; dW by its sum's error bound);
* RoPE: test_gpu_rope.assert_rope (table mode bit for bit, in-register 1 ulp);
* CE: loss within 1e-5 relative of the oracle, gradients within 1 ulp (fp32: 1e-5);
* SwiGLU: test_gpu_swiglu.check;
* linear CE: test_gpu_linear_ce.check_against_oracle / check_two_pass (loss rows
  against the oracle, every gradient element within its arithmetic bound).
The shapes are printed in each case's id, so a failure names its case.
"""
import math
import random

import pytest
import torch

import oracle
from helpers import assert_ulp
from test_gpu_ce import TINY, assert_loss_close
from test_gpu_linear_ce import check_against_oracle as lce_check
from test_gpu_linear_ce import check_two_pass
from test_gpu_rmsnorm import check_against_oracle as rms_check
from test_gpu_rope import assert_rope
from test_gpu_swiglu import check as swiglu_check
from trainscale_amd import ops
from trainscale_amd.kernels import apply_rope, apply_rope_theta

pytestmark = pytest.mark.gpu
BF, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def _cols(rng, hi):
    """A row length: a whole number of 16-byte vectors half the time."""
    c = int(math.exp(rng.uniform(0, math.log(hi))))
    return max(8, c // 8 * 8) if rng.random() < 0.5 else max(1, c)


def _rms_cases(n=24, seed=1):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        rows = rng.randint(1, 300)
        cols = _cols(rng, 9000)
        dtype = rng.choice([BF, BF, F16, F32])
        wdt = rng.choice([dtype, F32])
        out.append((rows, cols, dtype, wdt))
    return out


@pytest.mark.parametrize("rows,cols,dtype,wdt", _rms_cases())
def test_rmsnorm_sweep(gpu, rows, cols, dtype, wdt):
    g = torch.Generator().manual_seed(rows * 131 + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype).to(gpu)
    w = (1 + 0.05 * torch.randn(cols, generator=g)).to(wdt).to(gpu)
    dy = torch.randn(rows, cols, generator=g).to(dtype).to(gpu)
    rms_check(x, w, dy, 1e-6)


def _rope_cases(n=16, seed=2):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        D = 2 * rng.randint(1, 128)
        out.append((rng.randint(1, 3), rng.randint(1, 70), rng.randint(1, 40), rng.randint(1, 8),
                    D, rng.random() < 0.3, rng.choice([BF, BF, F16, F32]),
                    rng.choice(["table", "register"]), rng.choice(["ids", "offset"])))
    return out


@pytest.mark.parametrize("B,S,Hq,Hk,D,il,dtype,mode,pos", _rope_cases())
def test_rope_sweep(gpu, B, S, Hq, Hk, D, il, dtype, mode, pos):
    g = torch.Generator().manual_seed(B * 1000 + S * 10 + D)
    x = torch.randn(B, S, Hq + Hk, D, generator=g).to(dtype).to(gpu)
    n_pos = S + 9
    cos, sin = oracle.rope_tables(D, n_pos, 10000.0)
    if pos == "ids":
        pid = torch.stack([torch.randperm(n_pos, generator=g)[:S] for _ in range(B)]).to(gpu)
        kw, ref_pos = dict(position_ids=pid), oracle.rope_positions(B, S, pid.cpu())
    else:
        kw, ref_pos = dict(position_offset=9), oracle.rope_positions(B, S, position_offset=9)
    for backward in (False, True):
        xg = x.clone().requires_grad_()
        if mode == "table":
            y = apply_rope(xg, cos.to(gpu), sin.to(gpu), interleaved=il, inplace=False, **kw)
        else:
            y = apply_rope_theta(xg, 10000.0, interleaved=il, inplace=False, **kw)
        if not backward:
            assert_rope(y, x, cos, sin, ref_pos, il, what="fwd", exact=mode == "table")
        else:
            gr = torch.randn(y.shape, generator=g).to(dtype).to(gpu)
            y.backward(gr)
            assert_rope(xg.grad, gr, cos, sin, ref_pos, il, backward=True, what="bwd",
                        exact=mode == "table")


def _ce_cases(n=16, seed=3):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        V = int(math.exp(rng.uniform(math.log(2), math.log(200000))))
        xf = rng.choice([(0.0, 0.0, 0.0), (0.0, 0.0, 0.0), (0.7, 0.0, 0.0), (0.0, 20.0, 0.0),
                         (0.0, 0.0, 0.1)])
        out.append((rng.randint(1, 40), V, rng.choice([BF, BF, F16, F32]), *xf))
    return out


@pytest.mark.parametrize("N,V,dtype,scale,cap,smooth", _ce_cases())
def test_ce_sweep(gpu, N, V, dtype, scale, cap, smooth):
    g = torch.Generator().manual_seed(N * 7 + V)
    logits = (2 * torch.randn(N, V, generator=g)).to(dtype).to(gpu)
    labels = torch.randint(0, V, (N,), generator=g)
    labels[torch.rand(N, generator=g) < 0.2] = -100
    labels = labels.to(gpu)
    dl = (0.2 + torch.rand(N, generator=g)).to(gpu)
    ref, ref_lse = oracle.ce_fwd(logits.cpu(), labels.cpu(), -100, scale, cap, smooth)
    ref_g = oracle.ce_bwd(logits.cpu(), labels.cpu(), dl.cpu(), -100, scale, cap, smooth)
    valid = labels.cpu() != -100
    # one pass (schedule B) and forward-then-backward (schedule A)
    loss, lse, grad = ops.ce_forward_backward(logits, V, labels, dl, logit_scale=scale,
                                              softcap=cap, label_smoothing=smooth)
    l2, lse2 = ops.ce_forward(logits, V, labels, -100, scale, cap, smooth)
    g2 = torch.empty_like(logits)
    ops.ce_backward(logits, V, labels, lse2, dl, g2, V, 1.0, -100, scale, cap, smooth)
    for lo, ls, gr in ((loss, lse, grad), (l2, lse2, g2)):
        assert_loss_close(lo, ls, ref, ref_lse, valid)
        if dtype == F32:
            torch.testing.assert_close(gr.cpu(), ref_g, rtol=1e-5, atol=1e-9)
        elif smooth > 0:
            # p - a/V cancels: 32 fp32 ulps of a/V * dloss beside the 1-ulp bar
            tiny = 32 * 2.0 ** -23 * smooth / V * float(dl.max())
            assert_ulp(gr, ref_g, 1, tiny=max(tiny, TINY if dtype == BF else 1e-7))
        else:
            assert_ulp(gr, ref_g, 1, tiny=TINY if dtype == BF else 1e-7)


@pytest.mark.parametrize("n,dtype", [(n, d) for n, d in zip(
    [1, 7, 8, 1023, 65537, 300001, 2 ** 20 + 3, 4096 * 14336 // 64],
    [BF, F16, F32, BF, F16, BF, F32, BF])])
def test_swiglu_sweep(gpu, n, dtype):
    g = torch.Generator().manual_seed(n)
    gate = (3 * torch.randn(n, generator=g)).to(dtype).to(gpu)
    up = torch.randn(n, generator=g).to(dtype).to(gpu)
    dout = torch.randn(n, generator=g).to(dtype).to(gpu)
    swiglu_check(gate, up, dout, what=f"n={n}")


def _lce_cases(n=10, seed=5):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        out.append((rng.randint(1, 700), rng.randint(1, 300),
                    int(math.exp(rng.uniform(math.log(2), math.log(6000)))),
                    rng.choice(["mean", "sum"]), rng.choice([None, 256, 0]),
                    rng.choice(["fp32", "bf16"])))
    return out


@pytest.mark.parametrize("N,H,V,reduction,chunk,accum", _lce_cases())
def test_linear_ce_sweep(gpu, N, H, V, reduction, chunk, accum):
    g = torch.Generator().manual_seed(N + 31 * H + V)
    h = torch.randn(N, H, generator=g).to(BF).to(gpu)
    w = (0.5 / math.sqrt(H) * torch.randn(V, H, generator=g)).to(BF).to(gpu)
    labels = torch.randint(0, V, (N,), generator=g)
    labels[torch.rand(N, generator=g) < 0.1] = -100
    labels = labels.to(gpu)
    lce_check(h, w, labels, reduction=reduction, chunk=chunk, accum=accum)


def _lce_rl_cases(n=6, seed=6):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        out.append((rng.randint(1, 400), rng.randint(1, 200),
                    int(math.exp(rng.uniform(math.log(2), math.log(5000)))),
                    rng.choice([0.0, 3.0, 30.0]), rng.choice([0.0, 0.8]),
                    rng.choice([1.0, 0.7]), rng.choice([None, 256])))
    return out


@pytest.mark.parametrize("N,H,V,cap,scale,temp,chunk", _lce_rl_cases())
def test_linear_ce_rl_sweep(gpu, N, H, V, cap, scale, temp, chunk):
    """The two-pass schedule with the RL transforms and per-row upstream gradients."""
    g = torch.Generator().manual_seed(N * 3 + H + V)
    h = torch.randn(N, H, generator=g).to(BF).to(gpu)
    w = (1.0 / math.sqrt(H) * torch.randn(V, H, generator=g)).to(BF).to(gpu)
    labels = torch.randint(0, V, (N,), generator=g)
    labels[torch.rand(N, generator=g) < 0.1] = -100
    labels = labels.to(gpu)
    dloss = (torch.rand(N, generator=g) - 0.3).to(gpu)
    check_two_pass(h, w, labels, reduction="none", dloss=dloss, chunk=chunk,
                   logit_softcapping=cap, logit_scaling=scale, temperature=temp)


# ---------------------------------------------------------------------------
# The smallest shapes each op takes
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N", [1, 5])
def test_ce_one_class(gpu, N):
    """V = 1: lse is the logit itself, every loss 0 and every gradient 0 (both schedules)."""
    logits = torch.randn(N, 1, device=gpu).to(BF)
    labels = torch.zeros(N, dtype=torch.int64, device=gpu)
    ref, ref_lse = oracle.ce_fwd(logits.cpu(), labels.cpu())
    dl = torch.ones(1, device=gpu)
    loss, lse, grad = ops.ce_forward_backward(logits, 1, labels, dl)
    l2, lse2 = ops.ce_forward(logits, 1, labels)
    g2 = torch.empty_like(logits)
    ops.ce_backward(logits, 1, labels, lse2, dl, g2, 1)
    for lo, ls, g in ((loss, lse, grad), (l2, lse2, g2)):
        assert torch.equal(lo.cpu(), ref) and torch.count_nonzero(lo) == 0
        assert torch.equal(ls.cpu(), ref_lse)
        assert torch.count_nonzero(g) == 0


def test_linear_ce_one_class_and_one_row(gpu):
    """V = 1 (every loss exactly 0; the gradients 0 up to the rounding of exp(z - lse), which
    the element-wise bounds hold) and N = 1, H = 1, through the one-call and two-pass
    schedules."""
    from trainscale_amd.loss.linear_ce import linear_ce_forward, linear_ce_forward_backward
    g = torch.Generator().manual_seed(9)
    h = torch.randn(7, 16, generator=g).to(BF).to(gpu)
    w = torch.randn(1, 16, generator=g).to(BF).to(gpu)
    labels = torch.zeros(7, dtype=torch.int64, device=gpu)
    loss, rows, _, gh, gw = linear_ce_forward_backward(h, w, labels)
    assert loss.item() == 0.0 and torch.count_nonzero(rows) == 0
    assert float(gh.float().abs().max()) < 1e-4 and float(gw.float().abs().max()) < 1e-4
    lce_check(h, w, labels)
    loss2, _, _ = linear_ce_forward(h, w, labels)
    assert loss2.item() == 0.0
    check_two_pass(h, w, labels)
    # one token, a one-element hidden state
    h1 = torch.randn(1, 1, generator=g).to(BF).to(gpu)
    w1 = torch.randn(300, 1, generator=g).to(BF).to(gpu)
    lab1 = torch.tensor([17], device=gpu)
    lce_check(h1, w1, lab1)
    check_two_pass(h1, w1, lab1)


def test_rmsnorm_one_column_and_rope_one_pair(gpu):
    """RMSNorm over rows of one element (y = x / |x| * w up to eps) and RoPE with a
    head of one pair (D = 2), table and in-register."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(37, 1, generator=g).to(BF).to(gpu)
    w = (1 + 0.05 * torch.randn(1, generator=g)).to(BF).to(gpu)
    dy = torch.randn(37, 1, generator=g).to(BF).to(gpu)
    rms_check(x, w, dy, 1e-6)
    q = torch.randn(2, 5, 3, 2, generator=g).to(BF).to(gpu)
    cos, sin = oracle.rope_tables(2, 5, 10000.0)
    pos = oracle.rope_positions(2, 5)
    assert_rope(apply_rope(q, cos.to(gpu), sin.to(gpu), inplace=False), q, cos, sin, pos,
                exact=True)
    assert_rope(apply_rope_theta(q, 10000.0, inplace=False), q, cos, sin, pos)
