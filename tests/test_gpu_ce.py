"""Cross-entropy kernels vs the oracle and the golden vectors (GPU).

Bar (north star): loss within 1e-5 relative (fp32), gradients within 2e-2
absolute; since that absolute bound is vacuous for CE gradients (|g| <=
1/n_valid), gradients are also held to 1 bf16 ulp of the oracle.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_ulp, golden, round_to
from trainscale_amd import ops, workloads
from trainscale_amd.kernels import Fast_CrossEntropyLoss, fast_cross_entropy_loss
from trainscale_amd.loss import (ChunkedCrossEntropyLoss, CrossEntropyLoss,
                                 FusedCrossEntropyLoss)

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
TINY = 1e-37  # below bf16's normal range: v_exp_f32 flushes what the CPU keeps as a denormal


@pytest.mark.parametrize("case", ["ce_plain", "ce_odd_v", "ce_smooth", "ce_softcap_scale"])
def test_golden(gpu, case):
    g = golden(case)
    x = torch.from_numpy(g["logits"]).to(BF).to(gpu)
    labels = torch.from_numpy(g["labels"]).to(gpu)
    a, sc, cap = float(g["smoothing"]), float(g["scale"]), float(g["softcap"])
    loss, lse = ops.ce_forward(x, x.shape[1], labels, -100, sc, cap, a)
    np.testing.assert_allclose(loss.double().cpu().numpy(), g["loss"], rtol=1e-5, atol=1e-6)
    valid = g["labels"] != -100
    n_valid = max(int(valid.sum()), 1)
    grad = torch.empty_like(x)
    ops.ce_backward(x, x.shape[1], labels, lse, torch.tensor([1.0 / n_valid], device=gpu), grad,
                    x.shape[1], 1.0, -100, sc, cap, a)
    assert_ulp(grad, round_to(g["grad"], BF), 1, tiny=TINY, what="grad")


def test_c3_full(gpu):
    wl = workloads.ce_workload(gpu)
    logits, labels = wl.tensors["logits"], wl.tensors["labels"]
    N, V = logits.shape
    n_valid = int((labels != -100).sum())
    x = logits.clone().requires_grad_()
    loss = fast_cross_entropy_loss(x, labels)
    rows = Fast_CrossEntropyLoss.apply(logits.clone(), labels)
    # every row's loss against the oracle, in chunks of rows
    lab_cpu = labels.cpu()
    ref_rows = []
    for s in range(0, N, 1024):
        l, _ = oracle.ce_fwd(logits[s:s + 1024].cpu(), lab_cpu[s:s + 1024])
        ref_rows.append(l)
    ref_rows = torch.cat(ref_rows)
    torch.testing.assert_close(rows.cpu(), ref_rows, rtol=1e-5, atol=1e-6)
    ref_mean = ref_rows.double().sum() / n_valid
    assert abs(loss.item() - ref_mean.item()) <= 1e-5 * abs(ref_mean.item())
    loss.backward()
    grad = x.grad
    # gradients of a sample of rows (incl. ignored ones) at 1 ulp and 2e-2 absolute
    sample = torch.cat([torch.arange(0, 128), torch.arange(N - 128, N),
                        (labels == -100).nonzero().flatten()[:16].cpu()])
    ref_g = oracle.ce_bwd(logits[sample].cpu(), lab_cpu[sample], torch.tensor(1.0 / n_valid))
    assert_ulp(grad[sample], ref_g, 1, tiny=TINY, what="grad")
    assert (grad[sample].float().cpu() - ref_g.float()).abs().max() <= 2e-2
    # full-size properties: ignored rows are zero; a valid row's exact gradient
    # sums to 0, so its bf16-rounded sum is bounded by the rounding error of
    # each element (half an ulp, <= 2^-9 relative): |sum g| <= 2^-8 * sum |g|
    ign = labels == -100
    assert torch.count_nonzero(grad[ign]) == 0
    gv = grad[~ign].float()
    rs = gv.sum(-1).abs()
    bound = gv.abs().sum(-1) * 2.0 ** -8
    assert bool((rs <= bound).all()), float((rs / bound).max())


def test_fast_ce_backward_is_in_place(gpu):
    torch.manual_seed(0)
    logits = (2 * torch.randn(64, 1024, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, 1024, (64,), device=gpu)
    buf = logits.detach().clone().requires_grad_()
    loss = Fast_CrossEntropyLoss.apply(buf, labels).sum()
    loss.backward()
    # the gradient was written into the logits buffer saved by forward
    ref = oracle.ce_bwd(logits.detach().cpu(), labels.cpu(), torch.tensor(1.0))
    assert_ulp(buf.grad, ref, 1, tiny=TINY)


@pytest.mark.parametrize("V", [8, 37, 1000, 4096, 50257, 128256])
@pytest.mark.parametrize("dtype", [BF, torch.float16, torch.float32])
def test_vocab_sizes_and_dtypes(gpu, V, dtype):
    torch.manual_seed(V)
    N = 24
    logits = (2 * torch.randn(N, V, device=gpu)).to(dtype)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::5] = -100
    loss, lse = ops.ce_forward(logits, V, labels)
    ref, ref_lse = oracle.ce_fwd(logits.cpu(), labels.cpu())
    torch.testing.assert_close(loss.cpu(), ref, rtol=1e-5, atol=1e-6)
    grad = torch.empty_like(logits)
    ops.ce_backward(logits, V, labels, lse, torch.tensor([0.5], device=gpu), grad, V)
    ref_g = oracle.ce_bwd(logits.cpu(), labels.cpu(), torch.tensor(0.5))
    if dtype == torch.float32:
        torch.testing.assert_close(grad.cpu(), ref_g, rtol=1e-5, atol=1e-9)
    else:
        assert_ulp(grad, ref_g, 1, tiny=TINY if dtype == BF else 1e-7)


def test_modules_and_reductions(gpu):
    torch.manual_seed(1)
    N, V = 96, 3000
    logits = (2 * torch.randn(N, V, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[:7] = -100
    lab = labels.cpu()
    n_valid = int((lab != -100).sum())
    for a in (0.0, 0.1):
        rows, _ = oracle.ce_fwd(logits.cpu(), lab, label_smoothing=a)
        refs = {"mean": rows.sum() / n_valid, "sum": rows.sum(), "none": rows,
                "batchmean": rows.sum() / N}
        for red, ref in refs.items():
            for mod in (ChunkedCrossEntropyLoss(label_smoothing=a, reduction=red),
                        FusedCrossEntropyLoss(label_smoothing=a, reduction=red)):
                x = logits.clone().requires_grad_()
                out = mod(x.view(4, N // 4, V), labels.view(4, N // 4))
                torch.testing.assert_close(out.cpu().reshape(ref.shape), ref, rtol=1e-5, atol=1e-5)
                out.sum().backward()
                scale = {"mean": 1.0 / n_valid, "sum": 1.0, "none": 1.0, "batchmean": 1.0 / N}[red]
                ref_g = oracle.ce_bwd(logits.cpu(), lab, torch.tensor(scale), label_smoothing=a)
                # With smoothing a non-label gradient is dloss*(p - a/V): where p is
                # close to a/V both fp32 computations cancel, so the floor is 32 fp32
                # ulps of the dloss*a/V term rather than an ulp of the tiny result.
                tiny = max(TINY, 32 * 2.0 ** -24 * scale * a / V)
                assert_ulp(x.grad, ref_g, 1, tiny=tiny, what=f"{type(mod).__name__} {red} {a}")
        if True:
            ce = CrossEntropyLoss(label_smoothing=a)
            out = ce(logits, labels)
            torch.testing.assert_close(out.cpu(), refs["mean"], rtol=1e-5, atol=1e-6)


def test_all_rows_ignored(gpu):
    logits = torch.randn(8, 512, device=gpu).to(BF).requires_grad_()
    labels = torch.full((8,), -100, device=gpu)
    loss = ChunkedCrossEntropyLoss()(logits, labels)
    assert loss.item() == 0.0
    loss.backward()
    assert torch.count_nonzero(logits.grad) == 0


def test_softcap_scaling_fast_ce(gpu):
    torch.manual_seed(2)
    logits = (4 * torch.randn(40, 2048, device=gpu)).to(BF)
    labels = torch.randint(0, 2048, (40,), device=gpu)
    for cap, sc in ((30.0, 0.0), (0.0, 0.125), (5.0, 0.5)):
        x = logits.clone().requires_grad_()
        loss = fast_cross_entropy_loss(x, labels, logit_softcapping=cap, logit_scaling=sc)
        rows, _ = oracle.ce_fwd(logits.cpu(), labels.cpu(), logit_scale=sc, softcap=cap)
        assert abs(loss.item() - rows.mean().item()) <= 1e-5 * abs(rows.mean().item())
        loss.backward()
        ref_g = oracle.ce_bwd(logits.cpu(), labels.cpu(), torch.tensor(1.0 / 40),
                              logit_scale=sc, softcap=cap)
        assert_ulp(x.grad, ref_g, 1, tiny=TINY)


def test_out_of_range_label_is_nan(gpu):
    logits = torch.randn(3, 64, device=gpu).to(BF)
    labels = torch.tensor([1, 64, -100], device=gpu)
    loss, _ = ops.ce_forward(logits, 64, labels)
    l = loss.cpu()
    assert math.isnan(l[1]) and not math.isnan(l[0]) and l[2] == 0.0


# ---------------------------------------------------------------------------
# Schedule B: loss and gradient in one pass (ts_ce_fwd_bwd)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("V", [8, 1000, 4096, 32000, 128256, 140000])
@pytest.mark.parametrize("dtype", [BF, torch.float16, torch.float32])
def test_fused_fwd_bwd_matches_oracle(gpu, V, dtype):
    torch.manual_seed(V + 1)
    N = 20
    logits = (2 * torch.randn(N, V, device=gpu)).to(dtype)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::6] = -100
    dl = torch.tensor([0.25], device=gpu)
    loss, lse, grad = ops.ce_forward_backward(logits, V, labels, dl)
    ref, ref_lse = oracle.ce_fwd(logits.cpu(), labels.cpu())
    torch.testing.assert_close(loss.cpu(), ref, rtol=1e-5, atol=1e-6)
    ref_g = oracle.ce_bwd(logits.cpu(), labels.cpu(), torch.tensor(0.25))
    if dtype == torch.float32:
        torch.testing.assert_close(grad.cpu(), ref_g, rtol=1e-5, atol=1e-9)
    else:
        assert_ulp(grad, ref_g, 1, tiny=TINY if dtype == BF else 1e-7)
    # the two-pass schedule gives the same numbers
    l2, lse2 = ops.ce_forward(logits, V, labels)
    g2 = torch.empty_like(logits)
    ops.ce_backward(logits, V, labels, lse2, dl, g2, V)
    torch.testing.assert_close(loss, l2, rtol=1e-6, atol=1e-6)
    if dtype != torch.float32:
        assert max_ulp_gpu(grad, g2) <= 1


def extreme_rows(V, dtype, device):
    """Rows that push the lse fold off its fast path, with labels on finite values.

    0 plain; 1 every lane's first vector -inf; 2 half the values -inf at random;
    3 one value 100 above the rest (overflows a sum taken against an earlier
    reference); 4 values near -300 behind a -inf band (a sum against 0
    underflows); 5 -inf except two values; 6 values near 100; 7 ignored, all -inf.
    """
    g = torch.Generator().manual_seed(V)
    x = 2 * torch.randn(8, V, generator=g)
    band = min(8192, V // 2)
    hi = torch.randint(V // 2, V, (8,), generator=g)
    x[1, :band] = -math.inf
    x[2][torch.rand(V, generator=g) < 0.5] = -math.inf
    x[2, hi[2]] = 1.5
    x[3, (3 * V) // 5] = 100.0
    x[4] += -300.0
    x[4, :band] = -math.inf
    x[5] = -math.inf
    x[5, hi[5]] = 3.0
    x[5, (hi[5] + 1) % V] = 1.0
    x[6] += 100.0
    x[7] = -math.inf
    labels = hi.clone()
    labels[7] = -100
    return x.to(dtype).to(device), labels.to(device)


def assert_loss_close(loss, lse, ref, ref_lse, valid):
    """loss within 1e-5 relative, plus the fp32 resolution of lse - z at the row's lse."""
    loss, lse = loss.cpu().double(), lse.cpu().double()
    ref, ref_lse = ref.double(), ref_lse.double()
    slack = 4 * 2.0 ** -23 * ref_lse.abs().clamp(min=1.0)
    bad = (loss - ref).abs() > 1e-5 * ref.abs() + slack
    assert not bool(bad.any()), (loss, ref)
    assert bool(((lse - ref_lse).abs()[valid] <= 2 * slack[valid]).all()), (lse, ref_lse)


@pytest.mark.parametrize("schedule", ["fused", "two_pass"])
@pytest.mark.parametrize("V,dtype", [(128256, BF), (4096, BF), (1000, BF), (50257, BF),
                                     (128256, torch.float32)])
def test_extreme_logits(gpu, schedule, V, dtype):
    """-inf entries (masked vocab), offsets far from 0 and a value far above its
    neighbours give the oracle's loss and gradient; before the lse fold treated an
    all -inf first vector, these rows came out NaN."""
    x, labels = extreme_rows(V, dtype, gpu)
    n = x.shape[0]
    dl = torch.full((n,), 0.125, device=gpu)
    if schedule == "fused":
        loss, lse, grad = ops.ce_forward_backward(x, V, labels, dl)
    else:
        loss, lse = ops.ce_forward(x, V, labels)
        grad = torch.empty_like(x)
        ops.ce_backward(x, V, labels, lse, dl, grad, V)
    ref, ref_lse = oracle.ce_fwd(x.cpu(), labels.cpu())
    valid = (labels != -100).cpu()
    assert torch.isfinite(loss).all() and torch.isfinite(grad.float()).all()
    assert_loss_close(loss, lse, ref, ref_lse, valid)
    # Row 7 is ignored: zeros, as the reference kernel writes without reading the
    # row (the eager softmax of an all -inf row would be NaN times 0).
    assert torch.count_nonzero(grad[7]) == 0
    ref_g = oracle.ce_bwd(x[:7].cpu(), labels[:7].cpu(), dl[:7].cpu())
    if dtype == torch.float32:
        torch.testing.assert_close(grad[:7].cpu(), ref_g, rtol=2e-5, atol=1e-9)
    else:
        assert_ulp(grad[:7], ref_g, 1, tiny=TINY, what="grad")


@pytest.mark.parametrize("schedule", ["fused", "two_pass"])
def test_nan_logit_poisons_its_row_only(gpu, schedule):
    V = 4096
    torch.manual_seed(9)
    x = (2 * torch.randn(4, V, device=gpu)).to(BF)
    x[1, 77] = math.nan
    x[3, 5] = math.nan
    labels = torch.tensor([10, 20, 30, -100], device=gpu)
    dl = torch.full((4,), 0.25, device=gpu)
    if schedule == "fused":
        loss, lse, grad = ops.ce_forward_backward(x, V, labels, dl)
    else:
        loss, lse = ops.ce_forward(x, V, labels)
        grad = torch.empty_like(x)
        ops.ce_backward(x, V, labels, lse, dl, grad, V)
    ref, _ = oracle.ce_fwd(x.cpu(), labels.cpu())
    assert torch.isnan(loss[1]) and torch.isnan(ref[1])
    assert bool(torch.isnan(grad[1].float()).all())
    keep = torch.tensor([0, 2, 3])
    torch.testing.assert_close(loss.cpu()[keep], ref[keep], rtol=1e-5, atol=1e-6)
    ref_g = oracle.ce_bwd(x.cpu()[keep], labels.cpu()[keep], dl.cpu()[keep])
    assert_ulp(grad[keep.to(gpu)], ref_g, 1, tiny=TINY, what="grad")
    assert torch.count_nonzero(grad[3]) == 0


def max_ulp_gpu(a, b):
    from helpers import max_ulp
    return max_ulp(a.cpu(), b.cpu())


@pytest.mark.parametrize("cap,sc,a", [(30.0, 0.0, 0.0), (0.0, 0.5, 0.0), (0.0, 0.0, 0.1),
                                      (5.0, 0.5, 0.1)])
def test_fused_transforms(gpu, cap, sc, a):
    torch.manual_seed(3)
    N, V = 24, 3000
    logits = (4 * torch.randn(N, V, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[2] = -100
    dl = torch.full((N,), 0.5, device=gpu)
    loss, _, grad = ops.ce_forward_backward(logits, V, labels, dl, 1.0, -100, sc, cap, a,
                                            grad_dtype=torch.float32)
    ref, _ = oracle.ce_fwd(logits.cpu(), labels.cpu(), logit_scale=sc, softcap=cap,
                           label_smoothing=a)
    torch.testing.assert_close(loss.cpu(), ref, rtol=1e-5, atol=1e-5)
    ref_g = oracle.ce_bwd(logits.cpu(), labels.cpu(), torch.full((N,), 0.5), logit_scale=sc,
                          softcap=cap, label_smoothing=a, out_dtype=torch.float32)
    torch.testing.assert_close(grad.cpu(), ref_g, rtol=1e-4, atol=2e-8)


@pytest.mark.parametrize("red", ["mean", "sum", "batchmean"])
def test_loss_classes_upstream_scale_and_no_grad(gpu, red):
    torch.manual_seed(4)
    N, V = 64, 2048
    logits = (2 * torch.randn(N, V, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[:5] = -100
    lab = labels.cpu()
    n_valid = int((lab != -100).sum())
    rows, _ = oracle.ce_fwd(logits.cpu(), lab)
    w = {"mean": 1.0 / n_valid, "sum": 1.0, "batchmean": 1.0 / N}[red]
    for mod in (ChunkedCrossEntropyLoss(reduction=red), FusedCrossEntropyLoss(reduction=red)):
        x = logits.clone().requires_grad_()
        out = mod(x, labels)
        assert abs(out.item() - float(rows.sum()) * w) <= 1e-5 * abs(float(rows.sum()) * w)
        (-2.5 * out).backward()  # upstream gradient -2.5: scaled in place on the device
        ref_g = oracle.ce_bwd(logits.cpu(), lab, torch.tensor(-2.5 * w))
        assert_ulp(x.grad, ref_g, 1, tiny=TINY, what=f"{type(mod).__name__} {red}")
        with torch.no_grad():
            out2 = mod(logits, labels)
        assert abs(out2.item() - out.item()) <= 1e-6 * abs(out.item())


def test_c3_full_fused(gpu):
    wl = workloads.ce_workload(gpu)
    logits, labels = wl.tensors["logits"], wl.tensors["labels"]
    N, V = logits.shape
    n_valid = int((labels != -100).sum())
    dl = torch.tensor([1.0 / n_valid], device=gpu)
    loss, lse, grad = ops.ce_forward_backward(logits, V, labels, dl)
    lab_cpu = labels.cpu()
    sample = torch.cat([torch.arange(0, 256), torch.arange(N - 128, N)])
    ref_rows, _ = oracle.ce_fwd(logits[sample].cpu(), lab_cpu[sample])
    torch.testing.assert_close(loss[sample].cpu(), ref_rows, rtol=1e-5, atol=1e-6)
    ref_g = oracle.ce_bwd(logits[sample].cpu(), lab_cpu[sample], torch.tensor(1.0 / n_valid))
    assert_ulp(grad[sample], ref_g, 1, tiny=TINY, what="grad")
    ign = labels == -100
    assert torch.count_nonzero(grad[ign]) == 0
    # agrees with the two-pass schedule on every row's loss
    l2, _ = ops.ce_forward(logits, V, labels)
    torch.testing.assert_close(loss, l2, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("V", [4096, 128256])
@pytest.mark.parametrize("grad_dtype", [BF, torch.float32])
def test_fused_per_row_upstream_signs(gpu, V, grad_dtype):
    """Schedule B with one upstream gradient per row: negative, positive, +0, -0 and
    large values. The kernel applies the row's sign to the packed gradient words,
    so a row's sign must never leak into another row."""
    torch.manual_seed(V + 3)
    N = 24
    logits = (2 * torch.randn(N, V, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[5] = -100
    dl = torch.randn(N, device=gpu)
    dl[0], dl[1], dl[2], dl[3] = 0.0, -0.0, -3.5, 1e3
    loss, _, grad = ops.ce_forward_backward(logits, V, labels, dl, 0.5, grad_dtype=grad_dtype)
    ref, _ = oracle.ce_fwd(logits.cpu(), labels.cpu())
    torch.testing.assert_close(loss.cpu(), ref, rtol=1e-5, atol=1e-6)
    ref_g = oracle.ce_bwd(logits.cpu(), labels.cpu(), 0.5 * dl.cpu(), out_dtype=torch.float32)
    if grad_dtype == torch.float32:
        torch.testing.assert_close(grad.cpu(), ref_g, rtol=2e-5, atol=1e-30)
    else:
        assert_ulp(grad, ref_g, 1, tiny=TINY)
    signs = torch.sign(grad.float().cpu()) * torch.sign(ref_g)
    assert bool((signs >= 0).all())  # no element has the opposite sign


def test_upstream_grad_hint_across_steps(gpu):
    """A loss scaled the same way every step (1/4, as with 4 accumulation steps): the
    first backward rescales the gradient formed for 1, later steps form it for 1/4
    directly (ratio exactly 1, nothing rescaled); each step matches the oracle."""
    torch.manual_seed(6)
    N, V = 48, 4096
    logits = (2 * torch.randn(N, V, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[7] = -100
    lab = labels.cpu()
    n_valid = int((lab != -100).sum())
    mod = ChunkedCrossEntropyLoss()
    for step, up in enumerate([0.25, 0.25, 0.25, 0.0, 0.5]):
        x = logits.clone().requires_grad_()
        (mod(x, labels) * up).backward()
        ref_g = oracle.ce_bwd(logits.cpu(), lab, torch.tensor(up / n_valid))
        assert_ulp(x.grad, ref_g, 1, tiny=TINY, what=f"step {step} upstream {up}")
        hint = float(mod.grad_hint.get(x.device).item())
        assert hint == (up if up != 0.0 else 1.0), (step, hint)
    # two forwards before one backward: each node keeps the prediction it used
    x = logits.clone().requires_grad_()
    (0.5 * mod(x, labels) + 0.125 * mod(x, labels)).backward()
    ref_g = oracle.ce_bwd(logits.cpu(), lab, torch.tensor(0.625 / n_valid))
    assert_ulp(x.grad, ref_g, 2, tiny=TINY, what="two nodes")


def test_rescale_inplace_ratio_and_hint(gpu):
    t = torch.randn(4096, device=gpu).to(BF)
    orig = t.clone()
    now = torch.tensor([0.75], device=gpu)
    used = torch.tensor([0.75], device=gpu)
    hint = torch.zeros(1, device=gpu)
    ops.rescale_(t, now, used, hint)
    assert torch.equal(t, orig) and hint.item() == 0.75
    used.fill_(1.5)
    ops.rescale_(t, now, used, hint)
    torch.testing.assert_close(t.float(), (orig.float() * 0.5).to(BF).float(), rtol=0, atol=0)
    now.fill_(float("inf"))
    ops.rescale_(t[:0], now, used, hint)  # empty tensor: only the hint is written
    assert hint.item() == 1.0


@pytest.mark.parametrize("mod_cls", [FusedCrossEntropyLoss, ChunkedCrossEntropyLoss,
                                     CrossEntropyLoss])
def test_odd_sizes_through_modules_with_upstream_grad(gpu, mod_cls):
    # N * V = 5 * 37 elements: not a whole number of 16-byte vectors, so the in-place
    # application of the upstream gradient runs its element-wise tail
    g = golden("ce_odd_v")
    x = torch.from_numpy(g["logits"]).to(BF).to(gpu).requires_grad_()
    labels = torch.from_numpy(g["labels"]).to(gpu)
    mod = mod_cls()
    loss = mod(x, labels)
    assert abs(loss.item() - float(g["mean_loss"])) <= 1e-5 * float(g["mean_loss"])
    (2.5 * loss).backward()
    assert_ulp(x.grad, round_to(2.5 * g["grad"], BF), 1, tiny=TINY, what=mod_cls.__name__)
    # a second step with another upstream gradient (the hint's correction path)
    x2 = torch.from_numpy(g["logits"]).to(BF).to(gpu).requires_grad_()
    (-0.75 * mod(x2, labels)).backward()
    assert_ulp(x2.grad, round_to(-0.75 * g["grad"], BF), 1, tiny=TINY, what=mod_cls.__name__)


def test_scale_inplace_unaligned_and_tails(gpu):
    for n, off in ((185, 0), (1000, 1), (4099, 3), (7, 0)):
        base = torch.randn(n + off + 5, device=gpu).to(BF)
        before = base.clone()
        t = base[off:off + n]
        ops.scale_(t, torch.tensor([3.0], device=gpu))
        assert torch.equal(t, (before[off:off + n].float() * 3.0).to(BF)), (n, off)
        # nothing outside the view is written
        assert torch.equal(base[:off], before[:off]) and torch.equal(base[off + n:],
                                                                     before[off + n:])


@pytest.mark.parametrize("red", ["mean", "sum"])
def test_second_backward_is_refused(gpu, red):
    torch.manual_seed(3)
    logits = (2 * torch.randn(64, 1000, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, 1000, (64,), device=gpu)
    loss = ChunkedCrossEntropyLoss(reduction=red)(logits, labels)
    loss.backward(retain_graph=True)
    first = logits.grad.clone()
    with pytest.raises(RuntimeError, match="second time"):
        loss.backward()
    assert torch.equal(logits.grad, first)


def test_c3_full_schedule_b_equals_schedule_a_on_every_row(gpu):
    """The one-pass kernel the headline times (ce_fused_vec, schedule B) against the
    reference's two-pass contract (ce_fwd_vec then ce_bwd_vec, schedule A) on all
    16384 rows of C3: losses within 1e-6, gradients within 1 bf16 ulp; and every valid
    row of the one-pass gradient sums to zero within its elements' rounding."""
    wl = workloads.ce_workload(gpu)
    logits, labels = wl.tensors["logits"], wl.tensors["labels"]
    N, V = logits.shape
    n_valid = int((labels != -100).sum())
    dl = torch.tensor([1.0 / n_valid], device=gpu)
    loss_b, lse_b, grad_b = ops.ce_forward_backward(logits, V, labels, dl)
    loss_a, lse_a = ops.ce_forward(logits, V, labels)
    grad_a = torch.empty_like(logits)
    ops.ce_backward(logits, V, labels, lse_a, dl, grad_a, V)
    torch.testing.assert_close(loss_b, loss_a, rtol=1e-6, atol=1e-6)
    valid = labels != -100
    torch.testing.assert_close(lse_b[valid], lse_a[valid], rtol=1e-6, atol=1e-6)
    # ulp distance on the GPU, 1024 rows at a time
    worst = 0
    for s in range(0, N, 1024):
        a16 = grad_a[s:s + 1024].contiguous().view(torch.int16).int() & 0xFFFF
        b16 = grad_b[s:s + 1024].contiguous().view(torch.int16).int() & 0xFFFF
        a16 = torch.where(a16 < 0x8000, a16, 0x8000 - a16)
        b16 = torch.where(b16 < 0x8000, b16, 0x8000 - b16)
        worst = max(worst, int((a16 - b16).abs().max()))
    assert worst <= 1, worst
    assert torch.count_nonzero(grad_b[~valid]) == 0
    for s in range(0, N, 2048):
        gv = grad_b[s:s + 2048][valid[s:s + 2048]].float()
        rs = gv.sum(-1).abs()
        bound = gv.abs().sum(-1) * 2.0 ** -8
        assert bool((rs <= bound).all()), float((rs / bound).max())


def test_c3_full_gradient_every_row_against_fp32_softmax(gpu):
    """Both schedules' gradients on all 16384 rows of C3 against the oracle's arithmetic
    (oracle.ce_bwd: fp32 softmax of the bf16 logits minus the one-hot, times the upstream
    gradient, rounded once to bf16) evaluated with torch on the GPU, 1024 rows at a time:
    within 1 bf16 ulp on every element. Both roundings start from fp32 values a few fp32
    ulps apart, so they land at most one bf16 ulp apart."""
    wl = workloads.ce_workload(gpu)
    logits, labels = wl.tensors["logits"], wl.tensors["labels"]
    N, V = logits.shape
    valid = labels != -100
    n_valid = int(valid.sum())
    dl = torch.tensor([1.0 / n_valid], device=gpu)
    _, _, grad_b = ops.ce_forward_backward(logits, V, labels, dl)
    _, lse_a = ops.ce_forward(logits, V, labels)
    grad_a = torch.empty_like(logits)
    ops.ce_backward(logits, V, labels, lse_a, dl, grad_a, V)

    def ordered(t):
        u = t.contiguous().view(torch.int16).int() & 0xFFFF
        return torch.where(u < 0x8000, u, 0x8000 - u)

    worst = {"B": 0, "A": 0}
    for s in range(0, N, 1024):
        e = min(s + 1024, N)
        p = torch.softmax(logits[s:e].float(), dim=1)
        vc = valid[s:e]
        rows = torch.arange(e - s, device=gpu)
        p[rows[vc], labels[s:e][vc]] -= 1.0
        p[~vc] = 0.0
        ref = (p * dl).to(BF)
        for name, g in (("B", grad_b), ("A", grad_a)):
            d = (ordered(g[s:e]) - ordered(ref)).abs()
            tiny = (g[s:e].float() - ref.float()).abs() <= TINY
            d = torch.where(tiny, torch.zeros_like(d), d)
            worst[name] = max(worst[name], int(d.max()))
    assert worst["B"] <= 1 and worst["A"] <= 1, worst
