"""Fused linear cross-entropy (MFMA) vs the oracle (GPU).

Bar (north star): loss within 1e-5 relative (fp32), gradients within 2e-2
absolute in bf16. Since 2e-2 is loose next to these gradients' size, they are
also held to a relative Frobenius error of 1e-2 against the oracle, which
follows the reference's bf16 numerics (bf16 logits, bf16 dlogits, fp32
accumulation). With logits that are exact in bf16, GEMM results must agree to
fp32 rounding, which pins the MFMA tiling and index math. Per-row losses and lse
are held to 1e-5 on at least 98% of rows and, on every row, to that plus the
change one bf16 rounding flip per logit can cause (a logit within an fp32
rounding error of a bf16 midpoint rounds either way under another summation
order).
"""
import math

import numpy as np

import pytest
import torch

import oracle
from trainscale_amd import workloads
from trainscale_amd.loss import chunked_log_softmax, fused_linear_cross_entropy
from trainscale_amd.loss.linear_ce import (linear_ce_backward, linear_ce_forward,
                                           linear_ce_forward_backward)

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def rel_fro(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


def bf16_ulp(x):
    """Spacing of bf16 values at |x| (8 significant bits)."""
    e = torch.frexp(x.abs().clamp(min=2.0 ** -126))[1]
    return torch.ldexp(torch.ones_like(x), e - 8)


def flip_bound(h, w, labels):
    """Per-row bound on the change of lse and of the row loss when bf16 logits round
    one ulp the other way (the GEMM's fp32 sums are ordered differently from the CPU
    oracle's, so a logit within a rounding error of a bf16 midpoint may flip):
    sum_j p_j ulp(z_j) (+ ulp(z_label) for the loss)."""
    z = (h.float().cpu() @ w.float().cpu().t()).to(BF).float()
    p = torch.softmax(z, dim=1)
    u = bf16_ulp(z)
    lse_b = (p * u).sum(1)
    lab = labels.cpu().reshape(-1)
    valid = lab != -100
    lab_u = torch.zeros_like(lse_b)
    lab_u[valid] = u[valid.nonzero().squeeze(1), lab[valid]]
    return lse_b, lse_b + lab_u


def assert_rows_close(got, ref, bound, what):
    """Within 1e-5 (relative and absolute) of the oracle on at least 98% of rows, and
    within one bf16 rounding flip of the logits (bound) on every row."""
    got, ref = got.cpu().float(), ref.float()
    d = (got - ref).abs()
    tight = d <= 1e-5 + 1e-5 * ref.abs()
    assert int((~tight).sum()) <= max(1, len(ref) // 50), (what, int((~tight).sum()))
    assert bool((d <= 1e-5 + 1e-5 * ref.abs() + bound).all()), (what, float(d.max()))


def check_against_oracle(h, w, labels, reduction="mean", chunk=None, accum="fp32"):
    loss, rows, lse, gh, gw = linear_ce_forward_backward(h, w, labels, reduction=reduction,
                                                         chunk_tokens=chunk,
                                                         grad_weight_accum=accum)
    ref_loss, ref_gh, ref_gw, ref_rows, ref_lse = oracle.linear_ce(
        h, w, labels, reduction=reduction, bf16_logits=True, return_rows=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss)), (loss.item(),
                                                                              float(ref_loss))
    lse_bound, row_bound = flip_bound(h, w, labels)
    assert_rows_close(rows, ref_rows, row_bound, "loss rows")
    valid = labels.cpu() != -100
    assert_rows_close(lse[valid.to(lse.device)], ref_lse[valid], lse_bound[valid], "lse")
    for name, g, r in (("grad_hidden", gh, ref_gh), ("grad_weight", gw, ref_gw)):
        assert (g.float().cpu() - r.float()).abs().max().item() <= 2e-2, name
        assert rel_fro(g, r) <= 1e-2, (name, rel_fro(g, r))
    return loss, gh, gw


@pytest.mark.parametrize("N,H,V", [(512, 256, 1000), (520, 64, 256), (256, 512, 4096),
                                   (8, 32, 8), (264, 40, 520), (1032, 296, 776)])
def test_small_shapes(gpu, N, H, V):
    torch.manual_seed(N + H + V)
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::20] = -100
    check_against_oracle(h, w, labels)


@pytest.mark.parametrize("chunk", [256, 512])
@pytest.mark.parametrize("accum", ["fp32", "bf16"])
def test_token_chunks_accumulate_grad_weight(gpu, chunk, accum):
    torch.manual_seed(5)
    N, H, V = 1040, 128, 768
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::7] = -100
    _, gh1, gw1 = check_against_oracle(h, w, labels, chunk=chunk, accum=accum)
    # chunking changes only where (fp32) or how often (bf16) the sum of grad_weight is
    # rounded
    _, _, _, gh0, gw0 = linear_ce_forward_backward(h, w, labels, chunk_tokens=0)
    assert torch.equal(gh0, gh1)
    assert rel_fro(gw1, gw0) <= (4e-3 if accum == "fp32" else 8e-3)
    if accum == "bf16":
        # the first chunk's partial sum, then one bf16 rounding per further chunk: the
        # same as summing the per-chunk bf16 results the way autograd does
        parts = [linear_ce_forward_backward(h[s:s + chunk], w, labels[s:s + chunk],
                                            reduction="sum", chunk_tokens=0)[4]
                 for s in range(0, N, chunk)]
        n_valid = int((labels != -100).sum())
        assert rel_fro(gw1.float() * n_valid, sum(p.float() for p in parts)) <= 8e-3


@pytest.mark.parametrize("accum", ["fp32", "bf16"])
def test_token_chunks_partial_tiles(gpu, accum):
    # grad_weight [V, H] with neither dimension a multiple of the 256 x 256 tile (nor H of
    # the 128 columns a wave writes): the running-sum epilogues must mask rows and columns
    torch.manual_seed(9)
    N, H, V = 1032, 296, 776
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[3::11] = -100
    chunk = 256
    _, _, gw1 = check_against_oracle(h, w, labels, chunk=chunk, accum=accum)
    if accum == "bf16":
        parts = [linear_ce_forward_backward(h[s:s + chunk], w, labels[s:s + chunk],
                                            reduction="sum", chunk_tokens=0)[4]
                 for s in range(0, N, chunk)]
        n_valid = int((labels != -100).sum())
        assert rel_fro(gw1.float() * n_valid, sum(p.float() for p in parts)) <= 8e-3


def test_exact_logits_pin_the_gemms(gpu):
    # entries of hidden in {-1, 0, 1}, of weight in {0, +-0.5, +-1}, H = 64: every logit is
    # a multiple of 0.5 of magnitude <= 64, exact in bf16 however the sum is ordered
    torch.manual_seed(6)
    N, H, V = 264, 64, 520
    h = torch.randint(-1, 2, (N, H), device=gpu).float().to(BF)
    w = (torch.randint(-2, 3, (V, H), device=gpu).float() / 2).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[5] = -100
    loss, rows, lse, gh, gw = linear_ce_forward_backward(h, w, labels, reduction="sum")
    ref_loss, ref_gh, ref_gw, ref_rows, ref_lse = oracle.linear_ce(
        h, w, labels, reduction="sum", bf16_logits=True, return_rows=True)
    torch.testing.assert_close(rows.cpu(), ref_rows, rtol=2e-6, atol=2e-5)
    assert rel_fro(gh, ref_gh) <= 5e-3 and rel_fro(gw, ref_gw) <= 5e-3


def test_ignored_rows_and_reductions(gpu):
    torch.manual_seed(7)
    N, H, V = 64, 64, 128
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.full((N,), -100, device=gpu)
    loss, rows, _, gh, gw = linear_ce_forward_backward(h, w, labels)
    assert loss.item() == 0.0 and torch.count_nonzero(rows) == 0
    assert torch.count_nonzero(gh) == 0 and torch.count_nonzero(gw) == 0
    labels = torch.randint(0, V, (N,), device=gpu)
    check_against_oracle(h, w, labels, reduction="sum")


def test_autograd_and_upstream_scale(gpu):
    torch.manual_seed(8)
    B, L, H, V = 2, 64, 128, 512
    h = torch.randn(B, L, H, device=gpu).to(BF).requires_grad_()
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, V, (B, L), device=gpu)
    loss = fused_linear_cross_entropy(h, w, labels)
    (3.0 * loss).backward()
    ref_loss, ref_gh, ref_gw = oracle.linear_ce(h.detach().reshape(-1, H), w.detach(),
                                                labels.reshape(-1), bf16_logits=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    assert h.grad.shape == h.shape
    assert rel_fro(h.grad.reshape(-1, H), 3 * ref_gh.float()) <= 1e-2
    assert rel_fro(w.grad, 3 * ref_gw.float()) <= 1e-2


def test_strided_rows(gpu):
    # hidden and weight as column slices of wider buffers: row strides above H reach the
    # K-major logits GEMM and the MN-major gradient GEMMs (which step k by the stride)
    torch.manual_seed(8)
    N, H, V = 520, 72, 1032
    hb = torch.randn(N, H + 24, device=gpu).to(BF)
    wb = (0.05 * torch.randn(V, H + 40, device=gpu)).to(BF)
    h, w = hb[:, :H], wb[:, :H]
    assert h.stride(0) == H + 24 and w.stride(0) == H + 40
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::9] = -100
    _, gh, gw = check_against_oracle(h, w, labels)
    _, _, _, gh_c, gw_c = linear_ce_forward_backward(h.contiguous(), w.contiguous(), labels)
    assert torch.equal(gh, gh_c) and torch.equal(gw, gw_c)


def _c5_reference(h, w, labels, gw_rows):
    """Loss, grad_hidden and grad_weight[gw_rows] of C5 from torch on the GPU: bf16 matmul
    logits in row chunks, fp32 softmax, dlogits rounded to bf16 (as autograd hands them
    to the bf16 matmul's backward), fp32 products for the sampled grad_weight rows."""
    N = h.shape[0]
    n_valid = int((labels != -100).sum())
    ref_sum = 0.0
    ref_gh = torch.empty_like(h)
    d_cols = torch.empty((N, len(gw_rows)), dtype=torch.float32, device=h.device)
    for s in range(0, N, 1024):
        lg = (h[s:s + 1024] @ w.t()).float()
        lab = labels[s:s + 1024]
        l = torch.logsumexp(lg, -1)
        valid = lab != -100
        tgt = lg.gather(1, lab.clamp(min=0)[:, None]).squeeze(1)
        ref_sum += float(((l - tgt) * valid).sum())
        p = torch.softmax(lg, -1)
        p[valid.nonzero().squeeze(1), lab[valid]] -= 1.0
        p[~valid] = 0.0
        d = (p / n_valid).to(BF)
        ref_gh[s:s + 1024] = d @ w
        d_cols[s:s + 1024] = d[:, gw_rows].float()
        del lg, p, d
    ref_gw_rows = d_cols.t() @ h.float()
    return ref_sum / n_valid, ref_gh, ref_gw_rows


def _check_c5(h, w, labels, loss, rows, gh, gw):
    N, H = h.shape
    V = w.shape[0]
    # per-row loss of 32 rows against the CPU oracle (bf16 logits)
    sample = torch.arange(0, N, N // 32)
    logits = (h[sample].float().cpu() @ w.float().cpu().t()).to(BF)
    ref_rows, _ = oracle.ce_fwd(logits, labels[sample].cpu())
    _, row_bound = flip_bound(h[sample], w, labels[sample])
    assert_rows_close(rows[sample], ref_rows, row_bound, "loss rows")
    # 64 grad_weight rows, one in each 1/64 of the vocabulary (every group of eight
    # 256-row tiles), at varying offsets inside their tiles
    g = torch.Generator().manual_seed(9)
    step = V // 64
    gw_rows = torch.tensor([k * step + int(torch.randint(0, step, (1,), generator=g))
                            for k in range(64)], device=h.device)
    ref_loss, ref_gh, ref_gw_rows = _c5_reference(h, w, labels, gw_rows)
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss), (loss.item(), ref_loss)
    assert rel_fro(gh, ref_gh) <= 1e-2
    assert (gh.float() - ref_gh.float()).abs().max().item() <= 2e-2
    got = gw[gw_rows].float()
    assert rel_fro(got, ref_gw_rows) <= 1e-2, rel_fro(got, ref_gw_rows)
    assert (got - ref_gw_rows).abs().max().item() <= 2e-2
    # every row of dlogits sums to zero, so the column sums of grad_weight vanish
    col = gw.float().sum(0)
    assert col.abs().max().item() <= 1e-2 * gw.float().abs().sum(0).max().item()


def test_c5_full(gpu):
    """C5 at full size through the schedule fused_linear_cross_entropy picks for it by
    default (auto: the one-call schedule in token chunks of a quarter of the tokens,
    grad_weight summed in its bf16 output), the configuration of bench.py's C5 line:
    sampled rows against the CPU oracle, the loss, grad_hidden and 64 grad_weight rows
    spread over the vocabulary against an independent composition on the GPU (torch
    bf16 matmul + fp32 softmax)."""
    wl = workloads.linear_ce_workload(gpu)
    h, w, labels = wl.tensors["hidden"], wl.tensors["weight"], wl.tensors["labels"]
    loss, rows, lse, gh, gw = linear_ce_forward_backward(h, w, labels, chunk_tokens=None,
                                                         grad_weight_accum="bf16")
    _check_c5(h, w, labels, loss, rows, gh, gw)


def test_c5_full_two_pass(gpu):
    """C5 through the two-pass schedule (vocabulary-chunked recompute)."""
    wl = workloads.linear_ce_workload(gpu)
    h, w, labels = wl.tensors["hidden"], wl.tensors["weight"], wl.tensors["labels"]
    loss, rows, lse = linear_ce_forward(h, w, labels)
    gh, gw = linear_ce_backward(h, w, labels, lse, torch.ones((), device=gpu))
    _check_c5(h, w, labels, loss, rows, gh, gw)


@pytest.mark.parametrize("chunk", [None, 0])
def test_c5_full_fused_schedule(gpu, chunk):
    """C5 through the one-call schedule with grad_weight summed in fp32 (opt-in), at the
    default token chunk (a quarter of the tokens) and in one chunk (opt-in)."""
    wl = workloads.linear_ce_workload(gpu)
    h, w, labels = wl.tensors["hidden"], wl.tensors["weight"], wl.tensors["labels"]
    loss, rows, lse, gh, gw = linear_ce_forward_backward(h, w, labels, chunk_tokens=chunk,
                                                         grad_weight_accum="fp32")
    _check_c5(h, w, labels, loss, rows, gh, gw)


def test_c5_full_stored_logits(gpu):
    """C5 through the stored-logits schedule, and bit for bit against the recomputing
    backward in one vocabulary chunk (the same dz and the same two GEMMs)."""
    wl = workloads.linear_ce_workload(gpu)
    h, w, labels = wl.tensors["hidden"], wl.tensors["weight"], wl.tensors["labels"]
    loss, rows, lse, logits = linear_ce_forward(h, w, labels, keep_logits=True)
    one = torch.ones((), device=gpu)
    gh, gw = linear_ce_backward(h, w, labels, lse, one, logits=logits)
    del logits
    _check_c5(h, w, labels, loss, rows, gh, gw)
    gh0, gw0 = linear_ce_backward(h, w, labels, lse, one, vocab_chunk=w.shape[0])
    assert torch.equal(gh0, gh) and torch.equal(gw0, gw)


# ---------------------------------------------------------------------------
# Two-pass schedule (the default): vocabulary-chunked backward, RL transforms,
# per-row upstream gradients
# ---------------------------------------------------------------------------

def check_two_pass(h, w, labels, reduction="mean", dloss=None, chunk=None, **xf):
    loss, rows, lse = linear_ce_forward(h, w, labels, reduction=reduction, **xf)
    up = dloss if dloss is not None else torch.ones((), device=h.device)
    gh, gw = linear_ce_backward(h, w, labels, lse, up, reduction=reduction, vocab_chunk=chunk,
                                **xf)
    ref_loss, ref_gh, ref_gw, ref_rows, ref_lse = oracle.linear_ce(
        h, w, labels, reduction=reduction, bf16_logits=True, return_rows=True,
        dloss=None if dloss is None else dloss.cpu(), **xf)
    if reduction != "none":
        assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss)) + 1e-6, (
            loss.item(), float(ref_loss))
    else:
        assert loss is None
    if not xf:
        lse_bound, row_bound = flip_bound(h, w, labels)
    else:  # transformed logits: a flip moves t by at most ulp(z) * max|dt/dz|
        lse_bound, row_bound = flip_bound(h, w, labels)
        m = (xf.get("logit_scaling") or 1.0) / xf.get("temperature", 1.0)
        lse_bound, row_bound = lse_bound * m, row_bound * m
    assert_rows_close(rows, ref_rows, row_bound, "loss rows")
    valid = labels.cpu() != -100
    assert_rows_close(lse[valid.to(lse.device)], ref_lse[valid], lse_bound[valid], "lse")
    for name, g, r in (("grad_hidden", gh, ref_gh), ("grad_weight", gw, ref_gw)):
        assert (g.float().cpu() - r.float()).abs().max().item() <= 2e-2, name
        assert rel_fro(g, r) <= 1e-2, (name, rel_fro(g, r))
    return loss, rows, lse, gh, gw


@pytest.mark.parametrize("N,H,V,chunk", [(512, 256, 1000, None), (523, 64, 2048, 256),
                                         (257, 512, 4096, 768), (8, 32, 8, None),
                                         (1, 40, 520, 256), (1035, 296, 776, 512)])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_two_pass_shapes(gpu, N, H, V, chunk, reduction):
    torch.manual_seed(N + H + V)
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::20] = -100
    check_two_pass(h, w, labels, reduction, chunk=chunk)


@pytest.mark.parametrize("xf", [dict(logit_softcapping=30.0),
                                dict(logit_scaling=0.5, temperature=0.7),
                                dict(logit_softcapping=3.0, logit_scaling=0.8, temperature=1.3),
                                dict(temperature=2.0)])
@pytest.mark.parametrize("chunk", [None, 256])
def test_two_pass_rl_transforms_per_row_upstream(gpu, xf, chunk):
    torch.manual_seed(17)
    N, H, V = 333, 128, 1536
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.2 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::11] = -100
    dloss = torch.randn(N, device=gpu)  # per-token weights of both signs (advantages)
    check_two_pass(h, w, labels, "none", dloss=dloss, chunk=chunk, **xf)


def test_two_pass_rl_golden_on_gpu(gpu):
    from helpers import golden
    g = golden("linear_ce_rl")
    h = torch.from_numpy(g["hidden"]).to(BF).to(gpu)
    w = torch.from_numpy(g["weight"]).to(BF).to(gpu)
    labels = torch.from_numpy(g["labels"]).to(gpu)
    dloss = torch.from_numpy(g["dloss"]).float().to(gpu)
    kw = dict(logit_softcapping=float(g["softcap"]), logit_scaling=float(g["scale"]),
              temperature=float(g["temperature"]))
    _, rows, lse = linear_ce_forward(h, w, labels, reduction="none", **kw)
    gh, gw = linear_ce_backward(h, w, labels, lse, dloss, reduction="none", **kw)
    # the kernel rounds the logits to bf16, the golden values do not: bound the difference
    # by the rounding (|dz| <= ulp(z)/2, |dt/dz| <= scale / temperature)
    z = torch.from_numpy(g["hidden"]).double() @ torch.from_numpy(g["weight"]).double().t()
    dz = (z - z.to(BF).double()).abs().max().item()
    m = kw["logit_scaling"] / kw["temperature"]
    np.testing.assert_allclose(rows.double().cpu().numpy(), g["loss_rows"], atol=2 * m * dz + 1e-5)
    np.testing.assert_allclose(gh.double().cpu().numpy(), g["grad_hidden"], rtol=0.05, atol=0.02)
    np.testing.assert_allclose(gw.double().cpu().numpy(), g["grad_weight"], rtol=0.05, atol=0.02)


def test_two_pass_equals_one_call_schedule(gpu):
    torch.manual_seed(21)
    N, H, V = 520, 192, 2560
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::13] = -100
    loss1, rows1, lse1, gh1, gw1 = linear_ce_forward_backward(h, w, labels, chunk_tokens=0)
    loss2, rows2, lse2 = linear_ce_forward(h, w, labels)
    # the same GEMM and epilogue arithmetic: statistics and losses bit-identical
    assert torch.equal(rows1, rows2) and torch.equal(lse1, lse2) and torch.equal(loss1, loss2)
    one = torch.ones((), device=gpu)
    gh2, gw2 = linear_ce_backward(h, w, labels, lse2, one, vocab_chunk=V)  # one chunk
    assert torch.equal(gh1, gh2) and torch.equal(gw1, gw2)
    gh3, gw3 = linear_ce_backward(h, w, labels, lse2, one, vocab_chunk=512)  # five chunks
    assert torch.equal(gw1, gw3)  # grad_weight rows of a chunk: the same sums over tokens
    assert rel_fro(gh3, gh1) <= 4e-3  # grad_hidden: fp32 sums over chunks, rounded once


def test_module_api_schedules(gpu):
    torch.manual_seed(22)
    B, L, H, V = 2, 67, 128, 1024
    h = torch.randn(B, L, H, device=gpu).to(BF).requires_grad_()
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, V, (B, L), device=gpu)
    labels[0, :5] = -100
    # the default (auto: the one-call schedule here) against the two-pass schedule
    loss0 = fused_linear_cross_entropy(h, w, labels)
    (3.0 * loss0).backward()
    gh0, gw0 = h.grad.clone(), w.grad.clone()
    h.grad = None
    w.grad = None
    loss = fused_linear_cross_entropy(h, w, labels, schedule="two_pass")
    assert torch.equal(loss, loss0)
    (3.0 * loss).backward(retain_graph=True)
    assert rel_fro(h.grad, gh0) <= 4e-3 and rel_fro(w.grad, gw0) <= 8e-3
    ref_loss, ref_gh, ref_gw = oracle.linear_ce(h.detach().reshape(-1, H), w.detach(),
                                                labels.reshape(-1), bf16_logits=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    gh1, gw1 = h.grad.clone(), w.grad.clone()
    assert rel_fro(gh1.reshape(-1, H), 3 * ref_gh.float()) <= 1e-2
    assert rel_fro(gw1, 3 * ref_gw.float()) <= 1e-2
    # a second backward through the same graph recomputes: the gradients accumulate
    loss.backward()
    torch.testing.assert_close(h.grad.float(), gh1.float() * (4.0 / 3.0), rtol=1e-2, atol=1e-6)
    # reduction "none" with a per-row upstream gradient through autograd
    h.grad = None
    w.grad = None
    rows = fused_linear_cross_entropy(h, w, labels, reduction="none", logit_softcapping=20.0)
    assert rows.shape == labels.shape
    node = rows.grad_fn.next_functions[0][0]  # behind the view to labels' shape
    assert type(node).__name__ == "LinearCrossEntropyFunctionBackward"
    up = torch.randn(B, L, device=gpu)
    (rows * up).sum().backward()
    _, ref_gh2, ref_gw2 = oracle.linear_ce(h.detach().reshape(-1, H), w.detach(),
                                           labels.reshape(-1), reduction="none",
                                           bf16_logits=True, logit_softcapping=20.0,
                                           dloss=up.reshape(-1).cpu())
    assert rel_fro(h.grad.reshape(-1, H), ref_gh2.float()) <= 1e-2
    assert rel_fro(w.grad, ref_gw2.float()) <= 1e-2
    # forward only
    with torch.no_grad():
        l2 = fused_linear_cross_entropy(h, w, labels)
    assert torch.equal(l2, loss.detach())


def test_one_call_schedule_odd_tokens(gpu):
    torch.manual_seed(23)
    N, H, V = 8 * 40 + 3, 64, 512
    h = torch.randn(N, H, device=gpu).to(BF).requires_grad_()
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, V, (N,), device=gpu)
    loss = fused_linear_cross_entropy(h, w, labels, schedule="fused")
    loss.backward()
    ref_loss, ref_gh, ref_gw = oracle.linear_ce(h.detach(), w.detach(), labels,
                                                bf16_logits=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    assert h.grad.shape == (N, H)
    assert rel_fro(h.grad, ref_gh.float()) <= 1e-2 and rel_fro(w.grad, ref_gw.float()) <= 1e-2
    with pytest.raises(RuntimeError, match="second time"):
        l3 = fused_linear_cross_entropy(h, w, labels, schedule="fused")
        l3.backward(retain_graph=True)
        l3.backward()


def test_chunked_log_softmax_drop_in(gpu):
    """rl_training.chunked_log_softmax's call as GRPOCompute.compute_log_probs makes it
    (rl_training.py:544-550): hidden_states[:, :-1, :] (a strided view), lm_head,
    input_ids[:, 1:], temperature; log-probs [B, L-1] and their gradients."""
    torch.manual_seed(24)
    B, L, H, V = 3, 50, 128, 2048
    hs = torch.randn(B, L, H, device=gpu).to(BF).requires_grad_()
    lm_head = (0.1 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    ids = torch.randint(0, V, (B, L), device=gpu)
    lp = chunked_log_softmax(hs[:, :-1, :], lm_head, ids[:, 1:], num_chunks=4, temperature=0.9)
    assert lp.shape == (B, L - 1)
    up = torch.randn(B, L - 1, device=gpu)
    (lp * up).sum().backward()
    h2 = hs.detach()[:, :-1, :].reshape(-1, H)
    lab = ids[:, 1:].reshape(-1)
    rows, ref_gh, ref_gw = oracle.linear_ce(h2, lm_head.detach(), lab, reduction="none",
                                            bf16_logits=True, temperature=0.9,
                                            dloss=-up.reshape(-1).cpu())
    torch.testing.assert_close(lp.reshape(-1).cpu(), -rows, rtol=1e-5, atol=2e-5)
    assert torch.count_nonzero(hs.grad[:, -1]) == 0  # the last position takes no part
    assert rel_fro(hs.grad[:, :-1].reshape(-1, H), ref_gh.float()) <= 1e-2
    assert rel_fro(lm_head.grad, ref_gw.float()) <= 1e-2


@pytest.mark.parametrize("xf,reduction", [({}, "mean"), ({}, "none"),
                                          (dict(logit_softcapping=20.0, logit_scaling=0.5,
                                                temperature=0.9), "none"),
                                          (dict(temperature=0.7), "sum")])
def test_stored_logits_equal_the_recompute(gpu, xf, reduction):
    # ts_flce_forward_keep + ts_flce_backward_kept against the recomputing two-pass: the
    # same statistics, the logits bf16(hidden @ weight.T), and the same dz; with one
    # vocabulary chunk the recompute sums grad_hidden over all of V in one GEMM too, so
    # both gradients are bit-identical
    torch.manual_seed(31)
    N, H, V = 1035, 296, 776
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.1 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::9] = -100
    up = torch.randn(N, device=gpu) if reduction == "none" else torch.full((), 1.5, device=gpu)
    loss0, rows0, lse0 = linear_ce_forward(h, w, labels, reduction=reduction, **xf)
    loss1, rows1, lse1, logits = linear_ce_forward(h, w, labels, reduction=reduction,
                                                   keep_logits=True, **xf)
    assert torch.equal(rows0, rows1) and torch.equal(lse0, lse1)
    if reduction != "none":
        assert torch.equal(loss0, loss1)
    # the kept logits: bf16(hidden @ weight.T) to a bf16 ulp (the fp32 sums are ordered
    # differently from the CPU's; near 0 an absolute 1e-3 stands for that difference)
    z = (h.float().cpu() @ w.float().cpu().t()).to(BF)
    torch.testing.assert_close(logits.float().cpu(), z.float(), rtol=2 ** -7, atol=1e-3)
    gh0, gw0 = linear_ce_backward(h, w, labels, lse0, up, reduction=reduction, vocab_chunk=V,
                                  **xf)
    gh1, gw1 = linear_ce_backward(h, w, labels, lse1, up, reduction=reduction, logits=logits,
                                  **xf)
    assert torch.equal(gh0, gh1) and torch.equal(gw0, gw1)
    gh2, gw2 = linear_ce_backward(h, w, labels, lse0, up, reduction=reduction, vocab_chunk=256,
                                  **xf)
    assert torch.equal(gw2, gw1) and rel_fro(gh2, gh1) <= 4e-3
    # and against the oracle (the recompute is pinned there already; this pins the pair)
    _, ref_gh, ref_gw = oracle.linear_ce(h, w, labels, reduction=reduction, bf16_logits=True,
                                         dloss=up.cpu(), **xf)
    assert rel_fro(gh1, ref_gh.float()) <= 1e-2 and rel_fro(gw1, ref_gw.float()) <= 1e-2


def test_stored_logits_module_and_rl(gpu):
    torch.manual_seed(32)
    B, L, H, V = 2, 67, 128, 1024
    h = torch.randn(B, L, H, device=gpu).to(BF).requires_grad_()
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, V, (B, L), device=gpu)
    labels[0, :5] = -100
    grads = []
    for schedule in ("two_pass", "stored_logits"):
        h.grad = None
        w.grad = None
        rows = fused_linear_cross_entropy(h, w, labels, reduction="none", temperature=0.8,
                                          schedule=schedule, vocab_chunk=V)
        up = torch.linspace(-1.0, 1.0, B * L, device=gpu).reshape(B, L)
        (rows * up).sum().backward(retain_graph=True)
        g1 = (h.grad.clone(), w.grad.clone())
        # a second backward through the same graph: the kept logits were consumed, so it
        # recomputes (vocab_chunk=V: one chunk, bit-identical gradients); they accumulate
        (rows * up).sum().backward()
        grads.append((rows.detach(), g1, (h.grad.clone(), w.grad.clone())))
    (r0, g0, a0), (r1, g1, a1) = grads
    assert torch.equal(r0, r1)
    assert torch.equal(g0[0], g1[0]) and torch.equal(g0[1], g1[1])
    assert torch.equal(a0[0], a1[0]) and torch.equal(a0[1], a1[1])
    # chunked_log_softmax with and without the kept logits
    hs = torch.randn(B, L, H, device=gpu).to(BF).requires_grad_()
    ids = torch.randint(0, V, (B, L), device=gpu)
    out = []
    for store in (False, True):
        hs.grad = None
        w.grad = None
        lp = chunked_log_softmax(hs[:, :-1, :], w, ids[:, 1:], temperature=0.9,
                                 store_logits=store)
        (lp * torch.ones_like(lp)).sum().backward()
        out.append((lp.detach(), hs.grad.clone(), w.grad.clone()))
    assert torch.equal(out[0][0], out[1][0])
    assert torch.equal(out[0][2], out[1][2])  # grad_weight: the same sums over tokens
    assert rel_fro(out[1][1], out[0][1]) <= 4e-3  # grad_hidden: chunked vs one fp32 sum


def test_two_pass_strided_rows(gpu):
    torch.manual_seed(25)
    N, H, V = 519, 72, 1032
    hb = torch.randn(N, H + 24, device=gpu).to(BF)
    wb = (0.05 * torch.randn(V, H + 40, device=gpu)).to(BF)
    h, w = hb[:, :H], wb[:, :H]
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::9] = -100
    _, rows, lse, gh, gw = check_two_pass(h, w, labels, "sum", chunk=256)
    _, rows_c, lse_c, gh_c, gw_c = check_two_pass(h.contiguous(), w.contiguous(), labels, "sum",
                                                  chunk=256)
    assert torch.equal(rows, rows_c) and torch.equal(gh, gh_c) and torch.equal(gw, gw_c)
