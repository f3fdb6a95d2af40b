"""Fused linear cross-entropy (MFMA) vs the oracle (GPU).

Bars:
* Loss within 1e-5 relative (north star). Per-row losses and lse within 1e-5 on at
  least 98% of rows and, on every row, within that plus the change one bf16 rounding
  flip per logit can cause (a logit within an fp32 rounding error of a bf16 midpoint
  rounds either way under another summation order).
* The kernel's own bf16 dlogits (what ts_flce_backward_kept leaves in the logits it was
  handed; every schedule forms the same dlogits bits) within the bound U_d of the
  reference's on every element (tests/lce_bounds.py).
* grad_hidden and grad_weight on every element within the bound that the schedule's
  accumulation structure fixes (one GEMM, or an fp32 or bf16 running sum over chunks;
  tests/lce_bounds.py) around the float64 GEMM of the reference's bf16 dlogits. A copy of
  each gradient with two 32 x 32 blocks swapped must fail that comparison. The north
  star's 2e-2 absolute holds as well (one bf16 ulp where |g| >= 4 makes that larger).
With logits exact in bf16, the loss pins the logits GEMM's tiling and index math.
"""
import math
from types import SimpleNamespace

import numpy as np

import pytest
import torch

import lce_bounds
import oracle
from trainscale_amd import workloads
from trainscale_amd.loss import chunked_log_softmax, fused_linear_cross_entropy
from trainscale_amd.loss.linear_ce import (_chunk_rows, linear_ce_backward, linear_ce_forward,
                                           linear_ce_forward_backward)

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


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
    got, ref = got.cpu().float(), ref.float().cpu()
    bound = bound.cpu()
    d = (got - ref).abs()
    tight = d <= 1e-5 + 1e-5 * ref.abs()
    assert int((~tight).sum()) <= max(1, len(ref) // 50), (what, int((~tight).sum()))
    assert bool((d <= 1e-5 + 1e-5 * ref.abs() + bound).all()), (what, float(d.max()))


_XF = {"logit_softcapping": "softcap", "logit_scaling": "scale", "temperature": "temperature"}


def make_ref(h, w, labels, reduction="mean", dloss=None, token_chunk=None, ignore_index=-100,
             **xf):
    """The reference and bound terms (tests/lce_bounds.py) for these inputs, with the
    kernel's own dlogits taken from the stored-logits schedule (ts_flce_forward_keep then
    ts_flce_backward_kept, which leaves dz in the kept logits). The stored-logits
    gradients are checked on the way (one GEMM each)."""
    h2 = h.reshape(-1, h.shape[-1])
    lab = labels.reshape(-1)
    up = dloss if dloss is not None else torch.ones((), device=h.device)
    _, _, lse, logits = linear_ce_forward(h2, w, lab, ignore_index=ignore_index,
                                          reduction=reduction, keep_logits=True, **xf)
    gh, gw = linear_ce_backward(h2, w, lab, lse, up, ignore_index=ignore_index,
                                reduction=reduction, logits=logits, **xf)
    ref = lce_bounds.reference(h2, w, lab, logits, ignore_index=ignore_index,
                               reduction=reduction, dloss=dloss,
                               token_chunk=token_chunk or h2.shape[0],
                               **{_XF[k]: v for k, v in xf.items()})
    del logits
    assert ref.d_beyond == 0, f"{ref.d_beyond} dlogits beyond U_d ({ref.d_changed} differ)"
    check_grads(gh, gw, ref, what="stored logits")
    return ref


def _scaled(ref64, bound, s):
    """A gradient within `bound` of ref64, multiplied by s and rounded to bf16."""
    if s == 1.0:
        return ref64, bound
    b = abs(s) * bound
    return s * ref64, b + 0.5 * lce_bounds.bf16_ulp((s * ref64).abs().float() + b)


def check_grads(gh, gw, ref, vocab_chunks=1, gw_mode="one", scale=1.0, what=""):
    """Every element of grad_hidden / grad_weight within its bound; a copy with two
    32 x 32 blocks swapped is rejected; the north star's 2e-2 absolute."""
    for name, g, r, b in (
            ("grad_hidden", gh, ref.gh_ref, lambda: lce_bounds.gh_bound(ref, vocab_chunks)),
            ("grad_weight", gw, ref.gw_ref, lambda: lce_bounds.gw_bound(ref, gw_mode))):
        if g is None:
            continue
        g = g.reshape(r.shape)
        r, bound = _scaled(r, b(), scale)
        lce_bounds.assert_within(g, r, bound, f"{what} {name}")
        if g.shape[0] >= 64 and g.shape[1] >= 64:
            lce_bounds.assert_block_swap_rejected(g, r, bound, f"{what} {name}")
        # the north star's 2e-2 absolute, or one bf16 ulp where |g| >= 4 makes that larger
        north = torch.clamp(lce_bounds.bf16_ulp(r.abs().float()).double(), min=2e-2)
        assert lce_bounds.beyond(g, r, north) == 0, (what, name)


def _token_chunk(N, V, chunk_tokens):
    """The one-call schedule's token chunk (its kernel rounds to 256 rows; 0: one chunk)."""
    c = _chunk_rows(N, V, chunk_tokens)
    c = -(-c // 256) * 256 if c > 0 else 0
    return c if 0 < c < N else 0


def _vocab_chunks(V, chunk_cols):
    """Vocabulary chunks of the two-pass backward (ts_flce_backward's bwd_chunk_cols)."""
    if chunk_cols:
        c = -(-chunk_cols // 256) * 256
    else:
        c = max(4096, -(-(-(-V // 8)) // 256) * 256)
    c = min(c, -(-V // 8) * 8)
    return -(-V // c)


def check_against_oracle(h, w, labels, reduction="mean", chunk=None, accum="fp32"):
    loss, rows, lse, gh, gw = linear_ce_forward_backward(h, w, labels, reduction=reduction,
                                                         chunk_tokens=chunk,
                                                         grad_weight_accum=accum)
    ref_loss, _, _, ref_rows, ref_lse = oracle.linear_ce(
        h, w, labels, reduction=reduction, bf16_logits=True, return_rows=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss)), (loss.item(),
                                                                              float(ref_loss))
    lse_bound, row_bound = flip_bound(h, w, labels)
    assert_rows_close(rows, ref_rows, row_bound, "loss rows")
    valid = labels.cpu() != -100
    assert_rows_close(lse[valid.to(lse.device)], ref_lse[valid], lse_bound[valid], "lse")
    N, V = h.shape[0], w.shape[0]
    tc = _token_chunk(N, V, chunk)
    ref = make_ref(h, w, labels, reduction, token_chunk=tc or N)
    mode = "one" if tc == 0 else ("bf16_run" if accum == "bf16" else "f32_run")
    check_grads(gh, gw, ref, gw_mode=mode, what=f"one-call chunk {tc} {accum}")
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
    # rounded: grad_hidden is the same GEMM per row
    _, _, _, gh0, gw0 = linear_ce_forward_backward(h, w, labels, chunk_tokens=0)
    assert torch.equal(gh0, gh1)


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
    check_against_oracle(h, w, labels, chunk=256, accum=accum)


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
    ref_loss, _, _, ref_rows, ref_lse = oracle.linear_ce(
        h, w, labels, reduction="sum", bf16_logits=True, return_rows=True)
    torch.testing.assert_close(rows.cpu(), ref_rows, rtol=2e-6, atol=2e-5)
    ref = make_ref(h, w, labels, "sum", token_chunk=_token_chunk(N, V, None) or N)
    # exact logits: the kernel's dlogits can differ from the reference's only by the
    # rounding of values that the two exp implementations put on either side of a midpoint
    assert ref.d_changed <= ref.d_total // 1000, ref.d_changed
    check_grads(gh, gw, ref, gw_mode="f32_run", what="exact logits")


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
    ref_loss, _, _ = oracle.linear_ce(h.detach().reshape(-1, H), w.detach(),
                                      labels.reshape(-1), bf16_logits=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    assert h.grad.shape == h.shape
    # the one-call schedule (one chunk at 128 tokens) forms the gradients for 1 and the
    # backward multiplies them by 3 in place
    ref = make_ref(h.detach(), w.detach(), labels)
    check_grads(h.grad, w.grad, ref, scale=3.0, what="autograd x3")


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


@pytest.mark.parametrize("N,H,V", [(520, 256, 50257), (264, 72, 1001), (136, 100, 777),
                                   (64, 37, 512), (1032, 768, 50257)])
def test_vocab_and_hidden_not_multiples_of_8(gpu, N, H, V):
    """V not a multiple of 8 (GPT-2's 50257): the library pads its logits rows to whole
    16-byte vectors and masks the columns past V; H not a multiple of 8: the wrapper
    zero-pads hidden and weight. Every schedule against the oracle: the one-call schedule
    (default token chunks with an fp32 and a bf16 grad_weight sum, one chunk), the
    two-pass schedule (default and 256-column vocabulary chunks) and, through make_ref,
    the stored-logits schedule."""
    torch.manual_seed(N + H + V)
    h = torch.randn(N, H, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu)
    labels[::13] = -100
    labels[1] = V - 1  # the last column, in the partial last vector when V % 8 != 0
    for chunk, accum in ((None, "fp32"), (None, "bf16"), (0, "bf16")):
        _, gh, gw = check_against_oracle(h, w, labels, chunk=chunk, accum=accum)
        assert gh.shape == (N, H) and gw.shape == (V, H)
    for chunk in (None, 256):
        check_two_pass(h, w, labels, "mean", chunk=chunk)
    # the kept logits: [N, V] over rows padded to whole vectors
    _, _, _, logits = linear_ce_forward(h, w, labels, keep_logits=True)
    assert logits.shape == (N, V) and logits.stride(0) == -(-V // 8) * 8
    z = (h.float().cpu() @ w.float().cpu().t()).to(BF)
    torch.testing.assert_close(logits.float().cpu(), z.float(), rtol=2 ** -7, atol=1e-3)


def test_odd_vocab_through_autograd_and_rl(gpu):
    """fused_linear_cross_entropy (autograd, each schedule) and chunked_log_softmax at
    V = 50257, H = 72 with a non-contiguous hidden view."""
    torch.manual_seed(50257)
    B, L, H, V = 2, 70, 72, 50257
    hb = torch.randn(B, L, H + 8, device=gpu).to(BF)
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, V, (B, L), device=gpu)
    labels[0, :3] = -100
    hd = hb[..., :H]
    for schedule in ("fused", "two_pass", "stored_logits"):
        h = hd.detach().clone().requires_grad_()
        w.grad = None
        loss = fused_linear_cross_entropy(h, w, labels, schedule=schedule)
        loss.backward()
        ref_loss, _, _ = oracle.linear_ce(h.detach().reshape(-1, H), w.detach(),
                                          labels.reshape(-1), bf16_logits=True)
        assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss)), schedule
        ref = make_ref(h.detach(), w.detach(), labels,
                       token_chunk=_token_chunk(B * L, V, None) or B * L)
        mode = "one" if schedule != "fused" or not _token_chunk(B * L, V, None) else "bf16_run"
        check_grads(h.grad, w.grad, ref, gw_mode=mode, what=f"odd V {schedule}")
    hs = hd.detach().clone().requires_grad_()
    w.grad = None
    ids = torch.randint(0, V, (B, L), device=gpu)
    lp = chunked_log_softmax(hs[:, :-1, :], w, ids[:, 1:], temperature=0.8,
                             out_dtype=torch.float32)
    rows, _, _ = oracle.linear_ce(hs.detach()[:, :-1, :].reshape(-1, H), w.detach(),
                                  ids[:, 1:].reshape(-1), reduction="none", bf16_logits=True,
                                  temperature=0.8)
    torch.testing.assert_close(lp.reshape(-1).cpu(), -rows, rtol=1e-5, atol=2e-5)


# ---------------------------------------------------------------------------
# C5 at full size: every element of both gradients, for each schedule
# ---------------------------------------------------------------------------

C5_TOKEN_CHUNK = 4096  # the default schedule's token chunk at N = 8192


@pytest.fixture(scope="module")
def c5(gpu):
    """C5's inputs, the stored-logits schedule's outputs and the reference with its bound
    terms, in token chunks of the default schedule's 4096 rows (torch on the GPU: the
    oracle's arithmetic with fp32 logits GEMMs and float64 gradient GEMMs)."""
    wl = workloads.linear_ce_workload(gpu)
    h, w, labels = wl.tensors["hidden"], wl.tensors["weight"], wl.tensors["labels"]
    assert _token_chunk(h.shape[0], w.shape[0], None) == C5_TOKEN_CHUNK
    one = torch.ones((), device=gpu)
    loss, rows, lse, logits = linear_ce_forward(h, w, labels, keep_logits=True)
    gh, gw = linear_ce_backward(h, w, labels, lse, one, logits=logits)
    ref = lce_bounds.reference(h, w, labels, logits, token_chunk=C5_TOKEN_CHUNK)
    del logits
    torch.cuda.empty_cache()
    yield SimpleNamespace(h=h, w=w, labels=labels, ref=ref, stored=(loss, rows, lse, gh, gw))
    del ref
    torch.cuda.empty_cache()


def _check_c5_loss(c5, loss, rows):
    h, w, labels, ref = c5.h, c5.w, c5.labels, c5.ref
    N = h.shape[0]
    # per-row loss of 32 rows against the CPU oracle (bf16 logits)
    sample = torch.arange(0, N, N // 32)
    logits = (h[sample].float().cpu() @ w.float().cpu().t()).to(BF)
    ref_rows, _ = oracle.ce_fwd(logits, labels[sample].cpu())
    _, row_bound = flip_bound(h[sample], w, labels[sample])
    assert_rows_close(rows[sample], ref_rows, row_bound, "loss rows")
    # every row against the reference on the GPU, within its rounding bound
    assert_rows_close(rows, ref.loss_rows, ref.row_bound, "loss rows (all)")
    n_valid = int((labels != -100).sum())
    ref_loss = float(ref.loss_rows.double().sum()) / n_valid
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss), (loss.item(), ref_loss)


def test_c5_dlogits(c5):
    """The kernel's dlogits at C5 (all 8192 x 128256) within U_d of the reference's, and
    equal to them on all but a small fraction of elements."""
    ref = c5.ref
    assert ref.d_beyond == 0
    assert ref.d_changed <= ref.d_total // 100, (ref.d_changed, ref.d_total)


def test_c5_full(c5):
    """C5 through the schedule fused_linear_cross_entropy picks for it by default (auto:
    the one-call schedule in token chunks of half the tokens, grad_weight summed in its
    bf16 output), the configuration of bench.py's C5 line: the loss, every row's loss,
    and every element of grad_hidden and grad_weight within the bounds of that
    accumulation (a bf16 running sum over 2 chunks for grad_weight)."""
    loss, rows, lse, gh, gw = linear_ce_forward_backward(c5.h, c5.w, c5.labels,
                                                         chunk_tokens=None,
                                                         grad_weight_accum="bf16")
    _check_c5_loss(c5, loss, rows)
    # grad_hidden rows are the same GEMM as in the stored-logits schedule
    assert torch.equal(gh, c5.stored[3])
    check_grads(gh, gw, c5.ref, gw_mode="bf16_run", what="C5 default")


def test_c5_full_stored_logits(c5):
    """C5 through the stored-logits schedule (one GEMM per gradient), and bit for bit
    against the recomputing backward in one vocabulary chunk (the same dz and the same
    two GEMMs)."""
    loss, rows, lse, gh, gw = c5.stored
    _check_c5_loss(c5, loss, rows)
    check_grads(gh, gw, c5.ref, gw_mode="one", what="C5 stored logits")
    one = torch.ones((), device=c5.h.device)
    gh0, gw0 = linear_ce_backward(c5.h, c5.w, c5.labels, lse, one, vocab_chunk=c5.w.shape[0])
    assert torch.equal(gh0, gh) and torch.equal(gw0, gw)


@pytest.mark.parametrize("chunk", [None, 0])
def test_c5_full_fused_schedule(c5, chunk):
    """C5 through the one-call schedule with grad_weight summed in fp32 (opt-in), at the
    default token chunk (half the tokens) and in one chunk (opt-in)."""
    loss, rows, lse, gh, gw = linear_ce_forward_backward(c5.h, c5.w, c5.labels,
                                                         chunk_tokens=chunk,
                                                         grad_weight_accum="fp32")
    _check_c5_loss(c5, loss, rows)
    check_grads(gh, gw, c5.ref, gw_mode="f32_run" if chunk is None else "one",
                what=f"C5 fp32 sum chunk {chunk}")


def test_c5_full_two_pass(c5):
    """C5 through the two-pass schedule (vocabulary-chunked recompute: grad_hidden an fp32
    sum over 8 vocabulary chunks, grad_weight one GEMM per chunk's rows)."""
    loss, rows, lse = linear_ce_forward(c5.h, c5.w, c5.labels)
    gh, gw = linear_ce_backward(c5.h, c5.w, c5.labels, lse, torch.ones((), device=c5.h.device))
    _check_c5_loss(c5, loss, rows)
    check_grads(gh, gw, c5.ref, vocab_chunks=_vocab_chunks(c5.w.shape[0], None), gw_mode="one",
                what="C5 two-pass")


# ---------------------------------------------------------------------------
# Two-pass schedule: vocabulary-chunked backward, RL transforms, per-row upstream
# gradients
# ---------------------------------------------------------------------------

def check_two_pass(h, w, labels, reduction="mean", dloss=None, chunk=None, **xf):
    loss, rows, lse = linear_ce_forward(h, w, labels, reduction=reduction, **xf)
    up = dloss if dloss is not None else torch.ones((), device=h.device)
    gh, gw = linear_ce_backward(h, w, labels, lse, up, reduction=reduction, vocab_chunk=chunk,
                                **xf)
    ref_loss, _, _, ref_rows, ref_lse = oracle.linear_ce(
        h, w, labels, reduction=reduction, bf16_logits=True, return_rows=True,
        dloss=None if dloss is None else dloss.cpu(), **xf)
    if reduction != "none":
        assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss)) + 1e-6, (
            loss.item(), float(ref_loss))
    else:
        assert loss is None
    lse_bound, row_bound = flip_bound(h, w, labels)
    if xf:  # transformed logits: a flip moves t by at most ulp(z) * max|dt/dz|
        m = (xf.get("logit_scaling") or 1.0) / xf.get("temperature", 1.0)
        lse_bound, row_bound = lse_bound * m, row_bound * m
    assert_rows_close(rows, ref_rows, row_bound, "loss rows")
    valid = labels.cpu() != -100
    assert_rows_close(lse[valid.to(lse.device)], ref_lse[valid], lse_bound[valid], "lse")
    ref = make_ref(h, w, labels, reduction, dloss=dloss, **xf)
    check_grads(gh, gw, ref, vocab_chunks=_vocab_chunks(w.shape[0], chunk), gw_mode="one",
                what=f"two-pass chunk {chunk}")
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
    # grad_hidden: fp32 sums over the five chunks, rounded once
    ref = make_ref(h, w, labels)
    check_grads(gh3, None, ref, vocab_chunks=5, what="two-pass 5 chunks")


def test_module_api_schedules(gpu):
    torch.manual_seed(22)
    B, L, H, V = 2, 67, 128, 1024
    h = torch.randn(B, L, H, device=gpu).to(BF).requires_grad_()
    w = (0.05 * torch.randn(V, H, device=gpu)).to(BF).requires_grad_()
    labels = torch.randint(0, V, (B, L), device=gpu)
    labels[0, :5] = -100
    hd, wd = h.detach(), w.detach()
    # the default (auto: the one-call schedule here) against the reference, for 1 times 3
    loss0 = fused_linear_cross_entropy(h, w, labels)
    (3.0 * loss0).backward()
    ref1 = make_ref(hd, wd, labels)
    check_grads(h.grad, w.grad, ref1, scale=3.0, what="auto x3")
    h.grad = None
    w.grad = None
    loss = fused_linear_cross_entropy(h, w, labels, schedule="two_pass")
    assert torch.equal(loss, loss0)
    (3.0 * loss).backward(retain_graph=True)
    ref_loss, _, _ = oracle.linear_ce(hd.reshape(-1, H), wd, labels.reshape(-1),
                                      bf16_logits=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    # the two-pass backward forms the dlogits for the upstream gradient 3 itself
    ref3 = make_ref(hd, wd, labels, dloss=torch.tensor(3.0, device=gpu))
    check_grads(h.grad, w.grad, ref3, what="two-pass upstream 3")
    gh1, gw1 = h.grad.clone(), w.grad.clone()
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
    refn = make_ref(hd, wd, labels, "none", dloss=up.reshape(-1), logit_softcapping=20.0)
    check_grads(h.grad, w.grad, refn, what="none softcap per-row upstream")
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
    ref_loss, _, _ = oracle.linear_ce(h.detach(), w.detach(), labels, bf16_logits=True)
    assert abs(loss.item() - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    assert h.grad.shape == (N, H)
    # the kernel runs N rounded up to 8 rows (the extra rows ignored) in chunks of 256 with
    # grad_weight summed in bf16 (the module's default)
    tc = _token_chunk(N + 5, V, None)
    assert tc == 256
    ref = make_ref(h.detach(), w.detach(), labels, token_chunk=tc)
    check_grads(h.grad, w.grad, ref, gw_mode="bf16_run", what="odd tokens")
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
    assert lp.shape == (B, L - 1) and lp.dtype == BF  # the logits' dtype, as the reference
    lp32 = chunked_log_softmax(hs.detach()[:, :-1, :], lm_head.detach(), ids[:, 1:],
                               temperature=0.9, out_dtype=torch.float32)
    torch.testing.assert_close(lp, lp32.to(BF), rtol=0, atol=0)  # rounded once
    up = torch.randn(B, L - 1, device=gpu)
    (lp * up).sum().backward()
    h2 = hs.detach()[:, :-1, :].reshape(-1, H)
    lab = ids[:, 1:].reshape(-1)
    rows, _, _ = oracle.linear_ce(h2, lm_head.detach(), lab, reduction="none",
                                  bf16_logits=True, temperature=0.9, dloss=-up.reshape(-1).cpu())
    torch.testing.assert_close(lp32.reshape(-1).cpu(), -rows, rtol=1e-5, atol=2e-5)
    assert torch.count_nonzero(hs.grad[:, -1]) == 0  # the last position takes no part
    # autograd hands the bf16 log-probs their upstream gradient in bf16
    dl = -up.to(BF).float().reshape(-1)
    ref = make_ref(h2, lm_head.detach(), lab, "none", dloss=dl, ignore_index=-(1 << 62),
                   temperature=0.9)
    check_grads(hs.grad[:, :-1].reshape(-1, H), lm_head.grad, ref, what="chunked_log_softmax")


@pytest.mark.parametrize("kw", [dict(), dict(temperature=0.9),
                                dict(logit_softcapping=3.0, logit_scale=0.8, temperature=0.7),
                                dict(logit_softcapping=30.0), dict(logit_scale=1.7)])
@pytest.mark.parametrize("V", [1000, 50257])
def test_selective_log_softmax_on_explicit_logits(gpu, kw, V):
    """selective_log_softmax (rl_training.py:95-135) on explicit bf16 logits [B, L, V]:
    log-probs against the oracle (fp32) within 1e-5 and within one bf16 rounding in the
    default (logits') dtype; the gradient of the logits within 1 bf16 ulp of the
    oracle's -dout * (softmax - onehot) * dt/dz."""
    from trainscale_amd.loss import selective_log_softmax
    torch.manual_seed(V)
    B, L = 3, 37
    z = (3 * torch.randn(B, L, V, device=gpu)).to(BF).requires_grad_()
    ids = torch.randint(0, V, (B, L), device=gpu)
    lp = selective_log_softmax(z, ids, **kw)
    assert lp.shape == (B, L) and lp.dtype == BF
    lp32 = selective_log_softmax(z.detach(), ids, out_dtype=torch.float32, **kw)
    ref = oracle.selective_log_softmax(z.detach().cpu(), ids.cpu(), **kw)
    torch.testing.assert_close(lp32.cpu(), ref, rtol=1e-5, atol=1e-5)
    assert torch.equal(lp, lp32.to(BF))
    up = torch.randn(B, L, device=gpu)
    (lp.float() * up).sum().backward()
    t, dt = oracle.rl_logit_xform(z.detach().float().cpu(), kw.get("logit_softcapping", 0.0),
                                  kw.get("logit_scale", 0.0), kw.get("temperature", 1.0))
    dl = -up.to(BF).float().reshape(-1).cpu()  # lp is bf16: its upstream gradient is bf16
    g = (oracle.ce_bwd(t.reshape(-1, V), ids.reshape(-1).cpu(), dl, out_dtype=torch.float32)
         * dt.reshape(-1, V))
    from helpers import assert_ulp
    assert_ulp(z.grad.reshape(-1, V), g, 1, tiny=1e-30, what="grad logits")


def test_selective_log_softmax_golden_rl_case(gpu):
    """The golden RL case (softcap 3, scale 0.8, temperature 0.7; float64 per-token losses)
    through selective_log_softmax on its fp32 logits."""
    from helpers import golden
    from trainscale_amd.loss import selective_log_softmax
    g = golden("linear_ce_rl")
    z = torch.from_numpy(g["hidden"]).double() @ torch.from_numpy(g["weight"]).double().t()
    labels = torch.from_numpy(g["labels"])
    valid = labels != -100
    lp = selective_log_softmax(z.float().to(gpu), labels.clamp(min=0).to(gpu),
                               temperature=float(g["temperature"]),
                               logit_softcapping=float(g["softcap"]),
                               logit_scale=float(g["scale"]))
    assert lp.dtype == torch.float32
    np.testing.assert_allclose(lp.cpu()[valid].double().numpy(),
                               -g["loss_rows"][valid.numpy()], rtol=1e-5, atol=1e-5)


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
    assert torch.equal(gw2, gw1)
    # and against the reference (make_ref also checks the stored-logits pair itself)
    ref = make_ref(h, w, labels, reduction, dloss=up, **xf)
    check_grads(gh1, gw1, ref, what="stored logits")
    check_grads(gh2, None, ref, vocab_chunks=_vocab_chunks(V, 256), what="recompute 256")


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
    # chunked_log_softmax with and without the kept logits: at V = 1024 the recompute runs
    # one vocabulary chunk, so both gradients are the same GEMMs
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
    assert torch.equal(out[0][2], out[1][2]) and torch.equal(out[0][1], out[1][1])


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


@pytest.mark.parametrize("schedule", ["one_call", "two_pass", "stored_logits"])
def test_out_of_range_labels_give_nan_rows(gpu, schedule):
    """A label outside [0, V) that is not ignore_index (the reference's F.cross_entropy
    rejects it) gives that row a NaN loss, as the CE kernels do, and leaves the other
    rows' losses as they are; the reduced loss is then NaN."""
    g = torch.Generator().manual_seed(12)
    N, H, V = 64, 32, 1000
    h = torch.randn(N, H, generator=g).to(BF).to(gpu)
    w = (0.1 * torch.randn(V, H, generator=g)).to(BF).to(gpu)
    labels = torch.randint(0, V, (N,), generator=g).to(gpu)
    labels[3] = -100
    bad = labels.clone()
    bad[5], bad[9] = V, -7
    if schedule == "one_call":
        run = lambda lab: linear_ce_forward_backward(h, w, lab)[:2]
    else:
        run = lambda lab: linear_ce_forward(h, w, lab, reduction="mean",
                                            keep_logits=schedule == "stored_logits")[:2]
    loss_ok, rows_ok = run(labels)
    loss_bad, rows_bad = run(bad)
    assert math.isfinite(loss_ok.item()) and math.isnan(loss_bad.item())
    assert torch.isnan(rows_bad[5]) and torch.isnan(rows_bad[9])
    keep = torch.ones(N, dtype=torch.bool, device=gpu)
    keep[5] = keep[9] = False
    assert torch.equal(rows_bad[keep], rows_ok[keep])
