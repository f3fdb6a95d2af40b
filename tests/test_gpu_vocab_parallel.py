"""Vocabulary-parallel cross entropy (the kernels of one rank) vs the oracle (GPU).

Each test splits one full-vocabulary logits tensor into P column shards on one
GPU and runs every rank's forward and backward through
VocabParallelCrossEntropyLoss, with an exchange hook that hands each rank the
P partials an all-gather over P ranks would deliver (computed by the same
shard kernel). The shards are strided views of the full tensor, so the ranks'
gradients land side by side in its .grad.

Bar (north star): loss within 1e-5 relative in fp32 (plus the fp32 resolution
of lse - z at the row's lse), gradients within 1 bf16 ulp of the oracle
(fp32 gradients: 2e-5 relative).
"""
import math

import pytest
import torch

import lce_bounds
import oracle
from helpers import assert_ulp
from trainscale_amd import ops
from trainscale_amd.distributed import (VocabShardExchange, set_vocab_exchange,
                                        vocab_parallel_cross_entropy)

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
TINY = 1e-37  # below bf16's normal range: v_exp_f32 flushes what the CPU keeps as a denormal


def run_ranks(x, t, P, a):
    """Every rank's (loss, ) and the full tensor's gradient after all P backwards."""
    V = x.shape[-1]
    vp = V // P
    xg = x.clone().requires_grad_()
    stats = torch.stack([ops.ce_vocab_shard_stats(*ops.as_rows(x[..., p * vp:(p + 1) * vp]),
                                                  t.reshape(-1), p * vp) for p in range(P)])
    losses = []
    try:
        for p in range(P):
            def gather(st, p=p):
                assert torch.equal(st, stats[p])  # this rank's own partials
                return stats
            set_vocab_exchange(VocabShardExchange(gather, p, P))
            loss = vocab_parallel_cross_entropy(xg[..., p * vp:(p + 1) * vp], t, a)
            loss.backward()
            losses.append(loss.detach())
    finally:
        set_vocab_exchange(None)
    return losses, xg.grad, stats


def check_against_oracle(x, t, P, a, losses, grad):
    vp = x.shape[-1] // P
    ref = oracle.vocab_parallel_ce([x[..., p * vp:(p + 1) * vp].cpu() for p in range(P)],
                                   t.cpu(), a)
    lse_mag = torch.logsumexp(x.reshape(-1, x.shape[-1]).float().cpu(), -1).abs().max()
    slack = 4 * 2.0 ** -23 * max(float(lse_mag), 1.0)
    for p in range(P):
        r = ref[p][0].item()
        assert abs(losses[p].item() - r) <= 1e-5 * abs(r) + slack, (p, losses[p].item(), r)
    ref_g = torch.cat([g for _, g in ref], 1).reshape(grad.shape)
    if grad.dtype == torch.float32:
        torch.testing.assert_close(grad.cpu(), ref_g, rtol=2e-5, atol=1e-10)
    else:
        assert_ulp(grad, ref_g, 1, tiny=TINY, what="grad")


def make(V, dtype, seed, B=2, S=12):
    g = torch.Generator().manual_seed(seed)
    x = (2 * torch.randn(B, S, V, generator=g)).to(dtype)
    t = torch.randint(0, V, (B, S), generator=g)
    t[0, 3] = V + 5      # in no shard
    t[1, 7] = -100       # in no shard (the reference has no ignore_index)
    return x.cuda(), t.cuda()


@pytest.mark.parametrize("V,P,dtype,a", [
    (128256, 8, BF, 0.0), (128256, 8, BF, 0.1), (4096, 4, BF, 0.0), (1000, 2, BF, 0.1),
    (50264, 4, torch.float16, 0.0), (32000, 2, torch.float32, 0.1), (128256, 1, BF, 0.0),
    (262144, 1, BF, 0.0)])
def test_ranks_match_the_oracle(V, P, dtype, a):
    """Shard widths through every kernel path: 256 x {2, 4, 8, 16} and 1024 x 16
    register rows, element-wise rows for widths that are not a multiple of the
    vector or wider than 131072, bf16/fp16/fp32, smoothing on and off."""
    x, t = make(V, dtype, V + P)
    losses, grad, _ = run_ranks(x, t, P, a)
    check_against_oracle(x, t, P, a, losses, grad)


def test_masked_vocabulary_and_empty_shards():
    """-inf columns (a padded vocabulary), one rank's shard entirely -inf on a row
    (its partial lse is -inf and the merge skips it), and a value 100 above the
    rest of its row. Checked against the full-vocabulary CE oracle: the reference
    multiplies the gathered target logit by the shard's 0/1 mask
    (tensor_parallel.py:1569), so a -inf logit at the clamped index of a shard
    that does not hold the target makes its loss NaN; these kernels take 0 there,
    and every rank's loss is the full CE's."""
    V, P = 32768, 4
    x, t = make(V, BF, 3)
    x[..., V - 300:] = -math.inf
    x[0, 1, :V // P] = -math.inf
    t[0, 1] = V // P + 17
    x[1, 2, 12345] = 100.0
    losses, grad, stats = run_ranks(x, t, P, 0.0)
    assert stats[0, 1, 0].item() == -math.inf
    x2, t2 = x.reshape(-1, V).cpu(), t.reshape(-1).cpu()
    n = x2.shape[0]
    bad = (t2 < 0) | (t2 >= V)  # in no shard: the loss is the lse (target logit 0)
    full, _ = oracle.ce_fwd(x2, t2.clamp(0, V - 1), ignore_index=-(1 << 40))
    full = torch.where(bad, torch.logsumexp(x2.float(), -1), full)
    for p in range(P):
        assert abs(losses[p].item() - full.mean().item()) <= 1e-5 * abs(full.mean().item())
    ref_g = oracle.ce_bwd(x2, t2.clamp(0, V - 1), torch.tensor(1.0 / n),
                          ignore_index=-(1 << 40), out_dtype=torch.float32)
    soft = torch.softmax(x2.float(), -1) / n
    ref_g[bad] = soft[bad]
    assert_ulp(grad.reshape(-1, V), ref_g, 1, tiny=TINY, what="grad")


def test_merge_of_c3_shards_equals_the_full_ce():
    """At C3's shape with P = 8 (shards of [16384, 16032], the per-rank size): the
    merged lse equals the full-vocabulary CE kernel's lse, and the ranks' gradients
    side by side equal the full kernel's gradient within 1 bf16 ulp."""
    from trainscale_amd import workloads
    wl = workloads.ce_workload(torch.device("cuda"))
    x, labels = wl.tensors["logits"], wl.tensors["labels"]
    N, V = x.shape
    t = labels.clamp(min=0)  # every row counts here
    P, vp = 8, V // 8
    stats = torch.stack([ops.ce_vocab_shard_stats(x[:, p * vp:(p + 1) * vp], V, t, p * vp)
                         for p in range(P)])
    lse, loss = ops.ce_vocab_merge(stats, 0, vp)
    full_loss, full_lse = ops.ce_forward(x, V, t)
    torch.testing.assert_close(lse, full_lse, rtol=2e-6, atol=0)
    torch.testing.assert_close(loss, full_loss, rtol=2e-5, atol=2e-5)
    go = torch.ones((), device=x.device)
    g_full = torch.empty_like(x)
    ops.ce_backward(x, V, t, full_lse, torch.tensor([1.0 / N], device=x.device), g_full, V)
    for p in (0, 3, 7):
        gp = ops.ce_vocab_shard_backward(x[:, p * vp:(p + 1) * vp], V, t, lse, go, 1.0 / N, p * vp)
        d = (gp.float() - g_full[:, p * vp:(p + 1) * vp].float()).abs()
        ulp = g_full[:, p * vp:(p + 1) * vp].float().abs() * 2.0 ** -7
        assert bool((d <= ulp + TINY).all()), float((d - ulp).max())


# ---------------------------------------------------------------------------
# Vocabulary-parallel fused linear CE (one rank's two phases)
# ---------------------------------------------------------------------------

def lce_ranks(h, w, labels, P, reduction="mean"):
    """Every rank's (loss, loss_rows, lse, grad_hidden_partial, grad_weight_shard,
    dlogits_shard): P shards of V // P LM-head rows (V a multiple of P)."""
    from trainscale_amd.loss.linear_ce import linear_ce_vocab_phase1, linear_ce_vocab_phase2
    vp = w.shape[0] // P
    phase1 = [linear_ce_vocab_phase1(h, w[p * vp:(p + 1) * vp], labels, p * vp)
              for p in range(P)]
    stats_all = torch.stack([s for s, _ in phase1])
    outs = []
    for _, st in phase1:
        out = linear_ce_vocab_phase2(st, stats_all, -100, reduction)
        outs.append(out + (shard_dlogits(st),))
    return outs


def shard_dlogits(state):
    """The shard's bf16 dlogits [N, Vp] that phase 2 left in the workspace, where the
    library keeps them: the workspace's first bytes, rows of round_up(Vp, 8) columns."""
    ldl = -(-state.Vp // 8) * 8
    L = state.ws[:state.N * ldl * 2].view(BF).view(state.N, ldl)
    return L[:state.N0, :state.Vp].clone()


def check_rank_grads(outs, ref, P, what):
    """grad_weight: each shard is one K = N GEMM of its dlogits, so the shards side by
    side are held to lce_bounds.gw_bound(ref, "one"). grad_hidden: the float64 sum of
    the ranks' bf16 partials, each a K = Vp GEMM, within the sum of their GEMM bounds and
    roundings. Both reject a copy with two 32 x 32 blocks swapped."""
    vp = ref.gw_ref.shape[0] // P
    gw_cat = torch.cat([o[4] for o in outs], 0)
    bw = lce_bounds.gw_bound(ref, "one")
    lce_bounds.assert_within(gw_cat, ref.gw_ref, bw, f"{what} grad_weight shards")
    if min(gw_cat.shape) >= 64:
        lce_bounds.assert_block_swap_rejected(gw_cat, ref.gw_ref, bw, f"{what} grad_weight")
    # the partials summed in float64 (P bf16 values: exact but for 2^-52 of their size)
    gh_sum = sum(o[3].double() for o in outs)
    mag = sum(o[3].float().abs() for o in outs)
    rnd = sum(0.5 * lce_bounds.bf16_ulp(o[3].float()) for o in outs)  # each partial's rounding
    bh = (lce_bounds.gamma_mfma(vp) * 1.02 * ref.gh_S + 1.02 * ref.gh_D + rnd +
          2.0 ** -40 * ref.gh_S + P * 2.0 ** -52 * mag + lce_bounds.TINY)
    lce_bounds.assert_within(gh_sum, ref.gh_ref, bh, f"{what} grad_hidden sum")
    if min(gh_sum.shape) >= 64:
        lce_bounds.assert_block_swap_rejected(gh_sum, ref.gh_ref, bh, f"{what} grad_hidden")


@pytest.mark.parametrize("N,H,V,P", [(64, 128, 1024, 4), (264, 40, 2080, 2), (520, 256, 4096, 8),
                                     (1032, 296, 1552, 2), (263, 36, 2002, 2),
                                     (100, 72, 2331, 3), (517, 100, 8 * 6283, 8)])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_linear_ce_ranks_match_the_full_kernel(N, H, V, P, reduction):
    """The ranks' loss is the full kernel's and the oracle's; their dlogits side by side
    lie within U_d of the reference's (tests/lce_bounds.py), their grad_weight shards side
    by side and the sum of their grad_hidden partials within the bounds of that GEMM
    structure on every element. Shapes include shard widths that are not multiples of 8
    (1001, 777, 6283: GPT-2's vocabulary over 8 ranks) and N and H that are not."""
    from trainscale_amd.loss.linear_ce import linear_ce_forward_backward
    g = torch.Generator().manual_seed(N + V)
    h = torch.randn(N, H, generator=g).to(BF).cuda()
    w = (0.05 * torch.randn(V, H, generator=g)).to(BF).cuda()
    labels = torch.randint(0, V, (N,), generator=g)
    labels[::9] = -100
    labels = labels.cuda()
    loss, rows, lse, _, _ = linear_ce_forward_backward(h, w, labels, reduction=reduction)
    outs = lce_ranks(h, w, labels, P, reduction)
    ref_loss, _, _, _, _ = oracle.linear_ce(h.cpu(), w.cpu(), labels.cpu(), reduction=reduction,
                                            bf16_logits=True, return_rows=True)
    for lp, rp, lsep, _, _, _ in outs:
        assert abs(lp.item() - loss.item()) <= 2e-6 * abs(loss.item())
        assert abs(lp.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
        torch.testing.assert_close(lsep, lse, rtol=2e-6, atol=0)
        torch.testing.assert_close(rp, rows, rtol=2e-5, atol=2e-5)
    d = torch.cat([o[5] for o in outs], 1)
    ref = lce_bounds.reference(h, w, labels, d, reduction=reduction, token_chunk=N)
    assert ref.d_beyond == 0, f"{ref.d_beyond} dlogits beyond U_d"
    check_rank_grads(outs, ref, P, f"N={N} H={H} V={V} P={P}")


def test_linear_ce_single_rank_autograd_equals_fused():
    """One rank (world size 1): the autograd class gives fused_linear_cross_entropy's
    loss and gradients bit for bit (a merge of one partial leaves lse unchanged),
    including the upstream-gradient scale."""
    from trainscale_amd.distributed import vocab_parallel_linear_cross_entropy
    from trainscale_amd.loss import fused_linear_cross_entropy
    g = torch.Generator().manual_seed(7)
    h = torch.randn(2, 48, 128, generator=g).to(BF).cuda()
    w = (0.05 * torch.randn(1000, 128, generator=g)).to(BF).cuda()
    labels = torch.randint(0, 1000, (2, 48), generator=g)
    labels[0, :5] = -100
    labels = labels.cuda()
    res = []
    for fn in (fused_linear_cross_entropy, vocab_parallel_linear_cross_entropy):
        hg, wg = h.clone().requires_grad_(), w.clone().requires_grad_()
        loss = fn(hg, wg, labels)
        (0.5 * loss).backward()
        res.append((loss.detach(), hg.grad, wg.grad))
    assert torch.equal(res[0][0], res[1][0])
    assert torch.equal(res[0][1], res[1][1]) and torch.equal(res[0][2], res[1][2])


def test_linear_ce_ranks_at_c5_over_8_ranks():
    """The per-rank shape the bench measures: C5 (hidden [8192, 4096], LM head
    [128256, 4096], 5% ignored) split over 8 ranks of [16032, 4096]. Every rank's two
    phases against the full single-GPU kernel: the same loss, per-row loss and lse; the
    ranks' dlogits within U_d of the reference's, and every element of the grad_weight
    shards and of the summed grad_hidden partials within the bounds of that structure."""
    from trainscale_amd import workloads
    from trainscale_amd.loss.linear_ce import linear_ce_forward_backward
    wl = workloads.linear_ce_workload(torch.device("cuda"))
    h, w, labels = wl.tensors["hidden"], wl.tensors["weight"], wl.tensors["labels"]
    loss, rows, lse, _, _ = linear_ce_forward_backward(h, w, labels,
                                                       need_grad_hidden=False,
                                                       need_grad_weight=False)
    P = 8
    outs = lce_ranks(h, w, labels, P)
    for p, (lp, rp, lsep, _, _, _) in enumerate(outs):
        assert abs(lp.item() - loss.item()) <= 2e-6 * abs(loss.item()), p
        torch.testing.assert_close(lsep, lse, rtol=2e-6, atol=0)
        torch.testing.assert_close(rp, rows, rtol=2e-5, atol=2e-5)
    d = torch.cat([o[5] for o in outs], 1)
    outs = [o[:5] for o in outs]
    torch.cuda.empty_cache()
    ref = lce_bounds.reference(h, w, labels, d, token_chunk=h.shape[0])
    del d
    assert ref.d_beyond == 0, f"{ref.d_beyond} dlogits beyond U_d"
    check_rank_grads(outs, ref, P, "C5 over 8 ranks")
