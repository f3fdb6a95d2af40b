"""The linear-CE bound machinery (tests/lce_bounds.py) pinned to the oracle on the CPU.

`lce_bounds.reference` restates oracle.linear_ce's arithmetic chunk by chunk; here it
must agree with the oracle, accept the oracle's own outputs, and reject outputs with
planted mistakes: a dlogit off by 3%, two 32 x 32 blocks swapped, the label column
shifted, a 5% scale error, a bf16 running sum rounded with the wrong chunk boundaries.
"""
import pytest
import torch

import lce_bounds
import oracle

BF = torch.bfloat16


def _inputs(N=160, H=96, V=200, seed=0, ign=9):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(N, H, generator=g).to(BF)
    w = (0.1 * torch.randn(V, H, generator=g)).to(BF)
    labels = torch.randint(0, V, (N,), generator=g)
    labels[::ign] = -100
    return h, w, labels


def oracle_dlogits(h, w, labels, reduction="mean", dloss=None, softcap=0.0, scale=0.0,
                   temperature=1.0):
    """The oracle's bf16 dlogits (oracle.linear_ce before its gradient GEMMs)."""
    z = (h.float() @ w.float().t()).to(BF).float()
    t, dt = oracle.rl_logit_xform(z, softcap, scale, temperature)
    n_valid = max(int((labels != -100).sum()), 1)
    up = torch.ones(()) if dloss is None else dloss.float().reshape(-1)
    d = up if reduction == "none" else up.reshape(()) * (1.0 / n_valid if reduction == "mean"
                                                          else 1.0)
    return (oracle.ce_bwd(t, labels, d, out_dtype=torch.float32) * dt).to(BF)


def _gh_bound_any(ref):
    """gh bound with a CPU GEMM's accumulation (any order) in place of the MFMA chain."""
    V = ref.gw_ref.shape[0]
    err = lce_bounds.gamma_any(V) * 1.02 * ref.gh_S + 1.02 * ref.gh_D
    return err + 0.5 * lce_bounds.bf16_ulp(ref.gh_ref.abs().float() + err) + lce_bounds.TINY


def _gw_bound_any(ref):
    N = ref.gh_ref.shape[0]
    err = lce_bounds.gamma_any(N) * 1.02 * ref.gw_S + 1.02 * ref.gw_D
    return err + 0.5 * lce_bounds.bf16_ulp(ref.gw_ref.abs().float() + err) + lce_bounds.TINY


@pytest.mark.parametrize("xf,reduction", [({}, "mean"), ({}, "sum"),
                                          (dict(softcap=3.0, scale=0.8, temperature=1.3), "none"),
                                          (dict(temperature=0.7), "none")])
def test_reference_agrees_with_the_oracle(xf, reduction):
    h, w, labels = _inputs()
    dloss = torch.randn(h.shape[0]) if reduction == "none" else None
    okw = dict(logit_softcapping=xf.get("softcap", 0.0), logit_scaling=xf.get("scale", 0.0),
               temperature=xf.get("temperature", 1.0))
    loss, gh, gw, rows, lse = oracle.linear_ce(h, w, labels, reduction=reduction,
                                               bf16_logits=True, return_rows=True, dloss=dloss,
                                               **okw)
    dk = oracle_dlogits(h, w, labels, reduction, dloss, **xf)
    ref = lce_bounds.reference(h, w, labels, dk, reduction=reduction, dloss=dloss,
                               token_chunk=64, **xf)
    assert ref.d_beyond == 0
    assert ref.d_changed <= ref.d_total // 100
    torch.testing.assert_close(ref.loss_rows, rows, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(ref.lse, lse, rtol=1e-6, atol=1e-6)
    # the oracle's gradients (fp32 GEMMs of its dlogits, rounded once) lie within the bound
    lce_bounds.assert_within(gh, ref.gh_ref, _gh_bound_any(ref), "oracle grad_hidden")
    lce_bounds.assert_within(gw, ref.gw_ref, _gw_bound_any(ref), "oracle grad_weight")


def test_planted_mistakes_are_rejected():
    h, w, labels = _inputs(seed=1)
    loss, gh, gw = oracle.linear_ce(h, w, labels, bf16_logits=True)
    dk = oracle_dlogits(h, w, labels)
    # a dlogit off by 3%
    bad = dk.clone()
    r, c = 5, int(labels[5]) if labels[5] >= 0 else 0
    bad[r, c] = (bad[r, c].float() * 1.03).to(BF)
    assert lce_bounds.reference(h, w, labels, bad, token_chunk=64).d_beyond >= 1
    ref = lce_bounds.reference(h, w, labels, dk, token_chunk=64)
    bh, bw = _gh_bound_any(ref), _gw_bound_any(ref)
    # two swapped 32 x 32 blocks
    lce_bounds.assert_block_swap_rejected(gh, ref.gh_ref, bh, "grad_hidden")
    lce_bounds.assert_block_swap_rejected(gw, ref.gw_ref, bw, "grad_weight")
    # a 5% scale error
    assert lce_bounds.beyond((gh.float() * 1.05).to(BF), ref.gh_ref, bh) > 0
    assert lce_bounds.beyond((gw.float() * 1.05).to(BF), ref.gw_ref, bw) > 0
    # the label column shifted by one
    lab2 = torch.where(labels >= 0, (labels + 1) % w.shape[0], labels)
    _, gh2, gw2 = oracle.linear_ce(h, w, lab2, bf16_logits=True)
    assert lce_bounds.beyond(gh2, ref.gh_ref, bh) > 0
    assert lce_bounds.beyond(gw2, ref.gw_ref, bw) > 0


def test_running_sum_bounds():
    """A bf16 (and an fp32) running sum of grad_weight over token chunks, formed on the
    CPU from the oracle's dlogits, lies within the running-sum bounds; the bf16 sum
    with the wrong chunk boundary is rejected somewhere."""
    h, w, labels = _inputs(N=256, seed=2)
    dk = oracle_dlogits(h, w, labels)
    tc = 64
    ref = lce_bounds.reference(h, w, labels, dk, token_chunk=tc)

    def run(chunk, bf16):
        acc = None
        for s in range(0, h.shape[0], chunk):
            part = dk[s:s + chunk].float().t() @ h[s:s + chunk].float()
            if acc is None:
                acc = part.to(BF) if bf16 else part
            else:
                acc = (acc.float() + part).to(BF) if bf16 else acc + part
        return acc.to(BF)

    lce_bounds.assert_within(run(tc, True), ref.gw_ref, lce_bounds.gw_bound(ref, "bf16_run"),
                             "bf16 running sum")
    lce_bounds.assert_within(run(tc, False), ref.gw_ref, lce_bounds.gw_bound(ref, "f32_run"),
                             "fp32 running sum")
    # rounding after every 16 rows instead of every 64: more roundings than the bound allows
    # (the bf16 sum of 16 chunks drifts beyond the 4-chunk bound on some element)
    drift = run(16, True)
    assert lce_bounds.beyond(drift, ref.gw_ref, lce_bounds.gw_bound(ref, "one")) > 0
