"""Pins the CPU oracle (oracle/ops.py) before anything is checked against it.

Each oracle function is compared with formulations that do not share its code:
the float64 golden vectors (tests/golden/make_golden.py: closed forms, complex
rotation, smoothed-target cross-entropy, full-Jacobian RMSNorm backward),
torch.autograd on float64 forwards, finite differences, torch's own
F.cross_entropy, and invariants (scale/shift invariance, norm preservation,
transpose rotation, packed == per-document). The mutation tests at the end plant
plausible mistakes in the oracle's inputs/flags and check that these same
comparisons catch them.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from helpers import assert_ulp, golden, max_ulp, round_to

BF = torch.bfloat16


def t32(a):
    return torch.from_numpy(np.ascontiguousarray(a))


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["rmsnorm_64", "rmsnorm_4096", "rmsnorm_100"])
def test_rmsnorm_fwd_matches_golden(case):
    g = golden(case)
    x, w = t32(g["x"]).to(BF), t32(g["w"]).to(BF)
    y, rstd = oracle.rms_norm_fwd(x, w, float(g["eps"]))
    assert_ulp(y, round_to(g["y"], BF), 1, what=case)
    np.testing.assert_allclose(rstd.double().numpy(), g["rstd"], rtol=2e-6)


@pytest.mark.parametrize("case", ["rmsnorm_64", "rmsnorm_4096", "rmsnorm_100"])
def test_rmsnorm_bwd_matches_golden(case):
    g = golden(case)
    x, w, dy = t32(g["x"]).to(BF), t32(g["w"]).to(BF), t32(g["dy"]).to(BF)
    _, rstd = oracle.rms_norm_fwd(x, w, float(g["eps"]))
    dx, dw = oracle.rms_norm_bwd(dy, x, w, rstd)
    assert_ulp(dx, round_to(g["dx"], BF), 1, tiny=1e-4, what=case + " dx")
    assert_ulp(dw, round_to(g["dw"], BF), 1, tiny=1e-4, what=case + " dw")


def test_rmsnorm_bwd_matches_autograd_float64():
    torch.manual_seed(0)
    x = torch.randn(7, 48, dtype=torch.float64, requires_grad=True)
    w = (1 + 0.1 * torch.randn(48, dtype=torch.float64)).requires_grad_()
    dy = torch.randn(7, 48, dtype=torch.float64)
    eps = 1e-5
    y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w
    y.backward(dy)
    _, rstd = oracle.rms_norm_fwd(x.detach().float(), w.detach().float(), eps)
    dx, dw = oracle.rms_norm_bwd(dy.float(), x.detach().float(), w.detach().float(), rstd)
    torch.testing.assert_close(dx.double(), x.grad, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(dw.double(), w.grad, rtol=1e-5, atol=1e-5)


def test_rmsnorm_bwd_finite_differences():
    torch.manual_seed(1)
    x = torch.randn(2, 12, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(12, dtype=torch.float64)
    dy = torch.randn(2, 12, dtype=torch.float64)
    eps = 1e-6

    def L(xx):
        y = xx * torch.rsqrt((xx * xx).mean(-1, keepdim=True) + eps) * w
        return (y * dy).sum()

    _, rstd = oracle.rms_norm_fwd(x.float(), w.float(), eps)
    dx, _ = oracle.rms_norm_bwd(dy.float(), x.float(), w.float(), rstd)
    h = 1e-6
    for i in range(2):
        for j in range(0, 12, 3):
            e = torch.zeros_like(x)
            e[i, j] = h
            fd = (L(x + e) - L(x - e)) / (2 * h)
            assert abs(fd.item() - dx[i, j].item()) < 1e-4


def test_rmsnorm_invariants():
    torch.manual_seed(2)
    x = torch.randn(5, 64).to(BF)
    w = torch.ones(64, dtype=BF)
    y1, _ = oracle.rms_norm_fwd(x, w, 0.0)
    y2, _ = oracle.rms_norm_fwd((x.float() * 4).to(BF), w, 0.0)
    assert torch.equal(y1, y2)  # scale invariance (eps = 0, exact power-of-two scaling)
    rms = y1.float().pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones(5), atol=1e-2, rtol=0)
    z = torch.zeros(2, 64, dtype=BF)
    yz, _ = oracle.rms_norm_fwd(z, w, 1e-6)
    assert torch.count_nonzero(yz.float()) == 0


@pytest.mark.parametrize("case", ["add_rmsnorm_4096", "add_rmsnorm_72"])
def test_add_rmsnorm_matches_golden(case):
    g = golden(case)
    x, r, w = t32(g["x"]).to(BF), t32(g["r"]).to(BF), t32(g["w"]).to(BF)
    eps = float(g["eps"])
    y1, h, rstd = oracle.add_rms_norm_fwd(x, r, w, eps, round_twice=False)
    assert_ulp(y1, round_to(g["y"], BF), 1, what=case + " y once")
    assert torch.equal(h, round_to(g["h"], BF)), case + " h"
    np.testing.assert_allclose(rstd.double().numpy(), g["rstd"], rtol=2e-6)
    y2, _, _ = oracle.add_rms_norm_fwd(x, r, w, eps, round_twice=True)
    expect = (round_to(g["hn"], BF).double() * w.double()).numpy()
    assert_ulp(y2, round_to(expect, BF), 1, what=case + " y twice")
    # a plausible mistake, rstd taken from the rounded h, fails the rstd check
    hb = h.float()
    bad = 1.0 / torch.sqrt((hb * hb).sum(-1) / hb.shape[-1] + eps)
    assert not np.allclose(bad.double().numpy(), g["rstd"], rtol=2e-6, atol=0)


def test_add_rmsnorm_invariants():
    torch.manual_seed(5)
    x = torch.randn(6, 256).to(BF)
    r = torch.randn(6, 256).to(BF)
    w = (1 + 0.1 * torch.randn(256)).to(BF)
    # zero residual: plain RMSNorm with the same rounding, h == x
    y0, h0, rs0 = oracle.add_rms_norm_fwd(x, torch.zeros_like(x), w, 1e-6)
    yr, rsr = oracle.rms_norm_fwd(x, w, 1e-6, round_twice=True)
    assert torch.equal(y0, yr) and torch.equal(h0, x) and torch.equal(rs0, rsr)
    # x + r == r + x in fp32
    ya, ha, ra = oracle.add_rms_norm_fwd(x, r, w, 1e-6)
    yb, hb, rb = oracle.add_rms_norm_fwd(r, x, w, 1e-6)
    assert torch.equal(ya, yb) and torch.equal(ha, hb) and torch.equal(ra, rb)


def test_rmsnorm_round_twice_is_double_rounding():
    torch.manual_seed(3)
    x = torch.randn(64, 256).to(BF)
    w = (1 + 0.3 * torch.randn(256)).to(BF)
    y1, rstd = oracle.rms_norm_fwd(x, w, 1e-6)
    y2, _ = oracle.rms_norm_fwd(x, w, 1e-6, round_twice=True)
    expect = ((x.float() * rstd[:, None]).to(BF).float() * w.float()).to(BF)
    assert torch.equal(y2, expect)
    assert max_ulp(y1, y2) <= 1


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["rope_neox_seq", "rope_inter_seq", "rope_neox_packed",
                                  "rope_neox_far"])
def test_rope_matches_golden(case):
    g = golden(case)
    x, gr = t32(g["x"]).to(BF), t32(g["g"]).to(BF)
    pos = t32(g["positions"])
    D = x.shape[-1]
    cos, sin = oracle.rope_tables(D, int(pos.max()) + 1, float(g["theta"]))
    il = bool(g["interleaved"])
    fwd = oracle.rope_apply(x, cos, sin, pos, interleaved=il)
    bwd = oracle.rope_apply(gr, cos, sin, pos, interleaved=il, backward=True)
    assert_ulp(fwd, round_to(g["fwd"], BF), 1, what=case + " fwd")
    assert_ulp(bwd, round_to(g["bwd"], BF), 1, what=case + " bwd")


def test_rope_tables_match_float64():
    cos, sin = oracle.rope_tables(128, 4096, 500000.0)
    inv32 = oracle.rope_inv_freq(128, 500000.0).numpy()
    inv64 = 1.0 / (500000.0 ** (np.arange(0, 128, 2) / 128.0))
    np.testing.assert_allclose(inv32, inv64, rtol=3e-7)  # fp32 pow/divide of the reference
    # the reference forms the angle in fp32 (torch.outer of fp32 operands); cos/sin of
    # that fp32 angle must be accurate to fp32 rounding
    ang32 = np.arange(4096, dtype=np.float32)[:, None] * inv32[None, :]
    np.testing.assert_allclose(cos.numpy(), np.cos(ang32.astype(np.float64)), atol=2e-7)
    np.testing.assert_allclose(sin.numpy(), np.sin(ang32.astype(np.float64)), atol=2e-7)


def test_rope_invariants():
    torch.manual_seed(4)
    B, S, H, D = 2, 9, 3, 32
    x = torch.randn(B, S, H, D, dtype=torch.float64).float()
    cos, sin = oracle.rope_tables(D, 64, 10000.0)
    pos = oracle.rope_positions(B, S, position_offset=3)
    y = oracle.rope_apply(x, cos, sin, pos)
    # pair norms preserved
    n0 = x[..., :16] ** 2 + x[..., 16:] ** 2
    n1 = y[..., :16] ** 2 + y[..., 16:] ** 2
    torch.testing.assert_close(n0, n1, rtol=1e-5, atol=1e-5)
    # backward is the inverse and the transpose
    back = oracle.rope_apply(y, cos, sin, pos, backward=True)
    torch.testing.assert_close(back, x, rtol=1e-5, atol=1e-5)
    g = torch.randn_like(x)
    lhs = (y.double() * g.double()).sum()
    rhs = (x.double() * oracle.rope_apply(g, cos, sin, pos, backward=True).double()).sum()
    assert abs(lhs - rhs) < 1e-3
    # position 0 is the identity
    p0 = torch.zeros(B, S, dtype=torch.int64)
    torch.testing.assert_close(oracle.rope_apply(x, cos, sin, p0), x)


def test_rope_packed_equals_per_document():
    torch.manual_seed(5)
    lens = [5, 3, 8]
    T, H, D = sum(lens), 4, 16
    x = torch.randn(1, T, H, D).to(BF)
    pos = torch.cat([torch.arange(n) for n in lens])[None]
    cos, sin = oracle.rope_tables(D, 16, 10000.0)
    packed = oracle.rope_apply(x, cos, sin, pos)
    start = 0
    for n in lens:
        doc = x[:, start:start + n]
        ref = oracle.rope_apply(doc, cos, sin, oracle.rope_positions(1, n))
        assert torch.equal(packed[:, start:start + n], ref)
        start += n


# ---------------------------------------------------------------------------
# Cross-entropy
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", ["ce_plain", "ce_odd_v", "ce_smooth", "ce_softcap_scale"])
def test_ce_matches_golden(case):
    g = golden(case)
    x = t32(g["logits"]).to(BF)
    labels = t32(g["labels"])
    kw = dict(label_smoothing=float(g["smoothing"]), logit_scale=float(g["scale"]),
              softcap=float(g["softcap"]))
    loss, lse = oracle.ce_fwd(x, labels, **kw)
    np.testing.assert_allclose(loss.double().numpy(), g["loss"], rtol=1e-5, atol=1e-6)
    valid = g["labels"] != -100
    np.testing.assert_allclose(lse.double().numpy()[valid], g["lse"][valid], rtol=1e-6)
    n_valid = max(int(valid.sum()), 1)
    grad = oracle.ce_bwd(x, labels, torch.tensor(1.0 / n_valid), **kw)
    assert_ulp(grad, round_to(g["grad"], BF), 1, tiny=1e-30, what=case + " grad")


def test_ce_matches_torch_cross_entropy():
    torch.manual_seed(6)
    x = (2 * torch.randn(32, 1000)).to(BF)
    labels = torch.randint(0, 1000, (32,))
    labels[[3, 7]] = -100
    for a in (0.0, 0.2):
        loss, _ = oracle.ce_fwd(x, labels, label_smoothing=a)
        ref = F.cross_entropy(x.double(), labels, ignore_index=-100, reduction="none",
                              label_smoothing=a)
        torch.testing.assert_close(loss.double(), ref, rtol=1e-5, atol=1e-6)
        xr = x.double().requires_grad_()
        F.cross_entropy(xr, labels, ignore_index=-100, reduction="sum", label_smoothing=a).backward()
        grad = oracle.ce_bwd(x, labels, torch.tensor(1.0), label_smoothing=a,
                             out_dtype=torch.float32)
        torch.testing.assert_close(grad.double(), xr.grad, rtol=1e-4, atol=1e-6)


def test_ce_invariants():
    torch.manual_seed(7)
    V = 512
    x = torch.randn(8, V)
    labels = torch.randint(0, V, (8,))
    l1, _ = oracle.ce_fwd(x, labels)
    l2, _ = oracle.ce_fwd(x + 3.0, labels)
    torch.testing.assert_close(l1, l2, rtol=1e-5, atol=1e-5)
    lu, _ = oracle.ce_fwd(torch.zeros(3, V), torch.tensor([0, 5, 9]))
    torch.testing.assert_close(lu, torch.full((3,), math.log(V)), rtol=1e-6, atol=1e-6)
    g = oracle.ce_bwd(x, labels, torch.tensor(1.0), out_dtype=torch.float32)
    torch.testing.assert_close(g.sum(-1), torch.zeros(8), atol=1e-5, rtol=0)
    lab = labels.clone()
    lab[:] = -100
    lz, _ = oracle.ce_fwd(x, lab)
    assert torch.count_nonzero(lz) == 0
    gz = oracle.ce_bwd(x, lab, torch.tensor(1.0))
    assert torch.count_nonzero(gz.float()) == 0


def test_linear_ce_matches_golden():
    g = golden("linear_ce")
    h, w = t32(g["hidden"]).to(BF), t32(g["weight"]).to(BF)
    labels = t32(g["labels"])
    loss, gh, gw = oracle.linear_ce(h, w, labels)
    np.testing.assert_allclose(float(loss), float(g["loss"]), rtol=1e-5)
    assert_ulp(gh, round_to(g["grad_hidden"], BF), 1, tiny=1e-6, what="grad_hidden")
    assert_ulp(gw, round_to(g["grad_weight"], BF), 1, tiny=1e-6, what="grad_weight")


def _rl_case():
    g = golden("linear_ce_rl")
    h, w = t32(g["hidden"]).to(BF), t32(g["weight"]).to(BF)
    kw = dict(logit_softcapping=float(g["softcap"]), logit_scaling=float(g["scale"]),
              temperature=float(g["temperature"]))
    return g, h, w, t32(g["labels"]), torch.from_numpy(g["dloss"]).float(), kw


def test_linear_ce_rl_transforms_match_golden():
    """Per-token losses under softcap -> scale -> temperature with per-row upstream
    gradients, against float64 values whose gradients are finite differences."""
    g, h, w, labels, dloss, kw = _rl_case()
    rows, gh, gw, _, lse = oracle.linear_ce(h, w, labels, reduction="none", dloss=dloss,
                                            return_rows=True, **kw)
    np.testing.assert_allclose(rows.double().numpy(), g["loss_rows"], rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(lse.double().numpy(), g["lse"], rtol=2e-6, atol=2e-6)
    # gradients: bf16 outputs of fp32 arithmetic against float64 finite differences
    assert_ulp(gh, round_to(g["grad_hidden"], BF), 1, tiny=1e-5, what="grad_hidden")
    assert_ulp(gw, round_to(g["grad_weight"], BF), 1, tiny=1e-5, what="grad_weight")


def test_linear_ce_rl_mutations_fail_golden():
    """Plausible mistakes (scale applied before the softcap, a dropped tanh derivative,
    temperature multiplied instead of divided) each miss the golden vectors."""
    g, h, w, labels, dloss, kw = _rl_case()
    ref = g["loss_rows"]
    # scale before softcap (the CE kernels' order, not selective_log_softmax's)
    z = h.float() @ w.float().t()
    t = kw["logit_softcapping"] * torch.tanh(z * kw["logit_scaling"] / kw["logit_softcapping"])
    rows_bad, _ = oracle.ce_fwd(t / kw["temperature"], labels)
    assert np.abs(rows_bad.double().numpy() - ref).max() > 1e-3
    # temperature multiplied
    bad = dict(kw, temperature=1.0 / kw["temperature"])
    rows2, _, _ = oracle.linear_ce(h, w, labels, reduction="none", dloss=dloss, **bad)
    assert np.abs(rows2.double().numpy() - ref).max() > 1e-3
    # the softcap's derivative left out: d(loss)/dz without (1 - tanh^2)
    tt, d = oracle.rl_logit_xform(z, **{"logit_softcapping": kw["logit_softcapping"],
                                        "logit_scale": kw["logit_scaling"],
                                        "temperature": kw["temperature"]})
    gz = oracle.ce_bwd(tt, labels, dloss, out_dtype=torch.float32) * (
        kw["logit_scaling"] / kw["temperature"])
    gh_bad = gz @ w.float()
    assert np.abs(gh_bad.double().numpy() - g["grad_hidden"]).max() > 1e-3


def test_selective_log_softmax_matches_golden():
    """selective_log_softmax on the golden RL case's logits (float64 h @ w.T handed over
    in fp32): the log-probs are minus the golden per-token losses."""
    g, h, w, labels, dloss, kw = _rl_case()
    z = torch.from_numpy(g["hidden"]).double() @ torch.from_numpy(g["weight"]).double().t()
    valid = labels != -100
    lp = oracle.selective_log_softmax(z.float(), labels.clamp(min=0),
                                      temperature=kw["temperature"],
                                      logit_softcapping=kw["logit_softcapping"],
                                      logit_scale=kw["logit_scaling"])
    np.testing.assert_allclose(lp[valid].double().numpy(), -g["loss_rows"][valid.numpy()],
                               rtol=2e-6, atol=2e-6)
    # mutation: scale before the softcap misses the golden values
    bad = oracle.selective_log_softmax(z.float() * kw["logit_scaling"], labels.clamp(min=0),
                                       temperature=kw["temperature"],
                                       logit_softcapping=kw["logit_softcapping"])
    assert np.abs(bad[valid].double().numpy() + g["loss_rows"][valid.numpy()]).max() > 1e-3


def test_selective_log_softmax_matches_autograd_float64():
    """The log-probs and their gradient against torch's float64 log_softmax of the
    transformed logits (a separate formulation: F.log_softmax, autograd)."""
    torch.manual_seed(3)
    z = 3 * torch.randn(5, 7, 300)
    ids = torch.randint(0, 300, (5, 7))
    kw = dict(temperature=0.8, logit_softcapping=4.0, logit_scale=1.3)
    lp = oracle.selective_log_softmax(z, ids, **kw)
    z64 = z.double().requires_grad_()
    t = 4.0 * torch.tanh(z64 / 4.0) * 1.3 / 0.8
    ref = torch.gather(F.log_softmax(t, -1), -1, ids.unsqueeze(-1)).squeeze(-1)
    torch.testing.assert_close(lp.double(), ref.detach(), rtol=2e-6, atol=2e-6)
    # the gradient the kernels form: -dout * (softmax - onehot) * dt/dz
    up = torch.randn(5, 7).double()
    (ref * up).sum().backward()
    t32, dt = oracle.rl_logit_xform(z, 4.0, 1.3, 0.8)
    g = oracle.ce_bwd(t32.reshape(-1, 300), ids.reshape(-1), -up.reshape(-1).float(),
                      out_dtype=torch.float32) * dt.reshape(-1, 300)
    torch.testing.assert_close(g.double(), z64.grad.reshape(-1, 300), rtol=1e-4, atol=1e-6)


def test_linear_ce_reductions_agree():
    """mean = sum(rows) / n_valid with gradients equal to those of "none" under a
    constant upstream gradient 1 / n_valid; sum likewise with 1."""
    torch.manual_seed(11)
    N, H, V = 12, 32, 40
    h = torch.randn(N, H).to(BF)
    w = (0.2 * torch.randn(V, H)).to(BF)
    labels = torch.randint(0, V, (N,))
    labels[[1, 7]] = -100
    n_valid = N - 2
    for red, up in (("mean", 1.0 / n_valid), ("sum", 1.0)):
        loss, gh, gw = oracle.linear_ce(h, w, labels, reduction=red, logit_softcapping=5.0,
                                        temperature=1.3)
        rows, gh2, gw2 = oracle.linear_ce(h, w, labels, reduction="none",
                                          dloss=torch.full((N,), up), logit_softcapping=5.0,
                                          temperature=1.3)
        assert abs(float(loss) - float(rows.sum()) * (up if red == "mean" else 1.0)) <= 1e-6
        assert torch.equal(gh, gh2) and torch.equal(gw, gw2)


# ---------------------------------------------------------------------------
# Mutations: plausible mistakes in the oracle must fail the checks above.
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("P", [1, 3, 4])
def test_vocab_parallel_equals_full_ce(P):
    """Without smoothing every rank's loss is the full-vocabulary mean CE and the
    ranks' gradients side by side are the full gradient / n (the pinned CE oracle,
    itself checked against golden vectors and torch's cross_entropy)."""
    torch.manual_seed(P)
    n, v = 9, 60
    x = (2 * torch.randn(n, v)).to(torch.bfloat16)
    t = torch.randint(0, v, (n,))
    out = oracle.vocab_parallel_ce(list(x.split(v // P, dim=1)), t)
    full, _ = oracle.ce_fwd(x, t, ignore_index=-(1 << 40))
    g = oracle.ce_bwd(x, t, torch.tensor(1.0 / n), ignore_index=-(1 << 40), out_dtype=torch.float32)
    for loss, _ in out:
        assert abs(loss.item() - full.mean().item()) <= 1e-6 * abs(full.mean().item())
    torch.testing.assert_close(torch.cat([gp for _, gp in out], 1), g, rtol=1e-5, atol=1e-8)


def test_vocab_parallel_smoothing_follows_the_reference():
    """One rank: the loss is the standard smoothed CE; the reference's backward
    scales the softmax term by (1 - a), so its gradient is the true smoothed-CE
    gradient minus a * softmax / n. With P ranks the smoothed loss of rank p is
    the nll plus a * (lse - mean of p's shard), so two ranks differ by
    a * (mean_q - mean_p)."""
    torch.manual_seed(11)
    n, v, a = 7, 48, 0.1
    x = (3 * torch.randn(n, v)).to(torch.bfloat16)
    t = torch.randint(0, v, (n,))
    (loss, g), = oracle.vocab_parallel_ce([x], t, a)
    ref, _ = oracle.ce_fwd(x, t, ignore_index=-(1 << 40), label_smoothing=a)
    assert abs(loss.item() - ref.mean().item()) <= 1e-6 * abs(ref.mean().item())
    g_std = oracle.ce_bwd(x, t, torch.tensor(1.0 / n), ignore_index=-(1 << 40),
                          label_smoothing=a, out_dtype=torch.float32)
    soft = torch.softmax(x.double(), -1)
    torch.testing.assert_close(g.double(), g_std.double() - a * soft / n, rtol=1e-5, atol=1e-8)
    shards = list(x.split(v // 4, dim=1))
    out = oracle.vocab_parallel_ce(shards, t, a)
    means = [s.double().mean(-1) for s in shards]
    for p in range(4):
        for q in range(4):
            d = (out[p][0] - out[q][0]).item()
            assert abs(d - a * (means[q] - means[p]).mean().item()) <= 1e-5


def test_vocab_parallel_targets_outside_every_shard():
    """A target outside the vocabulary (or negative) is in no shard: the loss is the
    lse and the gradient the plain softmax / n, as the reference's masks give."""
    torch.manual_seed(5)
    n, v = 4, 32
    x = torch.randn(n, v)
    t = torch.tensor([3, v + 7, -100, v])
    out = oracle.vocab_parallel_ce(list(x.split(8, dim=1)), t)
    lse = torch.logsumexp(x.double(), -1)
    nll = lse - torch.tensor([x[0, 3].item(), 0.0, 0.0, 0.0], dtype=torch.float64)
    assert abs(out[0][0].item() - nll.mean().item()) <= 1e-5
    g = torch.cat([gp for _, gp in out], 1).double()
    soft = torch.softmax(x.double(), -1) / n
    torch.testing.assert_close(g[1:], soft[1:], rtol=1e-5, atol=1e-9)
    assert abs(g[0, 3].item() - (soft[0, 3].item() - 1.0 / n)) <= 1e-6


def test_mutation_vocab_parallel_smoothing_scale_is_caught():
    """Planted mistake (the true smoothed-CE gradient in place of the reference's
    (1 - a)-scaled softmax) fails the relation the test above checks."""
    torch.manual_seed(11)
    n, v, a = 7, 48, 0.1
    x = (3 * torch.randn(n, v)).to(torch.bfloat16)
    t = torch.randint(0, v, (n,))
    g_std = oracle.ce_bwd(x, t, torch.tensor(1.0 / n), ignore_index=-(1 << 40),
                          label_smoothing=a, out_dtype=torch.float32)
    soft = torch.softmax(x.double(), -1)
    with pytest.raises(AssertionError):
        torch.testing.assert_close(g_std.double(), g_std.double() - a * soft / n,
                                   rtol=1e-5, atol=1e-8)


def test_mutation_rope_sign_is_caught():
    g = golden("rope_neox_seq")
    x = t32(g["x"]).to(BF)
    pos = t32(g["positions"])
    cos, sin = oracle.rope_tables(16, 8, float(g["theta"]))
    wrong = oracle.rope_apply(x, cos, sin, pos, backward=True)  # sign of sin flipped
    with pytest.raises(AssertionError):
        assert_ulp(wrong, round_to(g["fwd"], BF), 1)
    wrong_layout = oracle.rope_apply(x, cos, sin, pos, interleaved=True)
    with pytest.raises(AssertionError):
        assert_ulp(wrong_layout, round_to(g["fwd"], BF), 1)


def test_mutation_rmsnorm_terms_are_caught():
    g = golden("rmsnorm_64")
    x, w, dy = t32(g["x"]).to(BF), t32(g["w"]).to(BF), t32(g["dy"]).to(BF)
    y_bad, _ = oracle.rms_norm_fwd(x, None, float(g["eps"]))  # weight dropped
    with pytest.raises(AssertionError):
        assert_ulp(y_bad, round_to(g["y"], BF), 1)
    _, rstd = oracle.rms_norm_fwd(x, w, float(g["eps"]))
    dx_bad, _ = oracle.rms_norm_bwd(dy, x, None, rstd)  # w missing from dx
    with pytest.raises(AssertionError):
        assert_ulp(dx_bad, round_to(g["dx"], BF), 1, tiny=1e-4)


def test_mutation_ce_label_is_caught():
    g = golden("ce_plain")
    x = t32(g["logits"]).to(BF)
    labels = t32(g["labels"])
    shifted = torch.where(labels >= 0, (labels + 1) % x.shape[1], labels)
    loss, _ = oracle.ce_fwd(x, shifted)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(loss.double().numpy(), g["loss"], rtol=1e-5, atol=1e-6)
    n_valid = int((labels != -100).sum())
    grad_bad = oracle.ce_bwd(x, labels, torch.tensor(1.0))  # dloss scale 1/n_valid dropped
    with pytest.raises(AssertionError):
        assert_ulp(grad_bad, round_to(g["grad"], BF), 1)
    assert n_valid > 1


def test_linear_ce_bf16_logits_mode():
    """bf16_logits restates a bf16 matmul: it agrees with torch's own bf16 matmul
    within 1 ulp, and equals the fp32 composition when the logits are exact in bf16."""
    torch.manual_seed(8)
    N, H, V = 16, 64, 40
    h = torch.randn(N, H).to(BF)
    w = (0.1 * torch.randn(V, H)).to(BF)
    labels = torch.randint(0, V, (N,))
    labels[3] = -100
    ref_logits = h @ w.t()  # torch's bf16 matmul (fp32 accumulate, bf16 result)
    ours = (h.float() @ w.float().t()).to(BF)
    assert max_ulp(ours, ref_logits) <= 1
    # exact logits: entries in {-1, 0, 1} x {0, +-0.5, +-1}, H = 16 -> multiples of 0.5 <= 16
    he = torch.randint(-1, 2, (N, 16)).float().to(BF)
    we = (torch.randint(-2, 3, (V, 16)).float() / 2).to(BF)
    a = oracle.linear_ce(he, we, labels, bf16_logits=True)
    b = oracle.linear_ce(he, we, labels, bf16_logits=False)
    assert float(a[0]) == float(b[0])
    # mean vs sum differ exactly by n_valid
    s = oracle.linear_ce(he, we, labels, reduction="sum", bf16_logits=True)
    n_valid = int((labels != -100).sum())
    assert abs(float(s[0]) - n_valid * float(a[0])) <= 1e-4 * abs(float(s[0]))


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def test_swiglu_matches_golden():
    g = golden("swiglu")
    gate, up, dout = t32(g["gate"]).to(BF), t32(g["up"]).to(BF), t32(g["dout"]).to(BF)
    # silu alone (up = 1): one rounding of the fp64 value, within 1 ulp
    silu = oracle.swiglu_fwd(gate, torch.ones_like(up))
    assert_ulp(silu, round_to(g["silu"], BF), 1, what="silu")
    # out = round(round(silu) * up): a silu rounding flip moves out by at most 2 ulps
    out = oracle.swiglu_fwd(gate, up)
    expect = round_to(g["silu"], BF).double() * up.double()
    assert_ulp(out, expect.to(BF), 2, what="out")
    dg, du = oracle.swiglu_bwd(dout, gate, up)
    # dsilu crosses zero near g = -1.28, where fp32 loses relative accuracy
    assert_ulp(dg, round_to(g["dgate"], BF), 1, tiny=1e-5, what="dgate")
    assert_ulp(du, round_to(g["dup"], BF), 1, what="dup")
    # a plausible mistake, sigmoid' in place of silu', fails the same check
    s = torch.sigmoid(gate.float())
    bad = (dout.float() * up.float() * s * (1 - s)).to(BF)
    with pytest.raises(AssertionError):
        assert_ulp(bad, round_to(g["dgate"], BF), 1, tiny=1e-5, what="mutated")


def test_swiglu_bwd_matches_autograd_float64():
    torch.manual_seed(9)
    gate = (3 * torch.randn(300, dtype=torch.float64)).requires_grad_()
    up = torch.randn(300, dtype=torch.float64).requires_grad_()
    dout = torch.randn(300, dtype=torch.float64)
    (F.silu(gate) * up).backward(dout)
    dg, du = oracle.swiglu_bwd(dout.float(), gate.detach().float(), up.detach().float())
    torch.testing.assert_close(dg.double(), gate.grad, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(du.double(), up.grad, rtol=1e-5, atol=1e-6)


def test_swiglu_invariants():
    g = torch.tensor([0.0, 40.0, -40.0, 2.0], dtype=BF)
    u = torch.tensor([5.0, 1.0, 1.0, 0.0], dtype=BF)
    out = oracle.swiglu_fwd(g, u)
    assert out[0].item() == 0.0 and out[3].item() == 0.0   # silu(0) = 0; up = 0
    assert out[1].item() == 40.0 and abs(out[2].item()) < 1e-15  # saturation


# ---------------------------------------------------------------------------
# The reference's eager sequences (oracle/eager.py, the CPU baseline) compute
# the same functions as the pinned oracle.
# ---------------------------------------------------------------------------
def test_eager_sequences_agree_with_oracle():
    from oracle import eager as E
    torch.manual_seed(12)
    x = torch.randn(16, 256).to(BF)
    w = (1 + 0.02 * torch.randn(256)).to(BF)
    dy = torch.randn(16, 256).to(BF)
    y, dx, dw = E.rmsnorm(x, w, dy)
    y_ref, rstd = oracle.rms_norm_fwd(x, w)
    dx_ref, dw_ref = oracle.rms_norm_bwd(dy, x, w, rstd)
    assert max_ulp(y, y_ref) <= 1
    # the eager backward rounds dy * w to bf16 before the products (the kernels do not)
    torch.testing.assert_close(dx.float(), dx_ref.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(dw.float(), dw_ref.float(), rtol=2e-2, atol=2e-2)
    q = torch.randn(2, 9, 4, 32).to(BF)
    k = torch.randn(2, 9, 2, 32).to(BF)
    cos, sin = oracle.rope_tables(32, 9, 10000.0)
    # fp32 tables: the products promote to fp32 (as the reference's fallback does with
    # precompute_freqs_cis's fp32 tables), rounded once here
    qo, ko, dqo, _ = (t.to(BF) for t in E.rope(q, k, q, k, cos, sin))
    pos = oracle.rope_positions(2, 9)
    assert max_ulp(qo, oracle.rope_apply(q, cos, sin, pos)) <= 1
    assert max_ulp(ko, oracle.rope_apply(k, cos, sin, pos)) <= 1
    assert max_ulp(dqo, oracle.rope_apply(q, cos, sin, pos, backward=True)) <= 1
    pid = torch.tensor([[0, 1, 2, 0, 1, 2, 3, 0, 1]] * 2)
    qp = E.rope(q, k, q, k, cos, sin, position_ids=pid)[0].to(BF)
    assert max_ulp(qp, oracle.rope_apply(q, cos, sin, pid)) <= 1
    logits = (2 * torch.randn(8, 300)).to(BF)
    labels = torch.randint(0, 300, (8,))
    labels[2] = -100
    rows, _ = oracle.ce_fwd(logits, labels)
    n_valid = 7
    for fn in (E.ce_chunked, E.ce_float):
        loss, g = fn(logits, labels) if fn is E.ce_float else fn(logits, labels, chunk_size=128)
        assert abs(float(loss) - float(rows.sum()) / n_valid) <= 1e-5
        ref_g = oracle.ce_bwd(logits, labels, torch.tensor(1.0 / n_valid))
        torch.testing.assert_close(g.float(), ref_g.float(), rtol=1e-2, atol=1e-4)
    h = torch.randn(6, 32).to(BF)
    wt = (0.1 * torch.randn(40, 32)).to(BF)
    lab = torch.randint(0, 40, (6,))
    loss, gh, gw = E.linear_ce(h, wt, lab)
    ref_loss, ref_gh, ref_gw = oracle.linear_ce(h, wt, lab, bf16_logits=True)
    assert abs(float(loss) - float(ref_loss)) <= 1e-4 * abs(float(ref_loss))
    torch.testing.assert_close(gh.float(), ref_gh.float(), rtol=2e-2, atol=2e-3)
    torch.testing.assert_close(gw.float(), ref_gw.float(), rtol=2e-2, atol=2e-3)
