"""Writes the golden vectors in tests/golden/*.npz.

TrainScale's own tests hold no golden vectors for this path, so these are
computed here in float64 with numpy from closed forms written independently of
oracle/ (no torch ops, no shared code):

* RMSNorm: y = x / sqrt(mean(x^2) + eps) * w; the backward from the analytic
  Jacobian of that map, dx_j = sum_i dy_i * dy_i/dx_j, formed as a full matrix
  product per row (not the simplified formula the kernels use).
* RoPE: rotation as complex multiplication (x1 + i*x2) * exp(i*theta_pos);
  backward as multiplication by exp(-i*theta_pos).
* Cross-entropy: log-sum-exp in float64 via the max shift; gradient
  softmax - onehot; label smoothing as the cross-entropy against the smoothed
  target distribution (1-a)*onehot + a/V.
* Linear cross-entropy: float64 matmul followed by the above.
* Linear cross-entropy with the RL logit transforms (softcap, scale,
  temperature) and per-row upstream gradients: losses from the float64
  composition, gradients by central finite differences of
  sum_r dloss_r * loss_r (no derivative formula).
* SwiGLU: silu(g) = g / (1 + exp(-g)) and its derivative
  1/(1+e^-g) + g e^-g / (1+e^-g)^2 (the quotient rule, not the reference's
  factored form).
* Residual add + RMSNorm: h = x + r in float64, then the RMSNorm forward above
  on the unrounded h (h * rstd stored separately for the round-twice form).

Inputs are rounded to bfloat16 values (stored as float32) so every kernel
dtype sees them exactly. Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32."""
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
def rmsnorm_case(seed, rows, cols, eps, zero_row=False):
    r = rng(seed)
    x = bf16_round(r.standard_normal((rows, cols)).astype(np.float32))
    if zero_row:
        x[0] = 0.0
    w = bf16_round((1.0 + 0.02 * r.standard_normal(cols)).astype(np.float32))
    dy = bf16_round(r.standard_normal((rows, cols)).astype(np.float32))
    X, W, DY = x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64)
    ms = (X * X).mean(axis=1)
    rstd = 1.0 / np.sqrt(ms + eps)
    y = X * rstd[:, None] * W[None, :]
    dx = np.empty_like(X)
    for i in range(rows):
        # Jacobian of y_k = x_k * w_k * (mean(x^2)+eps)^(-1/2) w.r.t. x_j
        r3 = rstd[i] ** 3
        J = np.diag(W * rstd[i]) - np.outer(W * X[i], X[i]) * r3 / cols
        dx[i] = DY[i] @ J
    dw = (DY * X * rstd[:, None]).sum(axis=0)
    return dict(x=x, w=w, dy=dy, eps=np.float64(eps), y=y, rstd=rstd, dx=dx, dw=dw)


def add_rmsnorm_case(seed, rows, cols, eps):
    r = rng(seed)
    x = bf16_round(r.standard_normal((rows, cols)).astype(np.float32))
    res = bf16_round(r.standard_normal((rows, cols)).astype(np.float32))
    w = bf16_round((1.0 + 0.02 * r.standard_normal(cols)).astype(np.float32))
    H = x.astype(np.float64) + res.astype(np.float64)
    rstd = 1.0 / np.sqrt((H * H).mean(axis=1) + eps)
    hn = H * rstd[:, None]
    return dict(x=x, r=res, w=w, eps=np.float64(eps), h=H, rstd=rstd, hn=hn,
                y=hn * w.astype(np.float64)[None, :])


# ---------------------------------------------------------------------------
def rope_case(seed, B, S, H, D, theta, positions, interleaved):
    r = rng(seed)
    x = bf16_round(r.standard_normal((B, S, H, D)).astype(np.float32))
    g = bf16_round(r.standard_normal((B, S, H, D)).astype(np.float32))
    inv = (1.0 / (theta ** (np.arange(0, D, 2, dtype=np.float64) / D)))
    ang = positions[:, :, None].astype(np.float64) * inv[None, None, :]  # [B,S,D/2]
    rot = np.exp(1j * ang)[:, :, None, :]
    X, G = x.astype(np.float64), g.astype(np.float64)
    if interleaved:
        zx = X[..., 0::2] + 1j * X[..., 1::2]
        zg = G[..., 0::2] + 1j * G[..., 1::2]
    else:
        zx = X[..., : D // 2] + 1j * X[..., D // 2:]
        zg = G[..., : D // 2] + 1j * G[..., D // 2:]
    fx = zx * rot
    bg = zg * np.conj(rot)

    def unz(z):
        if interleaved:
            out = np.empty(z.shape[:-1] + (D,))
            out[..., 0::2] = z.real
            out[..., 1::2] = z.imag
            return out
        return np.concatenate([z.real, z.imag], axis=-1)

    return dict(x=x, g=g, positions=positions.astype(np.int64), theta=np.float64(theta),
                interleaved=np.int64(interleaved), fwd=unz(fx), bwd=unz(bg))


# ---------------------------------------------------------------------------
def swiglu_case(seed, n, std):
    r = rng(seed)
    g = bf16_round((std * r.standard_normal(n)).astype(np.float32))
    g[:6] = np.array([0.0, -1.0, 1.0, -30.0, 30.0, -100.0], dtype=np.float32)
    u = bf16_round(r.standard_normal(n).astype(np.float32))
    d = bf16_round(r.standard_normal(n).astype(np.float32))
    G, U, D = g.astype(np.float64), u.astype(np.float64), d.astype(np.float64)
    e = np.exp(-G)
    silu = G / (1.0 + e)
    dsilu = 1.0 / (1.0 + e) + G * e / (1.0 + e) ** 2
    return dict(gate=g, up=u, dout=d, silu=silu, dgate=D * U * dsilu, dup=D * silu)


# ---------------------------------------------------------------------------
def ce_case(seed, N, V, ignore, smoothing=0.0, scale=0.0, softcap=0.0, std=2.0):
    r = rng(seed)
    x = bf16_round((std * r.standard_normal((N, V))).astype(np.float32))
    labels = r.integers(0, V, N).astype(np.int64)
    labels[ignore] = -100
    X = x.astype(np.float64)
    Z = X.copy()
    if scale != 0.0:
        Z = scale * Z
    if softcap != 0.0:
        T = np.tanh(Z / softcap)
        Z = softcap * T
    m = Z.max(axis=1)
    lse = m + np.log(np.exp(Z - m[:, None]).sum(axis=1))
    P = np.exp(Z - lse[:, None])
    valid = labels != -100
    loss = np.zeros(N)
    target = np.full((N, V), smoothing / V)
    for i in range(N):
        if valid[i]:
            target[i, labels[i]] += 1.0 - smoothing
            loss[i] = -(target[i] * (Z[i] - lse[i])).sum()
    n_valid = max(int(valid.sum()), 1)
    dl = 1.0 / n_valid
    grad = (P - target) * dl
    if softcap != 0.0:
        grad = grad * (1.0 - T * T)
    if scale != 0.0:
        grad = grad * scale
    grad[~valid] = 0.0
    return dict(logits=x, labels=labels, smoothing=np.float64(smoothing), scale=np.float64(scale),
                softcap=np.float64(softcap), loss=loss, lse=lse, grad=grad,
                mean_loss=np.float64(loss.sum() / n_valid))


def linear_ce_case(seed, N, H, V, ignore):
    r = rng(seed)
    h = bf16_round(r.standard_normal((N, H)).astype(np.float32))
    w = bf16_round((0.1 * r.standard_normal((V, H))).astype(np.float32))
    labels = r.integers(0, V, N).astype(np.int64)
    labels[ignore] = -100
    Hh, W = h.astype(np.float64), w.astype(np.float64)
    Z = Hh @ W.T
    m = Z.max(axis=1)
    lse = m + np.log(np.exp(Z - m[:, None]).sum(axis=1))
    valid = labels != -100
    n_valid = max(int(valid.sum()), 1)
    loss_rows = np.where(valid, lse - Z[np.arange(N), np.clip(labels, 0, None)], 0.0)
    G = np.exp(Z - lse[:, None])
    G[np.arange(N)[valid], labels[valid]] -= 1.0
    G[~valid] = 0.0
    G /= n_valid
    return dict(hidden=h, weight=w, labels=labels, loss=np.float64(loss_rows.sum() / n_valid),
                grad_hidden=G @ W, grad_weight=G.T @ Hh)


def linear_ce_rl_case(seed, N, H, V, ignore, softcap, scale, temperature):
    """Per-token losses (-log-probs) under the RL logit transforms of
    selective_log_softmax (softcap, then scale, then temperature) with per-row
    upstream gradients; the gradients of sum_r dloss_r * loss_r are central
    finite differences in float64, so no derivative formula is assumed."""
    r = rng(seed)
    h = bf16_round(r.standard_normal((N, H)).astype(np.float32))
    w = bf16_round((0.3 * r.standard_normal((V, H))).astype(np.float32))
    labels = r.integers(0, V, N).astype(np.int64)
    labels[ignore] = -100
    dloss = r.standard_normal(N)
    valid = labels != -100
    Hh, W = h.astype(np.float64), w.astype(np.float64)

    def rows(Hm, Wm):
        T = softcap * np.tanh((Hm @ Wm.T) / softcap) * scale / temperature
        m = T.max(axis=1)
        lse = m + np.log(np.exp(T - m[:, None]).sum(axis=1))
        return np.where(valid, lse - T[np.arange(N), np.clip(labels, 0, None)], 0.0), lse

    def f(Hm, Wm):
        return float((dloss * rows(Hm, Wm)[0]).sum())

    def fd(X, other_first):
        G = np.zeros_like(X)
        step = 1e-6
        for idx in np.ndindex(*X.shape):
            Xp, Xm = X.copy(), X.copy()
            Xp[idx] += step
            Xm[idx] -= step
            fp = f(Xp, W) if other_first else f(Hh, Xp)
            fm = f(Xm, W) if other_first else f(Hh, Xm)
            G[idx] = (fp - fm) / (2 * step)
        return G

    loss_rows, lse = rows(Hh, W)
    return dict(hidden=h, weight=w, labels=labels, dloss=dloss, softcap=np.float64(softcap),
                scale=np.float64(scale), temperature=np.float64(temperature),
                loss_rows=loss_rows, lse=lse, grad_hidden=fd(Hh, True), grad_weight=fd(W, False))


def main():
    cases = {}
    cases["rmsnorm_64"] = rmsnorm_case(10, 4, 64, 1e-6, zero_row=True)
    cases["rmsnorm_4096"] = rmsnorm_case(11, 3, 4096, 1e-6)
    cases["rmsnorm_100"] = rmsnorm_case(12, 5, 100, 1e-5)  # not a multiple of 8
    cases["add_rmsnorm_4096"] = add_rmsnorm_case(13, 3, 4096, 1e-6)
    cases["add_rmsnorm_72"] = add_rmsnorm_case(14, 4, 72, 1e-5)
    pos_seq = np.tile(np.arange(7), (2, 1))
    pos_packed = np.array([[0, 1, 2, 0, 1, 0, 1, 2, 3, 4, 5, 6, 0]])
    cases["rope_neox_seq"] = rope_case(20, 2, 7, 3, 16, 10000.0, pos_seq, False)
    cases["rope_inter_seq"] = rope_case(21, 2, 7, 3, 16, 10000.0, pos_seq, True)
    cases["rope_neox_packed"] = rope_case(22, 1, 13, 2, 128, 500000.0, pos_packed, False)
    cases["rope_neox_far"] = rope_case(23, 1, 4, 2, 128, 500000.0,
                                       np.array([[0, 1, 2047, 4095]]), False)
    cases["ce_plain"] = ce_case(30, 6, 256, ignore=[2])
    cases["ce_odd_v"] = ce_case(31, 5, 37, ignore=[0, 4])
    cases["ce_smooth"] = ce_case(32, 4, 128, ignore=[1], smoothing=0.1)
    cases["ce_softcap_scale"] = ce_case(33, 4, 96, ignore=[], scale=0.5, softcap=3.0, std=4.0)
    cases["linear_ce"] = linear_ce_case(40, 6, 32, 50, ignore=[3])
    cases["linear_ce_rl"] = linear_ce_rl_case(41, 6, 32, 48, ignore=[2], softcap=3.0, scale=0.8,
                                              temperature=0.7)
    cases["swiglu"] = swiglu_case(50, 4096, 3.0)
    for name, arrays in cases.items():
        np.savez(OUT / f"{name}.npz", **arrays)
    print(f"wrote {len(cases)} golden cases to {OUT}")


if __name__ == "__main__":
    main()
