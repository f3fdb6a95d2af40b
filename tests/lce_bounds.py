"""Element-wise parity bounds for the fused linear cross-entropy (test infrastructure).

The reference arithmetic is oracle.linear_ce's: logits bf16(h @ w.T) formed in fp32
(the reference's bf16 matmul, rl_training.py:177), the logit transforms of
rl_training.py:114-122, an fp32 softmax, and dlogits rounded to bf16 as autograd hands
them to the matmul's backward. `reference` runs that arithmetic chunk by chunk of token
rows on the tensors' own device, so the full C5 shape fits, and takes the reference's
gradient GEMMs in float64. Every bound below follows from the arithmetic of the kernel
and of the reference; none is a tolerance chosen to pass.

Two facts carry the bounds:

* A dot product of K terms summed in fp32, in any order, with one rounding per addition
  (any rounding mode, unit roundoff U = 2^-23), is within (K - 1) U sum|terms| of the
  exact sum (first order; the factor 1.01 covers the rest). Products of two bf16 values
  are exact in fp32. The kernel's dot products are chains of
  v_mfma_f32_32x32x16_bf16, each adding 16 exact products to the accumulator; however
  the matrix core orders those 17 terms, an MFMA contributes at most 16 U times their
  absolute sum, so a K-deep product is within (ceil(K / 16) + 16) U sum|terms|.
* Rounding to bf16 to nearest moves a value by at most half its bf16 ulp.

The gradients are then bounded element by element as
    |g_kernel - G(d_ref)| <= gamma * (|d_kernel| @ |B|) + (|d_kernel - d_ref| @ |B|)
                             + intermediate roundings + 1/2 ulp_bf16 of the result,
where G(d_ref) is the float64 GEMM of the reference's bf16 dlogits and d_kernel are the
kernel's own dlogits. Using the actual difference |d_kernel - d_ref| keeps the bound
tight; d_kernel itself is held element by element to a bound U_d derived from the
logits' accumulation (`reference` counts the elements beyond it).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

U = 2.0 ** -23            # unit roundoff of one fp32 operation, any rounding mode
EPS_P = 2.0 ** -16        # relative: the fp32 exp/fma/tanh/product chain of one probability
EPS_LSE = 2.0 ** -14      # absolute: an fp32 log-sum-exp whose summation depth is <= 1024
TINY = 1e-36              # values the GPU flushes below the normal range
SOFTCAP_D2 = 4.0 / (3.0 * math.sqrt(3.0))  # max |d/dx (1 - tanh(x)^2)| = max 2 tanh sech^2


def bf16_ulp(x: Tensor) -> Tensor:
    """Spacing of bf16 values at |x| (8 significant bits); 2^-133 below the normal range."""
    x = x.abs()
    e = torch.frexp(x.clamp(min=2.0 ** -126))[1]
    return torch.ldexp(torch.ones_like(x), e - 8)


def gamma_mfma(k: int) -> float:
    """Relative accumulation bound of a k-deep dot product on the kernel's MFMA chain."""
    return 1.01 * (math.ceil(k / 16) + 16) * U


def gamma_any(k: int) -> float:
    """Relative accumulation bound of a k-term fp32 sum in any order."""
    return 1.01 * max(k - 1, 1) * U


@dataclass
class Reference:
    loss_rows: Tensor      # fp32 [N] (0 on ignored rows), the oracle's arithmetic
    lse: Tensor            # fp32 [N]
    row_bound: Tensor      # fp32 [N]: |loss_kernel - loss_ref| allowed from the logits' rounding
    d_beyond: int          # elements of d_kernel outside U_d (must be 0)
    d_changed: int         # elements where d_kernel != d_ref
    d_total: int
    gh_ref: Tensor         # fp64 [N, H] = d_ref @ W
    gh_S: Tensor           # fp32 [N, H] = |d_kernel| @ |W|
    gh_D: Tensor           # fp32 [N, H] = |d_kernel - d_ref| @ |W|
    gw_ref: Tensor         # fp64 [V, H] = d_ref^T @ h
    gw_S: Tensor           # fp32 [V, H]
    gw_D: Tensor           # fp32 [V, H]
    gw_err_bf16_run: Tensor  # fp32 [V, H]: error of a bf16 running sum over token chunks
    gw_err_f32_run: Tensor   # fp32 [V, H]: error of an fp32 running sum over token chunks
    token_chunk: int


def _xform(z: Tensor, softcap: float, scale: float, temperature: float):
    """(t, dt/dz) in rl_training.py:114-122's order, as oracle.rl_logit_xform."""
    t = z
    d = torch.ones_like(z)
    if softcap > 0:
        th = torch.tanh(z / softcap)
        t = softcap * th
        d = 1 - th * th
    if scale > 0:
        t = t * scale
        d = d * scale
    if temperature != 1.0:
        t = t / temperature
        d = d / temperature
    return t, d


@torch.no_grad()
def reference(h: Tensor, w: Tensor, labels: Tensor, d_kernel: Tensor, *, ignore_index: int = -100,
              reduction: str = "mean", dloss: Optional[Tensor] = None, softcap: float = 0.0,
              scale: float = 0.0, temperature: float = 1.0, token_chunk: int = 2048) -> Reference:
    """The reference composition over token chunks of `token_chunk` rows, with the bound
    terms of each gradient. d_kernel: the kernel's bf16 dlogits [N, V] for the same
    reduction, upstream gradient and transforms (what ts_flce_backward_kept leaves in the
    logits it was handed). token_chunk must equal the kernel's token chunk for the
    running-sum error terms to apply to it."""
    prev_tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False  # fp32 GEMMs in fp32
    try:
        return _reference(h, w, labels.reshape(-1), d_kernel, ignore_index, reduction, dloss,
                          softcap, scale, temperature, token_chunk)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev_tf32


def _reference(h, w, labels, dk, ignore_index, reduction, dloss, softcap, scale, temperature,
               tc):
    dev = h.device
    N, H = h.shape
    V = w.shape[0]
    assert dk.shape == (N, V) and dk.dtype == torch.bfloat16
    valid = labels != ignore_index
    n_valid = max(int(valid.sum()), 1)
    up = torch.ones((), device=dev) if dloss is None else dloss.float().reshape(-1).to(dev)
    if reduction == "none":
        ds = up.expand(N) if up.numel() == 1 else up
    else:
        ds = (up.reshape(()) * (1.0 / n_valid if reduction == "mean" else 1.0)).expand(N)
    ds = torch.where(valid, ds, torch.zeros_like(ds)).float()
    mul = (scale if scale > 0 else 1.0) / temperature
    w32, aw = w.float(), w.float().abs()
    w64 = w.double()
    g_acc = gamma_mfma(H) + gamma_any(H)  # kernel logits vs reference logits (both fp32 sums)

    loss_rows = torch.empty(N, dtype=torch.float32, device=dev)
    lse_all = torch.empty(N, dtype=torch.float32, device=dev)
    row_bound = torch.empty(N, dtype=torch.float32, device=dev)
    gh_ref = torch.empty((N, H), dtype=torch.float64, device=dev)
    gh_S = torch.empty((N, H), dtype=torch.float32, device=dev)
    gh_D = torch.empty((N, H), dtype=torch.float32, device=dev)
    gw_ref = torch.zeros((V, H), dtype=torch.float64, device=dev)
    gw_S = torch.zeros((V, H), dtype=torch.float32, device=dev)
    gw_D = torch.zeros((V, H), dtype=torch.float32, device=dev)
    err_b = torch.zeros((V, H), dtype=torch.float32, device=dev)
    err_f = torch.zeros((V, H), dtype=torch.float32, device=dev)
    d_beyond = d_changed = 0
    for c, s in enumerate(range(0, N, tc)):
        e = min(s + tc, N)
        hc = h[s:e]
        lab = labels[s:e]
        vc = valid[s:e]
        rows = torch.arange(e - s, device=dev)
        lab_c = lab.clamp(min=0, max=V - 1)
        # logits: bf16 of an fp32 sum (the reference's bf16 matmul); the kernel forms the same
        # exact sum in another order, so the two bf16 values are within bz of each other
        acc = hc.float() @ w32.t()
        z = acc.to(torch.bfloat16).float()
        del acc
        Sz = hc.float().abs() @ aw.t()
        a = g_acc * 1.02 * Sz
        del Sz
        bz = a + 2 * bf16_ulp(z.abs() + a)
        del a
        t, dt = _xform(z, softcap, scale, temperature)
        lse = torch.logsumexp(t, dim=1)
        p = torch.exp(t - lse[:, None])
        tgt = t[rows, lab_c]
        loss_rows[s:e] = torch.where(vc, lse - tgt, torch.zeros_like(lse))
        lse_all[s:e] = lse
        # the transforms themselves round in fp32 (and tanh differs between libraries by a
        # few ulps): 8 U |t| on t, 8 U mul absolute on the cancelling 1 - tanh^2
        bt = mul * bz + 8 * U * t.abs()
        blse = (p * torch.expm1(bt)).sum(1) + EPS_LSE
        row_bound[s:e] = torch.where(vc, blse + bt[rows, lab_c], torch.zeros_like(blse))
        # dlogits: ds * (p - onehot) * dt/dz, rounded to bf16
        onehot = torch.zeros_like(p)
        onehot[rows[vc], lab[vc]] = 1.0
        pm = p - onehot
        g_pre = pm * ds[s:e, None] * dt
        d_ref = g_pre.to(torch.bfloat16)
        # U_d: how far the kernel's dlogits may lie from d_ref given |z_k - z_r| <= bz
        bp = p * torch.expm1(bt + blse[:, None] + EPS_P)
        bdt = ((mul * SOFTCAP_D2 / softcap) * bz + 8 * U * mul if softcap > 0
               else torch.zeros_like(bz))
        bg = ds[s:e, None].abs() * (bp * (dt.abs() + bdt) + pm.abs() * (bdt + EPS_P * dt.abs()))
        ud = (bg + bf16_ulp(g_pre.abs() + bg)) * (1 + 2.0 ** -10) + TINY
        del t, dt, p, onehot, pm, g_pre, bz, bt, bp, bdt, bg, z
        dkc = dk[s:e]
        diff = (dkc.float() - d_ref.float()).abs()
        d_beyond += int((diff > ud).sum())
        d_changed += int((diff != 0).sum())
        del ud
        adk = dkc.float().abs()
        d64 = d_ref.double()
        # grad_hidden rows of this chunk: one GEMM over all of V
        gh_ref[s:e] = d64 @ w64
        gh_S[s:e] = adk @ aw
        gh_D[s:e] = diff @ aw
        # grad_weight: this chunk's term
        h64, ah = hc.double(), hc.float().abs()
        E = d64.t() @ h64
        del d64
        S_c = adk.t() @ ah
        D_c = diff.t() @ ah
        del adk, diff
        gw_ref += E
        del E
        gw_S += S_c
        gw_D += D_c
        step = gamma_mfma(e - s) * 1.02 * S_c + 1.02 * D_c + 2.0 ** -40 * S_c
        del S_c, D_c
        P = gw_ref.abs().float()
        # bf16 running sum (TS_FLCE_ACCUM_BF16): chunk 0 rounded to bf16; then
        # bf16(fp32(old + acc)) per chunk
        err_b += step
        if c > 0:
            err_b += U * (P + err_b)
        err_b += 0.5 * bf16_ulp(P + err_b)
        # fp32 running sum: fp32 adds, one bf16 rounding at the end (left to the check)
        err_f += step
        if c > 0:
            err_f += U * (P + err_f)
        del P, step
    return Reference(loss_rows, lse_all, row_bound, d_beyond, d_changed, N * V, gh_ref, gh_S,
                     gh_D, gw_ref, gw_S, gw_D, err_b, err_f, tc)


def gh_bound(ref: Reference, vocab_chunks: int = 1) -> Tensor:
    """grad_hidden formed as one K = V GEMM per token row (vocab_chunks = 1), or summed in
    fp32 over vocab_chunks GEMMs and rounded once (the two-pass backward)."""
    V = ref.gw_ref.shape[0]
    g = gamma_mfma(V) + 17 * U * vocab_chunks
    err = g * 1.02 * ref.gh_S + 1.02 * ref.gh_D * (1 + U * vocab_chunks) + 2.0 ** -40 * ref.gh_S
    return err + 0.5 * bf16_ulp(ref.gh_ref.abs().float() + err) + TINY


def gw_bound(ref: Reference, mode: str) -> Tensor:
    """grad_weight as one K = N GEMM ("one"), a bf16 running sum over the token chunks
    ("bf16_run"), or an fp32 running sum rounded once ("f32_run")."""
    N = ref.gh_ref.shape[0]
    if mode == "one":
        err = gamma_mfma(N) * 1.02 * ref.gw_S + 1.02 * ref.gw_D + 2.0 ** -40 * ref.gw_S
        return err + 0.5 * bf16_ulp(ref.gw_ref.abs().float() + err) + TINY
    if mode == "bf16_run":
        return ref.gw_err_bf16_run + TINY
    if mode == "f32_run":
        err = ref.gw_err_f32_run
        return err + 0.5 * bf16_ulp(ref.gw_ref.abs().float() + err) + TINY
    raise ValueError(mode)


def beyond(got: Tensor, ref64: Tensor, bound: Tensor, rows: int = 16384) -> int:
    """Number of elements of got (bf16) farther than bound from the float64 reference."""
    n = 0
    for s in range(0, got.shape[0], rows):
        d = (got[s:s + rows].double() - ref64[s:s + rows]).abs()
        n += int((d > bound[s:s + rows]).sum())
    return n


def assert_within(got: Tensor, ref64: Tensor, bound: Tensor, what: str) -> None:
    assert got.shape == ref64.shape == bound.shape, (what, got.shape, ref64.shape, bound.shape)
    n = beyond(got, ref64, bound)
    if n:
        d = (got.double() - ref64).abs() / bound.double()
        idx = int(d.argmax())
        r, c = divmod(idx, got.shape[1])
        raise AssertionError(
            f"{what}: {n} elements beyond the bound; worst at ({r}, {c}): got "
            f"{got[r, c].item()!r}, reference {ref64[r, c].item()!r}, bound "
            f"{bound[r, c].item()!r}")


def assert_block_swap_rejected(got: Tensor, ref64: Tensor, bound: Tensor, what: str) -> int:
    """Swaps two 32 x 32 blocks (one MFMA tile's worth) of a copy of got and asserts that the
    comparison rejects the copy; returns how many of the 2048 moved elements it rejects."""
    R, C = got.shape
    assert R >= 64 and C >= 64, (what, got.shape)
    r0, c0 = 0, 0
    r1, c1 = (R // 64) * 32, (C // 64) * 32  # a block near the middle, whole and in range
    if (r1, c1) == (r0, c0):
        r1 = 32
    bad = got.clone()
    a = bad[r0:r0 + 32, c0:c0 + 32].clone()
    bad[r0:r0 + 32, c0:c0 + 32] = bad[r1:r1 + 32, c1:c1 + 32]
    bad[r1:r1 + 32, c1:c1 + 32] = a
    n = (beyond(bad[r0:r0 + 32], ref64[r0:r0 + 32], bound[r0:r0 + 32]) +
         beyond(bad[r1:r1 + 32], ref64[r1:r1 + 32], bound[r1:r1 + 32]))
    assert n > 0, f"{what}: a swap of two 32x32 blocks went unnoticed"
    return n
