"""RMSNorm kernels vs the oracle and the golden vectors (GPU).

Bar: outputs and gradients within 1 bf16 ulp of the oracle (plus the north
star's 2e-2 absolute for gradients), rstd within 1e-6 relative, dW
bit-reproducible run to run.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import assert_ulp, golden, max_ulp, round_to
from trainscale_amd import ops, workloads
from trainscale_amd.kernels import (Fast_RMS_LayerNorm, RMSLayerNormFunction, RMSNorm,
                                    rms_layernorm)

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def run_fwd_bwd(fn, x, w, dy, *args):
    xg = x.detach().clone().requires_grad_()
    wg = w.detach().clone().requires_grad_() if w is not None else None
    y = fn(xg, wg, *args)
    y.backward(dy)
    return y.detach(), xg.grad, (wg.grad if wg is not None else None)


@pytest.mark.parametrize("case", ["rmsnorm_64", "rmsnorm_4096", "rmsnorm_100"])
def test_golden(gpu, case):
    g = golden(case)
    x = torch.from_numpy(g["x"]).to(BF).to(gpu)
    w = torch.from_numpy(g["w"]).to(BF).to(gpu)
    dy = torch.from_numpy(g["dy"]).to(BF).to(gpu)
    y, dx, dw = run_fwd_bwd(Fast_RMS_LayerNorm.apply, x, w, dy, float(g["eps"]))
    assert_ulp(y, round_to(g["y"], BF), 1, what="y")
    assert_ulp(dx, round_to(g["dx"], BF), 1, tiny=1e-4, what="dx")
    assert_ulp(dw, round_to(g["dw"], BF), 1, tiny=1e-4, what="dw")


def check_against_oracle(x, w, dy, eps, round_twice=False, fn=None):
    fn = fn or (RMSLayerNormFunction.apply if round_twice else Fast_RMS_LayerNorm.apply)
    args = (eps, True) if round_twice else (eps,)
    y, dx, dw = run_fwd_bwd(fn, x, w, dy, *args)
    y_ref, rstd_ref = oracle.rms_norm_fwd(x, w, eps, round_twice=round_twice)
    dx_ref, dw_ref = oracle.rms_norm_bwd(dy, x, w, rstd_ref)
    # 16-bit outputs: 1 ulp. fp32 outputs carry rstd's summation-order error
    # (rstd itself is checked at 1e-6 relative below): 8 fp32 ulps.
    assert_ulp(y, y_ref, 1 if x.dtype != torch.float32 else 8, what="y")
    # rstd saved by the kernel
    x2d, ld = ops.as_rows(x)
    _, rstd = ops.rmsnorm_forward(x2d, ld, w, eps)
    torch.testing.assert_close(rstd.cpu(), rstd_ref, rtol=1e-6, atol=0)
    tiny = 1e-6 if x.dtype == torch.float32 else 1e-4
    assert_ulp(dx, dx_ref, 1 if x.dtype != torch.float32 else 64, tiny=tiny, what="dx")
    assert (dx.float().cpu() - dx_ref.float()).abs().max() <= 2e-2
    if w is not None:
        if w.dtype == torch.float32:
            # an fp32 column sum may cancel: bound its error by 16 fp32 ulps of the
            # sum of the absolute terms, the usual summation error bound
            xh = x.float().cpu().reshape(-1, x.shape[-1]) * rstd_ref[:, None]
            absum = (dy.float().cpu().reshape(xh.shape) * xh).abs().sum(0)
            err = (dw.float().cpu() - dw_ref.float()).abs()
            assert bool((err <= 16 * 2.0 ** -24 * absum + 1e-30).all()), float((err / absum).max())
        else:
            assert_ulp(dw, dw_ref, 1, tiny=tiny, what="dw")
        # dW sums over every row (|dW| ~ sqrt(rows)); above 4 one bf16 ulp exceeds
        # the north star's 2e-2 absolute bound, so the bound is max(2e-2, 1 ulp).
        ref = dw_ref.float()
        ulp = torch.where(ref == 0, torch.zeros_like(ref),
                          2.0 ** (torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7))
        if w.dtype != torch.bfloat16:
            ulp = torch.zeros_like(ref)
        assert bool(((dw.float().cpu() - ref).abs() <= torch.clamp(ulp, min=2e-2)).all())


def test_c1_full(gpu):
    wl = workloads.rmsnorm_workload(gpu)
    x, w, dy = wl.tensors["x"], wl.tensors["w"], wl.tensors["dy"]
    check_against_oracle(x, w, dy, 1e-6)


@pytest.mark.parametrize("cols", [8, 64, 100, 768, 4096, 5000, 8192, 12288, 16384, 20000])
@pytest.mark.parametrize("rows", [1, 37])
def test_shapes_bf16(gpu, rows, cols):
    torch.manual_seed(rows * 7 + cols)
    x = torch.randn(rows, cols, device=gpu).to(BF)
    w = (1 + 0.02 * torch.randn(cols, device=gpu)).to(BF)
    dy = torch.randn(rows, cols, device=gpu).to(BF)
    check_against_oracle(x, w, dy, 1e-6)


@pytest.mark.parametrize("rows,cols", [(5, 256), (3, 512), (7, 1024), (2, 2048), (9, 200),
                                       (1, 4096)])
def test_backward_fewer_rows_than_row_slots(gpu, rows, cols):
    """Backward launches whose last workgroup has row slots past the last row.

    Up to 256 vectors a row, a backward workgroup holds several rows at a time
    (8 at 256 columns of bf16); the slots past the matrix must load nothing
    outside it. Each case is its own allocation of exactly rows x cols.
    """
    torch.manual_seed(rows * 31 + cols)
    x = torch.randn(rows, cols, device=gpu).to(BF)
    w = (1 + 0.02 * torch.randn(cols, device=gpu)).to(BF)
    dy = torch.randn(rows, cols, device=gpu).to(BF)
    check_against_oracle(x, w, dy, 1e-6)


@pytest.mark.parametrize("rows,cols,dtype,wdtype", [(5000, 2048, BF, BF), (4099, 1024, BF, BF),
                                                    (3001, 1536, BF, torch.float32),
                                                    (2049, 1024, torch.float32, torch.float32),
                                                    (1027, 520, torch.float16, torch.float16)])
def test_backward_one_wave_per_row(gpu, rows, cols, dtype, wdtype):
    """Rows of 65-256 16-byte vectors take the one-wave-per-row backward (rms_bwd_wave):
    enough rows that every wave walks several steps, and a last step with rows past
    the matrix."""
    torch.manual_seed(rows + cols)
    x = torch.randn(rows, cols, device=gpu).to(dtype)
    w = (1 + 0.1 * torch.randn(cols, device=gpu)).to(wdtype)
    dy = torch.randn(rows, cols, device=gpu).to(dtype)
    check_against_oracle(x, w, dy, 1e-5)


@pytest.mark.parametrize("dtype,wdtype", [(torch.float16, torch.float16),
                                          (torch.float32, torch.float32),
                                          (BF, torch.float32), (torch.float16, torch.float32)])
def test_dtypes(gpu, dtype, wdtype):
    torch.manual_seed(11)
    x = torch.randn(129, 1024, device=gpu).to(dtype)
    w = (1 + 0.1 * torch.randn(1024, device=gpu)).to(wdtype)
    dy = torch.randn(129, 1024, device=gpu).to(dtype)
    check_against_oracle(x, w, dy, 1e-5)


def test_round_twice(gpu):
    torch.manual_seed(12)
    x = torch.randn(513, 4096, device=gpu).to(BF)
    w = (1 + 0.3 * torch.randn(4096, device=gpu)).to(BF)
    dy = torch.randn(513, 4096, device=gpu).to(BF)
    check_against_oracle(x, w, dy, 1e-6, round_twice=True)
    y = rms_layernorm(x, w)
    y_ref, _ = oracle.rms_norm_fwd(x, w, 1e-6, round_twice=True)
    assert max_ulp(y.cpu(), y_ref) <= 1


def test_no_weight_module(gpu):
    torch.manual_seed(13)
    m = RMSNorm(2048, eps=1e-6, elementwise_affine=False)
    x = torch.randn(4, 33, 2048, device=gpu).to(BF).requires_grad_()
    y = m(x)
    y_ref, rstd = oracle.rms_norm_fwd(x.detach(), None, 1e-6)
    assert_ulp(y, y_ref, 1)
    dy = torch.randn_like(y)
    y.backward(dy)
    dx_ref, _ = oracle.rms_norm_bwd(dy, x.detach(), None, rstd)
    assert_ulp(x.grad, dx_ref, 1, tiny=1e-4)


def test_strided_input(gpu):
    torch.manual_seed(14)
    big = torch.randn(64, 3 * 4096, device=gpu).to(BF)
    x = big[:, 4096:8192]  # row stride 3*4096, unit column stride
    w = (1 + 0.02 * torch.randn(4096, device=gpu)).to(BF)
    dy = torch.randn(64, 4096, device=gpu).to(BF)
    check_against_oracle(x, w, dy, 1e-6)


def test_gemma_norm_routing_as_the_reference(gpu):
    """registry/__init__.py:1058-1077 patches GemmaRMSNorm with the plain RMSNorm kernel:
    the patched module computes x * rstd * w (w = 0 at initialisation gives zeros) where
    its own forward computes x * rstd * (1 + w). KernelPatcher does the same by default;
    skip_inexact_norms keeps the module's own forward."""
    import torch.nn as nn
    from trainscale_amd import registry

    class GemmaRMSNorm(nn.Module):
        def __init__(self, n):
            super().__init__()
            self.weight = nn.Parameter(torch.zeros(n))
            self.eps = 1e-6

        def forward(self, h):
            var = h.float().pow(2).mean(-1, keepdim=True)
            return (h.float() * torch.rsqrt(var + self.eps) * (1.0 + self.weight.float())).to(h.dtype)

    torch.manual_seed(15)
    x = torch.randn(16, 512, device=gpu).to(BF)
    own = GemmaRMSNorm(512).to(gpu)
    y_own = own(x)
    patched = GemmaRMSNorm(512).to(gpu)
    registry.KernelPatcher().patch(patched)
    y_ref, _ = oracle.rms_norm_fwd(x, patched.weight.detach(), 1e-6)
    assert_ulp(patched(x), y_ref, 1)
    assert torch.count_nonzero(patched(x)) == 0 and torch.count_nonzero(y_own) > 0
    kept = GemmaRMSNorm(512).to(gpu)
    registry.KernelPatcher(skip_inexact_norms=True).patch(kept)
    assert torch.equal(kept(x), y_own)


def test_dw_deterministic(gpu):
    wl = workloads.rmsnorm_workload(gpu, scale=0.25)
    x, w, dy = wl.tensors["x"], wl.tensors["w"], wl.tensors["dy"]
    _, _, dw1 = run_fwd_bwd(Fast_RMS_LayerNorm.apply, x, w, dy, 1e-6)
    _, _, dw2 = run_fwd_bwd(Fast_RMS_LayerNorm.apply, x, w, dy, 1e-6)
    assert torch.equal(dw1, dw2)


def test_c4_packed_rmsnorm(gpu):
    wl = workloads.packed_workload(gpu, scale=0.25)
    x, w, dy = wl.tensors["x"], wl.tensors["w"], wl.tensors["dy"]
    check_against_oracle(x, w, dy, 1e-6)


def test_empty_batch(gpu):
    x = torch.empty(0, 4096, device=gpu, dtype=BF)
    w = torch.ones(4096, device=gpu, dtype=BF)
    y, dx, dw = run_fwd_bwd(Fast_RMS_LayerNorm.apply, x, w, torch.empty_like(x), 1e-6)
    assert y.shape == (0, 4096) and dx.shape == (0, 4096)
    assert torch.count_nonzero(dw) == 0


# ---------------------------------------------------------------------------
# Fused residual add + RMSNorm
# ---------------------------------------------------------------------------
from trainscale_amd.kernels import (FusedAddRMSLayerNormFunction, FusedRMSNorm,  # noqa: E402
                                    fused_add_rms_layernorm)


@pytest.mark.parametrize("case", ["add_rmsnorm_4096", "add_rmsnorm_72"])
def test_add_golden(gpu, case):
    g = golden(case)
    x = torch.from_numpy(g["x"]).to(BF).to(gpu)
    r = torch.from_numpy(g["r"]).to(BF).to(gpu)
    w = torch.from_numpy(g["w"]).to(BF).to(gpu)
    y, h = fused_add_rms_layernorm(x, r, w, float(g["eps"]), return_residual=True)
    assert torch.equal(h.cpu(), round_to(g["h"], BF))
    expect = (round_to(g["hn"], BF).double() * w.cpu().double()).numpy()
    assert_ulp(y, round_to(expect, BF), 1, what="y")
    x2d, ld = ops.as_rows(x)
    _, _, rstd = ops.add_rmsnorm_forward(x2d, ld, r, r.shape[1], w, float(g["eps"]))
    np.testing.assert_allclose(rstd.double().cpu().numpy(), g["rstd"], rtol=1e-6)


def check_add(x, r, w, dy, eps, store=True):
    xg = x.detach().clone().requires_grad_()
    rg = r.detach().clone().requires_grad_()
    wg = w.detach().clone().requires_grad_()
    out = FusedAddRMSLayerNormFunction.apply(xg, rg, wg, eps, store)
    y, h = out
    y.backward(dy)
    y_ref, h_ref, rstd_ref = oracle.add_rms_norm_fwd(x, r, w, eps)
    assert_ulp(y, y_ref, 1 if x.dtype != torch.float32 else 8, what="y")
    if store:
        assert torch.equal(h.cpu(), h_ref)
    else:
        assert h is None
    dx_ref, _ = oracle.rms_norm_bwd(dy, h_ref, w, rstd_ref)
    tiny = 1e-6 if x.dtype == torch.float32 else 1e-4
    assert_ulp(xg.grad, dx_ref, 1 if x.dtype != torch.float32 else 64, tiny=tiny, what="dx")
    assert torch.equal(xg.grad, rg.grad)
    assert wg.grad is None  # as the reference: no weight gradient


@pytest.mark.parametrize("rows,cols", [(64, 4096), (33, 8192), (17, 72), (5, 100), (8, 64)])
def test_add_shapes(gpu, rows, cols):
    torch.manual_seed(rows * 7 + cols)
    x = torch.randn(rows, cols, device=gpu).to(BF)
    r = torch.randn(rows, cols, device=gpu).to(BF)
    w = (1 + 0.02 * torch.randn(cols, device=gpu)).to(BF)
    dy = torch.randn(rows, cols, device=gpu).to(BF)
    check_add(x, r, w, dy, 1e-6)


@pytest.mark.parametrize("dtype,wdtype", [(BF, torch.float32), (torch.float16, torch.float16),
                                          (torch.float32, torch.float32)])
def test_add_dtypes(gpu, dtype, wdtype):
    torch.manual_seed(11)
    x = torch.randn(40, 512, device=gpu).to(dtype)
    r = torch.randn(40, 512, device=gpu).to(dtype)
    w = (1 + 0.1 * torch.randn(512, device=gpu)).to(wdtype)
    dy = torch.randn(40, 512, device=gpu).to(dtype)
    check_add(x, r, w, dy, 1e-5)


def test_add_no_store_and_strided(gpu):
    torch.manual_seed(12)
    base = torch.randn(32, 2 * 1024, device=gpu).to(BF)
    x = base[:, :1024]  # row stride 2048
    r = torch.randn(32, 1024, device=gpu).to(BF)
    w = (1 + 0.02 * torch.randn(1024, device=gpu)).to(BF)
    dy = torch.randn(32, 1024, device=gpu).to(BF)
    check_add(x, r, w, dy, 1e-6, store=False)
    mod = FusedRMSNorm(1024, eps=1e-6, device=gpu, dtype=BF)
    y1 = mod(x, r)
    y2, h2 = mod(x, r, return_residual=True)
    assert torch.equal(y1, y2) and torch.equal(h2, (x.float() + r.float()).to(BF))


def test_add_c1_full(gpu):
    wl = workloads.rmsnorm_workload(gpu)
    x, w, dy = wl.tensors["x"], wl.tensors["w"], wl.tensors["dy"]
    r = torch.flip(x, dims=[0]).contiguous()
    y, h = fused_add_rms_layernorm(x, r, w, 1e-6, return_residual=True)
    sample = torch.cat([torch.arange(0, 512), torch.arange(x.shape[0] * x.shape[1] - 512,
                                                            x.shape[0] * x.shape[1])])
    x2, r2 = x.reshape(-1, x.shape[-1]), r.reshape(-1, r.shape[-1])
    y_ref, h_ref, _ = oracle.add_rms_norm_fwd(x2[sample], r2[sample], w, 1e-6)
    assert_ulp(y.reshape(-1, y.shape[-1])[sample], y_ref, 1, what="y")
    assert torch.equal(h.reshape(-1, h.shape[-1])[sample].cpu(), h_ref)


def test_c4_full_rmsnorm(gpu):
    """C4 at its full 32768 tokens x 8192 through the ops the benchmark times: y, rstd and
    dx against the oracle in row chunks on the CPU; dW against the float64 sum over all
    rows (bf16 result: within 1 ulp, or 2e-2)."""
    wl = workloads.packed_workload(gpu)
    x, w, dy = wl.tensors["x"], wl.tensors["w"], wl.tensors["dy"]
    x2d, ldx = ops.as_rows(x)
    dy2d, lddy = ops.as_rows(dy)
    y, rstd = ops.rmsnorm_forward(x2d, ldx, w, 1e-6)
    dx, dw = ops.rmsnorm_backward(dy2d, lddy, x2d, ldx, w, rstd, need_dw=True)
    wc = w.cpu()
    dw64 = torch.zeros(x.shape[1], dtype=torch.float64)
    for s in range(0, x.shape[0], 4096):
        xs, dys = x2d[s:s + 4096].cpu(), dy2d[s:s + 4096].cpu()
        y_ref, rstd_ref = oracle.rms_norm_fwd(xs, wc, 1e-6)
        assert_ulp(y[s:s + 4096], y_ref, 1, what=f"y rows {s}")
        torch.testing.assert_close(rstd[s:s + 4096].cpu(), rstd_ref, rtol=1e-6, atol=0)
        dx_ref, _ = oracle.rms_norm_bwd(dys, xs, wc, rstd_ref)
        assert_ulp(dx[s:s + 4096], dx_ref, 1, tiny=1e-4, what=f"dx rows {s}")
        dw64 += (dys.double() * (xs.double() * rstd_ref.double()[:, None])).sum(0)
    ref = dw64.float()
    ulp = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7)
    assert bool(((dw.float().cpu() - ref).abs() <= torch.clamp(ulp, min=2e-2)).all())
    assert_ulp(dw, ref.to(BF), 1, tiny=1e-4, what="dw")
