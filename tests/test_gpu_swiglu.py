"""SwiGLU kernels vs the oracle and the golden vectors (GPU).

Bars: dgate/dup within 1 bf16 ulp of the oracle (fp32 math rounded once; near
g = -1.28, where silu' crosses zero, an absolute 1e-5 instead); out within 2
ulps, because the reference rounds silu to the data type before the product
and a 1-ulp difference there moves the product by up to 2 ulps.
"""
import pytest
import torch

import oracle
from helpers import assert_ulp, golden, round_to
from trainscale_amd import ops
from trainscale_amd.kernels import Fast_SwiGLU, swiglu_forward

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def check(gate, up, dout, what=""):
    g = gate.detach().clone().requires_grad_()
    u = up.detach().clone().requires_grad_()
    out = Fast_SwiGLU.apply(g, u)
    out.backward(dout)
    ref = oracle.swiglu_fwd(gate, up)
    dg_ref, du_ref = oracle.swiglu_bwd(dout, gate, up)
    f32 = gate.dtype == torch.float32
    assert_ulp(out, ref, 2 if not f32 else 8, tiny=1e-30, what=what + " out")
    assert_ulp(g.grad, dg_ref, 1 if not f32 else 16, tiny=1e-5, what=what + " dgate")
    assert_ulp(u.grad, du_ref, 1 if not f32 else 16, tiny=1e-30, what=what + " dup")


def test_golden(gpu):
    gd = golden("swiglu")
    gate = torch.from_numpy(gd["gate"]).to(BF).to(gpu)
    up = torch.from_numpy(gd["up"]).to(BF).to(gpu)
    dout = torch.from_numpy(gd["dout"]).to(BF).to(gpu)
    silu = ops.swiglu_forward(gate, torch.ones_like(up))
    assert_ulp(silu, round_to(gd["silu"], BF), 1, what="silu")
    out = swiglu_forward(gate, up)
    assert_ulp(out, (round_to(gd["silu"], BF).double() * up.cpu().double()).to(BF), 2, what="out")
    dg, du = ops.swiglu_backward(dout, gate, up)
    assert_ulp(dg, round_to(gd["dgate"], BF), 1, tiny=1e-5, what="dgate")
    assert_ulp(du, round_to(gd["dup"], BF), 1, what="dup")


@pytest.mark.parametrize("shape", [(4, 14336), (3, 7, 100), (8191,), (5,), (2, 2048, 1024)])
def test_shapes(gpu, shape):
    torch.manual_seed(len(shape) * 31 + shape[-1])
    gate = (3 * torch.randn(*shape, device=gpu)).to(BF)
    up = torch.randn(*shape, device=gpu).to(BF)
    dout = torch.randn(*shape, device=gpu).to(BF)
    check(gate, up, dout, str(shape))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_dtypes(gpu, dtype):
    torch.manual_seed(7)
    gate = (3 * torch.randn(64, 1000, device=gpu)).to(dtype)
    up = torch.randn(64, 1000, device=gpu).to(dtype)
    dout = torch.randn(64, 1000, device=gpu).to(dtype)
    check(gate, up, dout, str(dtype))


def test_unaligned_and_noncontiguous(gpu):
    torch.manual_seed(8)
    base = (3 * torch.randn(4097, device=gpu)).to(BF)
    gate = base[1:]  # 2-byte offset: element-wise kernels
    up = torch.randn(4096, device=gpu).to(BF)
    dout = torch.randn(4096, device=gpu).to(BF)
    check(gate, up, dout, "unaligned")
    g2 = (3 * torch.randn(64, 256, device=gpu)).to(BF).t()  # non-contiguous view
    u2 = torch.randn(256, 64, device=gpu).to(BF)
    d2 = torch.randn(256, 64, device=gpu).to(BF)
    check(g2, u2, d2, "transposed")


def test_extremes(gpu):
    gate = torch.tensor([0.0, -1.0, 1.0, -30.0, 30.0, -100.0, 100.0, -88.0], device=gpu).to(BF)
    up = torch.full((8,), 2.0, device=gpu).to(BF)
    dout = torch.ones(8, device=gpu).to(BF)
    check(gate, up, dout, "extremes")
    out = swiglu_forward(gate, up)
    assert torch.isfinite(out.float()).all()


def test_8b_shape(gpu):
    """Llama-3-8B MLP activation [8, 2048, 14336]: the first and last 2M elements."""
    torch.manual_seed(10)
    shape = (8, 2048, 14336)
    gate = (3 * torch.randn(shape, device=gpu)).to(BF)
    up = torch.randn(shape, device=gpu).to(BF)
    dout = torch.randn(shape, device=gpu).to(BF)
    out = swiglu_forward(gate, up)
    dg, du = ops.swiglu_backward(dout, gate, up)
    n = 1 << 21
    for sl in (slice(0, n), slice(gate.numel() - n, gate.numel())):
        fg, fu, fd = gate.reshape(-1)[sl], up.reshape(-1)[sl], dout.reshape(-1)[sl]
        assert_ulp(out.reshape(-1)[sl], oracle.swiglu_fwd(fg, fu), 2, what="out")
        rg, ru = oracle.swiglu_bwd(fd, fg, fu)
        assert_ulp(dg.reshape(-1)[sl], rg, 1, tiny=1e-5, what="dgate")
        assert_ulp(du.reshape(-1)[sl], ru, 1, what="dup")


def test_empty(gpu):
    e = torch.empty(0, 16, device=gpu, dtype=BF)
    assert swiglu_forward(e, e).shape == (0, 16)
    dg, du = ops.swiglu_backward(e, e, e)
    assert dg.numel() == 0 and du.numel() == 0


def test_registry_mlp_patch_on_gpu(gpu):
    from trainscale_amd import registry

    class LlamaMLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = torch.nn.Linear(64, 128, bias=False)
            self.up_proj = torch.nn.Linear(64, 128, bias=False)
            self.down_proj = torch.nn.Linear(128, 64, bias=False)

        def forward(self, x):
            return self.down_proj(torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))

    torch.manual_seed(3)
    m = LlamaMLP().to(gpu).to(BF)
    x = torch.randn(4, 16, 64, device=gpu).to(BF)
    g, u = m.gate_proj(x), m.up_proj(x)
    expect = m.down_proj(swiglu_forward(g, u))
    registry.KernelPatcher().patch(m)
    torch.testing.assert_close(m(x), expect, rtol=0, atol=0)
