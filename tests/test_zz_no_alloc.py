"""ts_rmsnorm_bwd_noalloc (device-scratch RMSNorm backward) against ts_rmsnorm_bwd (GPU).

The no-allocation entry point runs the same kernels with the dW partials in a
static device array instead of a caller workspace, so its results must equal
the workspace entry point's bit for bit. Two calls in a row, the second with a
smaller input, check that nothing left in the shared scratch by one call leaks
into the next. The refusal of a shape beyond the scratch, which happens before any
HIP call, is tested on the CPU (tests/test_abi.py).
"""
import pytest
import torch

from trainscale_amd import _lib, ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _inputs(dev, rows, cols, seed, wdtype=BF):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).to(BF).to(dev)
    dy = torch.randn(rows, cols, generator=g).to(BF).to(dev)
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(wdtype).to(dev)
    _, rstd = ops.rmsnorm_forward(x, cols, w, 1e-6)
    return x, dy, w, rstd


def _noalloc(x, dy, w, rstd, need_dw=True):
    rows, cols = x.shape
    dev = x.device
    lib = _lib.load()
    dx = torch.empty_like(x)
    dw = torch.empty_like(w) if need_dw else None
    with torch.cuda.device(dev):
        status = lib.ts_rmsnorm_bwd_noalloc(
            _lib.ptr(dy), cols, _lib.ptr(x), cols, _lib.TS_BF16, _lib.ptr(w),
            _lib.dtype_code(w, "w"), _lib.ptr(rstd), _lib.ptr(dx), cols, _lib.ptr(dw), rows, cols,
            _lib.stream_handle(dev))
    _lib.check(status, "ts_rmsnorm_bwd_noalloc")
    return dx, dw


@pytest.mark.parametrize("shapes", [((16384, 4096), (1000, 4096)),
                                    ((32768, 8192), (333, 1000)),
                                    ((4096, 512), (64, 512))])
def test_noalloc_matches_workspace_entry_point(gpu, shapes):
    for i, (rows, cols) in enumerate(shapes):
        print(f"noalloc call {i}: rows={rows} cols={cols}", flush=True)
        x, dy, w, rstd = _inputs(gpu, rows, cols, seed=rows + cols)
        dx_ref, dw_ref = ops.rmsnorm_backward(dy, cols, x, cols, w, rstd, need_dw=True)
        dx, dw = _noalloc(x, dy, w, rstd)
        torch.cuda.synchronize()
        assert torch.equal(dx, dx_ref), (rows, cols)
        assert torch.equal(dw, dw_ref), (rows, cols)


def test_noalloc_fp32_weight_and_no_dw(gpu):
    x, dy, w, rstd = _inputs(gpu, 2048, 4096, seed=3, wdtype=torch.float32)
    dx_ref, dw_ref = ops.rmsnorm_backward(dy, 4096, x, 4096, w, rstd, need_dw=True)
    dx, dw = _noalloc(x, dy, w, rstd)
    assert torch.equal(dx, dx_ref) and torch.equal(dw, dw_ref)
    dx2, _ = _noalloc(x, dy, w, rstd, need_dw=False)
    assert torch.equal(dx2, dx_ref)


def test_noalloc_under_graph_capture(gpu):
    """The entry point captured in a HIP graph (torch.cuda.graph) after one eager call on
    the device (which looks the scratch address up); four replays with new inputs copied
    in between, each equal bit for bit to the workspace entry point on the same inputs."""
    rows, cols = 4096, 4096
    x, dy, w, rstd = _inputs(gpu, rows, cols, seed=11)
    _noalloc(x, dy, w, rstd)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dx_g, dw_g = _noalloc(x, dy, w, rstd)
    for rep in range(4):
        x2, dy2, w2, rstd2 = _inputs(gpu, rows, cols, seed=100 + rep)
        for dst, src in ((x, x2), (dy, dy2), (w, w2), (rstd, rstd2)):
            dst.copy_(src)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        dx_ref, dw_ref = ops.rmsnorm_backward(dy, cols, x, cols, w, rstd, need_dw=True)
        torch.cuda.synchronize()
        assert torch.equal(dx_g, dx_ref) and torch.equal(dw_g, dw_ref), rep
