"""ts_rmsnorm_bwd_noalloc (device-scratch RMSNorm backward) against ts_rmsnorm_bwd (GPU).

The no-allocation entry point runs the same kernels with the dW partials in a
static device array instead of a caller workspace, so its results must equal
the workspace entry point's bit for bit. Two calls in a row, the second with a
smaller input, check that nothing left in the shared scratch by one call leaks
into the next; a shape beyond the scratch is refused before any launch.
"""
import ctypes

import pytest
import torch

from trainscale_amd import _lib, ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
TS_ERR_WORKSPACE = -4


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


def test_noalloc_rejects_shapes_beyond_the_scratch(gpu):
    lib = _lib.load()
    cap = int(lib.ts_rmsnorm_bwd_noalloc_max_bytes())
    assert cap == 16 << 20
    rows, cols = 65536, 65536  # the generic path's partials: rows / 64 x cols x 4 bytes
    assert int(lib.ts_rmsnorm_bwd_workspace_size(rows, cols)) > cap
    fake = ctypes.c_void_p(0x1000)
    status = lib.ts_rmsnorm_bwd_noalloc(fake, cols, fake, cols, _lib.TS_BF16, fake, _lib.TS_BF16,
                                        fake, fake, cols, fake, rows, cols, None)
    assert status == TS_ERR_WORKSPACE
    assert b"device scratch" in lib.ts_last_error()
