"""The headline step's ops captured in a HIP graph (torch.cuda.graph) and replayed.

The library allocates nothing, never synchronises and clears memory with
kernels rather than hipMemsetAsync, so a caller can capture its launches. The
graph is replayed several times, with eager work (new inputs copied in) and
synchronisations between the replays, and every replay is compared bit for bit
with the eager result on the same inputs: a replay that kept stale state, or a
launch whose arguments were not all captured, would differ.
"""
import pytest
import torch

from trainscale_amd import ops
from trainscale_amd.kernels.rope_kernels import _base_inv_freq

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def test_step_in_graph_matches_eager(gpu):
    g = torch.Generator(device=gpu).manual_seed(21)

    def randn(*shape, scale=1.0):
        return (scale * torch.randn(*shape, device=gpu, generator=g)).to(BF)

    rows, cols = 512, 4096
    B, S, Hq, Hk, D = 2, 128, 32, 8, 128
    N, V = 256, 32000
    x, dy = randn(rows, cols), randn(rows, cols)
    w = (1 + 0.02 * torch.randn(cols, device=gpu, generator=g)).to(BF)
    q, k = randn(B, S, Hq, D), randn(B, S, Hk, D)
    dq, dk = randn(B, S, Hq, D), randn(B, S, Hk, D)
    logits = randn(N, V, scale=2.0)
    labels = torch.randint(0, V, (N,), device=gpu, generator=g)
    labels[::10] = -100
    dloss = torch.full((1,), 1.0 / int((labels != -100).sum()), device=gpu)
    upstream = torch.ones((1,), device=gpu)
    inv = _base_inv_freq(500000.0, D, "cpu")
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    dqo, dko = torch.empty_like(dq), torch.empty_like(dk)
    grad = torch.empty_like(logits)

    def step():
        # forward C1, C2, C3, then backward C3, C2, C1, as the benchmark's step
        y, rstd = ops.rmsnorm_forward(x, cols, w, 1e-6)
        ops.rope_apply(q, qo, k, ko, inv_freq=inv)
        loss, lse, _ = ops.ce_forward_backward(logits, V, labels, dloss, grad=grad)
        ops.scale_(grad, upstream)
        ops.rope_apply(dq, dqo, dk, dko, inv_freq=inv, backward=True)
        dx, dw = ops.rmsnorm_backward(dy, cols, x, cols, w, rstd, need_dw=True)
        return [y, rstd, loss, lse, dx, dw]

    def shared():
        return [qo, ko, dqo, dko, grad]

    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        step()  # warm-up off the capture, as torch.cuda.graph expects
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()

    for rep in range(4):
        for t, scale in ((x, 1.0), (dy, 1.0), (q, 1.0), (k, 1.0), (dq, 1.0), (dk, 1.0),
                         (logits, 2.0)):
            t.copy_(randn(*t.shape, scale=scale))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs + shared()]
        ref = step()
        torch.cuda.synchronize()
        ref = [o.clone() for o in ref + shared()]
        names = ["y", "rstd", "loss", "lse", "dx", "dw", "q_out", "k_out", "dq_out", "dk_out",
                 "grad"]
        for name, a, b in zip(names, got, ref):
            assert torch.equal(a, b), (rep, name)
