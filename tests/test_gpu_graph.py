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


def _capture(gpu, step):
    """Warm up on a side stream, then capture step() into a graph; returns (graph, outs)."""
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    return graph, outs


@pytest.mark.parametrize("schedule", ["one_call", "two_pass", "stored_logits"])
def test_linear_ce_in_graph_matches_eager(gpu, schedule):
    """The fused linear CE captured and replayed: the one-call schedule in two token
    chunks with grad_weight summed in its bf16 output (the running sum starts from the
    first chunk's GEMM, not from memory that must be cleared), the two-pass schedule
    with the RL transforms and per-row upstream gradients, and the stored-logits one.
    N, H and V are off the 16-byte vector (the wrapper pads); four replays with new
    inputs in between, each equal to eager calls bit for bit."""
    from trainscale_amd.loss.linear_ce import (linear_ce_backward, linear_ce_forward,
                                               linear_ce_forward_backward)
    g = torch.Generator(device=gpu).manual_seed(5)
    N, H, V = 517, 100, 4099
    h = torch.randn(N, H, device=gpu, generator=g).to(BF)
    w = (0.1 * torch.randn(V, H, device=gpu, generator=g)).to(BF)
    labels = torch.randint(0, V, (N,), device=gpu, generator=g)
    labels[::9] = -100
    dloss = torch.rand(N, device=gpu, generator=g) - 0.3
    xf = dict(logit_softcapping=30.0, logit_scaling=0.9, temperature=0.8)

    def step():
        if schedule == "one_call":
            loss, rows, lse, gh, gw = linear_ce_forward_backward(h, w, labels,
                                                                 grad_weight_accum="bf16")
            return [loss, rows, lse, gh, gw]
        keep = schedule == "stored_logits"
        out = linear_ce_forward(h, w, labels, reduction="none", keep_logits=keep, **xf)
        gh, gw = linear_ce_backward(h, w, labels, out[2], dloss, reduction="none",
                                    logits=out[3] if keep else None, **xf)
        return [out[1], out[2], gh, gw]

    graph, outs = _capture(gpu, step)
    for rep in range(4):
        h.copy_(torch.randn(N, H, device=gpu, generator=g).to(BF))
        w.copy_((0.1 * torch.randn(V, H, device=gpu, generator=g)).to(BF))
        dloss.copy_(torch.rand(N, device=gpu, generator=g) - 0.3)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        ref = step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), (schedule, rep, i)
