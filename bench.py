"""Benchmark of the fused kernel layer on one MI355X.

One step = forward of C1 (RMSNorm x[8,2048,4096]), C2 (RoPE Q[8,2048,32,128] +
K[8,2048,8,128], theta 500000, in-register sin/cos) and C3 (cross-entropy over
logits[16384,128256] with 10% ignored labels), then their backwards in reverse
order (C3, C2, C1), as a training step runs them. Between the forward and the
backward of one op the other ops move gigabytes, so no op re-reads its inputs
from the 256 MB last-level cache. All inputs are synthetic, seeded and resident
in HBM before timing.

value = algorithmic bytes of the step / step time (GB/s); the roofline object is
computed for the dominant kernel from HIP-event durations taken on torch's
current stream (the stream every kernel is launched on).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "achieved HBM GB/s (% of 8TB/s) for RMSNorm/RoPE/CE fwd+bwd at 8B shapes"
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="approximate CPU time budget of the baseline sample")
    p.add_argument("--copy-probe", action="store_true",
                   help="before warm-up, copy a 1 GiB buffer 3 times (a plain copy of known "
                        "size, the reference point for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


def load_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc summary."""
    f = ROOT / "profiles" / "ce_bwd_c3_pmc.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text())
    except Exception:
        return None


def cpu_baseline(budget_s: float):
    """Times the oracle (a CPU port of the reference math) on bounded samples of C1-C3."""
    import torch

    import oracle
    from trainscale_amd import workloads as W

    torch.set_num_threads(os.cpu_count() or 1)
    cores = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    rows1, tok2, rows3 = 2048, 1024, 48
    x = torch.randn(rows1, 4096, generator=g).to(bf)
    w = (1 + 0.02 * torch.randn(4096, generator=g)).to(bf)
    dy = torch.randn(rows1, 4096, generator=g).to(bf)
    q = torch.randn(1, tok2, 32, 128, generator=g).to(bf)
    k = torch.randn(1, tok2, 8, 128, generator=g).to(bf)
    cos, sin = oracle.rope_tables(128, tok2, 500000.0)
    pos = oracle.rope_positions(1, tok2)
    logits = (2 * torch.randn(rows3, 128256, generator=g)).to(bf)
    labels = torch.randint(0, 128256, (rows3,), generator=g)
    labels[::10] = -100
    n_valid = int((labels != -100).sum())

    def one():
        y, rstd = oracle.rms_norm_fwd(x, w, 1e-6)
        oracle.rms_norm_bwd(dy, x, w, rstd)
        for t in (q, k):
            oracle.rope_apply(t, cos, sin, pos)
            oracle.rope_apply(t, cos, sin, pos, backward=True)
        oracle.ce_fwd(logits, labels)
        oracle.ce_bwd(logits, labels, torch.tensor(1.0 / n_valid))

    one()  # warm-up
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 50:
            break
    times.sort()
    t = times[len(times) // 2]
    b1 = W.rmsnorm_bytes(rows1, 4096)
    b2 = W.rope_bytes(tok2, 40, 128)
    b3 = W.ce_bytes(rows3, n_valid, 128256)
    sample_bytes = sum(b1.values()) + sum(b2.values()) + sum(b3.values())
    return {
        "value": round(sample_bytes / t / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle (torch CPU fp32 restatement of the reference math) fwd+bwd on "
                   f"C1 {rows1} rows x 4096, C2 {tok2} tokens x (32+8) heads x 128, "
                   f"C3 {rows3} rows x 128256; median of {len(times)} runs, "
                   f"{t * 1e3:.1f} ms per sample; CPU {platform.processor() or platform.machine()}"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is described in DESIGN.md)"}))
        sys.exit(2)

    import torch

    from trainscale_amd import ops
    from trainscale_amd import workloads as W
    from trainscale_amd.kernels.rope_kernels import _base_inv_freq

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    c1 = W.rmsnorm_workload(dev)
    c2 = W.rope_workload(dev)
    c3 = W.ce_workload(dev)
    x, w, dy = c1.tensors["x"], c1.tensors["w"], c1.tensors["dy"]
    x2d, ldx = ops.as_rows(x)
    dy2d, lddy = ops.as_rows(dy)
    q, k, dq, dk = (c2.tensors[n] for n in ("q", "k", "dq", "dk"))
    inv_freq = _base_inv_freq(500000.0, 128, "cpu")
    q_out, k_out = torch.empty_like(q), torch.empty_like(k)
    dq_out, dk_out = torch.empty_like(dq), torch.empty_like(dk)
    logits, labels = c3.tensors["logits"], c3.tensors["labels"]
    N, V = logits.shape
    n_valid = int((labels != -100).sum())
    grad = torch.empty_like(logits)
    dloss = torch.full((1,), 1.0 / n_valid, device=dev)
    torch.cuda.synchronize()

    if args.copy_probe:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    bytes_c1 = W.rmsnorm_bytes(x2d.shape[0], x2d.shape[1])
    bytes_c2 = W.rope_bytes(q.shape[0] * q.shape[1], q.shape[2] + k.shape[2], 128)
    bytes_c3 = W.ce_bytes(N, n_valid, V)
    op_bytes = {
        "rmsnorm_fwd": bytes_c1["fwd"], "rope_fwd": bytes_c2["fwd"], "ce_fwd": bytes_c3["fwd"],
        "ce_bwd": bytes_c3["bwd"], "rope_bwd": bytes_c2["bwd"], "rmsnorm_bwd": bytes_c1["bwd"],
    }
    step_bytes = sum(op_bytes.values())
    order = list(op_bytes)
    state = {}

    def step(events=None):
        def mark(i):
            if events is not None:
                events[i].record()
        mark(0)
        state["y"], state["rstd"] = ops.rmsnorm_forward(x2d, ldx, w, 1e-6)
        mark(1)
        ops.rope_apply(q, q_out, k, k_out, inv_freq=inv_freq)
        mark(2)
        _, state["lse"] = ops.ce_forward(logits, V, labels)
        mark(3)
        ops.ce_backward(logits, V, labels, state["lse"], dloss, grad, V)
        mark(4)
        ops.rope_apply(dq, dq_out, dk, dk_out, inv_freq=inv_freq, backward=True)
        mark(5)
        ops.rmsnorm_backward(dy2d, lddy, x2d, ldx, w, state["rstd"], need_dw=True)
        mark(6)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: exactly K steps, synchronised on both sides
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(7)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(ev[s])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    per_op = {name: [] for name in order}
    for s in range(args.steps):
        for i, name in enumerate(order):
            per_op[name].append(ev[s][i].elapsed_time(ev[s][i + 1]))  # ms
    ms_step = elapsed * 1e3 / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    kernels = {}
    for name in order:
        ms = sum(per_op[name]) / len(per_op[name])
        gbs = op_bytes[name] / (ms * 1e-3) / 1e9
        kernels[name] = {"ms": round(ms, 4), "bytes": op_bytes[name], "GB_s": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}
    dom = max(order, key=lambda n: kernels[n]["ms"])
    pmc = load_traffic()
    traffic = None
    if pmc and pmc.get("kernel_op") == dom:
        traffic = pmc.get("hbm_bytes_per_launch")
    roofline = {
        "kernel": dom,
        "bound": "hbm",
        "achieved": kernels[dom]["GB_s"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": kernels[dom]["frac"],
        "traffic": traffic,
        "algorithmic_bytes": op_bytes[dom],
    }
    tokens = c1.tokens + c2.tokens + c3.tokens
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("C1 RMSNorm x[8,2048,4096] + C2 RoPE Q[8,2048,32,128]/K[8,2048,8,128] "
                         "theta 5e5 in-register + C3 CE logits[16384,128256] 10% ignored; "
                         "fwd C1,C2,C3 then bwd C3,C2,C1"),
            "step_bytes": step_bytes,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(tokens / (ms_step * 1e-3), 1),
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "kernels": kernels,
        "device": torch.cuda.get_device_name(dev),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
