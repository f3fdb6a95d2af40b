"""Benchmark of the fused kernel layer on one MI355X.

Headline step (the metric's value): forward of C1 (RMSNorm x[8,2048,4096]),
C2 (RoPE Q[8,2048,32,128] + K[8,2048,8,128], theta 500000, in-register sin/cos)
and C3 (cross-entropy over logits[16384,128256] with 10% ignored labels), then
their backwards in reverse order (C3, C2, C1), as a training step runs them.
Between the forward and the backward of one op the other ops move gigabytes,
so no op re-reads its inputs from the 256 MB last-level cache. All inputs are
synthetic, seeded and resident in HBM before timing.

value = algorithmic bytes of the step / step time (GB/s). The roofline object is
for the dominant kernel of the step, from HIP-event durations taken on torch's
current stream (the stream every kernel is launched on); its `traffic` is the
HBM bytes per launch that rocprofv3 --pmc measured (profiles/pmc_traffic.txt).

Also reported, outside the timed step: C4 (packed varlen RMSNorm + RoPE with
position_ids at 70B shapes, GB/s) and C5 (fused linear cross-entropy, TFLOP/s
against the bf16 MFMA peak), each with its own timing.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--no-extra] [--copy-probe]
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
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true", help="skip the C4 and C5 sections")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="approximate CPU time budget of the baseline sample")
    p.add_argument("--copy-probe", action="store_true",
                   help="before warm-up, copy a 1 GiB buffer 3 times (a plain copy of known "
                        "size, the reference point for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


def load_traffic():
    """{kernel: HBM bytes per launch} from the committed rocprofv3 --pmc summary."""
    f = ROOT / "profiles" / "pmc_traffic.txt"
    out = {}
    if not f.exists():
        return out
    for line in f.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == "hbm_bytes_per_launch":
            try:
                out[parts[1]] = int(parts[2])
            except ValueError:
                pass
    return out


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
        if time.perf_counter() - t_start > budget_s or len(times) >= 1000:
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
                   f"{t * 1e3:.1f} ms per sample; CPU {cpu_model()}"),
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the machine type."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline_linear_ce(budget_s: float):
    """The oracle's linear CE (fp32 matmuls + CE) on 64 tokens of C5, in TFLOP/s."""
    import torch

    import oracle

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(4)
    n, h, v = 64, 4096, 128256
    hid = torch.randn(n, h, generator=g).to(torch.bfloat16)
    wt = (0.02 * torch.randn(v, h, generator=g)).to(torch.bfloat16)
    lab = torch.randint(0, v, (n,), generator=g)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        oracle.linear_ce(hid, wt, lab, bf16_logits=True)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s or len(times) >= 100:
            break
    times.sort()
    t = times[len(times) // 2]
    flops = 3 * 2 * n * h * v
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle linear_ce fwd+bwd on 64 tokens of C5 (H 4096, V 128256); "
                      f"median of {len(times)} runs, {t:.2f} s per sample; CPU {cpu_model()}"}


def time_ms(fn, steps: int, warmup: int) -> float:
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for e0, e1 in ev:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in ev) / steps


def device_reference(dev):
    """Measured reference points of this GPU, next to the published peaks: a plain
    device-to-device copy of 1 GiB (read + write, the HIP runtime's copy kernel) and a
    large bf16 GEMM from hipBLASLt (torch.matmul, 8192^3)."""
    import torch

    nbytes = 1 << 30
    bufs = [(torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1),
             torch.empty(nbytes, dtype=torch.uint8, device=dev)) for _ in range(2)]
    it = iter(range(1 << 30))

    def copy():
        a, b = bufs[next(it) % 2]
        b.copy_(a)

    copy_ms = time_ms(copy, 10, 2)
    del bufs
    g = torch.Generator(device=dev).manual_seed(7)
    m = 8192
    a = torch.randn(m, m, device=dev, generator=g).to(torch.bfloat16)
    b = torch.randn(m, m, device=dev, generator=g).to(torch.bfloat16)
    gemm_ms = time_ms(lambda: torch.matmul(a, b), 10, 2)
    del a, b
    torch.cuda.empty_cache()
    return {"d2d_copy_GB_s": round(2 * nbytes / (copy_ms * 1e-3) / 1e9, 1),
            "d2d_copy_bytes": nbytes,
            "hipblaslt_bf16_gemm_TFLOP_s": round(2 * m ** 3 / (gemm_ms * 1e-3) / 1e12, 1),
            "gemm_shape": [m, m, m]}


def bench_packed(dev, steps: int, warmup: int):
    """C4: packed varlen RMSNorm [32768, 8192] and RoPE (64q + 8k heads) with position_ids."""
    import torch

    from trainscale_amd import ops
    from trainscale_amd import workloads as W
    from trainscale_amd.kernels.rope_kernels import _base_inv_freq

    c4 = W.packed_workload(dev)
    t = c4.tensors
    x2d, ldx = ops.as_rows(t["x"])
    dy2d, lddy = ops.as_rows(t["dy"])
    q, k, dq, dk, pos = t["q"], t["k"], t["dq"], t["dk"], t["position_ids"]
    inv = _base_inv_freq(c4.params["theta"], 128, "cpu")
    qo, ko, dqo, dko = (torch.empty_like(a) for a in (q, k, dq, dk))
    state = {}

    def norm_fwd():
        state["y"], state["rstd"] = ops.rmsnorm_forward(x2d, ldx, t["w"], 1e-6)

    norm_fwd()

    def norm_bwd():
        ops.rmsnorm_backward(dy2d, lddy, x2d, ldx, t["w"], state["rstd"], need_dw=True)

    def rope_fwd():
        ops.rope_apply(q, qo, k, ko, inv_freq=inv, position_ids=pos)

    def rope_bwd():
        ops.rope_apply(dq, dqo, dk, dko, inv_freq=inv, position_ids=pos, backward=True)

    T, Hd = x2d.shape
    nb = W.rmsnorm_bytes(T, Hd)
    rb = W.rope_bytes(T, q.shape[2] + k.shape[2], 128, pos_bytes=T * 8)
    res = {}
    for name, fn, b in (("rmsnorm_fwd", norm_fwd, nb["fwd"]), ("rmsnorm_bwd", norm_bwd, nb["bwd"]),
                        ("rope_fwd", rope_fwd, rb["fwd"]), ("rope_bwd", rope_bwd, rb["bwd"])):
        ms = time_ms(fn, steps, warmup)
        gbs = b / (ms * 1e-3) / 1e9
        res[name] = {"ms": round(ms, 4), "bytes": b, "GB_s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)}
    tot_b = sum(v["bytes"] for v in res.values())
    tot_ms = sum(v["ms"] for v in res.values())
    return {"workload": ("C4 packed varlen: 32768 tokens, docs U[64,4096], position_ids reset per "
                         "doc; RMSNorm H 8192; RoPE 64q+8k heads x 128, theta 5e5 in-register"),
            "GB_s": round(tot_b / (tot_ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(tot_b / (tot_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "ms": round(tot_ms, 4), "tokens_per_s": round(T / (tot_ms * 1e-3), 1),
            "kernels": res}


def bench_next_rows(dev, steps: int, warmup: int):
    """Rows beyond the headline step: fused residual add + RMSNorm forward at
    the C1 and C4 shapes, SwiGLU forward + backward at the Llama-3-8B MLP shape
    [8, 2048, 14336], the two-pass CE of Fast_CrossEntropyLoss at C3, and one rank's vocabulary-parallel CE kernels at C3 / 8 ranks and fused
    linear-CE phases at C5 / 8 ranks.
    Synthetic seeded inputs, each op timed alone."""
    import torch

    from trainscale_amd import ops
    from trainscale_amd import workloads as W

    g = torch.Generator(device=dev).manual_seed(5)
    res = {}
    for name, rows, cols in (("add_rmsnorm_fwd_c1", 16384, 4096),
                             ("add_rmsnorm_fwd_c4", 32768, 8192)):
        x = torch.randn(rows, cols, device=dev, generator=g).to(torch.bfloat16)
        r = torch.randn(rows, cols, device=dev, generator=g).to(torch.bfloat16)
        w = (1 + 0.02 * torch.randn(cols, device=dev, generator=g)).to(torch.bfloat16)
        ms = time_ms(lambda: ops.add_rmsnorm_forward(x, cols, r, cols, w, 1e-6), steps, warmup)
        b = W.add_rmsnorm_bytes(rows, cols)
        res[name] = {"shape": [rows, cols], "ms": round(ms, 4), "bytes": b,
                     "GB_s": round(b / (ms * 1e-3) / 1e9, 1),
                     "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del x, r, w
    shape = (8, 2048, 14336)
    gate = (3 * torch.randn(shape, device=dev, generator=g)).to(torch.bfloat16)
    up = torch.randn(shape, device=dev, generator=g).to(torch.bfloat16)
    dout = torch.randn(shape, device=dev, generator=g).to(torch.bfloat16)
    n = gate.numel()
    sb = W.swiglu_bytes(n)
    for name, fn, b in (("swiglu_fwd", lambda: ops.swiglu_forward(gate, up), sb["fwd"]),
                        ("swiglu_bwd", lambda: ops.swiglu_backward(dout, gate, up), sb["bwd"])):
        ms = time_ms(fn, steps, warmup)
        res[name] = {"shape": list(shape), "ms": round(ms, 4), "bytes": b,
                     "GB_s": round(b / (ms * 1e-3) / 1e9, 1),
                     "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del gate, up, dout
    # The reference's own CE contract at C3 (Fast_CrossEntropyLoss, schedule A): the
    # forward reads each labelled row for loss and lse; the backward reads it again
    # and writes every row's gradient. Written to a separate buffer here so that every
    # repeat sees the same logits; the bytes are those of the in-place contract.
    c3 = W.ce_workload(dev)
    logits, labels = c3.tensors["logits"], c3.tensors["labels"]
    N3, V3 = logits.shape
    n_valid = int((labels != -100).sum())
    _, lse3 = ops.ce_forward(logits, V3, labels)
    g3 = torch.empty_like(logits)
    scale3 = torch.tensor([1.0 / n_valid], device=dev)
    cb = W.ce_bytes(N3, n_valid, V3)
    for name, fn, b in (
            ("ce_fwd_schedule_a", lambda: ops.ce_forward(logits, V3, labels), cb["fwd"]),
            ("ce_bwd_schedule_a",
             lambda: ops.ce_backward(logits, V3, labels, lse3, scale3, g3, V3), cb["bwd"])):
        ms = time_ms(fn, steps, warmup)
        res[name] = {"shape": [N3, V3], "ms": round(ms, 4), "bytes": b,
                     "GB_s": round(b / (ms * 1e-3) / 1e9, 1),
                     "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del c3, logits, labels, lse3, g3
    # Vocabulary-parallel CE: one rank's kernels at C3 split over 8 ranks, a
    # [16384, 16032] bf16 shard (the merge reads 8 ranks' partials).
    N, P = 16384, 8
    vp = 128256 // P
    xs = (2 * torch.randn(N, vp, device=dev, generator=g)).to(torch.bfloat16)
    tg = torch.randint(0, 128256, (N,), device=dev, generator=g)
    st_all = ops.ce_vocab_shard_stats(xs, vp, tg, vp).unsqueeze(0).repeat(P, 1, 1).contiguous()
    lse, _ = ops.ce_vocab_merge(st_all, 1, vp)
    go = torch.ones((), device=dev)
    vb = W.vocab_shard_bytes(N, vp, P)
    for name, fn, b in (
            ("vocab_shard_stats", lambda: ops.ce_vocab_shard_stats(xs, vp, tg, vp), vb["stats"]),
            ("vocab_merge", lambda: ops.ce_vocab_merge(st_all, 1, vp), vb["merge"]),
            ("vocab_shard_bwd",
             lambda: ops.ce_vocab_shard_backward(xs, vp, tg, lse, go, 1.0 / N, vp), vb["bwd"])):
        ms = time_ms(fn, steps, warmup)
        res[name] = {"shape": [N, vp], "ranks": P, "ms": round(ms, 4), "bytes": b,
                     "GB_s": round(b / (ms * 1e-3) / 1e9, 1),
                     "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del xs, tg, st_all, lse
    # Vocabulary-parallel fused linear CE: one rank of C5 over 8 ranks, hidden
    # [8192, 4096] against an LM head shard [16032, 4096]: phase 1 (logits GEMM and
    # partials) and phase 2 (merge of 8 ranks' partials, dlogits, grad_hidden
    # partial and grad_weight shard GEMMs).
    from trainscale_amd.loss.linear_ce import linear_ce_vocab_phase1, linear_ce_vocab_phase2
    Nt, H = 8192, 4096
    hid = torch.randn(Nt, H, device=dev, generator=g).to(torch.bfloat16)
    wsh = (0.02 * torch.randn(vp, H, device=dev, generator=g)).to(torch.bfloat16)
    lab = torch.randint(0, 128256, (Nt,), device=dev, generator=g)
    lab[::20] = -100

    def vocab_lce():
        stats, state = linear_ce_vocab_phase1(hid, wsh, lab, vp)
        linear_ce_vocab_phase2(state, stats.unsqueeze(0).expand(P, -1, -1), -100, "mean")

    ms = time_ms(vocab_lce, steps, warmup)
    fl = 3 * 2 * Nt * vp * H
    res["vocab_linear_ce"] = {"shape": {"hidden": [Nt, H], "weight_shard": [vp, H]}, "ranks": P,
                              "ms": round(ms, 4), "flop": fl,
                              "TFLOP_s": round(fl / (ms * 1e-3) / 1e12, 1),
                              "frac": round(fl / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}
    del hid, wsh, lab
    torch.cuda.empty_cache()
    return res


def bench_linear_ce(dev, steps: int, warmup: int, cpu: bool, cpu_seconds: float):
    """C5: fused linear CE fwd+bwd (loss, grad_hidden, grad_weight) in one call."""
    import torch

    from trainscale_amd import _lib
    from trainscale_amd import workloads as W
    from trainscale_amd.loss.linear_ce import _chunk_rows

    c5 = W.linear_ce_workload(dev)
    h, w, labels = c5.tensors["hidden"], c5.tensors["weight"], c5.tensors["labels"]
    N, H = h.shape
    V = w.shape[0]
    lib = _lib.load()
    chunk = _chunk_rows(N, V, None)
    ws_bytes = int(lib.ts_flce_workspace_size(N, H, V, chunk, 1))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    rows = torch.empty((N,), dtype=torch.float32, device=dev)
    lse = torch.empty((N,), dtype=torch.float32, device=dev)
    gh = torch.empty_like(h)
    gw = torch.empty_like(w)
    stream = _lib.stream_handle(dev)

    def step():
        _lib.check(lib.ts_flce_fwd_bwd(
            _lib.ptr(h), H, _lib.ptr(w), H, _lib.ptr(labels), N, H, V, -100, 0, _lib.ptr(loss),
            _lib.ptr(rows), _lib.ptr(lse), _lib.ptr(gh), _lib.ptr(gw), chunk, _lib.ptr(ws),
            ws_bytes, stream), "ts_flce_fwd_bwd")

    ms = time_ms(step, max(3, steps // 2), max(1, warmup // 2))
    flops = W.linear_ce_flops(N, H, V)
    tf = flops / (ms * 1e-3) / 1e12
    out = {"workload": (f"C5 fused linear CE: hidden [{N},{H}] bf16, lm_head [{V},{H}] bf16, "
                        f"5% ignored, mean; loss + grad_hidden + grad_weight; token chunk "
                        f"{chunk or N} rows"),
           "ms": round(ms, 4), "algorithmic_flop": flops, "TFLOP_s": round(tf, 1),
           "roofline": {"bound": "mfma", "achieved": round(tf, 1),
                        "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)},
           "tokens_per_s": round(N / (ms * 1e-3), 1)}
    if cpu:
        out["cpu_baseline"] = cpu_baseline_linear_ce(cpu_seconds)
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1 "
                                   "(every rank would run these kernels on its own shard: "
                                   "rows for RMSNorm/RoPE/CE, vocabulary columns for the "
                                   "vocab-parallel CE, whose per-rank kernels are measured "
                                   "at their shard shape)"}))
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
    upstream = torch.ones((1,), dtype=torch.float32, device=dev)
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
    bytes_c3 = W.ce_bytes_fused(N, n_valid, V)
    op_bytes = {
        "rmsnorm_fwd": bytes_c1["fwd"], "rope_fwd": bytes_c2["fwd"], "ce_fwd_bwd": bytes_c3,
        "ce_bwd_scale": 4, "rope_bwd": bytes_c2["bwd"], "rmsnorm_bwd": bytes_c1["bwd"],
    }
    kernel_names = {"rmsnorm_fwd": "rms_fwd_reg", "rope_fwd": "rope_tok_kernel",
                    "ce_fwd_bwd": "ce_fused_vec", "ce_bwd_scale": "scale_inplace",
                    "rope_bwd": "rope_tok_kernel", "rmsnorm_bwd": "rms_bwd_reg+rms_dw_reduce4"}
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
        # schedule B: the forward reads each valid row once and writes its gradient
        state["ce"] = ops.ce_forward_backward(logits, V, labels, dloss, grad=grad)
        mark(3)
        # the backward applies the upstream gradient: a device-side no-op when it is 1
        ops.scale_(grad, upstream)
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
        kernels[name] = {"kernel": kernel_names[name], "ms": round(ms, 4),
                         "bytes": op_bytes[name], "GB_s": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}
    dom = max(order, key=lambda n: kernels[n]["ms"])
    traffic = load_traffic().get(kernel_names[dom])
    roofline = {
        "kernel": kernel_names[dom],
        "op": dom,
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
                         "theta 5e5 in-register + C3 CE logits[16384,128256] 10% ignored "
                         "(schedule B: the forward reads each valid row once and writes the "
                         "gradient; the backward scales it by the upstream gradient, a "
                         "device-side no-op at 1); fwd C1,C2,C3 then bwd C3,C2,C1"),
            "ce_schedule": "B",
            "step_bytes": step_bytes,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(tokens / (ms_step * 1e-3), 1),
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "kernels": kernels,
        "device": torch.cuda.get_device_name(dev),
    }
    # free the headline step's buffers before the extra sections
    del c1, c2, c3, x, w, dy, x2d, dy2d, q, k, dq, dk, q_out, k_out, dq_out, dk_out
    del logits, labels, grad, state, upstream
    torch.cuda.empty_cache()
    out["device_reference"] = device_reference(dev)
    if not args.no_extra:
        out["c4_packed"] = bench_packed(dev, args.steps, args.warmup)
        out["c5_linear_ce"] = bench_linear_ce(dev, args.steps, args.warmup,
                                              cpu=not args.no_cpu_baseline,
                                              cpu_seconds=args.cpu_seconds)
        out["next_rows"] = bench_next_rows(dev, args.steps, args.warmup)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
