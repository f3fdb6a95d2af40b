"""bench.py's command-line contract and its reading of the committed profiles (CPU)."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    # the build measures one GPU: --gpus N > 1 exits with a message that says so, before
    # touching a GPU
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert proc.returncode == 2
    msg = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def _bench():
    sys.path.insert(0, str(ROOT))
    try:
        import bench
    finally:
        sys.path.remove(str(ROOT))
    return bench


def test_roofline_traffic_comes_from_the_committed_profile():
    bench = _bench()
    traffic, _ = bench.load_traffic()
    # the dominant kernel's measured HBM bytes per launch: within 5 % of the bytes it must
    # touch at C3 (valid rows read, every row written)
    touched = 7_985_480_704
    assert abs(traffic["ce_fused_vec"] - touched) <= 0.05 * touched


def test_traffic_is_left_out_when_the_kernels_changed(monkeypatch):
    bench = _bench()
    measured, src = bench.load_traffic()
    monkeypatch.setattr(bench, "kernel_source_hash", lambda: src)
    t, where = bench.traffic_for("ce_fused_vec")
    assert t == measured["ce_fused_vec"] and "pmc_traffic" in where
    monkeypatch.setattr(bench, "kernel_source_hash", lambda: "0" * 16)
    t, where = bench.traffic_for("ce_fused_vec")
    assert t is None and where.startswith("none")


def test_kernel_source_hash_is_stable():
    bench = _bench()
    a = bench.kernel_source_hash()
    assert len(a) == 16 and int(a, 16) >= 0 and a == bench.kernel_source_hash()
