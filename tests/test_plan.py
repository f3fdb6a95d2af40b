"""Host-side launch arithmetic (trainscale_amd/csrc/plan.hpp), checked on the CPU.

The plan functions decide grid sizes, how many fp32 dW partial rows the RMSNorm
backward writes, and the magic-number division the RoPE kernel uses for task
indices. A small C++ driver compiled with g++ sweeps many shapes and checks:

* every backward plan writes at most the partial rows ts_rmsnorm_bwd_workspace_size
  reports (regression: a split-row launch once wrote past a workspace sized
  for the unsplit launch);
* register plans cover every 16-byte vector of the row and stay within the
  template instantiations the launcher has;
* umulhi(n, ceil(2^32/d)) == n / d wherever magic_exact(n_max, d) admits it,
  including d == 1 (regression: ceil(2^32/1) once truncated to 0, sending every
  RoPE task of a one-task-per-head shape to head 0 and past the tensor).

It also checks the exported size query of the built library against the
driver's figure for the same shapes.
"""
import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

from trainscale_amd import _lib

CSRC = Path(__file__).resolve().parent.parent / "trainscale_amd" / "csrc"

DRIVER = r"""
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include "plan.hpp"
using namespace ts_plan;

static int fails = 0;
#define CHECK(c, ...) do { if (!(c)) { if (fails++ < 20) { std::printf(__VA_ARGS__); std::printf("\n"); } } } while (0)

int main() {
  const long long rows_list[] = {0, 1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 37, 63, 64, 65,
                                 100, 127, 128, 129, 255, 256, 257, 511, 512, 513, 1000,
                                 1023, 1024, 1025, 2047, 2048, 2049, 4096, 8192, 16384,
                                 32768, 65537};
  for (long long rows : rows_list) {
    for (long long cols = 4; cols <= 24000; cols += (cols < 256 ? 4 : cols < 4096 ? 52 : 764)) {
      const long long wsr = rms_bwd_workspace_rows(rows, cols);
      for (int elt : {2, 4}) {
        const int V = vec_elems(elt);
        for (bool vec : {true, false}) {
          for (bool dw : {true, false}) {
            RmsBwdPlan p = rms_bwd_plan(rows, cols, elt, vec, dw);
            CHECK(p.nparts <= wsr, "rows=%lld cols=%lld elt=%d vec=%d: nparts %lld > ws rows %lld",
                  rows, cols, elt, (int)vec, (long long)p.nparts, wsr);
            if (!dw) CHECK(p.nparts == 0, "nparts without dW");
            if (p.reg) {
              const long long nvec = cols / V;
              CHECK(cols % V == 0 && vec, "reg path for unaligned row");
              CHECK((long long)p.maxv * kWave * p.split >= nvec,
                    "rows=%lld cols=%lld: reg plan covers %lld of %lld vectors", rows, cols,
                    (long long)p.maxv * kWave * p.split, nvec);
              const bool inst = (p.split == 1 && (p.maxv == 1 || p.maxv == 2 || p.maxv == 4 ||
                                                  p.maxv == 8)) ||
                                (p.maxv == 8 && (p.split == 2 || p.split == 4));
              CHECK(inst, "no instantiation for maxv=%d split=%d", p.maxv, p.split);
              CHECK(p.grid >= (rows > 0 ? 1 : 0) && p.grid <= kBwdMaxGrid, "grid %lld", (long long)p.grid);
              CHECK(rows == 0 || p.grid * (kBwdWaves / p.split) <= rows + kBwdWaves,
                    "grid larger than the rows need");
              if (dw) CHECK(cols * 4 <= kBwdLdsLimit, "LDS fold row too long");
            }
          }
        }
        const long long nvec = cols / V;
        const int m = rms_fwd_maxv(nvec);
        if (m) CHECK((long long)m * kWave >= nvec && m <= kFwdMaxVec, "fwd maxv %d for %lld", m, nvec);
      }
    }
  }
  // magic-number division
  for (unsigned d = 1; d <= 70000; d += (d < 2048 ? 1 : 97)) {
    const unsigned mg = magic_for(d);
    unsigned long long nmax = (1ull << 32) / d;  // largest n admitted is < 2^32 / d
    while (nmax > 0 && !magic_exact(nmax, d)) --nmax;
    for (unsigned long long n = 0; n < nmax; n += (nmax > 5000 ? nmax / 4000 + 1 : 1)) {
      CHECK(magic_div((unsigned)n, mg) == n / d, "magic %llu/%u", n, d);
    }
    if (nmax) CHECK(magic_div((unsigned)(nmax - 1), mg) == (nmax - 1) / d, "magic edge %u", d);
  }
  std::printf("%d failures\n", fails);
  return fails != 0;
}
"""


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("plan")
    src = d / "plan_check.cpp"
    src.write_text(DRIVER)
    exe = d / "plan_check"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    return exe


def test_plan_bounds(driver):
    proc = subprocess.run([str(driver)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_workspace_query_matches_split_launches():
    lib = _lib.load()
    # shapes whose backward splits a row over 2 or 4 waves with few rows: the
    # case the old sizing got wrong
    for rows, cols in [(37, 8192), (37, 12288), (5, 8192), (129, 12288), (1, 8192)]:
        per_step = {8192: 4, 12288: 2}[cols]  # rows per workgroup step for bf16
        need_rows = -(-rows // per_step)
        got = lib.ts_rmsnorm_bwd_workspace_size(rows, cols)
        assert got >= need_rows * cols * 4, (rows, cols, got, need_rows)
    assert lib.ts_rmsnorm_bwd_workspace_size(0, 4096) == 0
    assert lib.ts_rmsnorm_bwd_workspace_size(16, 0) == 0
