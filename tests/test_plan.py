"""Host-side launch arithmetic (trainscale_amd/csrc/plan.hpp), checked on the CPU.

The plan functions decide grid sizes, how many fp32 dW partial rows the RMSNorm
backward writes, and the magic-number division the RoPE kernel uses for task
indices. A small C++ driver compiled with g++ sweeps many shapes and checks:

* every backward plan writes at most the partial rows ts_rmsnorm_bwd_workspace_size
  reports (regression: a split-row launch once wrote past a workspace sized
  for the unsplit launch);
* every 16-byte load the backward kernel issues (ts_plan::rms_bwd_load_offset,
  the function the kernel computes its addresses with) lies inside the matrix,
  including the lanes and row slots with nothing to load (regression: those
  once loaded their own row's start, past the matrix for the slots beyond the
  last row and for lanes beyond a short row);
* register plans cover every 16-byte vector of the row and stay within the
  template instantiations the launcher has;
* the grouped GEMM tile order visits every output tile exactly once;
* RoPE workgroups are whole waves within 256..1024 threads and their cos/sin
  staging fits the LDS bound;
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
#include <vector>
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
              const RmsRowPlan& r = p.row;
              CHECK(cols % V == 0 && vec, "reg path for unaligned row");
              CHECK((long long)r.tpr * r.kv >= nvec, "rows=%lld cols=%lld: plan covers %d of %lld vectors",
                    rows, cols, r.tpr * r.kv, nvec);
              if (p.wave) {
                CHECK(r.tpr == 64 && (r.kv == 2 || r.kv == 4),
                      "no wave instantiation for tpr=%d kv=%d", r.tpr, r.kv);
                CHECK(r.block == 64 * kWaveRowsPerBlock && r.rpb == kWaveRowsPerBlock,
                      "wave block shape");
                CHECK(nvec <= kWaveRowMaxVec, "wave dW staging exceeds its LDS array");
              } else {
                const bool inst = (r.kv == 1 && (r.tpr == 64 || r.tpr == 128 || r.tpr == 256 ||
                                                  r.tpr == 512)) ||
                                  (r.tpr == 512 && (r.kv == 2 || r.kv == 4));
                CHECK(inst, "no bwd instantiation for tpr=%d kv=%d", r.tpr, r.kv);
                CHECK(r.block == 512 && r.rpb * r.tpr == 512, "bwd block shape");
              }
              CHECK(p.steps >= 1 && p.grid >= (rows > 0 ? 1 : 0), "grid %lld steps %lld",
                    (long long)p.grid, (long long)p.steps);
              // every row is covered by exactly one (workgroup, step, slot)
              CHECK(p.grid * p.steps * r.rpb >= rows, "rows=%lld not covered", rows);
              CHECK(rows == 0 || (p.grid - 1) * p.steps * r.rpb < rows, "empty workgroup");
              CHECK(p.grid < (1ll << 31), "grid too large");
              if (dw) CHECK(p.nparts == (p.wave ? p.grid : p.grid * r.rpb), "nparts");
              // every 16-byte load of the backward kernel lies inside the [rows, ld] matrix
              // (ld = cols and a wider stride), for every workgroup, slot, step and lane
              if (rows > 0 && rows <= 2049 && cols <= 8192) {
                for (long long ld : {cols, cols + V}) {
                  const long long rstep = p.grid * r.rpb;
                  if (p.wave) {
                    // the buffer span of every (workgroup, slot, step) lies inside the matrix;
                    // lane offsets (v * 16 for v < nvec) lie inside a span of nvec * 16 bytes
                    const uint32_t rb = (uint32_t)(nvec * 16);
                    for (long long wg = 0; wg < p.grid; ++wg)
                      for (int sub = 0; sub < r.rpb; ++sub)
                        for (long long st = 0; st < p.steps + 1; ++st) {
                          const RowSpan sp = rms_bwd_wave_row(wg * r.rpb + sub, st, rstep,
                                                              p.steps, rows, ld, rb);
                          const long long row = wg * r.rpb + sub + st * rstep;
                          CHECK(sp.bytes == 0 || (sp.offset >= 0 && sp.offset * (16 / V) + sp.bytes <=
                                                  ((rows - 1) * ld + cols) * (16 / V)),
                                "rows=%lld cols=%lld ld=%lld wg=%lld sub=%d st=%lld: span past the "
                                "matrix", rows, cols, ld, wg, sub, st);
                          CHECK((sp.bytes != 0) == (st < p.steps && row < rows),
                                "span of a row that %s", sp.bytes ? "does not exist" : "exists");
                          CHECK(sp.bytes == 0 || sp.offset == row * ld, "span of another row");
                        }
                    continue;
                  }
                  for (long long wg = 0; wg < p.grid; wg += (p.grid > 64 ? p.grid / 17 : 1))
                    for (int sub = 0; sub < r.rpb; ++sub)
                      for (long long st = 0; st < p.steps + 1; ++st)
                        for (int t = 0; t < r.tpr; t += (r.tpr > 64 ? 7 : 1))
                          for (int k = 0; k < r.kv; ++k) {
                            const long long off = rms_bwd_load_offset(
                                wg * r.rpb + sub, st, rstep, p.steps, rows, t, k, r.tpr, V, nvec, ld);
                            CHECK(off >= 0 && off + V <= (rows - 1) * ld + cols,
                                  "rows=%lld cols=%lld ld=%lld wg=%lld sub=%d st=%lld t=%d k=%d: "
                                  "load at element %lld past the matrix", rows, cols, ld, wg, sub,
                                  st, t, k, off);
                          }
                }
              }
            }
          }
        }
        const long long nvec = cols / V;
        RmsRowPlan f = rms_fwd_plan(nvec);
        if (f.reg) {
          CHECK((long long)f.tpr * f.kv >= nvec, "fwd plan covers %d of %lld", f.tpr * f.kv, nvec);
          const bool inst = (f.tpr == 64 && (f.kv == 1 || f.kv == 2)) || (f.tpr == 128 && f.kv == 2) ||
                            (f.tpr == 256 && f.kv == 2) || (f.tpr == 512 && (f.kv == 2 || f.kv == 4));
          CHECK(inst, "no fwd instantiation for tpr=%d kv=%d", f.tpr, f.kv);
          CHECK(f.block == (f.tpr > 256 ? f.tpr : 256) && f.rpb * f.tpr == f.block, "fwd block shape");
        }
      }
    }
  }
  // RoPE workgroup shapes
  for (long long tpt = 1; tpt <= 40000; tpt += (tpt < 600 ? 1 : 37)) {
    for (int half : {1, 2, 8, 10, 32, 64, 128, 256}) {
      RopeBlock b = rope_block(tpt, half, 1024, 4096);
      CHECK(b.tpb >= 1 && (long long)b.tpb * half <= 4096, "rope tpb %d half %d", b.tpb, half);
      CHECK(b.threads % 64 == 0 && b.threads >= 256 && b.threads <= 1024, "rope threads %d", b.threads);
      if (tpt >= 256) CHECK(b.tpb == 1, "rope tpb %d for %lld tasks", b.tpb, tpt);
      else CHECK((long long)b.tpb * tpt <= 256 || b.tpb == 1, "rope over-filled block");
    }
  }
  // GEMM tile order is a bijection onto the MT x NT tiles
  for (long long MT : {1, 2, 15, 16, 17, 32, 33, 501}) {
    for (long long NT : {1, 3, 16, 501}) {
      std::vector<char> seen(MT * NT, 0);
      for (long long b = 0; b < MT * NT; ++b) {
        int64_t mt, nt;
        gemm_tile_of(b, MT, NT, mt, nt);
        const bool ok = mt >= 0 && mt < MT && nt >= 0 && nt < NT;
        CHECK(ok, "tile_of(%lld) out of range for %lld x %lld", b, MT, NT);
        if (ok) {
          CHECK(!seen[mt * NT + nt], "tile (%lld, %lld) twice", (long long)mt, (long long)nt);
          seen[mt * NT + nt] = 1;
        }
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
  // 64-bit magic-number division (RoPE token split): exact wherever admitted
  {
    const unsigned long long ds[] = {1, 2, 3, 7, 2048, 4095, 4096, 4097, 131071, 1000003,
                                     (1ull << 31) - 1, (1ull << 32) + 15, (1ull << 40) - 3};
    for (unsigned long long d : ds) {
      const unsigned long long mg = magic64_for(d);
      // largest admitted n: n * d < 2^64
      const unsigned long long nmax = d == 1 ? ~0ull : (~0ull) / d;
      CHECK(magic64_exact(nmax, d) || d == 1, "magic64 bound %llu", d);
      const unsigned long long probes[] = {0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d,
                                           nmax / 3, nmax / 2, nmax - 1, nmax};
      for (unsigned long long n : probes) {
        if (d > 1 && !magic64_exact(n, d)) continue;
        CHECK(magic64_div(n, mg) == n / d, "magic64 %llu/%llu", n, d);
      }
      for (unsigned long long q = 1; q < 2000 && d > 1; q += 7) {  // both sides of multiples
        const unsigned __int128 nn = (unsigned __int128)q * d;
        if (nn >= nmax) break;
        const unsigned long long n = (unsigned long long)nn;
        CHECK(magic64_div(n, mg) == q && magic64_div(n - 1, mg) == q - 1, "magic64 edge %llu*%llu", q, d);
      }
    }
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


def test_workspace_query_covers_every_partial_row():
    lib = _lib.load()
    # one partial row per row slot of every backward workgroup: rows small
    # enough that each row group gets its own workgroup
    for rows, cols in [(37, 8192), (37, 12288), (5, 8192), (129, 12288), (1, 8192), (300, 512)]:
        got = lib.ts_rmsnorm_bwd_workspace_size(rows, cols)
        assert got >= rows * cols * 4 or got >= 512 * cols * 4, (rows, cols, got)
    assert lib.ts_rmsnorm_bwd_workspace_size(0, 4096) == 0
    assert lib.ts_rmsnorm_bwd_workspace_size(16, 0) == 0
