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
* the streaming kernels' vector index (ts_plan::chunk_vec over the grid chunks_for
  gives; SwiGLU, the CE and vocabulary-shard backward, dlogits, dz, scale) and the
  CE forward's chunk-then-tail row loop visit every vector of a row exactly once,
  buffer offsets of register rows (vec_boffset) stay inside their resource or use
  the offset no resource covers, and row kernels' row_vec_in admits only vectors
  inside the matrix;
* every RoPE task of a workgroup (rope_task, and the token kernel's rope_head_task)
  maps to one (token slot, head, index) in range, each once, and its elements
  (rope_elems) lie inside the head, for the vector and generic paths and both
  layouts;
* one-wave-per-row kernels (wave_row over wave_row_blocks) own every row once,
  a label's logit is read only at a column inside its row (label_col), and a
  vocabulary split into shards gives each label to exactly one shard (shard_col);
* RoPE workgroups are whole waves within 256..1024 threads and their cos/sin
  staging fits the LDS bound;
* umulhi(n, ceil(2^32/d)) == n / d wherever magic_exact(n_max, d) admits it,
  including d == 1 (regression: ceil(2^32/1) once truncated to 0, sending every
  RoPE task of a one-task-per-head shape to head 0 and past the tensor).

It also checks the exported size query of the built library against the
driver's figure for the same shapes.
"""
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
#include <algorithm>
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
  // Streaming kernels: chunk_vec over the grid chunks_for gives (SwiGLU, CE and
  // vocabulary-shard backward, dlogits, dz, scale sweeps) visits every vector of
  // [0, nvec) exactly once; accesses are guarded by v < nvec
  for (int threads : {64, 256, 1024}) {
    for (int kv : {1, 2, 4, 16}) {
      for (long long nvec : {1ll, 7ll, 63ll, 64ll, 255ll, 256ll, 257ll, 1000ll, 1024ll, 4097ll,
                             16032ll, 16033ll}) {
        std::vector<int> seen(nvec, 0);
        const long long chunks = chunks_for(nvec, threads, kv);
        CHECK(chunks * threads * kv >= nvec && (chunks - 1) * threads * kv < nvec,
              "chunks_for(%lld, %d, %d) = %lld", nvec, threads, kv, chunks);
        for (long long c = 0; c < chunks; ++c)
          for (int k = 0; k < kv; ++k)
            for (int t = 0; t < threads; ++t) {
              const long long v = chunk_vec(c, k, t, threads, kv);
              CHECK(v >= 0, "negative vector index");
              if (v < nvec) seen[v]++;
            }
        for (long long v = 0; v < nvec; ++v)
          CHECK(seen[v] == 1, "nvec=%lld threads=%d kv=%d: vector %lld visited %d times", nvec,
                threads, kv, v, seen[v]);
        // the row loop of ce_fwd_vec: whole chunks, then the tail of chunk `full`
        // stepping by `threads` from chunk_vec(full, 0, t, ...)
        std::vector<int> seen2(nvec, 0);
        const long long full = nvec / ((long long)threads * kv);
        for (long long c = 0; c < full; ++c)
          for (int k = 0; k < kv; ++k)
            for (int t = 0; t < threads; ++t) {
              const long long v = chunk_vec(c, k, t, threads, kv);
              CHECK(v >= 0 && v < nvec, "whole chunk reaches vector %lld of %lld", v, nvec);
              if (v >= 0 && v < nvec) seen2[v]++;
            }
        for (int t = 0; t < threads; ++t)
          for (long long v = chunk_vec(full, 0, t, threads, kv); v < nvec; v += threads)
            if (v >= 0) seen2[v]++;
        for (long long v = 0; v < nvec; ++v) CHECK(seen2[v] == 1, "row loop visits %lld %d times", v, seen2[v]);
        // buffer offsets of register rows (ce_fused_vec, shard stats): inside a
        // resource of nvec vectors, or an offset no such resource covers
        for (int vb : {16, 32}) {
          if ((long long)nvec * vb >= (1ll << 31)) continue;
          for (long long v = 0; v < nvec + 3 * threads; ++v) {
            const int32_t o = vec_boffset(v, nvec, vb);
            if (v < nvec) CHECK(o == v * vb && o + vb <= nvec * vb, "boffset in range");
            else CHECK(o == kNoAccess && (uint32_t)o >= (uint64_t)nvec * vb, "boffset past the row");
          }
        }
      }
    }
  }
  // Row kernels (RMSNorm forward and add): row_vec_in admits exactly the vectors of
  // the matrix, whose element ranges lie inside [rows, ld]
  for (long long rows : {1ll, 3ll, 37ll}) {
    for (long long nvec : {1ll, 5ll, 64ll, 513ll}) {
      for (int V : {4, 8}) {
        for (long long ld : {nvec * V, nvec * V + V}) {
          const long long extent = (rows - 1) * ld + nvec * V;
          for (long long row = 0; row < rows + 2; ++row)
            for (long long v = 0; v < nvec + 70; ++v) {
              const bool in = row_vec_in(row, rows, v, nvec);
              CHECK(in == (row < rows && v < nvec), "row_vec_in");
              if (in) CHECK(row * ld + v * V + V <= extent, "row vector past the matrix");
            }
        }
      }
    }
  }
  // RoPE: every task f < tpb * tasks_per_token of a workgroup maps to one
  // (token slot, head, index) in range, each exactly once, and its elements lie
  // inside the head; the token kernel's per-token split likewise
  for (int heads : {1, 2, 3, 8, 9, 40, 72}) {
    for (int D : {2, 8, 16, 64, 128, 256, 512}) {
      const int half = D / 2;
      for (int W : {1, 4, 8}) {           // element width: 1 = generic path
        for (int il = 0; il < 2; ++il) {  // NeoX or interleaved
          const bool inter = il == 1;
          if (W > 1 && (inter ? D % W != 0 : half % W != 0)) continue;
          const int tph = W == 1 ? half : (inter ? 2 * half / W : half / W);
          const long long tpt = (long long)tph * heads;
          if (tpt >= (1 << 20)) continue;
          const RopeBlock blk = rope_block(tpt, half, 1024, 4096);
          const long long total = (long long)blk.tpb * tpt;
          if (!magic_exact((uint64_t)total, (uint64_t)tpt) || !magic_exact((uint64_t)tpt, (uint64_t)tph)) continue;
          const uint32_t mt = magic_for((uint32_t)tpt), mh = magic_for((uint32_t)tph);
          std::vector<char> hit(total, 0);
          for (long long f = 0; f < total; ++f) {
            const RopeTask t = rope_task((int)f, (int)tpt, mt, tph, mh);
            const bool ok = t.i >= 0 && t.i < blk.tpb && t.hh >= 0 && t.hh < heads && t.j >= 0 && t.j < tph;
            CHECK(ok, "rope task %lld of %d heads D=%d W=%d: (%d, %d, %d)", f, heads, D, W, t.i, t.hh, t.j);
            if (!ok) continue;
            const long long id = ((long long)t.i * heads + t.hh) * tph + t.j;
            CHECK(!hit[id], "rope task visited twice");
            hit[id] = 1;
            const RopeElems e = rope_elems(t.j, W, half, inter);
            const int w1 = W == 1 ? 1 : W;
            CHECK(e.e1 >= 0 && e.e1 + w1 <= D, "rope e1 %d (D=%d W=%d)", e.e1, D, W);
            if (W == 1 || !inter) CHECK(e.e2 >= 0 && e.e2 + w1 <= D, "rope e2 %d (D=%d W=%d)", e.e2, D, W);
            if (!inter) CHECK(e.e2 == e.e1 + half || (W == 1 && e.e2 == e.e1 + half), "NeoX pair");
            if (t.i == 0 && f < tpt) {
              const RopeTask u = rope_head_task((int)f, tph, mh);
              CHECK(u.hh == t.hh && u.j == t.j, "token-kernel task split");
            }
          }
        }
      }
    }
  }
  // One-wave-per-row kernels (flce_rows, flce_rows_t, flce_shard_rows): the grid
  // wave_row_blocks gives assigns each row to one wave, and the waves past the
  // last row are exactly those the kernel's row check sends home
  for (int waves : {1, 4, 16}) {
    for (long long rows : {1ll, 3ll, 4ll, 5ll, 2047ll, 2048ll, 8193ll}) {
      std::vector<int> seen(rows, 0);
      const long long blocks = wave_row_blocks(rows, waves);
      CHECK(blocks * waves >= rows && (blocks - 1) * waves < rows, "wave_row_blocks");
      for (long long b = 0; b < blocks; ++b)
        for (int w = 0; w < waves; ++w) {
          const long long r = wave_row(b, w, waves);
          if (r < rows) seen[r]++;
        }
      for (long long r = 0; r < rows; ++r) CHECK(seen[r] == 1, "row %lld owned %d times", r, seen[r]);
    }
  }
  // Label columns: a logit is read only at a column inside the row, and a
  // vocabulary split into shards gives every label in [0, V) to exactly one shard
  {
    const long long big = 0x7fffffffffffffffll;
    for (long long V : {1ll, 7ll, 50257ll, 128256ll}) {
      for (long long ign : {-100ll, 0ll, 5ll}) {
        for (long long lab : {-big - 1, -101ll, -100ll, -1ll, 0ll, 1ll, 5ll, 6ll, V - 1, V, V + 1, big}) {
          const long long c = label_col(lab, V, ign);
          if (lab == ign) CHECK(c == kLabelIgnored, "ignored label");
          else if (lab >= 0 && lab < V) CHECK(c == lab, "label column");
          else CHECK(c == kLabelOutside, "label outside");
        }
      }
      for (int P : {1, 2, 3, 8}) {
        const long long Vp = (V + P - 1) / P;
        for (long long lab : {-big - 1, -1ll, 0ll, 1ll, Vp - 1, Vp, V / 2, V - 1, V, big}) {
          int owners = 0;
          for (int p = 0; p < P; ++p) {
            const long long start = p * Vp, width = std::min(Vp, V - start);
            if (width <= 0) continue;
            const long long c = shard_col(lab, start, width);
            if (c != kLabelOutside) {
              owners++;
              CHECK(c >= 0 && c < width && start + c == lab, "shard column %lld of %lld", c, width);
            }
          }
          CHECK(owners == (lab >= 0 && lab < V ? 1 : 0), "label %lld held by %d shards", lab, owners);
        }
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
