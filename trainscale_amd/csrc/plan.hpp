// Launch planning shared by the C-ABI size queries and the kernel launches.
//
// Plain C++ with no HIP dependency, so the host-side bounds arithmetic can be
// compiled and checked on a machine without a GPU. Every quantity a launch
// writes to caller memory (number of dW partial rows, grid sizes) comes from
// these functions, and the workspace size reported to the caller is the
// maximum over every plan the launch may pick for the same (rows, cols).
#pragma once

#include <stdint.h>

namespace ts_plan {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// RMSNorm
// ---------------------------------------------------------------------------
constexpr int kFwdWaves = 4;          // rows per forward workgroup (one per wave)
constexpr int kFwdMaxVec = 16;        // 16-byte vectors per lane held in registers
constexpr int kBwdWaves = 8;          // waves per backward workgroup
constexpr int kBwdMaxVec = 8;         // 16-byte vectors per lane held in registers
constexpr int kBwdMaxSplit = 4;       // waves that may share one row
constexpr int64_t kBwdMaxGrid = 512;  // backward workgroups (2 per CU on 256 CUs)
constexpr int64_t kBwdLdsLimit = 65536 - 1024;  // bytes of the fp32 dW fold row
constexpr int64_t kGenericRowsPerGroup = 64;

// Elements per 16-byte vector.
inline int vec_elems(int elt_bytes) { return 16 / elt_bytes; }

// Vectors per lane of the forward register path (power of two), or 0 when
// the row is too long for registers.
inline int rms_fwd_maxv(int64_t nvec) {
  for (int m = 1; m <= kFwdMaxVec; m *= 2)
    if (nvec <= (int64_t)m * kWave) return m;
  return 0;
}

struct RmsBwdPlan {
  bool reg;        // register path (else the generic element-wise kernels)
  int maxv;        // vectors per lane (register path)
  int split;       // waves per row (register path)
  int64_t grid;    // workgroups of the dx kernel
  int64_t nparts;  // dW partial rows written (== rows of fp32 workspace used)
};

// Register-path feasibility given the row length in vectors; `vec_ok` says
// whether pointers/strides allow 16-byte access at all.
inline RmsBwdPlan rms_bwd_plan(int64_t rows, int64_t cols, int elt_bytes, bool vec_ok,
                               bool need_dw) {
  RmsBwdPlan p{false, 0, 0, 0, 0};
  const int V = vec_elems(elt_bytes);
  const int64_t nvec = cols / V;
  int split = 1;
  while (split <= kBwdMaxSplit && nvec > (int64_t)kWave * kBwdMaxVec * split) split *= 2;
  const bool lds_ok = !need_dw || cols * 4 <= kBwdLdsLimit;
  if (vec_ok && cols % V == 0 && split <= kBwdMaxSplit && lds_ok && nvec > 0) {
    p.reg = true;
    p.split = split;
    p.maxv = split == 1 ? rms_fwd_maxv(nvec) : kBwdMaxVec;
    if (p.maxv > kBwdMaxVec || p.maxv == 0) p.reg = false;
  }
  if (p.reg) {
    const int64_t per_step = kBwdWaves / p.split;
    const int64_t want = (rows + per_step - 1) / per_step;
    p.grid = want < kBwdMaxGrid ? want : kBwdMaxGrid;
    p.nparts = need_dw ? p.grid : 0;
  } else {
    p.split = 0;
    p.maxv = 0;
    p.grid = rows;
    p.nparts = need_dw ? (rows + kGenericRowsPerGroup - 1) / kGenericRowsPerGroup : 0;
  }
  return p;
}

// Rows of fp32 dW partials any backward launch for (rows, cols) may write:
// the maximum over element sizes 2 and 4 and over both paths.
inline int64_t rms_bwd_workspace_rows(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  int64_t m = 0;
  for (int e = 0; e < 4; ++e) {
    const RmsBwdPlan p = rms_bwd_plan(rows, cols, (e & 1) ? 4 : 2, (e & 2) != 0, true);
    if (p.nparts > m) m = p.nparts;
  }
  return m;
}

// ---------------------------------------------------------------------------
// Magic-number division used by the RoPE task decomposition:
// q = umulhi(n, ceil(2^32 / d)) equals n / d whenever n * d < 2^32 and d > 1.
// ceil(2^32 / 1) does not fit 32 bits, so d == 1 is encoded as magic 0 and
// divides by returning n (the device code makes the same choice).
// ---------------------------------------------------------------------------
inline uint32_t magic_for(uint32_t d) {
  return d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + d - 1) / d);
}
inline uint32_t magic_div(uint32_t n, uint32_t magic) {
  return magic == 0 ? n : (uint32_t)(((uint64_t)n * magic) >> 32);
}
inline bool magic_exact(uint64_t n_max, uint64_t d) { return n_max * d < ((uint64_t)1 << 32); }

}  // namespace ts_plan
