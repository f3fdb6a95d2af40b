// bf16 MFMA GEMM core for gfx950: C[M, N] = A[M, K] * B[N, K]^T, fp32 accumulation.
//
// Both operands are row-major with K contiguous (the layout of hidden [N, H]
// and of the LM head [V, H]), 16-byte aligned, row strides and K multiples of
// 8 elements.
//
// Workgroup tile 256 x 256, k-block 32, 256 threads = 4 waves in a 2 x 2 grid;
// each wave owns a 128 x 128 block of C as 4 x 4 tiles of
// v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane).
//
// Operands go from HBM straight into LDS with buffer_load_dwordx4 ... lds
// (no staging registers): a wave's load instruction fills 1 KiB of LDS, lane i
// at the wave's base + 16 * i. Four LDS stages of 32 KiB (A + B) keep two to
// three k-blocks of loads in flight while the MFMAs consume one (a fifth
// stage, the whole 160 KiB of a CU, measured slower on MI355X); one barrier
// per k-block, and the MFMA operand fragments are double-buffered in registers
// with the LDS reads and global loads interleaved between MFMAs (see
// mainloop). Buffer resources make
// out-of-range rows (and the k tail) read as zeros, so partial tiles need no
// branches.
//
// LDS rows are 64 B (32 bf16) with the four 16-byte chunks XOR-swizzled by
// (row >> 2) & 3 (see swz), which makes the MFMA operand ds_read_b128s free of
// bank conflicts.
//
// MFMA 32x32x16 bf16 lane layout (checked on the device): A lane l holds row
// l % 32, k = (l / 32) * 8 + e for e < 8; B lane l holds column l % 32 with the
// same k; accumulator element 4 * i + j is C[8 * i + 4 * (l / 32) + j][l % 32].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"
#include "plan.hpp"

namespace ts_gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint32_t* lds_ptr_t;

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 32;
#ifndef TS_GEMM_STAGES
#define TS_GEMM_STAGES 4
#endif
constexpr int kStages = TS_GEMM_STAGES;  // LDS stages of 32 KiB
static_assert(kStages >= 3 && kStages <= 5, "pipeline depth");
constexpr int kThreads = 256;
constexpr int kRowBytes = BK * 2;                       // 64
constexpr int kTileBytes = BM * kRowBytes;              // 16 KiB per operand per stage
constexpr int kStageBytes = 2 * kTileBytes;             // A + B
constexpr size_t kLdsBytes = (size_t)kStages * kStageBytes;
constexpr int kLoadsPerWave = BM * kRowBytes / 1024 / 4;      // 1 KiB loads per wave per operand
constexpr uint32_t kOob = 0x80000000u;  // voffset beyond every resource's range -> reads 0

struct Acc {
  f32x16 t[4][4];
};

__device__ void buffer_load_lds(i32x4 rsrc, lds_ptr_t lds, int size, int voffset, int soffset,
                                int offset, int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

// Raw buffer resource over [base, base + bytes) (gfx9 word 3).
__device__ inline i32x4 make_rsrc(const void* base, uint64_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = (int32_t)(uint32_t)a;
  r[1] = (int32_t)((uint32_t)(a >> 32) & 0xffffu);
  r[2] = (int32_t)(bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes);
  r[3] = 0x00020000;
  return r;
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS position of logical 16-byte chunk c (0..3) of LDS row `row` (64-byte
// rows). XOR with bits 2-3 of the row: among the rows one ds_read_b128 pass
// serves, rows that share a 128-byte bank line pair up with distinct chunk
// positions. Measured on MI355X with SQ_LDS_BANK_CONFLICT: 0 conflict cycles
// (XOR with bits 1-2 instead costs 12% of the main loop's cycles).
__device__ inline int swz(int row, int c) { return c ^ ((row >> 2) & 3); }

// Waits until at most `later` stages of this wave's loads are outstanding
// (each stage is 2 * kLoadsPerWave loads; vmcnt counts loads in issue order).
__device__ inline void wait_stage(int64_t later) {
  constexpr int kPer = 2 * kLoadsPerWave;
  static_assert(kPer * 3 < 64, "vmcnt range");
  if (later >= 3) wait_vmcnt<3 * kPer>();
  else if (later == 2) wait_vmcnt<2 * kPer>();
  else if (later == 1) wait_vmcnt<kPer>();
  else wait_vmcnt<0>();
}

// Per-thread byte offsets (relative to the tile's first row) of this lane's
// loads for logical chunk c of LDS row r: row * ld * 2 + chunk * 16.
struct TileLoader {
  i32x4 rsrc;
  uint32_t off[kLoadsPerWave];  // byte offset of this lane's chunk at k0 = 0
  int lds_row0;                 // first LDS row of the wave's first load
};

// Sets up the loads of one operand: rows [row0, row0 + 256) of a [nrows, ld]
// matrix; out-of-range rows read zeros.
__device__ inline TileLoader make_loader(const __bf16* g, int64_t ld, int64_t nrows,
                                         int64_t row0) {
  TileLoader t;
  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t valid = nrows - row0;
  if (valid > BM) valid = BM;
  if (valid < 0) valid = 0;
  t.rsrc = make_rsrc(g + row0 * ld, (uint64_t)valid * (uint64_t)ld * 2);
#pragma unroll
  for (int u = 0; u < kLoadsPerWave; ++u) {
    const int row = (u * 4 + wid) * 16 + (lane >> 2);
    const int chunk = swz(row, lane & 3);  // the logical chunk LDS position lane&3 holds
    t.off[u] = (uint32_t)(row * ld * 2 + chunk * 16);
  }
  t.lds_row0 = wid * 16;
  return t;
}

// Issues this wave's loads of k-block [k0, k0 + 32) into the LDS tile.
__device__ inline void issue_loads(const TileLoader& t, int64_t k0, int64_t K, uint8_t* lds_tile) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int u = 0; u < kLoadsPerWave; ++u) {
    // logical chunk of this lane for the load's row (same swizzle as make_loader)
    const int row = (u * 4 + (threadIdx.x >> 6)) * 16 + (lane >> 2);
    const int chunk = swz(row, lane & 3);
    const bool in_k = k0 + chunk * 8 < K;
    const uint32_t voff = in_k ? t.off[u] + (uint32_t)(k0 * 2) : kOob;
    uint8_t* dst = lds_tile + (u * 4 + (threadIdx.x >> 6)) * 16 * kRowBytes;
    buffer_load_lds(t.rsrc, (lds_ptr_t)dst, 16, (int)voff, 0, 0, 0);
  }
}

struct Frags {
  bf16x8 a[4];
  bf16x8 b[4];
};

// Operand fragments of k-step ks (0 or 1) of a staged k-block.
__device__ inline void read_frags(const uint8_t* As, const uint8_t* Bs, int wm, int wn, int lane,
                                  int ks, Frags& f) {
  const int r = lane & 31;
  const int c = ks * 2 + (lane >> 5);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wm * 128 + i * 32 + r;
    f.a[i] = *reinterpret_cast<const bf16x8*>(As + row * kRowBytes + (swz(row, c) << 4));
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = wn * 128 + j * 32 + r;
    f.b[j] = *reinterpret_cast<const bf16x8*>(Bs + row * kRowBytes + (swz(row, c) << 4));
  }
}

__device__ inline void mma_frags(const Frags& f, Acc& acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc.t[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc.t[i][j], 0, 0, 0);
}

// Instruction interleaving. A wave issues MFMAs one at a time and waits for
// the matrix core to accept each; other instructions placed between two MFMAs
// issue in the shadow of the first for free. These scheduling groups ask the
// compiler for such an order (the grouped instructions are independent of
// the MFMAs they sit between).
//
// 16 MFMAs, the first 8 each followed by one LDS read.
__device__ inline void sched_mfma_lds() {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
}
// 16 - kPreBarrier MFMAs: 8 each followed by a global->LDS load, then the rest
// each followed by an LDS read.
constexpr int kPreBarrier = 2;  // MFMAs issued before the barrier (see mainloop)
__device__ inline void sched_mfma_vmem_lds() {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (to LDS)
  }
#pragma unroll
  for (int i = 0; i < 8 - kPreBarrier; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
}

// MFMA q (0..15) of a k-step: tile (q / 4, q % 4).
__device__ inline void mma_one(const Frags& f, Acc& acc, int q) {
  acc.t[q / 4][q % 4] =
      __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[q / 4], f.b[q % 4], acc.t[q / 4][q % 4], 0, 0, 0);
}

// Main loop for the tile at (m0, n0). `smem` holds kLdsBytes (16-byte aligned).
//
// Steady state, per k-block kt (two 16-deep k-steps, 16 MFMAs each):
//   MFMAs (kt, 0), interleaved with the LDS reads of fragments (kt, 1)
//   kPreBarrier MFMAs of (kt, 1), so the matrix core stays busy while the
//   wave waits for stage kt+1 and the workgroup barrier
//   the other MFMAs of (kt, 1), interleaved with the global->LDS loads of
//   stage kt+3 (into the buffer of stage kt-1, which every wave finished
//   reading before the barrier) and the LDS reads of fragments (kt+1, 0)
// Global loads run two to three k-blocks ahead. The last kStages-1 k-blocks
// issue no loads and run a plain drain loop, so the steady-state body has no
// branches (a branch there splits the interleaved block and makes the
// register allocator shuffle the accumulators).
//
// Measured at 8192 x 128256 x 4096 (main loop only, on MI355X): 1446
// TFLOP/s, against 1219 TFLOP/s with the LDS reads and loads issued in
// blocks between the MFMA groups.
__device__ inline void mainloop(const __bf16* __restrict__ A, int64_t lda, int64_t M,
                                const __bf16* __restrict__ B, int64_t ldb, int64_t N, int64_t K,
                                int64_t m0, int64_t n0, uint8_t* smem, Acc& acc) {
  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wm = wid >> 1;
  const int wn = wid & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc.t[i][j][e] = 0.f;

  const TileLoader la = make_loader(A, lda, M, m0);
  const TileLoader lb = make_loader(B, ldb, N, n0);
  const int64_t KT = (K + BK - 1) / BK;
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) {
    if (s < KT) {
      issue_loads(la, (int64_t)s * BK, K, smem + s * kStageBytes);
      issue_loads(lb, (int64_t)s * BK, K, smem + s * kStageBytes + kTileBytes);
    }
  }
  // stage 0 landed (stages 1 .. kStages-2 may still be in flight)
  wait_stage(KT - 1 < kStages - 2 ? KT - 1 : kStages - 2);
  __builtin_amdgcn_s_barrier();
  Frags f0, f1;
  read_frags(smem, smem + kTileBytes, wm, wn, lane, 0, f0);

  int64_t kt = 0;
  for (; kt + kStages - 1 < KT; ++kt) {
    const uint8_t* As = smem + (kt % kStages) * kStageBytes;
    read_frags(As, As + kTileBytes, wm, wn, lane, 1, f1);
    mma_frags(f0, acc);
    sched_mfma_lds();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kPreBarrier; ++q) mma_one(f1, acc, q);
    __builtin_amdgcn_sched_barrier(0);
    // stage kt+1 landed: stages kt+2 .. kt+kStages-2 may remain in flight
    wait_stage(kStages - 3);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const int s = (int)((kt + kStages - 1) % kStages);
    issue_loads(la, (kt + kStages - 1) * BK, K, smem + s * kStageBytes);
    issue_loads(lb, (kt + kStages - 1) * BK, K, smem + s * kStageBytes + kTileBytes);
    const uint8_t* An = smem + ((kt + 1) % kStages) * kStageBytes;
    read_frags(An, An + kTileBytes, wm, wn, lane, 0, f0);
#pragma unroll
    for (int q = kPreBarrier; q < 16; ++q) mma_one(f1, acc, q);
    sched_mfma_vmem_lds();
    __builtin_amdgcn_sched_barrier(0);
  }
  // drain: the last k-blocks, no loads left to issue
  for (; kt < KT; ++kt) {
    const uint8_t* As = smem + (kt % kStages) * kStageBytes;
    read_frags(As, As + kTileBytes, wm, wn, lane, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    mma_frags(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < KT) {
      const int64_t later = KT - 2 - kt;
      wait_stage(later < kStages - 3 ? later : kStages - 3);
      __builtin_amdgcn_s_barrier();
      const uint8_t* An = smem + ((kt + 1) % kStages) * kStageBytes;
      read_frags(An, An + kTileBytes, wm, wn, lane, 0, f0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma_frags(f1, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Row / column (within the workgroup tile) of accumulator element e of tile (i, j).
__device__ inline int acc_row(int wm, int i, int e, int lane) {
  return wm * 128 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
__device__ inline int acc_col(int wn, int j, int lane) { return wn * 128 + j * 32 + (lane & 31); }

}  // namespace ts_gemm
