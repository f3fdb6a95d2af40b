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
//
// Either operand may instead be stored MN-major (element (r, k) at k * ld + r,
// e.g. dlogits [N, V] read as the [V, N] operand of the weight gradient, or
// the LM head [V, H] read as the [H, V] operand of the hidden gradient). Such
// a tile sits in LDS as 32 k-rows of 256 bf16 (512 B, 16-byte chunks XOR-
// swizzled by k & 3) and the MFMA fragments come out of it transposed by
// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element j of
// the 4 that lane 4j + i/4 addressed, element i % 4 of them (checked on the
// device). So lane s of group g addressing (k = kb + s / 4, r = rb + 4 (s % 4))
// makes lane i of the group receive X[rb + i][kb + j], j < 4: two such reads
// (kb and kb + 4) give the 8 k of an MFMA fragment without a transpose pass.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "common.hpp"
#include "plan.hpp"

namespace ts_gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4* lds_bf16x4_t;

// Storage of a GEMM operand: K-major (element (r, k) at r * ld + k) or
// MN-major (element (r, k) at k * ld + r).
enum Major : int { kKMajor = 0, kMNMajor = 1 };
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

// MN-major tile loads: rows [r0, r0 + 256) of the operand, k-block [k0,
// k0 + 32). LDS byte (kr, p) of the tile (kr < 32, p < 512) holds logical byte
// p ^ ((kr & 3) << 6) of k-row kr: the 16-byte chunk at p is 8 consecutive r.
// A half-wave of ds_read_b64_tr_b16 (see read_op_t) reads 64 bytes from each
// of 4 consecutive k-rows; the swizzle puts them in the 4 distinct 64-byte
// quarters of a 256-byte bank window (XOR in 32-byte units instead measured
// 8% of the kernel's cycles as bank conflicts per operand).
// Wave load u covers LDS chunks [(4u + wid) * 64, +64): k-rows 2 (4u + wid)
// and 2 (4u + wid) + 1.
struct TileLoaderT {
  const __bf16* base;           // element (k = 0, r = r0)
  int64_t ld;                   // elements between consecutive k
  uint32_t off[kLoadsPerWave];  // byte offset within a k-block window, kOob past the rows
  int kr[kLoadsPerWave];        // k-row (0..31) of this lane's chunk
};

__device__ inline int swz_t(int kr) { return (kr & 3) << 6; }

__device__ inline TileLoaderT make_loader_t(const __bf16* g, int64_t ld, int64_t nrows,
                                            int64_t r0) {
  TileLoaderT t;
  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  t.base = g + r0;
  t.ld = ld;
#pragma unroll
  for (int u = 0; u < kLoadsPerWave; ++u) {
    const int c = (u * 4 + wid) * 64 + lane;  // 16-byte LDS chunk of the tile
    const int kr = c >> 5;
    const int lbyte = ((c & 31) << 4) ^ swz_t(kr);  // logical byte within the k-row
    const int64_t r = r0 + (lbyte >> 1);
    t.kr[u] = kr;
    t.off[u] = r < nrows ? (uint32_t)(kr * ld * 2 + lbyte) : kOob;
  }
  return t;
}

// Issues this wave's loads of k-block [k0, k0 + 32) into the LDS tile. The
// buffer resource spans the k-block's 32 k-rows, so offsets stay 32-bit
// whatever the operand's size.
__device__ inline void issue_loads_t(const TileLoaderT& t, int64_t k0, int64_t K,
                                     uint8_t* lds_tile) {
  const i32x4 rsrc = make_rsrc(t.base + k0 * t.ld, (uint64_t)BK * (uint64_t)t.ld * 2);
#pragma unroll
  for (int u = 0; u < kLoadsPerWave; ++u) {
    const uint32_t voff = k0 + t.kr[u] < K ? t.off[u] : kOob;
    uint8_t* dst = lds_tile + (u * 4 + (threadIdx.x >> 6)) * 1024;
    buffer_load_lds(rsrc, (lds_ptr_t)dst, 16, (int)voff, 0, 0, 0);
  }
}

// Fragments (k-step ks) of four 32-row blocks starting at row r_base of a
// K-major tile: one ds_read_b128 each.
__device__ inline void read_op_k(const uint8_t* Xs, int r_base, int lane, int ks, bf16x8* f) {
  const int r = lane & 31;
  const int c = ks * 2 + (lane >> 5);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = r_base + i * 32 + r;
    f[i] = *reinterpret_cast<const bf16x8*>(Xs + row * kRowBytes + (swz(row, c) << 4));
  }
}

// The same fragments from an MN-major tile: two ds_read_b64_tr_b16 each.
__device__ inline void read_op_t(const uint8_t* Xs, int r_base, int lane, int ks, bf16x8* f) {
  const int g = lane >> 4;
  const int sl = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r_base + i * 32 + 16 * (g & 1) + 4 * (sl & 3);
    bf16x4 h[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int k = ks * 16 + 8 * (g >> 1) + 4 * hh + (sl >> 2);
      const int byte = k * 512 + ((2 * r) ^ swz_t(k));
      h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t)(Xs + byte));
    }
    f[i] = __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7);
  }
}

struct Frags {
  bf16x8 a[4];
  bf16x8 b[4];
};

// Loader of one operand of the given storage.
template <int kMajor> struct OpLoader;
template <> struct OpLoader<kKMajor> {
  TileLoader t;
  __device__ inline OpLoader(const __bf16* g, int64_t ld, int64_t nrows, int64_t r0)
      : t(make_loader(g, ld, nrows, r0)) {}
  __device__ inline void issue(int64_t k0, int64_t K, uint8_t* tile) const {
    issue_loads(t, k0, K, tile);
  }
};
template <> struct OpLoader<kMNMajor> {
  TileLoaderT t;
  __device__ inline OpLoader(const __bf16* g, int64_t ld, int64_t nrows, int64_t r0)
      : t(make_loader_t(g, ld, nrows, r0)) {}
  __device__ inline void issue(int64_t k0, int64_t K, uint8_t* tile) const {
    issue_loads_t(t, k0, K, tile);
  }
};

template <int kMajor>
__device__ inline void read_op(const uint8_t* Xs, int r_base, int lane, int ks, bf16x8* f) {
  if constexpr (kMajor == kKMajor) read_op_k(Xs, r_base, lane, ks, f);
  else read_op_t(Xs, r_base, lane, ks, f);
}

// Operand fragments of k-step ks (0 or 1) of a staged k-block.
template <int kMA, int kMB>
__device__ inline void read_frags(const uint8_t* As, const uint8_t* Bs, int wm, int wn, int lane,
                                  int ks, Frags& f) {
  read_op<kMA>(As, wm * 128, lane, ks, f.a);
  read_op<kMB>(Bs, wn * 128, lane, ks, f.b);
}

// LDS read instructions per k-step of read_frags.
template <int kMA, int kMB>
constexpr int lds_reads() {
  return (kMA == kMNMajor ? 8 : 4) + (kMB == kMNMajor ? 8 : 4);
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
template <int kMask, int kCount>
__device__ inline void sched_group() {
  if constexpr (kCount > 0) __builtin_amdgcn_sched_group_barrier(kMask, kCount, 0);
}

// 16 MFMAs, the first 8 each followed by kR / 8 LDS reads (kR = 8, 12 or 16
// reads per k-step: two ds_read_b64_tr_b16 per fragment of an MN-major
// operand).
template <int kR, int... I>
__device__ inline void sched_mfma_lds_impl(std::integer_sequence<int, I...>) {
  ((sched_group<0x008, 1>(), sched_group<0x100, (kR + 7 - I) / 8>()), ...);  // MFMA, LDS reads
}
template <int kR>
__device__ inline void sched_mfma_lds() {
  sched_mfma_lds_impl<kR>(std::make_integer_sequence<int, 8>());
  __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
}

// 16 - kPreBarrier MFMAs: 8 each followed by a global->LDS load, then the rest
// each followed by LDS reads. K-major operands (8 reads): one read per slot,
// the other two left to the scheduler, the order measured best; MN-major
// operands: every read placed.
constexpr int kPreBarrier = 2;  // MFMAs issued before the barrier (see mainloop)
constexpr int kLdsSlots = 8 - kPreBarrier;
template <int kR, int... I>
__device__ inline void sched_slots_impl(std::integer_sequence<int, I...>) {
  ((sched_group<0x008, 1>(),
    sched_group<0x100, kR == 8 ? 1 : (kR + kLdsSlots - 1 - I) / kLdsSlots>()),
   ...);
}
template <int kR>
__device__ inline void sched_mfma_vmem_lds() {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (to LDS)
  }
  sched_slots_impl<kR>(std::make_integer_sequence<int, kLdsSlots>());
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
template <int kMA, int kMB>
__device__ inline void mainloop(const __bf16* __restrict__ A, int64_t lda, int64_t M,
                                const __bf16* __restrict__ B, int64_t ldb, int64_t N, int64_t K,
                                int64_t m0, int64_t n0, uint8_t* smem, Acc& acc) {
  constexpr int kR = lds_reads<kMA, kMB>();
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

  const OpLoader<kMA> la(A, lda, M, m0);
  const OpLoader<kMB> lb(B, ldb, N, n0);
  const int64_t KT = (K + BK - 1) / BK;
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) {
    if (s < KT) {
      la.issue((int64_t)s * BK, K, smem + s * kStageBytes);
      lb.issue((int64_t)s * BK, K, smem + s * kStageBytes + kTileBytes);
    }
  }
  // stage 0 landed (stages 1 .. kStages-2 may still be in flight)
  wait_stage(KT - 1 < kStages - 2 ? KT - 1 : kStages - 2);
  __builtin_amdgcn_s_barrier();
  Frags f0, f1;
  read_frags<kMA, kMB>(smem, smem + kTileBytes, wm, wn, lane, 0, f0);

  int64_t kt = 0;
  for (; kt + kStages - 1 < KT; ++kt) {
    const uint8_t* As = smem + (kt % kStages) * kStageBytes;
    read_frags<kMA, kMB>(As, As + kTileBytes, wm, wn, lane, 1, f1);
    mma_frags(f0, acc);
    sched_mfma_lds<kR>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kPreBarrier; ++q) mma_one(f1, acc, q);
    __builtin_amdgcn_sched_barrier(0);
    // stage kt+1 landed: stages kt+2 .. kt+kStages-2 may remain in flight
    wait_stage(kStages - 3);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const int s = (int)((kt + kStages - 1) % kStages);
    la.issue((kt + kStages - 1) * BK, K, smem + s * kStageBytes);
    lb.issue((kt + kStages - 1) * BK, K, smem + s * kStageBytes + kTileBytes);
    const uint8_t* An = smem + ((kt + 1) % kStages) * kStageBytes;
    read_frags<kMA, kMB>(An, An + kTileBytes, wm, wn, lane, 0, f0);
#pragma unroll
    for (int q = kPreBarrier; q < 16; ++q) mma_one(f1, acc, q);
    sched_mfma_vmem_lds<kR>();
    __builtin_amdgcn_sched_barrier(0);
  }
  // drain: the last k-blocks, no loads left to issue
  for (; kt < KT; ++kt) {
    const uint8_t* As = smem + (kt % kStages) * kStageBytes;
    read_frags<kMA, kMB>(As, As + kTileBytes, wm, wn, lane, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    mma_frags(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < KT) {
      const int64_t later = KT - 2 - kt;
      wait_stage(later < kStages - 3 ? later : kStages - 3);
      __builtin_amdgcn_s_barrier();
      const uint8_t* An = smem + ((kt + 1) % kStages) * kStageBytes;
      read_frags<kMA, kMB>(An, An + kTileBytes, wm, wn, lane, 0, f0);
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
