// bf16 MFMA GEMM core for gfx950: C[M, N] = A[M, K] * B[N, K]^T, fp32 accumulation.
//
// Both operands are row-major with K contiguous (the layout of hidden [N, H]
// and of the LM head [V, H]), 16-byte aligned, row strides and K multiples of
// 8 elements.
//
// Workgroup tile 256 x 256, k-block 32. Two wave layouts (template kW):
//   kW = 4: 256 threads in a 2 x 2 grid, each wave a 128 x 128 block of C as
//           4 x 4 tiles of v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per
//           lane), one wave per SIMD;
//   kW = 8: 512 threads in a 4 x 2 grid, each wave a 64 x 128 block (2 x 4
//           tiles, 128 accumulators), two waves per SIMD, so one wave's MFMAs
//           can run while the other waits at the barrier or for LDS data.
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
constexpr int kRowBytes = BK * 2;                       // 64
constexpr int kTileBytes = BM * kRowBytes;              // 16 KiB per operand per stage
constexpr int kStageBytes = 2 * kTileBytes;             // A + B
constexpr size_t kLdsBytes = (size_t)kStages * kStageBytes;
constexpr uint32_t kOob = 0x80000000u;  // voffset beyond every resource's range -> reads 0

// Wave layout: kW waves, wave wid owns rows [wm * RW, +RW) and columns
// [wn * 128, +128) of the tile, wm = wid >> 1, wn = wid & 1.
template <int kW>
struct Cfg {
  static_assert(kW == 4 || kW == 8, "wave layout");
  static constexpr int kThreads = 64 * kW;
  static constexpr int kLoads = 16 / kW;  // 1 KiB loads per wave per operand per k-block
  static constexpr int kTI = 16 / kW;     // 32-row tiles per wave (4 or 2)
  static constexpr int kTJ = 4;           // 32-column tiles per wave
  static constexpr int RW = 32 * kTI;     // rows per wave
  static constexpr int kMfma = kTI * kTJ; // MFMAs per k-step
};

template <int kTI>
struct Acc {
  f32x16 t[kTI][4];
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
// (each stage is 2 * kLoads loads; vmcnt counts loads in issue order).
template <int kW>
__device__ inline void wait_stage(int64_t later) {
  constexpr int kPer = 2 * Cfg<kW>::kLoads;
  static_assert(kPer * 3 < 64, "vmcnt range");
  if (later >= 3) wait_vmcnt<3 * kPer>();
  else if (later == 2) wait_vmcnt<2 * kPer>();
  else if (later == 1) wait_vmcnt<kPer>();
  else wait_vmcnt<0>();
}

// K-major tile loads: rows [row0, row0 + 256) of a [nrows, ld] matrix,
// out-of-range rows read zeros. Wave load u fills LDS rows
// [(u * kW + wid) * 16, +16) (1 KiB); off[u] is this lane's byte offset
// (relative to the tile's first row) of the logical chunk its LDS position
// holds, at k0 = 0.
template <int kW>
struct TileLoader {
  i32x4 rsrc;
  uint32_t off[Cfg<kW>::kLoads];
};

template <int kW>
__device__ inline TileLoader<kW> make_loader(const __bf16* g, int64_t ld, int64_t nrows,
                                             int64_t row0) {
  TileLoader<kW> t;
  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t valid = nrows - row0;
  if (valid > BM) valid = BM;
  if (valid < 0) valid = 0;
  t.rsrc = make_rsrc(g + row0 * ld, (uint64_t)valid * (uint64_t)ld * 2);
#pragma unroll
  for (int u = 0; u < Cfg<kW>::kLoads; ++u) {
    const int row = (u * kW + wid) * 16 + (lane >> 2);
    const int chunk = swz(row, lane & 3);  // the logical chunk LDS position lane&3 holds
    t.off[u] = (uint32_t)(row * ld * 2 + chunk * 16);
  }
  return t;
}

// Issues this wave's loads of k-block [k0, k0 + 32) into the LDS tile.
template <int kW>
__device__ inline void issue_loads(const TileLoader<kW>& t, int64_t k0, int64_t K,
                                   uint8_t* lds_tile) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
#pragma unroll
  for (int u = 0; u < Cfg<kW>::kLoads; ++u) {
    // logical chunk of this lane for the load's row (same swizzle as make_loader)
    const int row = (u * kW + wid) * 16 + (lane >> 2);
    const int chunk = swz(row, lane & 3);
    const bool in_k = k0 + chunk * 8 < K;
    const uint32_t voff = in_k ? t.off[u] + (uint32_t)(k0 * 2) : kOob;
    uint8_t* dst = lds_tile + (u * kW + wid) * 16 * kRowBytes;
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
// Wave load u covers LDS chunks [(u * kW + wid) * 64, +64): k-rows
// 2 (u * kW + wid) and 2 (u * kW + wid) + 1.
template <int kW>
struct TileLoaderT {
  const __bf16* base;              // element (k = 0, r = r0)
  int64_t ld;                      // elements between consecutive k
  uint32_t off[Cfg<kW>::kLoads];   // byte offset within a k-block window, kOob past the rows
  int kr[Cfg<kW>::kLoads];         // k-row (0..31) of this lane's chunk
};

__device__ inline int swz_t(int kr) { return (kr & 3) << 6; }

template <int kW>
__device__ inline TileLoaderT<kW> make_loader_t(const __bf16* g, int64_t ld, int64_t nrows,
                                                int64_t r0) {
  TileLoaderT<kW> t;
  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  t.base = g + r0;
  t.ld = ld;
#pragma unroll
  for (int u = 0; u < Cfg<kW>::kLoads; ++u) {
    const int c = (u * kW + wid) * 64 + lane;  // 16-byte LDS chunk of the tile
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
template <int kW>
__device__ inline void issue_loads_t(const TileLoaderT<kW>& t, int64_t k0, int64_t K,
                                     uint8_t* lds_tile) {
  const i32x4 rsrc = make_rsrc(t.base + k0 * t.ld, (uint64_t)BK * (uint64_t)t.ld * 2);
  const int wid = threadIdx.x >> 6;
#pragma unroll
  for (int u = 0; u < Cfg<kW>::kLoads; ++u) {
    const uint32_t voff = k0 + t.kr[u] < K ? t.off[u] : kOob;
    uint8_t* dst = lds_tile + (u * kW + wid) * 1024;
    buffer_load_lds(rsrc, (lds_ptr_t)dst, 16, (int)voff, 0, 0, 0);
  }
}

// Fragments (k-step ks) of kN 32-row blocks starting at row r_base of a
// K-major tile: one ds_read_b128 each.
template <int kN>
__device__ inline void read_op_k(const uint8_t* Xs, int r_base, int lane, int ks, bf16x8* f) {
  const int r = lane & 31;
  const int c = ks * 2 + (lane >> 5);
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    const int row = r_base + i * 32 + r;
    f[i] = *reinterpret_cast<const bf16x8*>(Xs + row * kRowBytes + (swz(row, c) << 4));
  }
}

// The same fragments from an MN-major tile: two ds_read_b64_tr_b16 each.
template <int kN>
__device__ inline void read_op_t(const uint8_t* Xs, int r_base, int lane, int ks, bf16x8* f) {
  const int g = lane >> 4;
  const int sl = lane & 15;
#pragma unroll
  for (int i = 0; i < kN; ++i) {
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

template <int kTI>
struct Frags {
  bf16x8 a[kTI];
  bf16x8 b[4];
};

// Loader of one operand of the given storage.
template <int kMajor, int kW> struct OpLoader;
template <int kW> struct OpLoader<kKMajor, kW> {
  TileLoader<kW> t;
  __device__ inline OpLoader(const __bf16* g, int64_t ld, int64_t nrows, int64_t r0)
      : t(make_loader<kW>(g, ld, nrows, r0)) {}
  __device__ inline void issue(int64_t k0, int64_t K, uint8_t* tile) const {
    issue_loads<kW>(t, k0, K, tile);
  }
};
template <int kW> struct OpLoader<kMNMajor, kW> {
  TileLoaderT<kW> t;
  __device__ inline OpLoader(const __bf16* g, int64_t ld, int64_t nrows, int64_t r0)
      : t(make_loader_t<kW>(g, ld, nrows, r0)) {}
  __device__ inline void issue(int64_t k0, int64_t K, uint8_t* tile) const {
    issue_loads_t<kW>(t, k0, K, tile);
  }
};

template <int kMajor, int kN>
__device__ inline void read_op(const uint8_t* Xs, int r_base, int lane, int ks, bf16x8* f) {
  if constexpr (kMajor == kKMajor) read_op_k<kN>(Xs, r_base, lane, ks, f);
  else read_op_t<kN>(Xs, r_base, lane, ks, f);
}

// Operand fragments of k-step ks (0 or 1) of a staged k-block.
template <int kMA, int kMB, int kW>
__device__ inline void read_frags(const uint8_t* As, const uint8_t* Bs, int wm, int wn, int lane,
                                  int ks, Frags<Cfg<kW>::kTI>& f) {
  read_op<kMA, Cfg<kW>::kTI>(As, wm * Cfg<kW>::RW, lane, ks, f.a);
  read_op<kMB, 4>(Bs, wn * 128, lane, ks, f.b);
}

// LDS read instructions per k-step of read_frags.
template <int kMA, int kMB, int kW>
constexpr int lds_reads() {
  return (kMA == kMNMajor ? 2 : 1) * Cfg<kW>::kTI + (kMB == kMNMajor ? 2 : 1) * 4;
}

template <int kTI>
__device__ inline void mma_frags(const Frags<kTI>& f, Acc<kTI>& acc) {
#pragma unroll
  for (int i = 0; i < kTI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc.t[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc.t[i][j], 0, 0, 0);
}

// Instruction interleaving. A wave issues MFMAs one at a time and waits for
// the matrix core to accept each; other instructions placed between two MFMAs
// issue in the shadow of the first for free. These scheduling groups ask the
// compiler for such an order (the grouped instructions are independent of
// the MFMAs they sit between).
template <int kMask, int kCount>
__device__ inline void sched_group() {
  if constexpr (kCount > 0) __builtin_amdgcn_sched_group_barrier(kMask, kCount, 0);
}

// kM MFMAs of a k-step, the first kM / 2 each followed by LDS reads (kR in
// all: one ds_read_b128 per K-major fragment, two ds_read_b64_tr_b16 per
// MN-major one).
template <int kR, int kM, int... I>
__device__ inline void sched_mfma_lds_impl(std::integer_sequence<int, I...>) {
  constexpr int kSlots = kM / 2;
  ((sched_group<0x008, 1>(), sched_group<0x100, (kR + kSlots - 1 - I) / kSlots>()), ...);
}
template <int kR, int kM>
__device__ inline void sched_mfma_lds() {
  sched_mfma_lds_impl<kR, kM>(std::make_integer_sequence<int, kM / 2>());
  __builtin_amdgcn_sched_group_barrier(0x008, kM / 2, 0);
}

// The kM - kPre MFMAs after the barrier: the first kV each followed by a
// global->LDS load (kV = this wave's loads per k-block), the rest by LDS
// reads. With 4 waves and K-major operands (8 reads): one read per slot,
// the other two left to the scheduler, the order measured best; otherwise
// every read placed.
// MFMAs issued before the barrier (measured best: 2 with 4 waves; 1 with 8,
// where 0 and 2 were 0.5-1.5% slower at C5).
template <int kW>
constexpr int pre_barrier() { return kW == 4 ? 2 : 1; }
template <int kR, int kW, int... I>
__device__ inline void sched_slots_impl(std::integer_sequence<int, I...>) {
  constexpr int kSlots = sizeof...(I);
  ((sched_group<0x008, 1>(),
    sched_group<0x100, (kW == 4 && kR == 8) ? 1 : (kR + kSlots - 1 - I) / kSlots>()),
   ...);
}
template <int kR, int kW>
__device__ inline void sched_mfma_vmem_lds() {
  constexpr int kV = 2 * Cfg<kW>::kLoads;
  constexpr int kSlots = Cfg<kW>::kMfma - pre_barrier<kW>() - kV;
  static_assert(kSlots > 0, "schedule slots");
#pragma unroll
  for (int i = 0; i < kV; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read (to LDS)
  }
  sched_slots_impl<kR, kW>(std::make_integer_sequence<int, kSlots>());
}

// MFMA q (0..kTI*4-1) of a k-step: tile (q / 4, q % 4).
template <int kTI>
__device__ inline void mma_one(const Frags<kTI>& f, Acc<kTI>& acc, int q) {
  acc.t[q / 4][q % 4] =
      __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[q / 4], f.b[q % 4], acc.t[q / 4][q % 4], 0, 0, 0);
}

// Main loop for the tile at (m0, n0). `smem` holds kLdsBytes (16-byte aligned).
//
// Steady state, per k-block kt (two 16-deep k-steps):
//   MFMAs (kt, 0), interleaved with the LDS reads of fragments (kt, 1)
//   kPre MFMAs of (kt, 1), so the matrix core stays busy while the wave
//   waits for stage kt+1 and the workgroup barrier
//   the other MFMAs of (kt, 1), interleaved with the global->LDS loads of
//   stage kt+3 (into the buffer of stage kt-1, which every wave finished
//   reading before the barrier) and the LDS reads of fragments (kt+1, 0)
// Global loads run two to three k-blocks ahead. The last kStages-1 k-blocks
// issue no loads and run a plain drain loop, so the steady-state body has no
// branches (a branch there splits the interleaved block and makes the
// register allocator shuffle the accumulators).
//
// Measured at 8192 x 128256 x 4096 (main loop only, on MI355X, 4 waves): 1446
// TFLOP/s, against 1219 TFLOP/s with the LDS reads and loads issued in
// blocks between the MFMA groups.
template <int kMA, int kMB, int kW>
__device__ inline void mainloop(const __bf16* __restrict__ A, int64_t lda, int64_t M,
                                const __bf16* __restrict__ B, int64_t ldb, int64_t N, int64_t K,
                                int64_t m0, int64_t n0, uint8_t* smem, Acc<Cfg<kW>::kTI>& acc) {
  using C = Cfg<kW>;
  constexpr int kR = lds_reads<kMA, kMB, kW>();
  constexpr int kPre = pre_barrier<kW>();
  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wm = wid >> 1;
  const int wn = wid & 1;
#pragma unroll
  for (int i = 0; i < C::kTI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc.t[i][j][e] = 0.f;

  const OpLoader<kMA, kW> la(A, lda, M, m0);
  const OpLoader<kMB, kW> lb(B, ldb, N, n0);
  const int64_t KT = (K + BK - 1) / BK;
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) {
    if (s < KT) {
      la.issue((int64_t)s * BK, K, smem + s * kStageBytes);
      lb.issue((int64_t)s * BK, K, smem + s * kStageBytes + kTileBytes);
    }
  }
  // stage 0 landed (stages 1 .. kStages-2 may still be in flight)
  wait_stage<kW>(KT - 1 < kStages - 2 ? KT - 1 : kStages - 2);
  __builtin_amdgcn_s_barrier();
  Frags<C::kTI> f0, f1;
  read_frags<kMA, kMB, kW>(smem, smem + kTileBytes, wm, wn, lane, 0, f0);

  int64_t kt = 0;
  for (; kt + kStages - 1 < KT; ++kt) {
    const uint8_t* As = smem + (kt % kStages) * kStageBytes;
    read_frags<kMA, kMB, kW>(As, As + kTileBytes, wm, wn, lane, 1, f1);
    mma_frags(f0, acc);
    sched_mfma_lds<kR, C::kMfma>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kPre; ++q) mma_one(f1, acc, q);
    __builtin_amdgcn_sched_barrier(0);
    // stage kt+1 landed: stages kt+2 .. kt+kStages-2 may remain in flight
    wait_stage<kW>(kStages - 3);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const int s = (int)((kt + kStages - 1) % kStages);
    la.issue((kt + kStages - 1) * BK, K, smem + s * kStageBytes);
    lb.issue((kt + kStages - 1) * BK, K, smem + s * kStageBytes + kTileBytes);
    const uint8_t* An = smem + ((kt + 1) % kStages) * kStageBytes;
    read_frags<kMA, kMB, kW>(An, An + kTileBytes, wm, wn, lane, 0, f0);
#pragma unroll
    for (int q = kPre; q < C::kMfma; ++q) mma_one(f1, acc, q);
    sched_mfma_vmem_lds<kR, kW>();
    __builtin_amdgcn_sched_barrier(0);
  }
  // drain: the last k-blocks, no loads left to issue
  for (; kt < KT; ++kt) {
    const uint8_t* As = smem + (kt % kStages) * kStageBytes;
    read_frags<kMA, kMB, kW>(As, As + kTileBytes, wm, wn, lane, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    mma_frags(f0, acc);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < KT) {
      const int64_t later = KT - 2 - kt;
      wait_stage<kW>(later < kStages - 3 ? later : kStages - 3);
      __builtin_amdgcn_s_barrier();
      const uint8_t* An = smem + ((kt + 1) % kStages) * kStageBytes;
      read_frags<kMA, kMB, kW>(An, An + kTileBytes, wm, wn, lane, 0, f0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma_frags(f1, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
}

}  // namespace ts_gemm
