// Fused linear cross-entropy for gfx950: loss, grad_hidden and grad_weight of
//   logits = hidden [N, H] @ weight[V, H]^T,  loss = reduce_rows(lse - logits[label])
// without a library GEMM and without autograd.
//
// Token-chunked: for each chunk of Nc rows of hidden,
//   1. logits GEMM (MFMA, gemm.hpp). Its epilogue rounds the fp32 accumulators
//      to bf16 (the logits the reference's bf16 matmul produces,
//      rl_training.py:177), stores them to an [Nc, V] scratch, and from the
//      same bf16 values writes per (row, 128-column slice) max and sum of
//      exp.
//   2. row statistics -> lse; per-row loss = lse - the stored logit at the
//      label (0 on ignore_index rows).
//   3. dlogits = (softmax - onehot) * scale in bf16, written over the logits
//      scratch (scale = 1/n_valid for the mean, 1 for the sum).
//   4. grad_hidden[chunk] = dlogits @ weight   (MFMA; the weight is read in
//      place as the MN-major [H, V] operand)
//   5. grad_weight      += dlogits^T @ hidden  (MFMA; dlogits and hidden are
//      read in place as MN-major operands); with several chunks the sum is
//      carried in fp32 and rounded once, or (TS_FLCE_ACCUM_BF16) kept in the
//      bf16 output and rounded after every chunk.
//   No operand is transposed in memory: gemm.hpp reads MN-major tiles with
//   transposing LDS loads.
// Every reduction has a fixed order, so results are bit-reproducible.
//
// Scratch lives in a caller workspace (ts_flce_workspace_size): with one chunk
// the full [N, V] logits are staged (2.1 GB at N = 8192, V = 128256); the
// chunk size bounds that at Nc x V x 2 bytes.
#include <math.h>


#include "common.hpp"
#include "gemm.hpp"

namespace {

using namespace ts;
using ts_gemm::Acc;
using ts_gemm::BM;
using ts_gemm::BN;

constexpr int kStagePitch = 256;  // bytes per staged epilogue row (128 bf16)

enum EpiMode : int {
  kEpiLogits = 0,     // bf16 C + row statistics
  kEpiBf16 = 1,       // bf16 C
  kEpiF32 = 2,        // fp32 C32 = acc
  kEpiAccF32 = 3,     // fp32 C32 += acc
  kEpiAccBf16 = 4,    // bf16 C = C32 + acc
  kEpiStats = 5,      // row statistics of the transformed logits + the label's value (and,
                      // when C is not NULL, the bf16 logits in C)
  kEpiDlogits = 6,    // bf16 C = dlogits of the transformed logits (lse known)
  kEpiAddBf16 = 7     // bf16 C = bf16(C + acc): a running sum kept in the bf16 output
};

// Transform of the bf16-rounded logits z, in the order of selective_log_softmax
// (rl_training.py:114-122): softcapping, then scaling, then temperature:
//   t = (softcap > 0 ? softcap * tanh(z / softcap) : z) * mul,
//   mul = (scale > 0 ? scale : 1) / temperature,
//   dt/dz = (softcap > 0 ? 1 - tanh(z / softcap)^2 : 1) * mul.
struct LogitXform {
  float softcap;      // 0: off
  float inv_softcap;  // 1 / softcap
  float mul;
  __device__ inline bool on() const { return softcap > 0.f || mul != 1.f; }
  __device__ inline float apply(float z) const {
    return (softcap > 0.f ? softcap * tanhf(z * inv_softcap) : z) * mul;
  }
  // t and dt/dz
  __device__ inline float apply_d(float z, float& dt) const {
    if (softcap > 0.f) {
      const float th = tanhf(z * inv_softcap);
      dt = (1.f - th * th) * mul;
      return softcap * th * mul;
    }
    dt = mul;
    return z * mul;
  }
};

// A [M, K] and B [N, K] of C = A B^T; lda / ldb are the strides between
// consecutive rows of a K-major operand, or between consecutive k of an
// MN-major one (flce_gemm's kMA / kMB).
struct GemmArgs {
  const __bf16* A;
  int64_t lda;
  const __bf16* B;
  int64_t ldb;
  int64_t M, N, K;
  __bf16* C;      // bf16 output (modes 0, 1, 4, 6, 7; optional in 5)
  int64_t ldc;
  float* C32;     // fp32 accumulator (modes 2, 3, 4)
  int64_t ldc32;
  // logits epilogue
  float2* stats;          // [M][2 * NT] (max, sum exp) per 128-column slice
  // statistics / dlogits epilogues (kEpiStats, kEpiDlogits)
  const int64_t* labels;  // [M]; column of row r's label = labels[r] - label_offset
  int64_t label_offset;
  float* zlab;            // [M] transformed logit at the label (kEpiStats)
  const float* lse;       // [M] (kEpiDlogits)
  const float* dscale;    // [M] d(loss)/d(row loss), 0 on ignored rows (kEpiDlogits)
  LogitXform xf;
};

// Writes the wave's RW x 128 accumulator block (RW = 32 * kTI), rounded to
// bf16, into its private LDS region as [row][col] with 256-byte rows.
template <int kTI>
__device__ inline void stage_bf16(const Acc<kTI>& acc, uint8_t* region, int lane) {
#pragma unroll
  for (int i = 0; i < kTI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int col = j * 32 + (lane & 31);
        *reinterpret_cast<__bf16*>(region + row * kStagePitch + col * 2) = (__bf16)acc.t[i][j][e];
      }
}

// Writes rows [32 i, 32 i + 32) of the wave's fp32 accumulator block (tile
// row i) into its private LDS region as [row][col] fp32 with 512-byte rows
// (16 KiB).
template <int kTI>
__device__ inline void stage_f32_tile(const Acc<kTI>& acc, int i, uint8_t* region, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int row = 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      const int col = j * 32 + (lane & 31);
      *reinterpret_cast<float*>(region + row * 512 + col * 4) = acc.t[i][j][e];
    }
}

// One 256 x 256 tile of C = A B^T with kW waves (ts_gemm::Cfg) and the
// epilogue of kMode: tile number `bid` of the GEMM (ts_plan::gemm_tile_of
// maps it to a tile), `smem` the workgroup's kLdsBytes of LDS.
template <int kMode, int kMA, int kMB, int kW>
__device__ inline void gemm_tile(const GemmArgs& a, int64_t bid, uint8_t* smem) {
  using Cw = ts_gemm::Cfg<kW>;
  constexpr int kTI = Cw::kTI;
  const int64_t MT = (a.M + BM - 1) / BM;
  const int64_t NT = (a.N + BN - 1) / BN;
  int64_t mt, nt;
  ts_plan::gemm_tile_of(bid, MT, NT, mt, nt);
  const int64_t m0 = mt * BM;
  const int64_t n0 = nt * BN;
  Acc<kTI> acc;
  ts_gemm::mainloop<kMA, kMB, kW>(a.A, a.lda, a.M, a.B, a.ldb, a.N, a.K, m0, n0, smem, acc);

  const int wid = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wm = wid >> 1;
  const int wn = wid & 1;
  const int64_t mb = m0 + wm * Cw::RW;  // first row of this wave's block
  const int64_t nb = n0 + wn * 128;     // first column
  // Every wave is done with the pipeline's LDS before it is reused. Each wave
  // then works in its own region (kLdsBytes / kW: 32 KiB with 4 waves, 16 KiB
  // with 8); LDS operations of one wave complete in order, so it reads back
  // its own writes without a barrier.
  constexpr int kRegion = (int)(ts_gemm::kLdsBytes / kW);
  static_assert(kRegion >= Cw::RW * kStagePitch && kRegion >= 32 * 512, "epilogue region");
  __syncthreads();
  uint8_t* region = smem + wid * kRegion;

  if constexpr (kMode == kEpiAddBf16) {
    // bf16 running sum C = bf16(C + acc): a lane owns 8 consecutive columns (16 bytes of
    // C) of a 128-column row, 16 lanes a row, 4 rows a step. All 8 steps' old values of a
    // 32-row tile are loaded before that tile is staged, so their latency overlaps the
    // staging; the loads and stores are 16 bytes wide (measured on MI355X at the C5
    // chunk shape: the gradient pair 3.57-3.59 ms against 3.65 ms with 8-byte accesses,
    // 32 lanes a row).
    const int c8 = lane & 15;
    const int64_t gc = nb + c8 * 8;
#pragma unroll
    for (int i = 0; i < kTI; ++i) {
      const int64_t gm0 = mb + i * 32 + (lane >> 4);  // this lane's row at step s: gm0 + 4 s
      u32x4 old[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int64_t gm = gm0 + 4 * s;
        // N % 8 == 0: a lane's 8 columns are all in or all out
        old[s] = gm < a.M && gc < a.N ? ld16(a.C + gm * a.ldc + gc) : u32x4{0u, 0u, 0u, 0u};
      }
      stage_f32_tile(acc, i, region, lane);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int lrow = 4 * s + (lane >> 4);
        const int64_t gm = gm0 + 4 * s;
        if (gm < a.M && gc < a.N) {
          const float4 v0 = *reinterpret_cast<const float4*>(region + lrow * 512 + c8 * 32);
          const float4 v1 = *reinterpret_cast<const float4*>(region + lrow * 512 + c8 * 32 + 16);
          float f[8];
          Elt<__bf16>::unpack(old[s], f);
          f[0] += v0.x;
          f[1] += v0.y;
          f[2] += v0.z;
          f[3] += v0.w;
          f[4] += v1.x;
          f[5] += v1.y;
          f[6] += v1.z;
          f[7] += v1.w;
          st16(a.C + gm * a.ldc + gc, Elt<__bf16>::pack(f));
        }
      }
    }
  } else if constexpr (kMode == kEpiF32 || kMode == kEpiAccF32 || kMode == kEpiAccBf16) {
    // fp32 C32 rows of 128 columns = 512 B: 32 lanes x 16 B per row, 2 rows per step.
    // The modes that add to what C32 holds load the old values of 8 steps at a time
    // (16-byte fp32 values; more would exceed the register budget), the first batch
    // before the tile is staged, so the loads' latency overlaps the staging instead of
    // stalling step after step.
    const int c4 = lane & 31;
    const int64_t gc = nb + c4 * 4;
    constexpr bool kAddOld = kMode == kEpiAccF32 || kMode == kEpiAccBf16;
    constexpr int kPre = kAddOld ? 8 : 16;
#pragma unroll
    for (int i = 0; i < kTI; ++i) {
      const int64_t gm0 = mb + i * 32 + (lane >> 5);  // this lane's row at step it: gm0 + 2 it
#pragma unroll
      for (int h = 0; h < 16; h += kPre) {
        float4 old[kAddOld ? kPre : 1];
        if constexpr (kAddOld) {
#pragma unroll
          for (int q = 0; q < kPre; ++q) {
            const int64_t gm = gm0 + 2 * (h + q);
            const bool in = gm < a.M && gc < a.N;  // N % 8 == 0: 4 columns all in or all out
            old[q] = in ? *reinterpret_cast<const float4*>(a.C32 + gm * a.ldc32 + gc)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
        if (h == 0) stage_f32_tile(acc, i, region, lane);
#pragma unroll
        for (int q = 0; q < kPre; ++q) {
          const int it = h + q;
          const int lrow = it * 2 + (lane >> 5);
          const int64_t gm = gm0 + 2 * it;
          if (gm < a.M && gc < a.N) {
            float4 v = *reinterpret_cast<const float4*>(region + lrow * 512 + c4 * 16);
            if constexpr (kAddOld) {
              const float4 o = old[q];
              v.x += o.x;
              v.y += o.y;
              v.z += o.z;
              v.w += o.w;
            }
            if constexpr (kMode == kEpiAccBf16) {
              bf16x2_t lo = {(__bf16)v.x, (__bf16)v.y};
              bf16x2_t hi = {(__bf16)v.z, (__bf16)v.w};
              uint2 pk;
              pk.x = __builtin_bit_cast(uint32_t, lo);
              pk.y = __builtin_bit_cast(uint32_t, hi);
              *reinterpret_cast<uint2*>(a.C + gm * a.ldc + gc) = pk;
            } else {
              *reinterpret_cast<float4*>(a.C32 + gm * a.ldc32 + gc) = v;
            }
          }
        }
      }
    }
  } else {
    stage_bf16(acc, region, lane);
    const int c16 = lane & 15;  // 16-byte chunk of the 256-byte row
    const int64_t nparts = 2 * ((a.N + BN - 1) / BN);
    // Row operands of the statistics and dlogits epilogues: lane i holds those
    // of the wave's row mb + i; the 16 lanes that handle a row fetch them with
    // ds_bpermute. rel_lab is the label's column in C, -1 when outside it.
    int rel_lab = -1;
    float lse2 = 0.f, dsc = 0.f;
    if constexpr (kMode == kEpiStats || kMode == kEpiDlogits) {
      static_assert(Cw::RW == 64, "one row per lane");
      const int64_t r = mb + lane;
      if (r < a.M) {
        const int64_t c = a.labels[r] - a.label_offset;
        rel_lab = c >= 0 && c < a.N ? (int)c : -1;
        if constexpr (kMode == kEpiDlogits) {
          lse2 = a.lse[r] * kLog2e;
          dsc = a.dscale[r];
        }
      }
    }
    const bool xf_on = a.xf.on();
#pragma unroll 4
    for (int it = 0; it < Cw::RW / 4; ++it) {
      const int lrow = it * 4 + (lane >> 4);
      const int64_t gm = mb + lrow;
      const int64_t gc = nb + c16 * 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(region + lrow * kStagePitch + c16 * 16);
      // a chunk of 8 columns is stored whole when it starts inside C (rows of C are
      // padded to whole chunks: ldc >= round_up(N, 8)); nin of its columns are < N,
      // fewer than 8 only in the last chunk when N % 8 != 0
      const bool in = gm < a.M && gc < a.N;
      const int nin = in ? (a.N - gc < 8 ? (int)(a.N - gc) : 8) : 0;
      if constexpr (kMode == kEpiLogits || kMode == kEpiBf16) {
        if (in) st16(a.C + gm * a.ldc + gc, v);
      }
      if constexpr (kMode == kEpiStats) {
        // statistics of t over the row's 128-column slice, and t at the label; the
        // logits themselves when the caller keeps them for the backward
        if (in && a.C != nullptr) st16(a.C + gm * a.ldc + gc, v);
        float f[8];
        Elt<__bf16>::unpack(v, f);
        if (xf_on) {
#pragma unroll
          for (int q = 0; q < 8; ++q) f[q] = a.xf.apply(f[q]);
        }
        if (nin < 8) {  // columns past N take no part in the statistics
#pragma unroll
          for (int q = 0; q < 8; ++q) f[q] = q < nin ? f[q] : -INFINITY;
        }
        float lm = f[0];
#pragma unroll
        for (int q = 1; q < 8; ++q) lm = fmaxf(lm, f[q]);
        const float m = row_max(in ? lm : -INFINITY);  // over the 16 lanes of this row
        float ls = 0.f;
        if (in) {
          const float mb2 = m * kLog2e;
#pragma unroll
          for (int q = 0; q < 8; ++q) ls += fast_exp2(__builtin_fmaf(f[q], kLog2e, -mb2));
        }
        const float s = row_sum(ls);
        if (gm < a.M && c16 == 0) a.stats[gm * nparts + nt * 2 + wn] = make_float2(m, s);
        const int d = __shfl(rel_lab, lrow) - (int)gc;
        if (in && (unsigned)d < 8u) {
          float zl = f[0];
#pragma unroll
          for (int q = 1; q < 8; ++q) zl = d == q ? f[q] : zl;
          a.zlab[gm] = zl;
        }
      }
      if constexpr (kMode == kEpiDlogits) {
        // (exp(t - lse) - onehot) * dt/dz * dscale, rounded to bf16
        const float l2 = __shfl(lse2, lrow);
        const float ds = __shfl(dsc, lrow);
        const int d = __shfl(rel_lab, lrow) - (int)gc;
        float f[8], g[8];
        Elt<__bf16>::unpack(v, f);
        if (!xf_on) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pr = fast_exp2(__builtin_fmaf(f[e], kLog2e, -l2));
            g[e] = ds * (e == d ? pr - 1.f : pr);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float dt;
            const float t = a.xf.apply_d(f[e], dt);
            const float pr = fast_exp2(__builtin_fmaf(t, kLog2e, -l2));
            g[e] = ds * (e == d ? pr - 1.f : pr) * dt;
          }
        }
        if (nin < 8) {  // columns past N: zero, the gradient GEMMs read them
#pragma unroll
          for (int e = 0; e < 8; ++e) g[e] = e < nin ? g[e] : 0.f;
        }
        if (in) st16(a.C + gm * a.ldc + gc, Elt<__bf16>::pack(g));
      }
      if constexpr (kMode == kEpiLogits) {
        float f[8];
        Elt<__bf16>::unpack(v, f);
        if (nin < 8) {  // columns past N take no part in the statistics
#pragma unroll
          for (int q = 0; q < 8; ++q) f[q] = q < nin ? f[q] : -INFINITY;
        }
        float lm = f[0];
#pragma unroll
        for (int q = 1; q < 8; ++q) lm = fmaxf(lm, f[q]);
        const float m = row_max(in ? lm : -INFINITY);  // over the 16 lanes of this row
        float ls = 0.f;
        if (in) {
          const float mb = m * kLog2e;
#pragma unroll
          for (int q = 0; q < 8; ++q) ls += fast_exp2(__builtin_fmaf(f[q], kLog2e, -mb));
        }
        const float s = row_sum(ls);
        if (gm < a.M && c16 == 0) a.stats[gm * nparts + nt * 2 + wn] = make_float2(m, s);
      }
    }
  }
}

template <int kMode, int kMA, int kMB, int kW>
__global__ __launch_bounds__(64 * kW) __attribute__((amdgpu_waves_per_eu(kW / 4, kW / 4)))
void flce_gemm(const GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[ts_gemm::kLdsBytes];
  gemm_tile<kMode, kMA, kMB, kW>(a, blockIdx.x, smem);
}

// Two independent GEMMs in one grid: workgroups [0, tiles1) compute the first,
// the others the second. The two gradient GEMMs of a token chunk read the same
// dlogits; with few tokens per chunk the grad_hidden GEMM has fewer (and much
// longer) tiles than the GPU has CUs, and the grad_weight tiles, dispatched
// after them, fill the remaining CUs. With tiles1 a multiple of 8 both GEMMs
// keep their XCD tile grouping.
template <int kMode1, int kMA1, int kMB1, int kMode2, int kMA2, int kMB2, int kW>
__global__ __launch_bounds__(64 * kW) __attribute__((amdgpu_waves_per_eu(kW / 4, kW / 4)))
void flce_gemm_pair(const GemmArgs a1, const GemmArgs a2, int64_t tiles1) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[ts_gemm::kLdsBytes];
  const int64_t bid = blockIdx.x;
  if (bid < tiles1) gemm_tile<kMode1, kMA1, kMB1, kW>(a1, bid, smem);
  else gemm_tile<kMode2, kMA2, kMB2, kW>(a2, bid - tiles1, smem);
}

// n_valid = #labels != ignore_index over all N rows (one workgroup, fixed order).
__global__ __launch_bounds__(256) void flce_count(const int64_t* __restrict__ labels, int64_t N,
                                                  int64_t ignore_index, int* __restrict__ n_valid) {
  __shared__ float red[4];
  float c = 0.f;
  for (int64_t i = threadIdx.x; i < N; i += 256) c += labels[i] != ignore_index ? 1.f : 0.f;
  c = block_sum<4>(c, red);
  if (threadIdx.x == 0) *n_valid = (int)c;
}

// Row waves per workgroup of the one-wave-per-row kernels.
constexpr int kRowWaves = 4;

// Per row of a chunk (one wave per row): lse from the row's slice statistics
// (contiguous [nparts] float2), loss = lse - z[label] with z[label] read from
// the chunk's bf16 logits. Fixed combination order: lane-strided partial
// (max, sum) pairs, then a DPP/lane-read fold.
__global__ __launch_bounds__(64 * kRowWaves) void flce_rows(const float2* __restrict__ stats, int64_t nparts,
                                                 const __bf16* __restrict__ logits, int64_t ldl,
                                                 const int64_t* __restrict__ labels, int64_t M,
                                                 int64_t V, int64_t ignore_index,
                                                 float* __restrict__ lse_out,
                                                 float* __restrict__ loss_rows) {
  const int64_t r = ts_plan::wave_row(blockIdx.x, threadIdx.x >> 6, kRowWaves);
  const int lane = threadIdx.x & 63;
  if (r >= M) return;  // wave-uniform
  const float2* sr = stats + r * nparts;
  float m = -INFINITY;
  for (int64_t p = lane; p < nparts; p += 64) m = fmaxf(m, sr[p].x);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t p = lane; p < nparts; p += 64) {
    const float2 st = sr[p];
    s += st.y == 0.f ? 0.f : st.y * fast_exp2((st.x - m) * kLog2e);
  }
  s = wave_sum(s);
  if (lane != 0) return;
  const float l = m + logf(s);
  const int64_t col = ts_plan::label_col(labels[r], V, ignore_index);
  float out;
  if (col == ts_plan::kLabelIgnored) out = 0.f;
  else if (col == ts_plan::kLabelOutside) out = __builtin_nanf("");
  else out = l - Elt<__bf16>::load1(logits + r * ldl + col);
  lse_out[r] = l;
  loss_rows[r] = out;
}

// Two-pass schedule, forward: per row (one wave per row) lse from the slice
// statistics of the transformed logits t, and loss = lse - t[label] with
// t[label] from zlab, written by the statistics epilogue (0 on ignore_index
// rows, NaN for other labels outside [0, V)).
__global__ __launch_bounds__(64 * kRowWaves) void flce_rows_t(const float2* __restrict__ stats,
                                                   int64_t nparts, const float* __restrict__ zlab,
                                                   const int64_t* __restrict__ labels, int64_t M,
                                                   int64_t V, int64_t ignore_index,
                                                   float* __restrict__ lse_out,
                                                   float* __restrict__ loss_rows) {
  const int64_t r = ts_plan::wave_row(blockIdx.x, threadIdx.x >> 6, kRowWaves);
  const int lane = threadIdx.x & 63;
  if (r >= M) return;  // wave-uniform
  const float2* sr = stats + r * nparts;
  float m = -INFINITY;
  for (int64_t p = lane; p < nparts; p += 64) m = fmaxf(m, sr[p].x);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t p = lane; p < nparts; p += 64) {
    const float2 st = sr[p];
    s += st.y == 0.f ? 0.f : st.y * fast_exp2((st.x - m) * kLog2e);
  }
  s = wave_sum(s);
  if (lane != 0) return;
  const float l = m + logf(s);
  const int64_t col = ts_plan::label_col(labels[r], V, ignore_index);
  float out;
  if (col == ts_plan::kLabelIgnored) out = 0.f;
  else if (col == ts_plan::kLabelOutside) out = __builtin_nanf("");
  else out = l - zlab[r];
  lse_out[r] = l;
  loss_rows[r] = out;
}

// Two-pass schedule, backward: d(loss)/d(row loss) per row,
//   dscale[r] = dloss[r * stride] * (mean ? 1 / max(n_valid, 1) : 1),
// 0 on ignore_index rows.
__global__ __launch_bounds__(256) void flce_dscale(const int64_t* __restrict__ labels, int64_t N,
                                                   int64_t ignore_index,
                                                   const float* __restrict__ dloss,
                                                   int64_t stride, const int* __restrict__ n_valid,
                                                   int mean, float* __restrict__ dscale) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= N) return;
  const float sc = mean ? 1.f / (float)(*n_valid > 0 ? *n_valid : 1) : 1.f;
  dscale[r] = labels[r] == ignore_index ? 0.f : dloss[r * stride] * sc;
}

// Vocabulary-parallel linear CE, one rank. The 16-byte per-row partial the
// ranks exchange: {lse over the shard, the label's logit if the shard holds
// it (else 0), 0, 0} (the layout of ts_ce_vocab_shard_stats).
struct ShardStats {
  float lse, target, sum_z, pad;
};

// Per row of the shard's logits (one wave per row): the shard lse from the
// GEMM's slice statistics and the label's logit when vocab_start <= label <
// vocab_start + Vp, read from the bf16 logits.
__global__ __launch_bounds__(64 * kRowWaves) void flce_shard_rows(const float2* __restrict__ stats,
                                                       int64_t nparts,
                                                       const __bf16* __restrict__ logits,
                                                       int64_t ldl,
                                                       const int64_t* __restrict__ labels,
                                                       int64_t M, int64_t Vp,
                                                       int64_t vocab_start,
                                                       ShardStats* __restrict__ out) {
  const int64_t r = ts_plan::wave_row(blockIdx.x, threadIdx.x >> 6, kRowWaves);
  const int lane = threadIdx.x & 63;
  if (r >= M) return;  // wave-uniform
  const float2* sr = stats + r * nparts;
  float m = -INFINITY;
  for (int64_t p = lane; p < nparts; p += 64) m = fmaxf(m, sr[p].x);
  m = wave_max(m);
  float s = 0.f;
  for (int64_t p = lane; p < nparts; p += 64) {
    const float2 st = sr[p];
    s += st.y == 0.f ? 0.f : st.y * fast_exp2((st.x - m) * kLog2e);
  }
  s = wave_sum(s);
  if (lane != 0) return;
  const int64_t tl = ts_plan::shard_col(labels[r], vocab_start, Vp);
  const float zt = tl >= 0 ? Elt<__bf16>::load1(logits + r * ldl + tl) : 0.f;
  out[r] = ShardStats{m + logf(s), zt, 0.f, 0.f};
}

// Merges the P ranks' partials (rank-major [P][N]) into lse and the per-row
// loss: lse - sum of the target logits, 0 on rows whose label is ignore_index.
// One thread per row, eight ranks' partials loaded before they are folded.
__global__ __launch_bounds__(64) void flce_vocab_merge(const ShardStats* __restrict__ all,
                                                       int64_t P, int64_t N,
                                                       const int64_t* __restrict__ labels,
                                                       int64_t ignore_index,
                                                       float* __restrict__ lse_out,
                                                       float* __restrict__ rows_out) {
  const int64_t r = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (r >= N) return;
  float gm = -INFINITY, gs = 0.f, zt = 0.f;
  constexpr int kU = 8;
  for (int64_t p0 = 0; p0 < P; p0 += kU) {
    ShardStats st[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u)
      st[u] = p0 + u < P ? all[(p0 + u) * N + r] : ShardStats{-INFINITY, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (st[u].lse > gm) {  // false for -inf partials and NaN
        gs = gs == 0.f ? 0.f : gs * fast_exp2((gm - st[u].lse) * kLog2e);
        gm = st[u].lse;
      }
      gs += st[u].lse == -INFINITY ? 0.f : fast_exp2((st[u].lse - gm) * kLog2e);
      zt += st[u].target;
    }
  }
  const float lse = gm == -INFINITY ? -INFINITY : gm + logf(gs);
  lse_out[r] = lse;
  rows_out[r] = labels[r] == ignore_index ? 0.f : lse - zt;
}

// loss = scale * sum(loss_rows) over all N rows (one workgroup, fixed order);
// scale = 1/max(n_valid, 1) for the mean, 1 for the sum. Also stores the scale.
__global__ __launch_bounds__(256) void flce_loss(const float* __restrict__ loss_rows, int64_t N,
                                                 const int* __restrict__ n_valid, int mean,
                                                 float* __restrict__ loss,
                                                 float* __restrict__ scale_out) {
  __shared__ float red[4];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < N; i += 256) s += loss_rows[i];
  s = block_sum<4>(s, red);
  if (threadIdx.x == 0) {
    const float scale = mean ? 1.f / (float)(*n_valid > 0 ? *n_valid : 1) : 1.f;
    *loss = s * scale;
    *scale_out = scale;
  }
}

// dlogits of a chunk in place: D = (exp(z - lse) - onehot) * scale in bf16
// over the logits [M, V] with rows of ldl >= round_up(V, 8) elements (0 on
// ignored rows, which are not read, and in the columns from V up to the end
// of the last 16-byte vector, which the gradient GEMMs read). One-shot grid: a
// thread owns kDlKv 16-byte vectors of a row, spaced one workgroup apart;
// blockIdx.x = row * chunks + chunk.
constexpr int kDlKv = 1;
__global__ __launch_bounds__(256) void flce_dlogits(__bf16* __restrict__ L, int64_t ldl,
                                                    const float* __restrict__ lse,
                                                    const int64_t* __restrict__ labels,
                                                    int64_t V, int64_t chunks,
                                                    int64_t ignore_index,
                                                    const float* __restrict__ scale_p,
                                                    int64_t label_offset) {
  const int64_t r = (int64_t)blockIdx.x / chunks;
  const int64_t c = (int64_t)blockIdx.x % chunks;
  int64_t vk[kDlKv];  // this thread's vectors of row r (ts_plan::chunk_vec)
#pragma unroll
  for (int u = 0; u < kDlKv; ++u) vk[u] = ts_plan::chunk_vec(c, u, threadIdx.x, 256, kDlKv);
  const int64_t nvec = (V + 7) / 8;
  const int64_t raw = labels[r];
  const int64_t lab = raw - label_offset;  // the label's column in these logits
  __bf16* row = L + r * ldl;
  if (raw == ignore_index) {
    const u32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kDlKv; ++u) {
      const int64_t v = vk[u];
      if (v < nvec) st16_stream(row + v * 8, zero);
    }
    return;
  }
  u32x4 q[kDlKv];
#pragma unroll
  for (int u = 0; u < kDlKv; ++u) {
    const int64_t v = vk[u];
    if (v < nvec) q[u] = ld16_stream(row + v * 8);
  }
  const float scale = *scale_p;
  const float l2 = lse[r] * kLog2e;
#pragma unroll
  for (int u = 0; u < kDlKv; ++u) {
    const int64_t v = vk[u];
    if (v < nvec) {
      float z[8], g[8];
      Elt<__bf16>::unpack(q[u], z);
      const int64_t lim = V - v * 8;  // columns of this vector inside the row
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pr = fast_exp2(__builtin_fmaf(z[e], kLog2e, -l2));
        g[e] = e < lim ? scale * (v * 8 + e == lab ? pr - 1.f : pr) : 0.f;
      }
      st16_stream(row + v * 8, Elt<__bf16>::pack(g));
    }
  }
}

// dz of the logits a forward kept ([N, V] with rows of ldl >= round_up(V, 8)
// elements), in place over them: for row r and column j < V (0 from V on),
//   dz = bf16(dscale[r] * (exp(t - lse[r]) - [j == labels[r]]) * dt/dz),  t = xf(z),
// the arithmetic of the dlogits epilogue (kEpiDlogits) on the same bf16 z, so
// the result is bit-identical to what the recomputing backward forms (ignored
// rows have dscale 0 and give zeros of the same signs). Grid as flce_dlogits:
// blockIdx.x = row * chunks + chunk, one 16-byte vector a thread.
__global__ __launch_bounds__(256) void flce_dlogits_kept(__bf16* __restrict__ L, int64_t ldl,
                                                         const float* __restrict__ lse,
                                                         const int64_t* __restrict__ labels,
                                                         int64_t V, int64_t chunks,
                                                         const float* __restrict__ dscale,
                                                         LogitXform xf) {
  const int64_t r = (int64_t)blockIdx.x / chunks;
  const int64_t v = ts_plan::chunk_vec((int64_t)blockIdx.x % chunks, 0, threadIdx.x, 256, 1);
  if (v >= (V + 7) / 8) return;
  __bf16* p = L + r * ldl + v * 8;
  const float ds = dscale[r];
  const u32x4 q = ld16_stream(p);
  const float l2 = lse[r] * kLog2e;
  const int64_t d = labels[r] - v * 8;  // the label's position in this vector, if in [0, 8)
  float f[8], g[8];
  Elt<__bf16>::unpack(q, f);
  if (!xf.on()) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pr = fast_exp2(__builtin_fmaf(f[e], kLog2e, -l2));
      g[e] = ds * (e == d ? pr - 1.f : pr);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float dt;
      const float t = xf.apply_d(f[e], dt);
      const float pr = fast_exp2(__builtin_fmaf(t, kLog2e, -l2));
      g[e] = ds * (e == d ? pr - 1.f : pr) * dt;
    }
  }
  const int64_t lim = V - v * 8;  // the columns from V on are zero for the GEMMs
  if (lim < 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = e < lim ? g[e] : 0.f;
  }
  st16_stream(p, Elt<__bf16>::pack(g));
}

__global__ __launch_bounds__(256) void fill_zero_u32(uint32_t* __restrict__ p, int64_t n,
                                                     float* __restrict__ loss) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
  if (i == 0 && loss != nullptr) *loss = 0.f;
}

// x[i] *= *scale unless *scale == 1, over n elements of type T: nvec 16-byte
// vectors from x (x 16-byte aligned when nvec > 0), then the n - nvec * VE
// elements after them one at a time. The grid is capped at kScaleGrid
// workgroups (one per CU), each thread four vectors per sweep. Measured on
// MI355X over a [16384, 128256] bf16 gradient: factor 2 at 5.6 TB/s with 256 or
// 512 workgroups against 5.0 TB/s with 2048; the no-op (factor exactly 1) costs
// the same 5.9-6.0 us between HIP events for any grid from 64 to 2048
// workgroups, what an empty kernel costs there.
constexpr int kScaleGrid = 256;
constexpr int kScaleUnroll = 4;
// The factor is *num, or *num / *den when den is given. With hint_out, the
// first thread also stores *num there when it is finite and non-zero (else
// 1): the prediction a later forward pass uses for the upstream gradient.
template <typename T>
__global__ __launch_bounds__(256) void scale_inplace(T* __restrict__ x, int64_t nvec, int64_t n,
                                                     const float* __restrict__ num,
                                                     const float* __restrict__ den,
                                                     float* __restrict__ hint_out) {
  constexpr int VE = Elt<T>::kVec;
  const float g = *num;
  if (hint_out != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
    *hint_out = (__builtin_isfinite(g) && g != 0.f) ? g : 1.f;
  const float s = den != nullptr ? g / *den : g;
  if (s == 1.f) return;
  // sweep n takes chunk blockIdx.x + n * gridDim.x: v0 + u * 256 is
  // ts_plan::chunk_vec(chunk, u, threadIdx.x, 256, kScaleUnroll)
  const int64_t stride = (int64_t)gridDim.x * 256 * kScaleUnroll;
  for (int64_t v0 = ts_plan::chunk_vec(blockIdx.x, 0, threadIdx.x, 256, kScaleUnroll); v0 < nvec;
       v0 += stride) {
    u32x4 q[kScaleUnroll];
#pragma unroll
    for (int u = 0; u < kScaleUnroll; ++u) {
      const int64_t v = v0 + u * 256;
      if (v < nvec) q[u] = ld16_stream(x + v * VE);
    }
#pragma unroll
    for (int u = 0; u < kScaleUnroll; ++u) {
      const int64_t v = v0 + u * 256;
      if (v < nvec) {
        float f[VE];
        Elt<T>::unpack(q[u], f);
#pragma unroll
        for (int e = 0; e < VE; ++e) f[e] *= s;
        st16_stream(x + v * VE, Elt<T>::pack(f));
      }
    }
  }
  // elements after the last whole vector (all of them when x is not 16-byte aligned)
  for (int64_t i = nvec * VE + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    Elt<T>::store1(x + i, Elt<T>::load1(x + i) * s);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Row stride of the library's [rows, V] bf16 logits: whole 16-byte vectors, so any
// V (GPT-2's 50257 included) keeps every row 16-byte aligned.
inline int64_t logits_ld(int64_t V) { return round_up(V, 8); }

struct Layout {
  int64_t chunk, nchunks, nparts;
  size_t off_logits, off_stats, off_lse, off_rows, off_misc, off_acc, total;
};

Layout layout(int64_t N, int64_t H, int64_t V, int64_t chunk, bool grads, bool acc_bf16) {
  Layout l{};
  l.chunk = chunk <= 0 || chunk >= N ? round_up(N, 8) : round_up(chunk, 256);
  if (l.chunk > round_up(N, 8)) l.chunk = round_up(N, 8);
  l.nchunks = (N + l.chunk - 1) / l.chunk;
  l.nparts = 2 * ((V + BN - 1) / BN);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.off_logits = take((size_t)l.chunk * logits_ld(V) * 2);
  l.off_stats = take((size_t)l.nparts * l.chunk * sizeof(float2));
  l.off_lse = take((size_t)N * 4);
  l.off_rows = take((size_t)N * 4);
  l.off_misc = take(64);
  l.off_acc = grads && !acc_bf16 && l.nchunks > 1 ? take((size_t)V * H * 4) : 0;
  l.total = off;
  return l;
}

// The GEMMs run with 8 waves (two per SIMD): measured on MI355X at C5 against
// the 4-wave layout, logits 7.59 vs 7.88 ms, grad_hidden 6.96 vs 7.12 ms,
// grad_weight 6.93 vs 7.19 ms, bit-identical results. The matrix cores are busier
// per clock (69-76% against 58-67%); the box's clock under this load drops to
// 1.55-1.6 GHz from 1.75-1.85, which takes back part of the gain.
template <int kMode, int kMA = ts_gemm::kKMajor, int kMB = ts_gemm::kKMajor>
ts_status launch_gemm(const GemmArgs& a, hipStream_t st, const char* name) {
  constexpr int kW = 8;
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  if (tiles <= 0) return TS_OK;
  if (tiles > 0x7fffffffLL) return ts_host::fail(TS_ERR_SHAPE, "%s: too many tiles", name);
  hipLaunchKernelGGL((flce_gemm<kMode, kMA, kMB, kW>), dim3((unsigned)tiles),
                     dim3(ts_gemm::Cfg<kW>::kThreads), 0, st, a);
  return ts_host::check_launch(name);
}

template <int kMode1, int kMA1, int kMB1, int kMode2, int kMA2, int kMB2>
ts_status launch_gemm_pair(const GemmArgs& a1, const GemmArgs& a2, hipStream_t st,
                           const char* name) {
  constexpr int kW = 8;
  const int64_t t1 = ((a1.M + BM - 1) / BM) * ((a1.N + BN - 1) / BN);
  const int64_t t2 = ((a2.M + BM - 1) / BM) * ((a2.N + BN - 1) / BN);
  if (t1 + t2 <= 0) return TS_OK;
  if (t1 + t2 > 0x7fffffffLL) return ts_host::fail(TS_ERR_SHAPE, "%s: too many tiles", name);
  hipLaunchKernelGGL((flce_gemm_pair<kMode1, kMA1, kMB1, kMode2, kMA2, kMB2, kW>),
                     dim3((unsigned)(t1 + t2)), dim3(ts_gemm::Cfg<kW>::kThreads), 0, st, a1, a2,
                     t1);
  return ts_host::check_launch(name);
}

}  // namespace

#define TS_TRY(x)                  \
  do {                             \
    const ts_status s_ = (x);      \
    if (s_ != TS_OK) return s_;    \
  } while (0)

extern "C" size_t ts_flce_workspace_size(int64_t N, int64_t H, int64_t V, int64_t chunk,
                                         int32_t flags) {
  if (N <= 0 || H <= 0 || V <= 0) return 0;
  return layout(N, H, V, chunk, (flags & TS_FLCE_GRADS) != 0, (flags & TS_FLCE_ACCUM_BF16) != 0)
      .total;
}

extern "C" ts_status ts_flce_fwd_bwd(const void* hidden, int64_t ldh, const void* weight,
                                     int64_t ldw, const int64_t* labels, int64_t N, int64_t H,
                                     int64_t V, int64_t ignore_index, int32_t reduction,
                                     float* loss, float* loss_rows, float* lse,
                                     void* grad_hidden, void* grad_weight, int64_t chunk,
                                     int32_t flags, void* workspace, size_t workspace_bytes,
                                     ts_stream_t stream) {
  using ts_host::fail;
  if (N < 0 || H <= 0 || V <= 0)
    return fail(TS_ERR_SHAPE, "flce: bad shape N=%lld H=%lld V=%lld", (long long)N, (long long)H,
                (long long)V);
  // TS_FLCE_GRADS sizes the workspace; here the gradient pointers decide
  if ((flags & ~(TS_FLCE_ACCUM_BF16 | TS_FLCE_GRADS)) != 0)
    return fail(TS_ERR_INVALID_ARGUMENT, "flce: unknown flags 0x%x", (unsigned)flags);
  const bool acc_bf16 = (flags & TS_FLCE_ACCUM_BF16) != 0;
  if (N % 8 != 0 || H % 8 != 0)
    return fail(TS_ERR_SHAPE, "flce: N and H must be multiples of 8 (N=%lld H=%lld)",
                (long long)N, (long long)H);
  if (ldh < H || ldw < H || ldh % 8 != 0 || ldw % 8 != 0)
    return fail(TS_ERR_SHAPE, "flce: row strides must be >= H and multiples of 8");
  // Buffer offsets are 32-bit and must stay below 2^31: within a 256-row K-major tile
  // (row * ld * 2 bytes, ld = ldh, ldw or V) and within a 32-row k-block of an MN-major
  // operand (k * ld * 2, ld = ldh, ldw or V).
  if (V > ((int64_t)1 << 22) || H > ((int64_t)1 << 20) || N > ((int64_t)1 << 22))
    return fail(TS_ERR_SHAPE, "flce: shape beyond the kernel's index range");
  if (ldh > ((int64_t)1 << 22) || ldw > ((int64_t)1 << 22))
    return fail(TS_ERR_SHAPE, "flce: row strides beyond the kernel's index range (%lld, %lld)",
                (long long)ldh, (long long)ldw);
  if (reduction != 0 && reduction != 1)
    return fail(TS_ERR_INVALID_ARGUMENT, "flce: reduction must be 0 (mean) or 1 (sum)");
  if (loss == nullptr) return fail(TS_ERR_INVALID_ARGUMENT, "flce: loss is NULL");
  if (N > 0 && (hidden == nullptr || weight == nullptr || labels == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce: hidden, weight or labels is NULL");
  if (!ts_host::aligned16(hidden) || !ts_host::aligned16(weight) ||
      (grad_hidden != nullptr && !ts_host::aligned16(grad_hidden)) ||
      (grad_weight != nullptr && !ts_host::aligned16(grad_weight)))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce: tensors must be 16-byte aligned");
  const bool grads = grad_hidden != nullptr || grad_weight != nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (N == 0) {
    // no rows: loss 0, grad_weight 0 (grad_hidden is empty); no workspace needed
    const int64_t words = grad_weight != nullptr ? V * H / 2 : 1;
    hipLaunchKernelGGL(fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       grad_weight != nullptr ? static_cast<uint32_t*>(grad_weight) : nullptr,
                       grad_weight != nullptr ? words : 0, loss);
    return ts_host::check_launch("fill_zero_u32");
  }
  const Layout lay = layout(N, H, V, chunk, grads, acc_bf16);
  if (workspace == nullptr || workspace_bytes < lay.total || !ts_host::aligned16(workspace))
    return fail(TS_ERR_WORKSPACE, "flce: workspace needs %zu bytes (16-byte aligned), got %zu",
                lay.total, workspace == nullptr ? (size_t)0 : workspace_bytes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  __bf16* Lc = reinterpret_cast<__bf16*>(ws + lay.off_logits);
  float2* stats = reinterpret_cast<float2*>(ws + lay.off_stats);
  float* lse_ws = lse != nullptr ? lse : reinterpret_cast<float*>(ws + lay.off_lse);
  float* rows_ws = loss_rows != nullptr ? loss_rows : reinterpret_cast<float*>(ws + lay.off_rows);
  int* n_valid = reinterpret_cast<int*>(ws + lay.off_misc);
  float* scale = reinterpret_cast<float*>(ws + lay.off_misc + 16);
  float* acc32 = reinterpret_cast<float*>(ws + lay.off_acc);
  const __bf16* Hd = static_cast<const __bf16*>(hidden);
  const __bf16* Wd = static_cast<const __bf16*>(weight);
  const int64_t ldl = logits_ld(V);

  hipLaunchKernelGGL(flce_count, dim3(1), dim3(256), 0, st, labels, N, ignore_index, n_valid);
  TS_TRY(ts_host::check_launch("flce_count"));
  // Pass 1 over chunks: logits, statistics, per-row loss (and lse).
  // With gradients the dlogits of a chunk are consumed right away, so the
  // loss scale (which needs every row's label) is computed up front.
  if (grads) {
    hipLaunchKernelGGL(flce_loss, dim3(1), dim3(256), 0, st, rows_ws, (int64_t)0, n_valid,
                       reduction == 0 ? 1 : 0, loss, scale);
    TS_TRY(ts_host::check_launch("flce_loss"));
  }
  for (int64_t c = 0; c < lay.nchunks; ++c) {
    const int64_t r0 = c * lay.chunk;
    const int64_t Mc = N - r0 < lay.chunk ? N - r0 : lay.chunk;
    GemmArgs g{};
    g.A = Hd + r0 * ldh;
    g.lda = ldh;
    g.B = Wd;
    g.ldb = ldw;
    g.M = Mc;
    g.N = V;
    g.K = H;
    g.C = Lc;
    g.ldc = ldl;
    g.stats = stats;
    TS_TRY(launch_gemm<kEpiLogits>(g, st, "flce_gemm_logits"));
    hipLaunchKernelGGL(flce_rows, dim3((unsigned)ts_plan::wave_row_blocks(Mc, kRowWaves)), dim3(64 * kRowWaves), 0, st, stats,
                       lay.nparts, Lc, ldl, labels + r0, Mc, V, ignore_index, lse_ws + r0,
                       rows_ws + r0);
    TS_TRY(ts_host::check_launch("flce_rows"));
    if (!grads) continue;
    const int64_t dchunks = ts_plan::chunks_for((V + 7) / 8, 256, kDlKv);
    hipLaunchKernelGGL(flce_dlogits, dim3((unsigned)(Mc * dchunks)), dim3(256), 0, st, Lc, ldl,
                       lse_ws + r0, labels + r0, V, dchunks, ignore_index, scale, (int64_t)0);
    TS_TRY(ts_host::check_launch("flce_dlogits"));
    using ts_gemm::kKMajor;
    using ts_gemm::kMNMajor;
    GemmArgs dh{};
    dh.A = Lc;  // dlogits [Mc, V], K-major (zero from V to the end of the row's last vector)
    dh.lda = ldl;
    dh.B = Wd;  // weight [V, H] as the [H, V] operand: MN-major, k = v
    dh.ldb = ldw;
    dh.M = Mc;
    dh.N = H;
    dh.K = V;
    dh.C = static_cast<__bf16*>(grad_hidden) + r0 * H;
    dh.ldc = H;
    GemmArgs dw{};
    dw.A = Lc;             // dlogits [Mc, V] as the [V, Mc] operand: MN-major, k = token
    dw.lda = ldl;
    dw.B = Hd + r0 * ldh;  // hidden rows r0 .. r0 + Mc as the [H, Mc] operand: MN-major
    dw.ldb = ldh;
    dw.M = V;
    dw.N = H;
    dw.K = Mc;
    dw.C = static_cast<__bf16*>(grad_weight);
    dw.ldc = H;
    dw.C32 = acc32;
    dw.ldc32 = H;
    // grad_weight sums over the chunks: fp32 in the workspace, rounded once at the
    // end, or (TS_FLCE_ACCUM_BF16) in the bf16 output, rounded after every chunk
    const int wmode = lay.nchunks == 1 ? kEpiBf16
                      : acc_bf16       ? (c == 0 ? kEpiBf16 : kEpiAddBf16)
                      : c == 0         ? kEpiF32
                      : c + 1 < lay.nchunks ? kEpiAccF32
                                            : kEpiAccBf16;
    if (grad_hidden != nullptr && grad_weight != nullptr) {
      // both gradient GEMMs in one grid (grad_hidden's few long tiles first)
#define TS_PAIR(WM)                                                                         \
  TS_TRY((launch_gemm_pair<kEpiBf16, kKMajor, kMNMajor, WM, kMNMajor, kMNMajor>(dh, dw, st,   \
                                                                                "flce_gemm_grads")))
      if (wmode == kEpiBf16) TS_PAIR(kEpiBf16);
      else if (wmode == kEpiAddBf16) TS_PAIR(kEpiAddBf16);
      else if (wmode == kEpiF32) TS_PAIR(kEpiF32);
      else if (wmode == kEpiAccF32) TS_PAIR(kEpiAccF32);
      else TS_PAIR(kEpiAccBf16);
#undef TS_PAIR
    } else if (grad_hidden != nullptr) {
      TS_TRY((launch_gemm<kEpiBf16, kKMajor, kMNMajor>(dh, st, "flce_gemm_dhidden")));
    } else if (grad_weight != nullptr) {
      if (wmode == kEpiBf16) {
        TS_TRY((launch_gemm<kEpiBf16, kMNMajor, kMNMajor>(dw, st, "flce_gemm_dweight")));
      } else if (wmode == kEpiAddBf16) {
        TS_TRY((launch_gemm<kEpiAddBf16, kMNMajor, kMNMajor>(dw, st, "flce_gemm_dweight")));
      } else if (wmode == kEpiF32) {
        TS_TRY((launch_gemm<kEpiF32, kMNMajor, kMNMajor>(dw, st, "flce_gemm_dweight")));
      } else if (wmode == kEpiAccF32) {
        TS_TRY((launch_gemm<kEpiAccF32, kMNMajor, kMNMajor>(dw, st, "flce_gemm_dweight")));
      } else {
        TS_TRY((launch_gemm<kEpiAccBf16, kMNMajor, kMNMajor>(dw, st, "flce_gemm_dweight")));
      }
    }
  }
  hipLaunchKernelGGL(flce_loss, dim3(1), dim3(256), 0, st, rows_ws, N, n_valid,
                     reduction == 0 ? 1 : 0, loss, scale);
  return ts_host::check_launch("flce_loss");
}

// ---------------------------------------------------------------------------
// Two-pass fused linear CE: a forward that keeps only per-row statistics, and a
// backward that recomputes the logits one vocabulary chunk at a time.
// ---------------------------------------------------------------------------
namespace {

struct FwdLayout {
  int64_t nparts;
  size_t off_stats, off_zlab, off_rows, off_lse, off_misc, total;
};

FwdLayout fwd_layout(int64_t N, int64_t V) {
  FwdLayout l{};
  l.nparts = 2 * ((V + BN - 1) / BN);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.off_stats = take((size_t)l.nparts * (size_t)N * sizeof(float2));
  l.off_zlab = take((size_t)N * 4);
  l.off_rows = take((size_t)N * 4);
  l.off_lse = take((size_t)N * 4);
  l.off_misc = take(64);
  l.total = off;
  return l;
}

// Vocabulary chunk of the backward: the given width rounded up to whole
// 256-column tiles, or the default, about an eighth of V (at least 4096
// columns), so the dlogits buffer holds N x chunk bf16 values.
int64_t bwd_chunk_cols(int64_t V, int64_t chunk_cols) {
  int64_t c = chunk_cols > 0 ? chunk_cols : ((V + 7) / 8 + BN - 1) / BN * BN;
  if (chunk_cols <= 0 && c < 4096) c = 4096;
  c = (c + BN - 1) / BN * BN;
  const int64_t v8 = (V + 7) / 8 * 8;
  return c > v8 ? v8 : c;
}

struct BwdLayout {
  int64_t chunk, nchunks;
  size_t off_d, off_acc, off_dscale, off_misc, total;
};

BwdLayout bwd_layout(int64_t N, int64_t H, int64_t V, int64_t chunk_cols) {
  BwdLayout l{};
  l.chunk = bwd_chunk_cols(V, chunk_cols);
  l.nchunks = (V + l.chunk - 1) / l.chunk;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.off_d = take((size_t)N * (size_t)l.chunk * 2);
  l.off_acc = l.nchunks > 1 ? take((size_t)N * (size_t)H * 4) : 0;
  l.off_dscale = take((size_t)N * 4);
  l.off_misc = take(64);
  l.total = off;
  return l;
}

ts_status check_two_pass(const char* who, const void* hidden, int64_t ldh, const void* weight,
                         int64_t ldw, const int64_t* labels, int64_t N, int64_t H, int64_t V,
                         int32_t reduction, float softcap, float scale, float temperature,
                         LogitXform* xf) {
  using ts_host::fail;
  if (N < 0 || H <= 0 || V <= 0)
    return fail(TS_ERR_SHAPE, "%s: bad shape N=%lld H=%lld V=%lld", who, (long long)N,
                (long long)H, (long long)V);
  if (H % 8 != 0)
    return fail(TS_ERR_SHAPE, "%s: H must be a multiple of 8 (H=%lld)", who, (long long)H);
  if (ldh < H || ldw < H || ldh % 8 != 0 || ldw % 8 != 0)
    return fail(TS_ERR_SHAPE, "%s: row strides must be >= H and multiples of 8", who);
  // 32-bit buffer offsets within a 256-row K-major tile and a 32-row MN-major k-block
  if (V > ((int64_t)1 << 22) || H > ((int64_t)1 << 20) || N > ((int64_t)1 << 24) ||
      ldh > ((int64_t)1 << 22) || ldw > ((int64_t)1 << 22))
    return fail(TS_ERR_SHAPE, "%s: shape beyond the kernel's index range", who);
  if (reduction < 0 || reduction > 2)
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: reduction must be 0 (mean), 1 (sum) or 2 (none)",
                who);
  if (N > 0 && (hidden == nullptr || weight == nullptr || labels == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: hidden, weight or labels is NULL", who);
  if (!ts_host::aligned16(hidden) || !ts_host::aligned16(weight))
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: hidden and weight must be 16-byte aligned", who);
  if (!(softcap >= 0.f) || !(scale >= 0.f) || !(temperature > 0.f) ||
      !__builtin_isfinite(softcap) || !__builtin_isfinite(scale) ||
      !__builtin_isfinite(temperature))
    return fail(TS_ERR_INVALID_ARGUMENT,
                "%s: softcap and scale must be finite and >= 0 (0 = off), temperature > 0", who);
  xf->softcap = softcap;
  xf->inv_softcap = softcap > 0.f ? 1.f / softcap : 0.f;
  xf->mul = (scale > 0.f ? scale : 1.f) / temperature;
  return TS_OK;
}

}  // namespace

extern "C" size_t ts_flce_forward_workspace_size(int64_t N, int64_t V) {
  if (N <= 0 || V <= 0) return 0;
  return fwd_layout(N, V).total;
}

namespace {

// ts_flce_forward, and ts_flce_forward_keep when `logits` is not NULL.
ts_status flce_forward_impl(const char* who, const void* hidden, int64_t ldh, const void* weight,
                            int64_t ldw, const int64_t* labels, int64_t N, int64_t H, int64_t V,
                            int64_t ignore_index, int32_t reduction, float softcap, float scale,
                            float temperature, float* loss, float* loss_rows, float* lse,
                            void* logits, void* workspace, size_t workspace_bytes,
                            hipStream_t st) {
  using ts_host::fail;
  LogitXform xf{};
  TS_TRY(check_two_pass(who, hidden, ldh, weight, ldw, labels, N, H, V, reduction, softcap, scale,
                        temperature, &xf));
  if (reduction != 2 && loss == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: loss is NULL", who);
  if (N == 0) {
    if (loss == nullptr) return TS_OK;
    hipLaunchKernelGGL(fill_zero_u32, dim3(1), dim3(256), 0, st, nullptr, (int64_t)0, loss);
    return ts_host::check_launch("fill_zero_u32");
  }
  const FwdLayout lay = fwd_layout(N, V);
  if (workspace == nullptr || workspace_bytes < lay.total || !ts_host::aligned16(workspace))
    return fail(TS_ERR_WORKSPACE, "%s: workspace needs %zu bytes (16-byte aligned), got %zu", who,
                lay.total, workspace == nullptr ? (size_t)0 : workspace_bytes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float2* stats = reinterpret_cast<float2*>(ws + lay.off_stats);
  float* zlab = reinterpret_cast<float*>(ws + lay.off_zlab);
  float* rows_ws = loss_rows != nullptr ? loss_rows : reinterpret_cast<float*>(ws + lay.off_rows);
  float* lse_ws = lse != nullptr ? lse : reinterpret_cast<float*>(ws + lay.off_lse);
  int* n_valid = reinterpret_cast<int*>(ws + lay.off_misc);
  float* sc = reinterpret_cast<float*>(ws + lay.off_misc + 16);
  GemmArgs g{};
  g.A = static_cast<const __bf16*>(hidden);
  g.lda = ldh;
  g.B = static_cast<const __bf16*>(weight);
  g.ldb = ldw;
  g.M = N;
  g.N = V;
  g.K = H;
  g.stats = stats;
  g.labels = labels;
  g.label_offset = 0;
  g.zlab = zlab;
  g.xf = xf;
  g.C = static_cast<__bf16*>(logits);  // NULL: the statistics only
  g.ldc = logits_ld(V);
  TS_TRY(launch_gemm<kEpiStats>(g, st, "flce_gemm_stats"));
  hipLaunchKernelGGL(flce_rows_t, dim3((unsigned)ts_plan::wave_row_blocks(N, kRowWaves)), dim3(64 * kRowWaves), 0, st, stats,
                     lay.nparts, zlab, labels, N, V, ignore_index, lse_ws, rows_ws);
  TS_TRY(ts_host::check_launch("flce_rows_t"));
  if (loss == nullptr) return TS_OK;
  hipLaunchKernelGGL(flce_count, dim3(1), dim3(256), 0, st, labels, N, ignore_index, n_valid);
  TS_TRY(ts_host::check_launch("flce_count"));
  hipLaunchKernelGGL(flce_loss, dim3(1), dim3(256), 0, st, rows_ws, N, n_valid,
                     reduction == 0 ? 1 : 0, loss, sc);
  return ts_host::check_launch("flce_loss");
}

}  // namespace

extern "C" ts_status ts_flce_forward(const void* hidden, int64_t ldh, const void* weight,
                                     int64_t ldw, const int64_t* labels, int64_t N, int64_t H,
                                     int64_t V, int64_t ignore_index, int32_t reduction,
                                     float softcap, float scale, float temperature, float* loss,
                                     float* loss_rows, float* lse, void* workspace,
                                     size_t workspace_bytes, ts_stream_t stream) {
  return flce_forward_impl("flce_forward", hidden, ldh, weight, ldw, labels, N, H, V,
                           ignore_index, reduction, softcap, scale, temperature, loss, loss_rows,
                           lse, nullptr, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream));
}

extern "C" ts_status ts_flce_forward_keep(const void* hidden, int64_t ldh, const void* weight,
                                          int64_t ldw, const int64_t* labels, int64_t N,
                                          int64_t H, int64_t V, int64_t ignore_index,
                                          int32_t reduction, float softcap, float scale,
                                          float temperature, float* loss, float* loss_rows,
                                          float* lse, void* logits, void* workspace,
                                          size_t workspace_bytes, ts_stream_t stream) {
  if (N > 0 && (logits == nullptr || !ts_host::aligned16(logits)))
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "flce_forward_keep: logits NULL or unaligned");
  return flce_forward_impl("flce_forward_keep", hidden, ldh, weight, ldw, labels, N, H, V,
                           ignore_index, reduction, softcap, scale, temperature, loss, loss_rows,
                           lse, logits, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream));
}

extern "C" size_t ts_flce_backward_workspace_size(int64_t N, int64_t H, int64_t V,
                                                  int64_t chunk_cols) {
  if (N <= 0 || H <= 0 || V <= 0) return 0;
  return bwd_layout(N, H, V, chunk_cols).total;
}

extern "C" ts_status ts_flce_backward(const void* hidden, int64_t ldh, const void* weight,
                                      int64_t ldw, const int64_t* labels, int64_t N, int64_t H,
                                      int64_t V, int64_t ignore_index, int32_t reduction,
                                      float softcap, float scale, float temperature,
                                      const float* lse, const float* dloss, int64_t dloss_stride,
                                      void* grad_hidden, void* grad_weight, int64_t chunk_cols,
                                      void* workspace, size_t workspace_bytes,
                                      ts_stream_t stream) {
  using ts_host::fail;
  LogitXform xf{};
  TS_TRY(check_two_pass("flce_backward", hidden, ldh, weight, ldw, labels, N, H, V, reduction,
                        softcap, scale, temperature, &xf));
  if (dloss_stride < 0)
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_backward: dloss_stride must be >= 0");
  if (N > 0 && (lse == nullptr || dloss == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_backward: lse or dloss is NULL");
  if ((grad_hidden != nullptr && !ts_host::aligned16(grad_hidden)) ||
      (grad_weight != nullptr && !ts_host::aligned16(grad_weight)))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_backward: gradients must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (N == 0) {
    // no rows: grad_weight is 0 (grad_hidden is empty)
    if (grad_weight == nullptr) return TS_OK;
    const int64_t words = V * H / 2;
    hipLaunchKernelGGL(fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       static_cast<uint32_t*>(grad_weight), words, nullptr);
    return ts_host::check_launch("fill_zero_u32");
  }
  if (grad_hidden == nullptr && grad_weight == nullptr) return TS_OK;
  const BwdLayout lay = bwd_layout(N, H, V, chunk_cols);
  if (workspace == nullptr || workspace_bytes < lay.total || !ts_host::aligned16(workspace))
    return fail(TS_ERR_WORKSPACE, "flce_backward: workspace needs %zu bytes (16-byte aligned), "
                "got %zu", lay.total, workspace == nullptr ? (size_t)0 : workspace_bytes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  __bf16* D = reinterpret_cast<__bf16*>(ws + lay.off_d);
  float* acc32 = reinterpret_cast<float*>(ws + lay.off_acc);
  float* dscale = reinterpret_cast<float*>(ws + lay.off_dscale);
  int* n_valid = reinterpret_cast<int*>(ws + lay.off_misc);
  const __bf16* Hd = static_cast<const __bf16*>(hidden);
  const __bf16* Wd = static_cast<const __bf16*>(weight);

  hipLaunchKernelGGL(flce_count, dim3(1), dim3(256), 0, st, labels, N, ignore_index, n_valid);
  TS_TRY(ts_host::check_launch("flce_count"));
  hipLaunchKernelGGL(flce_dscale, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, labels, N,
                     ignore_index, dloss, dloss_stride, n_valid, reduction == 0 ? 1 : 0, dscale);
  TS_TRY(ts_host::check_launch("flce_dscale"));
  using ts_gemm::kKMajor;
  using ts_gemm::kMNMajor;
  for (int64_t c = 0; c < lay.nchunks; ++c) {
    const int64_t v0 = c * lay.chunk;
    const int64_t Vc = V - v0 < lay.chunk ? V - v0 : lay.chunk;
    // dlogits of the chunk: logits recomputed by the same GEMM as the forward's
    GemmArgs g{};
    g.A = Hd;
    g.lda = ldh;
    g.B = Wd + v0 * ldw;
    g.ldb = ldw;
    g.M = N;
    g.N = Vc;
    g.K = H;
    g.C = D;
    g.ldc = lay.chunk;
    g.labels = labels;
    g.label_offset = v0;
    g.lse = lse;
    g.dscale = dscale;
    g.xf = xf;
    TS_TRY(launch_gemm<kEpiDlogits>(g, st, "flce_gemm_dlogits"));
    if (grad_hidden != nullptr) {
      // grad_hidden (+)= D [N, Vc] @ W[v0 : v0 + Vc] (the chunk read as the MN-major [H, Vc]
      // operand); carried in fp32 across chunks and rounded once
      GemmArgs d{};
      d.A = D;
      d.lda = lay.chunk;
      d.B = Wd + v0 * ldw;
      d.ldb = ldw;
      d.M = N;
      d.N = H;
      d.K = Vc;
      d.C = static_cast<__bf16*>(grad_hidden);
      d.ldc = H;
      d.C32 = acc32;
      d.ldc32 = H;
      if (lay.nchunks == 1) {
        TS_TRY((launch_gemm<kEpiBf16, kKMajor, kMNMajor>(d, st, "flce_gemm_dhidden")));
      } else if (c == 0) {
        TS_TRY((launch_gemm<kEpiF32, kKMajor, kMNMajor>(d, st, "flce_gemm_dhidden")));
      } else if (c + 1 < lay.nchunks) {
        TS_TRY((launch_gemm<kEpiAccF32, kKMajor, kMNMajor>(d, st, "flce_gemm_dhidden")));
      } else {
        TS_TRY((launch_gemm<kEpiAccBf16, kKMajor, kMNMajor>(d, st, "flce_gemm_dhidden")));
      }
    }
    if (grad_weight != nullptr) {
      // grad_weight[v0 : v0 + Vc] = D^T @ hidden: D as the MN-major [Vc, N] operand, hidden
      // as the MN-major [H, N] operand
      GemmArgs d{};
      d.A = D;
      d.lda = lay.chunk;
      d.B = Hd;
      d.ldb = ldh;
      d.M = Vc;
      d.N = H;
      d.K = N;
      d.C = static_cast<__bf16*>(grad_weight) + v0 * H;
      d.ldc = H;
      TS_TRY((launch_gemm<kEpiBf16, kMNMajor, kMNMajor>(d, st, "flce_gemm_dweight")));
    }
  }
  return TS_OK;
}

// The backward from logits the forward kept (ts_flce_forward_keep): dz in place
// over them, then the two gradient GEMMs in one grid, as the one-call schedule
// runs them. Workspace: the per-row upstream gradients and the valid count.
namespace {

struct KeptLayout {
  size_t off_dscale, off_misc, total;
};

KeptLayout kept_layout(int64_t N) {
  KeptLayout l{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.off_dscale = take((size_t)N * 4);
  l.off_misc = take(64);
  l.total = off;
  return l;
}

}  // namespace

extern "C" size_t ts_flce_backward_kept_workspace_size(int64_t N) {
  if (N <= 0) return 0;
  return kept_layout(N).total;
}

extern "C" ts_status ts_flce_backward_kept(const void* hidden, int64_t ldh, const void* weight,
                                           int64_t ldw, const int64_t* labels, int64_t N,
                                           int64_t H, int64_t V, int64_t ignore_index,
                                           int32_t reduction, float softcap, float scale,
                                           float temperature, const float* lse,
                                           const float* dloss, int64_t dloss_stride,
                                           void* logits, void* grad_hidden, void* grad_weight,
                                           void* workspace, size_t workspace_bytes,
                                           ts_stream_t stream) {
  using ts_host::fail;
  LogitXform xf{};
  TS_TRY(check_two_pass("flce_backward_kept", hidden, ldh, weight, ldw, labels, N, H, V,
                        reduction, softcap, scale, temperature, &xf));
  if (dloss_stride < 0)
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_backward_kept: dloss_stride must be >= 0");
  if (N > 0 && (lse == nullptr || dloss == nullptr || logits == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_backward_kept: lse, dloss or logits is NULL");
  if ((logits != nullptr && !ts_host::aligned16(logits)) ||
      (grad_hidden != nullptr && !ts_host::aligned16(grad_hidden)) ||
      (grad_weight != nullptr && !ts_host::aligned16(grad_weight)))
    return fail(TS_ERR_INVALID_ARGUMENT,
                "flce_backward_kept: logits and gradients must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (N == 0) {
    // no rows: grad_weight is 0 (grad_hidden is empty)
    if (grad_weight == nullptr) return TS_OK;
    const int64_t words = V * H / 2;
    hipLaunchKernelGGL(fill_zero_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       static_cast<uint32_t*>(grad_weight), words, nullptr);
    return ts_host::check_launch("fill_zero_u32");
  }
  if (grad_hidden == nullptr && grad_weight == nullptr) return TS_OK;
  const int64_t ldl = logits_ld(V);
  const int64_t dchunks = ts_plan::chunks_for((V + 7) / 8, 256, 1);
  if (N * dchunks > 0x7fffffffLL)
    return fail(TS_ERR_SHAPE, "flce_backward_kept: too many rows for the dz grid");
  const KeptLayout lay = kept_layout(N);
  if (workspace == nullptr || workspace_bytes < lay.total || !ts_host::aligned16(workspace))
    return fail(TS_ERR_WORKSPACE,
                "flce_backward_kept: workspace needs %zu bytes (16-byte aligned), got %zu",
                lay.total, workspace == nullptr ? (size_t)0 : workspace_bytes);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* dscale = reinterpret_cast<float*>(ws + lay.off_dscale);
  int* n_valid = reinterpret_cast<int*>(ws + lay.off_misc);
  __bf16* L = static_cast<__bf16*>(logits);

  hipLaunchKernelGGL(flce_count, dim3(1), dim3(256), 0, st, labels, N, ignore_index, n_valid);
  TS_TRY(ts_host::check_launch("flce_count"));
  hipLaunchKernelGGL(flce_dscale, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, labels, N,
                     ignore_index, dloss, dloss_stride, n_valid, reduction == 0 ? 1 : 0, dscale);
  TS_TRY(ts_host::check_launch("flce_dscale"));
  hipLaunchKernelGGL(flce_dlogits_kept, dim3((unsigned)(N * dchunks)), dim3(256), 0, st, L, ldl,
                     lse, labels, V, dchunks, dscale, xf);
  TS_TRY(ts_host::check_launch("flce_dlogits_kept"));
  using ts_gemm::kKMajor;
  using ts_gemm::kMNMajor;
  GemmArgs dh{};
  dh.A = L;  // dz [N, V], K-major (rows of ldl, zero from V on)
  dh.lda = ldl;
  dh.B = static_cast<const __bf16*>(weight);  // weight [V, H] as the [H, V] operand: MN-major
  dh.ldb = ldw;
  dh.M = N;
  dh.N = H;
  dh.K = V;
  dh.C = static_cast<__bf16*>(grad_hidden);
  dh.ldc = H;
  GemmArgs dw{};
  dw.A = L;  // dz [N, V] as the [V, N] operand: MN-major
  dw.lda = ldl;
  dw.B = static_cast<const __bf16*>(hidden);  // hidden [N, H] as the [H, N] operand: MN-major
  dw.ldb = ldh;
  dw.M = V;
  dw.N = H;
  dw.K = N;
  dw.C = static_cast<__bf16*>(grad_weight);
  dw.ldc = H;
  if (grad_hidden != nullptr && grad_weight != nullptr)
    return launch_gemm_pair<kEpiBf16, kKMajor, kMNMajor, kEpiBf16, kMNMajor, kMNMajor>(
        dh, dw, st, "flce_gemm_grads_kept");
  if (grad_hidden != nullptr)
    return launch_gemm<kEpiBf16, kKMajor, kMNMajor>(dh, st, "flce_gemm_dhidden_kept");
  return launch_gemm<kEpiBf16, kMNMajor, kMNMajor>(dw, st, "flce_gemm_dweight_kept");
}

// ---------------------------------------------------------------------------
// Vocabulary-parallel fused linear CE: the two phases one rank runs around the
// exchange of the per-row partials. The shard's logits [N, Vp] stay in the
// workspace from phase 1 to phase 2 (no token chunking).
// ---------------------------------------------------------------------------
namespace {

struct VocabLayout {
  int64_t nparts;
  size_t off_logits, off_stats, off_lse, off_rows, off_misc, total;
};

VocabLayout vocab_layout(int64_t N, int64_t Vp) {
  VocabLayout l{};
  l.nparts = 2 * ((Vp + BN - 1) / BN);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  l.off_logits = take((size_t)N * logits_ld(Vp) * 2);  // rows of whole 16-byte vectors
  l.off_stats = take((size_t)l.nparts * N * sizeof(float2));
  l.off_lse = take((size_t)N * 4);
  l.off_rows = take((size_t)N * 4);
  l.off_misc = take(64);
  l.total = off;
  return l;
}

ts_status check_vocab(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                      const int64_t* labels, int64_t N, int64_t H, int64_t Vp,
                      int64_t vocab_start, const void* workspace, size_t workspace_bytes,
                      const char* who) {
  using ts_host::fail;
  if (N <= 0 || H <= 0 || Vp <= 0)
    return fail(TS_ERR_SHAPE, "%s: bad shape N=%lld H=%lld Vp=%lld", who, (long long)N,
                (long long)H, (long long)Vp);
  if (N % 8 != 0 || H % 8 != 0)
    return fail(TS_ERR_SHAPE, "%s: N and H must be multiples of 8", who);
  if (ldh < H || ldw < H || ldh % 8 != 0 || ldw % 8 != 0)
    return fail(TS_ERR_SHAPE, "%s: row strides must be >= H and multiples of 8", who);
  // 32-bit buffer offsets, as for ts_flce_fwd_bwd (the logits' row stride is
  // round_up(Vp, 8))
  if (Vp > ((int64_t)1 << 22) || H > ((int64_t)1 << 20) || N > ((int64_t)1 << 22) ||
      ldh > ((int64_t)1 << 22) || ldw > ((int64_t)1 << 22))
    return fail(TS_ERR_SHAPE, "%s: shape beyond the kernel's index range", who);
  if (vocab_start < 0) return fail(TS_ERR_INVALID_ARGUMENT, "%s: vocab_start < 0", who);
  if (hidden == nullptr || weight == nullptr || labels == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: hidden, weight or labels is NULL", who);
  if (!ts_host::aligned16(hidden) || !ts_host::aligned16(weight))
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: tensors must be 16-byte aligned", who);
  const VocabLayout lay = vocab_layout(N, Vp);
  if (workspace == nullptr || workspace_bytes < lay.total || !ts_host::aligned16(workspace))
    return fail(TS_ERR_WORKSPACE, "%s: workspace needs %zu bytes (16-byte aligned), got %zu", who,
                lay.total, workspace == nullptr ? (size_t)0 : workspace_bytes);
  return TS_OK;
}

}  // namespace

extern "C" size_t ts_flce_vocab_workspace_size(int64_t N, int64_t Vp) {
  if (N <= 0 || Vp <= 0) return 0;
  return vocab_layout(N, Vp).total;
}

extern "C" ts_status ts_flce_vocab_fwd(const void* hidden, int64_t ldh, const void* weight,
                                       int64_t ldw, const int64_t* labels, int64_t N, int64_t H,
                                       int64_t Vp, int64_t vocab_start, float* stats,
                                       void* workspace, size_t workspace_bytes,
                                       ts_stream_t stream) {
  TS_TRY(check_vocab(hidden, ldh, weight, ldw, labels, N, H, Vp, vocab_start, workspace,
                     workspace_bytes, "flce_vocab_fwd"));
  if (stats == nullptr || !ts_host::aligned16(stats))
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "flce_vocab_fwd: stats NULL or unaligned");
  const VocabLayout lay = vocab_layout(N, Vp);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  __bf16* L = reinterpret_cast<__bf16*>(ws + lay.off_logits);
  float2* part = reinterpret_cast<float2*>(ws + lay.off_stats);
  hipStream_t st = static_cast<hipStream_t>(stream);
  GemmArgs g{};
  g.A = static_cast<const __bf16*>(hidden);
  g.lda = ldh;
  g.B = static_cast<const __bf16*>(weight);
  g.ldb = ldw;
  g.M = N;
  g.N = Vp;
  g.K = H;
  g.C = L;
  g.ldc = logits_ld(Vp);
  g.stats = part;
  TS_TRY(launch_gemm<kEpiLogits>(g, st, "flce_vocab_gemm_logits"));
  hipLaunchKernelGGL(flce_shard_rows, dim3((unsigned)ts_plan::wave_row_blocks(N, kRowWaves)),
                     dim3(64 * kRowWaves), 0, st, part, lay.nparts, L, logits_ld(Vp), labels, N,
                     Vp, vocab_start,
                     reinterpret_cast<ShardStats*>(stats));
  return ts_host::check_launch("flce_shard_rows");
}

extern "C" ts_status ts_flce_vocab_bwd(const void* hidden, int64_t ldh, const void* weight,
                                       int64_t ldw, const int64_t* labels, int64_t N, int64_t H,
                                       int64_t Vp, int64_t vocab_start, const float* stats_all,
                                       int64_t P, int64_t ignore_index, int32_t reduction,
                                       float* loss, float* loss_rows, float* lse,
                                       void* grad_hidden_partial, void* grad_weight_shard,
                                       void* workspace, size_t workspace_bytes,
                                       ts_stream_t stream) {
  using ts_host::fail;
  TS_TRY(check_vocab(hidden, ldh, weight, ldw, labels, N, H, Vp, vocab_start, workspace,
                     workspace_bytes, "flce_vocab_bwd"));
  if (P < 1 || P > ((int64_t)1 << 20))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_vocab_bwd: bad rank count %lld", (long long)P);
  if (stats_all == nullptr || !ts_host::aligned16(stats_all))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_vocab_bwd: stats_all NULL or unaligned");
  if (reduction != 0 && reduction != 1)
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_vocab_bwd: reduction must be 0 (mean) or 1 (sum)");
  if (loss == nullptr) return fail(TS_ERR_INVALID_ARGUMENT, "flce_vocab_bwd: loss is NULL");
  if ((grad_hidden_partial != nullptr && !ts_host::aligned16(grad_hidden_partial)) ||
      (grad_weight_shard != nullptr && !ts_host::aligned16(grad_weight_shard)))
    return fail(TS_ERR_INVALID_ARGUMENT, "flce_vocab_bwd: gradients must be 16-byte aligned");
  const VocabLayout lay = vocab_layout(N, Vp);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  __bf16* L = reinterpret_cast<__bf16*>(ws + lay.off_logits);
  float* lse_ws = lse != nullptr ? lse : reinterpret_cast<float*>(ws + lay.off_lse);
  float* rows_ws = loss_rows != nullptr ? loss_rows : reinterpret_cast<float*>(ws + lay.off_rows);
  int* n_valid = reinterpret_cast<int*>(ws + lay.off_misc);
  float* scale = reinterpret_cast<float*>(ws + lay.off_misc + 16);
  hipStream_t st = static_cast<hipStream_t>(stream);

  hipLaunchKernelGGL(flce_count, dim3(1), dim3(256), 0, st, labels, N, ignore_index, n_valid);
  TS_TRY(ts_host::check_launch("flce_count"));
  hipLaunchKernelGGL(flce_vocab_merge, dim3((unsigned)((N + 63) / 64)), dim3(64), 0, st,
                     reinterpret_cast<const ShardStats*>(stats_all), P, N, labels, ignore_index,
                     lse_ws, rows_ws);
  TS_TRY(ts_host::check_launch("flce_vocab_merge"));
  hipLaunchKernelGGL(flce_loss, dim3(1), dim3(256), 0, st, rows_ws, N, n_valid,
                     reduction == 0 ? 1 : 0, loss, scale);
  TS_TRY(ts_host::check_launch("flce_loss"));
  if (grad_hidden_partial == nullptr && grad_weight_shard == nullptr) return TS_OK;
  const int64_t ldl = logits_ld(Vp);
  const int64_t dchunks = ts_plan::chunks_for((Vp + 7) / 8, 256, kDlKv);
  hipLaunchKernelGGL(flce_dlogits, dim3((unsigned)(N * dchunks)), dim3(256), 0, st, L, ldl,
                     lse_ws, labels, Vp, dchunks, ignore_index, scale, vocab_start);
  TS_TRY(ts_host::check_launch("flce_dlogits"));
  const __bf16* Hd = static_cast<const __bf16*>(hidden);
  const __bf16* Wd = static_cast<const __bf16*>(weight);
  using ts_gemm::kKMajor;
  using ts_gemm::kMNMajor;
  GemmArgs dh{};
  dh.A = L;  // dlogits [N, Vp], K-major (zero from Vp to the end of the row's last vector)
  dh.lda = ldl;
  dh.B = Wd;  // weight shard [Vp, H] as the [H, Vp] operand: MN-major
  dh.ldb = ldw;
  dh.M = N;
  dh.N = H;
  dh.K = Vp;
  dh.C = static_cast<__bf16*>(grad_hidden_partial);
  dh.ldc = H;
  GemmArgs dw{};
  dw.A = L;  // dlogits [N, Vp] as the [Vp, N] operand: MN-major
  dw.lda = ldl;
  dw.B = Hd;  // hidden [N, H] as the [H, N] operand: MN-major
  dw.ldb = ldh;
  dw.M = Vp;
  dw.N = H;
  dw.K = N;
  dw.C = static_cast<__bf16*>(grad_weight_shard);
  dw.ldc = H;
  if (grad_hidden_partial != nullptr && grad_weight_shard != nullptr) {
    // both GEMMs read the same dlogits: one grid
    return launch_gemm_pair<kEpiBf16, kKMajor, kMNMajor, kEpiBf16, kMNMajor, kMNMajor>(
        dh, dw, st, "flce_vocab_gemm_grads");
  }
  if (grad_hidden_partial != nullptr)
    return launch_gemm<kEpiBf16, kKMajor, kMNMajor>(dh, st, "flce_vocab_gemm_dhidden");
  return launch_gemm<kEpiBf16, kMNMajor, kMNMajor>(dw, st, "flce_vocab_gemm_dweight");
}

namespace {
ts_status scale_launch(const char* what, void* x, int64_t n, ts_dtype dtype, const float* num,
                       const float* den, float* hint_out, hipStream_t st) {
  if (!ts_host::valid_dtype(dtype))
    return ts_host::fail(TS_ERR_UNSUPPORTED_DTYPE, "%s: bad dtype", what);
  if (n < 0) return ts_host::fail(TS_ERR_SHAPE, "%s: n must be non-negative", what);
  if (num == nullptr) return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "%s: NULL factor", what);
  if (n > 0 && x == nullptr) return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "%s: NULL x", what);
  if (hint_out != nullptr && (hint_out == num || hint_out == den))
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "%s: hint_out aliases an input", what);
  if (n == 0 && hint_out == nullptr) return TS_OK;
  const int64_t per = dtype == TS_F32 ? 4 : 8;
  // whole 16-byte vectors when x is aligned; the rest element by element
  const int64_t nvec = ts_host::aligned16(x) ? n / per : 0;
  const int64_t tail = n - nvec * per;
  int64_t blocks = (nvec + 256 * kScaleUnroll - 1) / (256 * kScaleUnroll);
  const int64_t tail_blocks = (tail + 255) / 256;
  if (tail_blocks > blocks) blocks = tail_blocks;
  if (blocks > kScaleGrid) blocks = kScaleGrid;
  if (blocks < 1) blocks = 1;
  switch (dtype) {
    case TS_BF16:
      hipLaunchKernelGGL(scale_inplace<__bf16>, dim3((unsigned)blocks), dim3(256), 0, st,
                         static_cast<__bf16*>(x), nvec, n, num, den, hint_out);
      break;
    case TS_F16:
      hipLaunchKernelGGL(scale_inplace<_Float16>, dim3((unsigned)blocks), dim3(256), 0, st,
                         static_cast<_Float16*>(x), nvec, n, num, den, hint_out);
      break;
    case TS_F32:
      hipLaunchKernelGGL(scale_inplace<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                         static_cast<float*>(x), nvec, n, num, den, hint_out);
      break;
  }
  return ts_host::check_launch(what);
}
}  // namespace

extern "C" ts_status ts_scale_inplace(void* x, int64_t n, ts_dtype dtype, const float* scale,
                                      ts_stream_t stream) {
  return scale_launch("scale_inplace", x, n, dtype, scale, nullptr, nullptr,
                      static_cast<hipStream_t>(stream));
}

extern "C" ts_status ts_rescale_inplace(void* x, int64_t n, ts_dtype dtype, const float* now,
                                        const float* used, float* hint_out,
                                        ts_stream_t stream) {
  if (used == nullptr)
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "rescale_inplace: NULL used factor");
  return scale_launch("rescale_inplace", x, n, dtype, now, used, hint_out,
                      static_cast<hipStream_t>(stream));
}
