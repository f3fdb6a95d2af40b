// RMSNorm forward/backward for gfx950.
//
// Register path (ts_plan::rms_fwd_plan / rms_bwd_row_plan): a row is owned by
// TPR threads (whole waves), each holding KV 16-byte vectors spaced TPR
// vectors apart, so every load instruction of a wave covers 1 KiB of
// contiguous row and each thread has only one or two loads in flight per
// tensor; the row stays in VGPRs between the reduction and the output, so x
// (and dy) are read from HBM exactly once. The sum of squares (forward) and
// sum(dy*w*xhat) (backward) are reduced with DPP inside each wave and through
// LDS across the row's waves.
//
// Backward: each workgroup walks `steps` consecutive groups of rows and keeps
// dy*xhat for its threads' columns in fp32 registers, then writes one fp32
// partial row per row slot; rms_dw_reduce4 sums the partial rows in a fixed
// order. dW is therefore bit-reproducible run to run (no float atomics),
// unlike the reference's atomic_add variant.
//
// Generic path (row length not a multiple of the 16-byte vector, unaligned
// pointers, or rows longer than the register plans): one workgroup per row
// with element-wise loads and two passes over the row.
#include <mutex>

#include "common.hpp"
#include "plan.hpp"

// Device scratch of ts_rmsnorm_bwd_noalloc: the fp32 dW partial rows, for
// callers that cannot allocate. Each device that runs the library holds its
// own copy for the life of the process. Its contents need no clearing
// between calls: the dx kernel overwrites every partial row the reduction
// reads.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

using namespace ts;

// Loads V weights for the 16-byte data vector starting at element e.
template <typename W, int V>
__device__ inline void load_w(const W* __restrict__ w, int64_t e, float* f) {
  if constexpr (sizeof(W) == 4) {
#pragma unroll
    for (int h = 0; h < V / 4; ++h) Elt<float>::unpack(ld16(w + e + 4 * h), f + 4 * h);
  } else {
    static_assert(Elt<W>::kVec == V, "16-bit weight vector must match data vector");
    Elt<W>::unpack(ld16(w + e), f);
  }
}

// Sum of v over the TPR threads that own one row. `red` holds one float per
// wave of the workgroup; contains one barrier when TPR > 64 (every thread of
// the workgroup must call it).
template <int TPR, int kBlock>
__device__ inline float row_reduce(float v, float* red) {
  v = wave_sum(v);
  if constexpr (TPR == kWave) {
    return v;
  } else {
    constexpr int kWavesPerRow = TPR / kWave;
    const int wid = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) red[wid] = v;
    __syncthreads();
    const int first = (wid / kWavesPerRow) * kWavesPerRow;
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kWavesPerRow; ++i) t += red[first + i];
    return t;
  }
}

// Residual input of the fused add + RMSNorm (kAdd kernels): the normalised
// row is h = x + r in fp32; h rounded to the data type is stored to `h` when
// it is not null (the reference's residual_out).
template <typename T>
struct AddArgs {
  const T* r;
  int64_t ldr;
  T* h;
  int64_t ldh;
};

// x (+ r) of one 16-byte vector, in fp32.
template <typename T, bool kAdd>
__device__ inline void row_values(const u32x4& xq, const u32x4& rq, float* f) {
  Elt<T>::unpack(xq, f);
  if constexpr (kAdd) {
    float g[Elt<T>::kVec];
    Elt<T>::unpack(rq, g);
#pragma unroll
    for (int i = 0; i < Elt<T>::kVec; ++i) f[i] += g[i];
  }
}

// ---------------------------------------------------------------------------
// Forward, register path.
// ---------------------------------------------------------------------------
template <typename T, typename W, int TPR, int KV, bool kAdd>
__global__ __launch_bounds__(TPR > 256 ? TPR : 256) void rms_fwd_reg(
    const T* __restrict__ x, int64_t ldx, const W* __restrict__ w, T* __restrict__ y,
    int64_t ldy, float* __restrict__ rstd_out, int64_t rows, int nvec, float fcols, float eps,
    int twice, AddArgs<T> add) {
  constexpr int V = Elt<T>::kVec;
  constexpr int kBlock = TPR > 256 ? TPR : 256;
  constexpr int kRpb = kBlock / TPR;
  constexpr int KR = kAdd ? KV : 1;
  __shared__ float red[kBlock / kWave];
  const int sub = threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * kRpb + sub;
  const bool valid = row < rows;

  // this thread's vectors of the row (ts_plan::chunk_vec), accessed where
  // ts_plan::row_vec_in holds
  const T* xr = x + row * ldx;
  u32x4 xv[KV], rv[KR];
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = (int)ts_plan::chunk_vec(0, k, t, TPR, KV);
    xv[k] = ts_plan::row_vec_in(row, rows, v, nvec) ? ld16_stream(xr + (int64_t)v * V)
                                                    : u32x4{0, 0, 0, 0};
  }
  if constexpr (kAdd) {
    const T* rr = add.r + row * add.ldr;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      const int v = (int)ts_plan::chunk_vec(0, k, t, TPR, KV);
      rv[k] = ts_plan::row_vec_in(row, rows, v, nvec) ? ld16_stream(rr + (int64_t)v * V)
                                                      : u32x4{0, 0, 0, 0};
    }
  } else {
    rv[0] = u32x4{0, 0, 0, 0};
  }
  // The weights go out with the row's loads (they are shared by every row and
  // come from L2): loaded after the reduction they put an L2 round trip
  // between rstd and the stores of every workgroup.
  constexpr int kWq = sizeof(W) == 4 ? V / 4 : 1;  // 16-byte weight loads per data vector
  constexpr int kWe = 16 / (int)sizeof(W);         // weights per 16-byte load
  static_assert(kWq * kWe == V, "weight loads must cover one data vector");
  u32x4 wq[KV][kWq];
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = t + k * TPR;
#pragma unroll
    for (int h = 0; h < kWq; ++h)
      wq[k][h] = w != nullptr && v < nvec ? ld16(w + (int64_t)v * V + h * kWe) : u32x4{0, 0, 0, 0};
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    float f[V];
    row_values<T, kAdd>(xv[k], rv[kAdd ? k : 0], f);
#pragma unroll
    for (int i = 0; i < V; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    if constexpr (kAdd) {
      const int v = t + k * TPR;
      if (add.h != nullptr && valid && v < nvec)
        st16_stream(add.h + row * add.ldh + (int64_t)v * V, Elt<T>::pack(f));
    }
  }
  ss = row_reduce<TPR, kBlock>(ss, red);
  // mean(x^2) = sum / n (a division, as the reference divides by n_cols), then
  // 1/sqrt with correctly rounded sqrt and divide.
  const float rstd = 1.0f / __builtin_sqrtf(ss / fcols + eps);
  if (!valid) return;  // no barrier below
  if (t == 0) rstd_out[row] = rstd;

  T* yr = y + row * ldy;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = t + k * TPR;
    if (v < nvec) {
      float f[V];
      row_values<T, kAdd>(xv[k], rv[kAdd ? k : 0], f);
      if (w != nullptr) {
        float wf[V];
#pragma unroll
        for (int h = 0; h < kWq; ++h) Elt<W>::unpack(wq[k][h], wf + h * kWe);
        if (twice) {
#pragma unroll
          for (int i = 0; i < V; ++i) f[i] = Elt<T>::round(f[i] * rstd) * wf[i];
        } else {
#pragma unroll
          for (int i = 0; i < V; ++i) f[i] = (f[i] * rstd) * wf[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) f[i] = f[i] * rstd;
      }
      st16_stream(yr + (int64_t)v * V, Elt<T>::pack(f));
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, register path: dx plus one fp32 dW partial row per row slot.
// Workgroup b handles row groups b, b + G, b + 2G, ... (G = gridDim.x, at
// most `steps` of them), each of kRpb rows. At any moment the running
// workgroups then work on about G consecutive row groups, a compact window of
// HBM, rather than on G groups spread over the whole matrix: measured on
// MI355X at [16384, 4096] (G = 512), 73 us against 82 us for contiguous
// blocks of row groups per workgroup; 265 us against 300 us at [32768, 8192].
// ---------------------------------------------------------------------------
template <typename T, int KV>
struct BwdSlot {
  u32x4 xv[KV], dv[KV];  // raw loads; lanes outside the matrix hold other data
  float rstd;            // raw load
  bool valid;            // row inside this workgroup's range and the matrix
};

template <typename T, typename W, int TPR, int KV>
__global__ __launch_bounds__(512) void rms_bwd_reg(
    const T* __restrict__ dy, int64_t lddy, const T* __restrict__ x, int64_t ldx,
    const W* __restrict__ w, const float* __restrict__ rstd_in, T* __restrict__ dx,
    int64_t lddx, float* __restrict__ partial, int64_t rows, int64_t steps, int nvec,
    float fcols) {
  constexpr int V = Elt<T>::kVec;
  constexpr int kBlock = 512;
  constexpr int kRpb = kBlock / TPR;
  __shared__ float red[2][kBlock / kWave];
  const int sub = threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;

  float wf[KV][V];
  float acc[KV][V];
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = t + k * TPR;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      acc[k][i] = 0.f;
      wf[k][i] = 1.f;
    }
    if (w != nullptr && v < nvec) load_w<W, V>(w, (int64_t)v * V, wf[k]);
  }

  // Loads of row group st into `sl` (zeros past the end of this workgroup's
  // range or of the matrix).
  // This thread's first row; row group st adds st * rstep rows.
  const int64_t row0 = (int64_t)blockIdx.x * kRpb + sub;
  const int64_t rstep = (int64_t)gridDim.x * kRpb;
  // The loads are unconditional: a lane with nothing to load (a row past this
  // workgroup's range or the matrix, or a vector past the row) loads the
  // matrix's first element instead (ts_plan::rms_bwd_load_offset), which
  // exists whenever the kernel runs, and the data of such lanes is zeroed
  // where it is used, which keeps the loads free of branches.
  auto issue = [&](BwdSlot<T, KV>& sl, int64_t st) {
    const int64_t row = row0 + st * rstep;
    const bool valid = st < steps && row < rows;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      sl.xv[k] = ld16_stream(x + ts_plan::rms_bwd_load_offset(row0, st, rstep, steps, rows, t, k,
                                                              TPR, V, nvec, ldx));
      sl.dv[k] = ld16_stream(dy + ts_plan::rms_bwd_load_offset(row0, st, rstep, steps, rows, t,
                                                               k, TPR, V, nvec, lddy));
    }
    sl.rstd = rstd_in[valid ? row : 0];
    sl.valid = valid;
  };

  // dx of row group st from its loaded slot; dW contributions into acc.
  auto body = [&](BwdSlot<T, KV>& sl, int64_t st) {
    const int64_t row = row0 + st * rstep;
    const bool valid = sl.valid;
    const float rstd = valid ? sl.rstd : 0.f;
    const u32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      const bool ok = valid && t + k * TPR < nvec;
      sl.xv[k] = ok ? sl.xv[k] : zero;
      sl.dv[k] = ok ? sl.dv[k] : zero;
    }
    // c1 = mean(dy * w * xhat); rows that are not valid hold zeros.
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      float xf[V], df[V];
      Elt<T>::unpack(sl.xv[k], xf);
      Elt<T>::unpack(sl.dv[k], df);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float xh = xf[i] * rstd;
        s = __builtin_fmaf(df[i] * wf[k][i], xh, s);
        acc[k][i] = __builtin_fmaf(df[i], xh, acc[k][i]);
      }
    }
    const float c1 = row_reduce<TPR, kBlock>(s, red[st & 1]) / fcols;
    // dx unpacks the slot again: carrying the unpacked floats across the
    // reduction would double the slot's registers.
#pragma unroll
    for (int k = 0; k < KV; ++k) asm volatile("" : "+v"(sl.xv[k]), "+v"(sl.dv[k]));
    if (valid) {
      T* dxr = dx + row * lddx;
#pragma unroll
      for (int k = 0; k < KV; ++k) {
        const int v = t + k * TPR;
        if (v < nvec) {
          float xf[V], df[V], o[V];
          Elt<T>::unpack(sl.xv[k], xf);
          Elt<T>::unpack(sl.dv[k], df);
#pragma unroll
          for (int i = 0; i < V; ++i) o[i] = rstd * (df[i] * wf[k][i] - (xf[i] * rstd) * c1);
          st16_stream(dxr + (int64_t)v * V, Elt<T>::pack(o));
        }
      }
    }
  };

  // `steps` is uniform over the workgroup (barriers inside row_reduce when
  // TPR > 64).
  for (int64_t st = 0; st < steps; ++st) {
    BwdSlot<T, KV> sl;
    issue(sl, st);
    body(sl, st);
  }

  if (partial == nullptr) return;  // dW not requested
  const int ncols = nvec * V;
  float* prow = partial + ((int64_t)blockIdx.x * kRpb + sub) * ncols;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = t + k * TPR;
    if (v < nvec) {
#pragma unroll
      for (int h = 0; h < V / 4; ++h) {
        *reinterpret_cast<float4*>(prow + v * V + 4 * h) =
            make_float4(acc[k][4 * h], acc[k][4 * h + 1], acc[k][4 * h + 2], acc[k][4 * h + 3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, one wave per row (ts_plan::rms_bwd_wave_plan): lane l holds the
// row's 16-byte vectors l, l + 64, ... (KV of them), so sum(dy * w * xhat) is
// a wave reduction (DPP and lane reads: no LDS, no barrier). Wave j of
// workgroup b takes rows (b * kR + j) + s * gridDim.x * kR, s < steps: as in
// rms_bwd_reg, the running workgroups stay on a compact window of rows.
//
// Rows are addressed through buffer resources (ts_plan::rms_bwd_wave_row):
// a row's resource spans that row, or nothing for a row past the matrix, so
// loads past it read zeros and stores past it are dropped by the hardware,
// and the loop has no branches around memory operations. The next row's
// loads are issued before this row's dx stores: vmcnt counts loads and
// stores in issue order, so the wait for those loads at the top of the next
// step does not wait for the stores.
//
// dW: each lane keeps dy * xhat of its columns over its wave's rows in fp32;
// at the end the kR waves' sums are added in LDS in a fixed order and the
// workgroup writes one fp32 partial row (rms_dw_reduce4 sums those).
// ---------------------------------------------------------------------------
template <typename T, typename W, int KV>
__global__ __launch_bounds__(64 * ts_plan::kWaveRowsPerBlock)
__attribute__((amdgpu_waves_per_eu(2, 2))) void rms_bwd_wave(
    const T* __restrict__ dy, int64_t lddy, const T* __restrict__ x, int64_t ldx,
    const W* __restrict__ w, const float* __restrict__ rstd_in, T* __restrict__ dx,
    int64_t lddx, float* __restrict__ partial, int64_t rows, int64_t steps, int nvec,
    float fcols) {
  constexpr int V = Elt<T>::kVec;
  constexpr int kR = ts_plan::kWaveRowsPerBlock;
  constexpr int kWv = Elt<W>::kVec;
  constexpr int kWq = V / kWv;  // 16-byte weight vectors per data vector (1 or 2)
  // dW of the kR waves before they are combined: up to kWaveRowMaxVec vectors each
  __shared__ float4 dw_lds[kR * ts_plan::kWaveRowMaxVec * V / 4];
  const int lane = threadIdx.x & (kWave - 1);
  // uniform over the wave: keeps the row's buffer resources in SGPRs
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);

  // lane-invariant byte offsets of this lane's vectors within a row
  int voff[KV];
  u32x4 wq[KV][kWq];
  float acc[KV][V];
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = lane + k * kWave;
    voff[k] = v < nvec ? v * 16 : kBufOob;
#pragma unroll
    for (int i = 0; i < V; ++i) acc[k][i] = 0.f;
#pragma unroll
    for (int h = 0; h < kWq; ++h) {
      if (w != nullptr && v < nvec) {
        wq[k][h] = ld16(w + (int64_t)v * V + h * kWv);
      } else {
        float one[kWv];
#pragma unroll
        for (int i = 0; i < kWv; ++i) one[i] = 1.f;
        wq[k][h] = Elt<W>::pack(one);
      }
    }
  }

  const int64_t row0 = (int64_t)blockIdx.x * kR + wid;
  const int64_t rstep = (int64_t)gridDim.x * kR;
  const uint32_t row_bytes = (uint32_t)nvec * 16u;
  u32x4 xv[KV], dv[KV];
  auto issue = [&](int64_t st) {
    const ts_plan::RowSpan sx = ts_plan::rms_bwd_wave_row(row0, st, rstep, steps, rows, ldx,
                                                          row_bytes);
    const ts_plan::RowSpan sd = ts_plan::rms_bwd_wave_row(row0, st, rstep, steps, rows, lddy,
                                                          row_bytes);
    const Rsrc rx = buf_rsrc(x + sx.offset, sx.bytes);
    const Rsrc rd = buf_rsrc(dy + sd.offset, sd.bytes);
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      xv[k] = buf_ld16_stream(rx, voff[k]);
      dv[k] = buf_ld16_stream(rd, voff[k]);
    }
  };

  issue(0);
  {  // as in rms_bwd_reg: enter the loop with the back edge's loads-then-stores pattern
    const Rsrc none = buf_rsrc(dx, 0u);
#pragma unroll
    for (int k = 0; k < KV; ++k) buf_st16_stream(u32x4{0u, 0u, 0u, 0u}, none, voff[k]);
  }
  for (int64_t st = 0; st < steps; ++st) {
    const int64_t row = row0 + st * rstep;
    const bool valid = row < rows;
    const float rstd = valid ? rstd_in[row] : 0.f;
    // c1 = mean(dy * w * xhat); lanes and rows outside the matrix loaded zeros
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      float xf[V], df[V], wf[V];
      Elt<T>::unpack(xv[k], xf);
      Elt<T>::unpack(dv[k], df);
#pragma unroll
      for (int h = 0; h < kWq; ++h) Elt<W>::unpack(wq[k][h], wf + h * kWv);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float xh = xf[i] * rstd;
        s = __builtin_fmaf(df[i] * wf[i], xh, s);
        acc[k][i] = __builtin_fmaf(df[i], xh, acc[k][i]);
      }
    }
    const float c1 = wave_sum(s) / fcols;
    // dx unpacks the raw vectors again: carrying the unpacked floats across the
    // reduction would triple their registers
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      asm volatile("" : "+v"(xv[k]), "+v"(dv[k]));
#pragma unroll
      for (int h = 0; h < kWq; ++h) asm volatile("" : "+v"(wq[k][h]));
    }
    u32x4 o[KV];
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      float xf[V], df[V], wf[V], of[V];
      Elt<T>::unpack(xv[k], xf);
      Elt<T>::unpack(dv[k], df);
#pragma unroll
      for (int h = 0; h < kWq; ++h) Elt<W>::unpack(wq[k][h], wf + h * kWv);
#pragma unroll
      for (int i = 0; i < V; ++i) of[i] = rstd * (df[i] * wf[i] - (xf[i] * rstd) * c1);
      o[k] = Elt<T>::pack(of);
    }
    issue(st + 1);  // a step past `steps` spans nothing: its loads read zeros
    const ts_plan::RowSpan so = ts_plan::rms_bwd_wave_row(row0, st, rstep, steps, rows, lddx,
                                                          row_bytes);
    const Rsrc ro = buf_rsrc(dx + so.offset, so.bytes);
#pragma unroll
    for (int k = 0; k < KV; ++k) buf_st16_stream(o[k], ro, voff[k]);
  }

  if (partial == nullptr) return;  // dW not requested
  const int nq = nvec * V / 4;     // float4 quads of a row
  float4* mine = dw_lds + wid * nq;
#pragma unroll
  for (int k = 0; k < KV; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
#pragma unroll
      for (int h = 0; h < V / 4; ++h)
        mine[v * (V / 4) + h] =
            make_float4(acc[k][4 * h], acc[k][4 * h + 1], acc[k][4 * h + 2], acc[k][4 * h + 3]);
    }
  }
  __syncthreads();
  float4* prow = reinterpret_cast<float4*>(partial + (int64_t)blockIdx.x * nvec * V);
  for (int q = threadIdx.x; q < nq; q += kR * kWave) {
    float4 t = dw_lds[q];
#pragma unroll
    for (int j = 1; j < kR; ++j) {
      const float4 u = dw_lds[j * nq + q];
      t.x += u.x;
      t.y += u.y;
      t.z += u.z;
      t.w += u.w;
    }
    prow[q] = t;
  }
}

// Clears n bytes (a kernel rather than hipMemsetAsync, so a captured graph
// replays it like any other node).
__global__ __launch_bounds__(256) void zero_bytes(uint8_t* __restrict__ p, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// dW[c] = sum over partial rows, in a fixed order. cols % 4 == 0: a workgroup
// takes 16 columns (4 float4 quads) x 64 row groups, then a fixed tree over
// the 64 groups in LDS.
template <typename W>
__global__ __launch_bounds__(256) void rms_dw_reduce4(const float* __restrict__ partial,
                                                      int64_t nparts, int64_t cols,
                                                      W* __restrict__ dw) {
  __shared__ float4 red[64][4];
  const int cq = threadIdx.x & 3;
  const int g = threadIdx.x >> 2;
  const int64_t c = (int64_t)blockIdx.x * 16 + cq * 4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < cols) {
    for (int64_t b = g; b < nparts; b += 64) {
      const float4 v = *reinterpret_cast<const float4*>(partial + b * cols + c);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
  }
  red[g][cq] = s;
  __syncthreads();
#pragma unroll
  for (int h = 32; h >= 1; h >>= 1) {
    if (g < h) {
      const float4 o = red[g + h][cq];
      float4 m = red[g][cq];
      m.x += o.x;
      m.y += o.y;
      m.z += o.z;
      m.w += o.w;
      red[g][cq] = m;
    }
    __syncthreads();
  }
  if (g == 0 && c < cols) {
    const float4 t = red[0][cq];
    Elt<W>::store1(dw + c, t.x);
    Elt<W>::store1(dw + c + 1, t.y);
    Elt<W>::store1(dw + c + 2, t.z);
    Elt<W>::store1(dw + c + 3, t.w);
  }
}

// dW[c] for any column count: 64 columns per workgroup, 4 row groups per
// column combined in a fixed order through LDS.
template <typename W>
__global__ __launch_bounds__(256) void rms_dw_reduce1(const float* __restrict__ partial,
                                                      int64_t nparts, int64_t cols,
                                                      W* __restrict__ dw) {
  __shared__ float red[4][64];
  const int cl = threadIdx.x & 63;
  const int g = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + cl;
  float s = 0.f;
  if (c < cols) {
    for (int64_t b = g; b < nparts; b += 4) s += partial[b * cols + c];
  }
  red[g][cl] = s;
  __syncthreads();
  if (g == 0 && c < cols) {
    const float t = ((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl];
    Elt<W>::store1(dw + c, t);
  }
}

// ---------------------------------------------------------------------------
// Generic path: one 256-thread workgroup per row, element-wise.
// ---------------------------------------------------------------------------
template <typename T, typename W, bool kAdd>
__global__ __launch_bounds__(256) void rms_fwd_generic(const T* __restrict__ x, int64_t ldx,
                                                       const W* __restrict__ w,
                                                       T* __restrict__ y, int64_t ldy,
                                                       float* __restrict__ rstd_out,
                                                       int64_t cols, float eps, int twice,
                                                       AddArgs<T> add) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  const T* rr = kAdd ? add.r + row * add.ldr : nullptr;
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float f = Elt<T>::load1(xr + c);
    if constexpr (kAdd) {
      f += Elt<T>::load1(rr + c);
      if (add.h != nullptr) Elt<T>::store1(add.h + row * add.ldh + c, f);
    }
    ss = __builtin_fmaf(f, f, ss);
  }
  ss = block_sum<4>(ss, red);
  const float rstd = 1.0f / __builtin_sqrtf(ss / (float)cols + eps);
  if (threadIdx.x == 0) rstd_out[row] = rstd;
  T* yr = y + row * ldy;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    float f = Elt<T>::load1(xr + c);
    if constexpr (kAdd) f += Elt<T>::load1(rr + c);
    float o;
    if (w != nullptr) {
      const float wf = Elt<W>::load1(w + c);
      o = twice ? Elt<T>::round(f * rstd) * wf : (f * rstd) * wf;
    } else {
      o = f * rstd;
    }
    Elt<T>::store1(yr + c, o);
  }
}

template <typename T, typename W>
__global__ __launch_bounds__(256) void rms_bwd_dx_generic(
    const T* __restrict__ dy, int64_t lddy, const T* __restrict__ x, int64_t ldx,
    const W* __restrict__ w, const float* __restrict__ rstd_in, T* __restrict__ dx,
    int64_t lddx, int64_t cols) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  const T* dyr = dy + row * lddy;
  const float rstd = rstd_in[row];
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float wf = w != nullptr ? Elt<W>::load1(w + c) : 1.f;
    s = __builtin_fmaf(Elt<T>::load1(dyr + c) * wf, Elt<T>::load1(xr + c) * rstd, s);
  }
  const float c1 = block_sum<4>(s, red) / (float)cols;
  T* dxr = dx + row * lddx;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float wf = w != nullptr ? Elt<W>::load1(w + c) : 1.f;
    const float xh = Elt<T>::load1(xr + c) * rstd;
    Elt<T>::store1(dxr + c, rstd * (Elt<T>::load1(dyr + c) * wf - xh * c1));
  }
}

// partial[g][c] = sum over rows r in row-group g of dy[r,c] * x[r,c] * rstd[r]
template <typename T>
__global__ __launch_bounds__(256) void rms_bwd_dw_generic(
    const T* __restrict__ dy, int64_t lddy, const T* __restrict__ x, int64_t ldx,
    const float* __restrict__ rstd_in, float* __restrict__ partial, int64_t rows,
    int64_t cols, int64_t rows_per_group) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t g = blockIdx.y;
  if (c >= cols) return;
  const int64_t r0 = g * rows_per_group;
  const int64_t r1 = r0 + rows_per_group < rows ? r0 + rows_per_group : rows;
  float s = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    s = __builtin_fmaf(Elt<T>::load1(dy + r * lddy + c), Elt<T>::load1(x + r * ldx + c) * rstd_in[r],
                       s);
  }
  partial[g * cols + c] = s;
}

// ---------------------------------------------------------------------------
// Host dispatch. Grid sizes and the number of dW partial rows come from
// ts_plan (plan.hpp), the same functions the workspace-size query uses.
// ---------------------------------------------------------------------------
template <typename T, typename W>
bool vec_ok(const void* a, int64_t lda, int64_t cols, const void* w) {
  constexpr int V = sizeof(T) == 4 ? 4 : 8;
  return cols % V == 0 && lda % V == 0 && ts_host::aligned16(a) &&
         (w == nullptr || ts_host::aligned16(w));
}

template <typename T, typename W, bool kAdd = false>
ts_status fwd_typed(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy,
                    float* rstd, int64_t rows, int64_t cols, float eps, int twice,
                    hipStream_t st, AddArgs<T> add = AddArgs<T>{nullptr, 0, nullptr, 0}) {
  constexpr int V = sizeof(T) == 4 ? 4 : 8;
  const T* xp = static_cast<const T*>(x);
  const W* wp = static_cast<const W*>(w);
  T* yp = static_cast<T*>(y);
  const int64_t nvec = cols / V;
  const ts_plan::RmsRowPlan plan = ts_plan::rms_fwd_plan(nvec);
  const bool add_ok = !kAdd || (vec_ok<T, W>(add.r, add.ldr, cols, nullptr) &&
                                (add.h == nullptr || vec_ok<T, W>(add.h, add.ldh, cols, nullptr)));
  if (vec_ok<T, W>(x, ldx, cols, w) && vec_ok<T, W>(y, ldy, cols, nullptr) && add_ok &&
      plan.reg) {
    const dim3 grid((unsigned)((rows + plan.rpb - 1) / plan.rpb));
    const dim3 block(plan.block);
    bool launched = false;
#define TS_LAUNCH_FWD(TPR, KV)                                                                 \
  if (plan.tpr == TPR && plan.kv == KV) {                                                      \
    hipLaunchKernelGGL((rms_fwd_reg<T, W, TPR, KV, kAdd>), grid, block, 0, st, xp, ldx, wp,    \
                       yp, ldy, rstd, rows, (int)nvec, (float)cols, eps, twice, add);          \
    launched = true;                                                                           \
  }
    TS_LAUNCH_FWD(64, 1)
    TS_LAUNCH_FWD(64, 2)
    TS_LAUNCH_FWD(128, 2)
    TS_LAUNCH_FWD(256, 2)
    TS_LAUNCH_FWD(512, 2)
    TS_LAUNCH_FWD(512, 4)
#undef TS_LAUNCH_FWD
    if (!launched)
      return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_fwd: bad plan (tpr=%d kv=%d)",
                           plan.tpr, plan.kv);
    return ts_host::check_launch("rms_fwd_reg");
  }
  hipLaunchKernelGGL((rms_fwd_generic<T, W, kAdd>), dim3((unsigned)rows), dim3(256), 0, st, xp,
                     ldx, wp, yp, ldy, rstd, cols, eps, twice, add);
  return ts_host::check_launch("rms_fwd_generic");
}

template <typename T, typename W>
ts_status bwd_typed(const void* dy, int64_t lddy, const void* x, int64_t ldx, const void* w,
                    const float* rstd, void* dx, int64_t lddx, void* dw, float* ws,
                    size_t ws_bytes, int64_t rows, int64_t cols, hipStream_t st) {
  constexpr int V = sizeof(T) == 4 ? 4 : 8;
  const T* dyp = static_cast<const T*>(dy);
  const T* xp = static_cast<const T*>(x);
  const W* wp = static_cast<const W*>(w);
  T* dxp = static_cast<T*>(dx);
  const int64_t nvec = cols / V;
  const bool vec = vec_ok<T, W>(x, ldx, cols, w) && vec_ok<T, W>(dy, lddy, cols, nullptr) &&
                   vec_ok<T, W>(dx, lddx, cols, nullptr);
  const ts_plan::RmsBwdPlan plan =
      ts_plan::rms_bwd_plan(rows, cols, (int)sizeof(T), vec, dw != nullptr);
  if (dw != nullptr && (size_t)plan.nparts * (size_t)cols * sizeof(float) > ws_bytes)
    return ts_host::fail(TS_ERR_WORKSPACE, "rmsnorm_bwd: plan needs %lld partial rows",
                         (long long)plan.nparts);
  if (plan.wave) {
    float* part = dw != nullptr ? ws : nullptr;
    bool launched = false;
#define TS_LAUNCH_WAVE(KV)                                                                     \
  if (plan.row.kv == KV) {                                                                     \
    hipLaunchKernelGGL((rms_bwd_wave<T, W, KV>), dim3((unsigned)plan.grid),                    \
                       dim3(plan.row.block), 0, st, dyp, lddy, xp, ldx, wp, rstd, dxp, lddx,   \
                       part, rows, plan.steps, (int)nvec, (float)cols);                        \
    launched = true;                                                                           \
  }
    TS_LAUNCH_WAVE(2)
    TS_LAUNCH_WAVE(4)
#undef TS_LAUNCH_WAVE
    if (!launched)
      return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_bwd: bad wave plan (kv=%d)",
                           plan.row.kv);
    ts_status s = ts_host::check_launch("rms_bwd_wave");
    if (s != TS_OK) return s;
  } else if (plan.reg) {
    float* part = dw != nullptr ? ws : nullptr;
    bool launched = false;
#define TS_LAUNCH_BWD(TPR, KV)                                                                  \
  if (plan.row.tpr == TPR && plan.row.kv == KV) {                                               \
    hipLaunchKernelGGL((rms_bwd_reg<T, W, TPR, KV>), dim3((unsigned)plan.grid), dim3(512), 0,   \
                       st, dyp, lddy, xp, ldx, wp, rstd, dxp, lddx, part, rows, plan.steps,     \
                       (int)nvec, (float)cols);                                                 \
    launched = true;                                                                            \
  }
    TS_LAUNCH_BWD(64, 1)
    TS_LAUNCH_BWD(128, 1)
    TS_LAUNCH_BWD(256, 1)
    TS_LAUNCH_BWD(512, 1)
    TS_LAUNCH_BWD(512, 2)
    TS_LAUNCH_BWD(512, 4)
#undef TS_LAUNCH_BWD
    if (!launched)
      return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_bwd: bad plan (tpr=%d kv=%d)",
                           plan.row.tpr, plan.row.kv);
    ts_status s = ts_host::check_launch("rms_bwd_reg");
    if (s != TS_OK) return s;
  } else {
    hipLaunchKernelGGL((rms_bwd_dx_generic<T, W>), dim3((unsigned)rows), dim3(256), 0, st, dyp,
                       lddy, xp, ldx, wp, rstd, dxp, lddx, cols);
    ts_status s = ts_host::check_launch("rms_bwd_dx_generic");
    if (s != TS_OK) return s;
    if (dw != nullptr) {
      hipLaunchKernelGGL((rms_bwd_dw_generic<T>), dim3((unsigned)((cols + 255) / 256),
                                                       (unsigned)plan.nparts),
                         dim3(256), 0, st, dyp, lddy, xp, ldx, rstd, ws, rows, cols,
                         ts_plan::kGenericRowsPerGroup);
      s = ts_host::check_launch("rms_bwd_dw_generic");
      if (s != TS_OK) return s;
    }
  }
  if (dw != nullptr) {
    if (cols % 4 == 0) {
      hipLaunchKernelGGL((rms_dw_reduce4<W>), dim3((unsigned)((cols + 15) / 16)), dim3(256), 0,
                         st, ws, plan.nparts, cols, static_cast<W*>(dw));
      return ts_host::check_launch("rms_dw_reduce4");
    }
    hipLaunchKernelGGL((rms_dw_reduce1<W>), dim3((unsigned)((cols + 63) / 64)), dim3(256), 0, st,
                       ws, plan.nparts, cols, static_cast<W*>(dw));
    return ts_host::check_launch("rms_dw_reduce1");
  }
  return TS_OK;
}

ts_status check_common(const void* x, int64_t ldx, ts_dtype x_dtype, const void* w,
                       ts_dtype w_dtype, int64_t rows, int64_t cols) {
  using ts_host::fail;
  if (!ts_host::valid_dtype(x_dtype) || (w != nullptr && !ts_host::valid_dtype(w_dtype)))
    return fail(TS_ERR_UNSUPPORTED_DTYPE, "rmsnorm: unsupported dtype (x=%d, w=%d)", (int)x_dtype,
                (int)w_dtype);
  if (w != nullptr && w_dtype != x_dtype && w_dtype != TS_F32)
    return fail(TS_ERR_UNSUPPORTED_DTYPE,
                "rmsnorm: weight dtype must equal the data dtype or be float32");
  if (rows < 0 || cols <= 0)
    return fail(TS_ERR_SHAPE, "rmsnorm: bad shape rows=%lld cols=%lld", (long long)rows,
                (long long)cols);
  if (cols > (int64_t)1 << 30 || rows > ((int64_t)1 << 31) - 1)
    return fail(TS_ERR_SHAPE, "rmsnorm: shape too large rows=%lld cols=%lld", (long long)rows,
                (long long)cols);
  if (x == nullptr && rows > 0) return fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm: x is NULL");
  if (ldx < cols) return fail(TS_ERR_SHAPE, "rmsnorm: row stride %lld < cols %lld",
                              (long long)ldx, (long long)cols);
  return TS_OK;
}

}  // namespace

extern "C" ts_status ts_rmsnorm_fwd(const void* x, int64_t ldx, ts_dtype x_dtype, const void* w,
                                    ts_dtype w_dtype, void* y, int64_t ldy, float* rstd,
                                    int64_t rows, int64_t cols, float eps, int32_t round_mode,
                                    ts_stream_t stream) {
  using ts_host::fail;
  ts_status s = check_common(x, ldx, x_dtype, w, w_dtype, rows, cols);
  if (s != TS_OK) return s;
  if (rows > 0 && (y == nullptr || rstd == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_fwd: y or rstd is NULL");
  if (ldy < cols) return fail(TS_ERR_SHAPE, "rmsnorm_fwd: y row stride < cols");
  if (!(eps >= 0.f)) return fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_fwd: eps must be >= 0");
  if (round_mode != TS_RMS_ROUND_ONCE && round_mode != TS_RMS_ROUND_TWICE)
    return fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_fwd: bad round_mode %d", (int)round_mode);
  if (rows == 0) return TS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Double rounding only exists when the weight has the 16-bit data dtype.
  const int twice = round_mode == TS_RMS_ROUND_TWICE && w != nullptr && w_dtype == x_dtype &&
                    x_dtype != TS_F32;
  switch (x_dtype) {
    case TS_BF16:
      return w_dtype == TS_F32 && w != nullptr
                 ? fwd_typed<__bf16, float>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st)
                 : fwd_typed<__bf16, __bf16>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st);
    case TS_F16:
      return w_dtype == TS_F32 && w != nullptr
                 ? fwd_typed<_Float16, float>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st)
                 : fwd_typed<_Float16, _Float16>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice,
                                                 st);
    case TS_F32:
      return fwd_typed<float, float>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st);
  }
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "rmsnorm_fwd: unsupported dtype");
}

extern "C" ts_status ts_add_rmsnorm_fwd(const void* x, int64_t ldx, const void* residual,
                                        int64_t ldr, ts_dtype x_dtype, const void* w,
                                        ts_dtype w_dtype, void* y, int64_t ldy, void* h_out,
                                        int64_t ldh, float* rstd, int64_t rows, int64_t cols,
                                        float eps, int32_t round_mode, ts_stream_t stream) {
  using ts_host::fail;
  ts_status s = check_common(x, ldx, x_dtype, w, w_dtype, rows, cols);
  if (s != TS_OK) return s;
  if (rows > 0 && (residual == nullptr || y == nullptr || rstd == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "add_rmsnorm_fwd: residual, y or rstd is NULL");
  if (ldr < cols || ldy < cols || (h_out != nullptr && ldh < cols))
    return fail(TS_ERR_SHAPE, "add_rmsnorm_fwd: row stride < cols");
  if (!(eps >= 0.f)) return fail(TS_ERR_INVALID_ARGUMENT, "add_rmsnorm_fwd: eps must be >= 0");
  if (round_mode != TS_RMS_ROUND_ONCE && round_mode != TS_RMS_ROUND_TWICE)
    return fail(TS_ERR_INVALID_ARGUMENT, "add_rmsnorm_fwd: bad round_mode %d", (int)round_mode);
  if (rows == 0) return TS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int twice = round_mode == TS_RMS_ROUND_TWICE && w != nullptr && w_dtype == x_dtype &&
                    x_dtype != TS_F32;
#define TS_ADD_FWD(T)                                                                          \
  {                                                                                            \
    const AddArgs<T> add{static_cast<const T*>(residual), ldr, static_cast<T*>(h_out), ldh};   \
    return w_dtype == TS_F32 && w != nullptr                                                   \
               ? fwd_typed<T, float, true>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st, \
                                           add)                                                \
               : fwd_typed<T, T, true>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st,    \
                                       add);                                                   \
  }
  switch (x_dtype) {
    case TS_BF16: TS_ADD_FWD(__bf16)
    case TS_F16: TS_ADD_FWD(_Float16)
    case TS_F32: {
      const AddArgs<float> add{static_cast<const float*>(residual), ldr,
                               static_cast<float*>(h_out), ldh};
      return fwd_typed<float, float, true>(x, ldx, w, y, ldy, rstd, rows, cols, eps, twice, st,
                                           add);
    }
  }
#undef TS_ADD_FWD
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "add_rmsnorm_fwd: unsupported dtype");
}

extern "C" size_t ts_rmsnorm_bwd_workspace_size(int64_t rows, int64_t cols) {
  return (size_t)ts_plan::rms_bwd_workspace_rows(rows, cols) * (size_t)(cols > 0 ? cols : 0) *
         sizeof(float);
}

extern "C" ts_status ts_rmsnorm_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx,
                                    ts_dtype x_dtype, const void* w, ts_dtype w_dtype,
                                    const float* rstd, void* dx, int64_t lddx, void* dw,
                                    void* workspace, size_t workspace_bytes, int64_t rows,
                                    int64_t cols, ts_stream_t stream) {
  using ts_host::fail;
  ts_status s = check_common(x, ldx, x_dtype, w, w_dtype, rows, cols);
  if (s != TS_OK) return s;
  if (rows > 0 && (dy == nullptr || rstd == nullptr || dx == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_bwd: dy, rstd or dx is NULL");
  if (lddy < cols || lddx < cols) return fail(TS_ERR_SHAPE, "rmsnorm_bwd: row stride < cols");
  if (dw != nullptr && w == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "rmsnorm_bwd: dw requested without a weight");
  if (dw != nullptr && rows > 0) {
    const size_t need = ts_rmsnorm_bwd_workspace_size(rows, cols);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(TS_ERR_WORKSPACE, "rmsnorm_bwd: workspace needs %zu bytes, got %zu", need,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    if (!ts_host::aligned16(workspace))
      return fail(TS_ERR_WORKSPACE, "rmsnorm_bwd: workspace must be 16-byte aligned");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0) {
    // Empty batch: dW is all zeros.
    if (dw != nullptr) {
      const size_t nbytes = (size_t)cols * ts_host::dtype_size(w_dtype);
      hipLaunchKernelGGL(zero_bytes, dim3((unsigned)((nbytes + 255) / 256)), dim3(256), 0, st,
                         static_cast<uint8_t*>(dw), nbytes);
      return ts_host::check_launch("zero_bytes");
    }
    return TS_OK;
  }
  float* ws = static_cast<float*>(workspace);
  const size_t wsb = workspace == nullptr ? 0 : workspace_bytes;
  const bool w32 = w != nullptr && w_dtype == TS_F32;
#define TS_BWD_ARGS dy, lddy, x, ldx, w, rstd, dx, lddx, dw, ws, wsb, rows, cols, st
  switch (x_dtype) {
    case TS_BF16:
      return w32 ? bwd_typed<__bf16, float>(TS_BWD_ARGS) : bwd_typed<__bf16, __bf16>(TS_BWD_ARGS);
    case TS_F16:
      return w32 ? bwd_typed<_Float16, float>(TS_BWD_ARGS)
                 : bwd_typed<_Float16, _Float16>(TS_BWD_ARGS);
    case TS_F32:
      return bwd_typed<float, float>(TS_BWD_ARGS);
  }
#undef TS_BWD_ARGS
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "rmsnorm_bwd: unsupported dtype");
}

namespace {

// Device address of `scratch` on each device, looked up once per device with
// that device current (the name itself is a host-side stand-in that must
// never reach a kernel).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

ts_status scratch_on_current_device(void** out) {
  using ts_host::fail;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(TS_ERR_DEVICE, "rmsnorm_bwd_noalloc: no current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(TS_ERR_DEVICE, "rmsnorm_bwd_noalloc: hipGetSymbolAddress failed on device %d: %s",
                  dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TS_OK;
}

}  // namespace

extern "C" size_t ts_rmsnorm_bwd_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" ts_status ts_rmsnorm_bwd_noalloc(const void* dy, int64_t lddy, const void* x,
                                            int64_t ldx, ts_dtype x_dtype, const void* w,
                                            ts_dtype w_dtype, const float* rstd, void* dx,
                                            int64_t lddx, void* dw, int64_t rows, int64_t cols,
                                            ts_stream_t stream) {
  void* ws = nullptr;
  size_t need = 0;
  if (dw != nullptr && rows > 0 && cols > 0) {
    need = ts_rmsnorm_bwd_workspace_size(rows, cols);
    if (need > kNoAllocScratchBytes)
      return ts_host::fail(TS_ERR_WORKSPACE,
                           "rmsnorm_bwd_noalloc: rows=%lld cols=%lld need %zu bytes of dW "
                           "partials, above the %zu-byte device scratch; use ts_rmsnorm_bwd "
                           "with a workspace",
                           (long long)rows, (long long)cols, need, kNoAllocScratchBytes);
    const ts_status s = scratch_on_current_device(&ws);
    if (s != TS_OK) return s;
  }
  return ts_rmsnorm_bwd(dy, lddy, x, ldx, x_dtype, w, w_dtype, rstd, dx, lddx, dw, ws,
                        ws != nullptr ? kNoAllocScratchBytes : 0, rows, cols, stream);
}
