// Vocabulary cross-entropy forward/backward for gfx950.
//
// Forward: one 256-thread workgroup per row. Each lane streams the row with
// 16-byte non-temporal loads (kUnroll vectors in flight per lane) and keeps an
// online (max, sum of exp) pair: a new chunk's max rescales the running sum
// once per chunk, not once per element. exp is evaluated as
// exp2(z*log2(e) - m*log2(e)) with one FMA and one v_exp_f32. The per-lane
// pairs are folded with a wave64 DPP max, a rescale, and DPP sums, then across
// the four waves through LDS. Rows whose label is ignore_index are not read:
// their loss is 0 and their lse is stored as 0 (the backward never reads it).
//
// Backward: one read and one write per element, grad = dloss * (softmax -
// onehot) (with the label-smoothing, softcap and logit-scale chain rules),
// written with 16-byte stores; it may overwrite the logits in place. The grid
// is one-shot over (row, chunk of 256 vectors) with one vector per thread:
// on MI355X a streaming kernel with few accesses per thread keeps more of HBM
// busy than one that loops along a row, or than two vectors per thread. Ignored rows are written as zeros
// without being read.
#include <math.h>

#include "common.hpp"
#include "plan.hpp"

namespace {

using namespace ts;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kUnroll = 4;   // vectors in flight per lane in the forward's row loop
// Vectors per thread in the backward's one-shot grid: one measured 1.304 ms
// against 1.405 ms with two at C3 [16384, 128256] bf16 on MI355X.
constexpr int kBwdKv = 1;
constexpr int64_t kMaxGridY = 65535;  // rows per backward launch

struct Xform {
  float scale;    // 0 = off
  float softcap;  // 0 = off
};

// Applies logit scaling then softcapping, in the reference's order
// (kernels/triton_kernels.py:214-217).
template <bool kXform>
__device__ inline float xform(float x, const Xform& t) {
  if constexpr (kXform) {
    if (t.scale != 0.f) x = t.scale * x;
    if (t.softcap != 0.f) x = t.softcap * tanhf(x / t.softcap);
  }
  return x;
}

// Block-wide (max, sum exp, sum z) fold. Every thread receives the results.
__device__ inline void block_fold(float& m, float& s, float& sz, float* lds) {
  float bm = wave_max(m);
  const int wid = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (lane == 0) lds[wid] = bm;
  __syncthreads();
  bm = lds[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) bm = fmaxf(bm, lds[i]);
  __syncthreads();
  // Rescale this lane's sum to the row max. A lane that saw only -inf has
  // s == 0 and contributes nothing.
  const float scaled = s == 0.f ? 0.f : s * fast_exp2((m - bm) * kLog2e);
  float ws = wave_sum(scaled);
  float wz = wave_sum(sz);
  if (lane == 0) {
    lds[wid] = ws;
    lds[kWaves + wid] = wz;
  }
  __syncthreads();
  float ts = 0.f, tz = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    ts += lds[i];
    tz += lds[kWaves + i];
  }
  m = bm;
  s = ts;
  sz = tz;
}

template <typename T, bool kXform, bool kSmooth>
__global__ __launch_bounds__(kThreads) void ce_fwd_vec(const T* __restrict__ logits, int64_t ld,
                                                       const int64_t* __restrict__ labels,
                                                       int64_t V, int64_t nvec,
                                                       int64_t ignore_index, Xform xf,
                                                       float smoothing, float* __restrict__ loss,
                                                       float* __restrict__ lse_out) {
  constexpr int VE = Elt<T>::kVec;
  __shared__ float lds[2 * kWaves];
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  if (label == ignore_index) {
    if (threadIdx.x == 0) {
      loss[row] = 0.f;
      lse_out[row] = 0.f;
    }
    return;
  }
  const T* xr = logits + row * ld;
  float m = -INFINITY, s = 0.f, sz = 0.f;
  // whole chunks of kThreads * kUnroll vectors (ts_plan::chunk_vec), then the rest
  const int64_t full = nvec / ((int64_t)kThreads * kUnroll);
  int64_t c = 0;
  for (; c < full; ++c) {
    u32x4 buf[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      buf[u] = ld16_stream(xr + ts_plan::chunk_vec(c, u, threadIdx.x, kThreads, kUnroll) * VE);
    float z[kUnroll][VE];
    float lm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      Elt<T>::unpack(buf[u], z[u]);
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        z[u][i] = xform<kXform>(z[u][i], xf);
        lm = fmaxf(lm, z[u][i]);
        if constexpr (kSmooth) sz += z[u][i];
      }
    }
    if (lm > m) {
      s = s == 0.f ? 0.f : s * fast_exp2((m - lm) * kLog2e);
      m = lm;
    }
    // m is -inf only while every value seen is -inf: their terms are 0.
    const float mb = m == -INFINITY ? 0.f : m * kLog2e;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int i = 0; i < VE; ++i) s += fast_exp2(__builtin_fmaf(z[u][i], kLog2e, -mb));
  }
  // Tail: fewer than kThreads*kUnroll vectors remain.
  for (int64_t v = ts_plan::chunk_vec(c, 0, threadIdx.x, kThreads, kUnroll); v < nvec;
       v += kThreads) {  // chunk_vec(c, u, ...) for u = 0, 1, ...
    float z[VE];
    Elt<T>::unpack(ld16_stream(xr + v * VE), z);
    float lm = -INFINITY;
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      z[i] = xform<kXform>(z[i], xf);
      lm = fmaxf(lm, z[i]);
      if constexpr (kSmooth) sz += z[i];
    }
    if (lm > m) {
      s = s == 0.f ? 0.f : s * fast_exp2((m - lm) * kLog2e);
      m = lm;
    }
    // m is -inf only while every value seen is -inf: their terms are 0.
    const float mb = m == -INFINITY ? 0.f : m * kLog2e;
#pragma unroll
    for (int i = 0; i < VE; ++i) s += fast_exp2(__builtin_fmaf(z[i], kLog2e, -mb));
  }
  block_fold(m, s, sz, lds);
  if (threadIdx.x == 0) {
    const float l = m + logf(s);
    float out;
    const int64_t col = ts_plan::label_col(label, V, ignore_index);  // not ignored here
    if (col < 0) {
      out = __builtin_nanf("");
    } else {
      const float zt = xform<kXform>(Elt<T>::load1(xr + col), xf);
      out = l - zt;
      if constexpr (kSmooth) out = (1.f - smoothing) * out + smoothing * (l - sz / (float)V);
    }
    loss[row] = out;
    lse_out[row] = l;
  }
}

// Element-wise forward for rows that are not 16-byte aligned / divisible.
template <typename T, bool kXform, bool kSmooth>
__global__ __launch_bounds__(kThreads) void ce_fwd_generic(
    const T* __restrict__ logits, int64_t ld, const int64_t* __restrict__ labels, int64_t V,
    int64_t ignore_index, Xform xf, float smoothing, float* __restrict__ loss,
    float* __restrict__ lse_out) {
  __shared__ float lds[2 * kWaves];
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  if (label == ignore_index) {
    if (threadIdx.x == 0) {
      loss[row] = 0.f;
      lse_out[row] = 0.f;
    }
    return;
  }
  const T* xr = logits + row * ld;
  float m = -INFINITY, s = 0.f, sz = 0.f;
  for (int64_t j = threadIdx.x; j < V; j += kThreads) {
    const float z = xform<kXform>(Elt<T>::load1(xr + j), xf);
    if constexpr (kSmooth) sz += z;
    if (z > m) {
      s = s == 0.f ? 0.f : s * fast_exp2((m - z) * kLog2e);
      m = z;
    }
    s += z == -INFINITY ? 0.f : fast_exp2((z - m) * kLog2e);
  }
  block_fold(m, s, sz, lds);
  if (threadIdx.x == 0) {
    const float l = m + logf(s);
    float out;
    const int64_t col = ts_plan::label_col(label, V, ignore_index);  // not ignored here
    if (col < 0) {
      out = __builtin_nanf("");
    } else {
      const float zt = xform<kXform>(Elt<T>::load1(xr + col), xf);
      out = l - zt;
      if constexpr (kSmooth) out = (1.f - smoothing) * out + smoothing * (l - sz / (float)V);
    }
    loss[row] = out;
    lse_out[row] = l;
  }
}

struct BwdRow {
  float dl;     // upstream gradient of this row
  float lse2;   // lse * log2(e)
  int64_t label;
};

// Gradient of one element given its raw logit x at column j.
template <bool kXform, bool kSmooth>
__device__ inline float ce_grad(float x, int64_t j, const BwdRow& r, const Xform& xf,
                                float smoothing, float inv_v) {
  float z = x, t = 0.f;
  if constexpr (kXform) {
    if (xf.scale != 0.f) z = xf.scale * z;
    if (xf.softcap != 0.f) {
      t = tanhf(z / xf.softcap);
      z = xf.softcap * t;
    }
  }
  const float p = fast_exp2(__builtin_fmaf(z, kLog2e, -r.lse2));
  float g;
  if constexpr (kSmooth) {
    g = (1.f - smoothing) * (j == r.label ? p - 1.f : p) + smoothing * (p - inv_v);
  } else {
    g = j == r.label ? p - 1.f : p;
  }
  if constexpr (kXform) {
    if (xf.softcap != 0.f) g = g * (1.f - t * t);
    if (xf.scale != 0.f) g = g * xf.scale;
  }
  return r.dl * g;
}

// Stores one vector of VE gradients (as one or two 16-byte stores).
template <typename G, int VE>
__device__ inline void store_grad(G* p, const float* g) {
  if constexpr (sizeof(G) == 4 && VE == 8) {
    st16_stream(p, Elt<float>::pack(g));
    st16_stream(p + 4, Elt<float>::pack(g + 4));
  } else {
    st16_stream(p, Elt<G>::pack(g));
  }
}

// One-shot grid: blockIdx.y is the row (offset by row0), blockIdx.x a chunk
// of kThreads * kBwdKv vectors of it; each thread handles kBwdKv vectors.
template <typename T, typename G, bool kXform, bool kSmooth>
__global__ __launch_bounds__(kThreads) void ce_bwd_vec(
    const T* logits, int64_t ld, const int64_t* __restrict__ labels,
    const float* __restrict__ lse, const float* __restrict__ dloss, int64_t dloss_stride,
    float dloss_scale, G* grad, int64_t ld_grad, int64_t V, int64_t nvec, int64_t ignore_index,
    Xform xf, float smoothing, int64_t row0) {
  constexpr int VE = Elt<T>::kVec;
  static_assert(Elt<G>::kVec == VE || sizeof(G) == 4, "grad vector width");
  const int64_t row = row0 + blockIdx.y;
  const int64_t label = labels[row];
  G* gr = grad + row * ld_grad;
  int64_t vk[kBwdKv];  // this thread's vectors of the row (ts_plan::chunk_vec)
#pragma unroll
  for (int k = 0; k < kBwdKv; ++k)
    vk[k] = ts_plan::chunk_vec(blockIdx.x, k, threadIdx.x, kThreads, kBwdKv);
  if (label == ignore_index) {
    const float zero[VE] = {};
#pragma unroll
    for (int k = 0; k < kBwdKv; ++k) {
      if (vk[k] < nvec) store_grad<G, VE>(gr + vk[k] * VE, zero);
    }
    return;
  }
  BwdRow r;
  r.dl = dloss[row * dloss_stride] * dloss_scale;
  r.lse2 = lse[row] * kLog2e;
  r.label = label;
  const float inv_v = 1.f / (float)V;
  const T* xr = logits + row * ld;
  u32x4 buf[kBwdKv];
#pragma unroll
  for (int k = 0; k < kBwdKv; ++k) {
    const int64_t v = vk[k];
    buf[k] = v < nvec ? ld16_stream(xr + v * VE) : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int k = 0; k < kBwdKv; ++k) {
    const int64_t v = vk[k];
    if (v < nvec) {
      float x[VE], g[VE];
      Elt<T>::unpack(buf[k], x);
#pragma unroll
      for (int i = 0; i < VE; ++i)
        g[i] = ce_grad<kXform, kSmooth>(x[i], v * VE + i, r, xf, smoothing, inv_v);
      store_grad<G, VE>(gr + v * VE, g);
    }
  }
}

template <typename T, typename G, bool kXform, bool kSmooth>
__global__ __launch_bounds__(kThreads) void ce_bwd_generic(
    const T* logits, int64_t ld, const int64_t* __restrict__ labels,
    const float* __restrict__ lse, const float* __restrict__ dloss, int64_t dloss_stride,
    float dloss_scale, G* grad, int64_t ld_grad, int64_t V, int64_t ignore_index, Xform xf,
    float smoothing) {
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  G* gr = grad + row * ld_grad;
  if (label == ignore_index) {
    for (int64_t j = threadIdx.x; j < V; j += kThreads) Elt<G>::store1(gr + j, 0.f);
    return;
  }
  BwdRow r;
  r.dl = dloss[row * dloss_stride] * dloss_scale;
  r.lse2 = lse[row] * kLog2e;
  r.label = label;
  const float inv_v = 1.f / (float)V;
  const T* xr = logits + row * ld;
  for (int64_t j = threadIdx.x; j < V; j += kThreads) {
    const float x = Elt<T>::load1(xr + j);
    Elt<G>::store1(gr + j, ce_grad<kXform, kSmooth>(x, j, r, xf, smoothing, inv_v));
  }
}

// ---------------------------------------------------------------------------
// Forward + backward in one pass ("schedule B"): one row per 1024-thread
// workgroup, held in registers (kFusedKv 16-byte vectors per thread, so
// V <= 1024 * kFusedKv * vector width). Each thread folds its vectors into an
// online (max, sum of exp) pair as they arrive; one LDS exchange of the 16
// wave pairs gives the lse (a single barrier). The gradient is then written
// from the same registers: each valid row is read once and every row written
// once. Ignored rows are written as zeros without being read.
//
// The row is addressed through buffer resources (base and range in SGPRs,
// one VGPR of offset per lane), which keeps the 64 data VGPRs plus the
// working set inside the 128-VGPR budget of a 1024-thread workgroup. Without
// label smoothing or logit transforms an element's gradient is
// exp2(z*log2e - (lse*log2e - log2|dl|)) with the sign of dl applied to the
// packed result, one FMA and one exp per element; the label element is
// corrected by the one lane that holds it.
// ---------------------------------------------------------------------------
constexpr int kFusedThreads = 1024;
constexpr int kFusedWaves = kFusedThreads / kWave;
constexpr int kFusedKv = 16;

// Byte offset of this thread's k-th vector, past the row end one no row resource
// covers (ts_plan::vec_boffset: the hardware drops such stores, loads read 0).
__device__ inline int fused_voff(int k, int nvec, int vec_bytes) {
  return ts_plan::vec_boffset(ts_plan::chunk_vec(0, k, threadIdx.x, kFusedThreads, kFusedKv),
                              nvec, vec_bytes);
}

// Row lse (and, with kSmooth, the row sum of z) from every thread's online
// (max, sum of exp) pair. lds holds 3 * kFusedWaves floats. One barrier: the
// caller must not write lds again without another barrier in between.
template <bool kSmooth>
__device__ inline float fused_lse(float m, float s, float& sz, float* lds) {
  const float wm = wave_max(m);
  const float ws = wave_sum(s == 0.f ? 0.f : s * fast_exp2((m - wm) * kLog2e));
  const int wid = threadIdx.x / kWave;
  if constexpr (kSmooth) sz = wave_sum(sz);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    lds[wid] = wm;
    lds[kFusedWaves + wid] = ws;
    if constexpr (kSmooth) lds[2 * kFusedWaves + wid] = sz;
  }
  __syncthreads();
  float gm = lds[0];
#pragma unroll
  for (int i = 1; i < kFusedWaves; ++i) gm = fmaxf(gm, lds[i]);
  float gs = 0.f, gz = 0.f;
#pragma unroll
  for (int i = 0; i < kFusedWaves; ++i) {
    const float si = lds[kFusedWaves + i];
    gs += si == 0.f ? 0.f : si * fast_exp2((lds[i] - gm) * kLog2e);
    if constexpr (kSmooth) gz += lds[2 * kFusedWaves + i];
  }
  if constexpr (kSmooth) sz = gz;
  return gm + logf(gs);
}

template <typename G>
constexpr uint32_t sign_bits() {
  return sizeof(G) == 4 ? 0x80000000u : 0x80008000u;
}

template <typename T, typename G, bool kXform, bool kSmooth>
__global__ __launch_bounds__(kFusedThreads) void ce_fused_vec(
    const T* __restrict__ logits, int64_t ld, const int64_t* __restrict__ labels, int64_t V,
    int nvec, int64_t ignore_index, Xform xf, float smoothing, const float* __restrict__ dloss,
    int64_t dloss_stride, float dloss_scale, float* __restrict__ loss, float* __restrict__ lse_out,
    G* __restrict__ grad, int64_t ld_grad) {
  constexpr int VE = Elt<T>::kVec;
  constexpr int kGradBytes = VE * (int)sizeof(G);  // grad bytes per logits vector
  __shared__ float lds[3 * kFusedWaves];
  const int64_t row = blockIdx.x;
  const int64_t label = labels[row];
  const Rsrc go = buf_rsrc(grad + row * ld_grad, (uint32_t)nvec * kGradBytes);
  if (label == ignore_index) {
    const u32x4 zero = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < kFusedKv; ++k) {
      const int off = fused_voff(k, nvec, kGradBytes);
      buf_st16_stream(zero, go, off);
      if constexpr (kGradBytes == 32) buf_st16_stream(zero, go, off + 16);
    }
    if (threadIdx.x == 0) {
      loss[row] = 0.f;
      lse_out[row] = 0.f;
    }
    return;
  }
  const T* xr = logits + row * ld;
  const Rsrc xi = buf_rsrc(xr, (uint32_t)nvec * 16u);
  u32x4 buf[kFusedKv];
#pragma unroll
  for (int k = 0; k < kFusedKv; ++k) buf[k] = buf_ld16_stream(xi, fused_voff(k, nvec, 16));
  // Each lane sums exp(z - m) over its vectors against one reference m, the
  // largest value of its first vector (0 if that vector is all -inf): per
  // element one unpack, one FMA, one exp and one add, with no running max or
  // rescale. The sum is exact (terms that underflow lie below the resolution
  // of a sum that holds exp(0) = 1) unless it ends outside [0.5, inf): a
  // value more than 88 above m overflowed it, a NaN reached it, or an all
  // -inf first vector left a sum of values far below 0. Such a lane (only
  // with extreme logits) folds its vectors again from the registers with an
  // exact online max and rescale. Lanes without vectors keep m = -inf, s = 0.
  float m = -INFINITY, mb = 0.f, s = 0.f, sz = 0.f;
  auto sum_exp = [&](const float (&z)[VE], float bias) {
    float cs = fast_exp2(__builtin_fmaf(z[0], kLog2e, -bias));
#pragma unroll
    for (int i = 1; i < VE; ++i) cs += fast_exp2(__builtin_fmaf(z[i], kLog2e, -bias));
    return cs;
  };
  auto values = [&](const u32x4& q, float (&z)[VE]) {
    Elt<T>::unpack(q, z);
#pragma unroll
    for (int i = 0; i < VE; ++i) z[i] = xform<kXform>(z[i], xf);
  };
  auto vmax = [&](const float (&z)[VE]) {
    float cm = z[0];
#pragma unroll
    for (int i = 1; i < VE; ++i) cm = __builtin_fmaxf(cm, z[i]);
    return cm;
  };
  auto fold = [&](const u32x4& q, bool first) {
    float z[VE];
    values(q, z);
    if constexpr (kSmooth) {
#pragma unroll
      for (int i = 0; i < VE; ++i) sz += z[i];
    }
    if (first) {
      const float cm = vmax(z);
      m = cm == -INFINITY ? 0.f : cm;
      mb = m * kLog2e;
    }
    s += sum_exp(z, mb);
  };
#pragma unroll
  for (int k = 0; k < kFusedKv; ++k) {
    // Vectors every thread holds take a uniform branch; only the row's last
    // partial sweep tests each lane.
    if ((k + 1) * kFusedThreads <= nvec) fold(buf[k], k == 0);
    else if (threadIdx.x + k * kFusedThreads < nvec) fold(buf[k], k == 0);
  }
  if ((int)threadIdx.x < nvec && !(s >= 0.5f && s < INFINITY)) {
    m = -INFINITY;
    s = 0.f;
#pragma unroll
    for (int k = 0; k < kFusedKv; ++k) {
      if ((int)threadIdx.x + k * kFusedThreads < nvec) {
        float z[VE];
        values(buf[k], z);
        const float mn = __builtin_fmaxf(m, vmax(z));
        if (mn != -INFINITY) {
          s = (s == 0.f ? 0.f : s * fast_exp2((m - mn) * kLog2e)) + sum_exp(z, mn * kLog2e);
          m = mn;
        }
      }
    }
  }
  const float l = fused_lse<kSmooth>(m, s, sz, lds);
  // The gradient pass re-unpacks the stored vectors; this keeps the compiler
  // from carrying the first pass's unpacked floats (twice the registers).
#pragma unroll
  for (int k = 0; k < kFusedKv; ++k) asm volatile("" : "+v"(buf[k]));
  if (threadIdx.x == 0) {
    float out;
    const int64_t col = ts_plan::label_col(label, V, ignore_index);  // not ignored here
    if (col < 0) {
      out = __builtin_nanf("");
    } else {
      const float zt = xform<kXform>(Elt<T>::load1(xr + col), xf);
      out = l - zt;
      if constexpr (kSmooth) out = (1.f - smoothing) * out + smoothing * (l - sz / (float)V);
    }
    loss[row] = out;
    lse_out[row] = l;
  }
  // One upstream gradient per row, moved to a scalar register: its sign below
  // is then a wave-uniform mask (one XOR per packed dword, no per-lane select).
  const float dl = __builtin_bit_cast(
      float, __builtin_amdgcn_readfirstlane(
                 __builtin_bit_cast(int, dloss[row * dloss_stride] * dloss_scale)));
  if constexpr (!kXform && !kSmooth) {
    const float adl = fabsf(dl);
    const float l2 = l * kLog2e;
    const float l2d = l2 - __builtin_amdgcn_logf(adl);  // v_log_f32 is log2
    // The position of the label is uniform over the workgroup: its
    // correction is a uniform branch, and only the lane holding the label
    // runs it.
    const uint32_t smask = (__builtin_bit_cast(uint32_t, dl) >> 31) != 0 ? sign_bits<G>() : 0u;
    const int64_t lv = label >= 0 && label < V ? label / VE : -1;  // vector holding the label
    const int klab = lv < 0 ? -1 : (int)(lv / kFusedThreads);
    const int tlab = lv < 0 ? -1 : (int)(lv % kFusedThreads);
    const int elab = lv < 0 ? 0 : (int)(label % VE);
#pragma unroll
    for (int k = 0; k < kFusedKv; ++k) {
      float z[VE], g[VE];
      Elt<T>::unpack(buf[k], z);
#pragma unroll
      for (int i = 0; i < VE; ++i) g[i] = fast_exp2(__builtin_fmaf(z[i], kLog2e, -l2d));
      if (k == klab && (int)threadIdx.x == tlab) {
#pragma unroll
        for (int i = 0; i < VE; ++i)
          if (i == elab) g[i] = adl * (fast_exp2(__builtin_fmaf(z[i], kLog2e, -l2)) - 1.f);
      }
      const int off = fused_voff(k, nvec, kGradBytes);
      if constexpr (kGradBytes == 32) {
        u32x4 p0 = Elt<float>::pack(g), p1 = Elt<float>::pack(g + 4);
        p0 ^= smask;
        p1 ^= smask;
        buf_st16_stream(p0, go, off);
        buf_st16_stream(p1, go, off + 16);
      } else {
        u32x4 p = Elt<G>::pack(g);
        p ^= smask;
        buf_st16_stream(p, go, off);
      }
    }
  } else {
    BwdRow r;
    r.dl = dl;
    r.lse2 = l * kLog2e;
    r.label = label;
    const float inv_v = 1.f / (float)V;
#pragma unroll
    for (int k = 0; k < kFusedKv; ++k) {
      float x[VE], g[VE];
      Elt<T>::unpack(buf[k], x);
      const int64_t j0 = (int64_t)(threadIdx.x + k * kFusedThreads) * VE;
#pragma unroll
      for (int i = 0; i < VE; ++i)
        g[i] = ce_grad<kXform, kSmooth>(x[i], j0 + i, r, xf, smoothing, inv_v);
      const int off = fused_voff(k, nvec, kGradBytes);
      if constexpr (kGradBytes == 32) {
        buf_st16_stream(Elt<float>::pack(g), go, off);
        buf_st16_stream(Elt<float>::pack(g + 4), go, off + 16);
      } else {
        buf_st16_stream(Elt<G>::pack(g), go, off);
      }
    }
  }
}

// Schedule B when the row fits the registers of one workgroup and 16-byte
// access is possible; returns false (nothing launched) otherwise.
template <typename T, typename G>
bool fused_typed(const void* logits, int64_t ld, const int64_t* labels, int64_t N, int64_t V,
                 int64_t ignore_index, Xform xf, float smoothing, const float* dloss,
                 int64_t dloss_stride, float dloss_scale, float* loss, float* lse, void* grad,
                 int64_t ld_grad, hipStream_t st, ts_status* status) {
  constexpr int VE = sizeof(T) == 4 ? 4 : 8;
  const bool grad_ok = sizeof(G) == sizeof(T) || (sizeof(G) == 4 && VE == 8);
  const int64_t nvec = V / VE;
  if (!(V % VE == 0 && ld % VE == 0 && ld_grad % VE == 0 && ts_host::aligned16(logits) &&
        ts_host::aligned16(grad) && grad_ok && nvec <= (int64_t)kFusedThreads * kFusedKv &&
        N <= INT32_MAX))
    return false;
  const T* lp = static_cast<const T*>(logits);
  G* gp = static_cast<G*>(grad);
  const bool xform_on = xf.scale != 0.f || xf.softcap != 0.f;
  const bool smooth = smoothing != 0.f;
#define TS_CE_FUSED(X, S)                                                                        \
  if (xform_on == X && smooth == S) {                                                            \
    hipLaunchKernelGGL((ce_fused_vec<T, G, X, S>), dim3((unsigned)N), dim3(kFusedThreads), 0, st, \
                       lp, ld, labels, V, (int)nvec, ignore_index, xf, smoothing, dloss,        \
                       dloss_stride, dloss_scale, loss, lse, gp, ld_grad);                      \
    *status = ts_host::check_launch("ce_fused_vec");                                             \
    return true;                                                                                 \
  }
  TS_CE_FUSED(false, false)
  TS_CE_FUSED(false, true)
  TS_CE_FUSED(true, false)
  TS_CE_FUSED(true, true)
#undef TS_CE_FUSED
  return false;
}

template <typename T>
ts_status fwd_typed(const void* logits, int64_t ld, const int64_t* labels, int64_t N, int64_t V,
                    int64_t ignore_index, Xform xf, float smoothing, float* loss, float* lse,
                    hipStream_t st) {
  constexpr int VE = sizeof(T) == 4 ? 4 : 8;
  const T* lp = static_cast<const T*>(logits);
  const bool vec = V % VE == 0 && ld % VE == 0 && ts_host::aligned16(logits);
  const bool xform_on = xf.scale != 0.f || xf.softcap != 0.f;
  const bool smooth = smoothing != 0.f;
  const dim3 grid((unsigned)N), block(kThreads);
#define TS_CE_FWD(X, S)                                                                       \
  if (xform_on == X && smooth == S) {                                                         \
    if (vec) {                                                                                \
      hipLaunchKernelGGL((ce_fwd_vec<T, X, S>), grid, block, 0, st, lp, ld, labels, V,        \
                         V / VE, ignore_index, xf, smoothing, loss, lse);                     \
      return ts_host::check_launch("ce_fwd_vec");                                             \
    }                                                                                         \
    hipLaunchKernelGGL((ce_fwd_generic<T, X, S>), grid, block, 0, st, lp, ld, labels, V,      \
                       ignore_index, xf, smoothing, loss, lse);                               \
    return ts_host::check_launch("ce_fwd_generic");                                           \
  }
  TS_CE_FWD(false, false)
  TS_CE_FWD(false, true)
  TS_CE_FWD(true, false)
  TS_CE_FWD(true, true)
#undef TS_CE_FWD
  return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "ce_fwd: unreachable");
}

template <typename T, typename G>
ts_status bwd_typed(const void* logits, int64_t ld, const int64_t* labels, const float* lse,
                    const float* dloss, int64_t dloss_stride, float dloss_scale, void* grad,
                    int64_t ld_grad, int64_t N, int64_t V, int64_t ignore_index, Xform xf,
                    float smoothing, hipStream_t st) {
  constexpr int VE = sizeof(T) == 4 ? 4 : 8;
  const T* lp = static_cast<const T*>(logits);
  G* gp = static_cast<G*>(grad);
  // The vector path needs the grad rows to take the same vector width.
  const bool grad_ok = sizeof(G) == sizeof(T) || (sizeof(G) == 4 && VE == 8);
  const bool vec = V % VE == 0 && ld % VE == 0 && ld_grad % VE == 0 &&
                   ts_host::aligned16(logits) && ts_host::aligned16(grad) && grad_ok;
  const bool xform_on = xf.scale != 0.f || xf.softcap != 0.f;
  const bool smooth = smoothing != 0.f;
  const dim3 grid((unsigned)N), block(kThreads);
#define TS_CE_BWD(X, S)                                                                        \
  if (xform_on == X && smooth == S) {                                                          \
    if (vec) {                                                                                 \
      const int64_t nvec = V / VE;                                                             \
      const unsigned gx = (unsigned)ts_plan::chunks_for(nvec, kThreads, kBwdKv);    \
      for (int64_t r0 = 0; r0 < N; r0 += kMaxGridY) {                                          \
        const unsigned gy = (unsigned)(N - r0 < kMaxGridY ? N - r0 : kMaxGridY);               \
        hipLaunchKernelGGL((ce_bwd_vec<T, G, X, S>), dim3(gx, gy), block, 0, st, lp, ld,       \
                           labels, lse, dloss, dloss_stride, dloss_scale, gp, ld_grad, V,      \
                           nvec, ignore_index, xf, smoothing, r0);                             \
        ts_status s_ = ts_host::check_launch("ce_bwd_vec");                                    \
        if (s_ != TS_OK) return s_;                                                            \
      }                                                                                        \
      return TS_OK;                                                                            \
    }                                                                                          \
    hipLaunchKernelGGL((ce_bwd_generic<T, G, X, S>), grid, block, 0, st, lp, ld, labels, lse,  \
                       dloss, dloss_stride, dloss_scale, gp, ld_grad, V, ignore_index, xf,     \
                       smoothing);                                                             \
    return ts_host::check_launch("ce_bwd_generic");                                            \
  }
  TS_CE_BWD(false, false)
  TS_CE_BWD(false, true)
  TS_CE_BWD(true, false)
  TS_CE_BWD(true, true)
#undef TS_CE_BWD
  return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "ce_bwd: unreachable");
}

ts_status check_ce(const void* logits, int64_t ld, ts_dtype dtype, const int64_t* labels,
                   int64_t N, int64_t V, float logit_scale, float softcap,
                   float label_smoothing) {
  using ts_host::fail;
  if (!ts_host::valid_dtype(dtype)) return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce: bad dtype");
  if (N < 0 || V <= 0) return fail(TS_ERR_SHAPE, "ce: bad shape N=%lld V=%lld", (long long)N,
                                   (long long)V);
  if (N > 0x7fffffffLL) return fail(TS_ERR_SHAPE, "ce: too many rows (%lld)", (long long)N);
  if (ld < V) return fail(TS_ERR_SHAPE, "ce: row stride %lld < V %lld", (long long)ld,
                          (long long)V);
  if (N > 0 && (logits == nullptr || labels == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce: logits or labels is NULL");
  if (!(label_smoothing >= 0.f && label_smoothing < 1.f))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce: label_smoothing must be in [0, 1)");
  if (!isfinite(logit_scale) || !isfinite(softcap) || softcap < 0.f)
    return fail(TS_ERR_INVALID_ARGUMENT, "ce: bad logit_scale/softcap");
  return TS_OK;
}

}  // namespace

extern "C" ts_status ts_ce_fwd(const void* logits, int64_t ld, ts_dtype dtype,
                               const int64_t* labels, int64_t N, int64_t V,
                               int64_t ignore_index, float logit_scale, float softcap,
                               float label_smoothing, float* loss, float* lse,
                               ts_stream_t stream) {
  ts_status s = check_ce(logits, ld, dtype, labels, N, V, logit_scale, softcap, label_smoothing);
  if (s != TS_OK) return s;
  if (N > 0 && (loss == nullptr || lse == nullptr))
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "ce_fwd: loss or lse is NULL");
  if (N == 0) return TS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Xform xf{logit_scale, softcap};
  switch (dtype) {
    case TS_BF16:
      return fwd_typed<__bf16>(logits, ld, labels, N, V, ignore_index, xf, label_smoothing, loss,
                               lse, st);
    case TS_F16:
      return fwd_typed<_Float16>(logits, ld, labels, N, V, ignore_index, xf, label_smoothing,
                                 loss, lse, st);
    case TS_F32:
      return fwd_typed<float>(logits, ld, labels, N, V, ignore_index, xf, label_smoothing, loss,
                              lse, st);
  }
  return ts_host::fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_fwd: bad dtype");
}

extern "C" ts_status ts_ce_bwd(const void* logits, int64_t ld, ts_dtype dtype,
                               const int64_t* labels, const float* lse, const float* dloss,
                               int64_t dloss_stride, float dloss_scale, void* grad,
                               int64_t ld_grad, ts_dtype grad_dtype, int64_t N, int64_t V,
                               int64_t ignore_index, float logit_scale, float softcap,
                               float label_smoothing, ts_stream_t stream) {
  using ts_host::fail;
  ts_status s = check_ce(logits, ld, dtype, labels, N, V, logit_scale, softcap, label_smoothing);
  if (s != TS_OK) return s;
  if (!ts_host::valid_dtype(grad_dtype))
    return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_bwd: bad grad dtype");
  if (grad_dtype != dtype && grad_dtype != TS_F32)
    return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_bwd: grad dtype must equal logits dtype or be f32");
  if (N > 0 && (lse == nullptr || dloss == nullptr || grad == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_bwd: lse, dloss or grad is NULL");
  if (ld_grad < V) return fail(TS_ERR_SHAPE, "ce_bwd: grad row stride < V");
  if (dloss_stride < 0) return fail(TS_ERR_SHAPE, "ce_bwd: negative dloss stride");
  if (grad == logits && (ld_grad != ld || grad_dtype != dtype))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_bwd: in-place grad needs the logits layout");
  if (N == 0) return TS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Xform xf{logit_scale, softcap};
#define TS_CE_BWD_T(T)                                                                         \
  return grad_dtype == TS_F32 && dtype != TS_F32                                               \
             ? bwd_typed<T, float>(logits, ld, labels, lse, dloss, dloss_stride, dloss_scale,  \
                                   grad, ld_grad, N, V, ignore_index, xf, label_smoothing, st) \
             : bwd_typed<T, T>(logits, ld, labels, lse, dloss, dloss_stride, dloss_scale,      \
                               grad, ld_grad, N, V, ignore_index, xf, label_smoothing, st);
  switch (dtype) {
    case TS_BF16: TS_CE_BWD_T(__bf16)
    case TS_F16: TS_CE_BWD_T(_Float16)
    case TS_F32: TS_CE_BWD_T(float)
  }
#undef TS_CE_BWD_T
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_bwd: bad dtype");
}

extern "C" ts_status ts_ce_fwd_bwd(const void* logits, int64_t ld, ts_dtype dtype,
                                   const int64_t* labels, int64_t N, int64_t V,
                                   int64_t ignore_index, float logit_scale, float softcap,
                                   float label_smoothing, const float* dloss,
                                   int64_t dloss_stride, float dloss_scale, float* loss,
                                   float* lse, void* grad, int64_t ld_grad, ts_dtype grad_dtype,
                                   ts_stream_t stream) {
  using ts_host::fail;
  ts_status s = check_ce(logits, ld, dtype, labels, N, V, logit_scale, softcap, label_smoothing);
  if (s != TS_OK) return s;
  if (!ts_host::valid_dtype(grad_dtype))
    return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_fwd_bwd: bad grad dtype");
  if (grad_dtype != dtype && grad_dtype != TS_F32)
    return fail(TS_ERR_UNSUPPORTED_DTYPE,
                "ce_fwd_bwd: grad dtype must equal logits dtype or be f32");
  if (N > 0 && (loss == nullptr || lse == nullptr || dloss == nullptr || grad == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_fwd_bwd: loss, lse, dloss or grad is NULL");
  if (ld_grad < V) return fail(TS_ERR_SHAPE, "ce_fwd_bwd: grad row stride < V");
  if (dloss_stride < 0) return fail(TS_ERR_SHAPE, "ce_fwd_bwd: negative dloss stride");
  if (grad == logits)
    return fail(TS_ERR_INVALID_ARGUMENT,
                "ce_fwd_bwd: grad must not alias the logits (use ts_ce_fwd + ts_ce_bwd)");
  if (N == 0) return TS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Xform xf{logit_scale, softcap};
  bool done = false;
#define TS_CE_FB_T(T)                                                                           \
  done = grad_dtype == TS_F32 && dtype != TS_F32                                                \
             ? fused_typed<T, float>(logits, ld, labels, N, V, ignore_index, xf,                \
                                     label_smoothing, dloss, dloss_stride, dloss_scale, loss,   \
                                     lse, grad, ld_grad, st, &s)                                \
             : fused_typed<T, T>(logits, ld, labels, N, V, ignore_index, xf, label_smoothing,   \
                                 dloss, dloss_stride, dloss_scale, loss, lse, grad, ld_grad,    \
                                 st, &s);
  switch (dtype) {
    case TS_BF16: TS_CE_FB_T(__bf16) break;
    case TS_F16: TS_CE_FB_T(_Float16) break;
    case TS_F32: TS_CE_FB_T(float) break;
  }
#undef TS_CE_FB_T
  if (done) return s;
  // Rows too long for one workgroup's registers (or no 16-byte access): the
  // two-pass schedule, forward then backward.
  s = ts_ce_fwd(logits, ld, dtype, labels, N, V, ignore_index, logit_scale, softcap,
                label_smoothing, loss, lse, stream);
  if (s != TS_OK) return s;
  return ts_ce_bwd(logits, ld, dtype, labels, lse, dloss, dloss_stride, dloss_scale, grad,
                   ld_grad, grad_dtype, N, V, ignore_index, logit_scale, softcap,
                   label_smoothing, stream);
}
