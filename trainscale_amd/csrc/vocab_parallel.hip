// Vocabulary-parallel cross entropy: the kernels one rank runs (gfx950).
//
// The reference (distributed/tensor_parallel.py:1479-1666, the all-reduces at
// :1527, :1545 and :1573) splits the
// vocabulary over the tensor-parallel ranks and makes three all-reduces per
// step: the row max, the sum of exp and the target logit. Here a rank reads
// its shard once and emits one 16-byte partial per row,
//   { lse over the shard, the target's logit if the target lies in the shard
//     (else 0), the sum of the shard's logits (label smoothing), 0 },
// so one all-gather of [N, 4] floats replaces the three all-reduces, and every
// rank merges the P partials itself: lse = log sum_p exp(lse_p), target logit
// = sum_p target_p (one rank holds it). The backward reads the shard again
// and writes its gradient.
//
// Stats: one row per workgroup, held in registers (kKv 16-byte vectors per
// thread). Each lane sums exp(z - m) against one reference, the largest value
// of its first vector, and folds again with an exact online max only when the
// sum ends outside [0.5, inf) (extreme logits); then wave and workgroup
// combine the lanes' (m, s) pairs. Merge: one thread per row, one online
// pass over the P partials. Backward: one-shot grid over (row, chunk of 256
// vectors), one vector per thread.
#include <math.h>

#include "common.hpp"
#include "plan.hpp"

namespace {

using namespace ts;

constexpr int kBwdThreads = 256;
constexpr int kBwdKv = 1;  // 164 us against 182 us with 2 at [16384, 16032] bf16 (MI355X)
constexpr int kGenThreads = 256;
constexpr int64_t kMaxGridY = 65535;

struct Stats {
  float lse, target, sum_z, pad;
};

// Combines the lanes' (m, s, sum_z) into the row's lse and sum_z; every
// thread receives them. `lds` holds 3 * kWaves floats. One barrier.
template <int kWaves>
__device__ inline void block_lse(float m, float s, float sz, float* lds, float& lse,
                                 float& sz_out) {
  const float wm = wave_max(m);
  const float ws = wave_sum(s == 0.f ? 0.f : s * fast_exp2((m - wm) * kLog2e));
  const float wz = wave_sum(sz);
  const int wid = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    lds[wid] = wm;
    lds[kWaves + wid] = ws;
    lds[2 * kWaves + wid] = wz;
  }
  __syncthreads();
  float gm = lds[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) gm = fmaxf(gm, lds[i]);
  float gs = 0.f, gz = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const float si = lds[kWaves + i];
    gs += si == 0.f ? 0.f : si * fast_exp2((lds[i] - gm) * kLog2e);
    gz += lds[2 * kWaves + i];
  }
  lse = gm + logf(gs);  // -inf when every value is -inf
  sz_out = gz;
}

// Row statistics of a shard held in registers: kBlock threads x kKv vectors.
template <typename T, int kBlock, int kKv>
__global__ __launch_bounds__(kBlock) void shard_stats_vec(const T* __restrict__ logits,
                                                          int64_t ld,
                                                          const int64_t* __restrict__ targets,
                                                          int64_t Vp, int nvec,
                                                          int64_t vocab_start,
                                                          Stats* __restrict__ stats) {
  constexpr int VE = Elt<T>::kVec;
  constexpr int kWaves = kBlock / kWave;
  __shared__ float lds[3 * kWaves];
  const int64_t row = blockIdx.x;
  const T* xr = logits + row * ld;
  const Rsrc xi = buf_rsrc(xr, (uint32_t)nvec * 16u);
  u32x4 buf[kKv];
#pragma unroll
  for (int k = 0; k < kKv; ++k)  // past the row: an offset the resource does not cover
    buf[k] = buf_ld16_stream(
        xi, ts_plan::vec_boffset(ts_plan::chunk_vec(0, k, threadIdx.x, kBlock, kKv), nvec, 16));
  const int64_t tl = ts_plan::shard_col(targets[row], vocab_start, Vp);
  float zt = 0.f;
  if (threadIdx.x == 0 && tl >= 0) zt = Elt<T>::load1(xr + tl);

  float m = -INFINITY, mb = 0.f, s = 0.f, sz = 0.f;
  auto sum_exp = [&](const float (&z)[VE], float bias) {
    float cs = fast_exp2(__builtin_fmaf(z[0], kLog2e, -bias));
#pragma unroll
    for (int i = 1; i < VE; ++i) cs += fast_exp2(__builtin_fmaf(z[i], kLog2e, -bias));
    return cs;
  };
  auto vmax = [&](const float (&z)[VE]) {
    float cm = z[0];
#pragma unroll
    for (int i = 1; i < VE; ++i) cm = __builtin_fmaxf(cm, z[i]);
    return cm;
  };
  auto fold = [&](const u32x4& q, bool first) {
    float z[VE];
    Elt<T>::unpack(q, z);
#pragma unroll
    for (int i = 0; i < VE; ++i) sz += z[i];
    if (first) {
      const float cm = vmax(z);
      m = cm == -INFINITY ? 0.f : cm;
      mb = m * kLog2e;
    }
    s += sum_exp(z, mb);
  };
#pragma unroll
  for (int k = 0; k < kKv; ++k) {
    if ((k + 1) * kBlock <= nvec) fold(buf[k], k == 0);
    else if ((int)threadIdx.x + k * kBlock < nvec) fold(buf[k], k == 0);
  }
  if ((int)threadIdx.x < nvec && !(s >= 0.5f && s < INFINITY)) {
    // Extreme logits: fold again with an exact online max.
    m = -INFINITY;
    s = 0.f;
#pragma unroll
    for (int k = 0; k < kKv; ++k) {
      if ((int)threadIdx.x + k * kBlock < nvec) {
        float z[VE];
        Elt<T>::unpack(buf[k], z);
        const float mn = __builtin_fmaxf(m, vmax(z));
        if (mn != -INFINITY) {
          s = (s == 0.f ? 0.f : s * fast_exp2((m - mn) * kLog2e)) + sum_exp(z, mn * kLog2e);
          m = mn;
        }
      }
    }
  }
  if ((int)threadIdx.x >= nvec) m = -INFINITY;  // lanes without values
  float lse, gz;
  block_lse<kWaves>(m, s, sz, lds, lse, gz);
  if (threadIdx.x == 0) stats[row] = Stats{lse, zt, gz, 0.f};
}

// Any alignment and width: element-wise, one row per workgroup.
template <typename T>
__global__ __launch_bounds__(kGenThreads) void shard_stats_generic(
    const T* __restrict__ logits, int64_t ld, const int64_t* __restrict__ targets, int64_t Vp,
    int64_t vocab_start, Stats* __restrict__ stats) {
  __shared__ float lds[3 * (kGenThreads / kWave)];
  const int64_t row = blockIdx.x;
  const T* xr = logits + row * ld;
  float m = -INFINITY, s = 0.f, sz = 0.f;
  for (int64_t j = threadIdx.x; j < Vp; j += kGenThreads) {
    const float z = Elt<T>::load1(xr + j);
    sz += z;
    if (z > m) {
      s = s == 0.f ? 0.f : s * fast_exp2((m - z) * kLog2e);
      m = z;
    }
    s += z == -INFINITY ? 0.f : fast_exp2((z - m) * kLog2e);
  }
  float lse, gz;
  block_lse<kGenThreads / kWave>(m, s, sz, lds, lse, gz);
  if (threadIdx.x == 0) {
    const int64_t tl = ts_plan::shard_col(targets[row], vocab_start, Vp);
    const float zt = tl >= 0 ? Elt<T>::load1(xr + tl) : 0.f;
    stats[row] = Stats{lse, zt, gz, 0.f};
  }
}

// Merges the P ranks' partials of each row (rank-major [P][N]) in one online
// pass. 64-thread workgroups: a C3-sized merge (16384 rows) then spreads over
// 256 workgroups rather than 64.
constexpr int kMergeThreads = 64;

__global__ __launch_bounds__(kMergeThreads) void shard_merge(
    const Stats* __restrict__ all, int64_t P, int64_t self, int64_t N, float inv_vp,
    float smoothing, float* __restrict__ lse_out, float* __restrict__ loss_out) {
  const int64_t row = (int64_t)blockIdx.x * kMergeThreads + threadIdx.x;
  if (row >= N) return;
  float gm = -INFINITY, gs = 0.f, zt = 0.f, sz = 0.f;
  // Eight ranks' partials are loaded before any is folded, so their loads
  // overlap instead of each waiting on the previous fold.
  constexpr int kU = 8;
  for (int64_t p0 = 0; p0 < P; p0 += kU) {
    Stats st[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u)
      st[u] = p0 + u < P ? all[(p0 + u) * N + row] : Stats{-INFINITY, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (st[u].lse > gm) {  // false for -inf partials and NaN
        gs = gs == 0.f ? 0.f : gs * fast_exp2((gm - st[u].lse) * kLog2e);
        gm = st[u].lse;
      }
      gs += st[u].lse == -INFINITY ? 0.f : fast_exp2((st[u].lse - gm) * kLog2e);
      zt += st[u].target;
      if (p0 + u == self) sz = st[u].sum_z;
    }
  }
  const float lse = gm == -INFINITY ? -INFINITY : gm + logf(gs);
  float loss = lse - zt;
  if (smoothing != 0.f) loss = (1.f - smoothing) * loss + smoothing * (lse - sz * inv_vp);
  lse_out[row] = lse;
  loss_out[row] = loss;
}

// grad = dl * ((1 - a) * (softmax - onehot) - a / Vp), the reference's
// backward (tensor_parallel.py:1607-1632), dl = grad_output * dloss_scale.
struct ShardBwd {
  float a1;     // dl * (1 - a)
  float c;      // dl * a / Vp
  float lse2;   // lse * log2(e)
  int64_t tl;   // target column within the shard (any value when outside)
};

__device__ inline float shard_grad(float z, int64_t j, const ShardBwd& r) {
  const float p = fast_exp2(__builtin_fmaf(z, kLog2e, -r.lse2));
  return r.a1 * (j == r.tl ? p - 1.f : p) - r.c;
}

__device__ inline ShardBwd shard_bwd_row(const int64_t* targets, const float* lse,
                                         const float* grad_output, float dloss_scale,
                                         float smoothing, int64_t Vp, int64_t vocab_start,
                                         int64_t row) {
  const float dl = grad_output[0] * dloss_scale;
  ShardBwd r;
  r.a1 = dl * (1.f - smoothing);
  r.c = smoothing == 0.f ? 0.f : dl * smoothing / (float)Vp;
  r.lse2 = lse[row] * kLog2e;
  r.tl = ts_plan::shard_col(targets[row], vocab_start, Vp);  // no column matches kLabelOutside
  return r;
}

template <typename G, int VE>
__device__ inline void store_grad(G* p, const float* g) {
  if constexpr (sizeof(G) == 4 && VE == 8) {
    st16_stream(p, Elt<float>::pack(g));
    st16_stream(p + 4, Elt<float>::pack(g + 4));
  } else {
    st16_stream(p, Elt<G>::pack(g));
  }
}

template <typename T, typename G>
__global__ __launch_bounds__(kBwdThreads) void shard_bwd_vec(
    const T* logits, int64_t ld, const int64_t* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ grad_output, float dloss_scale,
    float smoothing, G* grad, int64_t ld_grad, int64_t Vp, int64_t nvec, int64_t vocab_start,
    int64_t row0) {
  constexpr int VE = Elt<T>::kVec;
  static_assert(Elt<G>::kVec == VE || sizeof(G) == 4, "grad vector width");
  const int64_t row = row0 + blockIdx.y;
  const ShardBwd r =
      shard_bwd_row(targets, lse, grad_output, dloss_scale, smoothing, Vp, vocab_start, row);
  const T* xr = logits + row * ld;
  G* gr = grad + row * ld_grad;
  int64_t vk[kBwdKv];  // this thread's vectors of the row (ts_plan::chunk_vec)
#pragma unroll
  for (int k = 0; k < kBwdKv; ++k)
    vk[k] = ts_plan::chunk_vec(blockIdx.x, k, threadIdx.x, kBwdThreads, kBwdKv);
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
      float z[VE], g[VE];
      Elt<T>::unpack(buf[k], z);
#pragma unroll
      for (int i = 0; i < VE; ++i) g[i] = shard_grad(z[i], v * VE + i, r);
      store_grad<G, VE>(gr + v * VE, g);
    }
  }
}

template <typename T, typename G>
__global__ __launch_bounds__(kGenThreads) void shard_bwd_generic(
    const T* logits, int64_t ld, const int64_t* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ grad_output, float dloss_scale,
    float smoothing, G* grad, int64_t ld_grad, int64_t Vp, int64_t vocab_start) {
  const int64_t row = blockIdx.x;
  const ShardBwd r =
      shard_bwd_row(targets, lse, grad_output, dloss_scale, smoothing, Vp, vocab_start, row);
  const T* xr = logits + row * ld;
  G* gr = grad + row * ld_grad;
  for (int64_t j = threadIdx.x; j < Vp; j += kGenThreads)
    Elt<G>::store1(gr + j, shard_grad(Elt<T>::load1(xr + j), j, r));
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

template <typename T>
ts_status stats_typed(const void* logits, int64_t ld, const int64_t* targets, int64_t N,
                      int64_t Vp, int64_t vocab_start, Stats* stats, hipStream_t st) {
  constexpr int VE = sizeof(T) == 4 ? 4 : 8;
  const T* lp = static_cast<const T*>(logits);
  const int64_t nvec = Vp / VE;
  const bool vec = Vp % VE == 0 && ld % VE == 0 && ts_host::aligned16(logits) &&
                   nvec <= 1024 * 16;
  const dim3 grid((unsigned)N);
#define TS_STATS(B, K)                                                                        \
  if (nvec <= (int64_t)(B) * (K)) {                                                           \
    hipLaunchKernelGGL((shard_stats_vec<T, B, K>), grid, dim3(B), 0, st, lp, ld, targets, Vp, \
                       (int)nvec, vocab_start, stats);                                        \
    return ts_host::check_launch("shard_stats_vec");                                          \
  }
  if (vec) {
    TS_STATS(256, 1)
    TS_STATS(256, 2)
    TS_STATS(256, 4)
    TS_STATS(256, 8)
    TS_STATS(256, 16)
    TS_STATS(1024, 16)
  }
#undef TS_STATS
  hipLaunchKernelGGL((shard_stats_generic<T>), grid, dim3(kGenThreads), 0, st, lp, ld, targets,
                     Vp, vocab_start, stats);
  return ts_host::check_launch("shard_stats_generic");
}

template <typename T, typename G>
ts_status bwd_typed(const void* logits, int64_t ld, const int64_t* targets, const float* lse,
                    const float* grad_output, float dloss_scale, float smoothing, void* grad,
                    int64_t ld_grad, int64_t N, int64_t Vp, int64_t vocab_start,
                    hipStream_t st) {
  constexpr int VE = sizeof(T) == 4 ? 4 : 8;
  const T* lp = static_cast<const T*>(logits);
  G* gp = static_cast<G*>(grad);
  const bool grad_ok = sizeof(G) == sizeof(T) || (sizeof(G) == 4 && VE == 8);
  const bool vec = Vp % VE == 0 && ld % VE == 0 && ld_grad % VE == 0 &&
                   ts_host::aligned16(logits) && ts_host::aligned16(grad) && grad_ok;
  if (vec) {
    const int64_t nvec = Vp / VE;
    const unsigned gx = (unsigned)ts_plan::chunks_for(nvec, kBwdThreads, kBwdKv);
    for (int64_t r0 = 0; r0 < N; r0 += kMaxGridY) {
      const unsigned gy = (unsigned)(N - r0 < kMaxGridY ? N - r0 : kMaxGridY);
      hipLaunchKernelGGL((shard_bwd_vec<T, G>), dim3(gx, gy), dim3(kBwdThreads), 0, st, lp, ld,
                         targets, lse, grad_output, dloss_scale, smoothing, gp, ld_grad, Vp,
                         nvec, vocab_start, r0);
      const ts_status s = ts_host::check_launch("shard_bwd_vec");
      if (s != TS_OK) return s;
    }
    return TS_OK;
  }
  hipLaunchKernelGGL((shard_bwd_generic<T, G>), dim3((unsigned)N), dim3(kGenThreads), 0, st, lp,
                     ld, targets, lse, grad_output, dloss_scale, smoothing, gp, ld_grad, Vp,
                     vocab_start);
  return ts_host::check_launch("shard_bwd_generic");
}

ts_status check_shard(const void* logits, int64_t ld, ts_dtype dtype, const int64_t* targets,
                      int64_t N, int64_t Vp, int64_t vocab_start, const char* who) {
  using ts_host::fail;
  if (!ts_host::valid_dtype(dtype)) return fail(TS_ERR_UNSUPPORTED_DTYPE, "%s: bad dtype", who);
  if (N < 0 || Vp <= 0 || ld < Vp)
    return fail(TS_ERR_SHAPE, "%s: bad shape N=%lld Vp=%lld ld=%lld", who, (long long)N,
                (long long)Vp, (long long)ld);
  if (N > INT32_MAX) return fail(TS_ERR_SHAPE, "%s: more than 2^31 - 1 rows", who);
  if (vocab_start < 0) return fail(TS_ERR_INVALID_ARGUMENT, "%s: vocab_start < 0", who);
  if (N > 0 && (logits == nullptr || targets == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "%s: logits or targets is NULL", who);
  // 16-byte offsets of a row must stay below the buffer range check's 2^31.
  if (Vp > ((int64_t)1 << 28)) return fail(TS_ERR_SHAPE, "%s: shard wider than 2^28", who);
  return TS_OK;
}

}  // namespace

extern "C" ts_status ts_ce_vocab_shard_stats(const void* logits, int64_t ld, ts_dtype dtype,
                                             const int64_t* targets, int64_t N, int64_t Vp,
                                             int64_t vocab_start, float* stats,
                                             ts_stream_t stream) {
  const ts_status c = check_shard(logits, ld, dtype, targets, N, Vp, vocab_start,
                                  "ce_vocab_shard_stats");
  if (c != TS_OK) return c;
  if (N > 0 && stats == nullptr)
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_shard_stats: stats is NULL");
  if (N > 0 && !ts_host::aligned16(stats))
    return ts_host::fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_shard_stats: stats not 16-byte aligned");
  if (N == 0) return TS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  Stats* sp = reinterpret_cast<Stats*>(stats);
  switch (dtype) {
    case TS_BF16: return stats_typed<__bf16>(logits, ld, targets, N, Vp, vocab_start, sp, st);
    case TS_F16: return stats_typed<_Float16>(logits, ld, targets, N, Vp, vocab_start, sp, st);
    case TS_F32: return stats_typed<float>(logits, ld, targets, N, Vp, vocab_start, sp, st);
  }
  return ts_host::fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_vocab_shard_stats: bad dtype");
}

extern "C" ts_status ts_ce_vocab_merge(const float* stats_all, int64_t P, int64_t self,
                                       int64_t N, int64_t Vp, float label_smoothing,
                                       float* lse, float* loss, ts_stream_t stream) {
  using ts_host::fail;
  if (P < 1 || self < 0 || self >= P)
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_merge: need 0 <= self < P (P=%lld self=%lld)",
                (long long)P, (long long)self);
  if (N < 0 || Vp <= 0)
    return fail(TS_ERR_SHAPE, "ce_vocab_merge: bad shape N=%lld Vp=%lld", (long long)N,
                (long long)Vp);
  if (!(label_smoothing >= 0.f && label_smoothing <= 1.f))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_merge: label_smoothing outside [0, 1]");
  if (N == 0) return TS_OK;
  if (stats_all == nullptr || lse == nullptr || loss == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_merge: NULL pointer");
  if (!ts_host::aligned16(stats_all))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_merge: stats not 16-byte aligned");
  if (P > ((int64_t)1 << 20) || N > INT32_MAX)
    return fail(TS_ERR_SHAPE, "ce_vocab_merge: too many ranks or rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(shard_merge, dim3((unsigned)((N + kMergeThreads - 1) / kMergeThreads)),
                     dim3(kMergeThreads), 0, st,
                     reinterpret_cast<const Stats*>(stats_all), P, self, N, 1.f / (float)Vp,
                     label_smoothing, lse, loss);
  return ts_host::check_launch("shard_merge");
}

extern "C" ts_status ts_ce_vocab_shard_bwd(const void* logits, int64_t ld, ts_dtype dtype,
                                           const int64_t* targets, const float* lse,
                                           const float* grad_output, float dloss_scale,
                                           int64_t N, int64_t Vp, int64_t vocab_start,
                                           float label_smoothing, void* grad, int64_t ld_grad,
                                           ts_dtype grad_dtype, ts_stream_t stream) {
  using ts_host::fail;
  const ts_status c = check_shard(logits, ld, dtype, targets, N, Vp, vocab_start,
                                  "ce_vocab_shard_bwd");
  if (c != TS_OK) return c;
  if (!ts_host::valid_dtype(grad_dtype))
    return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_vocab_shard_bwd: bad grad dtype");
  if (grad_dtype != dtype && grad_dtype != TS_F32)
    return fail(TS_ERR_UNSUPPORTED_DTYPE,
                "ce_vocab_shard_bwd: grad dtype must be the logits dtype or fp32");
  if (ld_grad < Vp) return fail(TS_ERR_SHAPE, "ce_vocab_shard_bwd: ld_grad < Vp");
  if (!(label_smoothing >= 0.f && label_smoothing <= 1.f))
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_shard_bwd: label_smoothing outside [0, 1]");
  if (N == 0) return TS_OK;
  if (lse == nullptr || grad_output == nullptr || grad == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "ce_vocab_shard_bwd: NULL pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define TS_SHARD_BWD(T, TC)                                                                     \
  case TC:                                                                                     \
    if (grad_dtype == TS_F32)                                                                  \
      return bwd_typed<T, float>(logits, ld, targets, lse, grad_output, dloss_scale,           \
                                 label_smoothing, grad, ld_grad, N, Vp, vocab_start, st);      \
    return bwd_typed<T, T>(logits, ld, targets, lse, grad_output, dloss_scale,                 \
                           label_smoothing, grad, ld_grad, N, Vp, vocab_start, st);
  switch (dtype) {
    TS_SHARD_BWD(__bf16, TS_BF16)
    TS_SHARD_BWD(_Float16, TS_F16)
    TS_SHARD_BWD(float, TS_F32)
  }
#undef TS_SHARD_BWD
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "ce_vocab_shard_bwd: bad dtype");
}
