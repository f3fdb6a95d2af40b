// SwiGLU forward/backward for gfx950:
//   out   = round(round(silu(gate)) * up),  silu(g) = g * sigmoid(g)
//   dgate = dout * up * sigmoid(g) * (1 + g * (1 - sigmoid(g)))
//   dup   = dout * silu(g)
// Arithmetic in fp32; the forward rounds silu to the data type before the
// product with up, as the reference's kernel does (silu.to(up.dtype) * up).
//
// Elementwise and HBM-bound (3 tensors of traffic forward, 5 backward), so
// the grid is one-shot: each thread owns kSwiKv 16-byte vectors spaced one
// workgroup apart, with every load issued before any arithmetic. A tensor
// whose length is not a multiple of the vector width, or that is not 16-byte
// aligned, goes through the element-wise kernels.
//
// sigmoid(g) = 1 / (1 + 2^(-g * log2 e)) with v_exp_f32 and v_rcp_f32 (each
// within 1 ulp); for g below about -88 the exponential overflows to +inf and
// sigmoid is 0, for g above about 104 it is exactly 1.
#include "common.hpp"
#include "plan.hpp"

namespace {

using namespace ts;

constexpr int kSwiThreads = 256;
// One 16-byte vector per thread: measured on MI355X at [8, 2048, 14336] bf16, the
// forward took 216 us against 230 us with two vectors per thread, the backward
// 376 against 387 us.
constexpr int kSwiKv = 1;

__device__ inline float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.f + fast_exp2(-g * kLog2e));
}

template <typename T>
__device__ inline float swiglu_out(float g, float u) {
  const float s = g * sigmoid_f(g);
  return Elt<T>::round(s) * u;
}

template <typename T>
__device__ inline void swiglu_grads(float d, float g, float u, float& dg, float& du) {
  const float sg = sigmoid_f(g);
  const float s = g * sg;
  dg = d * u * (sg * (1.f + g * (1.f - sg)));
  du = d * s;
}

template <typename T>
__global__ __launch_bounds__(kSwiThreads) void swiglu_fwd_vec(const T* __restrict__ gate,
                                                              const T* __restrict__ up,
                                                              T* __restrict__ out, int64_t nvec) {
  constexpr int VE = Elt<T>::kVec;
  int64_t vk[kSwiKv];  // this thread's vectors (ts_plan::chunk_vec)
#pragma unroll
  for (int k = 0; k < kSwiKv; ++k)
    vk[k] = ts_plan::chunk_vec(blockIdx.x, k, threadIdx.x, kSwiThreads, kSwiKv);
  u32x4 gq[kSwiKv], uq[kSwiKv];
#pragma unroll
  for (int k = 0; k < kSwiKv; ++k) {
    const int64_t v = vk[k];
    if (v < nvec) {
      gq[k] = ld16_stream(gate + v * VE);
      uq[k] = ld16_stream(up + v * VE);
    }
  }
#pragma unroll
  for (int k = 0; k < kSwiKv; ++k) {
    const int64_t v = vk[k];
    if (v < nvec) {
      float g[VE], u[VE];
      Elt<T>::unpack(gq[k], g);
      Elt<T>::unpack(uq[k], u);
#pragma unroll
      for (int i = 0; i < VE; ++i) g[i] = swiglu_out<T>(g[i], u[i]);
      st16_stream(out + v * VE, Elt<T>::pack(g));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kSwiThreads) void swiglu_bwd_vec(
    const T* __restrict__ dout, const T* __restrict__ gate, const T* __restrict__ up,
    T* __restrict__ dgate, T* __restrict__ dup, int64_t nvec) {
  constexpr int VE = Elt<T>::kVec;
  int64_t vk[kSwiKv];  // this thread's vectors (ts_plan::chunk_vec)
#pragma unroll
  for (int k = 0; k < kSwiKv; ++k)
    vk[k] = ts_plan::chunk_vec(blockIdx.x, k, threadIdx.x, kSwiThreads, kSwiKv);
  u32x4 dq[kSwiKv], gq[kSwiKv], uq[kSwiKv];
#pragma unroll
  for (int k = 0; k < kSwiKv; ++k) {
    const int64_t v = vk[k];
    if (v < nvec) {
      dq[k] = ld16_stream(dout + v * VE);
      gq[k] = ld16_stream(gate + v * VE);
      uq[k] = ld16_stream(up + v * VE);
    }
  }
#pragma unroll
  for (int k = 0; k < kSwiKv; ++k) {
    const int64_t v = vk[k];
    if (v < nvec) {
      float d[VE], g[VE], u[VE];
      Elt<T>::unpack(dq[k], d);
      Elt<T>::unpack(gq[k], g);
      Elt<T>::unpack(uq[k], u);
#pragma unroll
      for (int i = 0; i < VE; ++i) swiglu_grads<T>(d[i], g[i], u[i], g[i], u[i]);
      st16_stream(dgate + v * VE, Elt<T>::pack(g));
      st16_stream(dup + v * VE, Elt<T>::pack(u));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kSwiThreads) void swiglu_fwd_generic(const T* gate, const T* up,
                                                                  T* out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kSwiThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kSwiThreads)
    Elt<T>::store1(out + i, swiglu_out<T>(Elt<T>::load1(gate + i), Elt<T>::load1(up + i)));
}

template <typename T>
__global__ __launch_bounds__(kSwiThreads) void swiglu_bwd_generic(const T* dout, const T* gate,
                                                                  const T* up, T* dgate, T* dup,
                                                                  int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kSwiThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kSwiThreads) {
    float dg, du;
    swiglu_grads<T>(Elt<T>::load1(dout + i), Elt<T>::load1(gate + i), Elt<T>::load1(up + i), dg,
                    du);
    Elt<T>::store1(dgate + i, dg);
    Elt<T>::store1(dup + i, du);
  }
}

constexpr int64_t kGenericGrid = 4096;

template <typename T>
ts_status fwd_typed(const void* gate, const void* up, void* out, int64_t n, hipStream_t st) {
  constexpr int VE = Elt<T>::kVec;
  const T* g = static_cast<const T*>(gate);
  const T* u = static_cast<const T*>(up);
  T* o = static_cast<T*>(out);
  if (n % VE == 0 && ts_host::aligned16(gate) && ts_host::aligned16(up) &&
      ts_host::aligned16(out)) {
    const int64_t nvec = n / VE;
    const int64_t blocks = ts_plan::chunks_for(nvec, kSwiThreads, kSwiKv);
    if (blocks > 0x7fffffff) return ts_host::fail(TS_ERR_SHAPE, "swiglu: tensor too large");
    hipLaunchKernelGGL(swiglu_fwd_vec<T>, dim3((unsigned)blocks), dim3(kSwiThreads), 0, st, g, u,
                       o, nvec);
    return ts_host::check_launch("swiglu_fwd_vec");
  }
  int64_t blocks = (n + kSwiThreads - 1) / kSwiThreads;
  if (blocks > kGenericGrid) blocks = kGenericGrid;
  hipLaunchKernelGGL(swiglu_fwd_generic<T>, dim3((unsigned)blocks), dim3(kSwiThreads), 0, st, g,
                     u, o, n);
  return ts_host::check_launch("swiglu_fwd_generic");
}

template <typename T>
ts_status bwd_typed(const void* dout, const void* gate, const void* up, void* dgate, void* dup,
                    int64_t n, hipStream_t st) {
  constexpr int VE = Elt<T>::kVec;
  const T* d = static_cast<const T*>(dout);
  const T* g = static_cast<const T*>(gate);
  const T* u = static_cast<const T*>(up);
  T* dg = static_cast<T*>(dgate);
  T* du = static_cast<T*>(dup);
  if (n % VE == 0 && ts_host::aligned16(dout) && ts_host::aligned16(gate) &&
      ts_host::aligned16(up) && ts_host::aligned16(dgate) && ts_host::aligned16(dup)) {
    const int64_t nvec = n / VE;
    const int64_t blocks = ts_plan::chunks_for(nvec, kSwiThreads, kSwiKv);
    if (blocks > 0x7fffffff) return ts_host::fail(TS_ERR_SHAPE, "swiglu: tensor too large");
    hipLaunchKernelGGL(swiglu_bwd_vec<T>, dim3((unsigned)blocks), dim3(kSwiThreads), 0, st, d, g,
                       u, dg, du, nvec);
    return ts_host::check_launch("swiglu_bwd_vec");
  }
  int64_t blocks = (n + kSwiThreads - 1) / kSwiThreads;
  if (blocks > kGenericGrid) blocks = kGenericGrid;
  hipLaunchKernelGGL(swiglu_bwd_generic<T>, dim3((unsigned)blocks), dim3(kSwiThreads), 0, st, d,
                     g, u, dg, du, n);
  return ts_host::check_launch("swiglu_bwd_generic");
}

}  // namespace

extern "C" ts_status ts_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n,
                                   ts_dtype dtype, ts_stream_t stream) {
  using ts_host::fail;
  if (!ts_host::valid_dtype(dtype)) return fail(TS_ERR_UNSUPPORTED_DTYPE, "swiglu_fwd: bad dtype");
  if (n < 0) return fail(TS_ERR_SHAPE, "swiglu_fwd: negative size");
  if (n == 0) return TS_OK;
  if (gate == nullptr || up == nullptr || out == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "swiglu_fwd: NULL pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TS_BF16: return fwd_typed<__bf16>(gate, up, out, n, st);
    case TS_F16: return fwd_typed<_Float16>(gate, up, out, n, st);
    case TS_F32: return fwd_typed<float>(gate, up, out, n, st);
  }
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "swiglu_fwd: bad dtype");
}

extern "C" ts_status ts_swiglu_bwd(const void* dout, const void* gate, const void* up,
                                   void* dgate, void* dup, int64_t n, ts_dtype dtype,
                                   ts_stream_t stream) {
  using ts_host::fail;
  if (!ts_host::valid_dtype(dtype)) return fail(TS_ERR_UNSUPPORTED_DTYPE, "swiglu_bwd: bad dtype");
  if (n < 0) return fail(TS_ERR_SHAPE, "swiglu_bwd: negative size");
  if (n == 0) return TS_OK;
  if (dout == nullptr || gate == nullptr || up == nullptr || dgate == nullptr || dup == nullptr)
    return fail(TS_ERR_INVALID_ARGUMENT, "swiglu_bwd: NULL pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TS_BF16: return bwd_typed<__bf16>(dout, gate, up, dgate, dup, n, st);
    case TS_F16: return bwd_typed<_Float16>(dout, gate, up, dgate, dup, n, st);
    case TS_F32: return bwd_typed<float>(dout, gate, up, dgate, dup, n, st);
  }
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "swiglu_bwd: bad dtype");
}
