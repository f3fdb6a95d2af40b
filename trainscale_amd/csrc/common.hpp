// Shared device and host helpers for the gfx950 kernels.
//
// Device side: 16-byte vector access with fp32 unpacking for bf16/fp16/fp32
// elements, wave64 reductions built from DPP row operations plus lane reads
// (no LDS round trip inside a wave), and workgroup reductions that go
// through LDS once per wave.
//
// Host side: thread-local error reporting for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/trainscale_amd.h"

namespace ts {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Element types
// ---------------------------------------------------------------------------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Elements per 16-byte vector and conversions to/from fp32. The bf16 store
// path lowers to v_cvt_pk_bf16_f32 (round to nearest even, like torch).
//
// Note on vector elements: never pass an element of an ext_vector_type
// (v[i]) directly as the operand of __builtin_bit_cast. hipcc (ROCm 7.2)
// compiles that as a read of element 0 whatever i is; copy the element into
// a scalar first.
template <typename T> struct Elt;

template <> struct Elt<__bf16> {
  static constexpr int kVec = 8;
  __device__ static inline void unpack(const u32x4& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __builtin_bit_cast(float, v[i] << 16);
      f[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
    }
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bf16x2_t h = {(__bf16)f[2 * i], (__bf16)f[2 * i + 1]};
      v[i] = __builtin_bit_cast(uint32_t, h);
    }
    return v;
  }
  __device__ static inline float load1(const __bf16* p) {
    return __builtin_bit_cast(float, (uint32_t)(*(const uint16_t*)p) << 16);
  }
  __device__ static inline void store1(__bf16* p, float f) { *p = (__bf16)f; }
  __device__ static inline float round(float f) { return (float)(__bf16)f; }
};

template <> struct Elt<_Float16> {
  static constexpr int kVec = 8;
  __device__ static inline void unpack(const u32x4& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = v[i];  // see the note on vector elements above
      f16x2_t h = __builtin_bit_cast(f16x2_t, u);
      f[2 * i] = (float)h[0];
      f[2 * i + 1] = (float)h[1];
    }
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f16x2_t h = {(_Float16)f[2 * i], (_Float16)f[2 * i + 1]};
      v[i] = __builtin_bit_cast(uint32_t, h);
    }
    return v;
  }
  __device__ static inline float load1(const _Float16* p) { return (float)*p; }
  __device__ static inline void store1(_Float16* p, float f) { *p = (_Float16)f; }
  __device__ static inline float round(float f) { return (float)(_Float16)f; }
};

template <> struct Elt<float> {
  static constexpr int kVec = 4;
  __device__ static inline void unpack(const u32x4& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = v[i];  // see the note on vector elements above
      f[i] = __builtin_bit_cast(float, u);
    }
  }
  __device__ static inline u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_bit_cast(uint32_t, f[i]);
    return v;
  }
  __device__ static inline float load1(const float* p) { return *p; }
  __device__ static inline void store1(float* p, float f) { *p = f; }
  __device__ static inline float round(float f) { return f; }
};

template <typename T>
__device__ inline u32x4 ld16(const T* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Streaming load: data touched exactly once, keep it out of the way of
// reused lines (non-temporal hint).
template <typename T>
__device__ inline u32x4 ld16_stream(const T* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
template <typename T>
__device__ inline void st16(T* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
template <typename T>
__device__ inline void st16_stream(T* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Raw buffer access: a 128-bit resource (base, byte range) held in SGPRs and
// a 32-bit per-lane byte offset, so a row's addresses cost one VGPR instead
// of a 64-bit pointer per access. The hardware range check drops stores and
// zero-fills loads at offsets >= the range. It looks at the VGPR offset only
// (the SGPR offset operand is not range-checked), so every offset goes in the
// VGPR operand and an access that must not happen uses kBufOob. The range
// must stay below 2^31 bytes for kBufOob to lie outside it.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kBufOob = (int)0x80000000u;
constexpr int kBufNt = 2;  // non-temporal cache policy

__device__ inline Rsrc buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ inline u32x4 buf_ld16_stream(Rsrc r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kBufNt);
}
__device__ inline void buf_st16_stream(const u32x4& v, Rsrc r, int voff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, kBufNt);
}

// ---------------------------------------------------------------------------
// Wave64 reductions: DPP inside each 16-lane row (every lane of a row ends
// with the row's result), then the four row results are read with
// v_readlane_b32 and combined in a fixed order. Every lane gets the result.
//
// The gfx950 v_permlane16_swap/v_permlane32_swap builtins are not used: with
// the same value passed as both operands, hipcc (ROCm 7.2) keeps only the
// first of the two results, which turns the cross-row sum into a doubling.
// ---------------------------------------------------------------------------

template <int kCtrl>
__device__ inline float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

__device__ inline float lane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ inline float row_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

__device__ inline float row_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

// Requires all 64 lanes active.
__device__ inline float wave_sum(float v) {
  v = row_sum(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ inline float wave_max(float v) {
  v = row_max(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Sum over a workgroup of kWaves waves; `lds` holds kWaves floats. All
// threads receive the result. Contains two barriers.
template <int kWaves>
__device__ inline float block_sum(float v, float* lds) {
  v = wave_sum(v);
  const int wid = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) lds[wid] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) t += lds[i];
  __syncthreads();
  return t;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace ts

// ---------------------------------------------------------------------------
// Host-side helpers shared by the C ABI translation units.
// ---------------------------------------------------------------------------
namespace ts_host {

// Records `msg` as this thread's last error and returns `code`.
ts_status fail(ts_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Turns a launch error into TS_ERR_LAUNCH with the kernel name attached.
ts_status check_launch(const char* kernel);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t dtype_size(ts_dtype t) { return t == TS_F32 ? 4 : 2; }
inline bool valid_dtype(int t) { return t == TS_F32 || t == TS_BF16 || t == TS_F16; }

}  // namespace ts_host
