// Host-side status reporting and device queries for the C ABI.
#include <stdarg.h>
#include <stdio.h>


#include "common.hpp"

namespace ts_host {

static thread_local char g_last_error[512] = "no error";

ts_status fail(ts_status code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

ts_status check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(TS_ERR_LAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(e));
  }
  return TS_OK;
}

}  // namespace ts_host

extern "C" const char* ts_last_error(void) { return ts_host::g_last_error; }

extern "C" const char* ts_version(void) { return "trainscale_amd 0.1.0 gfx950"; }

// ---------------------------------------------------------------------------
// Reference copy: the flat streaming copy (one 16-byte vector per thread,
// 256-thread workgroups, non-temporal loads and stores) against which the
// benchmark sets each memory-bound kernel, for the same bytes moved.
// ---------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(256) void stream_copy(const ts::u32x4* __restrict__ src,
                                                   ts::u32x4* __restrict__ dst, int64_t nvec) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nvec) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

extern "C" ts_status ts_stream_copy(void* dst, const void* src, int64_t bytes,
                                    ts_stream_t stream) {
  using ts_host::fail;
  if (bytes < 0 || bytes % 16 != 0)
    return fail(TS_ERR_SHAPE, "stream_copy: bytes must be a non-negative multiple of 16");
  if (bytes == 0) return TS_OK;
  if (dst == nullptr || src == nullptr || !ts_host::aligned16(dst) || !ts_host::aligned16(src))
    return fail(TS_ERR_INVALID_ARGUMENT, "stream_copy: NULL or unaligned buffer");
  const int64_t nvec = bytes / 16;
  const int64_t blocks = (nvec + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TS_ERR_SHAPE, "stream_copy: too large");
  hipLaunchKernelGGL(stream_copy, dim3((unsigned)blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const ts::u32x4*>(src),
                     static_cast<ts::u32x4*>(dst), nvec);
  return ts_host::check_launch("stream_copy");
}
