// Rotary position embedding (RoPE) forward/backward for gfx950.
//
// A workgroup handles `tpb` consecutive tokens (b, s) and every head of both
// tensors (Q heads then K heads) at those tokens. A task is one 16-byte vector
// from each half of a head (NeoX layout: pairs (i, i + D/2)) or one 16-byte
// vector of adjacent pairs (interleaved layout); the workgroup has about one
// thread per task (320 threads for 32 + 8 heads of 128), so each thread keeps
// two 16-byte loads in flight and Q and K are read and written exactly once.
//
// Each thread issues the loads of its first task, then the workgroup fills
// LDS with cos/sin for its tokens: gathered from the caller's tables at
// pos(b, s), or evaluated from the fp32 angle fp32(pos / pos_div) * inv_freq[i]
// (times angle_scale when that is not 1)
// (the product torch.outer forms on the host), once per (token, frequency)
// and shared by all Hq + Hk heads. After one barrier the thread rotates and
// stores. Backward is the same kernel with sin negated (the transpose
// rotation).
//
// A generic element-wise kernel (a task is one pair) covers unaligned tensors
// and head dims whose half is not a multiple of the vector width.
#include <math.h>

#include "common.hpp"
#include "plan.hpp"

namespace {

using namespace ts;

constexpr int kMaxThreads = 1024;
constexpr int kMaxHalf = 256;        // head_dim <= 512
constexpr int kLdsAngles = 4096;     // max tpb * half (cos + sin = 32 KiB of LDS)

struct RopeArgs {
  const void* q_in;
  void* q_out;
  int64_t q_in_sb, q_in_ss, q_in_sh;
  int64_t q_out_sb, q_out_ss, q_out_sh;
  const void* k_in;
  void* k_out;
  int64_t k_in_sb, k_in_ss, k_in_sh;
  int64_t k_out_sb, k_out_ss, k_out_sh;
  int32_t Hq, Hk;
  int64_t S, ntok;
  int32_t half;
  const void* cos_tab;
  const void* sin_tab;
  int64_t tab_ld, table_rows;
  float pos_div;
  float angle_scale;         // multiplies the fp32 angle when != 1 (YaRN's mscale)
  const int64_t* position_ids;
  int64_t pos_sb, pos_ss, position_offset;
  int32_t backward;
  int32_t tpb;               // tokens per workgroup
  int32_t tasks_per_head;    // 16-byte tasks per head (vector path) or pairs per head
  int32_t tasks_per_token;   // tasks_per_head * (Hq + Hk)
  uint32_t tpt_magic;        // ts_plan::magic_for(tasks_per_token)
  uint32_t tph_magic;        // ts_plan::magic_for(tasks_per_head)
  uint64_t s_magic;          // ts_plan::magic64_for(S), exact for every token (tok kernel)
  float inv_freq[kMaxHalf];
};

template <typename TabT>
__device__ inline float tab_load(const void* p, int64_t idx) {
  return Elt<TabT>::load1(static_cast<const TabT*>(p) + idx);
}

// cos/sin of frequency f at position pos (sin negated for the backward).
template <typename TabT, bool kTable>
__device__ inline void angle_at(const RopeArgs& a, int64_t pos, int f, float& c, float& s) {
  if constexpr (kTable) {
    if (pos >= 0 && pos < a.table_rows) {
      c = tab_load<TabT>(a.cos_tab, pos * a.tab_ld + f);
      s = tab_load<TabT>(a.sin_tab, pos * a.tab_ld + f);
    } else {
      c = s = __builtin_nanf("");
    }
  } else {
    float ang = ((float)pos / a.pos_div) * a.inv_freq[f];
    if (a.angle_scale != 1.f) ang *= a.angle_scale;
    sincosf(ang, &s, &c);
  }
  if (a.backward) s = -s;
}

// cos/sin of the workgroup's tokens into LDS ([tpb][half] each).
template <typename TabT, bool kTable>
__device__ inline void fill_angles(const RopeArgs& a, int64_t tok0, float* cs, float* sn) {
  const int n = a.tpb * a.half;
  for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
    const int i = idx / a.half;
    const int f = idx - i * a.half;
    const int64_t t = tok0 + i;
    float c = 1.f, s = 0.f;
    if (t < a.ntok) {
      const int64_t b = t / a.S;
      const int64_t sq = t - b * a.S;
      const int64_t pos = a.position_ids != nullptr
                              ? a.position_ids[b * a.pos_sb + sq * a.pos_ss]
                              : sq + a.position_offset;
      angle_at<TabT, kTable>(a, pos, f, c, s);
    }
    cs[idx] = c;
    sn[idx] = s;
  }
}

// Task f of the workgroup starting at token tok0: source/destination head
// pointers, token slot i and index j of the task within its head.
template <typename T>
struct Task {
  const T* src;
  T* dst;
  int i;
  int j;
};

template <typename T>
__device__ inline Task<T> task_at(const RopeArgs& a, int64_t tok0, int f) {
  Task<T> k;
  // n / d as umulhi(n, ceil(2^32 / d)) (ts_plan::magic_div), exact while n * d < 2^32,
  // which the host checks for every launch
  const ts_plan::RopeTask rt =
      ts_plan::rope_task(f, a.tasks_per_token, a.tpt_magic, a.tasks_per_head, a.tph_magic);
  k.i = rt.i;
  const int hh = rt.hh;
  k.j = rt.j;
  const int64_t t = tok0 + k.i;
  const int64_t b = t / a.S;
  const int64_t sq = t - b * a.S;
  // Both candidates, then a select: choosing between the Q and K strides in a
  // branch lets the compiler fetch the chosen stride with a per-lane load from
  // the argument block, a memory round trip ahead of the data loads.
  const bool is_q = hh < a.Hq;
  const int kh = hh - a.Hq;
  const T* sq_src = static_cast<const T*>(a.q_in) + b * a.q_in_sb + sq * a.q_in_ss + hh * a.q_in_sh;
  T* sq_dst = static_cast<T*>(a.q_out) + b * a.q_out_sb + sq * a.q_out_ss + hh * a.q_out_sh;
  const T* sk_src = static_cast<const T*>(a.k_in) + b * a.k_in_sb + sq * a.k_in_ss + kh * a.k_in_sh;
  T* sk_dst = static_cast<T*>(a.k_out) + b * a.k_out_sb + sq * a.k_out_ss + kh * a.k_out_sh;
  k.src = is_q ? sq_src : sk_src;
  k.dst = is_q ? sq_dst : sk_dst;
  return k;
}

// Loads of one vector task: NeoX reads one vector from each half, the
// interleaved layout one vector of adjacent pairs (v2 unused).
template <typename T, bool kInterleaved>
__device__ inline void task_load(const RopeArgs& a, const Task<T>& k, u32x4& v1, u32x4& v2) {
  constexpr int V = Elt<T>::kVec;
  const ts_plan::RopeElems e = ts_plan::rope_elems(k.j, V, a.half, kInterleaved);
  v1 = ld16_stream(k.src + e.e1);
  v2 = kInterleaved ? u32x4{0, 0, 0, 0} : ld16_stream(k.src + e.e2);
}

// The rotation's two outputs, x1 c - x2 s and x2 c + x1 s, with each product
// rounded to fp32 before the sum (no fused multiply-add): the roundings of the
// reference's eager rotation (triton_kernels.py:908-925) and of the CPU
// restatement, so that from the same cos/sin values the outputs are bit-identical
// to theirs. The backward passes -s.
__device__ inline float rot_lo(float x1, float x2, float c, float s) {
#pragma clang fp contract(off)
  return x1 * c - x2 * s;
}
__device__ inline float rot_hi(float x1, float x2, float c, float s) {
#pragma clang fp contract(off)
  return x2 * c + x1 * s;
}

template <typename T, bool kInterleaved>
__device__ inline void task_rotate_store(const RopeArgs& a, const Task<T>& k, const u32x4& v1,
                                         const u32x4& v2, const float* cs, const float* sn) {
  constexpr int V = Elt<T>::kVec;
  const float* crow = cs + k.i * a.half;
  const float* srow = sn + k.i * a.half;
  const ts_plan::RopeElems el = ts_plan::rope_elems(k.j, V, a.half, kInterleaved);
  if constexpr (!kInterleaved) {
    const int e1 = el.e1;
    float x1[V], x2[V], o1[V], o2[V];
    Elt<T>::unpack(v1, x1);
    Elt<T>::unpack(v2, x2);
#pragma unroll
    for (int p = 0; p < V; ++p) {
      const float c = crow[e1 + p];
      const float s = srow[e1 + p];
      o1[p] = rot_lo(x1[p], x2[p], c, s);
      o2[p] = rot_hi(x1[p], x2[p], c, s);
    }
    st16_stream(k.dst + e1, Elt<T>::pack(o1));
    st16_stream(k.dst + el.e2, Elt<T>::pack(o2));
  } else {
    const int e = el.e1;
    float x[V], o[V];
    Elt<T>::unpack(v1, x);
#pragma unroll
    for (int p = 0; p < V / 2; ++p) {
      const float c = crow[e / 2 + p];
      const float s = srow[e / 2 + p];
      o[2 * p] = rot_lo(x[2 * p], x[2 * p + 1], c, s);
      o[2 * p + 1] = rot_hi(x[2 * p], x[2 * p + 1], c, s);
    }
    st16_stream(k.dst + e, Elt<T>::pack(o));
  }
}

template <typename T, typename TabT, bool kTable, bool kInterleaved>
__global__ __launch_bounds__(kMaxThreads) void rope_vec_kernel(const RopeArgs a) {
  extern __shared__ float lds[];
  float* cs = lds;
  float* sn = lds + a.tpb * a.half;
  const int64_t tok0 = (int64_t)blockIdx.x * a.tpb;
  const int64_t ntok_here = a.ntok - tok0 < a.tpb ? a.ntok - tok0 : a.tpb;
  const int total = (int)ntok_here * a.tasks_per_token;

  // First task's loads go out before the angle phase.
  int f = threadIdx.x;
  Task<T> k0{};
  u32x4 v1{0, 0, 0, 0}, v2{0, 0, 0, 0};
  if (f < total) {
    k0 = task_at<T>(a, tok0, f);
    task_load<T, kInterleaved>(a, k0, v1, v2);
  }
  fill_angles<TabT, kTable>(a, tok0, cs, sn);
  __syncthreads();
  if (f < total) task_rotate_store<T, kInterleaved>(a, k0, v1, v2, cs, sn);
  for (f += blockDim.x; f < total; f += blockDim.x) {
    const Task<T> k = task_at<T>(a, tok0, f);
    task_load<T, kInterleaved>(a, k, v1, v2);
    task_rotate_store<T, kInterleaved>(a, k, v1, v2, cs, sn);
  }
}

// One token per workgroup, for tokens of at least 256 vector tasks (the
// attention shapes, e.g. 32 + 8 or 64 + 8 heads of 128). The token's batch
// and position (token / S by a 64-bit magic number), its position id and both
// tensors' row pointers are uniform, so the scalar unit forms them once; a
// lane derives only its head and vector index and issues its loads a few
// instructions after it starts. Measured on MI355X at C2 this runs at the
// speed of a plain copy of the same bytes and launch shape (56.5 us against
// 62.5 us for rope_vec_kernel, whose lanes each split a token index into
// batch, position and head before their first load).
template <typename T, typename TabT, bool kTable, bool kInterleaved>
__global__ __launch_bounds__(kMaxThreads) void rope_tok_kernel(const RopeArgs a) {
  __shared__ float cs[kMaxHalf], sn[kMaxHalf];
  const int64_t t = blockIdx.x;
  const int64_t b = a.s_magic == 0 ? t : (int64_t)__umul64hi((uint64_t)t, a.s_magic);
  const int64_t sq = t - b * a.S;
  const T* qi = static_cast<const T*>(a.q_in) + b * a.q_in_sb + sq * a.q_in_ss;
  T* qo = static_cast<T*>(a.q_out) + b * a.q_out_sb + sq * a.q_out_ss;
  const T* ki = static_cast<const T*>(a.k_in) + b * a.k_in_sb + sq * a.k_in_ss;
  T* ko = static_cast<T*>(a.k_out) + b * a.k_out_sb + sq * a.k_out_ss;
  const int64_t q_in_sh = a.q_in_sh, q_out_sh = a.q_out_sh;
  const int64_t k_in_sh = a.k_in_sh, k_out_sh = a.k_out_sh;
  auto task = [&](int f) {
    Task<T> k;
    const ts_plan::RopeTask rt = ts_plan::rope_head_task(f, a.tasks_per_head, a.tph_magic);
    const int hh = rt.hh;
    k.i = 0;
    k.j = rt.j;
    const bool is_q = hh < a.Hq;  // a select, not a branch (see task_at)
    const T* src_q = qi + hh * q_in_sh;
    T* dst_q = qo + hh * q_out_sh;
    const T* src_k = ki + (hh - a.Hq) * k_in_sh;
    T* dst_k = ko + (hh - a.Hq) * k_out_sh;
    k.src = is_q ? src_q : src_k;
    k.dst = is_q ? dst_q : dst_k;
    return k;
  };
  const int total = a.tasks_per_token;
  int f = threadIdx.x;
  Task<T> k0{};
  u32x4 v1{0, 0, 0, 0}, v2{0, 0, 0, 0};
  if (f < total) {
    k0 = task(f);
    task_load<T, kInterleaved>(a, k0, v1, v2);
  }
  const int64_t pos = a.position_ids != nullptr ? a.position_ids[b * a.pos_sb + sq * a.pos_ss]
                                                : sq + a.position_offset;
  for (int i = threadIdx.x; i < a.half; i += blockDim.x) {
    float c, s;
    angle_at<TabT, kTable>(a, pos, i, c, s);
    cs[i] = c;
    sn[i] = s;
  }
  __syncthreads();
  if (f < total) task_rotate_store<T, kInterleaved>(a, k0, v1, v2, cs, sn);
  for (f += blockDim.x; f < total; f += blockDim.x) {
    const Task<T> k = task(f);
    task_load<T, kInterleaved>(a, k, v1, v2);
    task_rotate_store<T, kInterleaved>(a, k, v1, v2, cs, sn);
  }
}

// Element-wise fallback: a task is one rotation pair.
template <typename T, typename TabT, bool kTable, bool kInterleaved>
__global__ __launch_bounds__(kMaxThreads) void rope_generic_kernel(const RopeArgs a) {
  extern __shared__ float lds[];
  float* cs = lds;
  float* sn = lds + a.tpb * a.half;
  const int64_t tok0 = (int64_t)blockIdx.x * a.tpb;
  fill_angles<TabT, kTable>(a, tok0, cs, sn);
  __syncthreads();
  const int64_t ntok_here = a.ntok - tok0 < a.tpb ? a.ntok - tok0 : a.tpb;
  const int total = (int)ntok_here * a.tasks_per_token;
  for (int f = threadIdx.x; f < total; f += blockDim.x) {
    const Task<T> k = task_at<T>(a, tok0, f);
    const int p = k.j;  // pair index
    const ts_plan::RopeElems el = ts_plan::rope_elems(p, 1, a.half, kInterleaved);
    const int e1 = el.e1;
    const int e2 = el.e2;
    const float x1 = Elt<T>::load1(k.src + e1);
    const float x2 = Elt<T>::load1(k.src + e2);
    const float c = cs[k.i * a.half + p];
    const float s = sn[k.i * a.half + p];
    Elt<T>::store1(k.dst + e1, rot_lo(x1, x2, c, s));
    Elt<T>::store1(k.dst + e2, rot_hi(x1, x2, c, s));
  }
}

template <typename T, typename TabT, bool kTable, bool kInterleaved>
ts_status launch_typed(RopeArgs& a, bool vec, hipStream_t st) {
  constexpr int V = sizeof(T) == 4 ? 4 : 8;
  const int ntask_head = vec ? (kInterleaved ? 2 * a.half / V : a.half / V) : a.half;
  a.tasks_per_head = ntask_head;
  a.tasks_per_token = ntask_head * (a.Hq + a.Hk);
  const ts_plan::RopeBlock blk =
      ts_plan::rope_block(a.tasks_per_token, a.half, kMaxThreads, kLdsAngles);
  a.tpb = blk.tpb;
  // Task indices stay below tpb * tasks_per_token; both divisions must be exact.
  if (!ts_plan::magic_exact((uint64_t)a.tpb * a.tasks_per_token, (uint64_t)a.tasks_per_token) ||
      !ts_plan::magic_exact((uint64_t)a.tasks_per_token, (uint64_t)a.tasks_per_head))
    return ts_host::fail(TS_ERR_SHAPE,
                         "rope: %d heads x %d tasks per head exceed the kernel's index range",
                         a.Hq + a.Hk, a.tasks_per_head);
  a.tpt_magic = ts_plan::magic_for((uint32_t)a.tasks_per_token);
  a.tph_magic = ts_plan::magic_for((uint32_t)a.tasks_per_head);
  const dim3 grid((unsigned)((a.ntok + a.tpb - 1) / a.tpb));
  const size_t lds = 2 * sizeof(float) * (size_t)a.tpb * a.half;
  if (vec && a.tpb == 1 && ts_plan::magic64_exact((uint64_t)a.ntok, (uint64_t)a.S)) {
    a.s_magic = ts_plan::magic64_for((uint64_t)a.S);
    hipLaunchKernelGGL((rope_tok_kernel<T, TabT, kTable, kInterleaved>), grid,
                       dim3(blk.threads), 0, st, a);
    return ts_host::check_launch("rope_tok_kernel");
  }
  if (vec) {
    hipLaunchKernelGGL((rope_vec_kernel<T, TabT, kTable, kInterleaved>), grid,
                       dim3(blk.threads), lds, st, a);
    return ts_host::check_launch("rope_vec_kernel");
  }
  hipLaunchKernelGGL((rope_generic_kernel<T, TabT, kTable, kInterleaved>), grid,
                     dim3(blk.threads), lds, st, a);
  return ts_host::check_launch("rope_generic_kernel");
}

template <typename T, typename TabT>
ts_status dispatch_layout(RopeArgs& a, bool table, bool interleaved, bool vec, hipStream_t st) {
  if (table) {
    return interleaved ? launch_typed<T, TabT, true, true>(a, vec, st)
                       : launch_typed<T, TabT, true, false>(a, vec, st);
  }
  return interleaved ? launch_typed<T, TabT, false, true>(a, vec, st)
                     : launch_typed<T, TabT, false, false>(a, vec, st);
}

template <typename T>
ts_status dispatch_tab(RopeArgs& a, ts_dtype tab_dtype, bool table, bool interleaved, bool vec,
                       hipStream_t st) {
  if (!table) return dispatch_layout<T, float>(a, false, interleaved, vec, st);
  switch (tab_dtype) {
    case TS_F32: return dispatch_layout<T, float>(a, true, interleaved, vec, st);
    case TS_BF16: return dispatch_layout<T, __bf16>(a, true, interleaved, vec, st);
    case TS_F16: return dispatch_layout<T, _Float16>(a, true, interleaved, vec, st);
  }
  return ts_host::fail(TS_ERR_UNSUPPORTED_DTYPE, "rope: unsupported table dtype");
}

bool strides_vec_ok(int64_t sb, int64_t ss, int64_t sh, int V) {
  return sb % V == 0 && ss % V == 0 && sh % V == 0;
}

}  // namespace

extern "C" ts_status ts_rope_apply(
    const void* q_in, void* q_out, int64_t q_in_sb, int64_t q_in_ss, int64_t q_in_sh,
    int64_t q_out_sb, int64_t q_out_ss, int64_t q_out_sh, int64_t Hq, const void* k_in,
    void* k_out, int64_t k_in_sb, int64_t k_in_ss, int64_t k_in_sh, int64_t k_out_sb,
    int64_t k_out_ss, int64_t k_out_sh, int64_t Hk, ts_dtype dtype, int64_t B, int64_t S,
    int64_t D, const void* cos_tab, const void* sin_tab, ts_dtype tab_dtype, int64_t tab_ld,
    int64_t table_rows, const float* inv_freq, float pos_div, float angle_scale,
    const int64_t* position_ids,
    int64_t pos_sb, int64_t pos_ss, int64_t position_offset, int32_t interleaved,
    int32_t backward, ts_stream_t stream) {
  using ts_host::fail;
  if (!ts_host::valid_dtype(dtype)) return fail(TS_ERR_UNSUPPORTED_DTYPE, "rope: bad dtype");
  if (B < 0 || S < 0 || Hq < 0 || Hk < 0 || D <= 0)
    return fail(TS_ERR_SHAPE, "rope: bad shape B=%lld S=%lld Hq=%lld Hk=%lld D=%lld",
                (long long)B, (long long)S, (long long)Hq, (long long)Hk, (long long)D);
  if (D % 2 != 0 || D / 2 > kMaxHalf)
    return fail(TS_ERR_SHAPE, "rope: head_dim must be even and <= %d (got %lld)", 2 * kMaxHalf,
                (long long)D);
  if (Hq + Hk > 4096) return fail(TS_ERR_SHAPE, "rope: more than 4096 heads per token");
  // Tensors without tokens may have NULL data pointers (torch gives empty
  // tensors none); nothing is read or written for them.
  const bool any_tokens = B > 0 && S > 0;
  if (any_tokens && Hq > 0 && (q_in == nullptr || q_out == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "rope: q pointers are NULL");
  if (any_tokens && Hk > 0 && (k_in == nullptr || k_out == nullptr))
    return fail(TS_ERR_INVALID_ARGUMENT, "rope: k pointers are NULL");
  if (interleaved != 0 && interleaved != 1)
    return fail(TS_ERR_INVALID_ARGUMENT, "rope: interleaved must be 0 or 1");
  if (backward != 0 && backward != 1)
    return fail(TS_ERR_INVALID_ARGUMENT, "rope: backward must be 0 or 1");
  const bool table = cos_tab != nullptr || sin_tab != nullptr;
  if (table) {
    if (cos_tab == nullptr || sin_tab == nullptr)
      return fail(TS_ERR_INVALID_ARGUMENT, "rope: cos and sin tables must both be given");
    if (!ts_host::valid_dtype(tab_dtype))
      return fail(TS_ERR_UNSUPPORTED_DTYPE, "rope: bad table dtype");
    if (tab_ld < D / 2 || table_rows <= 0)
      return fail(TS_ERR_SHAPE, "rope: table must be [rows > 0, >= D/2] (ld=%lld rows=%lld)",
                  (long long)tab_ld, (long long)table_rows);
    if (position_ids == nullptr && S > 0 &&
        (position_offset < 0 || position_offset + S > table_rows))
      return fail(TS_ERR_SHAPE,
                  "rope: positions [%lld, %lld) exceed the %lld-row cos/sin table",
                  (long long)position_offset, (long long)(position_offset + S),
                  (long long)table_rows);
  } else {
    if (inv_freq == nullptr)
      return fail(TS_ERR_INVALID_ARGUMENT, "rope: need cos/sin tables or inv_freq");
    if (!(pos_div > 0.f)) return fail(TS_ERR_INVALID_ARGUMENT, "rope: pos_div must be > 0");
    if (!(angle_scale > 0.f) || !__builtin_isfinite(angle_scale))
      return fail(TS_ERR_INVALID_ARGUMENT, "rope: angle_scale must be finite and > 0");
  }
  const int64_t ntok = B * S;
  if (ntok == 0 || Hq + Hk == 0) return TS_OK;
  if (ntok > ((int64_t)1 << 40)) return fail(TS_ERR_SHAPE, "rope: too many tokens");

  RopeArgs a{};
  a.q_in = q_in; a.q_out = q_out;
  a.q_in_sb = q_in_sb; a.q_in_ss = q_in_ss; a.q_in_sh = q_in_sh;
  a.q_out_sb = q_out_sb; a.q_out_ss = q_out_ss; a.q_out_sh = q_out_sh;
  a.k_in = k_in; a.k_out = k_out;
  a.k_in_sb = k_in_sb; a.k_in_ss = k_in_ss; a.k_in_sh = k_in_sh;
  a.k_out_sb = k_out_sb; a.k_out_ss = k_out_ss; a.k_out_sh = k_out_sh;
  a.Hq = (int32_t)Hq; a.Hk = (int32_t)Hk;
  a.S = S; a.ntok = ntok; a.half = (int32_t)(D / 2);
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.tab_ld = tab_ld; a.table_rows = table_rows;
  a.pos_div = pos_div > 0.f ? pos_div : 1.f;
  a.angle_scale = table ? 1.f : angle_scale;
  a.position_ids = position_ids; a.pos_sb = pos_sb; a.pos_ss = pos_ss;
  a.position_offset = position_offset;
  a.backward = backward;
  if (!table) {
    for (int i = 0; i < a.half; ++i) a.inv_freq[i] = inv_freq[i];
  }

  const int V = dtype == TS_F32 ? 4 : 8;
  bool vec = (a.half % V) == 0;
  if (Hq > 0) {
    vec = vec && ts_host::aligned16(q_in) && ts_host::aligned16(q_out) &&
          strides_vec_ok(q_in_sb, q_in_ss, q_in_sh, V) &&
          strides_vec_ok(q_out_sb, q_out_ss, q_out_sh, V);
  }
  if (Hk > 0) {
    vec = vec && ts_host::aligned16(k_in) && ts_host::aligned16(k_out) &&
          strides_vec_ok(k_in_sb, k_in_ss, k_in_sh, V) &&
          strides_vec_ok(k_out_sb, k_out_ss, k_out_sh, V);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool il = interleaved != 0;
  switch (dtype) {
    case TS_BF16: return dispatch_tab<__bf16>(a, tab_dtype, table, il, vec, st);
    case TS_F16: return dispatch_tab<_Float16>(a, tab_dtype, table, il, vec, st);
    case TS_F32: return dispatch_tab<float>(a, tab_dtype, table, il, vec, st);
  }
  return fail(TS_ERR_UNSUPPORTED_DTYPE, "rope: bad dtype");
}
