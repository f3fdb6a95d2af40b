// Launch planning shared by the C-ABI size queries and the kernel launches.
//
// Plain C++ with no HIP dependency, so the host-side bounds arithmetic can be
// compiled and checked on a machine without a GPU. Every quantity a launch
// writes to caller memory (number of dW partial rows, grid sizes) comes from
// these functions, and the workspace size reported to the caller is the
// maximum over every plan the launch may pick for the same (rows, cols).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define TS_HOST_DEVICE __host__ __device__
#else
#define TS_HOST_DEVICE
#endif

namespace ts_plan {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// RMSNorm
//
// Register path: a row is owned by `tpr` threads (a power of two, whole
// waves), each holding `kv` 16-byte vectors spaced tpr vectors apart, so one
// load instruction of a wave covers 1 KiB of contiguous row. A workgroup holds
// rpb = block / tpr rows at a time. Few vectors per thread and many small
// workgroups keep the HBM queues full; loops over many vectors per thread do
// not (measured on MI355X: one 16-byte load per thread copies at ~6.4 TB/s,
// eight per thread at ~4.2 TB/s).
//
// Backward: each workgroup walks up to `steps` row groups spaced `grid` apart
// (grid * steps >= the number of row groups) and keeps the dW contributions
// of its threads' columns in registers; it writes rpb fp32 partial rows at
// the end, which a second kernel sums in a fixed order.
// ---------------------------------------------------------------------------
constexpr int kMaxKv = 4;                 // vectors per thread on the register path
// Backward workgroups, 2 per CU on 256 CUs (measured on MI355X at
// [16384, 4096]: 256, 1024 and 2048 workgroups were all slower).
constexpr int64_t kBwdGridTarget = 512;
constexpr int64_t kGenericRowsPerGroup = 64;

// Elements per 16-byte vector.
inline int vec_elems(int elt_bytes) { return 16 / elt_bytes; }

struct RmsRowPlan {
  bool reg;    // register path possible
  int tpr;     // threads per row (64..512)
  int kv;      // vectors per thread (1, 2 or 4)
  int block;   // threads per workgroup
  int rpb;     // rows per workgroup step (block / tpr)
};

// Forward: two vectors per thread where the row allows it.
inline RmsRowPlan rms_fwd_plan(int64_t nvec) {
  RmsRowPlan p{false, 0, 0, 0, 0};
  if (nvec <= 0 || nvec > 512 * kMaxKv) return p;
  if (nvec <= 64) { p.tpr = 64; p.kv = 1; }
  else if (nvec <= 128) { p.tpr = 64; p.kv = 2; }
  else if (nvec <= 256) { p.tpr = 128; p.kv = 2; }
  else if (nvec <= 512) { p.tpr = 256; p.kv = 2; }
  else if (nvec <= 1024) { p.tpr = 512; p.kv = 2; }
  else { p.tpr = 512; p.kv = 4; }
  p.reg = true;
  p.block = p.tpr > 256 ? p.tpr : 256;
  p.rpb = p.block / p.tpr;
  return p;
}

// Backward: one vector per thread where the row allows it (x and dy are both
// read, so a thread already has two loads in flight).
inline RmsRowPlan rms_bwd_row_plan(int64_t nvec) {
  RmsRowPlan p{false, 0, 0, 0, 0};
  if (nvec <= 0 || nvec > 512 * kMaxKv) return p;
  if (nvec <= 64) { p.tpr = 64; p.kv = 1; }
  else if (nvec <= 128) { p.tpr = 128; p.kv = 1; }
  else if (nvec <= 256) { p.tpr = 256; p.kv = 1; }
  else if (nvec <= 512) { p.tpr = 512; p.kv = 1; }
  else if (nvec <= 1024) { p.tpr = 512; p.kv = 2; }
  else { p.tpr = 512; p.kv = 4; }
  p.reg = true;
  p.block = 512;
  p.rpb = p.block / p.tpr;
  return p;
}

// Backward, one wave per row (rms_bwd_wave): rows of 65..256 vectors, kv = 2
// or 4 vectors per lane, kWaveRowsPerBlock waves (rows) per workgroup step.
// The row's sum is a wave reduction (no LDS, no barrier), and each lane has
// 2 kv loads in flight; the workgroup sums its waves' dW in LDS once at the
// end and writes one partial row. Measured on MI355X against the workgroup-
// per-row kernel (rms_bwd_reg): [16384, 2048] bf16 42.0 against 48.1 us,
// [16384, 1024] 35.5 against 36.6 us; at [16384, 4096] (8 vectors per lane,
// 233 VGPRs) it was slower, 80.4 against 74.7 us, so longer rows keep
// rms_bwd_reg.
constexpr int64_t kWaveRowMinVec = 65;
constexpr int64_t kWaveRowMaxVec = 256;
constexpr int kWaveRowsPerBlock = 4;

inline RmsRowPlan rms_bwd_wave_plan(int64_t nvec) {
  RmsRowPlan p{false, 0, 0, 0, 0};
  if (nvec < kWaveRowMinVec || nvec > kWaveRowMaxVec) return p;
  p.tpr = 64;
  p.kv = nvec <= 128 ? 2 : 4;
  p.reg = true;
  p.block = 64 * kWaveRowsPerBlock;
  p.rpb = kWaveRowsPerBlock;
  return p;
}

struct RmsBwdPlan {
  bool reg;        // register path (else the generic element-wise kernels)
  bool wave;       // register path with one wave per row (rms_bwd_wave)
  RmsRowPlan row;  // register-path shape
  int64_t steps;   // row groups (of rpb rows) per workgroup
  int64_t grid;    // workgroups of the dx kernel
  int64_t nparts;  // dW partial rows written (== rows of fp32 workspace used)
};

// `vec_ok` says whether pointers and strides allow 16-byte access.
inline RmsBwdPlan rms_bwd_plan(int64_t rows, int64_t cols, int elt_bytes, bool vec_ok,
                               bool need_dw) {
  RmsBwdPlan p{false, false, RmsRowPlan{false, 0, 0, 0, 0}, 0, 0, 0};
  const int V = vec_elems(elt_bytes);
  if (vec_ok && cols % V == 0) {
    p.row = rms_bwd_wave_plan(cols / V);
    p.wave = p.row.reg;
    if (!p.wave) p.row = rms_bwd_row_plan(cols / V);
  }
  p.reg = p.row.reg;
  if (p.reg) {
    const int64_t groups = (rows + p.row.rpb - 1) / p.row.rpb;
    int64_t steps = (groups + kBwdGridTarget - 1) / kBwdGridTarget;
    if (steps < 1) steps = 1;
    p.steps = steps;
    p.grid = (groups + steps - 1) / steps;
    // the wave kernel sums its rows' dW in LDS: one partial row per workgroup
    p.nparts = need_dw ? (p.wave ? p.grid : p.grid * p.row.rpb) : 0;
  } else {
    p.steps = 0;
    p.grid = rows;
    p.nparts = need_dw ? (rows + kGenericRowsPerGroup - 1) / kGenericRowsPerGroup : 0;
  }
  return p;
}

// Element offset, from the start of a [rows, ld] matrix, of the k-th 16-byte
// vector (V elements) that lane t of a backward row slot loads at step st:
// the slot's first row is row0, consecutive steps are rstep rows apart, and a
// row has nvec vectors. A lane with nothing to load there (a step past
// `steps`, a row past the matrix, a vector past the row) gets offset 0, the
// matrix's first element, so every load of the kernel stays inside the matrix.
TS_HOST_DEVICE inline int64_t rms_bwd_load_offset(int64_t row0, int64_t st, int64_t rstep,
                                                  int64_t steps, int64_t rows, int t, int k,
                                                  int tpr, int V, int64_t nvec, int64_t ld) {
  const int64_t row = row0 + st * rstep;
  const int64_t v = (int64_t)t + (int64_t)k * tpr;
  const bool ok = st < steps && row < rows && v < nvec;
  return ok ? row * ld + v * V : 0;
}

// The row that a wave-per-row backward slot (rms_bwd_wave) touches at step
// st, for a [rows, ld] matrix: the element offset of the row and its bytes
// (row_bytes), or {0, 0} for a step past `steps` or a row past the matrix. The
// kernel builds a buffer resource on it, so its accesses can only reach that
// row, or nothing (the hardware drops stores and zero-fills loads outside).
struct RowSpan {
  int64_t offset;
  uint32_t bytes;
};
TS_HOST_DEVICE inline RowSpan rms_bwd_wave_row(int64_t row0, int64_t st, int64_t rstep,
                                               int64_t steps, int64_t rows, int64_t ld,
                                               uint32_t row_bytes) {
  const int64_t row = row0 + st * rstep;
  const bool ok = st < steps && row < rows;
  return ok ? RowSpan{row * ld, row_bytes} : RowSpan{0, 0u};
}

// Rows of fp32 dW partials any backward launch for (rows, cols) may write:
// the maximum over element sizes 2 and 4 and over both paths.
inline int64_t rms_bwd_workspace_rows(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  int64_t m = 0;
  for (int e = 0; e < 4; ++e) {
    const RmsBwdPlan p = rms_bwd_plan(rows, cols, (e & 1) ? 4 : 2, (e & 2) != 0, true);
    if (p.nparts > m) m = p.nparts;
  }
  return m;
}

// ---------------------------------------------------------------------------
// RoPE workgroup shape: about one thread per task (a task is a 16-byte vector
// pair of one head, or one pair on the generic path), whole waves, at least
// 256 threads, at most max_threads; `tpb` tokens per workgroup, bounded so the
// cos/sin staging (tpb * half floats each) fits max_angles.
// ---------------------------------------------------------------------------
struct RopeBlock {
  int tpb;      // tokens per workgroup
  int threads;  // threads per workgroup (multiple of 64)
};

inline RopeBlock rope_block(int64_t tasks_per_token, int half, int max_threads, int max_angles) {
  RopeBlock b{1, 64};
  int64_t tpb = tasks_per_token >= 256 ? 1 : 256 / (tasks_per_token > 0 ? tasks_per_token : 1);
  const int64_t cap = max_angles / (half > 0 ? half : 1);
  if (tpb > cap) tpb = cap;
  if (tpb < 1) tpb = 1;
  int64_t threads = tpb * tasks_per_token;
  threads = (threads + kWave - 1) / kWave * kWave;
  if (threads < 256) threads = 256;
  if (threads > max_threads) threads = max_threads;
  b.tpb = (int)tpb;
  b.threads = (int)threads;
  return b;
}

// ---------------------------------------------------------------------------
// Magic-number division used by the RoPE task decomposition:
// q = umulhi(n, ceil(2^32 / d)) equals n / d whenever n * d < 2^32 and d > 1.
// ceil(2^32 / 1) does not fit 32 bits, so d == 1 is encoded as magic 0 and
// divides by returning n. The kernels divide with magic_div too.
// ---------------------------------------------------------------------------
inline uint32_t magic_for(uint32_t d) {
  return d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + d - 1) / d);
}
TS_HOST_DEVICE inline uint32_t magic_div(uint32_t n, uint32_t magic) {
#if defined(__HIP_DEVICE_COMPILE__)
  return magic == 0 ? n : __umulhi(n, magic);
#else
  return magic == 0 ? n : (uint32_t)(((uint64_t)n * magic) >> 32);
#endif
}
inline bool magic_exact(uint64_t n_max, uint64_t d) { return n_max * d < ((uint64_t)1 << 32); }

// The same rule one size up, for the RoPE token -> (batch, position) split:
// q = mulhi64(n, ceil(2^64 / d)) equals n / d whenever n * d < 2^64 and d > 1
// (with m = (2^64 + e) / d, 0 <= e < d, the error term n * e / (d * 2^64)
// stays below 1 / d, which cannot carry floor(n / d) over an integer).
inline uint64_t magic64_for(uint64_t d) {
  return d <= 1 ? 0u : (uint64_t)((((unsigned __int128)1 << 64) + d - 1) / d);
}
inline uint64_t magic64_div(uint64_t n, uint64_t magic) {
  return magic == 0 ? n : (uint64_t)(((unsigned __int128)n * magic) >> 64);
}
inline bool magic64_exact(uint64_t n_max, uint64_t d) {
  return (unsigned __int128)n_max * d < ((unsigned __int128)1 << 64);
}

// ---------------------------------------------------------------------------
// GEMM tile order. The dispatcher sends workgroup `bid` to XCD bid % 8, and
// each XCD has its own L2. Workgroups are first renumbered so that each XCD
// gets one contiguous range of logical tiles (XCD x takes the x-th eighth),
// and logical tiles run in groups of kGemmGroupM M-tiles with M-tiles
// varying fastest, then N-tiles. The 32 workgroups an XCD holds at a time
// then cover about 4 M-tiles x 8 N-tiles, whose operand panels its L2
// shares. Measured on MI355X at the fused linear-CE shapes (random bf16
// data): 4-11% faster than the same grouping without the XCD renumbering
// and 16 M-tiles per group.
// ---------------------------------------------------------------------------
constexpr int64_t kGemmGroupM = 4;
constexpr int64_t kXcds = 8;

TS_HOST_DEVICE inline void gemm_tile_of(int64_t bid, int64_t MT, int64_t NT, int64_t& mt,
                                        int64_t& nt) {
  const int64_t T = MT * NT;
  const int64_t x = bid % kXcds, i = bid / kXcds, q = T / kXcds, r = T % kXcds;
  const int64_t t = x * q + (x < r ? x : r) + i;  // logical tile
  const int64_t per_group = kGemmGroupM * NT;
  const int64_t g = t / per_group;
  const int64_t w = t - g * per_group;
  const int64_t gm = MT - g * kGemmGroupM < kGemmGroupM ? MT - g * kGemmGroupM : kGemmGroupM;
  mt = g * kGemmGroupM + w % gm;
  nt = w / gm;
}

// ---------------------------------------------------------------------------
// Addressing of the streaming and row kernels. The kernels compute their
// accesses with these functions, and tests/test_plan.py sweeps them with the
// launch shapes the host computes: every access lies inside its tensor and
// every element is visited once.
// ---------------------------------------------------------------------------

// Vector index that thread tid handles as its k-th vector of chunk c, for chunks
// of threads * kv consecutive 16-byte vectors whose k-th vectors lie `threads`
// apart (one wave's load instruction then covers 1 KiB of consecutive memory).
// Kernels touch it only when it is < the vector count.
TS_HOST_DEVICE inline int64_t chunk_vec(int64_t c, int k, int tid, int threads, int kv) {
  return c * threads * kv + tid + (int64_t)k * threads;
}

// Chunks of threads * kv vectors that cover nvec vectors.
TS_HOST_DEVICE inline int64_t chunks_for(int64_t nvec, int threads, int kv) {
  const int64_t per = (int64_t)threads * kv;
  return (nvec + per - 1) / per;
}

// Whether 16-byte vector v of row `row` lies inside a matrix of `rows` rows of
// nvec vectors (row and v are non-negative by construction); a kernel then
// accesses row * ld + v * V elements from the matrix's start.
TS_HOST_DEVICE inline bool row_vec_in(int64_t row, int64_t rows, int64_t v, int64_t nvec) {
  return row < rows && v < nvec;
}

// Byte offset of vector v for a buffer resource spanning nvec vectors of
// vec_bytes each, or kNoAccess past them: an offset no resource of this size
// covers (bit pattern 0x80000000), so the hardware drops the store or returns
// zeros. Requires nvec * vec_bytes < 2^31 (the hosts check).
constexpr int32_t kNoAccess = (int32_t)(-2147483647 - 1);
TS_HOST_DEVICE inline int32_t vec_boffset(int64_t v, int64_t nvec, int vec_bytes) {
  return v >= 0 && v < nvec ? (int32_t)(v * vec_bytes) : kNoAccess;
}

// Row owned by wave `wave` of workgroup `block` in a one-wave-per-row kernel
// with `waves` row waves per workgroup (flce_rows); such a kernel returns,
// wave-uniformly, for rows at or past its row count.
TS_HOST_DEVICE inline int64_t wave_row(int64_t block, int wave, int waves) {
  return block * waves + wave;
}
// Workgroups of `waves` row waves that cover `rows` rows.
TS_HOST_DEVICE inline int64_t wave_row_blocks(int64_t rows, int waves) {
  return (rows + waves - 1) / waves;
}

// A row's label as a column of its logits: the label itself when 0 <= label < V;
// kLabelIgnored for ignore_index (the row reads nothing and its loss is 0);
// kLabelOutside for any other label (nothing is read; the row's loss is NaN).
constexpr int64_t kLabelIgnored = -1;
constexpr int64_t kLabelOutside = -2;
TS_HOST_DEVICE inline int64_t label_col(int64_t label, int64_t V, int64_t ignore_index) {
  if (label == ignore_index) return kLabelIgnored;
  return label >= 0 && label < V ? label : kLabelOutside;
}
// The label's column in the vocabulary shard [vocab_start, vocab_start + Vp)
// (vocab_start >= 0), or kLabelOutside when the shard does not hold it.
TS_HOST_DEVICE inline int64_t shard_col(int64_t label, int64_t vocab_start, int64_t Vp) {
  return label >= vocab_start && label - vocab_start < Vp ? label - vocab_start : kLabelOutside;
}

// A RoPE task f of a workgroup: token slot i (0 .. tpb - 1), head hh (Q heads,
// then K heads) and j, its index within the head (a 16-byte vector pair on the
// vector path, a rotation pair on the generic path). The divisions are
// magic-number ones (magic_div), exact whenever f < tpb * tasks_per_token and
// the host's magic_exact checks hold.
struct RopeTask {
  int i, hh, j;
};
// Head and index within the head of task r of one token.
TS_HOST_DEVICE inline RopeTask rope_head_task(int r, int tasks_per_head, uint32_t tph_magic) {
  RopeTask t;
  t.i = 0;
  t.hh = (int)magic_div((uint32_t)r, tph_magic);
  t.j = r - t.hh * tasks_per_head;
  return t;
}
TS_HOST_DEVICE inline RopeTask rope_task(int f, int tasks_per_token, uint32_t tpt_magic,
                                         int tasks_per_head, uint32_t tph_magic) {
  const int i = (int)magic_div((uint32_t)f, tpt_magic);
  RopeTask t = rope_head_task(f - i * tasks_per_token, tasks_per_head, tph_magic);
  t.i = i;
  return t;
}

// Element offsets within its head of the two vectors (or elements) a RoPE task
// reads and writes: NeoX pairs (e, e + half), interleaved adjacent pairs in one
// vector (e2 unused, -1). `width` is the vector width (1 on the generic path).
struct RopeElems {
  int e1, e2;
};
TS_HOST_DEVICE inline RopeElems rope_elems(int j, int width, int half, bool interleaved) {
  if (width == 1) return interleaved ? RopeElems{2 * j, 2 * j + 1} : RopeElems{j, j + half};
  return interleaved ? RopeElems{j * width, -1} : RopeElems{j * width, half + j * width};
}

}  // namespace ts_plan
