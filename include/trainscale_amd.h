/*
 * trainscale_amd.h — C ABI of the MI355X (gfx950) fused kernel layer.
 *
 * Every entry point takes caller-owned device buffers as plain pointers, sizes
 * and strides counted in ELEMENTS, and the HIP stream to launch on. Nothing here
 * allocates device memory; scratch space is passed in as a workspace buffer whose
 * size the matching *_workspace_size() function reports. Launches are
 * asynchronous on `stream` and never synchronise. Every function returns a
 * ts_status; on failure ts_last_error() describes the problem (thread-local).
 *
 * Arguments are validated on the host before anything touches the GPU, so a bad
 * call returns an error code instead of launching.
 *
 * Each declaration cites the reference interface it replaces
 * (paths relative to generalaimodels/TrainScale, data_pipeline/trainer/).
 */
#ifndef TRAINSCALE_AMD_H
#define TRAINSCALE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ts_stream_t; /* a hipStream_t; NULL is the legacy default stream */

typedef int32_t ts_status;
enum {
  TS_OK = 0,
  TS_ERR_INVALID_ARGUMENT = -1, /* NULL pointer, negative size, bad flag */
  TS_ERR_UNSUPPORTED_DTYPE = -2,
  TS_ERR_SHAPE = -3,            /* inconsistent sizes / strides */
  TS_ERR_WORKSPACE = -4,        /* workspace missing or too small */
  TS_ERR_LAUNCH = -5,           /* the HIP runtime rejected a launch */
  TS_ERR_DEVICE = -6            /* device query failed */
};

typedef enum {
  TS_F32 = 0,
  TS_BF16 = 1,
  TS_F16 = 2
} ts_dtype;

/* Human-readable description of the last error raised on this thread. */
const char* ts_last_error(void);
/* Library version string, e.g. "trainscale_amd 0.1.0 gfx950". */
const char* ts_version(void);

/* ------------------------------------------------------------------------ */
/* RMSNorm                                                                   */
/* ------------------------------------------------------------------------ */

/* round_mode for ts_rmsnorm_fwd */
enum {
  /* y = round(x * rstd * w) in fp32, rounded once.
   * Replaces _rms_layernorm_forward_kernel, kernels/triton_kernels.py:477-514,
   * launched by Fast_RMS_LayerNorm.forward, triton_kernels.py:605-643. */
  TS_RMS_ROUND_ONCE = 0,
  /* y = round(round(x * rstd) * w) when w has the data dtype (bf16/fp16),
   * otherwise identical to ROUND_ONCE.
   * Replaces _rms_layernorm_forward_kernel, kernels/layernorm_kernels.py:143-199
   * (y = x_norm.to(w.dtype) * w), launched by RMSLayerNormFunction.forward,
   * layernorm_kernels.py:686-750. */
  TS_RMS_ROUND_TWICE = 1
};

/*
 * y[r, :] = x[r, :] * rstd[r] * w,   rstd[r] = 1 / sqrt(mean(x[r, :]^2) + eps)
 * x, y: [rows, cols] of x_dtype with row strides ldx, ldy (elements).
 * w: [cols] of w_dtype, or NULL for no weight (elementwise_affine=False).
 * rstd: [rows] fp32, written (saved for the backward pass).
 */
ts_status ts_rmsnorm_fwd(const void* x, int64_t ldx, ts_dtype x_dtype,
                         const void* w, ts_dtype w_dtype,
                         void* y, int64_t ldy,
                         float* rstd,
                         int64_t rows, int64_t cols, float eps,
                         int32_t round_mode, ts_stream_t stream);

/*
 * Fused residual add + RMSNorm:
 *   h = x + residual (fp32),  rstd[r] = 1 / sqrt(mean(h[r, :]^2) + eps),
 *   y = h * rstd * w with round_mode as in ts_rmsnorm_fwd,
 *   h_out = h rounded to x_dtype when h_out is not NULL.
 * x, residual, y, h_out: [rows, cols] of x_dtype with row strides ldx, ldr,
 * ldy, ldh. rstd comes from the unrounded h; the backward pass is
 * ts_rmsnorm_bwd with x = h_out (the rounded h, as the reference saves it).
 * Replaces _fused_add_rms_layernorm_kernel, kernels/layernorm_kernels.py:495-552,
 * launched by FusedAddRMSLayerNormFunction.forward, layernorm_kernels.py:957-1009
 * (which uses round-twice numerics: y = h_norm.to(w.dtype) * w).
 */
ts_status ts_add_rmsnorm_fwd(const void* x, int64_t ldx,
                             const void* residual, int64_t ldr, ts_dtype x_dtype,
                             const void* w, ts_dtype w_dtype,
                             void* y, int64_t ldy,
                             void* h_out, int64_t ldh,
                             float* rstd,
                             int64_t rows, int64_t cols, float eps,
                             int32_t round_mode, ts_stream_t stream);

/* Bytes of workspace ts_rmsnorm_bwd needs for these sizes (dW partial sums). */
size_t ts_rmsnorm_bwd_workspace_size(int64_t rows, int64_t cols);

/*
 * dx = rstd * (dy*w - xhat * mean(dy*w*xhat)),  xhat = x * rstd
 * dw = sum_rows(dy * xhat), accumulated in fp32 in a fixed order
 *      (deterministic: per-workgroup partials, then an ordered column sum).
 * dy, x, dx: [rows, cols] of x_dtype, row strides lddy, ldx, lddx.
 * w: [cols] of w_dtype or NULL. dw: [cols] of w_dtype, or NULL to skip dW.
 * Replaces _rms_layernorm_backward_kernel + _rms_layernorm_backward_dw_kernel,
 * kernels/triton_kernels.py:517-599 (Fast_RMS_LayerNorm.backward :646-684) and
 * _rms_layernorm_backward_dx_kernel + _rms_layernorm_backward_dw_kernel,
 * kernels/layernorm_kernels.py:203-308 (RMSLayerNormFunction.backward :752-807).
 */
ts_status ts_rmsnorm_bwd(const void* dy, int64_t lddy,
                         const void* x, int64_t ldx, ts_dtype x_dtype,
                         const void* w, ts_dtype w_dtype,
                         const float* rstd,
                         void* dx, int64_t lddx,
                         void* dw,
                         void* workspace, size_t workspace_bytes,
                         int64_t rows, int64_t cols, ts_stream_t stream);

/*
 * ts_rmsnorm_bwd without a workspace and without allocating: the dW partial
 * rows go to a device scratch array of ts_rmsnorm_bwd_noalloc_max_bytes()
 * bytes (16 MiB: C1 [16384, 4096] and C4 [32768, 8192] in bf16 fit) that the
 * library holds on every device it runs on until the process ends. Same
 * arguments, results and kernels as ts_rmsnorm_bwd. Calls whose partials
 * would not fit (ts_rmsnorm_bwd_workspace_size > the maximum) return
 * TS_ERR_WORKSPACE before launching anything. Every call on one device
 * shares that device's scratch, so calls that overlap on one device (two
 * streams, or two threads) race; calls in one stream are ordered. The
 * device of `stream` must be the current device. The first call on a device
 * looks the scratch array's address up there (hipGetSymbolAddress); a caller
 * that captures the call in a graph makes one call on that device outside the
 * capture first (torch.cuda.graph's warm-up is such a call).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).
 */
size_t ts_rmsnorm_bwd_noalloc_max_bytes(void);
ts_status ts_rmsnorm_bwd_noalloc(const void* dy, int64_t lddy,
                                 const void* x, int64_t ldx, ts_dtype x_dtype,
                                 const void* w, ts_dtype w_dtype,
                                 const float* rstd,
                                 void* dx, int64_t lddx,
                                 void* dw,
                                 int64_t rows, int64_t cols, ts_stream_t stream);

/* ------------------------------------------------------------------------ */
/* SwiGLU                                                                    */
/* ------------------------------------------------------------------------ */

/*
 * out = round(round(silu(gate)) * up),  silu(g) = g * sigmoid(g), fp32 math,
 * over n contiguous elements of dtype (silu is rounded to the data type
 * before the product, as the reference does).
 * Replaces _swiglu_forward_kernel, kernels/triton_kernels.py:1042-1067,
 * launched by Fast_SwiGLU.forward, triton_kernels.py:1108-1127.
 */
ts_status ts_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n,
                        ts_dtype dtype, ts_stream_t stream);

/*
 * dgate = dout * up * sigmoid(g) * (1 + g * (1 - sigmoid(g))),
 * dup = dout * silu(g), fp32 math, over n contiguous elements.
 * Replaces _swiglu_backward_kernel, kernels/triton_kernels.py:1069-1101,
 * launched by Fast_SwiGLU.backward, triton_kernels.py:1129-1143.
 */
ts_status ts_swiglu_bwd(const void* dout, const void* gate, const void* up,
                        void* dgate, void* dup, int64_t n, ts_dtype dtype,
                        ts_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Rotary position embedding                                                 */
/* ------------------------------------------------------------------------ */

/*
 * Rotates the head_dim pairs of up to two [B, S, H, D] tensors ("q" and "k") at
 * positions pos(b, s). The last dimension must be contiguous; other strides are
 * free. in == out rotates in place.
 *
 *   NeoX layout (interleaved=0): pairs (i, i + D/2);  interleaved=1: (2i, 2i+1)
 *   forward:  o1 = x1*cos - x2*sin,  o2 = x2*cos + x1*sin
 *   backward: the same with sin negated (the transpose rotation)
 *
 * pos(b, s) = position_ids[b*pos_sb + s*pos_ss] when position_ids != NULL
 *             (int64, device), else s + position_offset.
 *
 * Angle source, exactly one of:
 *   - tables: cos_tab/sin_tab != NULL, [table_rows, D/2] of tab_dtype with row
 *     stride tab_ld; cos/sin are read at row pos. Positions outside
 *     [0, table_rows) produce NaN outputs for that token instead of a fault.
 *   - in-register: cos_tab == sin_tab == NULL, inv_freq = HOST array of D/2
 *     fp32 values; angle_i = fp32(pos / pos_div) * inv_freq[i] (the fp32
 *     product torch.outer forms), then multiplied by angle_scale when that is
 *     not 1 (YaRN's mscale, kernels/rope_kernels.py:181-184: freqs * mscale),
 *     and sin/cos are evaluated on the GPU. angle_scale is ignored with tables.
 *
 * Replaces _rope_forward_kernel/_rope_backward_kernel (kernels/triton_kernels.py
 * :713-890, Fast_RoPE :893-981), _rope_fwd_kernel/_rope_bwd_kernel,
 * _rope_single_tensor_kernel and _rope_with_position_ids_kernel
 * (kernels/rope_kernels.py:385-804, launched by :837-951).
 * k may be NULL (Hk = 0) for the single-tensor forms.
 */
ts_status ts_rope_apply(const void* q_in, void* q_out,
                        int64_t q_in_sb, int64_t q_in_ss, int64_t q_in_sh,
                        int64_t q_out_sb, int64_t q_out_ss, int64_t q_out_sh,
                        int64_t Hq,
                        const void* k_in, void* k_out,
                        int64_t k_in_sb, int64_t k_in_ss, int64_t k_in_sh,
                        int64_t k_out_sb, int64_t k_out_ss, int64_t k_out_sh,
                        int64_t Hk,
                        ts_dtype dtype, int64_t B, int64_t S, int64_t D,
                        const void* cos_tab, const void* sin_tab,
                        ts_dtype tab_dtype, int64_t tab_ld, int64_t table_rows,
                        const float* inv_freq, float pos_div, float angle_scale,
                        const int64_t* position_ids, int64_t pos_sb, int64_t pos_ss,
                        int64_t position_offset,
                        int32_t interleaved, int32_t backward,
                        ts_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Cross-entropy over the vocabulary                                         */
/* ------------------------------------------------------------------------ */

/*
 * Per row r of logits [N, V] (row stride ld, dtype any of f32/bf16/f16):
 *   z = logit_scale != 0 ? logit_scale * x : x
 *   z = softcap != 0 ? softcap * tanh(z / softcap) : z
 *   lse[r] = log(sum_j exp(z_j))                      (fp32, online max)
 *   loss[r] = (1-a)*(lse - z[label]) + a*(lse - mean_j z_j), a = label_smoothing
 *   loss[r] = 0 and lse[r] = 0 when labels[r] == ignore_index (the row is not read).
 * labels: int64 [N], device. Labels outside [0, V) other than ignore_index
 * give loss NaN for that row.
 * Replaces _cross_entropy_forward_kernel/_chunked_cross_entropy_forward_kernel
 * (kernels/triton_kernels.py:122-235, Fast_CrossEntropyLoss.forward :320-397),
 * _fused_cross_entropy_fwd_kernel (loss/sota_losses.py:135-228) and
 * cross_entropy_fwd_kernel (loss/__init__.py:41-123).
 */
ts_status ts_ce_fwd(const void* logits, int64_t ld, ts_dtype dtype,
                    const int64_t* labels, int64_t N, int64_t V,
                    int64_t ignore_index, float logit_scale, float softcap,
                    float label_smoothing,
                    float* loss, float* lse, ts_stream_t stream);

/*
 * grad[r, j] = dloss[r] * dz/dx * (softmax(z)_j - (1-a)*[j == label] - a/V)
 * with dloss[r] = dloss_ptr[r * dloss_stride] * dloss_scale (stride 0
 * broadcasts one value) and grad = 0 on rows whose label is ignore_index.
 * grad may alias logits (in place, as the reference writes the gradient into
 * the saved logits buffer); grad has its own row stride ld_grad and dtype.
 * Replaces _cross_entropy_backward_kernel (kernels/triton_kernels.py:238-306,
 * Fast_CrossEntropyLoss.backward :400-424) and _fused_cross_entropy_bwd_kernel
 * (loss/sota_losses.py:230-289).
 */
ts_status ts_ce_bwd(const void* logits, int64_t ld, ts_dtype dtype,
                    const int64_t* labels, const float* lse,
                    const float* dloss, int64_t dloss_stride, float dloss_scale,
                    void* grad, int64_t ld_grad, ts_dtype grad_dtype,
                    int64_t N, int64_t V, int64_t ignore_index,
                    float logit_scale, float softcap, float label_smoothing,
                    ts_stream_t stream);

/*
 * ts_ce_fwd and ts_ce_bwd in one pass when the upstream gradient is known at
 * forward time (dloss as for ts_ce_bwd): loss[r], lse[r] and grad as those two
 * functions define them. Each valid row is read once and every row of grad
 * written once while a row of up to 1024 * 16 16-byte vectors (V <= 131072
 * for bf16) fits one workgroup's registers; longer rows run the two calls.
 * grad must not alias the logits. Replaces the forward + backward pair of
 * Fast_CrossEntropyLoss (kernels/triton_kernels.py:320-424) and
 * FusedCrossEntropyFunction (loss/sota_losses.py:437-532) for callers that
 * reduce the per-row losses with fixed weights (mean, sum, batchmean).
 */
ts_status ts_ce_fwd_bwd(const void* logits, int64_t ld, ts_dtype dtype,
                        const int64_t* labels, int64_t N, int64_t V,
                        int64_t ignore_index, float logit_scale, float softcap,
                        float label_smoothing, const float* dloss, int64_t dloss_stride,
                        float dloss_scale, float* loss, float* lse,
                        void* grad, int64_t ld_grad, ts_dtype grad_dtype, ts_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Vocabulary-parallel cross-entropy (the kernels of one rank)               */
/* ------------------------------------------------------------------------ */

/*
 * One rank's partials over its vocabulary shard: logits [N, Vp] (row stride
 * ld) are the columns vocab_start .. vocab_start + Vp - 1 of the full
 * vocabulary. For each row r, stats[4r .. 4r + 3] (16-byte aligned) receives
 *   { lse over the shard, the logit of targets[r] when the target lies in the
 *     shard (else 0), the sum of the shard's logits, 0 }.
 * Exchanging these 16 bytes per row (one all-gather over the ranks) replaces
 * the three all-reduces (row max, sum of exp, target logit) of
 * VocabParallelCrossEntropyLoss.forward, distributed/tensor_parallel.py:1522-1573.
 * No ignore_index: like the reference, every row counts.
 */
ts_status ts_ce_vocab_shard_stats(const void* logits, int64_t ld, ts_dtype dtype,
                                  const int64_t* targets, int64_t N, int64_t Vp,
                                  int64_t vocab_start, float* stats, ts_stream_t stream);

/*
 * Merges the P ranks' partials, stats_all [P][N][4] (rank-major, as an
 * all-gather lays them out), into lse[N] and the per-row loss[N] of rank
 * `self`:
 *   lse = log sum_p exp(lse_p),  nll = lse - sum_p target_p,
 *   loss = (1 - a) * nll + a * (lse - sum_z_self / Vp),  a = label_smoothing,
 * which is VocabParallelCrossEntropyLoss.forward's per-row loss
 * (tensor_parallel.py:1576-1597; the smoothing term, :1587-1588, uses the rank's own shard
 * mean, as there).
 */
ts_status ts_ce_vocab_merge(const float* stats_all, int64_t P, int64_t self, int64_t N,
                            int64_t Vp, float label_smoothing, float* lse, float* loss,
                            ts_stream_t stream);

/*
 * Gradient over the shard:
 *   grad[r, j] = dl * ((1 - a) * (exp(z - lse[r]) - [vocab_start + j == targets[r]]) - a / Vp),
 *   dl = grad_output[0] * dloss_scale,
 * VocabParallelCrossEntropyLoss.backward, tensor_parallel.py:1600-1632 (its
 * caller passes dloss_scale = 1 / (B * S) for the mean). grad_dtype is the
 * logits dtype or fp32; grad may alias the logits when both match.
 */
ts_status ts_ce_vocab_shard_bwd(const void* logits, int64_t ld, ts_dtype dtype,
                                const int64_t* targets, const float* lse,
                                const float* grad_output, float dloss_scale,
                                int64_t N, int64_t Vp, int64_t vocab_start,
                                float label_smoothing, void* grad, int64_t ld_grad,
                                ts_dtype grad_dtype, ts_stream_t stream);

/*
 * Vocabulary-parallel fused linear cross-entropy, the two phases of one rank
 * (no reference function: the vocabulary-parallel form of ts_flce_fwd_bwd for
 * an LM head split by rows over the tensor-parallel ranks, the layout of
 * VocabParallelEmbedding / ColumnParallelLinear, distributed/tensor_parallel.py).
 * weight: this rank's [Vp, H] rows, vocabulary columns vocab_start ..
 * vocab_start + Vp - 1, any Vp. N and H are multiples of 8 (the Python
 * wrapper pads other shapes: ignored rows, zero columns). Both phases take the
 * same workspace of ts_flce_vocab_workspace_size(N, Vp) bytes, which carries
 * the shard's logits (rows of round_up(Vp, 8) columns) from phase 1 to phase 2
 * and must not change in between.
 *
 * Phase 1: logits = hidden @ weight^T (bf16, into the workspace) and the
 * per-row partials stats[4r .. 4r + 3] = {lse over the shard, the logit of
 * labels[r] if the shard holds it (else 0), 0, 0}: the layout of
 * ts_ce_vocab_shard_stats, for the same all-gather.
 */
size_t ts_flce_vocab_workspace_size(int64_t N, int64_t Vp);
ts_status ts_flce_vocab_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                            const int64_t* labels, int64_t N, int64_t H, int64_t Vp,
                            int64_t vocab_start, float* stats, void* workspace,
                            size_t workspace_bytes, ts_stream_t stream);

/*
 * Phase 2, after the caller gathered every rank's partials into stats_all
 * [P][N][4] (rank-major): lse[r] = log sum_p exp(lse_p), the per-row loss
 * lse - (sum of the target logits) (0 where labels[r] == ignore_index; a
 * label in no rank's shard contributes a target logit of 0), loss = their
 * mean over non-ignored rows (reduction 0) or sum (1), the same on every rank.
 * Then the shard's dlogits ((softmax - onehot) * loss scale, bf16, in the
 * workspace) give grad_hidden_partial [N, H] = dlogits @ weight (bf16; the
 * caller sums it over the ranks) and grad_weight_shard [Vp, H] = dlogits^T @
 * hidden (bf16). Either gradient may be NULL; loss_rows and lse may be NULL.
 */
ts_status ts_flce_vocab_bwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                            const int64_t* labels, int64_t N, int64_t H, int64_t Vp,
                            int64_t vocab_start, const float* stats_all, int64_t P,
                            int64_t ignore_index, int32_t reduction, float* loss,
                            float* loss_rows, float* lse, void* grad_hidden_partial,
                            void* grad_weight_shard, void* workspace, size_t workspace_bytes,
                            ts_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Fused linear cross-entropy                                                */
/* ------------------------------------------------------------------------ */

/* flags of ts_flce_workspace_size / ts_flce_fwd_bwd */
enum {
  TS_FLCE_GRADS = 1,       /* workspace size: with the gradients' scratch */
  TS_FLCE_ACCUM_BF16 = 2   /* sum grad_weight over token chunks in the bf16 output (rounded
                              after each chunk, as autograd sums the per-chunk bf16 gradients
                              of the reference's chunked_log_softmax, rl_training.py:167-191)
                              instead of an fp32 V x H workspace rounded once */
};

/*
 * Bytes of workspace ts_flce_fwd_bwd needs for hidden [N, H], weight [V, H]
 * and a token chunk of `chunk` rows (chunk <= 0 or >= N: one chunk), with
 * (flags & TS_FLCE_GRADS) or without the backward scratch, and with
 * (TS_FLCE_ACCUM_BF16) or without the fp32 grad_weight sum.
 */
size_t ts_flce_workspace_size(int64_t N, int64_t H, int64_t V, int64_t chunk,
                              int32_t flags);

/*
 * Loss and gradients of logits = hidden @ weight^T without a library GEMM:
 *   loss_rows[r] = lse_r - logits[r, labels[r]]   (0 where labels[r] == ignore_index,
 *                                                   NaN for other labels outside [0, V))
 *   *loss = sum(loss_rows) * scale,  scale = 1/max(n_valid, 1) (reduction 0, mean)
 *                                    or 1 (reduction 1, sum)
 *   grad_hidden = dlogits @ weight,  grad_weight = dlogits^T @ hidden,
 *   dlogits = (softmax(logits) - onehot(labels)) * scale, 0 on ignored rows,
 * i.e. the gradients of *loss for an upstream gradient of 1.
 * hidden, weight, grad_hidden, grad_weight: bf16, row-major, 16-byte aligned,
 * row strides ldh/ldw (elements, multiples of 8; the gradients are dense).
 * N and H multiples of 8 (the Python wrapper pads other N and H); any V >= 1
 * (the library's logits rows are padded to whole 16-byte vectors and the
 * columns past V masked). Logits are formed in fp32 by MFMA and rounded to
 * bf16 (the rounding a bf16 matmul applies); softmax statistics, lse and loss
 * are fp32. loss_rows, lse ([N] fp32) may be NULL. grad_hidden and
 * grad_weight may be NULL (then their GEMM is skipped; both NULL: forward
 * only). Deterministic: every reduction has a fixed order.
 * The rows are processed in token chunks of `chunk` rows (0: one chunk); a
 * chunk's bf16 logits are the only [rows, V] scratch. Per chunk the two
 * gradient GEMMs run as one grid. grad_weight sums over the chunks in fp32 in
 * the workspace (rounded once), or with flags & TS_FLCE_ACCUM_BF16 in the
 * bf16 output (no V x H workspace). flags: the value given to
 * ts_flce_workspace_size (TS_FLCE_GRADS is accepted and ignored here: the
 * gradient pointers decide whether gradients are formed).
 * Has no counterpart in the reference, which has no fused linear-CE; it
 * replaces the composition logits = hidden @ lm_head.t() (rl_training.py:177,
 * chunked_log_softmax :138-191) followed by cross-entropy
 * (kernels/triton_kernels.py:427-467) and autograd's matmul backward.
 */
ts_status ts_flce_fwd_bwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                          const int64_t* labels, int64_t N, int64_t H, int64_t V,
                          int64_t ignore_index, int32_t reduction,
                          float* loss, float* loss_rows, float* lse,
                          void* grad_hidden, void* grad_weight, int64_t chunk,
                          int32_t flags, void* workspace, size_t workspace_bytes,
                          ts_stream_t stream);

/*
 * Two-pass fused linear cross-entropy (the schedule for any reduction and any
 * upstream gradient, and for forward-only calls): no [N, V] logits are stored.
 *
 * Logits z = bf16(hidden @ weight^T) (MFMA, fp32 accumulation, rounded to bf16
 * as a bf16 matmul rounds them), transformed in the order of
 * selective_log_softmax (rl_training.py:114-122):
 *   t = softcap > 0 ? softcap * tanh(z / softcap) : z;  t *= scale if scale > 0;
 *   t /= temperature
 * (softcap = scale = 0, temperature = 1: t = z). Per row, in fp32:
 *   lse[r] = log sum_j exp(t[r, j]),
 *   loss_rows[r] = lse[r] - t[r, labels[r]]  (0 where labels[r] == ignore_index,
 *                                            NaN for other labels outside [0, V)),
 *   reduction 0 (mean): *loss = sum(loss_rows) / max(n_valid, 1); 1 (sum):
 *   *loss = sum(loss_rows); 2 (none): loss may be NULL.
 * hidden [N, H], weight [V, H]: bf16, 16-byte aligned, row strides ldh/ldw
 * (multiples of 8); H a multiple of 8 (the Python wrapper pads other H); any
 * V >= 1; any N >= 0.
 *
 * Forward: one logits GEMM whose epilogue keeps per-(row, 128-column slice)
 * max and sum of exp and the label's t; workspace of
 * ts_flce_forward_workspace_size(N, V) bytes (N * V / 16 bytes of statistics).
 * loss_rows and lse may be NULL (lse is what the backward needs).
 * Replaces chunked_log_softmax + selective_log_softmax (rl_training.py:95-191,
 * which return -loss_rows, called by GRPOCompute.compute_log_probs :509-552)
 * and the composition logits = hidden @ lm_head.t() then cross-entropy
 * (kernels/triton_kernels.py:427-467), without their [B, chunk, V] logits.
 */
size_t ts_flce_forward_workspace_size(int64_t N, int64_t V);
ts_status ts_flce_forward(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                          const int64_t* labels, int64_t N, int64_t H, int64_t V,
                          int64_t ignore_index, int32_t reduction,
                          float softcap, float scale, float temperature,
                          float* loss, float* loss_rows, float* lse,
                          void* workspace, size_t workspace_bytes, ts_stream_t stream);

/*
 * Backward of ts_flce_forward for the upstream gradient dloss (device fp32:
 * dloss[r * dloss_stride], stride 0 broadcasts one value; for mean and sum
 * the scalar upstream gradient of *loss, for none that of each loss_rows[r]):
 *   dt[r, j] = dloss_r * s * (softmax(t[r])_j - [j == labels[r]]),
 *   s = 1 / max(n_valid, 1) for mean, else 1; 0 on ignore_index rows,
 *   dz = bf16(dt * dt/dz),  grad_hidden = dz @ weight,  grad_weight = dz^T @ hidden
 * (bf16 outputs, fp32 accumulation; either may be NULL). lse: the forward's.
 * The logits are recomputed one vocabulary chunk of chunk_cols columns at a
 * time (0: about V / 8, at least 4096; rounded up to 256) by the forward's
 * GEMM, whose epilogue forms the chunk's dz; grad_hidden accumulates over the
 * chunks in fp32, grad_weight's rows of a chunk are written once. Workspace:
 * ts_flce_backward_workspace_size(N, H, V, chunk_cols) bytes (N x chunk bf16
 * dz, plus N x H fp32 with more than one chunk). Deterministic.
 * Replaces autograd's backward through chunked_log_softmax /
 * selective_log_softmax (rl_training.py:95-191) and the lm_head matmul.
 */
size_t ts_flce_backward_workspace_size(int64_t N, int64_t H, int64_t V, int64_t chunk_cols);
ts_status ts_flce_backward(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                           const int64_t* labels, int64_t N, int64_t H, int64_t V,
                           int64_t ignore_index, int32_t reduction,
                           float softcap, float scale, float temperature,
                           const float* lse, const float* dloss, int64_t dloss_stride,
                           void* grad_hidden, void* grad_weight, int64_t chunk_cols,
                           void* workspace, size_t workspace_bytes, ts_stream_t stream);

/*
 * ts_flce_forward that also writes the bf16 logits z = bf16(hidden @ weight^T)
 * to `logits` ([N, V] with row stride round_up(V, 8), 16-byte aligned:
 * N * round_up(V, 8) * 2 bytes of caller memory, 2.1 GB at N = 8192,
 * V = 128256; the columns from V to the row's end are written too), for
 * ts_flce_backward_kept.
 * Everything else is bit-identical to ts_flce_forward's, and its workspace is
 * the same. The reference's chunked_log_softmax keeps each chunk's
 * [B, chunk, V] logits alive for autograd's backward (rl_training.py:175-189);
 * this keeps one bf16 copy, so the backward need not recompute them.
 */
ts_status ts_flce_forward_keep(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                               const int64_t* labels, int64_t N, int64_t H, int64_t V,
                               int64_t ignore_index, int32_t reduction,
                               float softcap, float scale, float temperature,
                               float* loss, float* loss_rows, float* lse, void* logits,
                               void* workspace, size_t workspace_bytes, ts_stream_t stream);

/*
 * ts_flce_backward from the logits ts_flce_forward_keep kept, which it
 * overwrites with dz (they are consumed: another backward needs
 * ts_flce_backward). dz is bit-identical to what ts_flce_backward forms, and
 * so is grad_weight; grad_hidden sums over all of V in one fp32 accumulation
 * instead of one per vocabulary chunk (the order of the fp32 sums differs).
 * Three GEMMs in all instead of four. Workspace:
 * ts_flce_backward_kept_workspace_size(N) bytes. Replaces autograd's backward
 * through chunked_log_softmax / selective_log_softmax (rl_training.py:95-191)
 * and the lm_head matmul, as ts_flce_backward does.
 */
size_t ts_flce_backward_kept_workspace_size(int64_t N);
ts_status ts_flce_backward_kept(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                                const int64_t* labels, int64_t N, int64_t H, int64_t V,
                                int64_t ignore_index, int32_t reduction,
                                float softcap, float scale, float temperature,
                                const float* lse, const float* dloss, int64_t dloss_stride,
                                void* logits, void* grad_hidden, void* grad_weight,
                                void* workspace, size_t workspace_bytes, ts_stream_t stream);

/*
 * x[i] *= *scale for n contiguous values of `dtype` (any n >= 0; 16-byte
 * vectors where x is 16-byte aligned, single elements for the rest); scale
 * is a device pointer, and when *scale == 1 nothing is written. Applies an upstream gradient other than 1
 * to gradients formed in a forward pass (ts_ce_fwd_bwd, ts_flce_fwd_bwd)
 * without a host synchronisation. Has no counterpart in the reference, whose
 * backward passes receive the upstream gradient directly.
 */
ts_status ts_scale_inplace(void* x, int64_t n, ts_dtype dtype, const float* scale,
                           ts_stream_t stream);

/*
 * x[i] *= *now / *used in place (same layout rules as ts_scale_inplace);
 * nothing is written to x when the ratio is exactly 1. If hint_out is not
 * NULL it receives *now when that is finite and non-zero, else 1 (it must
 * not alias now or used). This lets a forward pass form a gradient for a
 * predicted upstream gradient `used` (the previous step's, for a loss whose
 * scale is fixed across steps, such as 1 / gradient-accumulation steps),
 * and the backward pass correct it only when the prediction was wrong. No
 * counterpart in the reference (its backward passes get the upstream
 * gradient directly).
 */
ts_status ts_rescale_inplace(void* x, int64_t n, ts_dtype dtype, const float* now,
                             const float* used, float* hint_out, ts_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Measurement                                                               */
/* ------------------------------------------------------------------------ */

/*
 * dst[0 .. bytes) = src[0 .. bytes) with the flat streaming copy kernel (one
 * 16-byte vector per thread, 256-thread workgroups, non-temporal accesses);
 * bytes a multiple of 16, both buffers 16-byte aligned and not overlapping.
 * No counterpart in the reference: the copy against which the benchmark sets
 * each memory-bound kernel, for the same number of bytes moved.
 */
ts_status ts_stream_copy(void* dst, const void* src, int64_t bytes, ts_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TRAINSCALE_AMD_H */
