/* nanospec_hip.h -- C ABI of the MI355X (gfx950) draft-objective library.
 *
 * Drop-in for the arithmetic of nanospec's draft head + objective path
 * (reference paths relative to the jamesdborin/nanospec checkout):
 *   nanospec/objective.py:49-67   ce_kl_loss         -> ns_ce_kl_logits_fwd
 *   nanospec/objective.py:70-80   ce_kl_backward     -> ns_ce_kl_logits_bwd
 *   nanospec/objective.py:39-46   acceptance_length_counts (inside both fwd entries)
 *   nanospec/ops.py:34-35 via train.py:272-279, 291   linear + ce_kl_loss fused
 *                                                     -> ns_lmhead_ce_kl_fwd
 *   nanospec/objective.py:70-80 via train.py:301  ce_kl_backward after the fused
 *                                 forward (dl for the backward's accumulation_steps)
 *                                                     -> ns_lmhead_ce_kl_bwd
 *   nanospec/train.py:302         dh = dl @ lm_head.w -> ns_lmhead_bwd
 *   nanospec/train.py:276-279 (MarkovHead, layers.py:74-78: embedding + linear)
 *     fused into the LM head as a second K segment -> ns_lmhead_markov_ce_kl_fwd
 *   nanospec/train.py:302-307     dh, markov_w2.grad, markov_w1.grad -> ns_lmhead_markov_bwd
 *   nanospec/train.py:172-173, 280-290  teacher logits (producer LSE, gathered rows)
 *                                 -> ns_lmhead_teacher_logits, ns_teacher_args
 *   nanospec/train.py:271, 308-310 final_norm (ops.py:48-66) -> ns_rms_norm_fwd,
 *                                 ns_rms_norm_bwd, ns_lmhead_norm_bwd (fused after dh)
 *   nanospec/train.py:525-535, shard.py:318-330  pooled metrics, gradient factor
 *                                 -> ns_pooled_tail, ns_scale_gradient
 *
 * Conventions
 *   - All tensor arguments are device pointers; rows are `ld` elements apart,
 *     elements within a row are contiguous.
 *   - Every call is asynchronous on `stream` (the caller's current HIP stream);
 *     nothing synchronises the device and nothing is allocated: scratch
 *     memory is passed in as `workspace` (size from the *_workspace_bytes query).
 *   - Status: 0 ok; negative = invalid argument (shape, dtype, alignment,
 *     workspace size); positive = hipError_t from a launch.  ns_last_error()
 *     returns a thread-local description of the last failure.
 *   - dtype codes: NS_BF16 (raw bfloat16) or NS_F32.
 *   - Row metadata: labels int64 [N], weights fp32 [N] (valid * exp(-slot/gamma)),
 *     valid uint8 [N] (torch.bool); rows come in blocks of K consecutive slots.
 *     Label -100 is F.cross_entropy's ignore_index (objective.py:54): the row has no CE
 *     term (CE 0, and dl without it).  Any other label outside [0, V) makes the row's CE,
 *     and so the loss, NaN: the device cannot raise.
 *   - Outputs: metrics fp32 [6] in LossMetrics order (ce, kl, numerator,
 *     denominator, accept_len_sum, accept_len_total; objective.py:11-18) and
 *     row_stats fp32 [N][8] = (lse_z, lse_u, ce, kl, accept_rate, z_label, 0, 0).
 */
#ifndef NANOSPEC_HIP_H
#define NANOSPEC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NS_ABI_VERSION 6

#define NS_BF16 0
#define NS_F32 1

#define NS_OK 0
#define NS_EINVAL (-1)     /* bad shape or scalar argument */
#define NS_EDTYPE (-2)     /* unsupported dtype code */
#define NS_EALIGN (-3)     /* pointer / leading-dimension alignment */
#define NS_EWORKSPACE (-4) /* workspace missing or too small */
#define NS_ENULL (-5)      /* required pointer is NULL */

#define NS_WS_LOGITS 0   /* ns_ce_kl_logits_fwd */
#define NS_WS_LMHEAD 1   /* ns_lmhead_ce_kl_fwd */
#define NS_WS_LMHEAD_BWD 2 /* ns_lmhead_bwd */
#define NS_WS_FP8 3      /* ns_fp8_teacher_logits */
#define NS_WS_RMS_NORM_BWD 4     /* ns_rms_norm_bwd (v ignored) */
#define NS_WS_LMHEAD_NORM_BWD 5  /* ns_lmhead_norm_bwd */
#define NS_WS_TEACHER_LOGITS 6   /* ns_lmhead_teacher_logits with lse (d ignored) */

typedef struct ihipStream_t* ns_stream_t; /* == hipStream_t */

/* Operands of the rms_norm backward (ops.py:55-66) for final_norm (train.py:308-310):
 * x is the forward's input [N, d] bf16, inv its inverse RMS [N] fp32 (ns_rms_norm_fwd),
 * weight the norm weight [d] bf16; dx [N, d] bf16 and weight_grad [d] bf16 are written
 * (weight_grad overwritten, as the reference's copy_).  d % 8 == 0, d <= 16384,
 * 16-byte aligned base pointers and rows. */
/* Teacher logits as their producer left them (train.py:280-290).  Objective row t reads
 * row rows[t] of the teacher tensor, which has n_rows rows (rows NULL: row t, and n_rows
 * is n or 0): the gather of train.py:285-290 (teacher_indices, dspark.py:143) happens in
 * the load, with no gathered copy.  An index outside [0, n_rows) makes that row NaN.
 * lse, when not NULL, is the log-sum-exp of every teacher row (ns_lmhead_teacher_logits
 * writes it): the first pass then reads no teacher logits and the second forms KL. */
typedef struct ns_teacher_args {
  const int64_t* rows;
  int64_t n_rows;
  const float* lse;
} ns_teacher_args;

typedef struct ns_rms_norm_args {
  const void* x;
  int64_t ldx;
  const float* inv;
  const void* weight;
  void* dx;
  int64_t lddx;
  void* weight_grad;
} ns_rms_norm_args;

/* Library ABI version (NS_ABI_VERSION); the loader refuses a mismatch. */
int ns_abi_version(void);

/* Thread-local text of the last non-zero status. */
const char* ns_last_error(void);

/* Scratch bytes an entry point of `kind` needs (NS_WS_*); d is ignored by
 * NS_WS_LOGITS and NS_WS_TEACHER_LOGITS, v by NS_WS_RMS_NORM_BWD. */
size_t ns_workspace_bytes(int kind, int64_t n, int64_t v, int64_t d);

/* Forward objective over given logits (objective.py:49-67) plus, when dl is not
 * NULL, the derivative of objective.py:70-80 with scale inv_acc = 1/accumulation_steps.
 * z: draft logits [N, V] (z_dtype); u: teacher logits [N, V] (u_dtype);
 * dl: [N, V] in z_dtype, or NULL.  n % k == 0. */
int ns_ce_kl_logits_fwd(const void* z, int z_dtype, int64_t ldz, const void* u, int u_dtype, int64_t ldu,
                        const int64_t* labels, const float* weights, const uint8_t* valid, int64_t n,
                        int64_t v, int64_t k, float c_ce, float c_kl, float inv_acc, void* dl, int64_t ldd,
                        float* row_stats, float* metrics, void* workspace, size_t workspace_bytes,
                        ns_stream_t stream);

/* dl alone (objective.py:70-80) from row_stats of a previous forward. */
int ns_ce_kl_logits_bwd(const void* z, int z_dtype, int64_t ldz, const void* u, int u_dtype, int64_t ldu,
                        const int64_t* labels, const float* weights, int64_t n, int64_t v, float c_ce,
                        float c_kl, float inv_acc, const float* row_stats, void* dl, int64_t ldd,
                        ns_stream_t stream);

/* Fused LM head + objective forward (train.py:272-279 -> objective.py:49-67):
 * z = hidden . weight^T (+ markov) is formed tile by tile on bf16 MFMA and never
 * stored; pass 1 folds (max, sum-exp) of z and the teacher row and A = sum t(u - z);
 * pass 2 recomputes z and emits the accept rate and, when dl is not NULL,
 * dl = (w * inv_acc)[(c_ce + c_kl) p - c_kl t - c_ce e_y] as bf16.
 * hidden [N, d] bf16, weight [V, d] bf16 (the frozen LM head), markov [N, V] bf16
 * or NULL, teacher [N, V] (t_dtype), dl [N, V] bf16 or NULL.
 * Requires d % 64 == 0, V % 8 == 0, 16-byte aligned rows, n % k == 0. */
int ns_lmhead_ce_kl_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                        int64_t ldm, const void* teacher, int t_dtype, int64_t ldt,
                        const ns_teacher_args* teacher_args, const int64_t* labels, const float* weights,
                        const uint8_t* valid, int64_t n, int64_t d, int64_t v, int64_t k, float c_ce, float c_kl,
                        float inv_acc, void* dl, int64_t ldd, float* row_stats, float* metrics, void* workspace,
                        size_t workspace_bytes, ns_stream_t stream);

/* The fused forward in two parts, for a caller that runs pass 2 on a subset of its rows:
 * head.lm_head_ce_kl_loss(skip_masked_rows=True) runs pass 1 on every row, then pass 2 and
 * the dh GEMM only on the rows whose dl is not all zero (supervised rows, and unsupervised
 * rows whose log-normalisers are not finite), gathered with ns_copy_rows.  No counterpart in
 * the reference: objective.py:49-67 in steps.
 *   NS_PART_STATS: pass 1 and the merge; writes row_stats' lse_z, lse_u, ce, kl and z_label
 *                  (dl is ignored).
 *   NS_PART_EMIT:  pass 2 from row_stats' log-normalisers; writes dl (when not NULL) and the
 *                  accept rate (with teacher-LSE args also kl) into row_stats.
 * Arguments as ns_lmhead_ce_kl_fwd (labels, weights [n]; no valid, no metrics: those come from
 * ns_objective_metrics over every row).  Workspace NS_WS_LMHEAD for n rows. */
#define NS_PART_STATS 1
#define NS_PART_EMIT 2
int ns_lmhead_ce_kl_fwd_part(int part, const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                             const void* markov, int64_t ldm, const void* teacher, int t_dtype, int64_t ldt,
                             const ns_teacher_args* teacher_args, const int64_t* labels, const float* weights,
                             int64_t n, int64_t d, int64_t v, float c_ce, float c_kl, float inv_acc, void* dl,
                             int64_t ldd, float* row_stats, void* workspace, size_t workspace_bytes,
                             ns_stream_t stream);

/* The six LossMetrics from complete row statistics [n, 8] (objective.py:42-46, 53-60:
 * weighted CE and KL sums, accept_len from (accept_rate * valid).cumprod over blocks of k),
 * as the last step of ns_lmhead_ce_kl_fwd forms them. */
int ns_objective_metrics(const float* row_stats, const float* weights, const uint8_t* valid, int64_t n, int64_t k,
                         float c_ce, float c_kl, float* metrics, ns_stream_t stream);

/* dst row r = src row map[r] (row_bytes bytes each) for r < n_dst, and zeros where map[r] is
 * outside [0, n_src): the gather of the rows ns_lmhead_ce_kl_fwd_part runs pass 2 on, and the
 * scatter of their dl and dh back among zero rows.  Pitches in bytes; row_bytes and pitches
 * multiples of 4 (16-byte accesses when all are multiples of 16).  No counterpart in the
 * reference. */
int ns_copy_rows(const void* src, int64_t ld_src, int64_t n_src, const int64_t* map, int64_t n_dst, int64_t row_bytes,
                 void* dst, int64_t ld_dst, ns_stream_t stream);

/* ns_lmhead_ce_kl_fwd without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Its scratch is a static device array of 16 MiB per GPU,
 * held until the process ends (the fused forward needs about 2.6 MB at N = 4096 and
 * 10.6 MB at N = 32768 for V = 248,320); larger n * V is refused with NS_EWORKSPACE.
 * Nothing in the scratch has to start at zero.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (two streams, two threads) race; serialise them. */
/* Per-device set-up of ns_lmhead_ce_kl_fwd_noalloc, for callers that capture it into a
 * HIP graph: looks up the current device's static scratch (hipGetSymbolAddress) and raises
 * the fused forward's kernels' dynamic-LDS limit (hipFuncSetAttribute), so that no call
 * under capture makes either.  No counterpart in the reference.  Idempotent; call it once
 * per device, with that device current, before the first capture.  Without it the first
 * call on a device does the same. */
int ns_device_init(void);

int ns_lmhead_ce_kl_fwd_noalloc(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                                int64_t ldm, const void* teacher, int t_dtype, int64_t ldt,
                                const ns_teacher_args* teacher_args, const int64_t* labels, const float* weights,
                                const uint8_t* valid, int64_t n, int64_t d, int64_t v, int64_t k, float c_ce,
                                float c_kl, float inv_acc, void* dl, int64_t ldd, float* row_stats, float* metrics,
                                ns_stream_t stream);

/* The same forward with the Markov head in factored form (train.py:276-279):
 * z = hidden . weight^T + w1[prev] . w2^T, formed as one GEMM with K = d + r
 * ([hidden | w1[prev]] . [weight | w2]^T), so no [N, V] Markov tensor is read.
 * prev int64 [N]; w1 (markov_w1, nn.Embedding [V, r]) and w2 (markov_w2, nn.Linear
 * [V, r]) bf16 with r % 64 == 0.  A prev id outside [0, V) makes its row's logits
 * NaN (the reference's embedding lookup raises). */
int ns_lmhead_markov_ce_kl_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const int64_t* prev,
                               const void* w1, int64_t ldw1, const void* w2, int64_t ldw2, int64_t r,
                               const void* teacher, int t_dtype, int64_t ldt, const ns_teacher_args* teacher_args,
                               const int64_t* labels, const float* weights, const uint8_t* valid, int64_t n,
                               int64_t d, int64_t v, int64_t k, float c_ce, float c_kl, float inv_acc, void* dl,
                               int64_t ldd, float* row_stats, float* metrics, void* workspace,
                               size_t workspace_bytes, ns_stream_t stream);

/* dl alone for the fused head: ce_kl_backward (objective.py:70-80) as train.py:301 calls it,
 * with the backward's accumulation_steps (inv_acc = 1/accumulation_steps).  Runs pass 2 of
 * ns_lmhead_ce_kl_fwd / ns_lmhead_markov_ce_kl_fwd again over the same inputs, reading the
 * row log-normalisers from the row_stats that forward wrote: the same kernel, so dl holds
 * the bits a forward called with this inv_acc emits.  Markov head as in that forward:
 * markov [N, V] bf16 (dense addend), or prev, w1, w2 with r > 0 (factors), or neither
 * (markov NULL, r == 0).  dl [N, V] bf16 is required.  dh follows from dl through
 * ns_lmhead_bwd, ns_lmhead_markov_bwd or ns_lmhead_norm_bwd.  Workspace NS_WS_LMHEAD. */
int ns_lmhead_ce_kl_bwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                        int64_t ldm, const int64_t* prev, const void* w1, int64_t ldw1, const void* w2, int64_t ldw2,
                        int64_t r, const void* teacher, int t_dtype, int64_t ldt, const ns_teacher_args* teacher_args,
                        const int64_t* labels, const float* weights, int64_t n, int64_t d, int64_t v, float c_ce,
                        float c_kl, float inv_acc, const float* row_stats, void* dl, int64_t ldd, void* workspace,
                        size_t workspace_bytes, ns_stream_t stream);

/* Teacher-logit producer (train.py:172-173 and 281-284: ops.linear of the teacher's last
 * hidden state, gathered at teacher_indices, by the shared LM head):
 * out[t] = bf16(x[rows[t]] . weight^T), rows NULL: x[t].  When lse is not NULL, lse[t] =
 * log-sum-exp of out's bf16 row t, formed in the GEMM epilogue (workspace
 * NS_WS_TEACHER_LOGITS), for ns_teacher_args.lse.  x [n_rows, d] bf16 (d % 64 == 0),
 * out [n, V] bf16. */
int ns_lmhead_teacher_logits(const void* x, int64_t ldx, const int64_t* rows, int64_t n_rows, const void* weight,
                             int64_t ldw, void* out, int64_t ldo, float* lse, int64_t n, int64_t v, int64_t d,
                             void* workspace, size_t workspace_bytes, ns_stream_t stream);

/* LM-head backward dh = dl . weight (train.py:302): dl [N, V] bf16, weight [V, d]
 * bf16, dh [N, d] bf16.  Split-K over V with a fixed-order fp32 reduction. */
int ns_lmhead_bwd(const void* dl, int64_t ldd, const void* weight, int64_t ldw, void* dh, int64_t lddh,
                  int64_t n, int64_t v, int64_t d, void* workspace, size_t workspace_bytes, ns_stream_t stream);

/* final_norm forward, ops.rms_norm (ops.py:48-52) at train.py:271:
 * inv = rsqrt(mean(x^2) + eps) [N] fp32, normalized = bf16(x * inv) (written when not
 * NULL: the reference's saved activation), out = bf16(weight * normalized).
 * x, out, normalized [N, d] bf16; weight [d] bf16; d % 8 == 0, d <= 16384. */
int ns_rms_norm_fwd(const void* x, int64_t ldx, const void* weight, int64_t n, int64_t d, float eps, void* out,
                    int64_t ldo, void* normalized, int64_t ldn, float* inv, ns_stream_t stream);

/* rms_norm backward alone (ops.py:55-66): dy [N, d] bf16 -> norm->dx, norm->weight_grad.
 * Workspace NS_WS_RMS_NORM_BWD. */
int ns_rms_norm_bwd(const void* dy, int64_t lddy, const ns_rms_norm_args* norm, int64_t n, int64_t d, void* workspace,
                    size_t workspace_bytes, ns_stream_t stream);

/* dh = dl . weight (train.py:302) followed by final_norm's backward (train.py:308-310)
 * as the split-K reduction of the dh GEMM: dh is never stored unless dh is not NULL.
 * Workspace NS_WS_LMHEAD_NORM_BWD. */
int ns_lmhead_norm_bwd(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const ns_rms_norm_args* norm,
                       void* dh, int64_t lddh, int64_t n, int64_t v, int64_t d, void* workspace,
                       size_t workspace_bytes, ns_stream_t stream);

/* Scratch bytes ns_lmhead_markov_bwd needs for n slots, vocabulary v, hidden d, rank r. */
size_t ns_lmhead_markov_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t r);

/* Head backward with the factored Markov head (train.py:302-307):
 *   dh = dl . weight                                          (train.py:302)
 *   w2_grad = dl^T . w1[prev]      overwritten, bf16 [V, r]  (ops.py:38-45, copy_)
 *   w1_grad.index_add_(0, prev, dl . w2)   accumulated, bf16 (ops.py:73-74)
 * d(previous) = dl . w2 comes out of the dh GEMM as extra column tiles (fp32, never
 * rounded); each w1_grad row receives the fp32 sum of its tokens' rows, added in token
 * order (deterministic), rounded once.  Rows whose prev id is outside [0, V) add
 * nothing to w1_grad.  With norm not NULL, dh feeds final_norm's backward as in
 * ns_lmhead_norm_bwd (dh may then be NULL).  Requires V, d % 8 == 0, r % 64 == 0,
 * n < 2^31. */
int ns_lmhead_markov_bwd(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const int64_t* prev,
                         const void* w1, int64_t ldw1, const void* w2, int64_t ldw2, int64_t r, void* dh,
                         int64_t lddh, const ns_rms_norm_args* norm, void* w1_grad, int64_t ldg1, void* w2_grad,
                         int64_t ldg2, int64_t n, int64_t v, int64_t d, void* workspace, size_t workspace_bytes,
                         ns_stream_t stream);

/* Pooled-normalisation tail (train.py:525-535, shard.py:318-327): sums `count` LossMetrics
 * buffers metrics [count][6] in index order (the reference all-reduces numerator,
 * denominator, accept_len_sum and accept_len_total over ranks) and writes out fp32 [4] =
 * (loss = num / max(den, 1e-6), accept_len = sum / max(total, 1),
 *  gradient factor = den > 0 ? world_size * accumulation_steps / max(den, 1e-6) : 0, den). */
int ns_pooled_tail(const float* metrics, int64_t count, int64_t world_size, int64_t accumulation_steps, float* out,
                   ns_stream_t stream);

/* grad[0..n) *= *factor in place, the factor read on the device (shard.py:330,
 * shard.grad.mul_(factor)); grad bf16 (rounded once) or fp32, 16-byte aligned. */
int ns_scale_gradient(void* grad, int dtype, int64_t n, const float* factor, ns_stream_t stream);

/* Plain LM-head projection out = x . weight^T (+ addend), bf16 out (ops.py:34-35 for
 * the head: train.py:272, 279, 284).  x [N, d], weight [V, d], addend [N, V] or NULL. */
int ns_lmhead_linear(const void* x, int64_t ldx, const void* weight, int64_t ldw, const void* addend,
                     int64_t lda, void* out, int64_t ldo, int64_t n, int64_t v, int64_t d, ns_stream_t stream);

/* Teacher logits from a block-FP8 head with ops.fp8_linear numerics (ops.py:183-200):
 * x [N, d] bf16 is quantised per 1x128 block (scale amax/448, e4m3 round-to-nearest-
 * even), wq [V, d] holds e4m3 codes with one fp32 scale per 128x128 block in
 * scale [V/128, d/128] (the scale multiplies); out [N, V] bf16 = bf16 of the fp32
 * sum over K blocks of x_scale * w_scale * (fp8 dot product on MFMA).
 * lse, when not NULL, receives the log-sum-exp of each bf16 output row [N] fp32, formed in
 * the GEMM epilogue, for ns_teacher_args.lse.
 * Requires V % 128 == 0 and d % 128 == 0 (ValueError in the reference). */
int ns_fp8_teacher_logits(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const float* scale,
                          void* out, int64_t ldo, float* lse, int64_t n, int64_t v, int64_t d, void* workspace,
                          size_t workspace_bytes, ns_stream_t stream);

/* The activation half of the above alone: q [N, d] e4m3 codes (row stride d) and
 * xs [N, d/128] fp32 scales of x [N, d] bf16 (ops.py:189-196). */
int ns_fp8_quantize_rows(const void* x, int64_t ldx, int64_t n, int64_t d, uint8_t* q, float* xs,
                         ns_stream_t stream);

/* Objective inputs of every draft slot from sampled anchors (dspark.py:116-127, 143):
 * ids [b, s] int64, loss_mask [b, s] fp32, anchors [b, nb] int64 (each in [0, s)),
 * keep [b, nb] uint8 -> target_ids, previous [b, nb, k] int64, weights [b, nb, k]
 * fp32 (valid * exp(-slot / gamma); no decay when gamma <= 0), valid [b, nb, k]
 * uint8 (prefix product), teacher_indices [b, nb * k] int64.  s >= 1. */
int ns_prepare_slots(const int64_t* ids, const float* loss_mask, const int64_t* anchors, const uint8_t* keep,
                     int64_t b, int64_t s, int64_t nb, int64_t k, float gamma, int64_t* target_ids,
                     int64_t* previous, float* weights, uint8_t* valid, int64_t* teacher_indices,
                     ns_stream_t stream);

/* ---- timing instrumentation (opt-in) -------------------------------------
 * Between ns_profile_begin() and ns_profile_end(), every kernel the library
 * launches is bracketed by HIP events recorded on its launch stream.
 * ns_profile_end() waits for those events and fills up to `capacity` entries
 * (one per kernel name, in first-launch order); *count receives the number of
 * distinct kernels.  Not for use while another thread calls the library. */
typedef struct {
  char name[48];
  int launches;
  double total_ms;
} ns_kernel_time;

int ns_profile_begin(void);
int ns_profile_end(ns_kernel_time* out, int capacity, int* count);

/* Restricts the timing to launches whose timer name is in `names` (comma-separated,
 * e.g. "head_stats,head_emit"); NULL or "" times every launch.  The other launches run
 * without events, so a timed window is not lengthened by events around short kernels.
 * Applies from the next launch until changed. */
int ns_profile_select(const char* names);

#ifdef __cplusplus
}
#endif

#endif /* NANOSPEC_HIP_H */
