// Internal launch interface shared by the kernel sources and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

#include "ns_common.h"

namespace ns {

// Inputs shared by every objective entry point (all device pointers).
struct SlotArgs {
  const int64_t* labels;   // [N] target token ids (prepared.target_ids)
  const float* weights;    // [N] w = valid * exp(-slot/gamma) (prepared.weights)
  const uint8_t* valid;    // [N] supervision validity (prepared.valid, torch.bool)
  int64_t n;               // rows (draft slots)
  int64_t k;               // slots per block (accept_len prefix axis)
  float c_ce, c_kl;        // objective.ce, objective.kl
  float inv_acc;           // 1 / accumulation_steps
};

// ---- logits-level streaming path (stream.hip) -----------------------------
int stream_splits(int64_t n, int64_t v);
size_t stream_workspace_bytes(int64_t n, int64_t v);
hipError_t stream_forward(const void* z, int zdt, int64_t ldz, const void* u, int udt, int64_t ldu,
                          int64_t v, const SlotArgs& a, void* dl, int64_t ldd, float* row_stats,
                          float* metrics, void* ws, hipStream_t st);
hipError_t stream_backward(const void* z, int zdt, int64_t ldz, const void* u, int udt, int64_t ldu,
                           int64_t v, const SlotArgs& a, const float* row_stats, void* dl, int64_t ldd,
                           hipStream_t st);

// ---- shared tails (stream.hip) ---------------------------------------------
// Teacher logits as the producer left them: objective row t reads teacher row rows[t]
// (rows null: row t) of nt rows; lse (null: formed in pass 1) holds one log-normaliser per
// teacher row.
struct TeacherSpec {
  const int64_t* rows;
  int64_t nt;
  const float* lse;
};
// Merge first-pass partials part1[N][S] (+ z_y[N]) into row_stats (lse_z, lse_u, ce, kl, z_y).
// With ts (its lse given) lse_u comes from ts and KL is left to the finalize.
hipError_t launch_merge(const RowPart* part1, const float* zy, int64_t v, int splits, const SlotArgs& a,
                        float* row_stats, hipStream_t st, const TeacherSpec* ts = nullptr);
// Sum accept partials parta[N][S], form block lengths and the six metrics; with partk
// (pass-2 sums of t (u - z)), KL = sum partk - lse_u + lse_z first.  parta NULL: the metrics
// alone, from complete row_stats; metrics NULL: the row sums alone.
hipError_t launch_finalize(const float* parta, int splits, const SlotArgs& a, float* row_stats,
                           float* metrics, hipStream_t st, const float* partk = nullptr);
// lse[t] = log-sum-exp from (max, sum-exp) partials part1[N][S] (mz, sz), fixed order.
hipError_t launch_lse_merge(const RowPart* part1, int splits, int64_t n, float* lse, hipStream_t st);

// ---- final_norm around the head (norm.hip) ------------------------------------
constexpr int64_t kMaxNormD = 16384;   // hidden sizes the rms-norm kernels hold in registers
// rms_norm backward operands (ops.py:55-66): x the forward's input, inv its [N] inverse
// RMS, w the norm weight [d]; outputs dx [N, d] and wgrad [d] (overwritten), all bf16
struct NormBwd {
  const uint16_t* x;
  int64_t ldx;
  const float* inv;
  const uint16_t* w;
  uint16_t* dx;
  int64_t lddx;
  uint16_t* wgrad;
};
int norm_rows_per_block(int64_t n);
size_t norm_bwd_workspace_bytes(int64_t n, int64_t d);
hipError_t rms_norm_forward(const void* x, int64_t ldx, const void* weight, int64_t n, int64_t d, float eps,
                            void* out, int64_t ldo, void* normalized, int64_t ldn, float* inv, hipStream_t st);
// dy from split-K partials part[ksplit][N][d] (dh_out, if not NULL, receives bf16 dh) or,
// with part == NULL, from the bf16 tensor dy
hipError_t rms_norm_backward_rows(const float* part, int ksplit, const void* dy, int64_t lddy, const NormBwd& nb,
                                  void* dh_out, int64_t lddh, int64_t n, int64_t d, void* ws, hipStream_t st);

// ---- fused LM-head path (lmhead.hip) ---------------------------------------
// Markov head in factored form: logits += W1[prev] . W2^T (rank r, r % 64 == 0).
struct MarkovFactors {
  const int64_t* prev;   // [N] previous-token ids
  const void* w1;        // [V, r] bf16, row stride ldw1
  const void* w2;        // [V, r] bf16, row stride ldw2
  int64_t ldw1, ldw2, r;
};
size_t lmhead_workspace_bytes(int64_t n, int64_t v, int64_t d);
// Raises the dynamic-LDS limit of every head instantiation lmhead_forward can launch, on the
// current device (done lazily at launch otherwise; this lets a caller do it before capture).
hipError_t lmhead_forward_prepare();
// lmhead_forward's parts: pass 1 and the merge (row_stats' log-normalisers, CE, KL, z_label),
// then pass 2 with the per-row accept (and teacher-once KL) sums and, when metrics is not
// NULL, the metrics
constexpr int kHeadStats = 1, kHeadEmit = 2, kHeadParts = kHeadStats | kHeadEmit;
hipError_t lmhead_forward(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                          const void* markov, int64_t ldm, const MarkovFactors* factors, const void* teacher,
                          int tdt, int64_t ldt, int64_t d, int64_t v, const SlotArgs& a, const TeacherSpec* ts,
                          void* dl, int64_t ldd, float* row_stats, float* metrics, void* ws, hipStream_t st,
                          int parts = kHeadParts);
// dst row r = src row map[r] (row_bytes bytes), or zeros where map[r] is outside [0, n_src)
hipError_t copy_rows(const void* src, int64_t ld_src, int64_t n_src, const int64_t* map, int64_t n_dst,
                     int64_t row_bytes, void* dst, int64_t ld_dst, hipStream_t st);
// Pass 2 of lmhead_forward alone: dl for a.inv_acc from the row_stats a forward over the
// same inputs wrote (same kernel, so the same bits a forward with that inv_acc emits).
// Workspace: lmhead_workspace_bytes.
hipError_t lmhead_emit_dlogits(const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                               const void* markov, int64_t ldm, const MarkovFactors* factors, const void* teacher,
                               int tdt, int64_t ldt, int64_t d, int64_t v, const SlotArgs& a,
                               const TeacherSpec* ts, const float* row_stats, void* dl, int64_t ldd, void* ws,
                               hipStream_t st);
// dh workspace; r > 0 adds the Markov column tiles' partials, norm the rms-norm
// backward's column partials
size_t lmhead_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t r = 0, bool norm = false);
hipError_t lmhead_backward(const void* dl, int64_t ldd, const void* weight, int64_t ldw, void* dh,
                           int64_t lddh, int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st);
// dh = dl . weight and, when r > 0, dprev = dl . w2 (fp32 [N, r], row stride r) in the same
// GEMM.  With norm, the split-K reduction is the rms-norm backward: dx and the norm weight's
// gradient are written, and dh only if dh is not NULL.
hipError_t lmhead_backward_ext(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const void* w2,
                               int64_t ldw2, int64_t r, void* dh, int64_t lddh, float* dprev, const NormBwd* norm,
                               int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st);
// Markov-head backward (markov.hip): dh (or, with norm, dx and the norm weight's gradient),
// w2_grad = dl^T . w1[prev] (overwritten) and w1_grad.index_add_(prev, dl . w2)
// (accumulated, deterministic order)
size_t markov_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t r);
hipError_t markov_backward(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const MarkovFactors& f,
                           void* dh, int64_t lddh, const NormBwd* norm, void* w1_grad, int64_t ldg1, void* w2_grad,
                           int64_t ldg2, int64_t n, int64_t v, int64_t d, void* ws, size_t ws_bytes, hipStream_t st);
hipError_t lmhead_linear(const void* x, int64_t ldx, const void* weight, int64_t ldw, const void* addend,
                         int64_t lda, void* out, int64_t ldo, int64_t n, int64_t v, int64_t d,
                         hipStream_t st);
// The projection as a teacher-logit producer: out = x[rows] . weight^T (+ addend) with,
// when lse is not NULL, lse[t] = log-sum-exp of out's bf16 row t; rows (null: row t)
// index nrows rows of x.  Workspace: lmhead_linear_lse_workspace_bytes.
size_t lmhead_linear_lse_workspace_bytes(int64_t n, int64_t v);
hipError_t lmhead_linear_lse(const void* x, int64_t ldx, const int64_t* rows, int64_t nrows, const void* weight,
                             int64_t ldw, const void* addend, int64_t lda, void* out, int64_t ldo, float* lse,
                             int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st);

// ---- FP8 teacher head (fp8.hip) ---------------------------------------------
size_t fp8_workspace_bytes(int64_t n, int64_t v, int64_t d);
hipError_t fp8_quantize_rows(const void* x, int64_t ldx, int64_t n, int64_t d, uint8_t* q, float* xs,
                             hipStream_t st);
// lse (null: not formed): log-sum-exp of each stored bf16 output row, from the epilogue
hipError_t fp8_teacher_logits(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw,
                              const float* scale, void* out, int64_t ldo, float* lse, int64_t n, int64_t v,
                              int64_t d, void* ws, hipStream_t st);

// ---- slot preparation (prepare.hip) -----------------------------------------
hipError_t prepare_slots(const int64_t* ids, const float* loss_mask, const int64_t* anchors,
                         const uint8_t* keep, int64_t b, int64_t s, int64_t nb, int64_t k,
                         float gamma, int64_t* target_ids, int64_t* previous, float* weights,
                         uint8_t* valid, int64_t* teacher_indices, hipStream_t st);

// ---- pooled-normalisation tail (pooled.hip) ------------------------------------
// out[4] = (loss, accept_len, gradient factor, pooled denominator) from [count][6] metrics
hipError_t pooled_tail(const float* metrics, int64_t count, int64_t world_size, int64_t accumulation_steps,
                       float* out, hipStream_t st);
// grad[0..n) *= *factor in place (bf16 or fp32)
hipError_t scale_gradient(void* grad, int dtype, int64_t n, const float* factor, hipStream_t st);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device.  The attribute
// belongs to each device's copy of the kernel, so `done` keeps one bit per device id (ids
// of 64 and up set it on every call); concurrent first calls may both set it, harmlessly.
inline hipError_t ensure_dynamic_lds(const void* fn, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t(1) << dev) : 0;
  if (bit && (done.load(std::memory_order_relaxed) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_relaxed);
  return e;
}

}  // namespace ns
