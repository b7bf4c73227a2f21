// C ABI entry points: argument validation, workspace checks, error text.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/nanospec_hip.h"
#include "ns_internal.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return NS_OK;
  return fail((int)e, "%s: %s", where, hipGetErrorString(e));
}

bool dtype_ok(int dt) { return dt == NS_BF16 || dt == NS_F32; }

bool aligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_slots(const int64_t* labels, const float* weights, const uint8_t* valid, int64_t n, int64_t k,
                bool need_valid) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0 (got %lld)", (long long)n);
  if (n > 0 && (!labels || !weights || (need_valid && !valid)))
    return fail(NS_ENULL, "labels, weights and valid must be non-NULL");
  if (need_valid) {
    if (k < 1) return fail(NS_EINVAL, "block size k must be >= 1 (got %lld)", (long long)k);
    if (n % k) return fail(NS_EINVAL, "n (%lld) must be a multiple of the block size k (%lld)", (long long)n, (long long)k);
  }
  return NS_OK;
}

constexpr int64_t kMaxLd = int64_t(1) << 23;

int check_matrix(const void* p, int64_t n, int64_t cols, int64_t ld, const char* name) {
  if (n > 0 && cols > 0 && !p) return fail(NS_ENULL, "%s is NULL", name);
  if (ld < cols) return fail(NS_EINVAL, "%s: leading dimension %lld < columns %lld", name, (long long)ld, (long long)cols);
  // kernels address a 256-row tile with 32-bit byte offsets: 256 * ld * 2 bytes < 2^32
  if (ld > kMaxLd)
    return fail(NS_EINVAL, "%s: leading dimension %lld exceeds %lld elements", name, (long long)ld, (long long)kMaxLd);
  return NS_OK;
}

// Validate the rms-norm backward operands and convert them to the internal form.
int check_norm(const ns_rms_norm_args* nb, int64_t n, int64_t d, ns::NormBwd* out) {
  if (!nb) return fail(NS_ENULL, "norm is NULL");
  if (d % 8 || d > ns::kMaxNormD)
    return fail(NS_EINVAL, "rms-norm hidden size must be a multiple of 8 up to %lld (got %lld)",
                (long long)ns::kMaxNormD, (long long)d);
  int rc;
  if ((rc = check_matrix(nb->x, n, d, nb->ldx, "norm.x"))) return rc;
  if ((rc = check_matrix(nb->dx, n, d, nb->lddx, "norm.dx"))) return rc;
  if (n > 0 && (!nb->inv || !nb->weight || !nb->weight_grad))
    return fail(NS_ENULL, "norm.inv, norm.weight and norm.weight_grad must be non-NULL");
  if (!aligned(nb->x) || !aligned(nb->dx) || !aligned(nb->weight) || !aligned(nb->weight_grad) || nb->ldx % 8 ||
      nb->lddx % 8)
    return fail(NS_EALIGN, "rms-norm operands need 16-byte aligned base pointers and rows");
  *out = ns::NormBwd{static_cast<const uint16_t*>(nb->x), nb->ldx, nb->inv, static_cast<const uint16_t*>(nb->weight),
                     static_cast<uint16_t*>(nb->dx), nb->lddx, static_cast<uint16_t*>(nb->weight_grad)};
  return NS_OK;
}

}  // namespace

extern "C" {

int ns_abi_version(void) { return NS_ABI_VERSION; }

const char* ns_last_error(void) { return g_last_error; }

size_t ns_workspace_bytes(int kind, int64_t n, int64_t v, int64_t d) {
  if (n < 0 || v < 0 || d < 0) return 0;
  switch (kind) {
    case NS_WS_LOGITS:
      return ns::stream_workspace_bytes(n, v);
    case NS_WS_LMHEAD:
      return ns::lmhead_workspace_bytes(n, v, d);
    case NS_WS_LMHEAD_BWD:
      return ns::lmhead_bwd_workspace_bytes(n, v, d);
    case NS_WS_FP8:
      return ns::fp8_workspace_bytes(n, v, d);
    case NS_WS_RMS_NORM_BWD:
      return ns::norm_bwd_workspace_bytes(n, d);
    case NS_WS_LMHEAD_NORM_BWD:
      return ns::lmhead_bwd_workspace_bytes(n, v, d, 0, true);
    case NS_WS_TEACHER_LOGITS:
      return ns::lmhead_linear_lse_workspace_bytes(n, v);
    default:
      return 0;
  }
}

int ns_ce_kl_logits_fwd(const void* z, int z_dtype, int64_t ldz, const void* u, int u_dtype, int64_t ldu,
                        const int64_t* labels, const float* weights, const uint8_t* valid, int64_t n,
                        int64_t v, int64_t k, float c_ce, float c_kl, float inv_acc, void* dl, int64_t ldd,
                        float* row_stats, float* metrics, void* workspace, size_t workspace_bytes,
                        ns_stream_t stream) {
  if (!dtype_ok(z_dtype) || !dtype_ok(u_dtype))
    return fail(NS_EDTYPE, "unsupported dtype code (z %d, u %d)", z_dtype, u_dtype);
  if (v < 1) return fail(NS_EINVAL, "vocabulary size must be >= 1 (got %lld)", (long long)v);
  int rc;
  if ((rc = check_slots(labels, weights, valid, n, k, true))) return rc;
  if ((rc = check_matrix(z, n, v, ldz, "z"))) return rc;
  if ((rc = check_matrix(u, n, v, ldu, "u"))) return rc;
  if (dl && (rc = check_matrix(dl, n, v, ldd, "dl"))) return rc;
  if (!metrics || (n > 0 && !row_stats)) return fail(NS_ENULL, "metrics and row_stats must be non-NULL");
  const size_t need = ns::stream_workspace_bytes(n, v);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  ns::SlotArgs a{labels, weights, valid, n, k, c_ce, c_kl, inv_acc};
  return hip_status(ns::stream_forward(z, z_dtype, ldz, u, u_dtype, ldu, v, a, dl, ldd, row_stats, metrics,
                                       workspace, reinterpret_cast<hipStream_t>(stream)),
                    "ns_ce_kl_logits_fwd");
}

int ns_ce_kl_logits_bwd(const void* z, int z_dtype, int64_t ldz, const void* u, int u_dtype, int64_t ldu,
                        const int64_t* labels, const float* weights, int64_t n, int64_t v, float c_ce,
                        float c_kl, float inv_acc, const float* row_stats, void* dl, int64_t ldd,
                        ns_stream_t stream) {
  if (!dtype_ok(z_dtype) || !dtype_ok(u_dtype))
    return fail(NS_EDTYPE, "unsupported dtype code (z %d, u %d)", z_dtype, u_dtype);
  if (v < 1) return fail(NS_EINVAL, "vocabulary size must be >= 1 (got %lld)", (long long)v);
  int rc;
  if ((rc = check_slots(labels, weights, nullptr, n, 1, false))) return rc;
  if ((rc = check_matrix(z, n, v, ldz, "z"))) return rc;
  if ((rc = check_matrix(u, n, v, ldu, "u"))) return rc;
  if ((rc = check_matrix(dl, n, v, ldd, "dl"))) return rc;
  if (n > 0 && !row_stats) return fail(NS_ENULL, "row_stats must be non-NULL");
  ns::SlotArgs a{labels, weights, nullptr, n, 1, c_ce, c_kl, inv_acc};
  return hip_status(ns::stream_backward(z, z_dtype, ldz, u, u_dtype, ldu, v, a, row_stats, dl, ldd,
                                        reinterpret_cast<hipStream_t>(stream)),
                    "ns_ce_kl_logits_bwd");
}

}  // extern "C"

namespace {

// What check_head_inputs requires besides the head's inputs.
enum HeadCheck {
  kCheckForward,   // valid, metrics and row_stats; dl optional
  kCheckReemit,    // dl and row_stats (an input); metrics and valid unused
  kCheckParts,     // row_stats; dl optional; metrics and valid unused
};

// Validation shared by the fused forward, its parts and the dl re-emission (dense Markov
// addend or factors).
int check_head_inputs(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                      int64_t ldm, const ns::MarkovFactors* factors, const void* teacher, int t_dtype, int64_t ldt,
                      const ns_teacher_args* targs, const int64_t* labels, const float* weights,
                      const uint8_t* valid, int64_t n, int64_t d, int64_t v, int64_t k, const void* dl, int64_t ldd,
                      const float* row_stats, const float* metrics, const void* workspace, size_t workspace_bytes,
                      HeadCheck mode, int64_t* nt_out) {
  const bool reemit = mode == kCheckReemit;
  if (!dtype_ok(t_dtype)) return fail(NS_EDTYPE, "unsupported teacher dtype code %d", t_dtype);
  if (v < 8 || v % 8) return fail(NS_EINVAL, "vocabulary size must be a positive multiple of 8 (got %lld)", (long long)v);
  if (d < 64 || d % 64) return fail(NS_EINVAL, "hidden size must be a positive multiple of 64 (got %lld)", (long long)d);
  int rc;
  if ((rc = check_slots(labels, weights, valid, n, k, mode == kCheckForward))) return rc;
  if ((rc = check_matrix(hidden, n, d, ldh, "hidden"))) return rc;
  if ((rc = check_matrix(weight, v, d, ldw, "weight"))) return rc;
  if (markov && (rc = check_matrix(markov, n, v, ldm, "markov"))) return rc;
  // with teacher rows, the teacher tensor has its own row count (train.py:285-290 gathers it)
  const int64_t nt = targs && targs->rows ? targs->n_rows : n;
  if (targs && targs->rows && (nt < 1 || nt >= (int64_t(1) << 31)))
    return fail(NS_EINVAL, "teacher n_rows must be in [1, 2^31) (got %lld)", (long long)nt);
  if (targs && n > 0 && targs->n_rows > 0 && !targs->rows && targs->n_rows != n)
    return fail(NS_EINVAL, "teacher n_rows %lld without rows must equal n", (long long)targs->n_rows);
  if ((rc = check_matrix(teacher, nt, v, ldt, "teacher"))) return rc;
  if ((reemit || dl) && (rc = check_matrix(dl, n, v, ldd, "dl"))) return rc;
  if (mode != kCheckForward ? (n > 0 && !row_stats) : (!metrics || (n > 0 && !row_stats)))
    return fail(NS_ENULL, mode != kCheckForward ? "row_stats must be non-NULL" : "metrics and row_stats must be non-NULL");
  const int64_t tq = t_dtype == NS_BF16 ? 8 : 4;
  if (!aligned(hidden) || !aligned(weight) || !aligned(teacher) || (markov && !aligned(markov)) || (dl && !aligned(dl)) ||
      ldh % 8 || ldw % 8 || (markov && ldm % 8) || ldt % tq || (dl && ldd % 8))
    return fail(NS_EALIGN, "fused head needs 16-byte aligned base pointers and rows");
  if (factors) {
    const int64_t r = factors->r;
    if (r < 64 || r % 64) return fail(NS_EINVAL, "Markov rank must be a positive multiple of 64 (got %lld)", (long long)r);
    if (n > 0 && !factors->prev) return fail(NS_ENULL, "prev is NULL");
    if ((rc = check_matrix(factors->w1, v, r, factors->ldw1, "w1"))) return rc;
    if ((rc = check_matrix(factors->w2, v, r, factors->ldw2, "w2"))) return rc;
    if (!aligned(factors->w1) || !aligned(factors->w2) || factors->ldw1 % 8 || factors->ldw2 % 8)
      return fail(NS_EALIGN, "Markov factors need 16-byte aligned base pointers and rows");
    // gathered W1 rows are addressed with 32-bit byte offsets from its base
    if (v * factors->ldw1 * 2 >= (int64_t(1) << 32))
      return fail(NS_EINVAL, "w1 spans %lld bytes; at most 4 GiB", (long long)(v * factors->ldw1 * 2));
  }
  const size_t need = ns::lmhead_workspace_bytes(n, v, d);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  *nt_out = nt;
  return 0;
}

int lmhead_fwd_checked(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                       int64_t ldm, const ns::MarkovFactors* factors, const void* teacher, int t_dtype, int64_t ldt,
                       const ns_teacher_args* targs, const int64_t* labels, const float* weights, const uint8_t* valid,
                       int64_t n, int64_t d, int64_t v, int64_t k, float c_ce, float c_kl, float inv_acc, void* dl,
                       int64_t ldd, float* row_stats, float* metrics, void* workspace, size_t workspace_bytes,
                       ns_stream_t stream, const char* name) {
  int64_t nt = 0;
  const int rc = check_head_inputs(hidden, ldh, weight, ldw, markov, ldm, factors, teacher, t_dtype, ldt, targs, labels,
                                   weights, valid, n, d, v, k, dl, ldd, row_stats, metrics, workspace, workspace_bytes,
                                   kCheckForward, &nt);
  if (rc) return rc;
  ns::SlotArgs a{labels, weights, valid, n, k, c_ce, c_kl, inv_acc};
  const ns::TeacherSpec ts{targs ? targs->rows : nullptr, nt, targs ? targs->lse : nullptr};
  return hip_status(ns::lmhead_forward(hidden, ldh, weight, ldw, markov, ldm, factors, teacher, t_dtype, ldt, d, v,
                                       a, &ts, dl, ldd, row_stats, metrics, workspace,
                                       reinterpret_cast<hipStream_t>(stream)),
                    name);
}

}  // namespace

extern "C" {

int ns_lmhead_ce_kl_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                        int64_t ldm, const void* teacher, int t_dtype, int64_t ldt,
                        const ns_teacher_args* teacher_args, const int64_t* labels, const float* weights,
                        const uint8_t* valid, int64_t n, int64_t d, int64_t v, int64_t k, float c_ce, float c_kl,
                        float inv_acc, void* dl, int64_t ldd, float* row_stats, float* metrics, void* workspace,
                        size_t workspace_bytes, ns_stream_t stream) {
  return lmhead_fwd_checked(hidden, ldh, weight, ldw, markov, ldm, nullptr, teacher, t_dtype, ldt, teacher_args,
                            labels, weights, valid, n, d, v, k, c_ce, c_kl, inv_acc, dl, ldd, row_stats, metrics,
                            workspace, workspace_bytes, stream, "ns_lmhead_ce_kl_fwd");
}

int ns_lmhead_ce_kl_fwd_part(int part, const void* hidden, int64_t ldh, const void* weight, int64_t ldw,
                             const void* markov, int64_t ldm, const void* teacher, int t_dtype, int64_t ldt,
                             const ns_teacher_args* teacher_args, const int64_t* labels, const float* weights,
                             int64_t n, int64_t d, int64_t v, float c_ce, float c_kl, float inv_acc, void* dl,
                             int64_t ldd, float* row_stats, void* workspace, size_t workspace_bytes,
                             ns_stream_t stream) {
  if (part != NS_PART_STATS && part != NS_PART_EMIT) return fail(NS_EINVAL, "part must be NS_PART_STATS or NS_PART_EMIT");
  if (part == NS_PART_STATS) dl = nullptr;
  int64_t nt = 0;
  const int rc = check_head_inputs(hidden, ldh, weight, ldw, markov, ldm, nullptr, teacher, t_dtype, ldt, teacher_args,
                                   labels, weights, nullptr, n, d, v, 1, dl, ldd, row_stats, nullptr, workspace,
                                   workspace_bytes, kCheckParts, &nt);
  if (rc) return rc;
  ns::SlotArgs a{labels, weights, nullptr, n, 1, c_ce, c_kl, inv_acc};
  const ns::TeacherSpec ts{teacher_args ? teacher_args->rows : nullptr, nt, teacher_args ? teacher_args->lse : nullptr};
  return hip_status(ns::lmhead_forward(hidden, ldh, weight, ldw, markov, ldm, nullptr, teacher, t_dtype, ldt, d, v, a,
                                       &ts, dl, ldd, row_stats, nullptr, workspace,
                                       reinterpret_cast<hipStream_t>(stream),
                                       part == NS_PART_STATS ? ns::kHeadStats : ns::kHeadEmit),
                    "ns_lmhead_ce_kl_fwd_part");
}

int ns_objective_metrics(const float* row_stats, const float* weights, const uint8_t* valid, int64_t n, int64_t k,
                         float c_ce, float c_kl, float* metrics, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0 (got %lld)", (long long)n);
  if (k < 1 || n % k) return fail(NS_EINVAL, "n (%lld) must be a multiple of the block size k (%lld >= 1)", (long long)n, (long long)k);
  if (!metrics || (n > 0 && (!row_stats || !weights || !valid)))
    return fail(NS_ENULL, "row_stats, weights, valid and metrics must be non-NULL");
  ns::SlotArgs a{nullptr, weights, valid, n, k, c_ce, c_kl, 1.f};
  return hip_status(ns::launch_finalize(nullptr, 1, a, const_cast<float*>(row_stats), metrics,
                                        reinterpret_cast<hipStream_t>(stream)),
                    "ns_objective_metrics");
}

int ns_copy_rows(const void* src, int64_t ld_src, int64_t n_src, const int64_t* map, int64_t n_dst, int64_t row_bytes,
                 void* dst, int64_t ld_dst, ns_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || row_bytes < 0) return fail(NS_EINVAL, "row counts and row_bytes must be >= 0");
  if (row_bytes % 4 || ld_src % 4 || ld_dst % 4 || ld_src < row_bytes || ld_dst < row_bytes)
    return fail(NS_EINVAL, "row_bytes and the pitches must be multiples of 4 with pitches >= row_bytes");
  if (n_dst > 0 && row_bytes > 0 && (!map || !dst || (n_src > 0 && !src))) return fail(NS_ENULL, "src, map and dst must be non-NULL");
  if ((reinterpret_cast<uintptr_t>(src) & 3u) || (reinterpret_cast<uintptr_t>(dst) & 3u))
    return fail(NS_EALIGN, "src and dst need 4-byte aligned base pointers");
  return hip_status(ns::copy_rows(src, ld_src, n_src, map, n_dst, row_bytes, dst, ld_dst,
                                  reinterpret_cast<hipStream_t>(stream)),
                    "ns_copy_rows");
}

}  // extern "C"

namespace {

// Scratch of ns_lmhead_ce_kl_fwd_noalloc: one array per GPU for the life of the process.
// In host code `scratch` names a host-side stand-in, never the device memory: kernels get
// the address hipGetSymbolAddress returns for the current device (kept per device below).
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up once per device.
int scratch_for_current_device(void** out) {
  int dev = 0;
  if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(NS_EINVAL, "device %d beyond the %d devices supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
      return hip_status(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NS_OK;
}

}  // namespace

extern "C" {

int ns_device_init(void) {
  void* ws = nullptr;
  if (const int rc = scratch_for_current_device(&ws)) return rc;
  if (const hipError_t e = ns::lmhead_forward_prepare(); e != hipSuccess)
    return hip_status(e, "hipFuncSetAttribute (head kernels)");
  return NS_OK;
}

int ns_lmhead_ce_kl_fwd_noalloc(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                                int64_t ldm, const void* teacher, int t_dtype, int64_t ldt,
                                const ns_teacher_args* teacher_args, const int64_t* labels, const float* weights,
                                const uint8_t* valid, int64_t n, int64_t d, int64_t v, int64_t k, float c_ce,
                                float c_kl, float inv_acc, void* dl, int64_t ldd, float* row_stats, float* metrics,
                                ns_stream_t stream) {
  const size_t need = n > 0 && v > 0 ? ns::lmhead_workspace_bytes(n, v, d) : 0;
  if (need > kNoAllocScratchBytes)
    return fail(NS_EWORKSPACE,
                "ns_lmhead_ce_kl_fwd_noalloc: n = %lld, v = %lld need %zu bytes of scratch; its static scratch "
                "holds %zu (use ns_lmhead_ce_kl_fwd with a workspace)",
                (long long)n, (long long)v, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (n > 0) {
    const int rc = scratch_for_current_device(&ws);
    if (rc) return rc;
  }
  return lmhead_fwd_checked(hidden, ldh, weight, ldw, markov, ldm, nullptr, teacher, t_dtype, ldt, teacher_args,
                            labels, weights, valid, n, d, v, k, c_ce, c_kl, inv_acc, dl, ldd, row_stats, metrics, ws,
                            kNoAllocScratchBytes, stream, "ns_lmhead_ce_kl_fwd_noalloc");
}

int ns_lmhead_markov_ce_kl_fwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const int64_t* prev,
                               const void* w1, int64_t ldw1, const void* w2, int64_t ldw2, int64_t r,
                               const void* teacher, int t_dtype, int64_t ldt, const ns_teacher_args* teacher_args,
                               const int64_t* labels, const float* weights, const uint8_t* valid, int64_t n,
                               int64_t d, int64_t v, int64_t k, float c_ce, float c_kl, float inv_acc, void* dl,
                               int64_t ldd, float* row_stats, float* metrics, void* workspace,
                               size_t workspace_bytes, ns_stream_t stream) {
  const ns::MarkovFactors f{prev, w1, w2, ldw1, ldw2, r};
  return lmhead_fwd_checked(hidden, ldh, weight, ldw, nullptr, 0, &f, teacher, t_dtype, ldt, teacher_args, labels,
                            weights, valid, n, d, v, k, c_ce, c_kl, inv_acc, dl, ldd, row_stats, metrics, workspace,
                            workspace_bytes, stream, "ns_lmhead_markov_ce_kl_fwd");
}

int ns_lmhead_ce_kl_bwd(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                        int64_t ldm, const int64_t* prev, const void* w1, int64_t ldw1, const void* w2, int64_t ldw2,
                        int64_t r, const void* teacher, int t_dtype, int64_t ldt, const ns_teacher_args* teacher_args,
                        const int64_t* labels, const float* weights, int64_t n, int64_t d, int64_t v, float c_ce,
                        float c_kl, float inv_acc, const float* row_stats, void* dl, int64_t ldd, void* workspace,
                        size_t workspace_bytes, ns_stream_t stream) {
  if (markov && r != 0) return fail(NS_EINVAL, "pass either a dense Markov addend or factors (r > 0), not both");
  if (r < 0) return fail(NS_EINVAL, "Markov rank must be >= 0 (got %lld)", (long long)r);
  const ns::MarkovFactors f{prev, w1, w2, ldw1, ldw2, r};
  const ns::MarkovFactors* factors = r > 0 ? &f : nullptr;
  int64_t nt = 0;
  const int rc = check_head_inputs(hidden, ldh, weight, ldw, markov, ldm, factors, teacher, t_dtype, ldt, teacher_args,
                                   labels, weights, nullptr, n, d, v, 1, dl, ldd, row_stats, nullptr, workspace,
                                   workspace_bytes, kCheckReemit, &nt);
  if (rc) return rc;
  ns::SlotArgs a{labels, weights, nullptr, n, 1, c_ce, c_kl, inv_acc};
  const ns::TeacherSpec ts{teacher_args ? teacher_args->rows : nullptr, nt, teacher_args ? teacher_args->lse : nullptr};
  return hip_status(ns::lmhead_emit_dlogits(hidden, ldh, weight, ldw, markov, ldm, factors, teacher, t_dtype, ldt, d,
                                            v, a, &ts, row_stats, dl, ldd, workspace,
                                            reinterpret_cast<hipStream_t>(stream)),
                    "ns_lmhead_ce_kl_bwd");
}

int ns_lmhead_teacher_logits(const void* x, int64_t ldx, const int64_t* rows, int64_t n_rows, const void* weight,
                             int64_t ldw, void* out, int64_t ldo, float* lse, int64_t n, int64_t v, int64_t d,
                             void* workspace, size_t workspace_bytes, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (v < 8 || v % 8) return fail(NS_EINVAL, "vocabulary size must be a positive multiple of 8 (got %lld)", (long long)v);
  if (d < 64 || d % 64) return fail(NS_EINVAL, "hidden size must be a positive multiple of 64 (got %lld)", (long long)d);
  const int64_t nx = rows ? n_rows : n;
  if (rows && (nx < 1 || nx >= (int64_t(1) << 31)))
    return fail(NS_EINVAL, "n_rows must be in [1, 2^31) (got %lld)", (long long)nx);
  int rc;
  if ((rc = check_matrix(x, nx, d, ldx, "x"))) return rc;
  if ((rc = check_matrix(weight, v, d, ldw, "weight"))) return rc;
  if ((rc = check_matrix(out, n, v, ldo, "out"))) return rc;
  if (n > 0 && rows == nullptr && n_rows != 0 && n_rows != n)
    return fail(NS_EINVAL, "n_rows %lld without rows must equal n", (long long)n_rows);
  // gathered x rows are addressed with 32-bit byte offsets from its base
  if (rows && nx * ldx * 2 >= (int64_t(1) << 32))
    return fail(NS_EINVAL, "x spans %lld bytes; at most 4 GiB with rows", (long long)(nx * ldx * 2));
  if (!aligned(x) || !aligned(weight) || !aligned(out) || ldx % 8 || ldw % 8 || ldo % 8)
    return fail(NS_EALIGN, "teacher head needs 16-byte aligned base pointers and rows");
  if (lse) {
    const size_t need = ns::lmhead_linear_lse_workspace_bytes(n, v);
    if (n > 0 && (!workspace || workspace_bytes < need))
      return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  }
  return hip_status(ns::lmhead_linear_lse(x, ldx, rows, nx, weight, ldw, nullptr, 0, out, ldo, lse, n, v, d, workspace,
                                          reinterpret_cast<hipStream_t>(stream)),
                    "ns_lmhead_teacher_logits");
}

int ns_lmhead_bwd(const void* dl, int64_t ldd, const void* weight, int64_t ldw, void* dh, int64_t lddh,
                  int64_t n, int64_t v, int64_t d, void* workspace, size_t workspace_bytes, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (v < 8 || v % 8) return fail(NS_EINVAL, "vocabulary size must be a positive multiple of 8 (got %lld)", (long long)v);
  if (d < 8 || d % 8) return fail(NS_EINVAL, "hidden size must be a positive multiple of 8 (got %lld)", (long long)d);
  int rc;
  if ((rc = check_matrix(dl, n, v, ldd, "dl"))) return rc;
  if ((rc = check_matrix(weight, v, d, ldw, "weight"))) return rc;
  if ((rc = check_matrix(dh, n, d, lddh, "dh"))) return rc;
  if (!aligned(dl) || !aligned(weight) || !aligned(dh) || ldd % 8 || ldw % 8 || lddh % 4)
    return fail(NS_EALIGN, "dh GEMM needs 16-byte aligned base pointers and rows");
  const size_t need = ns::lmhead_bwd_workspace_bytes(n, v, d);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  return hip_status(ns::lmhead_backward(dl, ldd, weight, ldw, dh, lddh, n, v, d, workspace,
                                        reinterpret_cast<hipStream_t>(stream)),
                    "ns_lmhead_bwd");
}

size_t ns_lmhead_markov_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t r) {
  if (n < 0 || v < 0 || d < 0 || r < 0) return 0;
  return ns::markov_bwd_workspace_bytes(n, v, d, r);
}

int ns_lmhead_markov_bwd(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const int64_t* prev,
                         const void* w1, int64_t ldw1, const void* w2, int64_t ldw2, int64_t r, void* dh,
                         int64_t lddh, const ns_rms_norm_args* norm, void* w1_grad, int64_t ldg1, void* w2_grad,
                         int64_t ldg2, int64_t n, int64_t v, int64_t d, void* workspace, size_t workspace_bytes,
                         ns_stream_t stream) {
  if (n < 0 || n >= (int64_t(1) << 31)) return fail(NS_EINVAL, "n must be in [0, 2^31) (got %lld)", (long long)n);
  if (v < 8 || v % 8 || v >= (int64_t(1) << 31))
    return fail(NS_EINVAL, "vocabulary size must be a positive multiple of 8 below 2^31 (got %lld)", (long long)v);
  if (d < 8 || d % 8) return fail(NS_EINVAL, "hidden size must be a positive multiple of 8 (got %lld)", (long long)d);
  if (r < 64 || r % 64) return fail(NS_EINVAL, "Markov rank must be a positive multiple of 64 (got %lld)", (long long)r);
  if (n > 0 && !prev) return fail(NS_ENULL, "prev is NULL");
  int rc;
  if ((rc = check_matrix(dl, n, v, ldd, "dl"))) return rc;
  if ((rc = check_matrix(weight, v, d, ldw, "weight"))) return rc;
  if ((rc = check_matrix(w1, v, r, ldw1, "w1"))) return rc;
  if ((rc = check_matrix(w2, v, r, ldw2, "w2"))) return rc;
  if ((dh || !norm) && (rc = check_matrix(dh, n, d, lddh, "dh"))) return rc;
  ns::NormBwd nb{};
  if (norm && (rc = check_norm(norm, n, d, &nb))) return rc;
  if ((rc = check_matrix(w1_grad, v, r, ldg1, "w1_grad"))) return rc;
  if ((rc = check_matrix(w2_grad, v, r, ldg2, "w2_grad"))) return rc;
  if (!aligned(dl) || !aligned(weight) || !aligned(w1) || !aligned(w2) || !aligned(dh) || !aligned(w1_grad) ||
      !aligned(w2_grad) || ldd % 8 || ldw % 8 || ldw1 % 8 || ldw2 % 8 || lddh % (norm ? 8 : 4) || ldg1 % 8 ||
      ldg2 % 8)
    return fail(NS_EALIGN, "Markov backward needs 16-byte aligned base pointers and rows");
  const size_t need = ns::markov_bwd_workspace_bytes(n, v, d, r);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  const ns::MarkovFactors f{prev, w1, w2, ldw1, ldw2, r};
  return hip_status(ns::markov_backward(dl, ldd, weight, ldw, f, dh, lddh, norm ? &nb : nullptr, w1_grad, ldg1,
                                        w2_grad, ldg2, n, v, d, workspace, workspace_bytes,
                                        reinterpret_cast<hipStream_t>(stream)),
                    "ns_lmhead_markov_bwd");
}

int ns_rms_norm_fwd(const void* x, int64_t ldx, const void* weight, int64_t n, int64_t d, float eps, void* out,
                    int64_t ldo, void* normalized, int64_t ldn, float* inv, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (d < 8 || d % 8 || d > ns::kMaxNormD)
    return fail(NS_EINVAL, "rms-norm hidden size must be a multiple of 8 up to %lld (got %lld)",
                (long long)ns::kMaxNormD, (long long)d);
  int rc;
  if ((rc = check_matrix(x, n, d, ldx, "x"))) return rc;
  if ((rc = check_matrix(out, n, d, ldo, "out"))) return rc;
  if (normalized && (rc = check_matrix(normalized, n, d, ldn, "normalized"))) return rc;
  if (n > 0 && (!weight || !inv)) return fail(NS_ENULL, "weight and inv must be non-NULL");
  if (!aligned(x) || !aligned(out) || !aligned(weight) || (normalized && !aligned(normalized)) || ldx % 8 || ldo % 8 ||
      (normalized && ldn % 8))
    return fail(NS_EALIGN, "rms-norm operands need 16-byte aligned base pointers and rows");
  return hip_status(ns::rms_norm_forward(x, ldx, weight, n, d, eps, out, ldo, normalized, ldn, inv,
                                         reinterpret_cast<hipStream_t>(stream)),
                    "ns_rms_norm_fwd");
}

int ns_rms_norm_bwd(const void* dy, int64_t lddy, const ns_rms_norm_args* norm, int64_t n, int64_t d, void* workspace,
                    size_t workspace_bytes, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (d < 8) return fail(NS_EINVAL, "hidden size must be >= 8 (got %lld)", (long long)d);
  int rc;
  ns::NormBwd nb{};
  if ((rc = check_norm(norm, n, d, &nb))) return rc;
  if ((rc = check_matrix(dy, n, d, lddy, "dy"))) return rc;
  if (!aligned(dy) || lddy % 8) return fail(NS_EALIGN, "dy needs a 16-byte aligned base pointer and rows");
  const size_t need = ns::norm_bwd_workspace_bytes(n, d);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  return hip_status(ns::rms_norm_backward_rows(nullptr, 0, dy, lddy, nb, nullptr, 0, n, d, workspace,
                                               reinterpret_cast<hipStream_t>(stream)),
                    "ns_rms_norm_bwd");
}

int ns_lmhead_norm_bwd(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const ns_rms_norm_args* norm,
                       void* dh, int64_t lddh, int64_t n, int64_t v, int64_t d, void* workspace,
                       size_t workspace_bytes, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (v < 8 || v % 8) return fail(NS_EINVAL, "vocabulary size must be a positive multiple of 8 (got %lld)", (long long)v);
  if (d < 8) return fail(NS_EINVAL, "hidden size must be >= 8 (got %lld)", (long long)d);
  int rc;
  ns::NormBwd nb{};
  if ((rc = check_norm(norm, n, d, &nb))) return rc;
  if ((rc = check_matrix(dl, n, v, ldd, "dl"))) return rc;
  if ((rc = check_matrix(weight, v, d, ldw, "weight"))) return rc;
  if (dh && (rc = check_matrix(dh, n, d, lddh, "dh"))) return rc;
  if (!aligned(dl) || !aligned(weight) || !aligned(dh) || ldd % 8 || ldw % 8 || (dh && lddh % 8))
    return fail(NS_EALIGN, "dh GEMM needs 16-byte aligned base pointers and rows");
  const size_t need = ns::lmhead_bwd_workspace_bytes(n, v, d, 0, true);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  return hip_status(ns::lmhead_backward_ext(dl, ldd, weight, ldw, nullptr, 0, 0, dh, lddh, nullptr, &nb, n, v, d,
                                            workspace, reinterpret_cast<hipStream_t>(stream)),
                    "ns_lmhead_norm_bwd");
}

int ns_pooled_tail(const float* metrics, int64_t count, int64_t world_size, int64_t accumulation_steps, float* out,
                   ns_stream_t stream) {
  if (count < 1) return fail(NS_EINVAL, "count must be >= 1 (got %lld)", (long long)count);
  if (world_size < 1 || accumulation_steps < 1 || world_size * accumulation_steps > (int64_t(1) << 24))
    return fail(NS_EINVAL, "world_size and accumulation_steps must be >= 1 with a product <= 2^24");
  if (!metrics || !out) return fail(NS_ENULL, "metrics and out must be non-NULL");
  return hip_status(ns::pooled_tail(metrics, count, world_size, accumulation_steps, out,
                                    reinterpret_cast<hipStream_t>(stream)),
                    "ns_pooled_tail");
}

int ns_scale_gradient(void* grad, int dtype, int64_t n, const float* factor, ns_stream_t stream) {
  if (!dtype_ok(dtype)) return fail(NS_EDTYPE, "unsupported gradient dtype code %d", dtype);
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (n > 0 && (!grad || !factor)) return fail(NS_ENULL, "grad and factor must be non-NULL");
  if (!aligned(grad)) return fail(NS_EALIGN, "grad must be 16-byte aligned");
  return hip_status(ns::scale_gradient(grad, dtype, n, factor, reinterpret_cast<hipStream_t>(stream)),
                    "ns_scale_gradient");
}

int ns_lmhead_linear(const void* x, int64_t ldx, const void* weight, int64_t ldw, const void* addend,
                     int64_t lda, void* out, int64_t ldo, int64_t n, int64_t v, int64_t d, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (v < 8 || v % 8) return fail(NS_EINVAL, "vocabulary size must be a positive multiple of 8 (got %lld)", (long long)v);
  if (d < 64 || d % 64) return fail(NS_EINVAL, "hidden size must be a positive multiple of 64 (got %lld)", (long long)d);
  int rc;
  if ((rc = check_matrix(x, n, d, ldx, "x"))) return rc;
  if ((rc = check_matrix(weight, v, d, ldw, "weight"))) return rc;
  if (addend && (rc = check_matrix(addend, n, v, lda, "addend"))) return rc;
  if ((rc = check_matrix(out, n, v, ldo, "out"))) return rc;
  if (!aligned(x) || !aligned(weight) || !aligned(out) || (addend && !aligned(addend)) || ldx % 8 || ldw % 8 ||
      ldo % 8 || (addend && lda % 8))
    return fail(NS_EALIGN, "linear needs 16-byte aligned base pointers and rows");
  return hip_status(ns::lmhead_linear(x, ldx, weight, ldw, addend, lda, out, ldo, n, v, d,
                                      reinterpret_cast<hipStream_t>(stream)),
                    "ns_lmhead_linear");
}

int ns_fp8_teacher_logits(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const float* scale,
                          void* out, int64_t ldo, float* lse, int64_t n, int64_t v, int64_t d, void* workspace,
                          size_t workspace_bytes, ns_stream_t stream) {
  if (n < 0) return fail(NS_EINVAL, "n must be >= 0");
  if (v < 128 || v % 128 || d < 128 || d % 128) return fail(NS_EINVAL, "Expected checkpoint's 128x128 FP8 weight blocks");
  int rc;
  if ((rc = check_matrix(x, n, d, ldx, "x"))) return rc;
  if ((rc = check_matrix(wq, v, d, ldw, "wq"))) return rc;
  if ((rc = check_matrix(out, n, v, ldo, "out"))) return rc;
  if (!scale) return fail(NS_ENULL, "scale is NULL");
  if (!aligned(x) || !aligned(wq) || !aligned(out) || ldx % 8 || ldw % 16 || ldo % 8)
    return fail(NS_EALIGN, "fp8 head needs 16-byte aligned base pointers and rows");
  const size_t need = ns::fp8_workspace_bytes(n, v, d);
  if (n > 0 && (!workspace || workspace_bytes < need))
    return fail(NS_EWORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return fail(NS_EALIGN, "workspace must be 256-byte aligned");
  return hip_status(ns::fp8_teacher_logits(x, ldx, wq, ldw, scale, out, ldo, lse, n, v, d, workspace,
                                           reinterpret_cast<hipStream_t>(stream)),
                    "ns_fp8_teacher_logits");
}

int ns_fp8_quantize_rows(const void* x, int64_t ldx, int64_t n, int64_t d, uint8_t* q, float* xs,
                         ns_stream_t stream) {
  if (n < 0 || d < 128 || d % 128) return fail(NS_EINVAL, "d must be a positive multiple of 128");
  int rc;
  if ((rc = check_matrix(x, n, d, ldx, "x"))) return rc;
  if (n > 0 && (!q || !xs)) return fail(NS_ENULL, "q and xs must be non-NULL");
  if ((reinterpret_cast<uintptr_t>(x) & 3u) || ldx % 2) return fail(NS_EALIGN, "x rows must be 4-byte aligned");
  return hip_status(ns::fp8_quantize_rows(x, ldx, n, d, q, xs, reinterpret_cast<hipStream_t>(stream)),
                    "ns_fp8_quantize_rows");
}

int ns_prepare_slots(const int64_t* ids, const float* loss_mask, const int64_t* anchors, const uint8_t* keep,
                     int64_t b, int64_t s, int64_t nb, int64_t k, float gamma, int64_t* target_ids,
                     int64_t* previous, float* weights, uint8_t* valid, int64_t* teacher_indices,
                     ns_stream_t stream) {
  if (s < 1) return fail(NS_EINVAL, "Empty input sequence");
  if (b < 0 || nb < 0) return fail(NS_EINVAL, "batch and block counts must be >= 0");
  if (k < 1) return fail(NS_EINVAL, "block_size must be positive");
  if (b * nb > 0 && (!ids || !loss_mask || !anchors || !keep || !target_ids || !previous || !weights || !valid ||
                     !teacher_indices))
    return fail(NS_ENULL, "every tensor argument must be non-NULL");
  return hip_status(ns::prepare_slots(ids, loss_mask, anchors, keep, b, s, nb, k, gamma, target_ids, previous,
                                      weights, valid, teacher_indices, reinterpret_cast<hipStream_t>(stream)),
                    "ns_prepare_slots");
}

}  // extern "C"
