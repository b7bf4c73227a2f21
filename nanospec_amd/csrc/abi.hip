// C ABI entry points: argument validation, workspace checks, error text.
#include <stdarg.h>
#include <stdio.h>

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

int check_matrix(const void* p, int64_t n, int64_t cols, int64_t ld, const char* name) {
  if (n > 0 && cols > 0 && !p) return fail(NS_ENULL, "%s is NULL", name);
  if (ld < cols) return fail(NS_EINVAL, "%s: leading dimension %lld < columns %lld", name, (long long)ld, (long long)cols);
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
