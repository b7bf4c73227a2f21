// Row copies by an index map: dst row r = src row map[r], zeros where map[r] is outside
// [0, n_src).  The fused head uses them to run pass 2 and the dh GEMM on the rows whose
// outputs are not all zero (head.lm_head_ce_kl_loss(skip_masked_rows=True)): gathering those
// rows of hidden and the Markov logits, and scattering the compact dl and dh back with zero
// rows between.  HBM-bound: each byte is read and written once, with
// non-temporal 16-byte accesses (the compacted rows are not read again soon).
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

typedef uint32_t u32x4r_t __attribute__((ext_vector_type(4)));

// One thread per 16-byte chunk (W = 16) or 4-byte word (W = 4) of a destination row.
template <int W>
__global__ __launch_bounds__(256) void copy_rows_kernel(const char* __restrict__ src, int64_t ld_src, int64_t n_src,
                                                        const int64_t* __restrict__ map, int64_t n_dst,
                                                        int64_t row_bytes, char* __restrict__ dst, int64_t ld_dst) {
  const int64_t per_row = row_bytes / W;
  const int64_t total = n_dst * per_row;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / per_row, c = i - r * per_row;
    const int64_t s = map[r];
    char* to = dst + r * ld_dst + c * W;
    if constexpr (W == 16) {
      u32x4r_t x = {0u, 0u, 0u, 0u};
      if (s >= 0 && s < n_src) x = __builtin_nontemporal_load(reinterpret_cast<const u32x4r_t*>(src + s * ld_src + c * W));
      __builtin_nontemporal_store(x, reinterpret_cast<u32x4r_t*>(to));
    } else {
      uint32_t x = 0u;
      if (s >= 0 && s < n_src) x = *reinterpret_cast<const uint32_t*>(src + s * ld_src + c * W);
      *reinterpret_cast<uint32_t*>(to) = x;
    }
  }
}

}  // namespace

hipError_t copy_rows(const void* src, int64_t ld_src, int64_t n_src, const int64_t* map, int64_t n_dst,
                     int64_t row_bytes, void* dst, int64_t ld_dst, hipStream_t st) {
  if (n_dst == 0 || row_bytes == 0) return hipSuccess;
  const bool vec = row_bytes % 16 == 0 && ld_src % 16 == 0 && ld_dst % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(src) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
  const int64_t items = n_dst * (row_bytes / (vec ? 16 : 4));
  const int64_t blocks = (items + 255) / 256 < 8192 ? (items + 255) / 256 : 8192;
  NS_TIMED("copy_rows", st);
  if (vec)
    hipLaunchKernelGGL(copy_rows_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<const char*>(src),
                       ld_src, n_src, map, n_dst, row_bytes, static_cast<char*>(dst), ld_dst);
  else
    hipLaunchKernelGGL(copy_rows_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<const char*>(src),
                       ld_src, n_src, map, n_dst, row_bytes, static_cast<char*>(dst), ld_dst);
  return hipGetLastError();
}

}  // namespace ns
