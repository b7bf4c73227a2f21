// Pooled-normalisation tail: the metric pooling of the training loop
// (nanospec/train.py:525-535) and the gradient factor of the optimizer step
// (nanospec/shard.py:318-330), on the device so nothing waits for the host.
//
// The reference all-reduces [numerator, denominator, accept_len_sum, accept_len_total]
// over ranks; here the caller hands over `count` LossMetrics buffers ([count][6], one per
// micro-batch or per rank after a gather) and they are summed in index order.
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

// out = (loss, accept_len, gradient factor, pooled denominator)
__global__ __launch_bounds__(64) void pooled_tail_kernel(const float* __restrict__ metrics, int64_t count,
                                                         float world_acc, float* __restrict__ out) {
  if (threadIdx.x != 0) return;
  float num = 0.f, den = 0.f, asum = 0.f, atot = 0.f;
  for (int64_t i = 0; i < count; ++i) {
    const float* m = metrics + i * 6;   // ce, kl, numerator, denominator, accept_len_sum, accept_len_total
    num += m[2];
    den += m[3];
    asum += m[4];
    atot += m[5];
  }
  out[0] = num / fmaxf(den, 1e-6f);           // train.py:533
  out[1] = asum / fmaxf(atot, 1.0f);          // train.py:534
  // shard.py:323-327: world * accumulation_steps / max(den, 1e-6), 0 unless den > 0.  A
  // Python int over a tensor is evaluated as reciprocal(tensor) * int: two roundings, kept
  // here so the factor is the same fp32 value
  out[2] = den > 0.f ? (1.0f / fmaxf(den, 1e-6f)) * world_acc : 0.f;
  out[3] = den;
}

// grad *= *factor (shard.py:330), 8 elements per thread; the factor is read on the device.
// torch's mul_ of a bf16 tensor by a 0-d fp32 tensor casts the factor to the common dtype
// (bf16) first, then multiplies in fp32 and rounds once; bf16 gradients do the same.
template <typename T>
__global__ __launch_bounds__(256) void scale_kernel(T* __restrict__ g, int64_t n, const float* __restrict__ factor) {
  const float f = sizeof(T) == 2 ? bf16_to_f32(f32_to_bf16(*factor)) : *factor;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i + 8 <= n) {
    float x[8];
    load8(g + i, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= f;
    store8(g + i, x);
  } else {
    for (int64_t j = i; j < n; ++j) store1(g + j, load1(g + j) * f);
  }
}

}  // namespace

hipError_t pooled_tail(const float* metrics, int64_t count, int64_t world_size, int64_t accumulation_steps,
                       float* out, hipStream_t st) {
  NS_TIMED("pooled_tail", st);
  hipLaunchKernelGGL(pooled_tail_kernel, dim3(1), dim3(64), 0, st, metrics, count,
                     (float)(world_size * accumulation_steps), out);
  return hipGetLastError();
}

hipError_t scale_gradient(void* grad, int dtype, int64_t n, const float* factor, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int64_t threads = (n + 7) / 8;
  const dim3 grid((unsigned)((threads + 255) / 256));
  NS_TIMED("scale_gradient", st);
  if (dtype == kBF16)
    hipLaunchKernelGGL(scale_kernel<uint16_t>, grid, dim3(256), 0, st, static_cast<uint16_t*>(grad), n, factor);
  else
    hipLaunchKernelGGL(scale_kernel<float>, grid, dim3(256), 0, st, static_cast<float*>(grad), n, factor);
  return hipGetLastError();
}

}  // namespace ns
