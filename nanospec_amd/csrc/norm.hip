// final_norm around the LM head (nanospec/train.py:271, 308-310): ops.rms_norm
// (ops.py:48-52) before the head GEMM and ops.rms_norm_backward (ops.py:55-66) after the
// dh GEMM.  The backward reads dh straight from the dh GEMM's split-K partials, so dh
// itself never goes to HBM.
//
// Rounding follows torch's device kernels op by op: every product and sum of the
// reference expression is rounded where torch materialises it (no contraction into
// FMAs), the mean is sum * (1/d), inv^3 is (inv * inv) * inv, and dvar / d is
// dvar * (1/d) (torch divides by a host scalar through its reciprocal).  Only the order
// of the two row sums (sum x^2, sum dz x) differs from torch's reduction tree.
#pragma clang fp contract(off)

#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

constexpr int kThreads = 256;
constexpr int kChunk = kThreads * 8;     // columns per pass of a workgroup (8 per thread)
constexpr int kMaxChunks = kMaxNormD / kChunk;

__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Sum over the workgroup, fixed order (waves 0..3); red = 4 floats of LDS.
__device__ __forceinline__ float block_sum(float x, float* red) {
  x = wave_sum(x);
  const int wv = threadIdx.x >> 6;
  __syncthreads();   // red is free (a previous call's readers are done)
  if ((threadIdx.x & 63) == 0) red[wv] = x;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// One workgroup per row: inv = rsqrt(mean(x^2) + eps), normalized = bf16(x * inv),
// out = bf16(weight * normalized).
__global__ __launch_bounds__(kThreads) void rms_fwd_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const uint16_t* __restrict__ w, int64_t d, float eps,
                                                           uint16_t* __restrict__ out, int64_t ldo,
                                                           uint16_t* __restrict__ normalized, int64_t ldn,
                                                           float* __restrict__ inv_out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  float s = 0.f;
  for (int64_t c = threadIdx.x * 8; c < d; c += kChunk) {
    float xv[8];
    load8(xr + c, xv);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += xv[e] * xv[e];
  }
  const float total = block_sum(s, red);
  const float inv = rsqrtf(total * (1.0f / (float)d) + eps);
  if (threadIdx.x == 0) inv_out[row] = inv;
  for (int64_t c = threadIdx.x * 8; c < d; c += kChunk) {
    float xv[8], wv[8], nv[8], ov[8];
    load8(xr + c, xv);
    load8(w + c, wv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      nv[e] = bf16r(xv[e] * inv);
      ov[e] = wv[e] * nv[e];
    }
    if (normalized) store8(normalized + row * ldn + c, nv);
    store8(out + row * ldo + c, ov);
  }
}

// rms_norm backward over a block of `rows` rows per workgroup.  dy comes either from
// split-K partials part[ksplit][N][d] (fp32, summed in split order and rounded to bf16,
// which is the reference's bf16 dh) or from a bf16 tensor.  Writes dx (bf16) and this
// block's column sums of bf16(dy * normalized) into wpart[block][d] (fp32).
template <bool FROM_PARTS>
__global__ __launch_bounds__(kThreads) void rms_bwd_kernel(const float* __restrict__ part, int ksplit,
                                                           const uint16_t* __restrict__ dy_in, int64_t lddy,
                                                           NormBwd nb, uint16_t* __restrict__ dh_out, int64_t lddh,
                                                           int64_t n, int64_t d, int rows,
                                                           float* __restrict__ wpart) {
  __shared__ float red[4];
  float dwacc[kMaxChunks][8];
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) dwacc[j][e] = 0.f;
  const int64_t r0 = (int64_t)blockIdx.x * rows;
  const int64_t r1 = r0 + rows < n ? r0 + rows : n;
  for (int64_t row = r0; row < r1; ++row) {
    const float inv = nb.inv[row];
    const uint16_t* xr = nb.x + row * nb.ldx;
    float dz[kMaxChunks][8];
    float dinv_p = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
      const int64_t c = (int64_t)j * kChunk + threadIdx.x * 8;
      if (c < d) {
        float dy[8];
        if (FROM_PARTS) {
          load8(part + row * d + c, dy);
          for (int k = 1; k < ksplit; ++k) {
            float t[8];
            load8(part + ((int64_t)k * n + row) * d + c, t);
#pragma unroll
            for (int e = 0; e < 8; ++e) dy[e] += t[e];
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) dy[e] = bf16r(dy[e]);
          if (dh_out) store8(dh_out + row * lddh + c, dy);
        } else {
          load8(dy_in + row * lddy + c, dy);
        }
        float xv[8], wv[8];
        load8(xr + c, xv);
        load8(nb.w + c, wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dz[j][e] = bf16r(dy[e] * wv[e]);                     // (dy * weight).float()
          dwacc[j][e] += bf16r(dy[e] * bf16r(xv[e] * inv));    // dy * normalized, bf16
          dinv_p += dz[j][e] * xv[e];
        }
      }
    }
    const float dinv = block_sum(dinv_p, red);
    const float dvar = dinv * (-0.5f * ((inv * inv) * inv));
    const float q = dvar * (1.0f / (float)d);
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
      const int64_t c = (int64_t)j * kChunk + threadIdx.x * 8;
      if (c < d) {
        float xv[8], dx[8];
        load8(xr + c, xv);
#pragma unroll
        for (int e = 0; e < 8; ++e) dx[e] = dz[j][e] * inv + q * (2.0f * xv[e]);
        store8(nb.dx + row * nb.lddx + c, dx);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    const int64_t c = (int64_t)j * kChunk + threadIdx.x * 8;
    if (c < d) store8(wpart + (int64_t)blockIdx.x * d + c, dwacc[j]);
  }
}

// weight_grad[c] = bf16(sum over blocks of wpart[b][c]): 1024 threads per 256 columns,
// 16 strided groups of blocks each summed in order, then the groups in order.
__global__ __launch_bounds__(1024) void rms_wgrad_kernel(const float* __restrict__ wpart, int64_t nblk, int64_t d,
                                                         uint16_t* __restrict__ wgrad) {
  __shared__ float4 acc[16][64];
  const int q = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 256 + q * 4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < d) {
    for (int64_t b = grp; b < nblk; b += 16) {
      const float4 t = *reinterpret_cast<const float4*>(wpart + b * d + c);
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
  }
  acc[grp][q] = s;
  __syncthreads();
  if (grp == 0 && c < d) {
    float4 t = acc[0][q];
    for (int g = 1; g < 16; ++g) {
      t.x += acc[g][q].x; t.y += acc[g][q].y; t.z += acc[g][q].z; t.w += acc[g][q].w;
    }
    uint2 o;
    o.x = pack_bf16x2(t.x, t.y);
    o.y = pack_bf16x2(t.z, t.w);
    *reinterpret_cast<uint2*>(wgrad + c) = o;
  }
}

}  // namespace

int norm_rows_per_block(int64_t n) {
  // enough workgroups to cover the CUs several times over, few enough column partials
  return n >= 8192 ? 16 : (n >= 2048 ? 4 : 1);
}

size_t norm_bwd_workspace_bytes(int64_t n, int64_t d) {
  const int rows = norm_rows_per_block(n);
  return align_up((size_t)((n + rows - 1) / rows) * d * sizeof(float), 256);
}

hipError_t rms_norm_forward(const void* x, int64_t ldx, const void* weight, int64_t n, int64_t d, float eps,
                            void* out, int64_t ldo, void* normalized, int64_t ldn, float* inv, hipStream_t st) {
  if (n == 0) return hipSuccess;
  NS_TIMED("rms_norm_fwd", st);
  hipLaunchKernelGGL(rms_fwd_kernel, dim3((unsigned)n), dim3(kThreads), 0, st, static_cast<const uint16_t*>(x), ldx,
                     static_cast<const uint16_t*>(weight), d, eps, static_cast<uint16_t*>(out), ldo,
                     static_cast<uint16_t*>(normalized), ldn, inv);
  return hipGetLastError();
}

hipError_t rms_norm_backward_rows(const float* part, int ksplit, const void* dy, int64_t lddy, const NormBwd& nb,
                                  void* dh_out, int64_t lddh, int64_t n, int64_t d, void* ws, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int rows = norm_rows_per_block(n);
  const int64_t nblk = (n + rows - 1) / rows;
  float* wpart = static_cast<float*>(ws);
  hipError_t e;
  {
    NS_TIMED("rms_norm_bwd", st);
    if (part)
      hipLaunchKernelGGL(rms_bwd_kernel<true>, dim3((unsigned)nblk), dim3(kThreads), 0, st, part, ksplit, nullptr,
                         0, nb, static_cast<uint16_t*>(dh_out), lddh, n, d, rows, wpart);
    else
      hipLaunchKernelGGL(rms_bwd_kernel<false>, dim3((unsigned)nblk), dim3(kThreads), 0, st, nullptr, 0,
                         static_cast<const uint16_t*>(dy), lddy, nb, nullptr, 0, n, d, rows, wpart);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  NS_TIMED("rms_norm_wgrad", st);
  hipLaunchKernelGGL(rms_wgrad_kernel, dim3((unsigned)((d + 255) / 256)), dim3(1024), 0, st, wpart, nblk, d,
                     nb.wgrad);
  return hipGetLastError();
}

}  // namespace ns
