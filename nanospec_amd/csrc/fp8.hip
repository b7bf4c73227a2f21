// FP8 teacher head: logits = bf16( dequant(x) . dequant(W)^T ) with the numerics of
// nanospec/ops.py:183-200 (fp8_linear):
//   activations: per 1x128 block, xs = amax / 448, q = e4m3(clamp(x / max(xs, tiny), +-448))
//   weights:     e4m3 codes with one fp32 scale per 128 x 128 block (scale multiplies)
//   product:     sum over 128-wide K blocks of xs[t, kb] * s[v/128, kb] * (q_x . q_w)_kb,
//                accumulated in fp32 and rounded once to bf16.
// The block dot products run on gfx950's fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4 with
// unit e8m0 scales): e4m3 x e4m3 products are exact in fp32, so only the fp32
// accumulation order differs from the reference's dequantise-then-fp32-GEMM.
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_t;

constexpr int kQBlock = 128;     // quantisation block (K) and weight-scale block (rows, K)
constexpr int TM = 128;          // vocab rows per workgroup tile (one weight-scale row block)
constexpr int TN = 128;          // tokens per workgroup tile
constexpr int kThreads = 256;    // 4 waves as 2 (vocab) x 2 (tokens), 64 x 64 each
constexpr int kTileBytes = TM * kQBlock;         // 16 KB per operand per stage
constexpr int kLdsBytes = 4 * kTileBytes;        // 2 stages x 2 operands = 64 KB
constexpr int kNumXcd = 8;

// float in [-448, 448] -> OCP e4m3 (fn) code, round to nearest even; -0 keeps its sign.
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0.015625f) {               // below 2^-6: subnormal steps of 2^-9
    code = (uint32_t)rintf(a * 512.0f);
  } else {                           // keep 3 mantissa bits, RNE on the 20 dropped bits
    const uint32_t ab = __float_as_uint(a);
    const uint32_t r = ab + 0x7FFFFu + ((ab >> 20) & 1u);
    code = (r >> 20) - (120u << 3);  // exponent bias 127 -> 7
  }
  return code | sign;
}

// One wave per (row, 128-block): lane l owns elements 2l, 2l+1.
__global__ __launch_bounds__(256) void fp8_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t n,
                                                        int64_t d, uint8_t* __restrict__ q,
                                                        float* __restrict__ xs) {
  const int64_t nb = d / kQBlock;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= n * nb) return;
  const int64_t row = item / nb, kb = item % nb;
  const int lane = threadIdx.x & 63;
  const uint32_t w = *reinterpret_cast<const uint32_t*>(x + row * ldx + kb * kQBlock + 2 * lane);
  const float x0 = bf16_lo(w), x1 = bf16_hi(w);
  float amax = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float s = __fdiv_rn(amax, 448.0f);
  const float den = fmaxf(s, 1.17549435e-38f);   // clamp_min(torch.finfo(float32).tiny)
  const float q0 = fminf(fmaxf(__fdiv_rn(x0, den), -448.0f), 448.0f);
  const float q1 = fminf(fmaxf(__fdiv_rn(x1, den), -448.0f), 448.0f);
  const uint16_t codes = (uint16_t)(e4m3_code(q0) | (e4m3_code(q1) << 8));
  *reinterpret_cast<uint16_t*>(q + row * d + kb * kQBlock + 2 * lane) = codes;
  if (lane == 0) xs[row * nb + kb] = s;
}

__device__ __forceinline__ int swz(int row) { return ((row & 7) + ((row >> 3) & 1)) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 128 + ((chunk ^ swz(row)) << 4); }

struct Fp8Params {
  const uint8_t* qx;       // [N, d] e4m3 codes (row stride d)
  const float* xs;         // [N, d/128]
  const uint8_t* wq;       // [V, d] e4m3 codes
  const float* ws;         // [V/128, d/128]
  int64_t ldw;
  uint16_t* out;           // [N, V] bf16
  int64_t ldo;
  int64_t n, v, d;
  int vt, tt;              // vocab tiles, token tiles
};

// 128 rows x 128 bytes tile -> registers (4 x 16 B per thread), rows >= rmax clamped.
__device__ __forceinline__ void load_rows(uint4 (&r)[4], const uint8_t* base, int64_t ld, int64_t r0,
                                          int64_t rmax, int64_t k0) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t row = r0 + i * 32 + (tid >> 3);
    row = row < rmax ? row : rmax - 1;
    r[i] = *reinterpret_cast<const uint4*>(base + row * ld + k0 + (tid & 7) * 16);
  }
}

__device__ __forceinline__ void store_rows(const uint4 (&r)[4], lds_t* lds) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = i * 32 + (tid >> 3);
    const u32x4_t y = {r[i].x, r[i].y, r[i].z, r[i].w};
    *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(lds + lds_off(row, tid & 7)) = y;
  }
}

// 32 fp8 K-entries (two 16-byte chunks) of LDS row `row` for MFMA K-half `kk`.
__device__ __forceinline__ i32x8_t frag(const lds_t* base, int row, int kk, int kh) {
  const int c = kk * 4 + kh * 2;
  const u32x4_t lo = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(base + lds_off(row, c));
  const u32x4_t hi = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(base + lds_off(row, c + 1));
  i32x8_t r;
  r[0] = (int)lo[0]; r[1] = (int)lo[1]; r[2] = (int)lo[2]; r[3] = (int)lo[3];
  r[4] = (int)hi[0]; r[5] = (int)hi[1]; r[6] = (int)hi[2]; r[7] = (int)hi[3];
  return r;
}

__global__ __launch_bounds__(kThreads) void fp8_head_kernel(Fp8Params p) {
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_t* lds = (lds_t*)lds_raw;
  const int G = gridDim.x;
  int L = blockIdx.x;
  if (G % kNumXcd == 0) L = (L % kNumXcd) * (G / kNumXcd) + L / kNumXcd;
  const int tt = L % p.tt, vt = L / p.tt;   // consecutive ids share the weight tile
  const int64_t v0 = (int64_t)vt * TM, t0 = (int64_t)tt * TN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, kh = lane >> 5;
  const int KB = (int)(p.d / kQBlock);
  const float* wsrow = p.ws + (int64_t)vt * KB;     // the tile is one weight-scale row block

  int64_t tok[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t t = t0 + wn * 64 + j * 32 + r;
    tok[j] = t < p.n ? t : p.n - 1;
  }

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  uint4 ra[4], rb[4];
  load_rows(ra, p.wq, p.ldw, v0, p.v, 0);
  load_rows(rb, p.qx, p.d, t0, p.n, 0);
  store_rows(ra, lds);
  store_rows(rb, lds + kTileBytes);
  __syncthreads();
  if (KB > 1) {
    load_rows(ra, p.wq, p.ldw, v0, p.v, kQBlock);
    load_rows(rb, p.qx, p.d, t0, p.n, kQBlock);
  }
  for (int kb = 0; kb < KB; ++kb) {
    const lds_t* la = lds + (kb & 1) * 2 * kTileBytes;
    const lds_t* lb = la + kTileBytes;
    const float sw = wsrow[kb];
    float c[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) c[j] = p.xs[tok[j] * KB + kb] * sw;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x16_t part = {};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const i32x8_t a = frag(la, wm * 64 + i * 32 + r, kk, kh);
          const i32x8_t b = frag(lb, wn * 64 + j * 32 + r, kk, kh);
          part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, part, 0, 0, 0, 127, 0, 127);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = __builtin_fmaf(c[j], part[e], acc[i][j][e]);
      }
    }
    if (kb + 1 < KB) {
      lds_t* nxt = lds + ((kb + 1) & 1) * 2 * kTileBytes;
      store_rows(ra, nxt);
      store_rows(rb, nxt + kTileBytes);
    }
    __syncthreads();
    if (kb + 2 < KB) {
      load_rows(ra, p.wq, p.ldw, v0, p.v, (int64_t)(kb + 2) * kQBlock);
      load_rows(rb, p.qx, p.d, t0, p.n, (int64_t)(kb + 2) * kQBlock);
    }
  }

  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t t = t0 + wn * 64 + j * 32 + r;
    if (t >= p.n) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t v = v0 + wm * 64 + i * 32 + 8 * g + 4 * h;
        if (v < p.v) {
          uint2 o;
          o.x = pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
          o.y = pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          *reinterpret_cast<uint2*>(p.out + t * p.ldo + v) = o;
        }
      }
  }
}

}  // namespace

hipError_t fp8_quantize_rows(const void* x, int64_t ldx, int64_t n, int64_t d, uint8_t* q, float* xs,
                             hipStream_t st) {
  const int64_t items = n * (d / kQBlock);
  if (items == 0) return hipSuccess;
  NS_TIMED("fp8_quant", st);
  hipLaunchKernelGGL(fp8_quant_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st,
                     static_cast<const uint16_t*>(x), ldx, n, d, q, xs);
  return hipGetLastError();
}

size_t fp8_workspace_bytes(int64_t n, int64_t d) {
  return align_up((size_t)n * d, 256) + align_up((size_t)n * (d / kQBlock) * sizeof(float), 256);
}

hipError_t fp8_teacher_logits(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const float* scale,
                              void* out, int64_t ldo, int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st) {
  if (n == 0 || v == 0) return hipSuccess;
  uint8_t* qx = static_cast<uint8_t*>(ws);
  float* xs = reinterpret_cast<float*>(static_cast<char*>(ws) + align_up((size_t)n * d, 256));
  {
    hipError_t e = fp8_quantize_rows(x, ldx, n, d, qx, xs, st);
    if (e != hipSuccess) return e;
  }
  Fp8Params p;
  p.qx = qx; p.xs = xs; p.wq = wq; p.ws = scale; p.ldw = ldw;
  p.out = static_cast<uint16_t*>(out); p.ldo = ldo;
  p.n = n; p.v = v; p.d = d;
  p.vt = (int)((v + TM - 1) / TM);
  p.tt = (int)((n + TN - 1) / TN);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_head_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  NS_TIMED("fp8_head_gemm", st);
  hipLaunchKernelGGL(fp8_head_kernel, dim3((unsigned)(p.vt * p.tt)), dim3(kThreads), kLdsBytes, st, p);
  return hipGetLastError();
}

}  // namespace ns
