// Shared device helpers for the nanospec_amd HIP library (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ns {

constexpr float kLog2e = 1.4426950408889634f;   // log2(e)
constexpr float kLn2 = 0.6931471805599453f;     // ln(2)
constexpr float kNegBig = -3.402823466e+38f;    // running-max sentinel (finite: no inf-inf NaN)

// dtype tags shared with the C ABI (nanospec_hip.h)
enum DType : int { kBF16 = 0, kF32 = 1 };

// ---- bf16 <-> f32 --------------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even f32 -> bf16 pair, packed low|high<<16.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return (uint16_t)(__builtin_bit_cast(uint16_t, (__bf16)x));
}

// exp(x) as 2^(x*log2e) with the hardware exp2; callers fold the scale into an FMA.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// fminf(a, b) for a, b >= +0 or NaN (probabilities): on such values the unsigned order of
// the bit patterns is the float order, and a NaN pattern is above every number, so the
// integer min returns what fminf returns (the number when one side is NaN).  One v_min_u32,
// where fminf costs a v_max_f32 per operand (canonicalising the exp2 results) plus v_min_f32.
__device__ __forceinline__ float min_nonneg(float a, float b) {
  const uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
  return __uint_as_float(x < y ? x : y);
}

// The accept rate of a row, sum_v min(p_v, t_v), as torch.minimum(...).sum(-1) forms it
// (objective.py:42): NaN when any p_v or t_v is NaN.  softmax(x) holds a NaN exactly when x
// holds a NaN or a +inf or is -inf everywhere, and in each of those cases, and only then,
// the row's online log-normaliser is NaN or -inf (a NaN or +inf term makes the running sum
// NaN; an all -inf row leaves it 0).  So the per-entry sums may use min_nonneg, and the
// row's sum is replaced by NaN when either log-normaliser is not finite.
__device__ __forceinline__ float accept_rate_of(float sum, float lse_z, float lse_u) {
  const bool ok = __builtin_fabsf(lse_z) <= 3.402823466e+38f && __builtin_fabsf(lse_u) <= 3.402823466e+38f;
  return ok ? sum : __builtin_nanf("");
}

// ---- 8-element vector loads / stores (16 B for bf16, 32 B for f32) -----------

__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
  f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
  f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

__device__ __forceinline__ void load8(const float* p, float* f) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// Non-temporal loads for a read-once stream: on gfx950 a pure read stream reaches
// 6.7 TB/s with them against 6.0-6.25 TB/s without.
__device__ __forceinline__ void load8_nt(const uint16_t* p, float* f) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
  f[0] = bf16_lo(v[0]); f[1] = bf16_hi(v[0]);
  f[2] = bf16_lo(v[1]); f[3] = bf16_hi(v[1]);
  f[4] = bf16_lo(v[2]); f[5] = bf16_hi(v[2]);
  f[6] = bf16_lo(v[3]); f[7] = bf16_hi(v[3]);
}

__device__ __forceinline__ void load8_nt(const float* p, float* f) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  const f32x4v a = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(p));
  const f32x4v b = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(p) + 1);
  f[0] = a[0]; f[1] = a[1]; f[2] = a[2]; f[3] = a[3];
  f[4] = b[0]; f[5] = b[1]; f[6] = b[2]; f[7] = b[3];
}

__device__ __forceinline__ void store8(uint16_t* p, const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  *reinterpret_cast<uint4*>(p) = v;
}

// Eight values loaded as raw vectors, unpacked to fp32 later: keeping the unpack away from
// the load lets all of a row group's loads be in flight together.
template <typename T>
struct Raw8;
template <>
struct Raw8<uint16_t> {
  uint4 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void unpack(float* f) const {
    f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
  }
};
template <>
struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ void unpack(float* f) const {
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  }
};

// Non-temporal variant: a streamed output that nothing reads back soon.
__device__ __forceinline__ void store8_nt(uint16_t* p, const float* f) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const u32x4v v = {pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7])};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4v*>(p));
}

__device__ __forceinline__ void store8_nt(float* p, const float* f) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  const f32x4v a = {f[0], f[1], f[2], f[3]}, b = {f[4], f[5], f[6], f[7]};
  __builtin_nontemporal_store(a, reinterpret_cast<f32x4v*>(p));
  __builtin_nontemporal_store(b, reinterpret_cast<f32x4v*>(p) + 1);
}

__device__ __forceinline__ void store8(float* p, const float* f) {
  reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
}

__device__ __forceinline__ float load1(const uint16_t* p) { return bf16_to_f32(*p); }
__device__ __forceinline__ float load1(const float* p) { return *p; }
__device__ __forceinline__ void store1(uint16_t* p, float x) { *p = f32_to_bf16(x); }
__device__ __forceinline__ void store1(float* p, float x) { *p = x; }

// ---- online log-sum-exp states -------------------------------------------
// (m, s) represents sum_i exp(x_i) = s * exp(m).  A pair of streams (draft z,
// teacher u) also carries A = sum_i exp(u_i - m_u) (u_i - z_i), rescaled with s_u.

struct LseState {
  float m, s;
};

__device__ __forceinline__ LseState lse_merge(LseState a, LseState b) {
  const float m = fmaxf(a.m, b.m);
  return {m, a.s * fast_exp2((a.m - m) * kLog2e) + b.s * fast_exp2((b.m - m) * kLog2e)};
}

struct PairState {
  float mz, sz, mu, su, A;
};

__device__ __forceinline__ PairState pair_init() { return {kNegBig, 0.f, kNegBig, 0.f, 0.f}; }

__device__ __forceinline__ PairState pair_merge(const PairState& a, const PairState& b) {
  PairState r;
  r.mz = fmaxf(a.mz, b.mz);
  r.sz = a.sz * fast_exp2((a.mz - r.mz) * kLog2e) + b.sz * fast_exp2((b.mz - r.mz) * kLog2e);
  r.mu = fmaxf(a.mu, b.mu);
  const float ca = fast_exp2((a.mu - r.mu) * kLog2e);
  const float cb = fast_exp2((b.mu - r.mu) * kLog2e);
  r.su = a.su * ca + b.su * cb;
  r.A = a.A * ca + b.A * cb;
  return r;
}

// Fold a batch of values into a pair state (z and u of the same vocab entries).
template <int W>
__device__ __forceinline__ void pair_update(PairState& st, const float* z, const float* u) {
  float bz = z[0], bu = u[0];
#pragma unroll
  for (int i = 1; i < W; ++i) {
    bz = fmaxf(bz, z[i]);
    bu = fmaxf(bu, u[i]);
  }
  const float mz = fmaxf(st.mz, bz);
  const float mu = fmaxf(st.mu, bu);
  const float mzl = mz * kLog2e, mul = mu * kLog2e;
  float sz = st.sz * fast_exp2((st.mz - mz) * kLog2e);
  const float cu = fast_exp2((st.mu - mu) * kLog2e);
  float su = st.su * cu;
  float A = st.A * cu;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    sz += fast_exp2(__builtin_fmaf(z[i], kLog2e, -mzl));
    const float e = fast_exp2(__builtin_fmaf(u[i], kLog2e, -mul));
    su += e;
    A = __builtin_fmaf(e, u[i] - z[i], A);
  }
  st = {mz, sz, mu, su, A};
}

// ---- wave / block reductions (wave64) ---------------------------------------

__device__ __forceinline__ PairState wave_reduce(PairState s) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    PairState o;
    o.mz = __shfl_xor(s.mz, off);
    o.sz = __shfl_xor(s.sz, off);
    o.mu = __shfl_xor(s.mu, off);
    o.su = __shfl_xor(s.su, off);
    o.A = __shfl_xor(s.A, off);
    s = pair_merge(s, o);
  }
  return s;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// Per-row partial of the first (statistics) pass over one vocab range.
struct alignas(32) RowPart {
  float mz, sz, mu, su, A, pad0, pad1, pad2;
};

// F.cross_entropy's default ignore_index (objective.py:54): a row with this label has no
// CE term (CE 0) and no CE gradient.  Any other label outside [0, V) makes CE NaN.
constexpr int64_t kIgnoreIndex = -100;

// Per-row statistics returned to the host (layout of row_stats[N][8]).
enum RowStat : int {
  kLseZ = 0, kLseU = 1, kCE = 2, kKL = 3, kAccept = 4, kZy = 5, kRowStatWidth = 8
};

// Metrics layout (LossMetrics field order, objective.py:11-18).
enum Metric : int {
  kMetCE = 0, kMetKL = 1, kMetNum = 2, kMetDen = 3, kMetAccSum = 4, kMetAccTot = 5, kNumMetrics = 6
};

}  // namespace ns
