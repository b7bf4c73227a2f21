// Markov-head backward (nanospec/train.py:303-307):
//   d(previous) = dl . w2                    ops.linear_backward (ops.py:38-45), dx
//   w2.grad     = dl^T . w1[prev]            ops.linear_backward, dw (copied, not accumulated)
//   w1.grad    += index_add(prev, d(prev))   ops.embedding_backward (ops.py:73-74)
// d(previous) comes out of the dh GEMM as extra column tiles (lmhead_backward_ext);
// w2.grad is a K = N GEMM with both operands K-major; the index_add sorts (prev, t) with
// a stable radix sort and lets one wave per distinct id sum that id's rows in token order,
// so the result does not depend on scheduling (the reference's GPU index_add_ does).
#include <hipcub/hipcub.hpp>

#include "ns_gemm.h"
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

constexpr int TM = 256;          // w2.grad rows (vocab) per workgroup tile
constexpr int TN = 256;          // w2.grad columns (rank) per workgroup tile
constexpr int TK = 64;           // tokens per LDS stage
constexpr int kThreads = 256;    // 4 waves as 2 (vocab) x 2 (rank), 128 x 128 each
constexpr int kStage = TK * TN * 2;   // 32 KB per operand per stage (64 K rows x 512 B)
constexpr int kLds = 4 * kStage;      // 2 stages x 2 operands

// E[t] = w1[prev[t]] (bf16 rows of r entries); ids outside [0, V) read row 0 (the forward
// has already turned that row's loss NaN).
__global__ __launch_bounds__(256) void gather_rows_kernel(const int64_t* __restrict__ prev, const uint16_t* __restrict__ w1,
                                                          int64_t ldw1, int64_t n, int64_t v, int64_t r,
                                                          uint16_t* __restrict__ e) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (idx >= n * r) return;
  const int64_t t = idx / r, c = idx % r;
  int64_t id = prev[t];
  id = (id >= 0 && id < v) ? id : 0;
  *reinterpret_cast<uint4*>(e + t * r + c) = *reinterpret_cast<const uint4*>(w1 + id * ldw1 + c);
}

// One MFMA step (16 K rows) from two KN stages: A fragments (vocab rows) and B fragments
// (rank columns), both K-contiguous through transposed LDS reads.
struct KnFrags {
  TrFrag a[4], b[4];
};

__device__ __forceinline__ void read_kn_frags(KnFrags& f, const lds_t* sa, const lds_t* sb, int kk,
                                              const uint32_t (&ta)[4], const uint32_t (&tbv)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f.a[i].lo = tr_read(sa, ta[i] + kk * 8192);
    f.a[i].hi = tr_read(sa, ta[i] + kk * 8192 + 2048);
    f.b[i].lo = tr_read(sb, tbv[i] + kk * 8192);
    f.b[i].hi = tr_read(sb, tbv[i] + kk * 8192 + 2048);
  }
}

__device__ __forceinline__ void mma_kn(f32x16_t (&acc)[4][4], const KnFrags& f) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_join(f.a[i]), tr_join(f.b[j]), acc[i][j], 0, 0, 0);
}

// All four steps of one stage, fragments double-buffered across steps.
__device__ __forceinline__ void stage_kn(f32x16_t (&acc)[4][4], const lds_t* sa, const lds_t* sb,
                                         const uint32_t (&ta)[4], const uint32_t (&tbv)[4]) {
  KnFrags f[2];
  read_kn_frags(f[0], sa, sb, 0, ta, tbv);
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    if (kk < 3) read_kn_frags(f[(kk + 1) & 1], sa, sb, kk + 1, ta, tbv);
    mma_kn(acc, f[kk & 1]);
  }
}

// A partial stage of kvalid (< TK) rows through registers: rows past kvalid are zero,
// columns at or past cmax re-read column chunk 0 (their results are discarded).
__device__ __forceinline__ void load_kn_tail(lds_t* dst, const uint16_t* base, int64_t ld, int64_t c0, int64_t cmax,
                                             int kvalid) {
#pragma unroll
  for (int i = 0; i < (TK * TN / 8) / kThreads; ++i) {
    const int ci = i * kThreads + threadIdx.x;
    const int row = ci >> 5, cn = ci & 31;
    int64_t col = c0 + cn * 8;
    col = col < cmax ? col : c0;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (row < kvalid) x = *reinterpret_cast<const uint4*>(base + (int64_t)row * ld + col);
    const u32x4_t y = {x.x, x.y, x.z, x.w};
    *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(dst + row * 512 + ((cn ^ (4 * (row & 3))) << 4)) = y;
  }
}

struct Dw2Params {
  const uint16_t* dl;   // [N, V] bf16
  int64_t ldd;
  const uint16_t* e;    // [N, r] bf16 (w1[prev])
  uint16_t* w2g;        // [V, r] bf16
  int64_t ldg2;
  int64_t n, v, r;
  int ct;               // rank tiles
};

// w2.grad[v-tile, c-tile] = sum_t dl[t, v-tile]^T e[t, c-tile]: K = tokens, both operands
// filled row-major ([t][v], [t][c]) into LDS and read K-contiguous with tr_b16.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void dw2_kernel(Dw2Params p) {
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_t* lds = (lds_t*)lds_raw;
  const int vt = blockIdx.x / p.ct, ctile = blockIdx.x % p.ct;
  const int64_t v0 = (int64_t)vt * TM, c0 = (int64_t)ctile * TN;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv >> 1, wn = wv & 1;
  DmaTileKN ta, tb;
  ta.init(p.ldd, v0, p.v, wv);
  tb.init(p.r, c0, p.r, wv);
  uint32_t tra[4], trb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    tra[i] = tr_base(wm, i);
    trb[i] = tr_base(wn, i);
  }
  const char* pa = reinterpret_cast<const char*>(p.dl + v0);
  const char* pb = reinterpret_cast<const char*>(p.e + c0);
  const int64_t sa_bytes = (int64_t)TK * p.ldd * 2, sb_bytes = (int64_t)TK * p.r * 2;
  auto buf = [&](int t) -> lds_t* { return lds + (t & 1) * 2 * kStage; };
  const int KTf = (int)(p.n / TK);
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  if (KTf > 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ta.issue(pa, buf(0), wv, i);
      tb.issue(pb, buf(0) + kStage, wv, i);
    }
  }
  for (int t = 0; t < KTf; ++t) {
    fill_barrier();   // stage t landed; everyone is done with stage t - 1's buffer
    if (t + 1 < KTf) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ta.issue(pa + (t + 1) * sa_bytes, buf(t + 1), wv, i);
        tb.issue(pb + (t + 1) * sb_bytes, buf(t + 1) + kStage, wv, i);
      }
    }
    stage_kn(acc, buf(t), buf(t) + kStage, tra, trb);
  }
  const int kvalid = (int)(p.n - (int64_t)KTf * TK);
  if (kvalid > 0) {
    fill_barrier();
    const int64_t k0 = (int64_t)KTf * TK;
    load_kn_tail(lds, p.dl + k0 * p.ldd, p.ldd, v0, p.v, kvalid);
    load_kn_tail(lds + kStage, p.e + k0 * p.r, p.r, c0, p.r, kvalid);
    __syncthreads();
    stage_kn(acc, lds, lds + kStage, tra, trb);
  }
  const int lane = threadIdx.x & 63, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = c0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = v0 + wm * 128 + i * 32 + (e >> 2) * 8 + h * 4 + (e & 3);
        if (row < p.v && col < p.r) p.w2g[row * p.ldg2 + col] = f32_to_bf16(acc[i][j][e]);
      }
    }
}

// Sort keys: the row of w1 each token's d(previous) goes to (V for ids outside [0, V):
// they sort last and are skipped), paired with the token index.
__global__ __launch_bounds__(256) void markov_keys_kernel(const int64_t* __restrict__ prev, int64_t n, int64_t v,
                                                          uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int64_t id = prev[t];
  keys[t] = (id >= 0 && id < v) ? (uint32_t)id : (uint32_t)v;
  vals[t] = (uint32_t)t;
}

// One wave per sorted position; the first position of each id sums that id's rows of
// d(previous) in token order (fp32) and adds the sum into w1.grad's row (bf16).
__global__ __launch_bounds__(256) void markov_scatter_kernel(const uint32_t* __restrict__ keys,
                                                             const uint32_t* __restrict__ vals, int64_t n, int64_t v,
                                                             int64_t r, const float* __restrict__ dprev,
                                                             uint16_t* __restrict__ w1g, int64_t ldg1) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const uint32_t key = keys[i];
  if (key >= (uint32_t)v || (i > 0 && keys[i - 1] == key)) return;
  const int lane = threadIdx.x & 63;
  for (int64_t c = lane * 4; c < r; c += 256) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t j = i; j < n && keys[j] == key; ++j) {
      const float4 x = *reinterpret_cast<const float4*>(dprev + (int64_t)vals[j] * r + c);
      s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
    }
    uint16_t* g = w1g + (int64_t)key * ldg1 + c;
    const uint2 old = *reinterpret_cast<const uint2*>(g);
    uint2 o;
    o.x = pack_bf16x2(bf16_lo(old.x) + s.x, bf16_hi(old.x) + s.y);
    o.y = pack_bf16x2(bf16_lo(old.y) + s.z, bf16_hi(old.y) + s.w);
    *reinterpret_cast<uint2*>(g) = o;
  }
}

int key_bits(int64_t v) {
  int b = 1;
  while (b < 32 && (int64_t(1) << b) <= v) ++b;
  return b;
}

size_t sort_temp_bytes(int64_t n, int64_t v) {
  size_t bytes = 0;
  const hipError_t e = hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, static_cast<const uint32_t*>(nullptr),
                                                          static_cast<uint32_t*>(nullptr),
                                                          static_cast<const uint32_t*>(nullptr),
                                                          static_cast<uint32_t*>(nullptr), (int)n, 0, key_bits(v));
  // without a device the query cannot run; a generous bound keeps the size defined
  return e == hipSuccess ? bytes : (size_t)16 * n * 4 + (size_t(16) << 20);
}

struct MarkovWs {
  void* dh_ws;
  float* dprev;
  uint16_t* e;
  uint32_t *keys_in, *keys_out, *vals_in, *vals_out;
  void* sort_tmp;
  size_t sort_bytes;
};

size_t markov_ws_layout(int64_t n, int64_t v, int64_t d, int64_t r, void* base, MarkovWs* w) {
  const size_t b_dh = align_up(lmhead_bwd_workspace_bytes(n, v, d, r, true), 256);
  const size_t b_dp = align_up((size_t)n * r * sizeof(float), 256);
  const size_t b_e = align_up((size_t)n * r * 2, 256);
  const size_t b_k = align_up((size_t)n * 4, 256);
  const size_t b_s = align_up(sort_temp_bytes(n, v), 256);
  if (w) {
    char* p = static_cast<char*>(base);
    w->dh_ws = p; p += b_dh;
    w->dprev = reinterpret_cast<float*>(p); p += b_dp;
    w->e = reinterpret_cast<uint16_t*>(p); p += b_e;
    w->keys_in = reinterpret_cast<uint32_t*>(p); p += b_k;
    w->keys_out = reinterpret_cast<uint32_t*>(p); p += b_k;
    w->vals_in = reinterpret_cast<uint32_t*>(p); p += b_k;
    w->vals_out = reinterpret_cast<uint32_t*>(p); p += b_k;
    w->sort_tmp = p;
    w->sort_bytes = b_s;
  }
  return b_dh + b_dp + b_e + 4 * b_k + b_s;
}

}  // namespace

size_t markov_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t r) {
  return markov_ws_layout(n, v, d, r, nullptr, nullptr);
}

hipError_t markov_backward(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const MarkovFactors& f,
                           void* dh, int64_t lddh, const NormBwd* norm, void* w1_grad, int64_t ldg1, void* w2_grad,
                           int64_t ldg2, int64_t n, int64_t v, int64_t d, void* ws, size_t ws_bytes, hipStream_t st) {
  const int64_t r = f.r;
  MarkovWs w;
  markov_ws_layout(n, v, d, r, ws, &w);
  hipError_t e;
  // dh (or the rms-norm backward) and d(previous) in one GEMM
  if ((e = lmhead_backward_ext(dl, ldd, weight, ldw, f.w2, f.ldw2, r, dh, lddh, w.dprev, norm, n, v, d, w.dh_ws,
                               st)) != hipSuccess)
    return e;
  if (n == 0) return hipSuccess;
  {
    NS_TIMED("markov_gather", st);
    const int64_t items = n * r / 8;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, st, f.prev,
                       static_cast<const uint16_t*>(f.w1), f.ldw1, n, v, r, w.e);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    Dw2Params p;
    p.dl = static_cast<const uint16_t*>(dl); p.ldd = ldd;
    p.e = w.e;
    p.w2g = static_cast<uint16_t*>(w2_grad); p.ldg2 = ldg2;
    p.n = n; p.v = v; p.r = r;
    p.ct = (int)((r + TN - 1) / TN);
    static std::atomic<uint64_t> attr_done{0};
    if ((e = ensure_dynamic_lds(reinterpret_cast<const void*>(&dw2_kernel), kLds, attr_done)) != hipSuccess) return e;
    NS_TIMED("markov_dw2", st);
    const int grid = (int)((v + TM - 1) / TM) * p.ct;
    hipLaunchKernelGGL(dw2_kernel, dim3(grid), dim3(kThreads), kLds, st, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    NS_TIMED("markov_sort", st);
    hipLaunchKernelGGL(markov_keys_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, f.prev, n, v,
                       w.keys_in, w.vals_in);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    size_t tmp = w.sort_bytes;
    if ((e = hipcub::DeviceRadixSort::SortPairs(w.sort_tmp, tmp, w.keys_in, w.keys_out, w.vals_in, w.vals_out, (int)n,
                                                0, key_bits(v), st)) != hipSuccess)
      return e;
  }
  NS_TIMED("markov_scatter", st);
  hipLaunchKernelGGL(markov_scatter_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, w.keys_out, w.vals_out, n,
                     v, r, w.dprev, static_cast<uint16_t*>(w1_grad), ldg1);
  (void)ws_bytes;
  return hipGetLastError();
}

}  // namespace ns
