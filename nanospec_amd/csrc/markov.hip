// Markov-head backward (nanospec/train.py:303-307):
//   d(previous) = dl . w2                    ops.linear_backward (ops.py:38-45), dx
//   w2.grad     = dl^T . w1[prev]            ops.linear_backward, dw (copied, not accumulated)
//   w1.grad    += index_add(prev, d(prev))   ops.embedding_backward (ops.py:73-74)
// d(previous) comes out of the dh GEMM as extra column tiles (lmhead_backward_ext);
// w2.grad is a K = N GEMM with both operands K-major; the index_add sorts (prev, t) pairs
// (a bitonic chunk sort and merge passes, below) and sums each id's rows in a fixed order,
// so the result does not depend on scheduling (the reference's GPU index_add_ does).
#include <utility>

#include "ns_gemm.h"
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

constexpr int TM = 256;          // w2.grad rows (vocab) per workgroup tile
constexpr int TN = 256;          // w2.grad columns (rank) per workgroup tile
constexpr int TK = 32;           // tokens per LDS stage
constexpr int kThreads = 256;    // 4 waves as 2 (vocab) x 2 (rank), 128 x 128 each
constexpr int kStage = TK * TN * 2;   // 16 KB per operand per stage (32 K rows x 512 B)
constexpr int kRing = 4;              // stages in LDS: fills run three stages ahead
constexpr int kUnroll = 8;            // stages per loop iteration (a multiple of kRing)
constexpr int kFills = DmaTileKNR<TK>::NI;   // fills per wave per operand per stage

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

// All TK / 16 steps of one stage, fragments double-buffered across steps; mem(kk) issues
// step kk's share of a later stage's fills.
template <typename Mem>
__device__ __forceinline__ void stage_kn(f32x16_t (&acc)[4][4], const lds_t* sa, const lds_t* sb,
                                         const uint32_t (&ta)[4], const uint32_t (&tbv)[4], Mem&& mem) {
  KnFrags f[2];
  read_kn_frags(f[0], sa, sb, 0, ta, tbv);
#pragma unroll
  for (int kk = 0; kk < TK / 16; ++kk) {
    if (kk + 1 < TK / 16) read_kn_frags(f[(kk + 1) & 1], sa, sb, kk + 1, ta, tbv);
    __builtin_amdgcn_sched_barrier(0);
    mem(kk);
    __builtin_amdgcn_sched_barrier(0);
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
  // one LDS array per ring buffer: the compiler tells fills of one buffer from reads of
  // another only across distinct objects (with offsets into one array it waited for every
  // outstanding fill before each stage's fragment reads)
  __shared__ __attribute__((aligned(16))) char ring0[2 * kStage];
  __shared__ __attribute__((aligned(16))) char ring1[2 * kStage];
  __shared__ __attribute__((aligned(16))) char ring2[2 * kStage];
  __shared__ __attribute__((aligned(16))) char ring3[2 * kStage];
  static_assert(kRing == 4, "one array per ring buffer");
  auto ring = [&](int b) -> lds_t* {
    return b == 0 ? (lds_t*)ring0 : b == 1 ? (lds_t*)ring1 : b == 2 ? (lds_t*)ring2 : (lds_t*)ring3;
  };
  const int vt = blockIdx.x / p.ct, ctile = blockIdx.x % p.ct;
  const int64_t v0 = (int64_t)vt * TM, c0 = (int64_t)ctile * TN;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv >> 1, wn = wv & 1;
  DmaTileKNR<TK> ta, tb;
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
  const int KTf = (int)(p.n / TK);
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  // stage t lives in buffer t % kRing.  The loop below is unrolled by kUnroll so that every
  // buffer is a compile-time choice; only the first stage of an iteration still waits for all
  // outstanding fills (the compiler's count does not survive the loop's back edge).
  auto fill = [&](int t, int b, int i) {
    lds_t* dst = ring(b);
    ta.issue(pa + t * sa_bytes, dst, wv, i);
    tb.issue(pb + t * sb_bytes, dst + kStage, wv, i);
  };
  // stages 0 .. kRing - 2 go out first; stage t + kRing - 1 goes out during stage t, into
  // the buffer of stage t - 1, which every wave has finished reading at stage t's barrier
#pragma unroll
  for (int t = 0; t < kRing - 1; ++t)
    if (t < KTf)
#pragma unroll
      for (int i = 0; i < kFills; ++i) fill(t, t, i);
  for (int t0 = 0; t0 < KTf; t0 += kUnroll) {
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int t = t0 + j;
      if (t < KTf) {
        // stage t landed: this wave's later fills (stages t + 1, t + 2, 2 kFills each) may still fly
        if (t + 2 < KTf)
          vm_barrier<4 * kFills>();
        else if (t + 1 < KTf)
          vm_barrier<2 * kFills>();
        else
          vm_barrier<0>();
        const int tn = t + kRing - 1;
        const lds_t* cur = ring(j % kRing);
        stage_kn(acc, cur, cur + kStage, tra, trb, [&](int kk) {
          if (tn < KTf) {
#pragma unroll
            for (int i = kk * kFills / (TK / 16); i < (kk + 1) * kFills / (TK / 16); ++i)
              fill(tn, (j + kRing - 1) % kRing, i);
          }
        });
      }
    }
  }
  const int kvalid = (int)(p.n - (int64_t)KTf * TK);
  if (kvalid > 0) {
    fill_barrier();
    const int64_t k0 = (int64_t)KTf * TK;
    load_kn_tail(ring(0), p.dl + k0 * p.ldd, p.ldd, v0, p.v, kvalid);
    load_kn_tail(ring(0) + kStage, p.e + k0 * p.r, p.r, c0, p.r, kvalid);
    __syncthreads();
    stage_kn(acc, ring(0), ring(0) + kStage, tra, trb, [](int) {});
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

// ---- w1.grad.index_add_(prev, d(previous)), deterministic -------------------------------
// Each token's d(previous) row goes to w1.grad row prev[t].  The pairs are sorted by the
// composite key (row << 32) | t: the keys are unique, so any correct sort is the stable
// sort by row, and a row's tokens come out in token order.  Ids outside [0, V) get row V
// (sorted after every real row, skipped); padding up to a whole sort chunk gets row
// 0xFFFFFFFF (after those).  The sum of each row's d(previous) rows is then formed in two
// levels so that one frequent id does not serialise the step: fixed segments of kSeg
// sorted positions sum the pieces of the runs they hold (token order), and one wave per
// run adds the run's pieces in segment order and adds the result to w1.grad with one
// rounding.  Every order is fixed, so the result does not depend on scheduling.
constexpr int kSortChunk = 4096;   // keys per workgroup sorted in LDS (32 KB)
constexpr int kSortThreads = 1024;
constexpr int kSeg = 64;           // sorted positions per piece segment (one wave)

int64_t sort_padded(int64_t n) { return (n + kSortChunk - 1) / kSortChunk * kSortChunk; }

// Build the keys of one chunk and bitonic-sort it in LDS (ascending).
__global__ __launch_bounds__(kSortThreads) void markov_sort_chunks_kernel(const int64_t* __restrict__ prev, int64_t n,
                                                                         int64_t v, uint64_t* __restrict__ out) {
  __shared__ uint64_t sk[kSortChunk];
  const int64_t base = (int64_t)blockIdx.x * kSortChunk;
  for (int i = threadIdx.x; i < kSortChunk; i += kSortThreads) {
    const int64_t t = base + i;
    uint64_t k;
    if (t < n) {
      const int64_t id = prev[t];
      const uint64_t row = (id >= 0 && id < v) ? (uint64_t)id : (uint64_t)v;
      k = (row << 32) | (uint64_t)t;
    } else {
      k = (0xFFFFFFFFull << 32) | (uint64_t)t;
    }
    sk[i] = k;
  }
  __syncthreads();
  for (int size = 2; size <= kSortChunk; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int q = threadIdx.x; q < kSortChunk / 2; q += kSortThreads) {
        // pair q: element i with bit `stride` clear and its partner i + stride
        const int i = (q / stride) * 2 * stride + (q % stride);
        const int j = i + stride;
        const bool up = (i & size) == 0;
        const uint64_t a = sk[i], b = sk[j];
        if ((a > b) == up) {
          sk[i] = b;
          sk[j] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < kSortChunk; i += kSortThreads) out[base + i] = sk[i];
}

// Merge sorted runs of length len pairwise (runs 2m and 2m + 1) from src into dst, n_pad
// keys: a key's place is its position in its run plus the number of the other run's keys
// below it (a binary search; the keys are unique).  A run without a partner stays put.
__global__ __launch_bounds__(256) void markov_merge_kernel(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst,
                                                           int64_t n_pad, int64_t len) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_pad) return;
  const uint64_t x = src[i];
  const int64_t run = i / len, pos = i - run * len;
  const int64_t other = (run ^ 1) * len;
  int64_t olen = n_pad - other;
  olen = olen < 0 ? 0 : (olen > len ? len : olen);
  int64_t lo = 0, hi = olen;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (src[other + mid] < x) lo = mid + 1;
    else hi = mid;
  }
  dst[(run & ~int64_t(1)) * len + pos + lo] = x;
}

// One wave per segment of kSeg sorted positions: the fp32 sum, in sorted (token) order, of
// each run piece the segment holds, stored at the piece's first position.
__global__ __launch_bounds__(256) void markov_pieces_kernel(const uint64_t* __restrict__ keys, int64_t n, int64_t v,
                                                            int64_t r, const float* __restrict__ dprev,
                                                            float* __restrict__ piece) {
  const int64_t s0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kSeg;
  if (s0 >= n) return;
  const int lane = threadIdx.x & 63;
  const int cnt = n - s0 < kSeg ? (int)(n - s0) : kSeg;
  const uint64_t km = lane < cnt ? keys[s0 + lane] : ~0ull;
  const int row_m = (int)(uint32_t)(km >> 32), tok_m = (int)(uint32_t)km;
  // the column loop is uniform over the wave (its shuffles need every lane); lanes past r
  // only skip their loads and stores
  for (int64_t cb = 0; cb < r; cb += 256) {
    const int64_t c = cb + lane * 4;
    const bool act = c < r;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int start = 0;
    for (int j = 0; j < cnt; ++j) {
      const int row = __shfl(row_m, j), tok = __shfl(tok_m, j);
      const int next = __shfl(row_m, j + 1 < cnt ? j + 1 : j);
      if (act) {
        const float4 x = *reinterpret_cast<const float4*>(dprev + (int64_t)tok * r + c);
        acc.x += x.x; acc.y += x.y; acc.z += x.z; acc.w += x.w;
      }
      if (j + 1 == cnt || next != row) {
        if (act && (uint32_t)row < (uint64_t)v) *reinterpret_cast<float4*>(piece + (s0 + start) * r + c) = acc;
        acc = make_float4(0.f, 0.f, 0.f, 0.f);
        start = j + 1;
      }
    }
  }
}

// One wave per sorted position; the first position of each row adds the row's pieces
// (its own, then one per following segment it spans, in order) into w1.grad's row with one
// rounding to bf16.
__global__ __launch_bounds__(256) void markov_runs_kernel(const uint64_t* __restrict__ keys, int64_t n, int64_t v,
                                                          int64_t r, const float* __restrict__ piece,
                                                          uint16_t* __restrict__ w1g, int64_t ldg1) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const uint64_t row = keys[i] >> 32;
  if (row >= (uint64_t)v || (i > 0 && (keys[i - 1] >> 32) == row)) return;
  const int lane = threadIdx.x & 63;
  for (int64_t c = lane * 4; c < r; c += 256) {
    float4 s = *reinterpret_cast<const float4*>(piece + i * r + c);
    for (int64_t q = (i / kSeg + 1) * kSeg; q < n && (keys[q] >> 32) == row; q += kSeg) {
      const float4 x = *reinterpret_cast<const float4*>(piece + q * r + c);
      s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
    }
    uint16_t* g = w1g + (int64_t)row * ldg1 + c;
    const uint2 old = *reinterpret_cast<const uint2*>(g);
    uint2 o;
    o.x = pack_bf16x2(bf16_lo(old.x) + s.x, bf16_hi(old.x) + s.y);
    o.y = pack_bf16x2(bf16_lo(old.y) + s.z, bf16_hi(old.y) + s.w);
    *reinterpret_cast<uint2*>(g) = o;
  }
}

struct MarkovWs {
  void* dh_ws;
  float* dprev;
  uint16_t* e;
  uint64_t *keys_a, *keys_b;   // sort ping-pong, sort_padded(n) each
  float* piece;                // [n, r] run-piece sums
};

size_t markov_ws_layout(int64_t n, int64_t v, int64_t d, int64_t r, void* base, MarkovWs* w) {
  const size_t b_dh = align_up(lmhead_bwd_workspace_bytes(n, v, d, r, true), 256);
  const size_t b_dp = align_up((size_t)n * r * sizeof(float), 256);
  const size_t b_e = align_up((size_t)n * r * 2, 256);
  const size_t b_k = align_up((size_t)sort_padded(n) * sizeof(uint64_t), 256);
  if (w) {
    char* p = static_cast<char*>(base);
    w->dh_ws = p; p += b_dh;
    w->dprev = reinterpret_cast<float*>(p); p += b_dp;
    w->e = reinterpret_cast<uint16_t*>(p); p += b_e;
    w->keys_a = reinterpret_cast<uint64_t*>(p); p += b_k;
    w->keys_b = reinterpret_cast<uint64_t*>(p); p += b_k;
    w->piece = reinterpret_cast<float*>(p);
  }
  return b_dh + b_dp + b_e + 2 * b_k + b_dp;
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
    NS_TIMED("markov_dw2", st);
    const int grid = (int)((v + TM - 1) / TM) * p.ct;
    hipLaunchKernelGGL(dw2_kernel, dim3(grid), dim3(kThreads), 0, st, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  {
    NS_TIMED("markov_sort", st);
    const int64_t n_pad = sort_padded(n);
    hipLaunchKernelGGL(markov_sort_chunks_kernel, dim3((unsigned)(n_pad / kSortChunk)), dim3(kSortThreads), 0, st,
                       f.prev, n, v, w.keys_a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    for (int64_t len = kSortChunk; len < n_pad; len *= 2) {
      hipLaunchKernelGGL(markov_merge_kernel, dim3((unsigned)((n_pad + 255) / 256)), dim3(256), 0, st, w.keys_a,
                         w.keys_b, n_pad, len);
      if ((e = hipGetLastError()) != hipSuccess) return e;
      std::swap(w.keys_a, w.keys_b);
    }
  }
  NS_TIMED("markov_scatter", st);
  const int64_t segs = (n + kSeg - 1) / kSeg;
  hipLaunchKernelGGL(markov_pieces_kernel, dim3((unsigned)((segs + 3) / 4)), dim3(256), 0, st, w.keys_a, n, v, r,
                     w.dprev, w.piece);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(markov_runs_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, w.keys_a, n, v, r, w.piece,
                     static_cast<uint16_t*>(w1_grad), ldg1);
  (void)ws_bytes;
  return hipGetLastError();
}

}  // namespace ns
