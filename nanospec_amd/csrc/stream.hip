// Logits-level draft objective: CE + KL(target || draft) + accept rate and dl,
// streamed over given [N, V] draft (z) and teacher (u) logits.
//
// Restates nanospec/objective.py:49-80 (ce_kl_loss / ce_kl_backward) and
// objective.py:39-46 (acceptance_length_counts) without materialising any
// [N, V] probability tensor:
//   pass 1  (stats)   per (row, vocab split): online (max, sum-exp) of z and u and
//                     A = sum exp(u - m_u)(u - z)              -> RowPart partials
//   merge             per row: LSE_z, LSE_u, CE = LSE_z - z_y,
//                     KL = A / s_u - LSE_u + LSE_z              -> row_stats
//   pass 2  (emit)    per (row, vocab split): p, t; sum min(p, t); optionally
//                     dl = (w/acc)[(c_ce + c_kl) p - c_kl t - c_ce e_y]
//   finalize          one workgroup: accept rate per row, block prefix
//                     lengths, the six LossMetrics scalars (fixed order).
// bf16 rows of up to kRowCap entries take another route: stream_group_kernel, two
// workgroups per row, each keeping its half of z and u on chip between the statistics and
// the emit phase (both read once), then finalize.  fp32 logits, unaligned rows and longer rows
// take the split passes.
// Every reduction has a fixed order, so results are bitwise reproducible.
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {

constexpr int kStreamThreads = 256;
// Vocab entries per workgroup.  Pass 1 (read-only) is fastest with long ranges: few
// partials and one block reduction per 32K entries (0.59 ms at C1, against 0.625 ms at
// 16K and 0.65 ms at 8K).  Pass 2 reads two streams and writes
// one; it moves bytes fastest with one or two 16-byte vectors per thread and many short
// workgroups (3072 entries), five of them per CU: kEmitLds of (unused) LDS caps a CU at
// five.  Measured on MI355X at C1 (4096 x 248320 bf16): 0.955-0.964 ms, against 1.00-1.01
// ms for 2048 entries at eight workgroups per CU, 1.05 ms for 3072 at eight and 1.01 ms at
// four; 16K entries moved 5.1 TB/s against 6.3.  The cap is for the pass that writes dl
// only: the accept-only pass (no dl) runs 0.652 ms uncapped against 0.679 ms capped.
constexpr int64_t kStatsElems = 32768;
constexpr int kStatsMaxSplits = 64;
constexpr int64_t kEmitElems = 3072;
constexpr int kEmitMaxSplits = 256;
constexpr int kEmitLds = 28 * 1024;   // 160 KB of LDS per CU: five workgroups

static int splits_for(int64_t v, int64_t elems, int max_splits) {
  int64_t s = (v + elems - 1) / elems;
  if (s < 1) s = 1;
  if (s > max_splits) s = max_splits;
  return (int)s;
}

int stream_splits(int64_t n, int64_t v) {
  (void)n;
  return splits_for(v, kStatsElems, kStatsMaxSplits);
}

static int emit_splits(int64_t v) { return splits_for(v, kEmitElems, kEmitMaxSplits); }

static inline int64_t split_chunk(int64_t v, int splits) {
  const int64_t c = (v + splits - 1) / splits;
  return (c + 7) / 8 * 8;
}

struct StreamWs {
  RowPart* part1;
  float* parta;
  float* zy;
};

static size_t stream_ws_layout(int64_t n, int64_t v, void* base, StreamWs* out) {
  const int S = stream_splits(n, v);
  const size_t b1 = align_up((size_t)n * S * sizeof(RowPart), 256);
  const size_t b2 = align_up((size_t)n * emit_splits(v) * sizeof(float), 256);
  const size_t b3 = align_up((size_t)n * sizeof(float), 256);
  if (out) {
    char* p = static_cast<char*>(base);
    out->part1 = reinterpret_cast<RowPart*>(p);
    out->parta = reinterpret_cast<float*>(p + b1);
    out->zy = reinterpret_cast<float*>(p + b1 + b2);
  }
  return b1 + b2 + b3;
}

// Block-wide merge of pair states; thread 0 returns the result.
__device__ __forceinline__ PairState block_reduce_pair(PairState st) {
  __shared__ PairState sh[kStreamThreads / 64];
  st = wave_reduce(st);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[wave] = st;
  __syncthreads();
  PairState r = sh[0];
#pragma unroll
  for (int w = 1; w < kStreamThreads / 64; ++w) r = pair_merge(r, sh[w]);
  return r;
}

__device__ __forceinline__ float block_sum(float x) {
  __shared__ float sh[kStreamThreads / 64];
  x = wave_sum(x);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[wave] = x;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int w = 1; w < kStreamThreads / 64; ++w) r += sh[w];
  return r;
}

// ---------------------------------------------------------------- pass 1

template <typename TZ, typename TU, bool VEC>
__global__ __launch_bounds__(kStreamThreads) void stream_stats_kernel(
    const TZ* __restrict__ z, int64_t ldz, const TU* __restrict__ u, int64_t ldu, int64_t v,
    int64_t chunk, int splits, const int64_t* __restrict__ labels, RowPart* __restrict__ part1,
    float* __restrict__ zy) {
  const int s = (int)(blockIdx.x % (unsigned)splits);
  const int64_t r = blockIdx.x / (unsigned)splits;
  const int64_t lo = (int64_t)s * chunk;
  const int64_t hi = lo + chunk < v ? lo + chunk : v;
  const TZ* zr = z + r * ldz;
  const TU* ur = u + r * ldu;
  PairState st = pair_init();
  int64_t scalar_from = lo;
  if (VEC && lo < hi) {
    const int64_t nvec = (hi - lo) >> 3;
    const TZ* zb = zr + lo;
    const TU* ub = ur + lo;
    int64_t j = threadIdx.x;
    // z and u are read once here (pass 2 comes after the whole pass): non-temporal loads
    // took this kernel from 0.69 to 0.65 ms at C1 (pass 2's loads measured 2% slower so)
    for (; j + kStreamThreads < nvec; j += 2 * kStreamThreads) {
      float zf[16], uf[16];
      load8_nt(zb + j * 8, zf);
      load8_nt(ub + j * 8, uf);
      load8_nt(zb + (j + kStreamThreads) * 8, zf + 8);
      load8_nt(ub + (j + kStreamThreads) * 8, uf + 8);
      pair_update<16>(st, zf, uf);
    }
    if (j < nvec) {
      float zf[8], uf[8];
      load8(zb + j * 8, zf);
      load8(ub + j * 8, uf);
      pair_update<8>(st, zf, uf);
    }
    scalar_from = lo + nvec * 8;
  }
  for (int64_t i = scalar_from + threadIdx.x; i < hi; i += kStreamThreads) {
    float zf[1] = {load1(zr + i)}, uf[1] = {load1(ur + i)};
    pair_update<1>(st, zf, uf);
  }
  st = block_reduce_pair(st);
  if (threadIdx.x == 0) {
    RowPart p;
    p.mz = st.mz; p.sz = st.sz; p.mu = st.mu; p.su = st.su; p.A = st.A;
    p.pad0 = p.pad1 = p.pad2 = 0.f;
    part1[r * splits + s] = p;
    const int64_t y = labels[r];
    if (y >= lo && y < hi) zy[r] = load1(zr + y);
  }
}

// ---------------------------------------------------------------- merge

__global__ __launch_bounds__(256) void merge_kernel(const RowPart* __restrict__ part1,
                                                    const float* __restrict__ zy,
                                                    const int64_t* __restrict__ labels, int64_t v,
                                                    int splits, int64_t n, float* __restrict__ row_stats,
                                                    TeacherSpec ts) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const RowPart* p = part1 + r * splits;
  PairState st = {p[0].mz, p[0].sz, p[0].mu, p[0].su, p[0].A};
  for (int s = 1; s < splits; ++s) st = pair_merge(st, PairState{p[s].mz, p[s].sz, p[s].mu, p[s].su, p[s].A});
  const float lz = st.mz + logf(st.sz);
  float lu = st.mu + logf(st.su);
  if (ts.lse) {   // the teacher's producer formed its log-normaliser; KL follows pass 2
    const int64_t tr = ts.rows ? ts.rows[r] : r;
    lu = (tr >= 0 && tr < ts.nt) ? ts.lse[tr] : __builtin_nanf("");
  }
  // A label outside [0, V) has no logit: CE becomes NaN (the loss reports it, never masks
  // it), except kIgnoreIndex, whose CE is 0 (lz - lz keeps a poisoned row's NaN).
  const int64_t label = labels[r];
  const float y = (label >= 0 && label < v) ? zy[r] : __builtin_nanf("");
  float* o = row_stats + r * kRowStatWidth;
  o[kLseZ] = lz;
  o[kLseU] = lu;
  o[kCE] = label == kIgnoreIndex ? lz - lz : lz - y;
  o[kKL] = ts.lse ? 0.f : st.A / st.su - lu + lz;
  o[kZy] = y;
  o[6] = 0.f;   // reserved columns of the row_stats layout
  o[7] = 0.f;
}

hipError_t launch_merge(const RowPart* part1, const float* zy, int64_t v, int splits, const SlotArgs& a,
                        float* row_stats, hipStream_t st, const TeacherSpec* ts) {
  const int64_t blocks = (a.n + 255) / 256;
  const TeacherSpec none{nullptr, 0, nullptr};
  NS_TIMED("merge_rows", st);
  if (blocks > 0)
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)blocks), dim3(256), 0, st, part1, zy, a.labels, v,
                       splits, a.n, row_stats, ts ? *ts : none);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void lse_merge_kernel(const RowPart* __restrict__ part1, int splits, int64_t n,
                                                        float* __restrict__ lse) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const RowPart* p = part1 + r * splits;
  LseState st = {p[0].mz, p[0].sz};
  for (int s = 1; s < splits; ++s) st = lse_merge(st, LseState{p[s].mz, p[s].sz});
  lse[r] = st.m + logf(st.s);
}

hipError_t launch_lse_merge(const RowPart* part1, int splits, int64_t n, float* lse, hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  NS_TIMED("lse_merge", st);
  if (blocks > 0)
    hipLaunchKernelGGL(lse_merge_kernel, dim3((unsigned)blocks), dim3(256), 0, st, part1, splits, n, lse);
  return hipGetLastError();
}

// ---------------------------------------------------------------- pass 2

template <typename TZ, typename TU, typename TD, bool VEC, bool EMIT, bool ACCEPT>
__global__ __launch_bounds__(kStreamThreads) void stream_emit_kernel(
    const TZ* __restrict__ z, int64_t ldz, const TU* __restrict__ u, int64_t ldu, int64_t v,
    int64_t chunk, int splits, const float* __restrict__ row_stats, const int64_t* __restrict__ labels,
    const float* __restrict__ weights, float c_ce, float c_kl, float inv_acc, TD* __restrict__ dl,
    int64_t ldd, float* __restrict__ parta) {
  const int s = (int)(blockIdx.x % (unsigned)splits);
  const int64_t r = blockIdx.x / (unsigned)splits;
  const int64_t lo = (int64_t)s * chunk;
  const int64_t hi = lo + chunk < v ? lo + chunk : v;
  const TZ* zr = z + r * ldz;
  const TU* ur = u + r * ldu;
  TD* dr = EMIT ? dl + r * ldd : nullptr;
  const float lzl = row_stats[r * kRowStatWidth + kLseZ] * kLog2e;
  const float lul = row_stats[r * kRowStatWidth + kLseU] * kLog2e;
  const float w = weights[r] * inv_acc;
  const int64_t y = labels[r];
  // an ignored row has no CE term: dl = w c_kl (p - t) (its label matches no entry)
  const float cp = y == kIgnoreIndex ? w * c_kl : w * (c_ce + c_kl), ct = w * c_kl, cy = w * c_ce;
  float acc = 0.f;
  int64_t scalar_from = lo;
  if (VEC && lo < hi) {
    const int64_t nvec = (hi - lo) >> 3;
    // U groups of 8 per iteration: all 2U loads are issued before any is used
    auto body = [&](auto uc, int64_t j) {
      constexpr int U = decltype(uc)::value;
      Raw8<TZ> zraw[U];
      Raw8<TU> uraw[U];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        zraw[q].load(zr + lo + (j + q * kStreamThreads) * 8);
        uraw[q].load(ur + lo + (j + q * kStreamThreads) * 8);
      }
      float zf[U][8], uf[U][8];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        zraw[q].unpack(zf[q]);
        uraw[q].unpack(uf[q]);
      }
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int64_t i0 = lo + (j + q * kStreamThreads) * 8;
        float d[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float p = fast_exp2(__builtin_fmaf(zf[q][e], kLog2e, -lzl));
          const float t = fast_exp2(__builtin_fmaf(uf[q][e], kLog2e, -lul));
          if (ACCEPT) acc += min_nonneg(p, t);
          if (EMIT) d[e] = __builtin_fmaf(cp, p, -ct * t);
        }
        if (EMIT) {
          if ((uint64_t)(y - i0) < 8ull) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (i0 + e == y) d[e] -= cy;
          }
          store8_nt(dr + i0, d);   // dl is not read back by this pass: keep z, u in cache
        }
      }
    };
    int64_t j = threadIdx.x;
    for (; j + kStreamThreads < nvec; j += 2 * kStreamThreads) body(std::integral_constant<int, 2>{}, j);
    for (; j < nvec; j += kStreamThreads) body(std::integral_constant<int, 1>{}, j);
    scalar_from = lo + nvec * 8;
  }
  for (int64_t i = scalar_from + threadIdx.x; i < hi; i += kStreamThreads) {
    const float p = fast_exp2(__builtin_fmaf(load1(zr + i), kLog2e, -lzl));
    const float t = fast_exp2(__builtin_fmaf(load1(ur + i), kLog2e, -lul));
    if (ACCEPT) acc += min_nonneg(p, t);
    if (EMIT) {
      float d = __builtin_fmaf(cp, p, -ct * t);
      if (i == y) d -= cy;
      store1(dr + i, d);
    }
  }
  if (ACCEPT) {
    acc = block_sum(acc);
    if (threadIdx.x == 0) parta[r * splits + s] = acc;
  }
}

// ---------------------------------------------------------------- accept rate per row

// One wave per row: lane l sums the row's pass-2 partials l, l + 64, ... in order, then
// a butterfly sum (symmetric, so the result does not depend on the lane) -> row_stats.
__global__ __launch_bounds__(256) void accept_rows_kernel(const float* __restrict__ parta, int splits, int64_t n,
                                                          float* __restrict__ row_stats) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= n) return;
  const int lane = threadIdx.x & 63;
  const float* p = parta + r * splits;
  float a = 0.f;
  for (int s = lane; s < splits; s += 64) a += p[s];
  a = wave_sum(a);
  float* rs = row_stats + r * kRowStatWidth;
  if (lane == 0) rs[kAccept] = accept_rate_of(a, rs[kLseZ], rs[kLseU]);
}

static hipError_t launch_accept_rows(const float* parta, int splits, int64_t n, float* row_stats, hipStream_t st) {
  NS_TIMED("accept_rows", st);
  hipLaunchKernelGGL(accept_rows_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, parta, splits, n,
                     row_stats);
  return hipGetLastError();
}

// ---------------------------------------------------------------- finalize

constexpr int kFinalThreads = 1024;

// Per row, one thread, split partials summed in split order: the accept rate and, with
// partk, KL = sum t (u - z) - lse_u + lse_z (sum t = 1).  Its own grid: in finalize's single
// workgroup this loop took 0.05-0.1 ms at N = 4096.
__global__ __launch_bounds__(256) void row_parts_kernel(const float* __restrict__ parta,
                                                        const float* __restrict__ partk, int splits, int64_t n,
                                                        float* __restrict__ row_stats) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= n) return;
  const float* p = parta + r * splits;
  float a = p[0];
  for (int s = 1; s < splits; ++s) a += p[s];
  float* rs = row_stats + r * kRowStatWidth;
  rs[kAccept] = accept_rate_of(a, rs[kLseZ], rs[kLseU]);
  if (partk != nullptr) {
    const float* q = partk + r * splits;
    float k = q[0];
    for (int s = 1; s < splits; ++s) k += q[s];
    rs[kKL] = k - rs[kLseU] + rs[kLseZ];
  }
}

__global__ __launch_bounds__(kFinalThreads) void finalize_kernel(int64_t n, int64_t k,
                                                                 const float* __restrict__ weights,
                                                                 const uint8_t* __restrict__ valid, float c_ce,
                                                                 float c_kl, const float* __restrict__ row_stats,
                                                                 float* __restrict__ metrics) {
  // weighted sums and block prefix lengths (objective.py:42-46, 53-60)
  double den = 0.0, ce = 0.0, kl = 0.0, asum = 0.0, atot = 0.0;
  const int64_t nblocks = n / k;
  for (int64_t b = threadIdx.x; b < nblocks; b += kFinalThreads) {
    double prod = 1.0, len = 1.0;
    bool any = false;
    for (int64_t j = 0; j < k; ++j) {
      const int64_t r = b * k + j;
      const float* rs = row_stats + r * kRowStatWidth;
      const bool vr = valid[r] != 0;
      // (accept_rate * valid).cumprod(-1): a masked slot's NaN rate still poisons the block
      prod *= (double)rs[kAccept] * (vr ? 1.0 : 0.0);
      len += prod;
      any = any || vr;
      const double w = weights[r];
      den += w;
      ce += w * (double)rs[kCE];
      kl += w * (double)rs[kKL];
    }
    // (lengths * block_valid).sum(): a NaN length counts even in a block with no valid slot
    asum += len * (any ? 1.0 : 0.0);
    if (any) atot += 1.0;
  }
  __shared__ double sh[5][kFinalThreads / 64];
  double vals[5] = {den, ce, kl, asum, atot};
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const double x = wave_sum(vals[i]);
    if ((threadIdx.x & 63) == 0) sh[i][wave] = x;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double t[5];
    for (int i = 0; i < 5; ++i) {
      t[i] = sh[i][0];
      for (int w = 1; w < kFinalThreads / 64; ++w) t[i] += sh[i][w];
    }
    const double dc = t[0] > 1e-6 ? t[0] : 1e-6;
    metrics[kMetCE] = (float)(t[1] / dc);
    metrics[kMetKL] = (float)(t[2] / dc);
    metrics[kMetNum] = (float)((double)c_ce * t[1] + (double)c_kl * t[2]);
    metrics[kMetDen] = (float)t[0];
    metrics[kMetAccSum] = (float)t[3];
    metrics[kMetAccTot] = (float)t[4];
  }
}

hipError_t launch_finalize(const float* parta, int splits, const SlotArgs& a, float* row_stats,
                           float* metrics, hipStream_t st, const float* partk) {
  if (parta != nullptr && a.n > 0) {
    NS_TIMED("row_parts", st);
    hipLaunchKernelGGL(row_parts_kernel, dim3((unsigned)((a.n + 255) / 256)), dim3(256), 0, st, parta, partk,
                       splits, a.n, row_stats);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  if (metrics == nullptr) return hipSuccess;   // the row sums alone (metrics formed later)
  NS_TIMED("finalize_metrics", st);
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(kFinalThreads), 0, st, a.n, a.k, a.weights, a.valid, a.c_ce,
                     a.c_kl, row_stats, metrics);
  return hipGetLastError();
}

// ---------------------------------------------------------------- a group of workgroups per row

// bf16 z and u with V <= kRowCap: G workgroups of T threads share a row.  Member h keeps its
// contiguous share of both z and u on chip between the statistics phase and the emit phase,
// so each is read once: 6 V bytes per row with dl (4 V without), against 10 V (8 V) for
// stream_stats + stream_emit.  Between the phases the members swap their partial statistics
// (PairState and the label's logit) through the workspace and merge them in member order;
// the last member of a row to finish sums the accept partials in member order and writes the
// row's statistics.
//
// Workgroups take tickets from a counter: ticket t is member t % G of row t / G.  A member
// waits only for members holding tickets, which have started and so finish phase 1 without
// waiting, whatever order the workgroups are dispatched in.  An exchanged value is one
// 64-bit word, tag << 32 | bits, written and read with relaxed device-scope atomics (coherent
// across the XCDs' L2s): a word is complete once its tag is non-zero, so no fence orders it
// against other words.  group_clear_kernel zeroes the counter and the words before each
// launch.  Every wait is bounded (kGrpSpinLimit polls, seconds): one that runs out, which the
// argument above rules out, yields NaN statistics instead of a hang.
//
// Storage of member h's share (16-byte vectors b .. b + cnt of the row, b = h ceil(nvec / G)):
// thread t owns vectors b + i T + t.  Columns i < kGrpRegCols of z and u sit in registers,
// filled by ordinary loads; columns kGrpRegCols + c, c < kGrpLdsCols, in LDS (z at slot
// (c, t), u at slot (kGrpLdsCols + c, t), slot (k, t) at byte 16 (k T + t)), filled straight
// from memory (buffer_load ... lds).  All of a share's loads are issued, unconditionally,
// before any is used (vectors past the share read zeros through the buffer range and are
// never folded): the register columns first, which phase 1 then consumes in issue order while
// the rest land.  Loads under per-column conditions made the compiler wait for every load
// before the first fold.
constexpr int kGrpRegCols = 22;
constexpr int kGrpLdsCols = 9;
constexpr int kGrpCols = kGrpRegCols + kGrpLdsCols;
constexpr int kGrpMax = 4;               // largest group size the workspace is laid out for
constexpr uint32_t kGrpSpinLimit = 1u << 20;
constexpr int kGrpAux = 2;   // cache policy of the share's loads and dl's stores: each byte is used once
template <int T>
constexpr int grp_lds_bytes() { return 2 * kGrpLdsCols * T * 16; }
template <int T>
constexpr int64_t grp_share_cap() { return (int64_t)kGrpCols * T; }   // vectors per member

// Launch shape: 4 workgroups of 256 threads per row, two workgroups (72 KB of LDS each) per
// CU, so that one's loads overlap the other's arithmetic.  Measured at C1 (4096 x 248320), with
// an earlier register/LDS column split: 1.09 ms, against 1.33 ms for 2 x 512 threads (one
// workgroup per CU: loads, exchange and arithmetic in series) and the same 1.09 ms for 8 x 128
// threads; the kernel now runs 1.06 ms.
constexpr int kGrpThreads = 256;
constexpr int kGrp = 4;
constexpr int64_t kRowCap = kGrp * grp_share_cap<kGrpThreads>() * 8;   // 253,952 entries
static_assert(2 * (grp_lds_bytes<kGrpThreads>() + 512) <= 160 * 1024, "two group workgroups per CU");
static_assert(kGrp <= kGrpMax, "workspace layout");

// Test settings of the exchange (environment NS_DEBUG_GROUP_DROP_MEMBER, _SPIN_LIMIT): a
// member that publishes nothing, and the poll limit.  Unset: -1 and kGrpSpinLimit.
struct GrpDebug {
  int drop_member;
  uint32_t spin_limit;
};

static GrpDebug group_debug() {
  GrpDebug d{-1, kGrpSpinLimit};
  if (const char* e = getenv("NS_DEBUG_GROUP_DROP_MEMBER"); e && *e) d.drop_member = atoi(e);
  if (const char* e = getenv("NS_DEBUG_GROUP_SPIN_LIMIT"); e && *e) {
    const long x = atol(e);
    d.spin_limit = x < 1 ? 1u : x > (long)kGrpSpinLimit ? kGrpSpinLimit : (uint32_t)x;
  }
  return d;
}

struct alignas(64) GrpWords {
  uint64_t w[8];   // 0-4 PairState, 5 label logit (tag 2 when this member holds the label), 6 accept partial
};

typedef uint32_t u32x4n_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_c;
typedef __attribute__((address_space(3))) const u32x4n_t lds_vec;

__device__ __forceinline__ void unpack8(const u32x4n_t& w, float* f) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = bf16_lo(w[e]);
    f[2 * e + 1] = bf16_hi(w[e]);
  }
}

__device__ __forceinline__ void put_word(uint64_t* p, float x, uint32_t tag) {
  const uint64_t w = ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(x);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls until the word's tag is set; NaN (tag 1) once `limit` polls have gone by.
__device__ __forceinline__ uint64_t get_word(const uint64_t* p, uint32_t limit) {
  for (uint32_t k = 0;; ++k) {
    const uint64_t w = __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((w >> 32) != 0) return w;
    if (k >= limit) return (1ull << 32) | 0x7fc00000ull;
    __builtin_amdgcn_s_sleep(2);
  }
}

__device__ __forceinline__ float word_value(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Zeroes the ticket counter, the per-row finish counters and the exchange words.
__global__ __launch_bounds__(256) void group_clear_kernel(uint4* __restrict__ p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

template <int T, int G, bool EMIT>
__global__ __launch_bounds__(T) void stream_group_kernel(
    const uint16_t* __restrict__ z, int64_t ldz, const uint16_t* __restrict__ u, int64_t ldu, int64_t v,
    const int64_t* __restrict__ labels, const float* __restrict__ weights, float c_ce, float c_kl, float inv_acc,
    uint16_t* __restrict__ dl, int64_t ldd, float* __restrict__ row_stats, int64_t n, uint32_t* __restrict__ ctl,
    uint32_t* __restrict__ done, GrpWords* __restrict__ words, GrpDebug dbg) {
  static_assert(G * 6 <= 64 && G <= kGrpMax, "one wave polls every peer word; workspace layout");
  extern __shared__ __attribute__((aligned(16))) char grp_raw[];
  __shared__ PairState red[T / 64];
  __shared__ float red_a[T / 64];
  __shared__ uint32_t ticket_sh;
  __shared__ float peer[G][6];
  __shared__ uint32_t peer_tag[G];
  lds_c* lds = (lds_c*)grp_raw;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid == 0) ticket_sh = __hip_atomic_fetch_add(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const uint32_t ticket = __builtin_amdgcn_readfirstlane(ticket_sh);   // uniform: descriptors stay scalar
  const int64_t r = ticket / G;
  const int h = (int)(ticket % G);
  if (r >= n) return;   // only with a workspace that group_clear_kernel did not zero
  const int nvec = (int)(v >> 3);
  const int share = (nvec + G - 1) / G;
  const int b = h * share;
  const int cnt = nvec - b < share ? (nvec - b > 0 ? nvec - b : 0) : share;
  const int full = cnt / T, rem = cnt % T;   // vectors i < full exist in every thread
  auto has = [&](int i) { return i < full || (i == full && tid < rem); };
  // the share through buffer resources of its own length (accesses past it read 0, store nothing)
  const uint32_t share_bytes = (uint32_t)cnt * 16;
  const __amdgpu_buffer_rsrc_t zrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(z + r * ldz + (int64_t)b * 8), 0, share_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(u + r * ldu + (int64_t)b * 8), 0, share_bytes, 0x00020000);
  const int voff = tid * 16;
  // LDS slots of column i >= kGrpRegCols
  auto zcol = [](int i) { return i - kGrpRegCols; };
  auto ucol = [](int i) { return kGrpLdsCols + i - kGrpRegCols; };
  auto zslot = [&](int i) { return (lds_vec*)(lds + (zcol(i) * T + tid) * 16); };
  auto uslot = [&](int i) { return (lds_vec*)(lds + (ucol(i) * T + tid) * 16); };
  auto zblock = [&](int i) { return lds + (zcol(i) * T + wave * 64) * 16; };   // the wave's 1 KB of a column
  auto ublock = [&](int i) { return lds + (ucol(i) * T + wave * 64) * 16; };
  // phase 1: issue every load of the share, then (max, sum-exp) of z and u and
  // A = sum exp(u - m_u)(u - z) in issue order
  u32x4n_t zr[kGrpRegCols], ur[kGrpRegCols];
  // column offsets in the lane's own offset (the part the buffer range check is certain to
  // cover), the scalar offset 0
  uint32_t vo = voff;
#pragma unroll
  for (int i = 0; i < kGrpRegCols; ++i) {
    zr[i] = __builtin_amdgcn_raw_buffer_load_b128(zrs, vo, 0, kGrpAux);
    ur[i] = __builtin_amdgcn_raw_buffer_load_b128(urs, vo, 0, kGrpAux);
    vo += T * 16;   // formed here, not hoisted into one register per column
    asm volatile("" : "+v"(vo));
  }
#pragma unroll
  for (int i = kGrpRegCols; i < kGrpCols; ++i) {   // lane l of a wave fills the slot of thread 64 wave + l
    __builtin_amdgcn_raw_ptr_buffer_load_lds(zrs, (__attribute__((address_space(3))) void*)zblock(i), 16, vo, 0, 0,
                                             kGrpAux);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(urs, (__attribute__((address_space(3))) void*)ublock(i), 16, vo, 0, 0,
                                             kGrpAux);
    vo += T * 16;
    asm volatile("" : "+v"(vo));
  }
  // The label's entries are read on their own, after the share's loads (at a clamped index,
  // so without a branch that would wait for them): picking them out of the columns, or
  // patching dl[y] inside the emit loop, costs selects on every vector.
  const int64_t y = labels[r];
  const bool mine = y >= 8 * (int64_t)b && y < 8 * (int64_t)(b + cnt);   // this share holds the label
  const int lab_tid = mine ? (int)((y >> 3) - b) % T : -1;
  const int64_t yc = y < 0 ? 0 : (y < v ? y : v - 1);
  const float zy_at = bf16_to_f32(z[r * ldz + yc]), uy_at = bf16_to_f32(u[r * ldu + yc]);
  const float zy = mine ? zy_at : 0.f, uy = mine ? uy_at : 0.f;
  PairState st = pair_init();
  auto fold = [&](int i, const u32x4n_t& zv, const u32x4n_t& uv) {
    float zf[8], uf[8];
    unpack8(zv, zf);
    unpack8(uv, uf);
    pair_update<8>(st, zf, uf);
  };
#pragma unroll
  for (int i = 0; i < kGrpRegCols; ++i)
    if (has(i)) fold(i, zr[i], ur[i]);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this wave's LDS fills have landed
#pragma unroll
  for (int i = kGrpRegCols; i < kGrpCols; ++i)
    if (has(i)) {
      const u32x4n_t zv = *zslot(i), uv = *uslot(i);
      fold(i, zv, uv);
    }
  st = wave_reduce(st);
  if ((tid & 63) == 0) red[wave] = st;
  __syncthreads();

  // exchange: publish this member's partials, collect the others'
  GrpWords* mw = words + r * G;
  if (tid == 0) {
    PairState p = red[0];
#pragma unroll
    for (int w = 1; w < T / 64; ++w) p = pair_merge(p, red[w]);
    const float part[6] = {p.mz, p.sz, p.mu, p.su, p.A, zy};
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      if (h != dbg.drop_member) put_word(&mw[h].w[k], part[k], k == 5 && mine ? 2u : 1u);
      peer[h][k] = part[k];
    }
    peer_tag[h] = mine ? 2u : 1u;
  }
  if (wave == 0) {
    const int lane = tid & 63;
    const int m = lane / 6, k = lane % 6;
    if (m < G && m != h) {
      const uint64_t wd = get_word(&mw[m].w[k], dbg.spin_limit);
      peer[m][k] = word_value(wd);
      if (k == 5) peer_tag[m] = (uint32_t)(wd >> 32);
    }
  }
  __syncthreads();
  st = {peer[0][0], peer[0][1], peer[0][2], peer[0][3], peer[0][4]};
#pragma unroll
  for (int m = 1; m < G; ++m) st = pair_merge(st, PairState{peer[m][0], peer[m][1], peer[m][2], peer[m][3], peer[m][4]});
  float zy_row = 0.f;
#pragma unroll
  for (int m = 0; m < G; ++m)
    if (peer_tag[m] == 2u) zy_row = peer[m][5];
  const float lz = st.mz + logf(st.sz);
  const float lu = st.mu + logf(st.su);

  // phase 2: p, t, sum min(p, t) and dl, from chip.  The register columns pass through an
  // empty asm so that phase 1's unpacked (fp32) copies are not kept for reuse here: the
  // packed form is half the registers.
#pragma unroll
  for (int i = 0; i < kGrpRegCols; ++i) asm volatile("" : "+v"(zr[i]), "+v"(ur[i]));
  const float lzl = lz * kLog2e, lul = lu * kLog2e;
  const float w = weights[r] * inv_acc;
  const float cp = y == kIgnoreIndex ? w * c_kl : w * (c_ce + c_kl), ct = w * c_kl, cy = w * c_ce;
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc(
      EMIT ? dl + r * ldd + (int64_t)b * 8 : nullptr, 0, EMIT ? share_bytes : 0, 0x00020000);
  float acc = 0.f;
  int sout = 0;
  auto emit = [&](int i, const u32x4n_t& zv, const u32x4n_t& uv) {
    float zf[8], uf[8], d[8];
    unpack8(zv, zf);
    unpack8(uv, uf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pp = fast_exp2(__builtin_fmaf(zf[e], kLog2e, -lzl));
      const float tt = fast_exp2(__builtin_fmaf(uf[e], kLog2e, -lul));
      acc += min_nonneg(pp, tt);
      d[e] = __builtin_fmaf(cp, pp, -ct * tt);
    }
    if (EMIT) {
      const u32x4n_t o = {pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3]), pack_bf16x2(d[4], d[5]),
                          pack_bf16x2(d[6], d[7])};
      __builtin_amdgcn_raw_buffer_store_b128(o, drs, voff, sout, kGrpAux);
    }
  };
#pragma unroll
  for (int i = 0; i < kGrpCols; ++i) {
    if (has(i)) {
      if (i < kGrpRegCols)
        emit(i, zr[i < kGrpRegCols ? i : 0], ur[i < kGrpRegCols ? i : 0]);
      else
      {
        const u32x4n_t zv = *zslot(i), uv = *uslot(i);
        emit(i, zv, uv);
      }
    }
    sout += T * 16;
    asm volatile("" : "+s"(sout));
  }
  if (EMIT && tid == lab_tid) {   // dl[y] again, with - c_ce w, once the vector holding it is stored
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    const float pp = fast_exp2(__builtin_fmaf(zy, kLog2e, -lzl));
    const float tt = fast_exp2(__builtin_fmaf(uy, kLog2e, -lul));
    float d = __builtin_fmaf(cp, pp, -ct * tt);
    d -= cy;
    dl[r * ldd + y] = (uint16_t)(pack_bf16x2(d, 0.f) & 0xffffu);
  }
  acc = wave_sum(acc);
  if ((tid & 63) == 0) red_a[wave] = acc;
  __syncthreads();
  if (tid == 0) {
    float a = red_a[0];
#pragma unroll
    for (int w2 = 1; w2 < T / 64; ++w2) a += red_a[w2];
    if (h != dbg.drop_member) put_word(&mw[h].w[6], a, 1u);
    const uint32_t fin = __hip_atomic_fetch_add(done + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (fin == G - 1) {   // the row's last member: accept sum in member order, then the row's statistics
      float at = 0.f;
#pragma unroll
      for (int m = 0; m < G; ++m) at += m == h ? a : word_value(get_word(&mw[m].w[6], dbg.spin_limit));
      // CE and KL as merge_kernel forms them (labels outside [0, V) other than the ignore
      // index make CE NaN)
      const float yv = (y >= 0 && y < v) ? zy_row : __builtin_nanf("");
      float* o = row_stats + r * kRowStatWidth;
      o[kLseZ] = lz;
      o[kLseU] = lu;
      o[kCE] = y == kIgnoreIndex ? lz - lz : lz - yv;
      o[kKL] = st.A / st.su - lu + lz;
      o[kAccept] = accept_rate_of(at, lz, lu);
      o[kZy] = yv;
      o[6] = 0.f;
      o[7] = 0.f;
    }
  }
}

// Workspace of the group kernel: ticket counter, per-row finish counters, exchange words.
struct GroupWs {
  uint32_t* ctl;
  uint32_t* done;
  GrpWords* words;
  size_t bytes;
};

static size_t group_ws_layout(int64_t n, void* base, GroupWs* out) {
  const size_t b1 = 256;
  const size_t b2 = align_up((size_t)n * sizeof(uint32_t), 256);
  const size_t b3 = align_up((size_t)n * kGrpMax * sizeof(GrpWords), 256);
  if (out) {
    char* p = static_cast<char*>(base);
    out->ctl = reinterpret_cast<uint32_t*>(p);
    out->done = reinterpret_cast<uint32_t*>(p + b1);
    out->words = reinterpret_cast<GrpWords*>(p + b1 + b2);
    out->bytes = b1 + b2 + (size_t)n * kGrp * sizeof(GrpWords);
  }
  return b1 + b2 + b3;
}

template <bool EMIT>
static hipError_t launch_group(const void* z, int64_t ldz, const void* u, int64_t ldu, int64_t v, const SlotArgs& a,
                               void* dl, int64_t ldd, float* row_stats, const GroupWs& g, hipStream_t st) {
  static std::atomic<uint64_t> attr_done{0};
  constexpr int kLds = grp_lds_bytes<kGrpThreads>();
  if (const hipError_t e = ensure_dynamic_lds(
          reinterpret_cast<const void*>(&stream_group_kernel<kGrpThreads, kGrp, EMIT>), kLds, attr_done))
    return e;
  const int64_t n16 = (int64_t)(g.bytes / 16);
  {
    NS_TIMED("group_clear", st);
    hipLaunchKernelGGL(group_clear_kernel, dim3((unsigned)((n16 + 255) / 256 < 1024 ? (n16 + 255) / 256 : 1024)), dim3(256), 0,
                       st, reinterpret_cast<uint4*>(g.ctl), n16);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  NS_TIMED(EMIT ? "stream_group" : "stream_group_accept", st);
  hipLaunchKernelGGL((stream_group_kernel<kGrpThreads, kGrp, EMIT>), dim3((unsigned)(a.n * kGrp)), dim3(kGrpThreads), kLds, st, static_cast<const uint16_t*>(z),
                     ldz, static_cast<const uint16_t*>(u), ldu, v, a.labels, a.weights, a.c_ce, a.c_kl, a.inv_acc,
                     static_cast<uint16_t*>(dl), ldd, row_stats, a.n, g.ctl, g.done, g.words, group_debug());
  return hipGetLastError();
}

// The split passes and the group kernel use the workspace in turn, never together.
size_t stream_workspace_bytes(int64_t n, int64_t v) {
  const size_t a = stream_ws_layout(n, v, nullptr, nullptr), b = group_ws_layout(n, nullptr, nullptr);
  return a > b ? a : b;
}

// ---------------------------------------------------------------- host dispatch

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename TZ, typename TU>
static hipError_t stats_dispatch(const void* z, int64_t ldz, const void* u, int64_t ldu, int64_t v,
                                 const SlotArgs& a, const StreamWs& w, int S, hipStream_t st) {
  const TZ* zp = static_cast<const TZ*>(z);
  const TU* up = static_cast<const TU*>(u);
  const bool vec = aligned16(z) && aligned16(u) && (ldz * (int64_t)sizeof(TZ)) % 16 == 0 &&
                   (ldu * (int64_t)sizeof(TU)) % 16 == 0;
  const int64_t chunk = split_chunk(v, S);
  dim3 grid((unsigned)(S * a.n));
  NS_TIMED("stream_stats", st);
  if (vec)
    hipLaunchKernelGGL((stream_stats_kernel<TZ, TU, true>), grid, dim3(kStreamThreads), 0, st, zp, ldz, up,
                       ldu, v, chunk, S, a.labels, w.part1, w.zy);
  else
    hipLaunchKernelGGL((stream_stats_kernel<TZ, TU, false>), grid, dim3(kStreamThreads), 0, st, zp, ldz,
                       up, ldu, v, chunk, S, a.labels, w.part1, w.zy);
  return hipGetLastError();
}

template <typename TZ, typename TU, bool EMIT, bool ACCEPT>
static hipError_t emit_dispatch(const void* z, int64_t ldz, const void* u, int64_t ldu, int64_t v,
                                const SlotArgs& a, const float* row_stats, void* dl, int64_t ldd,
                                float* parta, int S, hipStream_t st) {
  const TZ* zp = static_cast<const TZ*>(z);
  const TU* up = static_cast<const TU*>(u);
  TZ* dp = static_cast<TZ*>(dl);  // dl has the logits dtype (objective.py:80)
  bool vec = aligned16(z) && aligned16(u) && (ldz * (int64_t)sizeof(TZ)) % 16 == 0 &&
             (ldu * (int64_t)sizeof(TU)) % 16 == 0;
  if (EMIT) vec = vec && aligned16(dl) && (ldd * (int64_t)sizeof(TZ)) % 16 == 0;
  const int64_t chunk = split_chunk(v, S);
  dim3 grid((unsigned)(S * a.n));
  NS_TIMED(EMIT ? "stream_emit" : "stream_accept", st);
  if (vec)
    hipLaunchKernelGGL((stream_emit_kernel<TZ, TU, TZ, true, EMIT, ACCEPT>), grid, dim3(kStreamThreads), EMIT ? kEmitLds : 0,
                       st, zp, ldz, up, ldu, v, chunk, S, row_stats, a.labels, a.weights, a.c_ce, a.c_kl,
                       a.inv_acc, dp, ldd, parta);
  else
    hipLaunchKernelGGL((stream_emit_kernel<TZ, TU, TZ, false, EMIT, ACCEPT>), grid, dim3(kStreamThreads), EMIT ? kEmitLds : 0,
                       st, zp, ldz, up, ldu, v, chunk, S, row_stats, a.labels, a.weights, a.c_ce, a.c_kl,
                       a.inv_acc, dp, ldd, parta);
  return hipGetLastError();
}

template <typename TZ, typename TU>
static hipError_t forward_typed(const void* z, int64_t ldz, const void* u, int64_t ldu, int64_t v,
                                const SlotArgs& a, void* dl, int64_t ldd, float* row_stats, float* metrics,
                                void* ws, hipStream_t st) {
  // bf16 rows that fit on chip, 16-byte aligned: a group of workgroups per row
  if (std::is_same<TZ, uint16_t>::value && std::is_same<TU, uint16_t>::value && v % 8 == 0 && v <= kRowCap &&
      aligned16(z) && aligned16(u) && ldz % 8 == 0 && ldu % 8 == 0 &&
      (dl == nullptr || (aligned16(dl) && ldd % 8 == 0))) {
    GroupWs g;
    group_ws_layout(a.n, ws, &g);
    hipError_t e = dl != nullptr ? launch_group<true>(z, ldz, u, ldu, v, a, dl, ldd, row_stats, g, st)
                                 : launch_group<false>(z, ldz, u, ldu, v, a, nullptr, 0, row_stats, g, st);
    if (e != hipSuccess) return e;
    return launch_finalize(nullptr, 1, a, row_stats, metrics, st);   // accept rates already in row_stats
  }
  StreamWs w;
  stream_ws_layout(a.n, v, ws, &w);
  const int S = stream_splits(a.n, v);
  hipError_t e = stats_dispatch<TZ, TU>(z, ldz, u, ldu, v, a, w, S, st);
  if (e != hipSuccess) return e;
  if ((e = launch_merge(w.part1, w.zy, v, S, a, row_stats, st)) != hipSuccess) return e;
  const int S2 = emit_splits(v);
  if (dl != nullptr)
    e = emit_dispatch<TZ, TU, true, true>(z, ldz, u, ldu, v, a, row_stats, dl, ldd, w.parta, S2, st);
  else
    e = emit_dispatch<TZ, TU, false, true>(z, ldz, u, ldu, v, a, row_stats, nullptr, 0, w.parta, S2, st);
  if (e != hipSuccess) return e;
  if ((e = launch_accept_rows(w.parta, S2, a.n, row_stats, st)) != hipSuccess) return e;
  return launch_finalize(nullptr, 1, a, row_stats, metrics, st);   // accept rates already in row_stats
}

hipError_t stream_forward(const void* z, int zdt, int64_t ldz, const void* u, int udt, int64_t ldu,
                          int64_t v, const SlotArgs& a, void* dl, int64_t ldd, float* row_stats,
                          float* metrics, void* ws, hipStream_t st) {
  if (a.n == 0) return launch_finalize(nullptr, 1, a, row_stats, metrics, st);
  if (zdt == kBF16 && udt == kBF16)
    return forward_typed<uint16_t, uint16_t>(z, ldz, u, ldu, v, a, dl, ldd, row_stats, metrics, ws, st);
  if (zdt == kBF16 && udt == kF32)
    return forward_typed<uint16_t, float>(z, ldz, u, ldu, v, a, dl, ldd, row_stats, metrics, ws, st);
  if (zdt == kF32 && udt == kBF16)
    return forward_typed<float, uint16_t>(z, ldz, u, ldu, v, a, dl, ldd, row_stats, metrics, ws, st);
  return forward_typed<float, float>(z, ldz, u, ldu, v, a, dl, ldd, row_stats, metrics, ws, st);
}

hipError_t stream_backward(const void* z, int zdt, int64_t ldz, const void* u, int udt, int64_t ldu,
                           int64_t v, const SlotArgs& a, const float* row_stats, void* dl, int64_t ldd,
                           hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  const int S = emit_splits(v);
  if (zdt == kBF16 && udt == kBF16)
    return emit_dispatch<uint16_t, uint16_t, true, false>(z, ldz, u, ldu, v, a, row_stats, dl, ldd, nullptr, S, st);
  if (zdt == kBF16 && udt == kF32)
    return emit_dispatch<uint16_t, float, true, false>(z, ldz, u, ldu, v, a, row_stats, dl, ldd, nullptr, S, st);
  if (zdt == kF32 && udt == kBF16)
    return emit_dispatch<float, uint16_t, true, false>(z, ldz, u, ldu, v, a, row_stats, dl, ldd, nullptr, S, st);
  return emit_dispatch<float, float, true, false>(z, ldz, u, ldu, v, a, row_stats, dl, ldd, nullptr, S, st);
}

}  // namespace ns
