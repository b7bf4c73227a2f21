// Fused LM head + draft objective on bf16 MFMA (gfx950, v_mfma_f32_32x32x16_bf16).
//
// Forward (nanospec/train.py:272-279 + objective.py:49-67), never storing logits:
//   z^T tile = W_lm[v-tile] . hidden[t-tile]^T   (vocab on the MFMA M axis, tokens on N)
//   pass 1 ("stats"): epilogue adds the Markov tile, reads the teacher tile and folds
//     (max, sum-exp) of z and u plus A = sum exp(u - m_u)(u - z) into per-token running
//     state kept in LDS across the workgroup's vocab range -> RowPart partials; the lane
//     that owns (token, label) writes z_label.
//   merge (shared with the logits path): LSE_z, LSE_u, CE, KL per token.
//   pass 2 ("emit"): recomputes the z tile, p = exp(z - LSE_z), t = exp(u - LSE_u),
//     accumulates sum min(p, t) and writes dl = (w/acc)[(c_ce + c_kl) p - c_kl t - c_ce e_y]
//     as bf16.
// Backward (train.py:302): dh = dl . W_lm as a long-K (K = V) split-K MFMA GEMM with a
// fixed-order fp32 reduction of the split partials.
//
// Layout choices (MI355X): one 256-thread workgroup per CU (4 waves, 2 x 2, each a
// 128 x 128 accumulator tile = 256 AGPRs/lane), 256 x 256 x 64 LDS stages double
// buffered with an XOR swizzle on 16-byte chunks, an epilogue that works on the
// accumulators in place while the tile's Markov and teacher rows come into the freed
// stage buffers, persistent workgroups that walk a contiguous vocab range with per-token
// running statistics, and a workgroup -> tile map that puts the workgroups sharing a W
// stream on the same XCD (shared L2).
#include <type_traits>

#include "ns_gemm.h"
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int BM = 256;          // MFMA rows per workgroup tile
constexpr int BN = 256;          // MFMA columns per workgroup tile
constexpr int BK = 64;           // K per LDS stage
constexpr int kThreads = 256;    // 4 waves as 2 (M) x 2 (N), 128 x 128 each
constexpr int kStageBytes = BM * BK * 2;    // 32 KB per operand per stage
constexpr int kGemmLds = 4 * kStageBytes;   // 2 stages x 2 operands = 128 KB

// Wait states between the K loop's last v_mfma_f32_32x32x16_bf16 and the epilogue's
// inline-asm v_accvgpr_read_b32 of its result, which the compiler's hazard tracking does
// not see.  CDNA3/CDNA4 ask for (passes + 2) wait states between an XDL write and a VALU
// read of the same register; the 32x32x16 bf16 form is taken at 16 passes (the count of
// its 32x32x8 predecessor, an upper bound on gfx950).  Each s_nop 7 gives 8.  A change of
// the K loop's MFMA must change kAccMfmaPasses with it.
constexpr int kAccMfmaPasses = 16;
constexpr int kAccReadWaitStates = kAccMfmaPasses + 2;
constexpr int kAccReadNops = (kAccReadWaitStates + 7) / 8;
static_assert(kAccReadNops * 8 >= kAccReadWaitStates, "too few s_nop 7 before the accumulator reads");
static_assert(kAccReadNops == 3, "the epilogue's s_nop sequence below is written out for 3");



// MFMA operand fragments of one 16-wide K step for this wave's 128 x 128 block.
struct Frags {
  bf16x8_t a[4], b[4];
};

__device__ __forceinline__ void zero_acc(f32x16_t (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
}

// Operand rows i of fragment step kk (one A and one B fragment).
__device__ __forceinline__ void load_frag_pair(Frags& f, const lds_t* la, const lds_t* lb, int kk, int i) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r = lane & 31, kh = lane >> 5;
  f.a[i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
      la + lds_off(wm * 128 + i * 32 + r, kk * 2 + kh));
  f.b[i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
      lb + lds_off(wn * 128 + i * 32 + r, kk * 2 + kh));
}

// Wait for this wave's LDS operations only, then a workgroup barrier (outstanding global
// loads, LDS fills included, keep flying).  s_waitcnt encoding: vmcnt 63, expcnt 7,
// lgkmcnt 0.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// acc += A[a0:a0+256, :K] . B[b0:b0+256, :K]^T, both row-major with K contiguous and
// K a multiple of BK.
//
// Operands go global -> LDS without registers; stage t lives in LDS buffer t & 1.  A
// stage's 64 MFMAs run one per instruction slot (slot 4 q + j of step kk) with the other
// work of the stage between them:
//   steps 0-2: fragment reads for the next step in slots 0-7;
//   step 3: fill_barrier first (stage t + 1 complete; every wave's reads of buffer t & 1,
//           the last issued in step 2, done), then in slots 0-7 the fragment reads of
//           stage t + 1 step 0.
// The barrier cannot come earlier: step 2 still reads buffer t & 1 and the step-0
// fragment registers.  Placing it at the start of step 3 rather than after two of its
// MFMA groups gives the next stage's first reads 8 more slots: 3.6-3.9% off each head
// pass at C2.
//
// A stage's 16 fills per wave (f = 0..7: A blocks, 8..15: B blocks) go out one every
// third slot across three steps: fills 0-5 of stage t + 2 in step 3 of stage t (slots
// 0, 3, .., 15, into buffer t & 1 just freed), fills 6-10 of stage t + 1 in step 0
// (slots 1, 4, .., 13) and 11-15 in step 1 (slots 0, 3, .., 12).  Eight fills in
// consecutive slots (four waves: 256 lines) stalled each wave's issue behind its own
// burst: the CU then averaged 60-62 line misses in flight to the L2, 74 with the spread
// (TCP_TCC_READ_REQ_LATENCY over cycles).  Spreading them over three steps took 1.5-2.7%
// off each head pass at C2 and 1.5-2.5% at C3; over all four, the fills of step 2 land
// after the barrier wants them (4-6% slower).
//
// The last stages would fill stages past the end.  With `tail.on` and KT >= 2 the slots
// of two of those fills issue the caller's next loads instead (the epilogue's first
// stream step, into the buffer the GEMM is done with): tail.issue(sb, 0, i, buf) in
// slots 0-7 of step 3 of stage KT - 2 (buffer KT & 1, free after that stage's barrier)
// and tail.issue(sb, 1, i, buf) in slots 8-15 of step 0 of stage KT - 1 (the same
// buffer); the last stage issues no fills, and its step-3 barrier waits for LDS reads
// only, not for those loads.  Returns true in that case, with the loads still in flight;
// otherwise fills past the last stage re-read the last stage into the idle buffer and the
// function ends with a full barrier (LDS free).
//
// The operand tiles come in ready-made: `ta`/`tb` hold the per-lane offsets of the
// 256 rows of each operand from the uniform bases `pa`/`pb` (stage 0), and stage t reads
// 128 bytes further along K each step; KT stages.
template <typename Tail>
__device__ __forceinline__ bool gemm_nt_tiles(f32x16_t (&acc)[4][4], const DmaTile<256>& ta, const char* pa,
                                              const DmaTile<256>& tb, const char* pb, int KT, lds_t* lds,
                                              const Tail& tail) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool tl = tail.on && KT >= 2;
  auto stage_k = [&](int t) -> int64_t { return (int64_t)(t < KT - 1 ? t : KT - 1) * BK * 2; };
  auto buf = [&](int t) -> lds_t* { return lds + (t & 1) * 2 * kStageBytes; };
#pragma unroll
  for (int i = 0; i < 8; ++i) ta.issue(pa, buf(0), wv, i);
#pragma unroll
  for (int i = 0; i < 8; ++i) tb.issue(pb, buf(0) + kStageBytes, wv, i);
  fill_barrier();
  Frags f[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) load_frag_pair(f[0], buf(0), buf(0) + kStageBytes, 0, i);
  {
    const int64_t k1 = stage_k(1);
#pragma unroll
    for (int f = 0; f < 6; ++f) ta.issue(pa + k1, buf(1), wv, f);   // stage 1's fills 0-5
  }
  // stage t; MODE 0: an ordinary stage, 1: stage KT - 2 and 2: stage KT - 1 with the tail
  auto stage = [&](auto mode, int t) {
    constexpr int M = decltype(mode)::value;
    decltype(tail.bases()) sb{};
    if constexpr (M != 0) sb = tail.bases();
    const lds_t* cur = buf(t);
    lds_t* nxt = buf(t + 1);
    const int64_t k1 = stage_k(t + 1), k2 = stage_k(t + 2);
    const int lane = threadIdx.x & 63;
    const int wm = wv >> 1, wn = wv & 1;
    const int r = lane & 31, kh = lane >> 5;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int cb = kk & 1;
      if (kk == 3) {
        if (M == 2) lds_barrier();
        else fill_barrier();
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[q][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[cb].a[q], f[cb].b[j], acc[q][j], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
          const int i = 2 * (q & 1) + (j >> 1);
          if (kk < 3 && q < 2) {
            if ((j & 1) == 0)
              f[cb ^ 1].a[i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
                  cur + lds_off(wm * 128 + i * 32 + r, (kk + 1) * 2 + kh));
            else
              f[cb ^ 1].b[i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
                  cur + kStageBytes + lds_off(wn * 128 + i * 32 + r, (kk + 1) * 2 + kh));
          }
          const int sl = 4 * q + j;
          if (kk == 0 && q >= 2 && M == 2) tail.issue(sb, 1, (q - 2) * 4 + j, nxt);
          // fills 6-10 and 11-15 of stage t + 1
          if (M != 2 && ((kk == 0 && sl % 3 == 1) || (kk == 1 && sl % 3 == 0 && sl < 15))) {
            const int f = kk == 0 ? 6 + sl / 3 : 11 + sl / 3;
            if (f < 8) ta.issue(pa + k1, nxt, wv, f);
            else tb.issue(pb + k1, nxt + kStageBytes, wv, f - 8);
          }
          if (kk == 3 && q < 2) {
            if (M != 2) {
              if ((j & 1) == 0)
                f[0].a[i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
                    nxt + lds_off(wm * 128 + i * 32 + r, kh));
              else
                f[0].b[i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
                    nxt + kStageBytes + lds_off(wn * 128 + i * 32 + r, kh));
            }
            if (M == 1) tail.issue(sb, 0, q * 4 + j, buf(t));
          }
          // fills 0-5 of stage t + 2 (A blocks 0-5) into the buffer just freed
          if (kk == 3 && M == 0 && sl % 3 == 0) ta.issue(pa + k2, buf(t), wv, sl / 3);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };
  const int tmain = tl ? KT - 2 : KT;
  for (int t = 0; t < tmain; ++t) stage(std::integral_constant<int, 0>(), t);
  if (tl) {
    stage(std::integral_constant<int, 1>(), KT - 2);
    stage(std::integral_constant<int, 2>(), KT - 1);
  }
  if (!tl) fill_barrier();
  return tl;
}



// acc += A[a0:a0+256, :K] . B[b0:b0+256, :K]^T (row-major, K contiguous, K % BK == 0);
// rows at or past amax / bmax re-read the last row.
template <typename Tail>
__device__ __forceinline__ bool gemm_nt(f32x16_t (&acc)[4][4], const uint16_t* __restrict__ A, int64_t lda,
                                        int64_t a0, int64_t amax, const uint16_t* __restrict__ B, int64_t ldb,
                                        int64_t b0, int64_t bmax, int64_t K, lds_t* lds, const Tail& tail) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  DmaTile<256> ta, tb;
  ta.init(lda * 2, a0, amax, wv);
  tb.init(ldb * 2, b0, bmax, wv);
  return gemm_nt_tiles(acc, ta, reinterpret_cast<const char*>(A + a0 * lda), tb,
                       reinterpret_cast<const char*>(B + b0 * ldb), (int)(K / BK), lds, tail);
}

// ---- dh GEMM: 32-K stages in a 4-deep LDS ring ----------------------------------------------
// acc += A[a0:a0+256, k0:k0+32 S] . B[k0:k0+32 S, c0:c0+256] (+ a partial stage of kv < 32
// K entries), A row-major (K contiguous), B row-major [K, cols].  Both operands go straight into
// LDS; the fills of stage t + 3 go out during stage t, so every fill has two to three stages of
// lead (with 64-K stages in two buffers the last fills of a stage had about half a stage).  The
// fills are issued through inline asm (dma16_asm): with the builtin the compiler, unable to tell
// a stage's fragment reads from a later stage's fills, waited for every outstanding fill before
// each read (9.37 ms against 7.57 ms at C2); the explicit vmcnt waits below order them.  The
// four ring buffers are separate LDS arrays and the stage loop is unrolled by 8, so every
// fragment address is a constant offset: with a computed buffer index the loop ran 2% slower.
//
// A stage: 256 rows x 64 B (32 bf16 along K); chunk c of row m at m * 64 + ((c ^ sw4(m)) << 4),
// sw4(m) = (m >> 2) & 3, so the 16 rows of a ds_read_b128 lane group hit 16 distinct 16-byte
// bank slots.  B stage: 32 rows x 512 B, as DmaTileKNR<32> (transposed fragment reads).
constexpr int BK2 = 32;                     // K per ring stage
constexpr int kRingStage = BM * BK2 * 2;    // 16 KB per operand per stage
constexpr int kRingBuf = 2 * kRingStage;    // one ring buffer: A then B
constexpr int kRingUnroll = 8;              // stages per loop iteration (a multiple of 4)

__device__ __forceinline__ int a32_off(int m, int c) { return m * 64 + ((c ^ ((m >> 2) & 3)) << 4); }

// A stage fetched straight into LDS: fill i of wave wv writes rows 16 (4 wv + i) .. +15; lane l
// fetches logical chunk (l & 3) ^ sw4(row) of row 16 (4 wv + i) + l / 4.  Rows at or past rmax
// re-read row rmax - 1 (their results are discarded).
struct DmaTileA32 {
  uint32_t off[4];
  __device__ __forceinline__ void init(int64_t ld_bytes, int64_t r0, int64_t rmax, int wv) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (wv * 4 + i) * 16 + (lane >> 2);
      int64_t r = r0 + row;
      r = r < rmax ? r : rmax - 1;
      const int chunk = (lane & 3) ^ ((row >> 2) & 3);
      off[i] = (uint32_t)((r - r0) * ld_bytes + chunk * 16);
    }
  }
  __device__ __forceinline__ void issue(const char* base, lds_t* dst, int wv, int i) const {
    dma16_asm(base, off[i], dst + (wv * 4 + i) * 1024);
  }
};

// A partial stage (kv < BK2 valid K entries, a multiple of 8) through registers into one ring
// buffer: K entries at or past kv are zero; A rows at or past amax and B columns at or past cmax
// re-read row a0 / column c0 (their results are discarded).
__device__ __forceinline__ void load_ring_tail(lds_t* dst, const uint16_t* A, int64_t lda, int64_t a0, int64_t amax,
                                               const uint16_t* B, int64_t ldb, int64_t c0, int64_t cmax, int kv) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {   // A: 256 rows x 4 chunks
    const int ci = i * 256 + tid;
    const int m = ci >> 2, c = ci & 3;
    int64_t row = a0 + m;
    row = row < amax ? row : a0;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (c * 8 < kv) x = *reinterpret_cast<const uint4*>(A + row * lda + c * 8);
    const u32x4_t y = {x.x, x.y, x.z, x.w};
    *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(dst + a32_off(m, c)) = y;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {   // B: 32 K rows x 32 chunks of 8 columns
    const int ci = i * 256 + tid;
    const int k = ci >> 5, cn = ci & 31;
    int64_t col = c0 + cn * 8;
    col = col < cmax ? col : c0;
    uint4 x = make_uint4(0, 0, 0, 0);
    if (k < kv) x = *reinterpret_cast<const uint4*>(B + (int64_t)k * ldb + col);
    const u32x4_t y = {x.x, x.y, x.z, x.w};
    *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(dst + kRingStage + k * 512 +
                                                                  ((cn ^ (4 * (k & 3))) << 4)) = y;
  }
}

// S full stages from k0, then (kv > 0) one partial stage.  `ring(b)` is ring buffer b (b < 4).
// Per stage t (two 16-K MFMA steps, one fragment read per MFMA slot in slots 0-11):
//   step 0: stage t's step-1 fragments; fills 0-3 of stage t + 3 in slots 1, 5, 9, 13;
//   step 1: first a barrier (stage t + 1 landed, and every wave is past stage t - 1's reads),
//           then stage t + 1's step-0 fragments and fills 4-7 of stage t + 3 in slots 1, 5, 9,
//           13, into stage t - 1's buffer.
// Fills and reads past the last stage re-read the last stage into a buffer nobody reads, so the
// loop body has no conditions but its stage count (branches in it made the compiler shuttle
// the accumulators between register files).  Ends with a barrier.
template <typename Ring>
__device__ __forceinline__ void gemm_nn_ring(f32x16_t (&acc)[4][4], const uint16_t* __restrict__ A, int64_t lda,
                                             int64_t a0, int64_t amax, const uint16_t* __restrict__ B,
                                             int64_t ldb, int64_t c0, int64_t cmax, int64_t k0, int S, int kv,
                                             const Ring& ring) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wv >> 1, wn = wv & 1;
  const int r = lane & 31, kh = lane >> 5;
  uint32_t tb_addr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) tb_addr[i] = tr_base(wn, i);
  bf16x8_t fa[2][4];
  TrFrag fb[2][4];
  // read op o (0..11) of step kk from stage buffer `sb` into set `c`: A i, B i lo, B i hi
  auto read_op = [&](int c, const lds_t* sb, int kk, int o) {
    const int i = o / 3, part = o % 3;
    if (part == 0)
      fa[c][i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
          sb + a32_off(wm * 128 + i * 32 + r, kk * 2 + kh));
    else if (part == 1)
      fb[c][i].lo = tr_read(sb + kRingStage, tb_addr[i] + kk * 8192);
    else
      fb[c][i].hi = tr_read(sb + kRingStage, tb_addr[i] + kk * 8192 + 2048);
  };
  auto mma = [&](int c, int q, int j) {
    acc[q][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[c][q], tr_join(fb[c][j]), acc[q][j], 0, 0, 0);
  };
  if (S > 0) {
    DmaTileA32 ta;
    DmaTileKNR<BK2> tb;
    ta.init(lda * 2, a0, amax, wv);
    tb.init(ldb, c0, cmax, wv);
    const char* pa = reinterpret_cast<const char*>(A + a0 * lda + k0);
    const char* pb = reinterpret_cast<const char*>(B + k0 * ldb + c0);
    const int64_t sb_bytes = (int64_t)BK2 * ldb * 2;
    auto fill = [&](int t, lds_t* dst, int f) {   // fill f (0-7) of stage min(t, S - 1): A 0-3, B 4-7
      const int64_t tc = t < S - 1 ? t : S - 1;
      if (f < 4)
        ta.issue(pa + tc * BK2 * 2, dst, wv, f);
      else
        tb.issue_asm(pb + tc * sb_bytes, dst + kRingStage, wv, f - 4);
    };
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int f = 0; f < 8; ++f) fill(t, ring(t), f);
    vm_barrier<16>();   // stage 0 landed; stages 1 and 2 may still fly
#pragma unroll
    for (int o = 0; o < 12; ++o) read_op(0, ring(0), 0, o);
    for (int t0 = 0; t0 < S; t0 += kRingUnroll) {
#pragma unroll
      for (int j = 0; j < kRingUnroll; ++j) {
        const int t = t0 + j;
        if (t < S) {
          const lds_t* cur = ring(j % 4);
          const lds_t* nxt = ring((j + 1) % 4);
          lds_t* far = ring((j + 3) % 4);
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            // stage t + 1 landed: stage t + 2's 8 fills and stage t + 3's first 4 may fly
            if (kk == 1) vm_barrier<12>();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) {
                const int sl = q * 4 + jj;
                mma(kk, q, jj);
                __builtin_amdgcn_sched_barrier(0);
                if (sl < 12) read_op(kk ^ 1, kk == 0 ? cur : nxt, kk ^ 1, sl);
                if ((sl & 3) == 1) fill(t + 3, far, kk * 4 + (sl >> 2));
                __builtin_amdgcn_sched_barrier(0);
              }
            }
          }
        }
      }
    }
  }
  if (kv > 0) {
    fill_barrier();   // every fill landed; every wave is past its last ring read
    const int64_t kt = k0 + (int64_t)S * BK2;
    load_ring_tail(ring(0), A + kt, lda, a0, amax, B + kt * ldb, ldb, c0, cmax, kv);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int o = 0; o < 12; ++o) read_op(0, ring(0), kk, o);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) mma(0, q, jj);
    }
  }
  fill_barrier();
}

// ------------------------------------------------------------------ head kernel

struct HeadParams {
  const uint16_t* hidden;   // [N, d] bf16
  const uint16_t* weight;   // [V, d] bf16
  const uint16_t* markov;   // [N, V] bf16 or null
  const void* teacher;      // [N, V] bf16 / f32
  int64_t ldh, ldw, ldm, ldt;
  int64_t n, d, v;
  int tt, vt, splits;       // token tiles, vocab tiles, vocab splits
  int xa, xb;               // XCD round block (wg_coords), 0 = unblocked
  // Markov head as a second K segment (r > 0): z += W1[prev] . W2^T
  const int64_t* prev;      // [N] previous-token ids
  const uint16_t* w1;       // [V, r] bf16 (embedding)
  const uint16_t* w2;       // [V, r] bf16 (projection)
  int64_t ldw1, ldw2, r;
  const int64_t* labels;
  const float* weights;
  float c_ce, c_kl, inv_acc;
  const float* row_stats;   // pass 2 input
  RowPart* part1;           // pass 1 output [N][splits]
  float* zy;                // pass 1 output [N]
  float* parta;             // pass 2 output [N][splits]
  uint16_t* dl;             // pass 2 output [N, V] bf16 or null
  int64_t ldd;
  uint16_t* out;            // MODE_STORE output [N, V] bf16
  int64_t ldo;
  // teacher rows (the gather of train.py:285-290): objective row t reads teacher row
  // trows[t] of nt rows; an index outside [0, nt) makes the row's teacher NaN.  null: row t
  const int64_t* trows;
  int64_t nt;
  // gathered bf16 teacher rows that may lie 4 GiB or more apart: the epilogue reads them
  // itself instead of loading them into LDS (whose loads take 32-bit offsets)
  bool tdirect;
  // teacher log-normalisers from the teacher's producer, one per teacher row (kTeacherLse):
  // pass 1 reads no teacher, pass 2 writes partk[N][splits] = sum t (u - z) for KL
  const float* tlse;
  float* partk;
  // MODE_STORE: B rows gathered as hidden[hrows[t]] of nh rows (null: row t); with
  // kStoreLse, part1 receives the (max, sum-exp) partials of the stored bf16 values
  const int64_t* hrows;
  int64_t nh;
  // launches by round (launch_head): this launch's first workgroup id and the whole grid; 0: one launch
  int wg0, wg_total;
};

enum { MODE_STATS = 0, MODE_EMIT = 1, MODE_STORE = 2 };
// head_kernel variants: the teacher's log-normaliser is given (STATS / EMIT), the stored
// values' log-sum-exp partials are formed (STORE)
enum { kTeacherLse = 1, kStoreLse = 2 };

// Head-kernel LDS beyond the GEMM stages: per-token running state and per-token
// constants of the workgroup's 256 tokens (they persist across vocab tiles).  The state
// is kept per vocab half (the two waves holding a token each cover 128 of a tile's 256
// vocab entries) and the halves are merged once, after the last tile.
constexpr int kStateOff = kGemmLds;                   // [2][256][8] fp32: mz sz mu su A | arate kl
constexpr int kConstOff = kStateOff + 2 * 256 * 8 * 4;  // [256][8] fp32: lzl lul cp ct cy zy
constexpr int kLabelOff = kConstOff + 256 * 8 * 4;    // [256] int64 labels
constexpr int kPrevOff = kLabelOff + 256 * 8;        // [256] int32 W1 rows (ids clamped to [0, V))
constexpr int kBadOff = kPrevOff + 256 * 4;          // [256] uint8: id outside [0, V)
constexpr int kTrowOff = kBadOff + 256;             // [256] int32 teacher rows (0 when out of range)
constexpr int kTbadOff = kTrowOff + 256 * 4;        // [256] uint8: teacher (STORE: B) row out of range
constexpr int kHrowOff = kTbadOff + 256;            // [256] int32 gathered B rows (MODE_STORE)
constexpr int kHeadLdsBytes = kHrowOff + 256 * 4;
static_assert(kHeadLdsBytes <= 160 * 1024, "head kernel LDS");

// Lanes l and l ^ 32 hold the same token (vocab entries 4 h .. 4 h + 3 of each 8-entry
// chunk, h = l / 32).  v_permlane32_swap hands every lane both lanes' values in the same
// order, so a symmetric merge of the two leaves identical bits in both.
__device__ __forceinline__ void half_pair(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

__device__ __forceinline__ float half_sum(float x) {
  float a, b;
  half_pair(x, a, b);
  return a + b;
}

__device__ __forceinline__ PairState half_merge(const PairState& s) {
  PairState a, b;
  half_pair(s.mz, a.mz, b.mz);
  half_pair(s.sz, a.sz, b.sz);
  half_pair(s.mu, a.mu, b.mu);
  half_pair(s.su, a.su, b.su);
  half_pair(s.A, a.A, b.A);
  return pair_merge(a, b);
}

__device__ __forceinline__ LseState half_merge(const LseState& s) {
  LseState a, b;
  half_pair(s.m, a.m, b.m);
  half_pair(s.s, a.s, b.s);
  return lse_merge(a, b);
}

// One distribution's online (max, sum-exp) over W values.
template <int W>
__device__ __forceinline__ void lse_update(LseState& st, const float* z) {
  float b = z[0];
#pragma unroll
  for (int i = 1; i < W; ++i) b = fmaxf(b, z[i]);
  const float m = fmaxf(st.m, b);
  const float ml = m * kLog2e;
  float s = st.s * fast_exp2((st.m - m) * kLog2e);
#pragma unroll
  for (int i = 0; i < W; ++i) s += fast_exp2(__builtin_fmaf(z[i], kLog2e, -ml));
  st = {m, s};
}

// pair_update<32> / lse_update<32> with f(g) called after each group of 8 exponentials
// (the same arithmetic in the same order; the group's sums are pinned before the call)
template <typename F>
__device__ __forceinline__ void pair_update32(PairState& st, const float* z, const float* u, F&& f) {
  float bz = z[0], bu = u[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) {
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
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int i = 8 * g; i < 8 * g + 8; ++i) {
      sz += fast_exp2(__builtin_fmaf(z[i], kLog2e, -mzl));
      const float e = fast_exp2(__builtin_fmaf(u[i], kLog2e, -mul));
      su += e;
      A = __builtin_fmaf(e, u[i] - z[i], A);
    }
    asm volatile("" : "+v"(sz), "+v"(su), "+v"(A));
    f(g);
  }
  st = {mz, sz, mu, su, A};
}

template <typename F>
__device__ __forceinline__ void lse_update32(LseState& st, const float* z, F&& f) {
  float b = z[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) b = fmaxf(b, z[i]);
  const float m = fmaxf(st.m, b);
  const float ml = m * kLog2e;
  float s = st.s * fast_exp2((st.m - m) * kLog2e);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int i = 8 * g; i < 8 * g + 8; ++i) s += fast_exp2(__builtin_fmaf(z[i], kLog2e, -ml));
    asm volatile("" : "+v"(s));
    f(g);
  }
  st = {m, s};
}

// ---- the epilogue's stream
//
// The epilogue works on the accumulators where the MFMAs left them: lane 32 h + r of wave
// (wm, wn) holds, for each 32-token column block j, token 128 wn + 32 j + r at the vocab
// entries 128 wm + 32 i + 8 g + 4 h + q (i, g, q = 0..3) as acc[i][j][4 g + q].  It runs
// in four steps; step s takes column block s of both 128-token halves, 64 tokens.  Their
// Markov and teacher rows (the tile's 256 entries: 512 bytes of bf16 per row) come
// straight into LDS, into the step's slot: one of the two 64 KB GEMM stage buffers, with
// the Markov rows at +0 and the teacher rows at +kSlotU.  Step 0 is loaded during the
// GEMM's last stages (gemm_nt_tiles' tail).  Step s + 1 goes into the other slot while step
// s is worked, one load after each piece of work: issued at once, a step's loads filled
// the memory queue of the CU and stalled the wave's issue for about as long as the work.
// (These rows come from HBM, unlike the GEMM's operands, which mostly hit the L2.)
//
// A slot half holds 32 blocks of 1 KB, each written by one 64-lane load: block b holds
// step tokens 2b and 2b + 1 (step token e is tile token 128 (e / 32) + 32 s + e % 32), and
// its 16-byte slot 32 pb + (c ^ sw) holds chunk c (entries 8c .. 8c + 7) of token 2b + pb,
// sw = 2 (b & 7) + pb.  The lane reading chunk c of token 32 wn + r finds its 8 bytes at
// 16 KB wn + 512 r + 16 (c ^ (r & 15)) + 8 h, so the 16 lanes r = 0..15 (or 16..31) of one
// read hit 16 distinct 16-byte bank groups.
//
// EMIT and STORE write their bf16 outputs over the Markov rows they read (each lane over
// its own 8 bytes), then read them back as whole 256-byte row pieces (16 lanes per token,
// the wave's vocab half) and store those as coalesced rows.  Every lane stores (out-of-
// range lanes into a sink), so the next step's wait can leave exactly these eight stores
// in flight.
constexpr int kSlotU = 64 * 512;   // teacher rows after the 64 Markov rows

// A row of zeros standing in for the dense Markov addend when there is none, so every step
// loads the same number of blocks (1 KB: the widest offset is 496 + 16 bytes).
__device__ uint4 kZeroRow[64] = {};

// Where the epilogue's out-of-range lanes store (their values are never read).
__device__ u32x4_t kStoreSink[64];

// One 64-lane load into the 1 KB LDS block dst of block b: lane l fetches chunk
// c = (l % 32) ^ (2 (b & 7) + l / 32), entries 8c .. 8c + 7 of the tile, of the row at byte
// offset `row` from the uniform tile base (chunks at or past v - v0 re-read chunk 0).
__device__ __forceinline__ void stream_dma(const char* base, uint32_t row, int64_t vleft, lds_t* dst, int b,
                                           int lane) {
  const int c = (lane & 31) ^ (2 * (b & 7) + (lane >> 5));
  dma16(base, row + (uint32_t)((8 * c < vleft ? c : 0) * 16), dst);
}

// Uniform operands of the stream loads of one tile, read from the kernel arguments where
// they are used (see StreamTail::bases).
struct StreamBases {
  const char* mbase;   // Markov rows: the tile's first row at column v0 (or the zero row)
  const char* ubase;   // teacher rows: likewise, or the teacher's row 0 for gathered rows
  uint32_t mld, uld;   // row pitches in bytes (0 for the zero row)
  int umode;           // 0: the tile's rows, 1: gathered rows, 2: none (zero row)
  int rlast;           // the tile's last row below N (rows past it re-read it)
  int64_t vleft;       // V - v0
};

template <int MODE, typename TT, int FLAGS>
struct StreamTail {
  // the teacher is read in pass 2, and in pass 1 unless its log-normaliser is given
  static constexpr bool kReadU = MODE == MODE_EMIT || (MODE == MODE_STATS && !(FLAGS & kTeacherLse));
  // bf16 teacher rows come through LDS; fp32 rows are read by the epilogue itself
  static constexpr bool kDmaU = kReadU && sizeof(TT) == 2;
  static constexpr int kLoads = kDmaU ? 16 : 8;   // loads per wave per step
  const lds_t* lds;
  int64_t t0, v0;
  bool on;
  // the thread index, opaque to the compiler: address arithmetic derived from it stays in
  // the vocab-tile loop instead of being hoisted out and kept live across the K loop
  int tid;

  // The bases, from the kernel arguments (scalar loads) and opaque copies of t0 and v0, so
  // that nothing of them is computed ahead and held across the K loop.  Offsets are 32-bit
  // from a uniform base: the tile's first row (rows within 256 of it; the C ABI caps leading
  // dimensions at 2^23 elements, so 255 rows and a row's 512 bytes stay below 4 GiB), or the
  // teacher's row 0 for gathered rows (all within 4 GiB unless tdirect, where the epilogue
  // reads them).
  __device__ __forceinline__ StreamBases bases() const {
    const __attribute__((address_space(4))) HeadParams* kp =
        (const __attribute__((address_space(4))) HeadParams*)__builtin_amdgcn_kernarg_segment_ptr();
    int64_t t0o = t0, v0o = v0;
    asm volatile("" : "+s"(kp), "+s"(t0o), "+s"(v0o));
    StreamBases sb;
    const uint16_t* m = kp->markov;
    sb.mbase = m ? reinterpret_cast<const char*>(m + t0o * kp->ldm + v0o) : reinterpret_cast<const char*>(kZeroRow);
    sb.mld = m ? (uint32_t)(kp->ldm * 2) : 0u;
    sb.rlast = (int)(kp->n - 1 - t0o);
    sb.vleft = kp->v - v0o;
    sb.umode = 2;
    sb.ubase = reinterpret_cast<const char*>(kZeroRow);
    sb.uld = 0;
    if (kDmaU && !kp->tdirect) {
      const uint16_t* u = static_cast<const uint16_t*>(kp->teacher);
      sb.umode = kp->trows ? 1 : 0;
      sb.ubase = reinterpret_cast<const char*>(kp->trows ? u + v0o : u + t0o * kp->ldt + v0o);
      sb.uld = (uint32_t)(kp->ldt * 2);
    }
    return sb;
  }

  // load i (0..7) of this wave's Markov (region 0) or teacher (region 1) rows of step s
  __device__ __forceinline__ void load(const StreamBases& sb, int s, int region, int i, lds_t* slot) const {
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int b = 8 * wv + i;
    const int tk = (b >> 4) * 128 + 32 * s + 2 * (b & 15) + (lane >> 5);   // this lane's token
    const int rl = tk < sb.rlast ? tk : sb.rlast;
    lds_t* dst = slot + (region ? kSlotU : 0) + b * 1024;
    if (region == 0) {
      stream_dma(sb.mbase, (uint32_t)rl * sb.mld, sb.vleft, dst, b, lane);
    } else if (kDmaU) {
      uint32_t row = (uint32_t)rl * sb.uld;
      if (sb.umode == 1)   // gathered teacher rows (checked and clamped at kernel start)
        row = (uint32_t)reinterpret_cast<const __attribute__((address_space(3))) int*>(lds + kTrowOff)[tk] * sb.uld;
      stream_dma(sb.ubase, row, sb.vleft, dst, b, lane);
    }
  }
  __device__ __forceinline__ void load_step(int s, lds_t* slot) const {
    const StreamBases sb = bases();
#pragma unroll
    for (int ci = 0; ci < 16; ++ci) load_part(sb, s, ci, slot);
  }
  // gemm_nt_tiles' tail: part 0 = step 0's Markov rows, 1 = step 0's teacher rows
  __device__ __forceinline__ void issue(const StreamBases& sb, int part, int i, lds_t* slot) const {
    load(sb, 0, part, i, slot);
  }
  // load ci (0..15) of step s, the loads of a step spread over the previous step's work:
  // Markov load ci / 2 for even ci, teacher load ci / 2 for odd ci (none without them)
  __device__ __forceinline__ void load_part(const StreamBases& sb, int s, int ci, lds_t* slot) const {
    if ((ci & 1) == 0 || kDmaU) load(sb, s, ci & 1, ci >> 1, slot);
  }

  // The epilogue's own loads (steps 1-3) from per-lane offsets set up once per tile, for
  // tiles whose 256 rows all lie below N and whose teacher rows are the tile's own (or
  // none): load i of a region reads base + off[i] + s * 32 rows, the step term as the
  // instruction's scalar offset.  load() re-derives each address from the thread index,
  // about 15 instructions a load, and with one wave per SIMD every instruction of the
  // epilogue costs an issue slot.  Such a tile never reads teacher rows itself (tdirect
  // implies gathered rows), so its epilogue has no global loads of its own.
  struct Offsets {
    uint32_t m[8], u[8];
    int wv;
  };
  __device__ __forceinline__ static bool direct(const StreamBases& sb) {
    return sb.rlast >= BN - 1 && (kDmaU ? sb.umode == 0 : true);
  }
  __device__ __forceinline__ void offsets(const StreamBases& sb, Offsets& o) const {
    const int lane = tid & 63;
    o.wv = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int b = 8 * o.wv + i;
      const int tk = (b >> 4) * 128 + 2 * (b & 15) + (lane >> 5);   // the lane's token in step 0
      const int c = (lane & 31) ^ (2 * (b & 7) + (lane >> 5));
      const uint32_t cc = (uint32_t)((8 * c < sb.vleft ? c : 0) * 16);
      o.m[i] = (uint32_t)tk * sb.mld + cc;
      o.u[i] = (uint32_t)tk * sb.uld + cc;
      // held in registers for the epilogue, not re-derived at each use
      asm volatile("" : "+v"(o.m[i]), "+v"(o.u[i]));
    }
  }
  __device__ __forceinline__ void load_direct(const StreamBases& sb, const Offsets& o, int s, int ci,
                                              lds_t* slot) const {
    const int i = ci >> 1;
    lds_t* dst = slot + (8 * o.wv + i) * 1024;
    if ((ci & 1) == 0)
      dma16(sb.mbase, o.m[i], dst, (uint32_t)(32 * s) * sb.mld);
    else if (kDmaU)
      dma16(sb.ubase, o.u[i], dst + kSlotU, (uint32_t)(32 * s) * sb.uld);
  }
};

typedef uint32_t u32x2v_t __attribute__((ext_vector_type(2)));

// Objective epilogue of one 256 x 256 tile (layout above).  Each lane folds its token's
// 64 entries per step locally, the two lanes of a token combine (half_merge / half_sum),
// and the lane of the lower half folds the result into the token's running state for
// this wave's vocab half.  Sums over a tile are formed locally first: one running fp32
// sum over a whole vocab range (up to ~10^5 terms) would lose the many small terms.
// V % 8 == 0, so each 8-entry chunk is wholly inside or outside the vocabulary.
// `pre`: step 0 was loaded by the GEMM's tail (otherwise the K loop ended with a full
// barrier and it is loaded here).  Ends with every wave's LDS reads done.
template <int MODE, typename TT, int FLAGS, bool FULL, bool DIRECT>
__device__ __forceinline__ void epilogue_tile(const HeadParams& p, lds_t* lds, const f32x16_t (&acc)[4][4],
                                              const StreamTail<MODE, TT, FLAGS>& st, int KT, bool pre) {
  using ST = StreamTail<MODE, TT, FLAGS>;
  constexpr bool kReadU = ST::kReadU, kDmaU = ST::kDmaU;
  constexpr bool kOut = MODE == MODE_EMIT || MODE == MODE_STORE;
  const int64_t t0 = st.t0, v0 = st.v0;
  const int wv = __builtin_amdgcn_readfirstlane(st.tid >> 6);
  const int lane = st.tid & 63;
  const int wm = wv >> 1, wn = wv & 1;
  lds_f32* state = reinterpret_cast<lds_f32*>(lds + kStateOff) + wm * 256 * 8;
  const lds_f32* cst = reinterpret_cast<const lds_f32*>(lds + kConstOff);
  const __attribute__((address_space(3))) int64_t* lab =
      reinterpret_cast<const __attribute__((address_space(3))) int64_t*>(lds + kLabelOff);
  const __attribute__((address_space(3))) uint8_t* badf =
      reinterpret_cast<const __attribute__((address_space(3))) uint8_t*>(lds + kBadOff);
  const __attribute__((address_space(3))) uint8_t* tbadf =
      reinterpret_cast<const __attribute__((address_space(3))) uint8_t*>(lds + kTbadOff);
  auto slot = [&](int s) -> lds_t* { return lds + ((KT + s) & 1) * 2 * kStageBytes; };
  if (!pre) st.load_step(0, slot(0));
  // outputs go through LDS and out as rows (EMIT without dl writes nothing)
  const bool write = MODE == MODE_STORE || (MODE == MODE_EMIT && p.dl != nullptr);
  uint16_t* const out = MODE == MODE_STORE ? p.out : p.dl;
  const int64_t ldo = MODE == MODE_STORE ? p.ldo : p.ldd;
  const float nan = __builtin_nanf("");
  const StreamBases sb = st.bases();
  typename ST::Offsets so;
  if (DIRECT) st.offsets(sb, so);
  // Teacher rows read here rather than through LDS.  A direct tile never takes that path (it
  // implies gathered rows), and pass 1 drops it there: the compiler then sees no global loads
  // feeding the teacher values and no longer waits, in each step's second half, for the
  // stream loads the first half issued (0.8% off pass 1).  Pass 2 keeps the runtime test and
  // with it those waits and one for the previous step's row stores; dropping it there was
  // 0-1.5% slower (two boxes, C2 and C3).
  const bool tdirect = (MODE == MODE_STATS && DIRECT) ? false : p.tdirect;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    // this step's loads landed in every wave (after step 0, the previous step's eight row
    // stores may still fly), and every wave is done with the previous step's slot, which
    // the next step's loads go to while this step works
    if (s == 0) {
      vm_barrier<0>();
      // the K loop's last MFMAs may still be writing accumulators that the volatile reads
      // below take without the compiler's hazard wait states: kAccReadNops x 8 wait states
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    } else if (kOut && write) {
      vm_barrier<8>();
    } else {
      vm_barrier<0>();
    }
    // per-step copy of the lane index, opaque: the step's address arithmetic stays after
    // its barrier instead of being computed early and held in registers
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r = ln & 31, h = ln >> 5;
    // this lane's 8 bytes of chunk k (= 4 i + g) of its vocab half sit at lb + 16 (k ^ (r & 15))
    const int lb = wn * 16384 + r * 512 + wm * 256 + 8 * h;
    lds_t* sl = slot(s);
    // load ci of the next step, issued between this step's chunks so that the wave never
    // waits on a full memory queue with work left (a step's loads at once stalled issue)
    auto next = [&](int ci) {
      if (s < 3) {
        __builtin_amdgcn_sched_barrier(0);
        if (DIRECT)
          st.load_direct(sb, so, s + 1, ci, slot(s + 1));
        else
          st.load_part(sb, s + 1, ci, slot(s + 1));
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    const int tk = wn * 128 + 32 * s + r;   // this lane's token
    const int64_t t = t0 + tk;
    const bool tok_ok = t < p.n;
    const bool bad = badf[tk] != 0;
    const bool ubad = tbadf[tk] != 0;
    const int64_t y = MODE == MODE_STORE ? -1 : lab[tk];
    const int64_t yr = y - v0;
    // this lane holds entry y (labels outside [0, V) match nothing; the merge flags them)
    const bool mine = MODE != MODE_STORE && tok_ok && yr >= 0 && yr < BM && y < p.v && (int)(yr >> 7) == wm &&
                      (int)((yr >> 2) & 1) == h;
    const lds_f32* cr = cst + tk * 8;
    float lzl = 0.f, lul = 0.f, cp = 0.f, ct = 0.f;
    if (MODE == MODE_EMIT) {
      lzl = cr[0]; lul = cr[1]; cp = cr[2]; ct = cr[3];
    }
    const TT* urow = nullptr;
    if (kReadU && (!kDmaU || tdirect)) {
      const int trw = reinterpret_cast<const __attribute__((address_space(3))) int*>(lds + kTrowOff)[tk];
      urow = static_cast<const TT*>(p.teacher) + (int64_t)trw * p.ldt + v0;
    }
    PairState ploc = pair_init();
    LseState lloc = {kNegBig, 0.f};
    float aloc = 0.f, kloc = 0.f;
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
      __builtin_amdgcn_sched_barrier(0);   // one half-step's values live at a time
      // the accumulators are read where they are used (volatile: not hoisted above the
      // step's barrier, which would hold all 256 in VGPRs at once)
      float z[32], u[32];
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(z[16 * ii + e]) : "a"(acc[2 * hs + ii][s][e]));
      u32x2v_t mraw[8], uraw[8];
      int off[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int k = 8 * hs + c;   // chunk 4 i + g of the wave's vocab half
        off[c] = lb + ((k ^ (r & 15)) << 4);
        mraw[c] = *reinterpret_cast<const __attribute__((address_space(3))) u32x2v_t*>(sl + off[c]);
      }
      if (kDmaU) {
        if (tdirect) {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const int vl = wm * 128 + 8 * (8 * hs + c) + 4 * h;
            const bool in = FULL || v0 + wm * 128 + 8 * (8 * hs + c) < p.v;
            uraw[c] = *reinterpret_cast<const u32x2v_t*>(urow + (in ? vl : 0));
          }
        } else {
#pragma unroll
          for (int c = 0; c < 8; ++c)
            uraw[c] = *reinterpret_cast<const __attribute__((address_space(3))) u32x2v_t*>(sl + kSlotU + off[c]);
        }
      }
      // chunk c is inside the vocabulary; the first one of the half-step decides whether
      // the lane has any entry (a fold over sentinels only would form inf - inf)
      bool okc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) okc[c] = FULL || v0 + wm * 128 + 8 * (8 * hs + c) < p.v;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float mk[4];
        mk[0] = bf16_lo(mraw[c][0]); mk[1] = bf16_hi(mraw[c][0]);
        mk[2] = bf16_lo(mraw[c][1]); mk[3] = bf16_hi(mraw[c][1]);
        if (kDmaU) {
          u[4 * c + 0] = bf16_lo(uraw[c][0]); u[4 * c + 1] = bf16_hi(uraw[c][0]);
          u[4 * c + 2] = bf16_lo(uraw[c][1]); u[4 * c + 3] = bf16_hi(uraw[c][1]);
        } else if (kReadU) {
          const int vl = wm * 128 + 8 * (8 * hs + c) + 4 * h;
          const float4 x = *reinterpret_cast<const float4*>(urow + (okc[c] ? vl : 0));
          u[4 * c + 0] = x.x; u[4 * c + 1] = x.y; u[4 * c + 2] = x.z; u[4 * c + 3] = x.w;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float& zq = z[4 * c + q];
          if (MODE == MODE_STORE) {
            // a gathered B row outside its matrix: the output row is NaN
            zq = okc[c] ? (ubad ? nan : zq + mk[q]) : kNegBig;
          } else {
            zq = okc[c] ? zq + mk[q] : kNegBig;
            if (kReadU && !FULL) u[4 * c + q] = okc[c] ? u[4 * c + q] : kNegBig;
          }
        }
      }
      const bool any = FULL || okc[0];
      if (MODE == MODE_STATS) {
        auto next2 = [&](int g) {
          next(2 * (4 * hs + g));
          next(2 * (4 * hs + g) + 1);
        };
        if (FLAGS & kTeacherLse) {
          if (any) lse_update32(lloc, z, next2);
          else for (int g = 0; g < 4; ++g) next2(g);
        } else {
          if (any) pair_update32(ploc, z, u, next2);
          else for (int g = 0; g < 4; ++g) next2(g);
        }
        // the label entry, when this half-step holds it (rare: the label is in this tile)
        const bool here = mine && (int)((yr >> 6) & 1) == hs;
        if (__any(here)) {
          const int idx = (int)((((yr >> 5) & 1) << 4) | (((yr >> 3) & 3) << 2) | (yr & 3));
          float zv = 0.f;
#pragma unroll
          for (int k2 = 0; k2 < 32; ++k2) zv = k2 == idx ? z[k2] : zv;
          if (here) p.zy[t] = bad ? nan : zv;
        }
      } else if (MODE == MODE_EMIT) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float d[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float zq = z[4 * c + q], uq = u[4 * c + q];
            const float pp = fast_exp2(__builtin_fmaf(zq, kLog2e, -lzl));
            const float tt = fast_exp2(__builtin_fmaf(uq, kLog2e, -lul));
            aloc += min_nonneg(pp, tt);
            // KL's sum t (u - z) (entries past V: t = 0 and u = z)
            if (FLAGS & kTeacherLse) kloc = __builtin_fmaf(tt, uq - zq, kloc);
            d[q] = __builtin_fmaf(cp, pp, -ct * tt);
          }
          // written even without dl (never read back then): no branch in the loop
          const u32x2v_t o = {pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])};
          *reinterpret_cast<__attribute__((address_space(3))) u32x2v_t*>(sl + off[c]) = o;
          // the chunk's sums are formed here, not deferred with every chunk's values live
          asm volatile("" : "+v"(aloc), "+v"(kloc));
          next(8 * hs + c);
        }
      } else {   // MODE_STORE
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const u32x2v_t o = {pack_bf16x2(z[4 * c], z[4 * c + 1]), pack_bf16x2(z[4 * c + 2], z[4 * c + 3])};
          *reinterpret_cast<__attribute__((address_space(3))) u32x2v_t*>(sl + off[c]) = o;
          next(8 * hs + c);
        }
        if (FLAGS & kStoreLse) {
          // log-sum-exp of the values as stored (bf16), which is what a consumer reads
#pragma unroll
          for (int i = 0; i < 32; ++i) z[i] = bf16_to_f32(f32_to_bf16(z[i]));
          if (any) lse_update<32>(lloc, z);
        }
      }
    }
    // fold the step into the token's state (lanes of the lower half write)
    if (MODE == MODE_STATS && !(FLAGS & kTeacherLse)) {
      PairState loc = half_merge(ploc);
      if (bad) { loc.mz = nan; loc.sz = nan; }
      if (ubad) { loc.mu = nan; loc.su = nan; loc.A = nan; }
      if (h == 0) {
        lds_f32* sr = state + tk * 8;
        const PairState m2 = pair_merge(PairState{sr[0], sr[1], sr[2], sr[3], sr[4]}, loc);
        sr[0] = m2.mz; sr[1] = m2.sz; sr[2] = m2.mu; sr[3] = m2.su; sr[4] = m2.A;
      }
    } else if (MODE == MODE_STATS || (MODE == MODE_STORE && (FLAGS & kStoreLse))) {
      LseState loc = half_merge(lloc);
      if (MODE == MODE_STATS && bad) loc = {nan, nan};
      if (h == 0) {
        lds_f32* sr = state + tk * 8;
        const LseState m2 = lse_merge(LseState{sr[0], sr[1]}, loc);
        sr[0] = m2.m; sr[1] = m2.s;
      }
    } else if (MODE == MODE_EMIT) {
      aloc = half_sum(aloc);
      if (h == 0) state[tk * 8] += aloc;
      if (FLAGS & kTeacherLse) {
        kloc = half_sum(kloc);
        if (h == 0) state[tk * 8 + 1] += kloc;
      }
    }
    if (kOut && write) {
      if (MODE == MODE_EMIT && __any(mine)) {
        // the label entry: rewrite dl[y] with the -c_ce term over this lane's own store
        // (a bad row's NaN comes through its log-normaliser); z_y is pass 1's value
        if (mine) {
          const int k = (int)((yr >> 3) & 15);
          const int a = lb - 8 * h + ((k ^ (r & 15)) << 4) + 2 * (int)(yr & 7);
          const float uy = kDmaU && !tdirect
                               ? bf16_to_f32(*reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
                                     sl + kSlotU + a))
                               : load1(urow + yr);
          const float pp = fast_exp2(__builtin_fmaf(cr[5], kLog2e, -lzl));
          const float tt = fast_exp2(__builtin_fmaf(uy, kLog2e, -lul));
          *reinterpret_cast<__attribute__((address_space(3))) uint16_t*>(sl + a) =
              f32_to_bf16(__builtin_fmaf(cp, pp, -ct * tt) - cr[4]);
        }
      }
      // read back this wave's rows, 16 lanes per token and 4 tokens per read, and store
      // them; every lane stores (rows past N and chunks past V into a sink), so a step
      // always issues exactly eight stores, which the next step's wait counts on
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int r2 = 4 * k + (ln >> 4), cl = ln & 15;
        const u32x4_t x = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
            sl + (lb - r * 512 - 8 * h) + r2 * 512 + ((cl ^ (r2 & 15)) << 4));
        const int64_t t2 = t0 + wn * 128 + 32 * s + r2;
        const int64_t col = v0 + 8 * (wm * 16 + cl);
        const bool in = t2 < p.n && (FULL || col < p.v);
        *(in ? reinterpret_cast<u32x4_t*>(out + t2 * ldo + col) : &kStoreSink[ln]) = x;
      }
    }
  }
  lds_barrier();
}

template <int MODE, typename TT, int FLAGS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void head_kernel(HeadParams p) {
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_t* lds = (lds_t*)lds_raw;
  int tile_t, split;
  wg_coords(p.wg0 + (int)blockIdx.x, p.wg_total > 0 ? p.wg_total : (int)gridDim.x, p.tt, p.xa, p.xb, tile_t, split);
  const int vt_begin = (int)((int64_t)split * p.vt / p.splits);
  const int vt_end = (int)((int64_t)(split + 1) * p.vt / p.splits);
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)tile_t * BN;

  // per-token state and constants of this workgroup's 256 tokens (thread tid: token tid);
  // first read after the GEMM's barriers
  if (p.r > 0) {
    const int64_t t = t0 + tid;
    const int64_t id = p.prev[t < p.n ? t : p.n - 1];
    const bool ok = id >= 0 && id < p.v;
    reinterpret_cast<__attribute__((address_space(3))) int*>(lds + kPrevOff)[tid] = ok ? (int)id : 0;
    reinterpret_cast<__attribute__((address_space(3))) uint8_t*>(lds + kBadOff)[tid] = ok ? 0 : 1;
  } else {
    reinterpret_cast<__attribute__((address_space(3))) uint8_t*>(lds + kBadOff)[tid] = 0;
  }
  {
    // teacher row (MODE_STORE: gathered B row) of token tid, checked against its tensor
    const int64_t t = t0 + tid;
    const int64_t trow = t < p.n ? t : p.n - 1;
    const int64_t* rows = MODE == MODE_STORE ? p.hrows : p.trows;
    const int64_t lim = MODE == MODE_STORE ? p.nh : p.nt;
    const int64_t rr = rows ? rows[trow] : trow;
    const bool ok = !rows || (rr >= 0 && rr < lim);
    reinterpret_cast<__attribute__((address_space(3))) int*>(lds + kTrowOff)[tid] = ok ? (int)rr : 0;
    reinterpret_cast<__attribute__((address_space(3))) uint8_t*>(lds + kTbadOff)[tid] = ok ? 0 : 1;
    if (MODE == MODE_STORE)
      reinterpret_cast<__attribute__((address_space(3))) int*>(lds + kHrowOff)[tid] = ok ? (int)rr : 0;
  }
  if (MODE == MODE_STORE && (FLAGS & kStoreLse)) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      lds_f32* sr = reinterpret_cast<lds_f32*>(lds + kStateOff) + (half * 256 + tid) * 8;
      sr[0] = kNegBig;
      sr[1] = 0.f;
    }
  }
  // gathered B rows are read from LDS by every wave's fill offsets before the first barrier
  if (MODE == MODE_STORE && p.hrows) __syncthreads();
  if (MODE != MODE_STORE) {
    const int64_t t = t0 + tid;
    const int64_t trow = t < p.n ? t : p.n - 1;
    const PairState z0 = pair_init();
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      lds_f32* sr = reinterpret_cast<lds_f32*>(lds + kStateOff) + (half * 256 + tid) * 8;
      sr[0] = MODE == MODE_STATS ? z0.mz : 0.f;
      sr[1] = z0.sz; sr[2] = z0.mu; sr[3] = z0.su; sr[4] = z0.A;
    }
    reinterpret_cast<__attribute__((address_space(3))) int64_t*>(lds + kLabelOff)[tid] = p.labels[trow];
    if (MODE == MODE_EMIT) {
      lds_f32* cr = reinterpret_cast<lds_f32*>(lds + kConstOff) + tid * 8;
      const float w = p.weights[trow] * p.inv_acc;
      cr[0] = p.row_stats[trow * kRowStatWidth + kLseZ] * kLog2e;
      cr[1] = p.row_stats[trow * kRowStatWidth + kLseU] * kLog2e;
      // an ignored row has no CE term: dl = w c_kl (p - t) (its label matches no entry)
      cr[2] = p.labels[trow] == kIgnoreIndex ? w * p.c_kl : w * (p.c_ce + p.c_kl);
      cr[3] = w * p.c_kl;
      cr[4] = w * p.c_ce;
      cr[5] = p.row_stats[trow * kRowStatWidth + kZy];   // pass 1's z + Markov at the label
    }
  }

  f32x16_t acc[4][4];
  for (int vt = vt_begin; vt < vt_end; ++vt) {
    const int64_t v0 = (int64_t)vt * BM;
    zero_acc(acc);
    // the epilogue's first two stream steps load during the last K segment's final stages
    int tid_o = tid;
    asm volatile("" : "+v"(tid_o));
    StreamTail<MODE, TT, FLAGS> tail{lds, t0, v0, p.r == 0, tid_o};
    int KT = (int)(p.d / BK);
    bool pre;
    if (MODE == MODE_STORE && p.hrows) {   // B = hidden[hrows[t-tile]]
      const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
      DmaTile<256> ta, tb;
      ta.init(p.ldw * 2, v0, p.v, wv);
      tb.init_gather(p.ldh * 2, reinterpret_cast<const __attribute__((address_space(3))) int*>(lds + kHrowOff), wv);
      pre = gemm_nt_tiles(acc, ta, reinterpret_cast<const char*>(p.weight + v0 * p.ldw), tb,
                          reinterpret_cast<const char*>(p.hidden), KT, lds, tail);
    } else {
      pre = gemm_nt(acc, p.weight, p.ldw, v0, p.v, p.hidden, p.ldh, t0, p.n, p.d, lds, tail);
    }
    if (p.r > 0) {   // Markov K segment: W2[v-tile] . W1[prev[t-tile]]^T
      const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
      DmaTile<256> ta, tb;
      ta.init(p.ldw2 * 2, v0, p.v, wv);
      tb.init_gather(p.ldw1 * 2, reinterpret_cast<const __attribute__((address_space(3))) int*>(lds + kPrevOff), wv);
      tail.on = true;
      KT = (int)(p.r / BK);
      pre = gemm_nt_tiles(acc, ta, reinterpret_cast<const char*>(p.w2 + v0 * p.ldw2), tb,
                          reinterpret_cast<const char*>(p.w1), KT, lds, tail);
    }
    if (v0 + BM > p.v)
      epilogue_tile<MODE, TT, FLAGS, false, false>(p, lds, acc, tail, KT, pre);
    else if (StreamTail<MODE, TT, FLAGS>::direct(tail.bases()))
      epilogue_tile<MODE, TT, FLAGS, true, true>(p, lds, acc, tail, KT, pre);
    else
      epilogue_tile<MODE, TT, FLAGS, true, false>(p, lds, acc, tail, KT, pre);
  }

  if (MODE == MODE_STORE && !(FLAGS & kStoreLse)) return;
  // this split's partial of every token: the two vocab halves' states merged (complete:
  // the last epilogue ended with a barrier)
  const int64_t t = t0 + tid;
  if (t < p.n) {
    const lds_f32* s0 = reinterpret_cast<const lds_f32*>(lds + kStateOff) + tid * 8;
    const lds_f32* s1 = s0 + 256 * 8;
    if (MODE == MODE_STATS && !(FLAGS & kTeacherLse)) {
      const PairState m2 = pair_merge(PairState{s0[0], s0[1], s0[2], s0[3], s0[4]},
                                      PairState{s1[0], s1[1], s1[2], s1[3], s1[4]});
      RowPart rp;
      rp.mz = m2.mz; rp.sz = m2.sz; rp.mu = m2.mu; rp.su = m2.su; rp.A = m2.A;
      rp.pad0 = rp.pad1 = rp.pad2 = 0.f;
      p.part1[t * p.splits + split] = rp;
    } else if (MODE == MODE_STATS || MODE == MODE_STORE) {
      // pass 1 with the teacher's log-normaliser given and the stored values' partials
      // carry (mz, sz) only
      const LseState m2 = lse_merge(LseState{s0[0], s0[1]}, LseState{s1[0], s1[1]});
      RowPart rp;
      rp.mz = m2.m; rp.sz = m2.s;
      rp.mu = kNegBig; rp.su = 0.f; rp.A = 0.f;
      rp.pad0 = rp.pad1 = rp.pad2 = 0.f;
      p.part1[t * p.splits + split] = rp;
    } else {
      p.parta[t * p.splits + split] = s0[0] + s1[0];
      if (FLAGS & kTeacherLse) p.partk[t * p.splits + split] = s0[1] + s1[1];
    }
  }
}

// ------------------------------------------------------------------ dh = dl . W kernel

struct BwdParams {
  const uint16_t* dl;      // [N, V] bf16
  const uint16_t* weight;  // [V, d] bf16
  int64_t ldd, ldw;
  int64_t n, v, d;
  int mt, ct, ksplit;      // token tiles, d tiles, K splits
  int xa, xb;              // XCD block: xa token tiles x xb d tiles per round (0 = unblocked)
  int kt_total;            // ceil(V / BK)
  int grid_main;           // mt * ct * ksplit workgroups of dh tiles (padded to whole rounds)
  float* part;             // [ksplit][N][d] fp32
  // Markov extension (r > 0): workgroups past grid_main take mt x ct2 column tiles of
  // w2 [V, r] with their own K split count ksplit2, into part2 [ksplit2][N][r]
  // (d(previous) = dl . w2)
  const uint16_t* w2;
  int64_t ldw2, r;
  int ct2, ksplit2;
  float* part2;
  int wg0;                 // workgroup id of this launch's first workgroup (launches by round)
};

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void dh_kernel(BwdParams p) {
  // the GEMM's LDS ring: one array per buffer (see gemm_nn_ring)
  __shared__ __attribute__((aligned(16))) char ring0[kRingBuf];
  __shared__ __attribute__((aligned(16))) char ring1[kRingBuf];
  __shared__ __attribute__((aligned(16))) char ring2[kRingBuf];
  __shared__ __attribute__((aligned(16))) char ring3[kRingBuf];
  auto ring = [&](int b) -> lds_t* {
    return b == 0 ? (lds_t*)ring0 : b == 1 ? (lds_t*)ring1 : b == 2 ? (lds_t*)ring2 : (lds_t*)ring3;
  };
  // Tile order.  Workgroups go round-robin to the 8 XCDs and run in rounds of
  // C = xa * xb per XCD (one per CU).  With xa > 0 each round of one XCD is a block of
  // xa token tiles x xb d tiles of one K split, so a K stage reads xa + xb distinct
  // operand tiles through that XCD's L2; blocks are numbered token group fastest, then
  // d group, then K split.  xa = 0: consecutive ids per XCD, token tile fastest.
  const int G = p.grid_main;
  const int g = p.wg0 + (int)blockIdx.x;
  int mt, ct, ks, nsplit = p.ksplit;
  const bool mk = g >= G;   // a Markov column tile (after every dh tile)
  if (mk) {
    const int q = g - G;
    mt = q % p.mt;
    ct = (q / p.mt) % p.ct2;
    ks = q / (p.mt * p.ct2);
    nsplit = p.ksplit2;
  } else if (p.xa > 0) {
    const int C = p.xa * p.xb;
    const int i = g / kNumXcd;
    const int blk = (i / C) * kNumXcd + g % kNumXcd, r = i % C;
    const int gm = p.mt / p.xa, gc = p.ct / p.xb;
    mt = (blk % gm) * p.xa + r % p.xa;
    ct = ((blk / gm) % gc) * p.xb + r / p.xa;
    ks = blk / (gm * gc);
    if (ks >= nsplit) return;   // a block past the last (the grid is padded to whole rounds)
  } else {
    int L = g;
    if (G % kNumXcd == 0) L = (L % kNumXcd) * (G / kNumXcd) + L / kNumXcd;
    mt = L % p.mt;
    const int rest = L / p.mt;
    ct = rest % p.ct;
    ks = rest / p.ct;
  }
  const int kt0 = (int)((int64_t)ks * p.kt_total / nsplit);
  const int kt1 = (int)((int64_t)(ks + 1) * p.kt_total / nsplit);
  // the column tile reads W_lm, or w2 for the Markov extension tiles
  const uint16_t* B = mk ? p.w2 : p.weight;
  const int64_t ldb = mk ? p.ldw2 : p.ldw;
  const int64_t cols = mk ? p.r : p.d;
  const int64_t m0 = (int64_t)mt * BM, c0 = (int64_t)ct * BN;
  f32x16_t acc[4][4];
  zero_acc(acc);
  // this split's K range [kt0 BK, min(kt1 BK, V)): full 32-K stages straight into LDS, a
  // partial last one (V % 32 != 0) through registers with entries past V zeroed
  const int64_t kb = (int64_t)kt0 * BK, ke = (int64_t)kt1 * BK < p.v ? (int64_t)kt1 * BK : p.v;
  const int S = (int)((ke - kb) / BK2), kv = (int)(ke - kb - (int64_t)S * BK2);
  gemm_nn_ring(acc, p.dl, p.ldd, m0, p.n, B, ldb, c0, cols, kb, S, kv, ring);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5;
  float* out = (mk ? p.part2 : p.part) + (int64_t)ks * p.n * cols;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = c0 + wn * 128 + j * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * 128 + i * 32 + (e >> 2) * 8 + h * 4 + (e & 3);
        if (row < p.n && col < cols) out[row * cols + col] = acc[i][j][e];
      }
    }
}

// fp32 sum of split partials [ksplit][N][d] into fp32 out [N][d] (row stride ldo), fixed order.
__global__ __launch_bounds__(256) void sum_partials_kernel(const float* __restrict__ part, int ksplit, int64_t n,
                                                           int64_t d, float* __restrict__ out, int64_t ldo) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t total = n * d;
  if (idx >= total) return;
  const int64_t row = idx / d, col = idx % d;
  float4 s = *reinterpret_cast<const float4*>(part + idx);
  for (int k = 1; k < ksplit; ++k) {
    const float4 x = *reinterpret_cast<const float4*>(part + (int64_t)k * total + idx);
    s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
  }
  *reinterpret_cast<float4*>(out + row * ldo + col) = s;
}

__global__ __launch_bounds__(256) void dh_reduce_kernel(const float* __restrict__ part, int ksplit, int64_t n,
                                                        int64_t d, uint16_t* __restrict__ dh, int64_t lddh) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t total = n * d;
  if (idx >= total) return;
  const int64_t row = idx / d, col = idx % d;
  float4 s = *reinterpret_cast<const float4*>(part + idx);
  for (int k = 1; k < ksplit; ++k) {
    const float4 x = *reinterpret_cast<const float4*>(part + (int64_t)k * total + idx);
    s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
  }
  uint2 o;
  o.x = pack_bf16x2(s.x, s.y);
  o.y = pack_bf16x2(s.z, s.w);
  *reinterpret_cast<uint2*>(dh + row * lddh + col) = o;
}

// CUs of the current device (cached per device id below 64; 256 when the query fails, as
// on a host without a GPU, where only workspace sizes are asked for)
int device_cus() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev >= 0 && dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev >= 0 && dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

struct HeadPlan {
  int tt, vt, splits, grid;
  int xa, xb;  // XCD round block (wg_coords): token tiles x splits, 0 = unblocked
};


HeadPlan head_plan(int64_t n, int64_t v) {
  HeadPlan pl;
  pl.tt = (int)((n + BN - 1) / BN);
  pl.vt = (int)((v + BM - 1) / BM);
  // both operands stage 256 rows x 64 bf16 per K step, so the block only counts tiles
  const SplitPlan sp = split_plan(pl.tt, pl.vt, device_cus());
  pl.splits = sp.splits;
  pl.grid = pl.tt * sp.splits;
  pl.xa = sp.xa;
  pl.xb = sp.xb;
  return pl;
}

struct HeadWs {
  RowPart* part1;
  float* parta;
  float* zy;
  float* partk;   // pass-2 KL partials (teacher log-normaliser given)
};

size_t head_ws_layout(int64_t n, int64_t v, void* base, HeadWs* out) {
  const HeadPlan pl = head_plan(n, v);
  const size_t b1 = align_up((size_t)n * pl.splits * sizeof(RowPart), 256);
  const size_t b2 = align_up((size_t)n * pl.splits * sizeof(float), 256);
  const size_t b3 = align_up((size_t)n * sizeof(float), 256);
  if (out) {
    char* c = static_cast<char*>(base);
    out->part1 = reinterpret_cast<RowPart*>(c);
    out->parta = reinterpret_cast<float*>(c + b1);
    out->zy = reinterpret_cast<float*>(c + b1 + b2);
    out->partk = reinterpret_cast<float*>(c + b1 + b2 + b3);
  }
  return b1 + b2 + b3 + b2;
}

struct BwdPlan {
  int mt, ct, ksplit, kt_total, grid_main, grid;
  int ct2, ksplit2;  // Markov column tiles (r > 0) and their K splits
  int xa, xb;        // XCD block (dh_kernel's tile order), 0 = unblocked
};

BwdPlan bwd_plan(int64_t n, int64_t v, int64_t d, int64_t r = 0) {
  BwdPlan pl;
  pl.mt = (int)((n + BM - 1) / BM);
  pl.ct = (int)((d + BN - 1) / BN);
  pl.ct2 = (int)((r + BN - 1) / BN);
  pl.kt_total = (int)((v + BK - 1) / BK);
  const int tiles = pl.mt * pl.ct;
  const int cus = device_cus();
  int ks = tiles > 0 ? (4 * cus + tiles - 1) / tiles : 1;   // no tiles: nothing launches
  if (ks < 1) ks = 1;
  if (ks > 16) ks = 16;
  if (ks > pl.kt_total) ks = pl.kt_total;
  pl.ksplit = ks;
  pl.grid_main = tiles * ks;
  // Markov tiles run after the dh tiles as one extra round: enough K splits to give
  // every CU one (each then covers a fraction of V), at least the dh count
  pl.ksplit2 = 0;
  pl.grid = pl.grid_main;
  if (pl.ct2 > 0) {
    const int tiles2 = pl.mt * pl.ct2;
    int ks2 = tiles2 > 0 ? (cus + tiles2 - 1) / tiles2 : 1;
    if (ks2 < ks) ks2 = ks;
    if (ks2 > 64) ks2 = 64;
    if (ks2 > pl.kt_total) ks2 = pl.kt_total;
    pl.ksplit2 = ks2;
    pl.grid += tiles2 * ks2;
  }
  // XCD block (dh_kernel's tile order): xa * xb = CUs per XCD, xa | mt, xb | ct, whole
  // rounds on every XCD; the smallest xa + xb.  Failing whole rounds, the grid of blocks is
  // padded to them (the workgroups past the last block return at once) when that adds at most
  // an eighth: blocked, a K stage reads xa + xb operand tiles through an XCD's L2, against up to
  // C unblocked.
  pl.xa = pl.xb = 0;
  if (cus % kNumXcd == 0) {
    const int C = cus / kNumXcd;
    int pad_main = 0;
    for (int pass = 0; pass < 2 && pl.xa == 0; ++pass) {
      for (int a = 1; a <= C; ++a) {
        const int b = C / a;
        if (C % a || pl.mt % a || pl.ct % b) continue;
        int g_main = pl.grid_main;
        if (g_main % (kNumXcd * C)) {
          if (pass == 0) continue;
          const int64_t blocks = (int64_t)(pl.mt / a) * (pl.ct / b) * pl.ksplit;
          g_main = (int)((blocks + kNumXcd - 1) / kNumXcd * kNumXcd * C);
          if ((int64_t)g_main * 8 > (int64_t)pl.grid_main * 9) continue;
        }
        if (pl.xa == 0 || a + b < pl.xa + pl.xb || (a + b == pl.xa + pl.xb && g_main < pad_main)) {
          pl.xa = a;
          pl.xb = b;
          pad_main = g_main;
        }
      }
    }
    if (pl.xa > 0 && pad_main != pl.grid_main) {
      pl.grid += pad_main - pl.grid_main;
      pl.grid_main = pad_main;
    }
  }
  return pl;
}

// The dynamic-LDS limit of one head instantiation, raised once per device.
template <int MODE, typename TT, int FLAGS = 0>
hipError_t head_lds_attr() {
  static std::atomic<uint64_t> attr_done{0};
  return ensure_dynamic_lds(reinterpret_cast<const void*>(&head_kernel<MODE, TT, FLAGS>), kHeadLdsBytes, attr_done);
}

template <int MODE, typename TT, int FLAGS = 0>
hipError_t launch_head(const HeadParams& p, int grid, hipStream_t st, const char* name) {
  if (const hipError_t e = head_lds_attr<MODE, TT, FLAGS>()) return e;
  NS_TIMED(name, st);
  // Past five rounds of XCD blocks each round is its own launch, as for the dh GEMM: the
  // rounds start together instead of drifting apart (nine rounds, the compact pass 2 of 18,326
  // rows: 40.6 against 41.8 ms; four, C3: unchanged).
  const int cus = device_cus();
  if (p.xa > 0 && grid % cus == 0 && grid / cus > 5) {
    HeadParams q = p;
    q.wg_total = grid;
    for (int r0 = 0; r0 < grid; r0 += cus) {
      q.wg0 = r0;
      hipLaunchKernelGGL((head_kernel<MODE, TT, FLAGS>), dim3(cus), dim3(kThreads), kHeadLdsBytes, st, q);
    }
    return hipGetLastError();
  }
  hipLaunchKernelGGL((head_kernel<MODE, TT, FLAGS>), dim3(grid), dim3(kThreads), kHeadLdsBytes, st, p);
  return hipGetLastError();
}

template <typename TT, int FLAGS>
hipError_t head_forward_typed(HeadParams& p, const HeadPlan& pl, const SlotArgs& a, float* row_stats,
                              float* metrics, const HeadWs& w, hipStream_t st, int parts) {
  hipError_t e;
  if (parts & kHeadStats) {
    if ((e = launch_head<MODE_STATS, TT, FLAGS>(p, pl.grid, st, "head_stats")) != hipSuccess) return e;
    const TeacherSpec tl{p.trows, p.nt, p.tlse};
    if ((e = launch_merge(w.part1, w.zy, p.v, pl.splits, a, row_stats, st, p.tlse ? &tl : nullptr)) != hipSuccess)
      return e;
  }
  if (!(parts & kHeadEmit)) return hipSuccess;
  p.row_stats = row_stats;
  if ((e = launch_head<MODE_EMIT, TT, FLAGS>(p, pl.grid, st, "head_emit")) != hipSuccess) return e;
  return launch_finalize(w.parta, pl.splits, a, row_stats, metrics, st, p.tlse ? w.partk : nullptr);
}

}  // namespace

hipError_t lmhead_forward_prepare() {
  hipError_t e;
  if ((e = head_lds_attr<MODE_STATS, uint16_t, 0>()) || (e = head_lds_attr<MODE_EMIT, uint16_t, 0>()) ||
      (e = head_lds_attr<MODE_STATS, float, 0>()) || (e = head_lds_attr<MODE_EMIT, float, 0>()) ||
      (e = head_lds_attr<MODE_STATS, uint16_t, kTeacherLse>()) || (e = head_lds_attr<MODE_EMIT, uint16_t, kTeacherLse>()) ||
      (e = head_lds_attr<MODE_STATS, float, kTeacherLse>()) || (e = head_lds_attr<MODE_EMIT, float, kTeacherLse>()))
    return e;
  return hipSuccess;
}

size_t lmhead_workspace_bytes(int64_t n, int64_t v, int64_t d) {
  (void)d;
  return head_ws_layout(n, v, nullptr, nullptr);
}

namespace {

// The fused head's kernel arguments, shared by the forward and the dl re-emission.
HeadParams head_params(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                       int64_t ldm, const MarkovFactors* factors, const void* teacher, int64_t ldt, int64_t d,
                       int64_t v, const SlotArgs& a, const TeacherSpec* ts, void* dl, int64_t ldd,
                       const HeadPlan& pl, const HeadWs& w) {
  HeadParams p = {};
  p.hidden = static_cast<const uint16_t*>(hidden);
  p.weight = static_cast<const uint16_t*>(weight);
  p.markov = static_cast<const uint16_t*>(markov);
  p.teacher = teacher;
  p.ldh = ldh; p.ldw = ldw; p.ldm = ldm; p.ldt = ldt;
  p.n = a.n; p.d = d; p.v = v;
  p.tt = pl.tt; p.vt = pl.vt; p.splits = pl.splits; p.xa = pl.xa; p.xb = pl.xb;
  p.labels = a.labels; p.weights = a.weights;
  p.c_ce = a.c_ce; p.c_kl = a.c_kl; p.inv_acc = a.inv_acc;
  p.part1 = w.part1; p.zy = w.zy; p.parta = w.parta; p.partk = w.partk;
  p.dl = static_cast<uint16_t*>(dl); p.ldd = ldd;
  if (ts) {
    p.trows = ts->rows; p.nt = ts->nt; p.tlse = ts->lse;
    // any two gathered rows within 4 GiB of each other (bf16 rows through LDS)
    p.tdirect = ts->rows && ts->nt > 1 && (ts->nt - 1) * ldt * 2 + 512 > (int64_t)0xffffffffLL;
  }
  if (factors) {
    p.prev = factors->prev;
    p.w1 = static_cast<const uint16_t*>(factors->w1);
    p.w2 = static_cast<const uint16_t*>(factors->w2);
    p.ldw1 = factors->ldw1; p.ldw2 = factors->ldw2; p.r = factors->r;
  }
  return p;
}

}  // namespace

hipError_t lmhead_forward(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                          int64_t ldm, const MarkovFactors* factors, const void* teacher, int tdt, int64_t ldt,
                          int64_t d, int64_t v, const SlotArgs& a, const TeacherSpec* ts, void* dl, int64_t ldd,
                          float* row_stats, float* metrics, void* ws, hipStream_t st, int parts) {
  if (a.n == 0) return metrics ? launch_finalize(nullptr, 1, a, row_stats, metrics, st) : hipSuccess;
  const HeadPlan pl = head_plan(a.n, v);
  HeadWs w;
  head_ws_layout(a.n, v, ws, &w);
  HeadParams p = head_params(hidden, ldh, weight, ldw, markov, ldm, factors, teacher, ldt, d, v, a, ts, dl, ldd, pl, w);
  if (p.tlse) {
    if (tdt == kBF16) return head_forward_typed<uint16_t, kTeacherLse>(p, pl, a, row_stats, metrics, w, st, parts);
    return head_forward_typed<float, kTeacherLse>(p, pl, a, row_stats, metrics, w, st, parts);
  }
  if (tdt == kBF16) return head_forward_typed<uint16_t, 0>(p, pl, a, row_stats, metrics, w, st, parts);
  return head_forward_typed<float, 0>(p, pl, a, row_stats, metrics, w, st, parts);
}

hipError_t lmhead_emit_dlogits(const void* hidden, int64_t ldh, const void* weight, int64_t ldw, const void* markov,
                               int64_t ldm, const MarkovFactors* factors, const void* teacher, int tdt, int64_t ldt,
                               int64_t d, int64_t v, const SlotArgs& a, const TeacherSpec* ts,
                               const float* row_stats, void* dl, int64_t ldd, void* ws, hipStream_t st) {
  if (a.n == 0) return hipSuccess;
  const HeadPlan pl = head_plan(a.n, v);
  HeadWs w;
  head_ws_layout(a.n, v, ws, &w);
  HeadParams p = head_params(hidden, ldh, weight, ldw, markov, ldm, factors, teacher, ldt, d, v, a, ts, dl, ldd, pl, w);
  // pass 2 alone: the row log-normalisers come from the forward's row_stats, the accept
  // and KL partials it also forms go to the workspace and are not read
  p.row_stats = row_stats;
  if (p.tlse) {
    if (tdt == kBF16) return launch_head<MODE_EMIT, uint16_t, kTeacherLse>(p, pl.grid, st, "head_emit");
    return launch_head<MODE_EMIT, float, kTeacherLse>(p, pl.grid, st, "head_emit");
  }
  if (tdt == kBF16) return launch_head<MODE_EMIT, uint16_t, 0>(p, pl.grid, st, "head_emit");
  return launch_head<MODE_EMIT, float, 0>(p, pl.grid, st, "head_emit");
}

size_t lmhead_bwd_workspace_bytes(int64_t n, int64_t v, int64_t d, int64_t r, bool norm) {
  const BwdPlan pl = bwd_plan(n, v, d, r);
  return align_up((size_t)pl.ksplit * n * d * sizeof(float), 256) +
         align_up((size_t)pl.ksplit2 * n * r * sizeof(float), 256) + (norm ? norm_bwd_workspace_bytes(n, d) : 0);
}

hipError_t lmhead_backward(const void* dl, int64_t ldd, const void* weight, int64_t ldw, void* dh, int64_t lddh,
                           int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st) {
  return lmhead_backward_ext(dl, ldd, weight, ldw, nullptr, 0, 0, dh, lddh, nullptr, nullptr, n, v, d, ws, st);
}

hipError_t lmhead_backward_ext(const void* dl, int64_t ldd, const void* weight, int64_t ldw, const void* w2,
                               int64_t ldw2, int64_t r, void* dh, int64_t lddh, float* dprev, const NormBwd* norm,
                               int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st) {
  if (n == 0 || d == 0) return hipSuccess;
  const BwdPlan pl = bwd_plan(n, v, d, r);
  BwdParams p = {};
  p.dl = static_cast<const uint16_t*>(dl);
  p.weight = static_cast<const uint16_t*>(weight);
  p.ldd = ldd; p.ldw = ldw; p.n = n; p.v = v; p.d = d;
  p.mt = pl.mt; p.ct = pl.ct; p.ksplit = pl.ksplit; p.kt_total = pl.kt_total;
  p.grid_main = pl.grid_main; p.ct2 = pl.ct2; p.ksplit2 = pl.ksplit2;
  p.xa = pl.xa; p.xb = pl.xb;
  p.part = static_cast<float*>(ws);
  p.w2 = static_cast<const uint16_t*>(w2); p.ldw2 = ldw2; p.r = r;
  const size_t b_part = align_up((size_t)pl.ksplit * n * d * sizeof(float), 256);
  const size_t b_part2 = align_up((size_t)pl.ksplit2 * n * r * sizeof(float), 256);
  p.part2 = reinterpret_cast<float*>(static_cast<char*>(ws) + b_part);
  void* norm_ws = static_cast<char*>(ws) + b_part + b_part2;
  {
    NS_TIMED("dh_gemm", st);   // 128 KB of static LDS (the ring), none dynamic
    // With more than five rounds of dh tiles each round is its own launch, so every round's
    // XCDs start together and read their shared W and dl stages through the Infinity Cache
    // at about the same time; in one launch later rounds drift apart.  Ten rounds (N =
    // 32,768): 60.5 against 61.9 ms; five (N = 4096): unchanged.  The Markov tiles follow
    // as one more launch.
    const int cus = device_cus();
    const int rounds = pl.xa > 0 && pl.grid_main % cus == 0 ? pl.grid_main / cus : 0;
    if (rounds > 5) {
      BwdParams q = p;
      for (int r0 = 0; r0 < pl.grid; r0 += cus) {
        q.wg0 = r0;
        const int g = pl.grid - r0 < cus ? pl.grid - r0 : cus;
        hipLaunchKernelGGL(dh_kernel, dim3(g), dim3(kThreads), 0, st, q);
      }
    } else {
      hipLaunchKernelGGL(dh_kernel, dim3(pl.grid), dim3(kThreads), 0, st, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (norm) {
    hipError_t e = rms_norm_backward_rows(p.part, pl.ksplit, nullptr, 0, *norm, dh, lddh, n, d, norm_ws, st);
    if (e != hipSuccess) return e;
  } else {
    const int64_t quads = (n * d + 3) / 4;
    NS_TIMED("dh_reduce", st);
    hipLaunchKernelGGL(dh_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, p.part, pl.ksplit,
                       n, d, static_cast<uint16_t*>(dh), lddh);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (r > 0) {
    const int64_t quads = (n * r + 3) / 4;
    NS_TIMED("dprev_reduce", st);
    hipLaunchKernelGGL(sum_partials_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, p.part2,
                       pl.ksplit2, n, r, dprev, r);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t lmhead_linear(const void* x, int64_t ldx, const void* weight, int64_t ldw, const void* addend,
                         int64_t lda, void* out, int64_t ldo, int64_t n, int64_t v, int64_t d, hipStream_t st) {
  return lmhead_linear_lse(x, ldx, nullptr, 0, weight, ldw, addend, lda, out, ldo, nullptr, n, v, d, nullptr, st);
}

size_t lmhead_linear_lse_workspace_bytes(int64_t n, int64_t v) {
  const HeadPlan pl = head_plan(n, v);
  return align_up((size_t)n * pl.splits * sizeof(RowPart), 256);
}

hipError_t lmhead_linear_lse(const void* x, int64_t ldx, const int64_t* rows, int64_t nrows, const void* weight,
                             int64_t ldw, const void* addend, int64_t lda, void* out, int64_t ldo, float* lse,
                             int64_t n, int64_t v, int64_t d, void* ws, hipStream_t st) {
  if (n == 0 || v == 0) return hipSuccess;
  const HeadPlan pl = head_plan(n, v);
  HeadParams p = {};
  p.hidden = static_cast<const uint16_t*>(x);
  p.weight = static_cast<const uint16_t*>(weight);
  p.markov = static_cast<const uint16_t*>(addend);
  p.ldh = ldx; p.ldw = ldw; p.ldm = lda;
  p.n = n; p.d = d; p.v = v;
  p.tt = pl.tt; p.vt = pl.vt; p.splits = pl.splits; p.xa = pl.xa; p.xb = pl.xb;
  p.out = static_cast<uint16_t*>(out); p.ldo = ldo;
  p.teacher = nullptr;
  p.hrows = rows; p.nh = nrows;
  if (!lse) return launch_head<MODE_STORE, uint16_t, 0>(p, pl.grid, st, "head_linear");
  p.part1 = static_cast<RowPart*>(ws);
  hipError_t e = launch_head<MODE_STORE, uint16_t, kStoreLse>(p, pl.grid, st, "head_linear_lse");
  if (e != hipSuccess) return e;
  return launch_lse_merge(p.part1, pl.splits, n, lse, st);
}

}  // namespace ns
