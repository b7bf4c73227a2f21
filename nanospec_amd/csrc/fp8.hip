// FP8 teacher head: logits = bf16( dequant(x) . dequant(W)^T ) with the numerics of
// nanospec/ops.py:183-200 (fp8_linear):
//   activations: per 1x128 block, xs = amax / 448, q = e4m3(clamp(x / max(xs, tiny), +-448))
//   weights:     e4m3 codes with one fp32 scale per 128 x 128 block (scale multiplies)
//   product:     sum over 128-wide K blocks of xs[t, kb] * s[v/128, kb] * (q_x . q_w)_kb,
//                accumulated in fp32 and rounded once to bf16.
// The block dot products run on gfx950's fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4 with
// unit e8m0 scales): e4m3 x e4m3 products are exact in fp32, so only the fp32
// accumulation order differs from the reference's dequantise-then-fp32-GEMM.
#include <type_traits>

#include "ns_gemm.h"
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kQBlock = 128;     // quantisation block (K) and weight-scale block (rows, K)

// float in [-448, 448] or NaN -> OCP e4m3 (fn) code, round to nearest even; -0 keeps its
// sign; NaN gives the NaN code 0x7F (the sign of a NaN carries nothing).
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  if (x != x) return 0x7Fu;
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

// torch's clamp keeps a NaN (fminf / fmaxf would replace it by the bound)
__device__ __forceinline__ float clamp448(float q) { return q != q ? q : fminf(fmaxf(q, -448.0f), 448.0f); }

// One wave per (row, 128-block): lane l owns elements 2l, 2l+1.  Non-finite inputs follow
// the reference's tensor ops: a NaN makes the block's amax, so its scale and every code,
// NaN; an infinity makes the scale inf, the finite entries' codes +-0 and its own code NaN
// (inf / inf).  Either way the block dequantises to NaN and so do the row's logits.
// Scale of (row, block kb) at xs[row * xs_row + kb * xs_blk]: [N, d/128] for callers,
// [d/128, N] (contiguous over rows within a block) for the fp8 head.
__global__ __launch_bounds__(256) void fp8_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t n,
                                                        int64_t d, uint8_t* __restrict__ q,
                                                        float* __restrict__ xs, int64_t xs_row, int64_t xs_blk) {
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
  // abs().amax() propagates a NaN, which fmaxf drops
  if (__any((x0 != x0) || (x1 != x1))) amax = __builtin_nanf("");
  const float s = __fdiv_rn(amax, 448.0f);
  // clamp_min(torch.finfo(float32).tiny), keeping a NaN scale
  const float den = s != s ? s : fmaxf(s, 1.17549435e-38f);
  const float q0 = clamp448(__fdiv_rn(x0, den));
  const float q1 = clamp448(__fdiv_rn(x1, den));
  const uint16_t codes = (uint16_t)(e4m3_code(q0) | (e4m3_code(q1) << 8));
  *reinterpret_cast<uint16_t*>(q + row * d + kb * kQBlock + 2 * lane) = codes;
  if (lane == 0) xs[row * xs_row + kb * xs_blk] = s;
}

struct Fp8Params {
  const uint8_t* qx;       // [N, d] e4m3 codes (row stride d)
  const float* xs;         // [d/128, N]: each 128-K block's scales, contiguous over tokens
  const uint8_t* wq;       // [V, d] e4m3 codes
  const float* ws;         // [V/128, d/128]
  int64_t ldw;
  uint16_t* out;           // [N, V] bf16
  int64_t ldo;
  int64_t n, v, d;
  int tt, vt, splits;      // token tiles, vocab tiles, vocab splits
  int xa, xb;              // XCD round block (wg_coords), 0 = unblocked
  RowPart* part;           // [N][splits] (max, sum-exp) of the stored bf16 values, or null
};

// Workgroup tile: 256 vocab rows (two weight-scale row blocks) x 256 tokens on 8 waves, two
// per SIMD, as 2 (vocab) x 4 (tokens), each 128 x 64 = 4 x 2 blocks of 32 x 32 with its
// accumulator in 128 VGPRs.  K advances one 128-entry quantisation block per stage; a stage
// is 32 KB of weight codes plus 32 KB of activation codes, in a 2-deep LDS ring.  Against a
// 256 x 128 tile on 4 waves this moves a third fewer fill bytes per MFMA, and a wave that
// stalls on a fill or on its fold leaves the SIMD's matrix core to the other wave.
constexpr int FM = 256;
constexpr int FN = 256;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kAStage = FM * kQBlock;        // 32 KB of weight codes
constexpr int kBStage = FN * kQBlock;        // 32 KB of activation codes
constexpr int kStage = kAStage + kBStage;
constexpr int kRing = 2;
constexpr int kRingLds = kRing * kStage;     // 128 KB
constexpr int kOutRow = FM * 2 + 16;         // bf16 output row in the LDS transpose (+16 B)
constexpr int kOutTokens = 128;              // tokens per output pass (two passes per tile)
constexpr int kOutOff = kStage;              // the transpose: ring buffer 1 and 3.5 KB past it
constexpr int kLseOff = kOutOff + kOutTokens * kOutRow;   // [FN][2] fp32 running (max, sum-exp)
constexpr int kFp8Lds = kLseOff + FN * 8;
static_assert(kOutOff + kOutTokens * kOutRow <= kLseOff && kLseOff % 16 == 0, "LDS layout");
static_assert(kFp8Lds <= 160 * 1024, "fp8 head LDS");

// s_waitcnt vmcnt(0) lgkmcnt(0) (expcnt not waited): gfx9 encoding, vmcnt[3:0] in bits
// 3:0, expcnt in 6:4, lgkmcnt in 11:8, vmcnt[5:4] in 15:14.
constexpr int kWaitAll = 0 | (7 << 4);
// vmcnt(4): everything but the last 4 vector-memory operations (stage 1's A fills)
constexpr int kWaitPrologue = 4 | (7 << 4) | (15 << 8);

__device__ __forceinline__ u32x4_t rd16(const lds_t* base, int row, int chunk) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(base + lds_off(row, chunk));
}

// One lane's 32-byte fp8 MFMA operand: logical chunks c0 and c0 + 1 of `row` (c0 even),
// read straight into the two halves of one 8-register vector.
__device__ __forceinline__ i32x8_t rd32(const lds_t* base, int row, int c0) {
  const u32x4_t lo = rd16(base, row, c0), hi = rd16(base, row, c0 + 1);
  return __builtin_bit_cast(i32x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// One fp8 MFMA block product: 32 x 32 outputs over 64 K-entries.  Operand lane layout:
// lane r + 32 kh holds row r, K entries 32 kh .. 32 kh + 31 of the 64 (two 16-byte
// chunks); unit e8m0 scales (127).
__device__ __forceinline__ f32x16_t mfma_f8(const i32x8_t& a, const i32x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// Reductions over the 16 lanes of a DPP row with every lane receiving the result:
// xor 1, xor 2, then the half-row and row mirrors, which pair the 4- and 8-lane groups
// once their values agree (so all 16 lanes end with the same bits).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));
  x = fmaxf(x, dpp_mov<0x4E>(x));
  x = fmaxf(x, dpp_mov<0x141>(x));
  return fmaxf(x, dpp_mov<0x140>(x));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x141>(x);
  return x + dpp_mov<0x140>(x);
}

// acc[e0 .. e0 + 8) += c * part[e0 .. e0 + 8).  The empty asm statements pin each sum where
// it is formed: the optimiser otherwise sinks these FMAs to the end of the stage, which
// keeps every 32 x 32 block's partial alive at once.
__device__ __forceinline__ void fold8(f32x16_t& acc, const f32x16_t& part, float c, int e0) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = __builtin_fmaf(c, part[e0 + e], acc[e0 + e]);
    asm volatile("" : "+v"(x));
    acc[e0 + e] = x;
  }
}

template <int WAITCNT>
__device__ __forceinline__ void wait_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(WAITCNT);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The lane's index in its wave, formed where it is used (mbcnt over an opaque zero) rather
// than kept from the thread-id register, which the stage loop would otherwise spill.
__device__ __forceinline__ int lane_here() {
  uint32_t z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, z));
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fp8_head_kernel(Fp8Params p) {
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_t* lds = (lds_t*)lds_raw;
  int tile_t, split;
  wg_coords(blockIdx.x, gridDim.x, p.tt, p.xa, p.xb, tile_t, split);
  const int vt_begin = (int)((int64_t)split * p.vt / p.splits);
  const int vt_end = (int)((int64_t)(split + 1) * p.vt / p.splits);
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv >> 2, wn = wv & 3;
  const int lane = tid & 63, r = lane & 31, kh = lane >> 5;
  // Waves w and w + 4 share a SIMD.  With one of them ahead whenever both are ready, their
  // fragment waits and folds fall at different times and the matrix core takes the other's
  // MFMA (with the barrier move below, 1-1.5% at C4).
  if (wm == 0) __builtin_amdgcn_s_setprio(1);
  const int KB = (int)(p.d / kQBlock);
  const int64_t t0 = (int64_t)tile_t * FN;
  const int nvb = (int)(p.v / kQBlock);
  auto buf = [&](int t) -> lds_t* { return lds + (t & 1) * kStage; };

  DmaTile<FN, kWaves> tb;
  tb.init(p.d, t0, p.n, wv);
  const char* pb = reinterpret_cast<const char*>(p.qx + t0 * p.d);
  // this lane's two tokens (rows past N re-read the last); a block's scales are
  // contiguous over tokens, so the 32 tokens of a load share one 128-byte line (from the
  // callers' [N, d/128] layout a load touched 32 lines, which the fills evict from the
  // L1: about 390 extra L2 requests per CU per stage, 7% of the kernel's time at C4)
  uint32_t xsoff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t t = t0 + wn * 64 + j * 32 + r;
    xsoff[j] = (uint32_t)(t < p.n ? t : p.n - 1);
  }
  lds_f32* lse_st = reinterpret_cast<lds_f32*>(lds + kLseOff);
  if (p.part && tid < FN) {   // first read after the first tile's barriers
    lse_st[2 * tid] = kNegBig;
    lse_st[2 * tid + 1] = 0.f;
  }

  auto a_src = [&](int vt) -> const char* { return reinterpret_cast<const char*>(p.wq + (int64_t)vt * FM * p.ldw); };
  auto ws_row = [&](int vt) -> const float* {   // this wave's weight-scale row block of tile vt
    int vb = vt * (FM / kQBlock) + wm;
    vb = vb < nvb ? vb : nvb - 1;                // a tile half past V: rows discarded
    return p.ws + (int64_t)vb * KB;
  };
  DmaTile<FM, kWaves> ta;
  bool staged = false;   // this tile's first stage in buffer 0, its fragments in a / b and its
                         // block scales in c_cur (set up by the previous tile)
  float c_cur[2], c_prev[2], xn[2], wnx;
  i32x8_t a[2];            // [kk]: block row q's A fragments, reloaded after their last use
  i32x8_t b[2][2];         // [j][kk]
  f32x16_t part[2];        // [j]: the pair of MFMAs of one 32 x 32 block over 128 K
  for (int vt = vt_begin; vt < vt_end; ++vt) {
    const int64_t v0 = (int64_t)vt * FM;
    const char* pa = a_src(vt);
    const float* wsrow = ws_row(vt);
    // With an even number of stages the tile's last one sits in buffer 1, and the next tile's
    // first stage fills buffer 0 during this tile's last two stages (its weight codes in
    // slots 12-15 of stage KB - 2, its activation codes in slots 0-3 of stage KB - 1) while the
    // epilogue transposes through buffer 1; otherwise each tile starts with its own fills.
    // Waiting at each tile's start for its first fills took 11.8K cycles of a 143K-cycle tile.
    const bool pf = vt + 1 < vt_end && (KB & 1) == 0;
    const char* pan = a_src(vt + 1);
    const float* wsn = ws_row(vt + 1);

    f32x16_t acc[4][2];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[q][j][e] = 0.f;

    // the blocks carried into the first stage's folds start at zero (they add nothing)
    c_prev[0] = c_prev[1] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) part[j][e] = 0.f;
    auto read_frags = [&]() {
      const int fl = lane_here(), fr = fl & 31, fkh = fl >> 5;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) b[j][kk] = rd32(buf(0) + kAStage, wn * 64 + j * 32 + fr, kk * 4 + fkh * 2);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) a[kk] = rd32(buf(0), wm * 128 + fr, kk * 4 + fkh * 2);
    };
    if (!staged) {
      // prologue: stage 0's scales, then the fills of stage 0 and stage 1's A fills (its B
      // fills go out in stage 0); wait for stage 0 only (vector-memory operations complete
      // in order)
      ta.init(p.ldw, v0, p.v, wv, lane_here());
      {
        const float w0 = wsrow[0];
        c_cur[0] = p.xs[xsoff[0]] * w0;
        c_cur[1] = p.xs[xsoff[1]] * w0;
      }
      const int64_t k1 = KB > 1 ? kQBlock : 0;
#pragma unroll
      for (int i = 0; i < DmaTile<FM, kWaves>::NI; ++i) ta.issue(pa, buf(0), wv, i);
#pragma unroll
      for (int i = 0; i < DmaTile<FN, kWaves>::NI; ++i) tb.issue(pb, buf(0) + kAStage, wv, i);
#pragma unroll
      for (int i = 0; i < DmaTile<FM, kWaves>::NI; ++i) ta.issue(pa + k1, buf(1), wv, i);
      static_assert(DmaTile<FM, kWaves>::NI == 4 && DmaTile<FN, kWaves>::NI == 4, "fill slots");
      wait_barrier<kWaitPrologue>();
      read_frags();
    }

    for (int t = 0; t < KB; ++t) {
      const lds_t* cb = buf(t);
      const lds_t* nb = buf(t + 1);
      lds_t* db = buf(t);              // stage t + 2 lands where stage t was
      const int64_t k2 = (int64_t)(t + 2) * kQBlock;
      const bool more = t + 1 < KB, fill2 = t + 2 < KB;
      const int kn = more ? t + 1 : 0;              // the next stage: this tile's or the next tile's first
      const float* wsk = more ? wsrow : wsn;
      const bool fill_next = pf && t == KB - 2;     // slots 12-15 fill the next tile's first stage
      if (fill_next) ta.init(p.ldw, v0 + FM, p.v, wv, lane_here());
      // 16 MFMA slots s = 4 q + 2 j + kk; the pair (q, j) accumulates over the stage's two
      // 64-K halves into part[j], which is folded into the accumulator with the block
      // scale in slot (q + 1, j, 0), before the next pair overwrites it (sched_barrier
      // keeps the order)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const int s = 4 * q + 2 * j + kk;
            // block (q - 1, j) (the previous stage's (3, j) when q = 0) is folded with its
            // scale just before its partial is overwritten: its last MFMA was issued three
            // slots ago and has completed, so the fold does not wait on the matrix core
            if (kk == 0) {
              if (q > 0)
                fold8(acc[q - 1][j], part[j], c_cur[j], 0), fold8(acc[q - 1][j], part[j], c_cur[j], 8);
              else   // at t = 0 part[j] and c_prev[j] are 0, which adds nothing
                fold8(acc[3][j], part[j], c_prev[j], 0), fold8(acc[3][j], part[j], c_prev[j], 8);
            }
            part[j] = mfma_f8(a[kk], b[j][kk], kk == 0 ? f32x16_t{} : part[j]);
            asm volatile("" : "+v"(part[j]));   // keep the MFMAs in program order
            __builtin_amdgcn_sched_barrier(0);
            if (s == 0) {   // next stage's scales (complete by this stage's barrier)
              const float* xsb = p.xs + (int64_t)kn * p.n;
              xn[0] = xsb[xsoff[0]];
              xn[1] = xsb[xsoff[1]];
              wnx = wsk[kn];
            }
            // stage t + 1's B fills (activation codes), one per slot in slots 0-3 (the last
            // stage re-reads itself into the idle buffer).  That half of buffer t + 1 was last
            // read in slots 12-15 of stage t - 2, before the previous barrier; this stage's
            // barrier waits for them.  Issued with stage t + 2's A fills, eight per wave in
            // slots 12-15, a CU's 64 fills overfilled its L1's miss queue and stalled the
            // waves' issue: 7% slower at C4.
            if (q == 0) tb.issue(pb + (int64_t)kn * kQBlock, buf(t + 1) + kAStage, wv, s);
            // block row q + 1's A fragment kk, after its last use by block (q, 1)
            if (q < 3 && j == 1) a[kk] = rd32(cb, wm * 128 + (q + 1) * 32 + r, kk * 4 + kh * 2);
            // stage t + 1 landed everywhere, every wave done reading stage t.  After slot 12's
            // MFMA rather than before it: block row 3's fragments, read in slots 10-11, have
            // had that MFMA to arrive before the wait for every LDS read (0.5% at C4).
            if (s == 12) {
              wait_barrier<kWaitAll>();
            }
            if (q == 3) {
              const int u = s - 12;   // 0..3
              // stage t + 2's A fills (weight codes) into stage t's buffer, one per slot
              if (fill2) ta.issue(pa + k2, db, wv, u);
              else if (fill_next) ta.issue(pan, db, wv, u);
              // stage t + 1's fragments, each right after its last use in this stage: B (j, kk)
              // in its own slot, A row 0 in the slots of block (3, 1)
              if (more) {
                b[j][kk] = rd32(nb + kAStage, wn * 64 + j * 32 + r, kk * 4 + kh * 2);
                if (j == 1) a[kk] = rd32(nb, wm * 128 + r, kk * 4 + kh * 2);
              }
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      c_prev[0] = c_cur[0];
      c_prev[1] = c_cur[1];
      c_cur[0] = xn[0] * wnx;
      c_cur[1] = xn[1] * wnx;
    }
    // the last stage's blocks (3, 0) and (3, 1)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[3][j][e] = __builtin_fmaf(c_prev[j], part[j][e], acc[3][j][e]);
    // no fill in flight (the next tile's first stage, when prefetched, has landed), every
    // wave done with the ring
    wait_barrier<kWaitAll>();

    // bf16 tile transposed through LDS in two passes of 128 tokens, then whole 16-byte
    // chunks of output rows
    const int etid = wv * 64 + lane_here(), er = etid & 31, ekh = (etid >> 5) & 1;   // == tid
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if ((wn >> 1) == half) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int tl = (wn & 1) * 64 + j * 32 + er;
              const int vl = wm * 128 + q * 32 + 8 * g + 4 * ekh;
              const u32x2_t y = {pack_bf16x2(acc[q][j][4 * g], acc[q][j][4 * g + 1]),
                                 pack_bf16x2(acc[q][j][4 * g + 2], acc[q][j][4 * g + 3])};
              *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(lds + kOutOff + tl * kOutRow + vl * 2) = y;
            }
      }
      __syncthreads();
      // 16 lanes per output row (one DPP row), each taking 16-byte chunks c and c + 16
#pragma unroll 2
      for (int i = 0; i < kOutTokens * (FM / 16) / kThreads; ++i) {
        const int ci = i * kThreads + etid;
        const int row = ci >> 4, c = ci & 15;
        const int tk = half * kOutTokens + row;   // token within the tile
        const int64_t t = t0 + tk;
        float f[2][8];
        bool in[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int chunk = c + 16 * h;
          const int64_t v = v0 + chunk * 8;
          in[h] = t < p.n && v < p.v;
          const u32x4_t x =
              *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(lds + kOutOff + row * kOutRow + chunk * 16);
          if (in[h]) *reinterpret_cast<uint4*>(p.out + t * p.ldo + v) = make_uint4(x[0], x[1], x[2], x[3]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f[h][2 * e] = bf16_lo(x[e]);
            f[h][2 * e + 1] = bf16_hi(x[e]);
          }
        }
        if (p.part) {
          // log-sum-exp of the stored bf16 row over this tile: the row maximum first, then
          // one exponential per entry against it, then the sum
          float m = kNegBig;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (in[h]) {
#pragma unroll
              for (int e = 0; e < 8; ++e) m = fmaxf(m, f[h][e]);
            }
          m = row16_max(m);
          const float ml = m * kLog2e;
          float sum = 0.f;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (in[h]) {
#pragma unroll
              for (int e = 0; e < 8; ++e) sum += fast_exp2(__builtin_fmaf(f[h][e], kLog2e, -ml));
            }
          sum = row16_sum(sum);
          if (c == 0) {
            const LseState r2 = lse_merge(LseState{lse_st[2 * tk], lse_st[2 * tk + 1]}, LseState{m, sum});
            lse_st[2 * tk] = r2.m;
            lse_st[2 * tk + 1] = r2.s;
          }
        }
      }
      __syncthreads();
    }
    staged = pf;
    if (pf) {   // the next tile's first fragments (landed before the epilogue), then its
                // stage-1 weight fills into buffer 1, free again after the epilogue's last barrier
      read_frags();
#pragma unroll
      for (int i = 0; i < DmaTile<FM, kWaves>::NI; ++i) ta.issue(pan + kQBlock, buf(1), wv, i);
    }
  }
  if (p.part && tid < FN && t0 + tid < p.n) {
    RowPart rp;
    rp.mz = lse_st[2 * tid]; rp.sz = lse_st[2 * tid + 1];
    rp.mu = kNegBig; rp.su = 0.f; rp.A = 0.f; rp.pad0 = rp.pad1 = rp.pad2 = 0.f;
    p.part[(t0 + tid) * p.splits + split] = rp;
  }
}

struct Fp8Plan {
  int tt, vt, splits, xa, xb;
};

Fp8Plan fp8_plan(int64_t n, int64_t v) {
  Fp8Plan pl;
  pl.vt = (int)((v + FM - 1) / FM);
  pl.tt = (int)((n + FN - 1) / FN);
  int cus = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  // one stage reads FN x 128 activation codes per token tile and FM x 128 weight codes per
  // split: at N = 4096 this picks 16 splits in blocks of 4 token tiles x 8 splits per XCD
  // (8 x 4, the other block of equal cost, ran the same: 4.694 against 4.695 ms)
  const SplitPlan sp = split_plan(pl.tt, pl.vt, cus, FN, FM);
  pl.splits = sp.splits;
  pl.xa = sp.xa;
  pl.xb = sp.xb;
  return pl;
}

}  // namespace

namespace {

hipError_t launch_quant(const void* x, int64_t ldx, int64_t n, int64_t d, uint8_t* q, float* xs, int64_t xs_row,
                        int64_t xs_blk, hipStream_t st) {
  const int64_t items = n * (d / kQBlock);
  if (items == 0) return hipSuccess;
  NS_TIMED("fp8_quant", st);
  hipLaunchKernelGGL(fp8_quant_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st,
                     static_cast<const uint16_t*>(x), ldx, n, d, q, xs, xs_row, xs_blk);
  return hipGetLastError();
}

}  // namespace

hipError_t fp8_quantize_rows(const void* x, int64_t ldx, int64_t n, int64_t d, uint8_t* q, float* xs,
                             hipStream_t st) {
  return launch_quant(x, ldx, n, d, q, xs, d / kQBlock, 1, st);
}

size_t fp8_workspace_bytes(int64_t n, int64_t v, int64_t d) {
  const size_t part = v > 0 ? align_up((size_t)n * fp8_plan(n, v).splits * sizeof(RowPart), 256) : 0;
  return align_up((size_t)n * d, 256) + align_up((size_t)n * (d / kQBlock) * sizeof(float), 256) + part;
}

hipError_t fp8_teacher_logits(const void* x, int64_t ldx, const uint8_t* wq, int64_t ldw, const float* scale,
                              void* out, int64_t ldo, float* lse, int64_t n, int64_t v, int64_t d, void* ws,
                              hipStream_t st) {
  if (n == 0 || v == 0) return hipSuccess;
  uint8_t* qx = static_cast<uint8_t*>(ws);
  float* xs = reinterpret_cast<float*>(static_cast<char*>(ws) + align_up((size_t)n * d, 256));
  RowPart* part = reinterpret_cast<RowPart*>(static_cast<char*>(ws) + align_up((size_t)n * d, 256) +
                                             align_up((size_t)n * (d / kQBlock) * sizeof(float), 256));
  {
    hipError_t e = launch_quant(x, ldx, n, d, qx, xs, 1, n, st);   // scales [d/128, N] for the head
    if (e != hipSuccess) return e;
  }
  Fp8Params p;
  p.qx = qx; p.xs = xs; p.wq = wq; p.ws = scale; p.ldw = ldw;
  p.out = static_cast<uint16_t*>(out); p.ldo = ldo;
  p.n = n; p.v = v; p.d = d;
  const Fp8Plan pl = fp8_plan(n, v);
  p.vt = pl.vt; p.tt = pl.tt; p.splits = pl.splits; p.xa = pl.xa; p.xb = pl.xb;
  const int sp = pl.splits;
  p.part = lse ? part : nullptr;
  static std::atomic<uint64_t> attr_done{0};
  if (const hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&fp8_head_kernel), kFp8Lds, attr_done))
    return e;
  {
    NS_TIMED("fp8_head_gemm", st);
    hipLaunchKernelGGL(fp8_head_kernel, dim3((unsigned)(p.tt * sp)), dim3(kThreads), kFp8Lds, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !lse) return e;
  }
  return launch_lse_merge(part, sp, n, lse, st);
}

}  // namespace ns
