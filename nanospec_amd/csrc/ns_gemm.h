// Building blocks shared by the MFMA GEMM kernels (lmhead.hip, fp8.hip): the swizzled
// LDS tile layout, direct-to-LDS operand fills, the fill barrier and the XCD-aware
// workgroup -> tile maps.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ns {

typedef __attribute__((address_space(3))) char lds_t;   // LDS byte pointer
typedef __attribute__((address_space(3))) float lds_f32;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kNumXcd = 8;   // MI355X: 8 XCDs, workgroups dispatched round-robin over them

// LDS tiles hold rows of 128 bytes (64 bf16 or 128 fp8 K-entries) as eight 16-byte
// chunks.  Swizzle: chunk c of row r sits at c ^ swz(r); rows r and r + 8 rotate, so 8-
// and 16-lane groups reading one logical chunk of consecutive rows hit distinct banks.
__device__ __forceinline__ int swz(int row) { return ((row & 7) + ((row >> 3) & 1)) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * 128 + ((chunk ^ swz(row)) << 4); }

// One 16-byte-per-lane fill straight into LDS: lane l's 16 bytes at base + voff land in
// slot l of the 1 KB block at dst.  Issued as buffer_load_dwordx4 ... lds (a raw buffer
// over base, offsets < 4 GiB) rather than global_load_lds: the compiler treats a pending
// FLAT-encoded LDS fill as able to complete out of order with LDS reads, so it waits
// for every outstanding LDS read (lgkmcnt(0)) before any fragment use; with the buffer
// form it waits only for the reads a fragment needs.  Same bytes, same LDS layout.
// `soff`: a wave-uniform byte offset added to every lane's (the instruction's scalar offset).
__device__ __forceinline__ void dma16(const char* base, uint32_t voff, lds_t* dst, uint32_t soff = 0) {
  // word 3: 32-bit data format, the raw-buffer setting for gfx9-family descriptors
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, -1, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, reinterpret_cast<__attribute__((address_space(3))) void*>(dst), 16,
                                           voff, soff, 0, 0);
}

// dma16 issued through inline asm.  The compiler then sees no LDS write in flight, so it adds
// no waits for one before LDS reads (with the builtin it waited for every outstanding fill
// before a read it could not prove disjoint); the caller's own vmcnt waits must order each
// fill before the reads of its data.  Same instruction, descriptor and LDS layout as dma16.
// M0 is reserved to the compiler, which does not honour the clobber: a kernel using this
// must not also use dma16 or anything else that sets M0 (the dh GEMM uses only this form).
__device__ __forceinline__ void dma16_asm(const char* base, uint32_t voff, lds_t* dst) {
  typedef uint32_t u32x4s_t __attribute__((ext_vector_type(4)));
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const u32x4s_t rs = {(uint32_t)b, (uint32_t)(b >> 32) & 0xffffu, 0xffffffffu, 0x00020000u};
  const uint32_t m0v = (uint32_t)reinterpret_cast<uintptr_t>(dst);
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "s"(m0v)
               : "memory", "m0");
}

// A ROWS-row operand tile (128-byte rows) fetched straight into LDS (dma16).  Each of the
// WAVES waves issues NI = ROWS / (8 WAVES) instructions per stage; instruction i of wave wv
// fills the 1 KB LDS block wv * NI + i, i.e. rows 8 (wv * NI + i) .. +8.  Lane l writes the
// block's 16-byte slot l, which is physical chunk l % 8 of row 8 (wv * NI + i) + l / 8; the
// lane therefore fetches the logical chunk (l % 8) ^ swz(row), so the tile lands in the
// swizzled lds_off layout.  Rows at or past rmax re-read row rmax - 1 (their results are
// discarded by the caller).
template <int ROWS, int WAVES = 4>
struct DmaTile {
  static constexpr int NI = ROWS / (8 * WAVES);
  static_assert(NI * 8 * WAVES == ROWS, "whole 8-row blocks per wave");
  uint32_t off[NI];  // per-lane byte offsets from the tile's first row, stage 0
  // ld_bytes: row pitch in bytes; r0: first row; rmax: rows in the matrix
  __device__ __forceinline__ void init(int64_t ld_bytes, int64_t r0, int64_t rmax, int wv) {
    init(ld_bytes, r0, rmax, wv, threadIdx.x & 63);
  }
  // the same with the lane's index in its wave given
  __device__ __forceinline__ void init(int64_t ld_bytes, int64_t r0, int64_t rmax, int wv, int lane) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (wv * NI + i) * 8 + (lane >> 3);
      int64_t r = r0 + row;
      r = r < rmax ? r : rmax - 1;
      const int chunk = (lane & 7) ^ swz(row);
      off[i] = (uint32_t)((r - r0) * ld_bytes + chunk * 16);
    }
  }
  // Gathered rows: tile row j is matrix row rows[j] (rows[] in LDS, already in range),
  // offsets from the matrix base.
  __device__ __forceinline__ void init_gather(int64_t ld_bytes, const __attribute__((address_space(3))) int* rows,
                                              int wv) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = (wv * NI + i) * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ swz(row);
      off[i] = (uint32_t)((int64_t)rows[row] * ld_bytes + chunk * 16);
    }
  }
  // instruction i of one stage: `base` = the tile's first row at this stage's K offset,
  // `dst` = the operand's LDS stage buffer (wave-uniform)
  __device__ __forceinline__ void issue(const char* base, lds_t* dst, int wv, int i) const {
    dma16(base, off[i], dst + (wv * NI + i) * 1024);
  }
};

// B operand [K rows, cols] (cols contiguous) fetched straight into a row-major LDS stage
// of ROWS K rows of 512 bytes (ROWS = 8 x fills per wave, four waves), the 16-byte chunk cn
// of row k stored at physical chunk cn ^ (4 (k & 3)), which keeps the transposed fragment
// reads (tr_b16) free of bank conflicts.  Fill i of wave wv writes rows 2 (wv NI + i) + {0,
// 1}; lane l writes physical chunk l % 32 of row 2 (wv NI + i) + l / 32.  Column chunks at or
// past cmax re-read the tile's first chunk (discarded by the caller).
template <int ROWS>
struct DmaTileKNR {
  static constexpr int NI = ROWS / 8;
  static_assert(NI * 8 == ROWS, "two rows per fill, four waves");
  uint32_t off[NI];
  __device__ __forceinline__ void init(int64_t ld, int64_t c0, int64_t cmax, int wv) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = 2 * (wv * NI + i) + (lane >> 5);
      const int cn = (lane & 31) ^ (4 * (row & 3));
      int64_t col = c0 + cn * 8;
      col = col < cmax ? col : c0;
      off[i] = (uint32_t)((row * ld + (col - c0)) * 2);
    }
  }
  __device__ __forceinline__ void issue(const char* base, lds_t* dst, int wv, int i) const {
    dma16(base, off[i], dst + (wv * NI + i) * 1024);
  }
  __device__ __forceinline__ void issue_asm(const char* base, lds_t* dst, int wv, int i) const {
    dma16_asm(base, off[i], dst + (wv * NI + i) * 1024);
  }
};

typedef short i16x4_t __attribute__((ext_vector_type(4)));

// B fragment i (32 columns) of step kk from a DmaTileKNR stage, as two transposed reads:
// ds_read_b64_tr_b16 gives lane 16 g + x of a 16-lane group element x % 4 of the
// 8-byte pieces addressed by lanes 16 g + 4 j + x / 4, j = 0..3.  Lane 16 g + 4 j + m
// addresses row kbase + j, columns nb + 4 m .. +3, so lane 16 g + x receives
// B[kbase + 0..3][nb + x]: K-contiguous, as the MFMA B operand wants.
struct TrFrag {
  i16x4_t lo, hi;  // K 0..3 and 4..7 of this lane's eight
};

__device__ __forceinline__ uint32_t tr_base(int wn, int i) {
  // byte address of this lane's piece for step 0, half 0 (add 2048 for half 1, 8192 per step)
  const int lane = threadIdx.x & 63;
  const int x = lane & 15;
  const int row = 8 * (lane >> 5) + (x >> 2);                       // + 16 kk + 4 half
  const int col = wn * 128 + i * 32 + 16 * ((lane >> 4) & 1) + 4 * (x & 3);
  const int cn = (col >> 3) ^ (4 * (row & 3));
  return (uint32_t)(row * 512 + (cn << 4) + (col & 7) * 2);
}

__device__ __forceinline__ i16x4_t tr_read(const lds_t* buf, uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) i16x4_t*>(const_cast<lds_t*>(buf) + addr));
}

__device__ __forceinline__ bf16x8_t tr_join(const TrFrag& f) {
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(f.lo, f.hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Wait for this wave's LDS fills and all outstanding memory operations, then a
// workgroup barrier.  The empty asm statements keep the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void fill_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait until at most N of this wave's global loads and stores are outstanding and every
// LDS operation is done, then a workgroup barrier (vmcnt N in bits 3:0 and 15:14,
// expcnt 7, lgkmcnt 0).
template <int N>
__device__ __forceinline__ void vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup -> (tile t, split s) map for a grid of TT x S workgroups, one per CU at a
// time.  Workgroups are dispatched round-robin over the 8 XCDs, and the workgroups of
// one XCD share its L2.  With xa > 0 the grid runs in rounds of xa * xb workgroups per
// XCD (one per CU), and each round of an XCD is a block of xa t-tiles x xb splits, so one
// K stage of the round reads xa + xb distinct operand tiles through that L2 (12 for a
// 4 x 8 block, against 18 for 16 x 2).  Block b = round * 8 + XCD walks the
// (TT / xa) x (S / xb) block grid, t-blocks fastest.  Requires G % (8 xa xb) == 0,
// TT % xa == 0 and S % xb == 0 (split_plan).  xa = 0: consecutive ids per XCD, t fastest.
__host__ __device__ inline void wg_coords(int g, int G, int TT, int xa, int xb, int& t, int& s) {
  if (xa > 0) {
    const int C = xa * xb;
    const int x = g % kNumXcd, i = g / kNumXcd;
    const int blk = (i / C) * kNumXcd + x, r = i % C;
    const int gm = TT / xa;
    t = (blk % gm) * xa + r % xa;
    s = (blk / gm) * xb + r / xa;
    return;
  }
  int L = g;
  if (G % kNumXcd == 0) L = (g % kNumXcd) * (G / kNumXcd) + g / kNumXcd;
  s = L / TT;
  t = L % TT;
}

struct SplitPlan {
  int splits;   // S: vocab (or column) ranges, one workgroup each per t-tile
  int xa, xb;   // round block for wg_coords, 0 = unblocked
};

// Splits and XCD block for a TT-tile grid over `vt` splittable tiles (vocab tiles) on
// `cus` CUs, one workgroup per CU at a time.  Candidates are the split counts S up to
// max(64, cus / TT) (and at most vt) whose grid TT * S fills whole rounds of cus
// workgroups.  Each gets the block a x b = cus / 8 with a | TT and b | S minimising the
// distinct operand bytes one L2 serves per K stage, a * t_stage + b * s_stage (t_stage:
// one t-tile's operand stage, shared by the block's splits; s_stage: one split's).  The
// cheapest wins.  Ties go to the block with more splits (b), so each t-tile's stage is
// shared by more workgroups of an L2: for the head kernels the t-tiles are the hidden
// rows, re-read for every vocab tile, and at N = 32768 the 4 x 8 block (8 splits) ran
// both passes about 2% faster than 8 x 4 (4 splits), which lost 8% once the fill
// barrier moved earlier.  Then fewer splits, then the smaller a.  Without a candidate:
// floor(cus / TT) splits (at least 1), unblocked, so no round is left with a few
// stragglers.
inline SplitPlan split_plan(int tt, int vt, int cus, int64_t t_stage = 1, int64_t s_stage = 1) {
  int s0 = tt > 0 && tt <= cus ? cus / tt : 1;   // no tiles: nothing launches
  if (s0 > vt) s0 = vt;
  if (s0 < 1) s0 = 1;
  SplitPlan best = {s0, 0, 0};
  if (tt <= 0 || cus <= 0 || cus % kNumXcd) return best;
  const int C = cus / kNumXcd;
  int64_t best_cost = -1;
  int s_max = cus / tt > 64 ? cus / tt : 64;
  if (s_max > vt) s_max = vt;
  for (int sp = 1; sp <= s_max; ++sp) {
    if (((int64_t)tt * sp) % cus) continue;
    for (int a = 1; a <= C; ++a) {
      if (C % a || tt % a || sp % (C / a)) continue;
      const int64_t cost = a * t_stage + (C / a) * s_stage;
      if (best_cost < 0 || cost < best_cost || (cost == best_cost && C / a > best.xb)) {
        best_cost = cost;
        best = {sp, a, C / a};
      }
    }
  }
  return best;
}

}  // namespace ns
