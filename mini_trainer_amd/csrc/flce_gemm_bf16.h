// bf16 MFMA main loop shared by the GEMM-shaped kernels of the bf16 path
// (gfx950).
//
// Workgroup = 4 waves (256 threads), one per CU, output tile 256 (A rows) x
// 256 (B rows).  Wave w = (wm, wn) = (w >> 1, w & 1) owns a 128 x 128 block =
// 8 x 8 fragments of v_mfma_f32_16x16x32_bf16: 256 accumulator registers
// (the AGPR file), one wave per SIMD.  Per bf16 of K a wave reads 256
// operand values from LDS for 16384 MACs, a third fewer LDS bytes per flop
// than a 128 x 64 wave tile.
//
// K advances in stages of 64 bf16 (128 bytes per operand row, whole cache
// lines); each stage is two halves kk of 32.  A stage's operands sit in
// 32 KiB LDS slots (A 256 rows x 128 bytes, B the same) of a 160 KiB ring --
// two slots for one operand, three for the other -- filled by LDS DMA
// (buffer_load_dwordx4 ... lds: no VGPR staging, 32-bit lane offsets, the K
// advance is the scalar offset).  With one wave per SIMD nothing else hides a
// stall, so the loop is software pipelined inside the wave.  With F0 / F1 =
// the kk = 0 / kk = 1 fragments of stage g:
//
//   phase 1   64 MFMAs on F0(g)        | 16 LDS reads of F1(g)
//                                      | 8 DMA instructions: three-slot
//                                      |   operand, stage g + 2
//   sync      own LDS reads retired, own DMA of stage g + 1 landed, s_barrier
//   phase 2   64 MFMAs on F1(g)        | 8 DMA instructions: two-slot
//                                      |   operand, stage g + 2 (into the
//                                      |   slot of its stage g)
//                                      | 16 LDS reads of F0(g + 1)
//
// The barrier sits between two MFMA blocks whose operands are already in
// registers; it publishes every wave's DMA of stage g + 1 and retires every
// read of stage g, whose slots are then refilled.  Inside a phase the order
// is fixed with scheduling fences: groups of kMpg MFMAs, each followed by one
// LDS read (and every other group by one DMA instruction).  Measured on
// gfx950 with s_memtime around each part of the loop: a DS or VMEM
// instruction issued within a couple of MFMAs of the previous one stalls the
// wave's MFMA issue (a burst of 16 LDS reads costs more than the 64 MFMAs it
// sits beside), so the memory instructions are spread thinly, and the third
// slot halves the DMA instructions per phase; LDS layouts are conflict-free.
//
// LDS tile formats (per operand per stage, 32 KiB):
//   KC  operand rows contiguous along K (X rows, W rows in the logits GEMM,
//       G rows in dX, X^T rows in dW): tile_off(row, chunk) of
//       flce_device.h; a fragment is one ds_read_b128.
//   TR  operand stored K-major (W in dX, G in dW): 64 K rows x 512 bytes,
//       16-byte chunk j (8 columns) of K row k at k * 512 + (j ^ tr_swz(k)) *
//       16.  A fragment is two ds_read_b64_tr_b16: within each 16-lane group
//       the instruction hands lane i element (i & 3) of the 8-byte read of
//       lane 4 e + (i >> 2), e = 0..3, so lanes reading (K row k0 + e,
//       columns c0 + 4 q .. + 3) deliver to lane i column c0 + i at K rows
//       k0 .. k0 + 3, which is the MFMA operand layout.  The reads are issued
//       from inline asm (the compiler would otherwise wait for every
//       in-flight LDS DMA before each one); their registers are tied to the
//       explicit lgkmcnt wait that ends the phase.
// Accumulator layout (B fragment issued as the MFMA's first operand): lane l
// holds for fragment (fm, fn) four consecutive columns of one row:
//   row = wm * 128 + fm * 16 + (l & 15),  col = wn * 128 + fn * 16 + 4 (l >> 4) + r.
#pragma once

#include "flce_gemm.h"

namespace mtf {

constexpr int kThreadsBf = 256;
constexpr int kBKBf = 64;                   // bf16 K elements per stage
constexpr int kTileBf = 256 * 128;          // one operand, one stage: 32 KiB
constexpr int kLdsBf = 5 * kTileBf;         // ring of 2 + 3 operand slots: 160 KiB
constexpr int kNIBf = 8;                    // DMA instructions of 1 KiB per wave per operand tile
// MFMAs per memory-instruction group inside a phase (see the header comment;
// 2 and 3 measure the same on the logits GEMM, 1 and bursts are slower).
constexpr int kMpg = 3;

// XOR applied to the 16-byte chunk index of K row k in a TR tile.  The eight
// K rows {0..3, 8..11} (+16, +32 ...) read by one half-wave of a transposing
// fragment read get eight distinct even values, i.e. distinct 32-byte bank
// groups; bit 3 also differs between rows 16 apart so that the halves
// (lanes 0-15, 32-47) and (16-31, 48-63) are spread as well.
__device__ __forceinline__ uint32_t tr_swz(uint32_t k) {
  return ((k & 3u) << 1) | ((((k >> 3) ^ (k >> 4)) & 1u) << 3);
}

// Byte offset of an LDS location (address space 3) from a generic pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ds_read_b64_tr_b16 outside the compiler's view of LDS accesses.
__device__ __forceinline__ u32x2_t ds_read_tr(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
// The same at addr + 2048 through the instruction's offset field (no
// address add between a fragment's two reads).
__device__ __forceinline__ u32x2_t ds_read_tr_2k(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:2048" : "=v"(r) : "v"(addr));
  return r;
}

// s_waitcnt vmcnt(0) only (expcnt and lgkmcnt left at their maximum).
__device__ __forceinline__ void wait_vm0() {
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0) (memory operations do not move across it).  Issued
// through the builtin so that the compiler's wait insertion sees it: after it
// every LDS read counts as complete, and the next phase's MFMAs on fragments
// read before it get no lgkmcnt waits of their own (as inline asm it was
// invisible, and each first use of a fragment waited on the LDS reads the
// phase itself had issued since).
__device__ __forceinline__ void lgkm_wait0() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));
  asm volatile("" ::: "memory");
}

// Nothing is scheduled across this point.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Raw buffer resource over `bytes` bytes from `base` (stride 0, dword 3 =
// the gfx9 raw-buffer format word).  Operand loads go through buffer
// instructions so that a lane's address is a 32-bit offset (one VGPR instead
// of two) and the K advance of a stage is a scalar offset.  Operand DMA is
// kept in range by the callers, the bound only backs that up; the dW tile
// accesses use it: a lane outside the tile gets an offset past the bound,
// whose load returns 0 and whose store is dropped.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16-byte LDS DMA of one lane: LDS[dst + 16 lane] = mem[rsrc + voff + soff].
__device__ __forceinline__ void dma16(rsrc_t r, char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)dst, 16, voff, soff, 0, 0);
}

// Operand whose rows are contiguous along K.  The 32 KiB tile is filled by
// 32 DMA instructions of 1 KiB (8 per wave); lane l of instruction q lands at
// q * 1024 + 16 l, so the lane -> (row, chunk) assignment is the inverse of
// tile_off().
struct KcOp {
  static constexpr bool kTr = false;
  rsrc_t rsrc;
  uint32_t off[kNIBf];
  uint32_t frag[2];  // LDS offset of this lane's fragment 0 for K halves 0, 1
  uint32_t tail_bad;  // bit i: DMA instruction i's chunk lies past K in the last stage

  __device__ __forceinline__ static uint32_t row_of(uint32_t i) {
    const uint32_t l = lane_id(), q = wave_id() * kNIBf + i;
    return (q >> 1) * 16 + ((l >> 3) & 1u) * 8 + (q & 1u) * 4 + (l >> 4);
  }
  __device__ __forceinline__ static uint32_t chunk_of(uint32_t i) {
    const uint32_t l = lane_id(), q = wave_id() * kNIBf + i;
    return (l & 7u) ^ ((q & 1u) * 4 + (l >> 4));
  }
  // row_off(r) = byte offset from the resource base of K element 0 of tile row r.
  template <class RowOff>
  __device__ __forceinline__ void set_rows(rsrc_t r, RowOff row_off) {
    rsrc = r;
#pragma unroll
    for (uint32_t i = 0; i < kNIBf; ++i) off[i] = row_off(row_of(i)) + chunk_of(i) * 16u;
  }
  // c_lim: 16-byte chunks (of 8) of the last K stage that lie below K.
  __device__ __forceinline__ void set_tail(uint32_t c_lim) {
    uint32_t m = 0;
#pragma unroll
    for (uint32_t i = 0; i < kNIBf; ++i) m |= (chunk_of(i) >= c_lim ? 1u : 0u) << i;
    tail_bad = m;
  }
  // wave_row0: first tile row of this wave's fragments.
  __device__ __forceinline__ void init_frag(uint32_t wave_row0) {
    const uint32_t l = lane_id();
#pragma unroll
    for (uint32_t kk = 0; kk < 2; ++kk) frag[kk] = tile_off(wave_row0 + (l & 15u), kk * 4 + (l >> 4));
  }
  // DMA instruction i (0..7) of this wave for stage kt.
  __device__ __forceinline__ void issue_one(char* tile, int kt, int i) const {
    dma16(rsrc, tile + (wave_id() * kNIBf + (uint32_t)i) * 1024u, off[i], (uint32_t)kt * 128u);
  }
  __device__ __forceinline__ void issue(char* tile, int kt) const {
#pragma unroll
    for (int i = 0; i < kNIBf; ++i) issue_one(tile, kt, i);
  }
  // The same with a possibly partial last K stage (tail: kt is that stage):
  // chunks past K re-read chunk 0 of their row, which is in bounds, and the
  // fragments holding them are zeroed after they are read (mask_tail), so no
  // byte past a row's K extent -- past the end of the array for its last
  // row -- is touched.  Branch-free: the choice is a select on the offsets.
  __device__ __forceinline__ void issue_one_k(char* tile, int kt, int i, bool tail) const {
    const bool bad = tail && ((tail_bad >> i) & 1u);
    const uint32_t voff = bad ? off[i] - chunk_of(i) * 16u : (tail ? off[i] + (uint32_t)kt * 128u : off[i]);
    dma16(rsrc, tile + (wave_id() * kNIBf + (uint32_t)i) * 1024u, voff, tail ? 0u : (uint32_t)kt * 128u);
  }
  __device__ __forceinline__ void issue_k(char* tile, int kt, bool tail) const {
#pragma unroll
    for (int i = 0; i < kNIBf; ++i) issue_one_k(tile, kt, i, tail);
  }
  __device__ __forceinline__ u32x4_t read(const char* tile, int kk, int f) const {
    return lds_read16(tile, frag[kk] + (uint32_t)f * 2048u);
  }
};

// Zero the fragments of K half kk of the last (partial) K stage in the lanes
// whose 8 K values lie at or past K: lane l holds K chunk kk * 4 + (l >> 4)
// of the stage, and the stage's first c_lim chunks lie below K.
__device__ __forceinline__ void mask_tail(u32x4_t (&fr)[8], int kk, uint32_t c_lim) {
  const bool bad = (uint32_t)kk * 4u + (lane_id() >> 4) >= c_lim;
#pragma unroll
  for (int f = 0; f < 8; ++f) fr[f] = bad ? u32x4_t{0u, 0u, 0u, 0u} : fr[f];
}

// Operand stored K-major: row-major [K, 256-column tile].  Instruction q of
// the tile covers K rows 2 q and 2 q + 1; lane l writes LDS chunk l & 31 of
// K row 2 q + (l >> 5) and so loads global chunk (l & 31) ^ tr_swz(k).
// The per-lane state is small: the K row of instruction i is krow0 + 2 i,
// and with k = 16 w + (l >> 5) + 2 i, tr_swz(k) depends on i only through
// (i & 1, i >= 4), so the column offsets take four values; the fragment
// reads' bases differ by constants and share one XOR mask (the lane's K row
// inside a fragment read, 8 g + 4 h + (L >> 2), fixes tr_swz independently
// of kk and h).
// A DMA's address is split into a per-lane part, min(row offset, limit) +
// column offset, and a uniform scalar offset, base + stage * 64 rows: two
// full-rate VALU instructions per DMA.  (Formed as base + k ld_b with k
// clamped per lane, it took a quarter-rate 64-bit multiply-add right before
// every DMA, which stalled the MFMA issue behind it.)
struct TrOp {
  static constexpr bool kTr = true;
  rsrc_t rsrc;
  uint32_t base, ld_b;
  int32_t k_limit;
  uint32_t rowoff[kNIBf];  // (16 w + (l >> 5) + 2 i) ld_b: instruction i's K row
  uint32_t moff[4];        // [(i >= 4) * 2 + (i & 1)]
  uint32_t fbase, fxor;

  // r, base: resource and byte offset of (K row 0, column 0) of the tile;
  // k_limit: K rows that exist (rows at or beyond it read row k_limit - 1,
  // whose products the caller discards or multiplies by zero); m_valid: tile
  // columns that exist (the others read column 0 and are discarded later);
  // wave_col0: first tile column of this wave's fragments, a multiple of 128
  // (fragments f = 0..7 then stay inside one group of 16 chunks, so the XOR
  // of tr_swz never leaves it).
  __device__ __forceinline__ void init(rsrc_t r, uint32_t base_, uint32_t ld_b_, int32_t k_limit_,
                                       int32_t m_valid, uint32_t wave_col0) {
    rsrc = r;
    base = base_;
    ld_b = ld_b_;
    k_limit = k_limit_;
    const uint32_t l = lane_id(), w = wave_id();
    const uint32_t krow0 = 16u * w + (l >> 5);
#pragma unroll
    for (int i = 0; i < kNIBf; ++i) rowoff[i] = (krow0 + 2u * (uint32_t)i) * ld_b;
#pragma unroll
    for (uint32_t p = 0; p < 4; ++p) {
      const uint32_t i = (p >> 1) * 4 + (p & 1);  // representative i of the pattern
      const uint32_t j = (l & 31u) ^ tr_swz(krow0 + 2 * i);
      const int32_t m0 = (int32_t)j * 8;
      moff[p] = m0 < m_valid ? (uint32_t)m0 * 2u : 0u;
    }
    const uint32_t g = l >> 4, L = l & 15u, c0 = wave_col0 / 8u;
    const uint32_t k = 8 * g + (L >> 2);
    // fragment f sits at chunk c0 + 2 f + ((L & 3) >> 1); c0's low four bits
    // and that lane bit join the XOR mask, so f enters as 32 f ^ mask
    fbase = k * 512u + (c0 & ~15u) * 16u + (L & 1u) * 8u;
    fxor = ((c0 & 15u) ^ tr_swz(k) ^ ((L & 3u) >> 1)) * 16u;
  }
  // K row kb + r (kb = 64 kt, r = the lane's row in the stage) clamped to
  // k_limit - 1: kb ld_b goes to the scalar offset and the lane's part is
  // min(r ld_b, (k_limit - 1 - kb) ld_b); the bound is uniform and at least
  // 63 ld_b in every stage but a partial last one.
  __device__ __forceinline__ void issue_one(char* tile, int kt, int i) const {
    const int32_t kb = kt * kBKBf;
    const int32_t rem = k_limit - 1 - kb;
    const uint32_t lim = (uint32_t)(rem > 0 ? rem : 0) * ld_b;
    const uint32_t r = rowoff[i] < lim ? rowoff[i] : lim;
    dma16(rsrc, tile + (wave_id() * kNIBf + (uint32_t)i) * 1024u,
          r + moff[(i >= 4 ? 2 : 0) + (i & 1)], base + (uint32_t)kb * ld_b);
  }
  __device__ __forceinline__ void issue(char* tile, int kt) const {
#pragma unroll
    for (int i = 0; i < kNIBf; ++i) issue_one(tile, kt, i);
  }
  // Two transposing reads into one 128-bit register tuple (inline asm; the
  // phase ends with lgkm_wait0 and tie_frags before any use).  K half kk and
  // read h add (32 kk + 4 h) K rows of 512 bytes to the base.
  __device__ __forceinline__ u32x4_t read(const char* tile, int kk, int f) const {
    const uint32_t t = lds_addr(tile) + fbase + ((32u * (uint32_t)f) ^ fxor);
    const uint32_t tk = t + (uint32_t)kk * 32u * 512u;
    const u32x2_t lo = ds_read_tr(tk);
    const u32x2_t hi = ds_read_tr_2k(tk);  // 4 K rows of 512 bytes on
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
  }
};

// Make fragments read by inline asm depend on the preceding explicit wait
// (the compiler does not know that those reads complete only then).
template <class Op>
__device__ __forceinline__ void tie_frags(u32x4_t (&fr)[8]) {
  if constexpr (Op::kTr) {
#pragma unroll
    for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(fr[i]));
  }
}

// MFMA i (0..63) of a phase: fragment row fm = i / 8, column fn = i % 8.
__device__ __forceinline__ void mfma_one(f32x4_t (&acc)[8][8], const u32x4_t (&fa)[8],
                                         const u32x4_t (&fb)[8], int i) {
  acc[i >> 3][i & 7] = mma_chunk<__bf16>(fb[i & 7], fa[i >> 3], acc[i >> 3][i & 7]);
}

// Accumulators start at zero (the init hook of every kernel but dW).
struct ZeroInit {
  __device__ __forceinline__ void operator()(int, f32x4_t (&acc)[8][8]) const {
#pragma unroll
    for (int fm = 0; fm < 8; ++fm)
#pragma unroll
      for (int fn = 0; fn < 8; ++fn) acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
};

// s_waitcnt vmcnt(8): every DMA but the last eight issued has landed.
__device__ __forceinline__ void wait_vm8() {
  __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8));
}

// Stream of ntiles output tiles of KT stages each (see the header comment);
// retarget(tile) re-points the operands before the first DMA of a tile,
// init(tile, acc) sets a tile's accumulators before its first MFMA (zero, or
// values loaded from memory that the tile adds to), and
// epilogue(tile, acc, scratch) runs after a tile's last MFMA;
// `scratch` is a 32 KiB LDS buffer that is free until the next phase 1 (the
// epilogue ends with a barrier if it uses it).
//
// LDS ring (160 KiB): the operand named by kThreeA (A if true, else B) has
// three 32 KiB slots, the other two.  The three-slot operand's DMA of stage
// g + 2 goes into the slot of its stage g - 1 during phase 1 (free since the
// barrier that closed phase 1 of g - 1), the two-slot operand's into the
// slot of its stage g during phase 2: eight DMA instructions per wave per
// phase instead of sixteen in phase 2 alone, and one and a half stages of
// lead for the three-slot operand, which is the one streamed from HBM (W;
// G in dW).  The sync between the phases waits for all but the newest eight
// DMAs (the three-slot operand's stage g + 2).
//
// Each phase is one basic block: the retarget branch sits before phase 1,
// and every phase issues its DMA -- the two stages past the end reload the
// last tile's final stage into slots that are never read again.
// kKTail (both operands KcOp, K contiguous in their rows): the last K stage
// holds only c_lim of its 8 chunks below K; its DMA keeps to the rows' K
// extent and its fragments are masked (KcOp::issue_one_k, mask_tail).
// more(t): does tile t exist?  It is asked in increasing order of t, at most
// one tile ahead of the one being multiplied when KT >= 2 (two ahead when
// KT == 1) -- a tile stream whose length is found as it runs (a work queue)
// answers from what it has fetched so far.
// kCarry: one accumulator array for all tiles; init runs for tile 0 only and
// the epilogue of tile t leaves tile t + 1's starting values in it (dW: its
// stores of tile t interleaved with the loads of tile t + 1).
template <bool kThreeA, bool kKTail = false, bool kCarry = false, class A, class B, class More,
          class Retarget, class Epi, class Init = ZeroInit>
__device__ __forceinline__ void mainloop_bf16_seq(char* lds, A& a, B& b, int KT, More more,
                                                  Retarget retarget, Epi epilogue,
                                                  Init init = Init(), uint32_t c_lim = 8) {
  if (KT <= 0 || !more(0)) return;
  // With a transposed operand (two ds_read_b64_tr_b16 per fragment) each DMA
  // instruction goes one MFMA into the group after the LDS read it used to
  // follow, so that no two memory instructions are adjacent (dX -3% on the
  // same box); the logits GEMMs keep the DMA right after the read (measured
  // 1% faster that way).
  constexpr bool kSpread = A::kTr || B::kTr;
  // (tile2, kt2) = coordinates of stage g + 2, the next stage to be loaded;
  // they stop at the last stage of the last tile
  int tile2 = 0, kt2 = 0;
  auto advance = [&]() __attribute__((always_inline)) {
    if (kt2 + 1 < KT) {
      ++kt2;
    } else if (more(tile2 + 1)) {
      kt2 = 0;
      ++tile2;
      retarget(tile2);
    }
  };
  // slots: the two-slot operand at [0, 64 KiB), the three-slot one above
  char* const two0 = lds;
  char* const three0 = lds + 2 * kTileBf;
  auto slot_a = [&](int s2, int s3) __attribute__((always_inline)) {
    return kThreeA ? three0 + s3 * kTileBf : two0 + s2 * kTileBf;
  };
  auto slot_b = [&](int s2, int s3) __attribute__((always_inline)) {
    return kThreeA ? two0 + s2 * kTileBf : three0 + s3 * kTileBf;
  };
  // DMA of stage kt2 of the current tile: the last stage may be partial
  auto issue_a = [&](char* dst, int kt) __attribute__((always_inline)) {
    if constexpr (kKTail) a.issue_k(dst, kt, kt == KT - 1);
    else a.issue(dst, kt);
  };
  auto issue_b = [&](char* dst, int kt) __attribute__((always_inline)) {
    if constexpr (kKTail) b.issue_k(dst, kt, kt == KT - 1);
    else b.issue(dst, kt);
  };
  auto issue_one_a = [&](char* dst, int kt, int i) __attribute__((always_inline)) {
    if constexpr (kKTail) a.issue_one_k(dst, kt, i, kt == KT - 1);
    else a.issue_one(dst, kt, i);
  };
  auto issue_one_b = [&](char* dst, int kt, int i) __attribute__((always_inline)) {
    if constexpr (kKTail) b.issue_one_k(dst, kt, i, kt == KT - 1);
    else b.issue_one(dst, kt, i);
  };
  retarget(0);
  issue_a(slot_a(0, 0), kt2);
  issue_b(slot_b(0, 0), kt2);
  advance();
  issue_a(slot_a(1, 1), kt2);
  issue_b(slot_b(1, 1), kt2);
  wait_vm0();
  __builtin_amdgcn_s_barrier();
  u32x4_t fa0[8], fb0[8], fa1[8], fb1[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    fa0[f] = a.read(slot_a(0, 0), 0, f);
    fb0[f] = b.read(slot_b(0, 0), 0, f);
  }
  lgkm_wait0();
  tie_frags<A>(fa0);
  tie_frags<B>(fb0);
  int g = 0, g3 = 0;  // stage being multiplied, g % 3
  f32x4_t acc_carried[8][8];
  for (int tile = 0; more(tile); ++tile) {
    f32x4_t acc_own[8][8];
    f32x4_t(&acc)[8][8] = kCarry ? acc_carried : acc_own;
    if (!kCarry || tile == 0) init(tile, acc);
    for (int kt = 0; kt < KT; ++kt, ++g, g3 = (g3 == 2 ? 0 : g3 + 1)) {
      advance();
      if constexpr (kKTail) {
        if (kt == KT - 1) {
          mask_tail(fa0, 0, c_lim);
          mask_tail(fb0, 0, c_lim);
        }
      }
      sched_fence();
      const int g2 = g & 1, g2n = g2 ^ 1;
      const int g3n = g3 == 2 ? 0 : g3 + 1, g3p = g3 == 0 ? 2 : g3 - 1;  // (g+1)%3, (g+2)%3
      const char* ra = slot_a(g2, g3);
      const char* rb = slot_b(g2, g3);
      // phase 1: MFMAs on F0(g), LDS reads of F1(g), DMA of the three-slot
      // operand's stage g + 2 (into the slot of its stage g - 1)
      char* w3 = three0 + g3p * kTileBf;
      auto dma3 = [&](int d) __attribute__((always_inline)) {
        sched_fence();
        if (kThreeA) issue_one_a(w3, kt2, d);
        else issue_one_b(w3, kt2, d);
        sched_fence();
      };
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        mfma_one(acc, fa0, fb0, kMpg * i);
        if (kSpread && (i & 1) == 0 && i >= 2) dma3((i - 2) >> 1);
#pragma unroll
        for (int j = 1; j < kMpg; ++j) mfma_one(acc, fa0, fb0, kMpg * i + j);
        if (i & 1) fb1[i >> 1] = b.read(rb, 1, i >> 1);
        else fa1[i >> 1] = a.read(ra, 1, i >> 1);
        if (!kSpread && (i & 1)) {
          if (kThreeA) issue_one_a(w3, kt2, i >> 1);
          else issue_one_b(w3, kt2, i >> 1);
        }
        sched_fence();
      }
      mfma_one(acc, fa0, fb0, 16 * kMpg);
      if (kSpread) dma3(7);
#pragma unroll
      for (int i = 16 * kMpg + 1; i < 64; ++i) mfma_one(acc, fa0, fb0, i);
      sched_fence();
      // every wave: reads of stage g retired, own DMA of stage g + 1 landed
      // (the three-slot operand's stage g + 2 may still be in flight)
      lgkm_wait0();
      tie_frags<A>(fa1);
      tie_frags<B>(fb1);
      wait_vm8();
      __builtin_amdgcn_s_barrier();
      if constexpr (kKTail) {
        if (kt == KT - 1) {
          mask_tail(fa1, 1, c_lim);
          mask_tail(fb1, 1, c_lim);
        }
      }
      sched_fence();
      // phase 2: MFMAs on F1(g), DMA of the two-slot operand's stage g + 2
      // into the slot of its stage g, LDS reads of F0(g + 1) (stale after the
      // last stage, never used)
      char* w2 = two0 + g2 * kTileBf;
      const char* ra1 = slot_a(g2n, g3n);
      const char* rb1 = slot_b(g2n, g3n);
      auto dma2 = [&](int d) __attribute__((always_inline)) {
        sched_fence();
        if (kThreeA) issue_one_b(w2, kt2, d);
        else issue_one_a(w2, kt2, d);
        sched_fence();
      };
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        mfma_one(acc, fa1, fb1, kMpg * i);
        if (kSpread && (i & 1) == 0 && i >= 2) dma2((i - 2) >> 1);
#pragma unroll
        for (int j = 1; j < kMpg; ++j) mfma_one(acc, fa1, fb1, kMpg * i + j);
        if (!kSpread && (i & 1)) {
          if (kThreeA) issue_one_b(w2, kt2, i >> 1);
          else issue_one_a(w2, kt2, i >> 1);
        }
        if (i & 1) fb0[i >> 1] = b.read(rb1, 0, i >> 1);
        else fa0[i >> 1] = a.read(ra1, 0, i >> 1);
        sched_fence();
      }
      mfma_one(acc, fa1, fb1, 16 * kMpg);
      if (kSpread) dma2(7);
#pragma unroll
      for (int i = 16 * kMpg + 1; i < 64; ++i) mfma_one(acc, fa1, fb1, i);
      sched_fence();
      lgkm_wait0();
      tie_frags<A>(fa0);
      tie_frags<B>(fb0);
    }
    // the three-slot operand's slot of the last stage (g - 1) is free until
    // phase 1 of stage g refills it
    epilogue(tile, acc, three0 + (g3 == 0 ? 2 : g3 - 1) * kTileBf);
    // The next tile's first fragments were read in the last phase; reading
    // them again here (stage g is resident until phase 2 of stage g refills
    // the two-slot operand's other buffer) keeps their 64 registers free
    // during the epilogue.
    if (more(tile + 1)) {
      // (the memory clobber keeps these reads from being hoisted into the
      // epilogue, where their registers would be live again)
      lgkm_wait0();
      const char* ra = slot_a(g & 1, g3);
      const char* rb = slot_b(g & 1, g3);
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        fa0[f] = a.read(ra, 0, f);
        fb0[f] = b.read(rb, 0, f);
      }
      lgkm_wait0();
      tie_frags<A>(fa0);
      tie_frags<B>(fb0);
    }
  }
  wait_vm0();
}

// The same over a fixed number of tiles.
template <bool kThreeA, bool kKTail = false, class A, class B, class Retarget, class Epi,
          class Init = ZeroInit>
__device__ __forceinline__ void mainloop_bf16(char* lds, A& a, B& b, int KT, int ntiles,
                                              Retarget retarget, Epi epilogue, Init init = Init(),
                                              uint32_t c_lim = 8) {
  mainloop_bf16_seq<kThreeA, kKTail>(
      lds, a, b, KT, [ntiles](int t) __attribute__((always_inline)) { return t < ntiles; },
      retarget, epilogue, init, c_lim);
}

}  // namespace mtf
