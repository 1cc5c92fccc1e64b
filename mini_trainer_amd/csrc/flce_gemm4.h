// bf16 MFMA main loop of the eight-wave workgroup (gfx950).
//
// Workgroup = 8 waves (512 threads), one per CU, output tile 256 (A rows) x
// 256 (B rows).  Wave w = (wm, wn) = (w >> 2, w & 3) owns a 128 x 64 block =
// 8 x 4 fragments of 16 x 16, so its accumulators take 128 registers and two
// waves share each SIMD: while one waits on LDS data or a barrier, the other
// issues MFMAs.
//
// K advances in stages of 64 bf16 (128 bytes per operand row, whole cache
// lines).  A stage holds the A tile and the B tile, 32 KiB each; two stages
// use 128 KiB of the 160 KiB LDS.  Stages are filled by
// global_load_lds_dwordx4 (no VGPR staging) one stage ahead: the loads of
// stage g + 1 are issued right after the barrier that opens stage g.
//
// LDS tile formats (per operand per stage, 32 KiB):
//   KC  operand rows contiguous along K (X rows, W rows in the logits GEMM,
//       G rows in dX, X^T rows in dW): tile_off(row, chunk) of
//       flce_device.h; a fragment is one ds_read_b128.
//   TR  operand stored K-major (W in dX, G in dW): 64 K rows x 512 bytes,
//       16-byte chunk j (8 columns) of K row k at k * 512 + (j ^ tr4_swz(k)) *
//       16.  A fragment is two ds_read_b64_tr_b16: within each 16-lane group
//       the instruction hands lane i element (i & 3) of the 8-byte read of
//       lane 4 e + (i >> 2), e = 0..3, so lanes reading (K row k0 + e,
//       columns c0 + 4 q .. + 3) deliver to lane i column c0 + i at K rows
//       k0 .. k0 + 3, which is the MFMA operand layout.  tr4_swz spreads the
//       eight K rows that one half-wave reads over distinct bank groups.
//       The reads are issued from inline asm (the compiler would otherwise
//       wait for every in-flight LDS DMA before each one) and are followed by
//       an explicit lgkmcnt wait tied to the fragment registers.
// Accumulator layout (B fragment issued as the MFMA's first operand): lane l
// holds for fragment (fm, fn) four consecutive columns of one row:
//   row = wm * 128 + fm * 16 + (l & 15),  col = wn * 64 + fn * 16 + 4 (l >> 4) + r.
#pragma once

#include "flce_gemm.h"

namespace mtf {

constexpr int kThreads4 = 512;
constexpr int kBK4 = 64;                   // bf16 K elements per stage
constexpr int kTile4 = 256 * 128;          // one operand, one stage: 32 KiB
constexpr int kStage4 = 2 * kTile4;        // A + B
constexpr int kLds4 = 2 * kStage4;         // two stages: 128 KiB

// XOR applied to the 16-byte chunk index of K row k in a TR tile.  The eight
// K rows {0..3, 8..11} (+16, +32 ...) read by one half-wave of a transposing
// fragment read get eight distinct even values, i.e. distinct 32-byte bank
// groups; bit 3 also differs between rows 16 apart so that the halves
// (lanes 0-15, 32-47) and (16-31, 48-63) are spread as well.
__device__ __forceinline__ uint32_t tr4_swz(uint32_t k) {
  return ((k & 3u) << 1) | ((((k >> 3) ^ (k >> 4)) & 1u) << 3);
}

// Byte offset of an LDS location (address space 3) from a generic pointer.
__device__ __forceinline__ uint32_t lds_addr4(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ds_read_b64_tr_b16 outside the compiler's view of LDS accesses.
__device__ __forceinline__ u32x2_t ds_read_tr4(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

// s_waitcnt vmcnt(0) only (expcnt and lgkmcnt left at their maximum).
__device__ __forceinline__ void wait_vm0() {
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

// Raw buffer resource over `bytes` bytes from `base` (stride 0, dword 3 =
// the gfx9 raw-buffer format word).  Operand loads go through buffer
// instructions so that a lane's address is a 32-bit offset (one VGPR instead
// of two) and the K advance of a stage is a scalar offset; every access is
// kept in range by the callers, the resource bound only backs that up.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
constexpr uint32_t kWholeRange = 0xffffffffu;

// 16-byte LDS DMA of one lane: LDS[dst + 16 lane] = mem[rsrc + voff + soff].
__device__ __forceinline__ void dma16(rsrc_t r, char* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)dst, 16, voff, soff, 0, 0);
}

// Operand whose rows are contiguous along K.  The 32 KiB tile is filled by
// 32 DMA instructions of 1 KiB (4 per wave); lane l of instruction q lands at
// q * 1024 + 16 l, so the lane -> (row, chunk) assignment is the inverse of
// tile_off().
struct Kc4 {
  static constexpr bool kTr = false;
  rsrc_t rsrc;
  uint32_t off[4];
  uint32_t frag[2];  // LDS offset of this lane's fragment 0 for K halves 0, 1

  __device__ __forceinline__ static uint32_t row_of(uint32_t i) {
    const uint32_t l = lane_id(), q = wave_id() * 4 + i;
    return (q >> 1) * 16 + ((l >> 3) & 1u) * 8 + (q & 1u) * 4 + (l >> 4);
  }
  __device__ __forceinline__ static uint32_t chunk_of(uint32_t i) {
    const uint32_t l = lane_id(), q = wave_id() * 4 + i;
    return (l & 7u) ^ ((q & 1u) * 4 + (l >> 4));
  }
  // row_off(r) = byte offset from the resource base of K element 0 of tile row r.
  template <class RowOff>
  __device__ __forceinline__ void set_rows(rsrc_t r, RowOff row_off) {
    rsrc = r;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) off[i] = row_off(row_of(i)) + chunk_of(i) * 16u;
  }
  // wave_row0: first tile row of this wave's fragments.
  __device__ __forceinline__ void init_frag(uint32_t wave_row0) {
    const uint32_t l = lane_id();
#pragma unroll
    for (uint32_t kk = 0; kk < 2; ++kk) frag[kk] = tile_off(wave_row0 + (l & 15u), kk * 4 + (l >> 4));
  }
  __device__ __forceinline__ void issue(char* tile, int kt) const {
    const uint32_t w = wave_id();
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) dma16(rsrc, tile + (w * 4 + i) * 1024u, off[i], (uint32_t)kt * 128u);
  }
  __device__ __forceinline__ u32x4_t read(const char* tile, int kk, int f) const {
    return lds_read16(tile, frag[kk] + (uint32_t)f * 2048u);
  }
};

// Operand stored K-major: row-major [K, 256-column tile].  Instruction q of
// the tile covers K rows 2 q and 2 q + 1; lane l writes LDS chunk l & 31 of
// K row 2 q + (l >> 5) and so loads global chunk (l & 31) ^ tr4_swz(k).
struct Tr4 {
  static constexpr bool kTr = true;
  rsrc_t rsrc;
  uint32_t base, ld_b;
  int32_t k_limit;
  uint32_t moff[4];
  uint32_t krow[4];
  uint32_t fbase[2][2], fxor[2][2];  // [kk][h]

  // r, base: resource and byte offset of (K row 0, column 0) of the tile;
  // k_limit: K rows that exist (rows at or beyond it read row k_limit - 1,
  // whose products the caller discards or multiplies by zero); m_valid: tile
  // columns that exist (the others read column 0 and are discarded later);
  // wave_col0: first tile column of this wave's fragments.
  __device__ __forceinline__ void init(rsrc_t r, uint32_t base_, uint32_t ld_b_, int32_t k_limit_,
                                       int32_t m_valid, uint32_t wave_col0) {
    rsrc = r;
    base = base_;
    ld_b = ld_b_;
    k_limit = k_limit_;
    const uint32_t l = lane_id(), w = wave_id();
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      const uint32_t q = w * 4 + i;
      const uint32_t k = 2 * q + (l >> 5);
      const uint32_t j = (l & 31u) ^ tr4_swz(k);
      krow[i] = k;
      const int32_t m0 = (int32_t)j * 8;
      moff[i] = m0 < m_valid ? (uint32_t)m0 * 2u : 0u;
    }
    const uint32_t g = l >> 4, L = l & 15u, c0 = wave_col0 / 8u;
#pragma unroll
    for (uint32_t kk = 0; kk < 2; ++kk)
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t k = 32 * kk + 8 * g + 4 * h + (L >> 2);
        // fragment f sits at chunk c0 + 2 f + ((L & 3) >> 1); c0's low four
        // bits and that lane bit join the XOR mask, so f enters as 32 f ^ mask
        fbase[kk][h] = k * 512u + (c0 & ~15u) * 16u + (L & 1u) * 8u;
        fxor[kk][h] = ((c0 & 15u) ^ tr4_swz(k) ^ ((L & 3u) >> 1)) * 16u;
      }
  }
  __device__ __forceinline__ void issue(char* tile, int kt) const {
    const uint32_t w = wave_id();
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
      int32_t k = kt * kBK4 + (int32_t)krow[i];
      k = k < k_limit ? k : k_limit - 1;
      dma16(rsrc, tile + (w * 4 + i) * 1024u, base + (uint32_t)k * ld_b + moff[i], 0u);
    }
  }
  // Two transposing reads into one 128-bit register tuple (inline asm; the
  // caller waits with tr4_wait before use).
  __device__ __forceinline__ u32x4_t read(const char* tile, int kk, int f) const {
    const uint32_t t = lds_addr4(tile);
    const u32x2_t lo = ds_read_tr4(t + fbase[kk][0] + ((32u * (uint32_t)f) ^ fxor[kk][0]));
    const u32x2_t hi = ds_read_tr4(t + fbase[kk][1] + ((32u * (uint32_t)f) ^ fxor[kk][1]));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
  }
};

// Wait for all LDS reads and make the fragment registers depend on it.
template <int N>
__device__ __forceinline__ void tr4_wait(u32x4_t (&fr)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(fr[i]));
}

__device__ __forceinline__ void mfma4_8x4(f32x4_t (&acc)[8][4], const u32x4_t (&fa)[8],
                                          const u32x4_t (&fb)[4]) {
#pragma unroll
  for (int fm = 0; fm < 8; ++fm)
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) acc[fm][fn] = mma_chunk<__bf16>(fb[fn], fa[fm], acc[fm][fn]);
}

// Wave coordinates of the eight-wave workgroup.
struct Wave4 {
  uint32_t wm, wn;
  __device__ __forceinline__ Wave4() {
    const uint32_t w = wave_id();
    wm = w >> 2;
    wn = w & 3u;
  }
};

// Stream of ntiles output tiles of KT stages each; the two-stage DMA ring
// runs across tile boundaries.  retarget(tile) re-points the operands before
// the first load of a tile; epilogue(tile, acc) runs after a tile's last MFMA
// and must not touch LDS (the next tile's first stage is in flight).
template <class A, class B, class Retarget, class Epi>
__device__ __forceinline__ void mainloop4(char* lds, A& a, B& b, int KT, int ntiles,
                                          Retarget retarget, Epi epilogue) {
  const int total = KT * ntiles;
  if (total <= 0) return;
  auto issue = [&](int g) __attribute__((always_inline)) {
    const int tile = g / KT, kt = g - tile * KT;
    if (kt == 0) retarget(tile);
    char* st = lds + (g & 1) * kStage4;
    a.issue(st, kt);
    b.issue(st + kTile4, kt);
  };
  issue(0);
  int g = 0;
  for (int tile = 0; tile < ntiles; ++tile) {
    f32x4_t acc[8][4];
#pragma unroll
    for (int fm = 0; fm < 8; ++fm)
#pragma unroll
      for (int fn = 0; fn < 4; ++fn) acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kt = 0; kt < KT; ++kt, ++g) {
      // this wave's loads of stage g have landed; the barrier publishes every
      // wave's and retires all reads of stage g - 1, whose buffer is refilled next
      wait_vm0();
      __builtin_amdgcn_s_barrier();
      if (g + 1 < total) issue(g + 1);
      const char* st = lds + (g & 1) * kStage4;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        u32x4_t fa[8], fb[4];
#pragma unroll
        for (int f = 0; f < 8; ++f) fa[f] = a.read(st, kk, f);
#pragma unroll
        for (int f = 0; f < 4; ++f) fb[f] = b.read(st + kTile4, kk, f);
        if constexpr (A::kTr) tr4_wait(fa);
        if constexpr (B::kTr) tr4_wait(fb);
        mfma4_8x4(acc, fa, fb);
      }
    }
    epilogue(tile, acc);
  }
}

}  // namespace mtf
