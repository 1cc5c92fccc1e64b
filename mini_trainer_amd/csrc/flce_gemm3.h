// bf16 MFMA main loop for two resident workgroups per CU (gfx950).
//
// Workgroup = 4 waves, output tile 256 (A rows) x 128 (B rows); wave (wm, wn)
// owns a 128 x 64 quadrant = 8 x 4 fragments of 16 x 16, so its accumulators
// take 128 registers and two workgroups (8 waves, 2 per SIMD) stay resident.
// The two waves sharing a SIMD come from different workgroups; while one
// waits on LDS data, a barrier or global loads, the other issues MFMAs, which
// is what keeps the matrix cores busy (no per-wave software pipelining).
//
// K advances in stages of 32 bf16.  A stage holds the A tile (256 x 64 B =
// 16 KiB) and the B tile (128 x 64 B = 8 KiB); NS = 3 stages = 72 KiB per
// workgroup (two workgroups use 144 of the 160 KiB).  Stages are filled by
// global_load_lds_dwordx4 (no VGPR staging) NS - 1 stages ahead.
//
// LDS tile formats (per stage):
//   KC  operand rows contiguous along K (X rows, W rows in the forward, G
//       rows in dX, X^T rows in dW): ROWS x 64 B, 16-byte chunk c of row r at
//       r * 64 + ((c ^ (r >> 2)) & 3) * 16.  Fragment = one ds_read_b128.
//   TR  operand stored K-major (W in dX, G in dW): 32 K rows x (COLS * 2) B,
//       16-byte chunk j (8 columns) of K row k at
//       k * COLS * 2 + (j ^ tr_swz(k)) * 16.  Fragment = two
//       ds_read_b64_tr_b16: within each 16-lane group the instruction hands
//       lane i element (i & 3) of the 8-byte read of lane 4 e + (i >> 2),
//       e = 0..3, so lanes reading (k0 + e, col0 + 4 q .. + 3) deliver to lane
//       i the column col0 + i at K rows k0 .. k0 + 3 -- the MFMA operand.
//       The TR reads are issued from inline asm (the compiler would otherwise
//       wait for every in-flight LDS DMA before each one) and are followed by
//       an explicit lgkmcnt wait tied to the fragment registers.
// Accumulator layout (B fragment issued as the MFMA's first operand): lane l
// holds for fragment (fm, fn) four consecutive columns of one row:
//   row = wm * 128 + fm * 16 + (l & 15),  col = wn * 64 + fn * 16 + 4 (l >> 4) + r.
#pragma once

#include "flce_gemm.h"

namespace mtf {

constexpr int kBK3 = 32;              // bf16 K elements per stage
constexpr int kRowsA3 = 256, kRowsB3 = 128;
constexpr int kTileA3 = kRowsA3 * 64;  // 16 KiB
constexpr int kTileB3 = kRowsB3 * 64;  // 8 KiB
constexpr int kStage3 = kTileA3 + kTileB3;
constexpr int kNS3 = 3;
constexpr int kLds3 = kNS3 * kStage3;  // 72 KiB

__device__ __forceinline__ uint32_t kc3_off(uint32_t row, uint32_t c) {
  return row * 64u + (((c ^ (row >> 2)) & 3u) << 4);
}
__device__ __forceinline__ uint32_t tr3_swz(uint32_t k) { return ((k + 4u * (k >> 3)) & 7u) << 1; }

// Byte offset of an LDS location (address space 3) from a generic pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ds_read_b64_tr_b16 outside the compiler's view of LDS accesses.
__device__ __forceinline__ u32x2_t ds_read_tr_asm(uint32_t addr) {
  u32x2_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

// s_waitcnt vmcnt(N) only.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Operand whose rows are contiguous along K.  ROWS = 256 (A) or 128 (B).
template <int ROWS>
struct KcOp {
  static constexpr int kInstr = ROWS / 64;  // 1 KiB DMA instructions per wave per stage
  static constexpr int kTrReads = 0;
  const char* p[kInstr];
  uint32_t frag;

  __device__ __forceinline__ static uint32_t row_of(uint32_t i) {
    return (wave_id() * kInstr + i) * 16 + (lane_id() >> 2);
  }
  template <class RowPtr>
  __device__ __forceinline__ void set_rows(RowPtr row_ptr) {
    const uint32_t l = lane_id();
    const uint32_t c = ((l & 3u) ^ ((l >> 4) & 3u)) * 16u;
#pragma unroll
    for (uint32_t i = 0; i < kInstr; ++i) p[i] = row_ptr(row_of(i)) + c;
  }
  __device__ __forceinline__ void init_frag(uint32_t wave_row0) {
    const uint32_t l = lane_id();
    frag = kc3_off(wave_row0 + (l & 15u), l >> 4);
  }
  __device__ __forceinline__ void issue(char* tile, int kt) const {
    const uint32_t w = wave_id();
    const int64_t koff = (int64_t)kt * 64;
#pragma unroll
    for (uint32_t i = 0; i < kInstr; ++i)
      __builtin_amdgcn_global_load_lds(p[i] + koff, (lds_void_t*)(tile + (w * kInstr + i) * 1024u),
                                       16, 0, 0);
  }
  __device__ __forceinline__ u32x4_t read(const char* tile, int f) const {
    return lds_read16(tile, frag + (uint32_t)f * 1024u);
  }
};

// Operand stored K-major: row-major [K, COLS-wide tile], COLS = 256 or 128.
template <int COLS>
struct TrOp {
  static constexpr int kRowB = COLS * 2;          // bytes per K row
  static constexpr int kInstr = COLS / 64;        // DMA instructions per wave per stage
  static constexpr int kRowsPerInstr = 1024 / kRowB;
  static constexpr int kTrReads = 2;
  const char* base;
  int64_t ld_b;
  int32_t k_limit;
  uint32_t moff[kInstr];
  uint32_t krow[kInstr];
  uint32_t fbase[2], fxor[2];

  // base: (k = 0, column 0 of the tile); k_limit: K rows that exist;
  // m_valid: tile columns that exist (others read column 0, discarded later);
  // wave_col0: first tile column of this wave's fragments.
  __device__ __forceinline__ void init(const char* base_, int64_t ld_b_, int32_t k_limit_,
                                       int32_t m_valid, uint32_t wave_col0) {
    base = base_;
    ld_b = ld_b_;
    k_limit = k_limit_;
    const uint32_t l = lane_id(), w = wave_id();
    constexpr uint32_t kChunks = kRowB / 16;  // 16-byte chunks per K row
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)kInstr; ++i) {
      const uint32_t q = w * kInstr + i;
      const uint32_t k = q * kRowsPerInstr + l / kChunks;
      const uint32_t j = (l % kChunks) ^ tr3_swz(k);
      krow[i] = k;
      const int32_t m0 = (int32_t)j * 8;
      moff[i] = m0 < m_valid ? (uint32_t)m0 * 2u : 0u;
    }
    const uint32_t g = l >> 4, L = l & 15u;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t k = 8 * g + 4 * h + (L >> 2);
      // fragment f sits at chunk c0 + 2 f + ((L & 3) >> 1), c0 = wave_col0 / 8; the
      // swizzle XORs chunk bits 1..3, so c0's low 4 bits join the XOR mask
      const uint32_t c0 = wave_col0 / 8u;
      fbase[h] = k * kRowB + ((c0 & ~15u) + ((L & 3u) >> 1)) * 16u + (L & 1u) * 8u;
      fxor[h] = (tr3_swz(k) ^ (c0 & 15u)) * 16u;
    }
  }
  __device__ __forceinline__ void issue(char* tile, int kt) const {
    const uint32_t w = wave_id();
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)kInstr; ++i) {
      int32_t k = kt * kBK3 + (int32_t)krow[i];
      k = k < k_limit ? k : k_limit - 1;
      __builtin_amdgcn_global_load_lds(base + (int64_t)k * ld_b + moff[i],
                                       (lds_void_t*)(tile + (w * kInstr + i) * 1024u), 16, 0, 0);
    }
  }
  // Two transposing reads into one 128-bit register tuple (inline asm; the
  // caller waits with tr_wait before use).
  __device__ __forceinline__ u32x4_t read(const char* tile, int f) const {
    const uint32_t t = lds_addr(tile);
    const u32x2_t lo = ds_read_tr_asm(t + fbase[0] + ((32u * (uint32_t)f) ^ fxor[0]));
    const u32x2_t hi = ds_read_tr_asm(t + fbase[1] + ((32u * (uint32_t)f) ^ fxor[1]));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
  }
};

template <class Op>
struct is_tr_op {
  static constexpr bool value = Op::kTrReads != 0;
};

// Wait for all LDS reads and make the fragment registers depend on it.
template <int N>
__device__ __forceinline__ void tr_wait(u32x4_t (&fr)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(fr[i]));
}

__device__ __forceinline__ void mfma_8x4(f32x4_t (&acc)[8][4], const u32x4_t (&fa)[8],
                                         const u32x4_t (&fb)[4]) {
#pragma unroll
  for (int fm = 0; fm < 8; ++fm)
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) acc[fm][fn] = mma_chunk<__bf16>(fb[fn], fa[fm], acc[fm][fn]);
}

// Stream of ntiles tiles of KT stages each; the DMA ring runs across tile
// boundaries.  retarget(tile) re-points the operands before the first load
// of a tile; epilogue(tile, acc) runs after a tile's last MFMA (it must not
// touch LDS and may only store to global memory).
template <class A, class B, class Retarget, class Epi>
__device__ __forceinline__ void mainloop3(char* lds, A& a, B& b, int KT, int ntiles,
                                          Retarget retarget, Epi epilogue) {
  constexpr int NS = kNS3;
  constexpr int kVm = A::kInstr + B::kInstr;  // DMA instructions per wave per stage
  const int total = KT * ntiles;
  if (total <= 0) return;
  auto issue = [&](int g) __attribute__((always_inline)) {
    const int tile = g / KT, kt = g - tile * KT;
    if (kt == 0) retarget(tile);
    char* st = lds + (g % NS) * kStage3;
    a.issue(st, kt);
    b.issue(st + kTileA3, kt);
  };
  wait_vmcnt<0>();
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < total) issue(p);

  int g = 0;
  for (int tile = 0; tile < ntiles; ++tile) {
    f32x4_t acc[8][4];
#pragma unroll
    for (int fm = 0; fm < 8; ++fm)
#pragma unroll
      for (int fn = 0; fn < 4; ++fn) acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kt = 0; kt < KT; ++kt, ++g) {
      // stage g landed: stages g + 1 .. min(g + NS - 2, total - 1) may stay in flight
      if (g + NS - 2 < total) wait_vmcnt<(NS - 2) * kVm>();
      else wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      if (g + NS - 1 < total) issue(g + NS - 1);
      const char* st = lds + (g % NS) * kStage3;
      u32x4_t fa[8], fb[4];
#pragma unroll
      for (int f = 0; f < 8; ++f) fa[f] = a.read(st, f);
#pragma unroll
      for (int f = 0; f < 4; ++f) fb[f] = b.read(st + kTileA3, f);
      if constexpr (is_tr_op<A>::value) tr_wait(fa);
      if constexpr (is_tr_op<B>::value) tr_wait(fb);
      mfma_8x4(acc, fa, fb);
    }
    epilogue(tile, acc);
  }
}

}  // namespace mtf
