// Device-side building blocks of the fused linear + cross-entropy kernels
// (gfx950 / CDNA4 only).
//
// Tiling
//   A workgroup is 256 threads = 4 waves of 64 and owns a 256 x 256 output
//   tile.  Wave w owns the 128 x 128 quadrant (wm = w / 2, wn = w % 2).  The
//   contraction runs in steps of one 128-byte K slab (64 bf16 or 32 fp32),
//   double-buffered in LDS: 2 stages x (A tile + B tile) x 32 KiB = 128 KiB
//   of the 160 KiB LDS, one workgroup per CU.
//
// LDS tile layout
//   A tile holds 256 rows x 128 bytes of K.  A row is 8 chunks of 16 bytes.
//   Rows r and r + 8 of a 16-row group share one 256-byte line (halves 0/1);
//   the chunk index is XOR-swizzled with (r & 7).  With this layout the
//   16-lane groups of an MFMA operand read (16 consecutive rows, one chunk)
//   and the 8-lane / 16-lane groups of every writer below touch distinct
//   16-byte slots of a 256-byte window, so neither 32- nor 64-bank LDS
//   organisations see conflicts on ds_read_b128 / ds_write_b128.
//
// Accumulator layout (v_mfma_f32_16x16x32_bf16 with the B fragment issued
// as the MFMA's first operand): lane l of a wave holds, for fragment
// (fm, fn), four consecutive output columns of one output row:
//   row = wm*128 + fm*16 + (l & 15),  col = wn*128 + fn*16 + 4*(l >> 4) + r.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kThreads = 256;
constexpr int kTileRows = 256;
constexpr int kRowBytes = 128;
constexpr int kTileBytes = kTileRows * kRowBytes;  // 32 KiB
constexpr int kStageBytes = 2 * kTileBytes;        // A + B
constexpr int kLdsBytes = 2 * kStageBytes;         // double buffered

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegBig = -1.0e30f;  // "minus infinity" that keeps exp2(a - b) finite

template <typename T>
struct Elt;
template <>
struct Elt<__bf16> {
  static constexpr int kBytes = 2;
  static constexpr int kPerChunk = 8;  // elements per 16-byte chunk
  static constexpr int kBK = 64;       // K elements per LDS stage
};
template <>
struct Elt<float> {
  static constexpr int kBytes = 4;
  static constexpr int kPerChunk = 4;
  static constexpr int kBK = 32;
};

// Byte offset of (row, logical 16-byte chunk) inside one 256-row tile.
__device__ __forceinline__ uint32_t tile_off(uint32_t row, uint32_t chunk) {
  return ((row >> 4) << 11) | ((row & 7u) << 8) | (((row >> 3) & 1u) << 7) |
         (((chunk ^ row) & 7u) << 4);
}

__device__ __forceinline__ u32x4_t lds_read16(const char* lds, uint32_t off) {
  return *reinterpret_cast<const u32x4_t*>(lds + off);
}
__device__ __forceinline__ void lds_write16(char* lds, uint32_t off, u32x4_t v) {
  *reinterpret_cast<u32x4_t*>(lds + off) = v;
}

// One 16-byte chunk of A and of B per lane -> 16x16 fp32 fragment update.
// bf16: one v_mfma_f32_16x16x32_bf16.  fp32: four v_mfma_f32_16x16x4_f32
// (element j of every lane's chunk is one K column of the j-th MFMA; A and
// B use the same pairing, so the sum over K is unchanged).
template <typename T>
__device__ __forceinline__ f32x4_t mma_chunk(u32x4_t a, u32x4_t b, f32x4_t c);

template <>
__device__ __forceinline__ f32x4_t mma_chunk<__bf16>(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mma_chunk<float>(u32x4_t a, u32x4_t b, f32x4_t c) {
  // Bit-cast whole vectors, then index: a bit-cast of a single vector element
  // (e.g. __builtin_bit_cast(float, a.y)) is read from element 0 by this
  // compiler.
  const f32x4_t af = __builtin_bit_cast(f32x4_t, a), bf = __builtin_bit_cast(f32x4_t, b);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], c, 0, 0, 0);
  return c;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair (v_cvt_pk_bf16_f32: round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// Values of (lo, hi) after a round trip through the storage type T.
template <typename T>
__device__ __forceinline__ void round_pair(float& lo, float& hi);
template <>
__device__ __forceinline__ void round_pair<__bf16>(float& lo, float& hi) {
  const uint32_t p = pack_bf16x2(lo, hi);
  lo = __builtin_bit_cast(float, p << 16);
  hi = __builtin_bit_cast(float, p & 0xffff0000u);
}
template <>
__device__ __forceinline__ void round_pair<float>(float&, float&) {}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// tanh(x) from exp2: 1 - 2 / (exp(2|x|) + 1), sign restored.
__device__ __forceinline__ float tanh_approx(float x) {
  float ax = fabsf(x);
  float e = fast_exp2(ax * (2.0f * kLog2e));
  float t = 1.0f - 2.0f / (e + 1.0f);
  return copysignf(t, x);
}

// Online log-sum-exp state merge in the log2 domain: (m, d) represents
// d * 2^m.
__device__ __forceinline__ void lse_merge(float& m, float& d, float m2, float d2) {
  float mn = fmaxf(m, m2);
  d = d * fast_exp2(m - mn) + d2 * fast_exp2(m2 - mn);
  m = mn;
}

// Workgroup id -> logical tile id such that the workgroups resident on one
// XCD (hardware dispatches id i to XCD i % 8) get a contiguous logical range.
// A bijection of [0, nwg) for any nwg: XCD x < nwg % 8 owns one id more than
// the others, and the ranges are laid out XCD after XCD.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t nwg) {
  const uint32_t kXcd = 8;
  const uint32_t q = nwg / kXcd, r = nwg % kXcd;
  const uint32_t x = bid % kXcd, i = bid / kXcd;
  return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

// Logical tile id -> (tile_m, tile_n) walking groups of `group_m` tile rows
// column by column, so concurrently running tiles share operand panels.
__device__ __forceinline__ void grouped_tile(uint32_t lid, uint32_t tiles_m, uint32_t tiles_n,
                                             uint32_t group_m, uint32_t& tm, uint32_t& tn) {
  uint32_t per_group = group_m * tiles_n;
  uint32_t g = lid / per_group;
  uint32_t first_m = g * group_m;
  uint32_t gm = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  uint32_t in = lid - g * per_group;
  tm = first_m + in % gm;
  tn = in / gm;
  // lid is uniform (a workgroup's tile index), but the divisions above run
  // in vector registers and the compiler does not always prove the results
  // uniform; a pointer or buffer resource built from them then becomes a
  // per-lane waterfall loop around every memory instruction that uses it.
  tm = __builtin_amdgcn_readfirstlane(tm);
  tn = __builtin_amdgcn_readfirstlane(tn);
}

}  // namespace mtf
