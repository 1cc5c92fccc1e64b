// Operand loaders and the double-buffered MFMA main loop shared by every
// GEMM-shaped kernel of the fused linear + cross-entropy path.
#pragma once

#include "flce_device.h"

namespace mtf {

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint32_t wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// ---------------------------------------------------------------------------
// DirectLoader: operand whose rows are contiguous along K (row-major [R, K]).
// The 32 KiB tile is filled with 32 global_load_lds_dwordx4 instructions of
// 1 KiB each (8 per wave); lane i of an instruction lands at LDS byte
// base + 16 i, so the lane -> (row, chunk) assignment below is the inverse of
// tile_off().  Row addresses are resolved once (gathers included), then
// advanced by 128 bytes per K slab.
// ---------------------------------------------------------------------------
struct DirectLoader {
  const char* p[8];
  uint32_t tail_bad;  // bit i: load i's chunk lies past K in the last stage

  // Tile row handled by load instruction i of this lane.
  __device__ __forceinline__ static uint32_t row_of(uint32_t i) {
    uint32_t lane = lane_id(), w = wave_id();
    return (w * 4 + (i >> 1)) * 16 + ((lane >> 3) & 1u) * 8 + (i & 1u) * 4 + (lane >> 4);
  }
  __device__ __forceinline__ static uint32_t chunk_of(uint32_t i) {
    uint32_t lane = lane_id();
    return (lane & 7u) ^ ((i & 1u) * 4 + (lane >> 4));
  }

  // row_ptr(r) returns the byte address of K element 0 of tile row r.
  template <class RowPtr>
  __device__ __forceinline__ void init(RowPtr row_ptr) {
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) p[i] = row_ptr(row_of(i)) + chunk_of(i) * 16u;
  }

  __device__ __forceinline__ void issue(char* lds_tile, int kt) const {
    const uint32_t w = wave_id();
    const int64_t koff = (int64_t)kt * kRowBytes;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      __builtin_amdgcn_global_load_lds(p[i] + koff, (lds_void_t*)(lds_tile + (w * 8 + i) * 1024u),
                                       16, 0, 0);
    }
  }
  // c_lim: 16-byte chunks of the last K stage that lie below K.
  __device__ __forceinline__ void set_tail(uint32_t c_lim) {
    uint32_t m = 0;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) m |= (chunk_of(i) >= c_lim ? 1u : 0u) << i;
    tail_bad = m;
  }
  // The last (partial) K stage: chunks past K re-read chunk 0 of their row
  // (in bounds); the fragments holding them are zeroed after the LDS read.
  __device__ __forceinline__ void issue_tail(char* lds_tile, int kt) const {
    const uint32_t w = wave_id();
    const int64_t koff = (int64_t)kt * kRowBytes;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const char* src = ((tail_bad >> i) & 1u) ? p[i] - chunk_of(i) * 16u : p[i] + koff;
      __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds_tile + (w * 8 + i) * 1024u), 16, 0, 0);
    }
  }
  __device__ __forceinline__ void commit(char*) {}
};

// ---------------------------------------------------------------------------
// TransLoader: operand stored K-major (row-major [K, R], contiguous along the
// tile's row dimension).  Each thread loads KR K-rows x 16 bytes (one KR x KR
// block for bf16, two 4 x 4 blocks for fp32), transposes in registers
// (v_perm_b32 for bf16) and writes one 16-byte chunk per tile row.
// Thread t: kb = t & 7 (K block), mb = t >> 3 (row block).
// ---------------------------------------------------------------------------
template <typename T>
struct TransLoader {
  static constexpr int KR = Elt<T>::kPerChunk;  // K rows per block
  static constexpr int NB = 8 / KR;             // blocks per thread
  static constexpr int BK = Elt<T>::kBK;

  const char* base;    // byte address of K row 0, tile row 0
  int64_t ld_b;        // bytes between K rows
  int32_t k_limit;     // K rows >= k_limit are read from row k_limit - 1
  uint32_t m_off[NB];  // byte offset of this thread's 16-byte piece of each row
  uint32_t kb, mb;
  u32x4_t r[8];

  // m_valid: number of tile rows that exist in memory (pieces beyond it are
  // read from offset 0 and produce garbage that the epilogue discards).
  __device__ __forceinline__ void init(const char* base_, int64_t ld_b_, int32_t k_limit_,
                                       int32_t m_valid) {
    base = base_;
    ld_b = ld_b_;
    k_limit = k_limit_;
    kb = threadIdx.x & 7u;
    mb = threadIdx.x >> 3;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      int32_t m0 = (int32_t)((mb + 32u * b) * KR);
      m_off[b] = m0 < m_valid ? (uint32_t)(m0 * Elt<T>::kBytes) : 0u;
    }
  }

  __device__ __forceinline__ void issue(char*, int kt) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int i = 0; i < KR; ++i) {
        int32_t k = kt * BK + (int32_t)kb * KR + i;
        k = k < k_limit ? k : k_limit - 1;
        r[b * KR + i] = *reinterpret_cast<const u32x4_t*>(base + (int64_t)k * ld_b + m_off[b]);
      }
    }
  }

  __device__ __forceinline__ void commit(char* lds_tile);
};

template <>
__device__ __forceinline__ void TransLoader<__bf16>::commit(char* lds_tile) {
  // r[i] holds tile rows mb*8 .. mb*8+7 (2 per dword) of K row kb*8 + i.
  // Output row j = 2e + h takes half h of dword e of every r[i].
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t sel = h ? 0x07060302u : 0x05040100u;
      u32x4_t o;
      o.x = __builtin_amdgcn_perm(r[1][e], r[0][e], sel);
      o.y = __builtin_amdgcn_perm(r[3][e], r[2][e], sel);
      o.z = __builtin_amdgcn_perm(r[5][e], r[4][e], sel);
      o.w = __builtin_amdgcn_perm(r[7][e], r[6][e], sel);
      lds_write16(lds_tile, tile_off(mb * 8 + 2 * e + h, kb), o);
    }
  }
}

template <>
__device__ __forceinline__ void TransLoader<float>::commit(char* lds_tile) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t o;
      o.x = r[b * 4 + 0][j];
      o.y = r[b * 4 + 1][j];
      o.z = r[b * 4 + 2][j];
      o.w = r[b * 4 + 3][j];
      lds_write16(lds_tile, tile_off((mb + 32u * b) * 4 + j, kb), o);
    }
  }
}

// LDS byte offsets of this lane's fragment reads: kk selects the K half
// (chunks 0-3 or 4-7) of a slab; fragment f of the wave adds f * 2048.
struct FragOffsets {
  uint32_t a[2], b[2];
  __device__ __forceinline__ void init() {
    uint32_t lane = lane_id(), w = wave_id();
    uint32_t wm = w >> 1, wn = w & 1u;
    uint32_t ra = wm * 128 + (lane & 15u), rb = wn * 128 + (lane & 15u);
#pragma unroll
    for (uint32_t kk = 0; kk < 2; ++kk) {
      a[kk] = tile_off(ra, kk * 4 + (lane >> 4));
      b[kk] = tile_off(rb, kk * 4 + (lane >> 4));
    }
  }
};

// tail: the stage's 16-byte chunks at or past c_lim lie past K; lane l holds
// chunk kk * 4 + (l >> 4), zeroed in both operands when it does.
template <typename T>
__device__ __forceinline__ void compute_stage(const char* ldsA, const char* ldsB,
                                              f32x4_t (&acc)[8][8], const FragOffsets& fo,
                                              bool tail = false, uint32_t c_lim = 8) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    u32x4_t a[8], b[8];
#pragma unroll
    for (int f = 0; f < 8; ++f) a[f] = lds_read16(ldsA, fo.a[kk] + f * 2048u);
#pragma unroll
    for (int f = 0; f < 8; ++f) b[f] = lds_read16(ldsB, fo.b[kk] + f * 2048u);
    if (tail && (uint32_t)kk * 4u + (lane_id() >> 4) >= c_lim) {
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        a[f] = u32x4_t{0u, 0u, 0u, 0u};
        b[f] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int fm = 0; fm < 8; ++fm)
#pragma unroll
      for (int fn = 0; fn < 8; ++fn) acc[fm][fn] = mma_chunk<T>(b[fn], a[fm], acc[fm][fn]);
  }
}

// C_tile[256 x 256] = sum over KT slabs of A_tile * B_tile^T, fp32 in acc.
// kKTail (both loaders DirectLoader): the last slab holds only c_lim of its
// 8 chunks below K (DirectLoader::issue_tail, compute_stage's mask).
template <typename T, bool kKTail = false, class LA, class LB>
__device__ __forceinline__ void mainloop(char* lds, f32x4_t (&acc)[8][8], LA& la, LB& lb, int KT,
                                         const FragOffsets& fo, uint32_t c_lim = 8) {
#pragma unroll
  for (int fm = 0; fm < 8; ++fm)
#pragma unroll
    for (int fn = 0; fn < 8; ++fn) acc[fm][fn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (KT <= 0) return;

  if constexpr (kKTail) {
    if (KT == 1) {
      la.issue_tail(lds, 0);
      lb.issue_tail(lds + kTileBytes, 0);
    } else {
      la.issue(lds, 0);
      lb.issue(lds + kTileBytes, 0);
    }
  } else {
    la.issue(lds, 0);
    lb.issue(lds + kTileBytes, 0);
  }
  la.commit(lds);
  lb.commit(lds + kTileBytes);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    char* cur = lds + (kt & 1) * kStageBytes;
    char* nxt = lds + ((kt + 1) & 1) * kStageBytes;
    const bool more = kt + 1 < KT;
    if (more) {
      if (kKTail && kt + 1 == KT - 1) {
        if constexpr (kKTail) {
          la.issue_tail(nxt, kt + 1);
          lb.issue_tail(nxt + kTileBytes, kt + 1);
        }
      } else {
        la.issue(nxt, kt + 1);
        lb.issue(nxt + kTileBytes, kt + 1);
      }
    }
    compute_stage<T>(cur, cur + kTileBytes, acc, fo, kKTail && kt == KT - 1, c_lim);
    if (more) {
      la.commit(nxt);
      lb.commit(nxt + kTileBytes);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
}

}  // namespace mtf
