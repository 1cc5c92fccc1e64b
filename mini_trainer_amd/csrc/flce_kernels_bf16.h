// bf16 kernels on the four-wave main loop (flce_gemm_bf16.h): output tiles
// of 256 x 256, wave tiles 128 x 128.  Arguments, accumulation order and
// epilogues are those of the generic kernels in flce_kernels.h (the fp32
// path).
#pragma once

#include "flce_gemm_bf16.h"
#include "flce_kernels.h"

namespace mtf {

#define MT_GEMM_BF16_KERNEL \
  __global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))

// Cache policy of streamed accesses (the tiled dW's read-modify-write and
// the narrowing pass over it): non-temporal, streamed past the caches that
// hold the GEMM operand panels.  (The chunk's exponentials stored so were
// slower to write: forward +1.2%.)
constexpr int kCpolNt = 2;

// Wave (wm, wn) of the 2 x 2 wave grid, 8 x 8 fragments each.
typedef EpiCoordsT<8, 2> EpiCoordsBf;

// A copy of the wave coordinates that the compiler cannot treat as invariant
// across the persistent tile loop: an epilogue's per-lane address arithmetic
// is then formed inside the epilogue instead of being hoisted out of the
// loop and spilled across the main loop.
__device__ __forceinline__ EpiCoordsBf fresh(const EpiCoordsBf& ec) {
  EpiCoordsBf e = ec;
  asm volatile("" : "+v"(e.lane));
  return e;
}

// Persistent schedule of the single-pass GEMM kernels: the grid holds
// P <= #tiles workgroups (one per CU) and workgroup b takes the logical tiles
// k * P + xcd_remap(b, P), k = 0, 1, ...  In every round the workgroups of one
// XCD therefore hold a contiguous logical range (neighbouring tiles share
// operand panels in that XCD's L2), and a tile's epilogue overlaps the first
// operand loads of the workgroup's next tile.
struct TileSeq {
  uint32_t first, stride, total;
  __device__ __forceinline__ explicit TileSeq(uint32_t total_) : total(total_) {
    stride = gridDim.x;
    first = xcd_remap(blockIdx.x, gridDim.x);
  }
  // workgroup b of nb (a launch that also holds other work)
  __device__ __forceinline__ TileSeq(uint32_t total_, uint32_t b, uint32_t nb) : total(total_) {
    stride = nb;
    first = xcd_remap(b, nb);
  }
  __device__ __forceinline__ int count() const {
    return first < total ? (int)((total - first + stride - 1) / stride) : 0;
  }
  __device__ __forceinline__ uint32_t logical(int k) const { return first + (uint32_t)k * stride; }
};

// Forward: one 256 x 256 logits tile per work unit (A = gathered X rows, B =
// W rows), persistent over the (row tile, vocabulary tile) grid.  The
// epilogue reduces the tile to a (max, sum) partial per row -- lanes that
// share a row through shuffles, the two wave columns through 2 KiB of the
// ring slot the main loop hands to the epilogue -- and writes it to
// part[vocab tile][row];
// the lane that holds a row's label logit writes it to xy[row].  Nothing is
// carried in registers from one tile to the next.
// kStore = kStoreLogits: the tile's bf16-rounded logits (before the softcap)
// are also written to S, row = compacted row of the chunk, column =
// vocabulary index, and the fused path forms G from them in place once the
// row's lse is known.  kStore = kStoreExp: S receives E = exp(z) (1 - (z /
// cap)^2) instead, z the soft-capped logit (fwd_epilogue_exp_bf16): G is
// then s E with a per-row factor s applied downstream (see
// fused_row_scale_kernel), which saves the pass over S that forms G.
// Row tiles per group of the forward's tile walk: W (the larger operand) is
// streamed once per group, so wider groups cut its re-reads.  Up to 12 row
// tiles walk as one group, more in groups of 8.  Measured in same-box
// rotations: 8 against 4, 2% faster at config 3; a config-3 chunk's 12 row
// tiles as one group, a further 0.4% against 8 and 6; config 5's 26 row
// tiles in groups of 12, 0.8% slower than in groups of 8; config 4's 23
// the same in groups of 8, 12 and 16.
__device__ __forceinline__ uint32_t fwd_group(uint32_t tiles_m) { return tiles_m <= 12u ? tiles_m : 8u; }

// Forward tile epilogue of the bf16 kernels, one fragment row fm at a time
// (a scheduling fence after each keeps a single row group's values in
// registers; the unrolled whole-tile form spilled): the lane's 32 logits of
// the row are rounded to bf16 once, stored to S (kStore = kStoreLogits,
// before the softcap), soft-capped, masked past V, merged into the row's
// running (max, sum) and scanned for the label (same arithmetic as
// fwd_tile_epilogue).
enum FwdStore : int { kStoreNone = 0, kStoreLogits = 1, kStoreExp = 2 };
template <bool kCap, int kStore, bool kTail>
__device__ __forceinline__ void fwd_epilogue_bf16(const f32x4_t (&acc)[8][8], float (&m2)[8],
                                                  float (&d)[8], const int32_t (&lbl)[8],
                                                  const int32_t (&rglob)[8], int32_t vrow0,
                                                  const EpiCoordsBf& ec, const FwdArgs& a) {
  // vrow0: the tile's first column from W's row 0; labels and S columns are
  // global vocabulary indices (a.vcol0 + local)
  const int32_t lcol0 = vrow0 + ec.col(0);
  const int32_t ncol0 = a.vcol0 + lcol0;
  int32_t rel[8];
  bool hit = false;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    rel[fm] = lbl[fm] - ncol0;
    hit |= lane_holds<8>(rel[fm]);
  }
  const bool any_hit = __builtin_amdgcn_ballot_w64(hit) != 0;
  const float cap = a.softcap, inv_cap = kCap ? 1.0f / a.softcap : 0.f;
  // S stores go through one buffer resource at the chunk base (the planner
  // keeps the chunk below 4 GiB): a 32-bit row offset per fragment row and
  // the fragment pair as a constant.  A lane holds 4 consecutive columns of
  // each fragment (8 bytes); one v_permlane16_swap per dword pairs fragments
  // fn = 2p, 2p + 1 so that lane group q (= lane / 16) holds 8 consecutive
  // columns, 8 (2 (q & 1) + (q >> 1)) + 32 p, for one 16-byte store: half the
  // store instructions, each writing 64 contiguous bytes per row instead of
  // 32 (the store pipeline's cost goes with instructions x rows touched).
  constexpr bool kStoreS = kStore == kStoreLogits;
  const rsrc_t srs = make_rsrc(kStoreS ? static_cast<const void*>(a.S) : a.xy,
                               kStoreS ? a.s_range : 0u);
  const uint32_t q = ec.lane >> 4;
  const uint32_t scol = (uint32_t)(a.vcol0 + vrow0) + ec.wn * 128u + 8u * (2u * (q & 1u) + (q >> 1));
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    // vocabulary columns of this lane below V, re-formed per fragment row
    // through an empty asm so that the 32 compares are not hoisted out of
    // the row loop (their masks spilled from the scalar registers)
    int32_t lim = a.V - lcol0;
    if (kTail) asm volatile("" : "+v"(lim));
    float v[8][4];
    uint32_t slo[8], shi[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int fn = 0; fn < 8; ++fn) {
      const uint32_t lo = pack_bf16x2(acc[fm][fn][0], acc[fm][fn][1]);
      const uint32_t hi = pack_bf16x2(acc[fm][fn][2], acc[fm][fn][3]);
      slo[fn] = lo;
      shi[fn] = hi;
      v[fn][0] = __builtin_bit_cast(float, lo << 16);
      v[fn][1] = __builtin_bit_cast(float, lo & 0xffff0000u);
      v[fn][2] = __builtin_bit_cast(float, hi << 16);
      v[fn][3] = __builtin_bit_cast(float, hi & 0xffff0000u);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = v[fn][r];
        if (kCap) x = cap * tanh_approx(x * inv_cap);
        if (kTail) x = fn * 16 + r < lim ? x : -INFINITY;
        v[fn][r] = x;
        tmax = fmaxf(tmax, x);
      }
    }
    if (kStoreS) {
      const uint32_t soff = (uint32_t)rglob[fm] * (uint32_t)a.lds_b + scol * 2u;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const auto l2 = __builtin_amdgcn_permlane16_swap(slo[2 * p], slo[2 * p + 1], false, false);
        const auto h2 = __builtin_amdgcn_permlane16_swap(shi[2 * p], shi[2 * p + 1], false, false);
        u32x4_t o;
        o[0] = l2[0];
        o[1] = h2[0];
        o[2] = l2[1];
        o[3] = h2[1];
        __builtin_amdgcn_raw_buffer_store_b128(o, srs, soff + (uint32_t)p * 64u, 0, 0);
      }
    }
    const float mn = fmaxf(m2[fm], tmax * kLog2e);
    float sum = 0.f;
#pragma unroll
    for (int fn = 0; fn < 8; ++fn)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += fast_exp2(fmaf(v[fn][r], kLog2e, -mn));
    d[fm] = fmaf(d[fm], fast_exp2(m2[fm] - mn), sum);
    m2[fm] = mn;
    if (any_hit) {
      const int rl = rel[fm];
      if (lane_holds<8>(rl) && rglob[fm] < a.N) {
        float hitv = 0.f;
#pragma unroll
        for (int fn = 0; fn < 8; ++fn)
#pragma unroll
          for (int r = 0; r < 4; ++r) hitv = (rl == fn * 16 + r) ? v[fn][r] : hitv;
        a.xy[rglob[fm]] = hitv;
      }
    }
    sched_fence();
  }
}

// Forward tile epilogue with kStore = kStoreExp, two passes per fragment row
// over the row's bf16-rounded logits, held packed in 16 registers rather
// than as 32 floats.  Pass 1 finds the lane's row maximum of the
// soft-capped, masked logits; pass 2 re-forms each logit x, adds
// exp2(x log2e - max) to the row's sum and stores E = exp2(x log2e)
// (1 - (x / cap)^2) through the same paired 16-byte stores as the logits,
// half a row per fenced group.  E takes a
// second exponential rather than the sum's term times exp2(max): that extra
// per-row factor, live across the half rows, pushed the register allocator
// into spilling the main loop's DMA offsets (a scratch reload and a full
// vmcnt wait in every K stage), as did the float form of the logits.
// Columns past V give E = 0; rows past N repeat row N - 1's values (the
// gather clamps the row index) and meet zero rows of the gathered X^T.  The
// label's logit is scanned in the (rare) branch of the wave that holds it.
template <bool kCap, bool kTail>
__device__ __forceinline__ void fwd_epilogue_exp_bf16(const f32x4_t (&acc)[8][8], float (&m2)[8],
                                                      float (&d)[8], const int32_t (&lbl)[8],
                                                      const int32_t (&rglob)[8], int32_t vrow0,
                                                      const EpiCoordsBf& ec, const FwdArgs& a) {
  const int32_t lcol0 = vrow0 + ec.col(0);
  const int32_t ncol0 = a.vcol0 + lcol0;
  int32_t rel[8];
  bool hit = false;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    rel[fm] = lbl[fm] - ncol0;
    hit |= lane_holds<8>(rel[fm]);
  }
  const bool any_hit = __builtin_amdgcn_ballot_w64(hit) != 0;
  const float cap = a.softcap, inv_cap = kCap ? 1.0f / a.softcap : 0.f;
  const rsrc_t srs = make_rsrc(a.S, a.s_range);
  const uint32_t q = ec.lane >> 4;
  const uint32_t scol = (uint32_t)(a.vcol0 + vrow0) + ec.wn * 128u + 8u * (2u * (q & 1u) + (q >> 1));
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    int32_t lim = a.V - lcol0;
    if (kTail) asm volatile("" : "+v"(lim));
    // logit r of fragment fn from the packed pair, soft-capped and masked;
    // dz = the softcap's derivative
    uint32_t slo[8], shi[8];
    auto logit = [&](int fn, int r, float& dz) __attribute__((always_inline)) {
      const uint32_t w = r < 2 ? slo[fn] : shi[fn];
      float x = __builtin_bit_cast(float, (r & 1) ? (w & 0xffff0000u) : (w << 16));
      dz = 1.f;
      if (kCap) {
        const float t = tanh_approx(x * inv_cap);
        x = cap * t;
        dz = fmaf(-t, t, 1.f);
      }
      if (kTail) x = fn * 16 + r < lim ? x : -INFINITY;
      return x;
    };
    float tmax = -INFINITY;
#pragma unroll
    for (int fn = 0; fn < 8; ++fn) {
      slo[fn] = pack_bf16x2(acc[fm][fn][0], acc[fm][fn][1]);
      shi[fn] = pack_bf16x2(acc[fm][fn][2], acc[fm][fn][3]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float dz;
        tmax = fmaxf(tmax, logit(fn, r, dz));
      }
    }
    if (any_hit) {
      const int rl = rel[fm];
      if (lane_holds<8>(rl) && rglob[fm] < a.N) {
        float hitv = 0.f;
#pragma unroll
        for (int fn = 0; fn < 8; ++fn)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float dz;
            hitv = (rl == fn * 16 + r) ? logit(fn, r, dz) : hitv;
          }
        a.xy[rglob[fm]] = hitv;
      }
    }
    const float mn = fmaxf(m2[fm], tmax * kLog2e);
    const uint32_t soff = (uint32_t)rglob[fm] * (uint32_t)a.lds_b + scol * 2u;
    float sum = 0.f;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      uint32_t plo[4], phi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int fn = 4 * hh + j;
        float e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float dz;
          const float x = logit(fn, r, dz);
          const float t = fast_exp2(fmaf(x, kLog2e, -mn));
          sum += t;
          const float ex = fast_exp2(x * kLog2e);
          e[r] = kCap ? ex * dz : ex;
        }
        plo[j] = pack_bf16x2(e[0], e[1]);
        phi[j] = pack_bf16x2(e[2], e[3]);
      }
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const auto l2 = __builtin_amdgcn_permlane16_swap(plo[2 * pp], plo[2 * pp + 1], false, false);
        const auto h2 = __builtin_amdgcn_permlane16_swap(phi[2 * pp], phi[2 * pp + 1], false, false);
        u32x4_t o;
        o[0] = l2[0];
        o[1] = h2[0];
        o[2] = l2[1];
        o[3] = h2[1];
        __builtin_amdgcn_raw_buffer_store_b128(o, srs, soff + (uint32_t)(2 * hh + pp) * 64u, 0, 0);
      }
      sched_fence();
    }
    d[fm] = fmaf(d[fm], fast_exp2(m2[fm] - mn), sum);
    m2[fm] = mn;
    sched_fence();
  }
}

// Forward body over ntiles logits tiles; map(k, tm, tv) gives tile k's row
// tile and vocabulary tile.  kTail: the tiles have columns past V (the
// epilogue masks them).
template <bool kCap, int kStore, bool kTail, bool kKTail, class Map>
__device__ __forceinline__ void fwd_bf16_body(char* lds, const FwdArgs& a, int ntiles, Map map) {
  const EpiCoordsBf ec0;
  const int KT = (a.H + kBKBf - 1) / kBKBf;
  const uint32_t c_lim = (uint32_t)(a.H - (KT - 1) * kBKBf) / 8u;
  KcOp A, B;
  A.init_frag(ec0.wm * 128);
  B.init_frag(ec0.wn * 128);
  if constexpr (kKTail) {
    A.set_tail(c_lim);
    B.set_tail(c_lim);
  }
  mainloop_bf16<false, kKTail>(
      lds, A, B, KT, ntiles,
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tv;
        map(k, tm, tv);
        const int32_t row0 = (int32_t)tm * 256, vrow0 = (int32_t)tv * 256;
        A.set_rows(make_rsrc(a.X, a.x_range), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t rr = row0 + (int32_t)r;
          rr = rr < a.N ? rr : a.N - 1;
          return (uint32_t)a.row_index[rr] * (uint32_t)a.ldx_b;
        });
        B.set_rows(make_rsrc(a.W, a.w_range), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t v = vrow0 + (int32_t)r;
          v = v < a.V ? v : a.V - 1;
          return (uint32_t)v * (uint32_t)a.ldw_b;
        });
      },
      [&](int k, f32x4_t(&acc)[8][8], char* scratch) __attribute__((always_inline)) {
        const EpiCoordsBf ec = fresh(ec0);
        uint32_t tm, tv;
        map(k, tm, tv);
        const int32_t row0 = (int32_t)tm * 256;
        int32_t rglob[8], lbl[8];
        float m2[8], d[8];
#pragma unroll
        for (int fm = 0; fm < 8; ++fm) {
          rglob[fm] = row0 + ec.row(fm);
          lbl[fm] = rglob[fm] < a.N ? a.row_label[rglob[fm]] : -1;
          m2[fm] = kNegBig;
          d[fm] = 0.f;
        }
        if constexpr (kStore == kStoreExp)
          fwd_epilogue_exp_bf16<kCap, kTail>(acc, m2, d, lbl, rglob, (int32_t)tv * 256, ec, a);
        else
          fwd_epilogue_bf16<kCap, kStore, kTail>(acc, m2, d, lbl, rglob, (int32_t)tv * 256, ec, a);
        fwd_final_merge(scratch, m2, d, rglob, (uint32_t)a.vcol0 / 256u + tv, ec, a);
        // the merge's LDS is the ring slot refilled in the next phase 1
        __syncthreads();
      },
      ZeroInit(), c_lim);
}

// kTail: V is not a multiple of 256.  Only the last vocabulary tile column
// has columns past V, and only its tiles take the masked epilogue, in a
// tile loop of their own (a select per logit in every tile cost 10k cycles
// per tile, measured, and the masked and unmasked epilogues in one tile loop
// spilled): the persistent schedule covers the full columns, and the
// workgroups that get one full tile fewer in it (their logical start lies
// in [r, r + tiles_m), r = full tiles mod grid) each run one tile of the
// last column first (rel, rel + grid, ... when tiles_m exceeds the grid).
// kKTail: H is not a multiple of 64, so the last K stage is partial.
// run_if (non-null): the launch does nothing unless *run_if != 0 (the fused
// path's recomputation of a chunk whose exponentials are out of range);
// guard_reset (non-null): set to 0 (its readers run after this launch).
template <bool kCap, int kStore, bool kTail, bool kKTail>
MT_GEMM_BF16_KERNEL void fwd_bf16_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBf];
  if (a.run_if && *a.run_if == 0) return;
  if (a.guard_reset && blockIdx.x == 0 && threadIdx.x == 0) *a.guard_reset = 0;
  const uint32_t vt_full = (uint32_t)a.vt_total - (kTail ? 1u : 0u);
  const TileSeq seq((uint32_t)a.tiles_m * vt_full);
  if constexpr (kTail) {
    const uint32_t P = gridDim.x, r = seq.total % P;
    const uint32_t rel = seq.first >= r ? seq.first - r : seq.first + P - r;
    const uint32_t tm_n = (uint32_t)a.tiles_m;
    if (rel < tm_n) {
      fwd_bf16_body<kCap, kStore, true, kKTail>(
          lds, a, (int)((tm_n - rel + P - 1) / P),
          [&](int k, uint32_t& tm, uint32_t& tv) __attribute__((always_inline)) {
            tm = rel + (uint32_t)k * P;
            tv = vt_full;
          });
      __syncthreads();
    }
  }
  fwd_bf16_body<kCap, kStore, false, kKTail>(
      lds, a, seq.count(), [&](int k, uint32_t& tm, uint32_t& tv) __attribute__((always_inline)) {
        grouped_tile(seq.logical(k), a.tiles_m, vt_full, fwd_group((uint32_t)a.tiles_m), tm, tv);
      });
}

// Backward recompute epilogue of the bf16 kernel, one fragment row at a
// time: G = g (softmax - onehot), times 1 - tanh^2 under softcap, with the
// arithmetic of recompute_epilogue.  G is written as the fused forward
// writes S: v_permlane16_swap pairs fragments fn = 2p, 2p + 1 so that each
// lane stores 8 consecutive columns in one 16-byte store, through one buffer
// resource at the block's G base (the planner keeps G below 4 GiB).  G holds
// whole tiles; rows past Cn and (kTail: cv is not a multiple of 256) columns
// past cv are written as zeros.
template <bool kCap, bool kTail>
__device__ __forceinline__ void recompute_epilogue_bf16(const f32x4_t (&acc)[8][8],
                                                        const RecompArgs& a, const EpiCoordsBf& ec,
                                                        int32_t row0, int32_t col0) {
  const float cap = a.softcap, inv_cap = kCap ? 1.0f / a.softcap : 0.f;
  const int32_t ncol0 = col0 + ec.col(0);  // block-local column of fn = 0, r = 0
  int32_t rel[8], rowl[8];
  float lse2[8], g[8];
  bool hit = false;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    rowl[fm] = row0 + ec.row(fm);
    const bool rv = rowl[fm] < a.Cn;
    const int32_t rr = rv ? rowl[fm] : 0;
    lse2[fm] = a.lse[rr] * kLog2e;
    g[fm] = rv ? a.grad[(int64_t)a.row_index[rr] * a.gstride] : 0.f;
    rel[fm] = rv ? a.row_label[rr] - a.v0 - ncol0 : -1;
    hit |= lane_holds<8>(rel[fm]);
  }
  const bool any_hit = __builtin_amdgcn_ballot_w64(hit) != 0;
  const rsrc_t grs = make_rsrc(a.G, a.g_range);
  const uint32_t q = ec.lane >> 4;
  const uint32_t gcol = (uint32_t)col0 + ec.wn * 128u + 8u * (2u * (q & 1u) + (q >> 1));
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const bool rv = rowl[fm] < a.Cn;
    // columns this lane may write, re-formed per fragment row through an
    // empty asm: otherwise the 32 column compares are hoisted out of the row
    // loop and their masks spill from the scalar registers
    int32_t lim = a.cv - ncol0;
    if (kTail) asm volatile("" : "+v"(lim));
    uint32_t glo[8], ghi[8];
#pragma unroll
    for (int fn = 0; fn < 8; ++fn) {
      float xr[4] = {acc[fm][fn][0], acc[fm][fn][1], acc[fm][fn][2], acc[fm][fn][3]};
      round_pair<__bf16>(xr[0], xr[1]);
      round_pair<__bf16>(xr[2], xr[3]);
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = xr[r];
        float dcap = 1.f;
        if (kCap) {
          const float t = tanh_approx(x * inv_cap);
          x = cap * t;
          dcap = 1.f - t * t;
        }
        float p = fast_exp2(fmaf(x, kLog2e, -lse2[fm]));
        if (any_hit) p -= (rel[fm] == fn * 16 + r) ? 1.f : 0.f;
        const bool ok = kTail ? rv && (fn * 16 + r < lim) : rv;
        o[r] = ok ? p * g[fm] * dcap : 0.f;
      }
      glo[fn] = pack_bf16x2(o[0], o[1]);
      ghi[fn] = pack_bf16x2(o[2], o[3]);
    }
    const uint32_t goff = (uint32_t)rowl[fm] * (uint32_t)a.ldg_b + gcol * 2u;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const auto l2 = __builtin_amdgcn_permlane16_swap(glo[2 * p], glo[2 * p + 1], false, false);
      const auto h2 = __builtin_amdgcn_permlane16_swap(ghi[2 * p], ghi[2 * p + 1], false, false);
      u32x4_t o;
      o[0] = l2[0];
      o[1] = h2[0];
      o[2] = l2[1];
      o[3] = h2[1];
      __builtin_amdgcn_raw_buffer_store_b128(o, grs, goff + (uint32_t)p * 64u, 0, 0);
    }
    sched_fence();
  }
}

// Backward step 1: A = X rows of the block (256 tokens), B = W rows (256
// vocabulary entries); the epilogue writes G.  kTail: the block's vocabulary
// width cv is not a multiple of 256 (only the last block, and only when V is
// not), so its last tile masks the columns past cv.
template <bool kCap, bool kTail, bool kKTail>
MT_GEMM_BF16_KERNEL void recompute_bf16_kernel(RecompArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBf];
  if (a.zero_words && blockIdx.x == 0 && threadIdx.x < (uint32_t)kQueueWords)
    a.zero_words[threadIdx.x] = 0u;
  if (a.run_if && *a.run_if == 0) return;
  const TileSeq seq((uint32_t)(a.tiles_m * a.tiles_n));
  const EpiCoordsBf ec0;
  const int KT = (a.H + kBKBf - 1) / kBKBf;
  const uint32_t c_lim = (uint32_t)(a.H - (KT - 1) * kBKBf) / 8u;
  KcOp A, B;
  A.init_frag(ec0.wm * 128);
  B.init_frag(ec0.wn * 128);
  if constexpr (kKTail) {
    A.set_tail(c_lim);
    B.set_tail(c_lim);
  }
  mainloop_bf16<false, kKTail>(
      lds, A, B, KT, seq.count(),
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        // W points at the block's first vocabulary row (v0)
        const int32_t row0 = (int32_t)tm * 256, vloc0 = (int32_t)tn * 256;
        A.set_rows(make_rsrc(a.X, a.x_range), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t rr = row0 + (int32_t)r;
          rr = rr < a.Cn ? rr : a.Cn - 1;
          return (uint32_t)a.row_index[rr] * (uint32_t)a.ldx_b;
        });
        B.set_rows(make_rsrc(a.W, a.w_range), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t v = vloc0 + (int32_t)r;
          v = v < a.cv ? v : a.cv - 1;  // rows past the block repeat its last one
          return (uint32_t)v * (uint32_t)a.ldw_b;
        });
      },
      [&](int k, f32x4_t(&acc)[8][8], char* scratch) __attribute__((always_inline)) {
        const EpiCoordsBf ec = fresh(ec0);
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t row0 = (int32_t)tm * 256, col0 = (int32_t)tn * 256;
        recompute_epilogue_bf16<kCap, kTail>(acc, a, ec, row0, col0);
      },
      ZeroInit(), c_lim);
}

// dX tile epilogue of the bf16 kernels (one mode of dx_epilogue per
// instantiation: a kernel holding all four spilled accumulators), half a
// fragment row at a time: bounds checks guard single stores, and a scheduling
// fence after each half row -- in uniform control flow -- keeps one group's
// values in registers.
// kMode >= kDxTiledAcc: the accumulator of tile (row0, h0) is one 256 KiB
// tile in the accumulators' own order (the wave's 64 KiB, fragment (fm, fn)
// at (fm * 8 + fn) KiB of it, the lane's 16 bytes at lane * 16), so every
// load and store covers one contiguous KiB.  Rows past Cn are neither
// stored nor emitted (their accumulators are never read); the control flow
// is that of the row-major modes (with unconditional stores the compiler
// spilled the main loop's registers).
template <int kMode>
__device__ __forceinline__ void dx_epilogue_tiled_acc(const f32x4_t (&acc)[8][8], const DxArgs& a,
                                                      const EpiCoordsBf& ec, int32_t row0,
                                                      int32_t h0) {
  constexpr int kM = kMode - kDxTiledAcc;
  const int64_t tile = (int64_t)(row0 / 256) * a.tiles_n + h0 / 256;
  float* const base =
      a.accbuf + tile * 65536 + (int64_t)((ec.wm * 2u + ec.wn) * 16384u + ec.lane * 4u);
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const int32_t rowl = row0 + ec.row(fm);
    const bool rv = rowl < a.Cn;
    char* xrow = kM == kDxAddEmit ? a.dX + (int64_t)a.row_index[rv ? rowl : 0] * a.lddx_b : nullptr;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int fn = 4 * half + q;
        const int32_t h = h0 + ec.col(fn);
        float* const slot = base + (fm * 8 + fn) * 256;
        f32x4_t v = acc[fm][fn];
        if (rv && h < a.H) {
          if (kM == kDxAdd || kM == kDxAddEmit)
            v += __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(slot));
          if (kM <= kDxAdd) {
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t*>(slot));
          } else {
            u32x2_t o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<u32x2_t*>(xrow + (int64_t)h * 2) = o;
          }
        }
      }
      sched_fence();
    }
  }
}

template <int kMode>
__device__ __forceinline__ void dx_epilogue_bf16(const f32x4_t (&acc)[8][8], const DxArgs& a,
                                                 const EpiCoordsBf& ec, int32_t row0, int32_t h0) {
  if constexpr (kMode >= kDxTiledAcc) {
    dx_epilogue_tiled_acc<kMode>(acc, a, ec, row0, h0);
    return;
  }
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const int32_t rowl = row0 + ec.row(fm);
    const bool rv = rowl < a.Cn;
    float* arow = a.accbuf + (int64_t)(rv ? rowl : 0) * a.ld_acc;
    char* xrow = kMode >= kDxAddEmit ? a.dX + (int64_t)a.row_index[rv ? rowl : 0] * a.lddx_b
                                     : nullptr;
    const float sc = kMode == kDxEmit && a.row_scale ? a.row_scale[rv ? rowl : 0] : 1.f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int fn = 4 * half + q;
        const int32_t h = h0 + ec.col(fn);
        f32x4_t v = acc[fm][fn];
        if (rv && h < a.H) {
          if (kMode == kDxAdd || kMode == kDxAddEmit)
            v += *reinterpret_cast<const f32x4_t*>(arow + h);
          if (kMode <= kDxAdd) {
            *reinterpret_cast<f32x4_t*>(arow + h) = v;
          } else {
            if (kMode == kDxEmit) v *= sc;
            u32x2_t o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<u32x2_t*>(xrow + (int64_t)h * 2) = o;
          }
        }
      }
      sched_fence();
    }
  }
}

// Backward step 2: A = G rows (256 tokens, K = vocabulary), B = W read
// K-major (256 hidden columns).
// dX: one workgroup per output tile (grid = tiles_m x tiles_n, launched
// that way by the host).  K = the block's vocabulary columns is long (hundreds
// to thousands of stages), so a persistent tile loop gains nothing here, and
// with one the compiler rotated accumulators through VGPRs and spilled inside
// the K loop (the next tile's operand set-up lives in that loop); with a
// single tile the loop compiles to the MFMAs, LDS reads and DMA only.
// Workgroup b of nb (b = blockIdx.x unless the launch holds dW as well).
template <int kMode>
__device__ __forceinline__ void dx_bf16_tile(char* lds, const DxArgs& a, uint32_t tile);

template <int kMode>
__device__ __forceinline__ void dx_bf16_body(char* lds, DxArgs a, uint32_t b, uint32_t nb) {
  // K split (nsplit > 1): workgroup b takes slice b % nsplit of tile b / nsplit:
  // the slice's first vocabulary entry becomes K = 0 of E and of W, and its
  // fp32 result goes to its own plane of accbuf
  if (a.nsplit > 1) {
    const uint32_t z = b % (uint32_t)a.nsplit;
    b /= (uint32_t)a.nsplit;
    nb /= (uint32_t)a.nsplit;
    const int32_t k0 = (int32_t)z * a.kslice;
    a.G += (int64_t)k0 * 2;
    a.g_range -= (uint32_t)k0 * 2u;
    a.W += (int64_t)k0 * a.ldw_b;
    a.w_range -= (uint32_t)k0 * (uint32_t)a.ldw_b;
    a.v0 += k0;
    a.kv = min(a.kslice, a.kv - k0);
    a.accbuf += (int64_t)z * a.split_stride;
  }
  dx_bf16_tile<kMode>(lds, a, xcd_remap(b, nb));
}

// One dX output tile (logical id `tile`, none if past the grid).
template <int kMode>
__device__ __forceinline__ void dx_bf16_tile(char* lds, const DxArgs& a, uint32_t tile) {
  const int ntiles = tile < (uint32_t)(a.tiles_m * a.tiles_n) ? 1 : 0;
  const EpiCoordsBf ec0;
  KcOp A;
  TrOp B;
  A.init_frag(ec0.wm * 128);
  mainloop_bf16<false>(
      lds, A, B, (a.kv + kBKBf - 1) / kBKBf, ntiles,
      [&](int) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(tile, a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t row0 = (int32_t)tm * 256, h0 = (int32_t)tn * 256;
        A.set_rows(make_rsrc(a.G, a.g_range), [&](uint32_t r) __attribute__((always_inline)) {
          return (uint32_t)(row0 + (int32_t)r) * (uint32_t)a.ldg_b;
        });
        // W points at the block's (or slice's) first vocabulary row (v0)
        B.init(make_rsrc(a.W, a.w_range), (uint32_t)h0 * 2u, (uint32_t)a.ldw_b, a.V - a.v0,
               a.H - h0, ec0.wn * 128);
      },
      [&](int, f32x4_t(&acc)[8][8], char*) __attribute__((always_inline)) {
        const EpiCoordsBf ec = fresh(ec0);
        uint32_t tm, tn;
        grouped_tile(tile, a.tiles_m, a.tiles_n, 4, tm, tn);
        dx_epilogue_bf16<kMode>(acc, a, ec, (int32_t)tm * 256, (int32_t)tn * 256);
      });
}

template <int kMode>
MT_GEMM_BF16_KERNEL void dx_bf16_kernel(DxArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBf];
  dx_bf16_body<kMode>(lds, a, blockIdx.x, gridDim.x);
}

// dW tiles accumulate in place: a tile's accumulators start from the fp32
// values already in dW (when the kernel accumulates) -- 64 loads per lane in
// flight together, straight into the accumulator registers -- and the
// epilogue only stores.  Every tile, whole or at the edge (rows past cv,
// columns past H), takes the same branch-free code: one buffer resource per
// tile that ends at its last element, and a lane whose element lies outside
// the tile gets an offset past that end (loads return 0, stores are
// dropped).  The whole offset is in the per-lane register (no scalar part),
// which is what the range check covers.
constexpr uint32_t kDwOut = 0x80000000u;  // beyond any tile resource (< 2 GiB)

struct DwTile {
  rsrc_t r;
  uint32_t rows, cols;  // valid extent (<= 256 each)
};
__device__ __forceinline__ DwTile dw_tile(const DwArgs& a, int32_t m0, int32_t h0) {
  DwTile t;
  t.rows = (uint32_t)min(256, a.cv - m0);
  t.cols = (uint32_t)min(256, a.H - h0);
  t.r = make_rsrc(a.dW + (int64_t)(a.v0 + m0) * a.lddw + h0,
                  ((t.rows - 1u) * (uint32_t)a.lddw + t.cols) * 4u);
  return t;
}

// Tiled dW (DwArgs::tiled): a tile's 256 KiB are contiguous and ordered by
// wave, fragment and lane, so every load and store of the accumulators is
// one contiguous KiB per instruction -- no transpose, no bounds (the tile
// grid is padded; rows past V and columns past H are never read back).
__device__ __forceinline__ rsrc_t dw_tiled_rsrc(const DwArgs& a, int32_t m0, int32_t h0) {
  const int32_t tm = (a.v0 + m0) / 256;
  const float* base = tm < a.lo_rows ? a.dW + a.tile_pad + (int64_t)tm * a.tiles_n * 65536
                                     : a.dW_hi + (int64_t)(tm - a.lo_rows) * a.tiles_n * 65536;
  return make_rsrc(base + (int64_t)(h0 / 256) * 65536, 262144u);
}
__device__ __forceinline__ uint32_t dw_tiled_off(const EpiCoordsBf& ec, int fm, int fn) {
  return ((((ec.wm * 2u + ec.wn) * 64u + (uint32_t)fm * 8u + (uint32_t)fn) * 64u) + ec.lane) * 16u;
}

// Zero starting values of a tile the compiler cannot see as constants (with
// known-zero accumulators it restructured the K loop and spilled).
__device__ __forceinline__ f32x4_t opaque_zero4() {
  uint32_t z = 0;
  asm volatile("" : "+v"(z));
  const float f = __builtin_bit_cast(float, z);
  return f32x4_t{f, f, f, f};
}

// Accumulators of tile (m0, h0) from dW (or zero), fragment row fm of the
// wave (its fragments' 16 rows x 4 columns per lane).
__device__ __forceinline__ void dw_load_row(f32x4_t (&accrow)[8], const DwArgs& a,
                                            const EpiCoordsBf& ec, const DwTile& t, int fm,
                                            bool load) {
  const uint32_t row = (uint32_t)ec.row(fm);
#pragma unroll
  for (int fn = 0; fn < 8; ++fn) {
    const uint32_t col = (uint32_t)ec.col(fn);
    const uint32_t off = row < t.rows && col < t.cols ? (row * (uint32_t)a.lddw + col) * 4u : kDwOut;
    accrow[fn] = load ? __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(t.r, off, 0, kCpolNt))
                      : f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
}

template <int kOut>
__device__ __forceinline__ void dw_load_acc(f32x4_t (&acc)[8][8], const DwArgs& a,
                                            const EpiCoordsBf& ec, int32_t m0, int32_t h0,
                                            bool load) {
  if constexpr (kOut == kDwNarrow) {
    const f32x4_t z = opaque_zero4();
#pragma unroll
    for (int fm = 0; fm < 8; ++fm)
#pragma unroll
      for (int fn = 0; fn < 8; ++fn) acc[fm][fn] = z;
    return;
  }
  if constexpr (kOut == kDwTiles) {
    const rsrc_t r = dw_tiled_rsrc(a, m0, h0);
#pragma unroll
    for (int fm = 0; fm < 8; ++fm)
#pragma unroll
      for (int fn = 0; fn < 8; ++fn)
        acc[fm][fn] = load ? __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                          r, dw_tiled_off(ec, fm, fn), 0, kCpolNt))
                           : f32x4_t{0.f, 0.f, 0.f, 0.f};
    return;
  }
  const DwTile t = dw_tile(a, m0, h0);
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) dw_load_row(acc[fm], a, ec, t, fm, load);
}

// Stores leave through LDS: a store instruction straight from the
// accumulators covers 16 rows x 64 bytes (each lane holds 4 consecutive
// columns of one row), and the memory pipeline takes such scattered half
// lines at a quarter of its rate (16.8k cycles per tile against 5.2k for
// the same bytes in whole rows, measured).  Per fragment row fm each wave
// writes its 16 x 128 fp32 block (8 KiB) into its own quarter of `scratch`
// (the epilogue's free ring slot, 32 KiB), reads it back two rows of 512
// contiguous bytes per instruction and stores those.  The 16-byte chunk c
// of row i sits at i * 512 + ((c ^ i) & 31) * 16, so that any 8 consecutive
// lanes of a write or a read touch 8 different 16-byte bank groups.  Each
// wave uses only its own 8 KiB (LDS operations of one wave complete in
// order); the barrier at the end keeps the next phase's DMA into the slot
// behind every wave's reads.
__device__ __forceinline__ void dw_store_row(const f32x4_t (&accrow)[8], const DwArgs& a,
                                             const EpiCoordsBf& ec, const DwTile& t, int fm,
                                             char* R) {
  const uint32_t i = ec.lane & 15u, q = ec.lane >> 4;
  const uint32_t rr = ec.lane >> 5, c = ec.lane & 31u;
#pragma unroll
  for (int fn = 0; fn < 8; ++fn)
    lds_write16(R, i * 512u + ((((uint32_t)fn * 4u + q) ^ i) & 31u) * 16u,
                __builtin_bit_cast(u32x4_t, accrow[fn]));
  const uint32_t col = ec.wn * 128u + 4u * c;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t lrow = 2u * (uint32_t)j + rr;
    const uint32_t row = ec.wm * 128u + (uint32_t)fm * 16u + lrow;
    const u32x4_t v = lds_read16(R, lrow * 512u + ((c ^ lrow) & 31u) * 16u);
    const uint32_t off = row < t.rows && col < t.cols ? (row * (uint32_t)a.lddw + col) * 4u : kDwOut;
    __builtin_amdgcn_raw_buffer_store_b128(v, t.r, off, 0, kCpolNt);
  }
}

// kDwNarrow: one fragment row of the tile's final values as bf16 rows
// (round to nearest even), through the epilogue's free ring slot as
// dw_store_row does: the wave writes its 16 x 128 fp32 fragment row into LDS
// (XOR-swizzled 16-byte chunks) and reads it back as two rows of 512
// contiguous bytes per instruction, each lane narrowing its 4 columns into
// one 8-byte store -- 256 contiguous bytes per row and instruction.  (Packing
// straight from the accumulators made the compiler spill them.)  The
// resource ends at the tile's last element; lanes past it (rows past cv,
// columns past H) get an offset beyond that end.
__device__ __forceinline__ void dw_narrow_row(const f32x4_t (&accrow)[8], const EpiCoordsBf& ec,
                                              const rsrc_t& dst, uint32_t rows, uint32_t cols,
                                              uint32_t ldo_b, int fm, char* R) {
  const uint32_t i = ec.lane & 15u, q = ec.lane >> 4;
  const uint32_t rr = ec.lane >> 5, c = ec.lane & 31u;
#pragma unroll
  for (int fn = 0; fn < 8; ++fn)
    lds_write16(R, i * 512u + ((((uint32_t)fn * 4u + q) ^ i) & 31u) * 16u,
                __builtin_bit_cast(u32x4_t, accrow[fn]));
  const uint32_t col = ec.wn * 128u + 4u * c;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t lrow = 2u * (uint32_t)j + rr;
    const uint32_t row = ec.wm * 128u + (uint32_t)fm * 16u + lrow;
    const f32x4_t v = __builtin_bit_cast(f32x4_t, lds_read16(R, lrow * 512u + ((c ^ lrow) & 31u) * 16u));
    u32x2_t o;
    o[0] = pack_bf16x2(v[0], v[1]);
    o[1] = pack_bf16x2(v[2], v[3]);
    const uint32_t off = row < rows && col < cols ? row * ldo_b + col * 2u : kDwOut;
    __builtin_amdgcn_raw_buffer_store_b64(o, dst, off, 0, kCpolNt);
  }
}

// The bf16 rows of tile (m0, h0): resource and valid extent.
struct DwNarrowTile {
  rsrc_t r;
  uint32_t rows, cols, ldo_b;
};
__device__ __forceinline__ DwNarrowTile dw_narrow_tile(const DwArgs& a, int32_t m0, int32_t h0) {
  DwNarrowTile t;
  t.rows = (uint32_t)min(256, a.cv - m0);
  t.cols = (uint32_t)min(256, a.H - h0);
  t.ldo_b = (uint32_t)(a.lddw * 2);
  t.r = make_rsrc(reinterpret_cast<char*>(a.dW) + (int64_t)(a.v0 + m0) * a.lddw * 2 + (int64_t)h0 * 2,
                  (t.rows - 1u) * t.ldo_b + t.cols * 2u);
  return t;
}

template <int kOut>
__device__ __forceinline__ void dw_store_acc(const f32x4_t (&acc)[8][8], const DwArgs& a,
                                             const EpiCoordsBf& ec, int32_t m0, int32_t h0,
                                             char* scratch) {
  if constexpr (kOut == kDwNarrow) {
    const DwNarrowTile t = dw_narrow_tile(a, m0, h0);
    char* R = scratch + (ec.wm * 2u + ec.wn) * 8192u;
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
      dw_narrow_row(acc[fm], ec, t.r, t.rows, t.cols, t.ldo_b, fm, R);
      sched_fence();
    }
    lgkm_wait0();
    __builtin_amdgcn_s_barrier();
    return;
  }
  if constexpr (kOut == kDwTiles) {
    const rsrc_t r = dw_tiled_rsrc(a, m0, h0);
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
#pragma unroll
      for (int fn = 0; fn < 8; ++fn)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[fm][fn]), r,
                                               dw_tiled_off(ec, fm, fn), 0, kCpolNt);
      sched_fence();
    }
    return;
  }
  const DwTile t = dw_tile(a, m0, h0);
  char* R = scratch + (ec.wm * 2u + ec.wn) * 8192u;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    dw_store_row(acc[fm], a, ec, t, fm, R);
    sched_fence();
  }
  lgkm_wait0();
  __builtin_amdgcn_s_barrier();
}

// Epilogue of a dW tile when the workgroup has a next tile (nm0, nh0): the
// stores of this tile and the loads of the next tile's starting values into
// the same accumulators, so that the loads' latency runs beside the
// remaining stores instead of before the next tile's first multiplication.
// Row-major: interleaved fragment row by fragment row (each row's stores go
// through the LDS transpose).  Tiled: all 64 stores, then all 64 loads, so
// that the next tile's first multiplications wait for the vector-memory
// counter to drop to the loads issued after their own, which it can count
// (at most 63 outstanding); interleaved, they also waited for stores and
// loads of later rows (phase -0.5% at config 3 on one box).
template <int kOut>
__device__ __forceinline__ void dw_store_then_load(f32x4_t (&acc)[8][8], const DwArgs& a,
                                                   const EpiCoordsBf& ec, int32_t m0, int32_t h0,
                                                   char* scratch, int32_t nm0, int32_t nh0) {
  if constexpr (kOut == kDwNarrow) {
    (void)nm0;
    (void)nh0;
    const DwNarrowTile t = dw_narrow_tile(a, m0, h0);
    char* R = scratch + (ec.wm * 2u + ec.wn) * 8192u;
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
      dw_narrow_row(acc[fm], ec, t.r, t.rows, t.cols, t.ldo_b, fm, R);
      const f32x4_t z = opaque_zero4();
#pragma unroll
      for (int fn = 0; fn < 8; ++fn) acc[fm][fn] = z;
      sched_fence();
    }
    lgkm_wait0();
    __builtin_amdgcn_s_barrier();
    return;
  }
  if constexpr (kOut == kDwTiles) {
    const rsrc_t r = dw_tiled_rsrc(a, m0, h0), nr = dw_tiled_rsrc(a, nm0, nh0);
    const bool load = a.accumulate != 0;
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
#pragma unroll
      for (int fn = 0; fn < 8; ++fn)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[fm][fn]), r,
                                               dw_tiled_off(ec, fm, fn), 0, kCpolNt);
      sched_fence();
    }
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
#pragma unroll
      for (int fn = 0; fn < 8; ++fn)
        acc[fm][fn] = load ? __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                          nr, dw_tiled_off(ec, fm, fn), 0, kCpolNt))
                           : f32x4_t{0.f, 0.f, 0.f, 0.f};
      sched_fence();
    }
    return;
  }
  const DwTile t = dw_tile(a, m0, h0), nt = dw_tile(a, nm0, nh0);
  char* R = scratch + (ec.wm * 2u + ec.wn) * 8192u;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    dw_store_row(acc[fm], a, ec, t, fm, R);
    dw_load_row(acc[fm], a, ec, nt, fm, a.accumulate != 0);
    sched_fence();
  }
  lgkm_wait0();
  __builtin_amdgcn_s_barrier();
}

// Work queue of the persistent dW schedule.  The logical tiles are split
// into 8 contiguous shares, one per XCD (workgroup b runs on XCD b mod 8, as
// in xcd_remap), and the workgroups of an XCD take the tiles of its share in
// the order they ask for them (one atomic per tile on the share's counter):
// workgroups that start late -- on CUs that dX holds when dW is launched
// beside it -- simply take fewer tiles.  A workgroup whose share is used up
// goes on to the next XCD's share, and so on round the eight: without that,
// the XCDs that dX leaves earlier or that run faster finished their shares
// ~0.8 ms before the last one at config 3 (a mean of 300 us idle per CU
// per chunk, measured).  Wave 0 asks two tiles ahead (the main loop
// re-points its DMA at tile t + 1 while it multiplies tile t); the answer
// reaches the other waves through LDS in the tile's epilogue.
struct DwQueue {
  uint32_t* ctrs;      // the 8 counters
  uint32_t total;      // logical tiles
  uint32_t x, steps;   // share being drawn from; shares found used up
  uint32_t cur, nxt;   // logical ids of tiles base, base + 1 (>= total: none)
  int base;            // main-loop index of `cur`
  uint32_t asked;      // wave 0, lane 0: the id of tile base + 2

  __device__ __forceinline__ static uint32_t share_lo(uint32_t total, uint32_t s) {
    return (uint32_t)((uint64_t)total * s / 8u);
  }
  // next tile for this workgroup (wave 0, lane 0 only), total when none is left
  __device__ __forceinline__ uint32_t fetch() {
    while (steps < 8u) {
      const uint32_t r = __hip_atomic_fetch_add(ctrs + x, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t t = share_lo(total, x) + r;
      if (t < share_lo(total, x + 1u)) return t;
      x = (x + 1u) & 7u;
      ++steps;
    }
    return total;
  }
  // first two tiles, broadcast through LDS (before the ring uses it)
  __device__ __forceinline__ void start(const DwArgs& a, uint32_t total_, char* lds) {
    ctrs = a.queue;
    total = total_;
    x = blockIdx.x & 7u;
    steps = 0;
    base = 0;
    uint32_t* box = reinterpret_cast<uint32_t*>(lds);
    if (threadIdx.x == 0) {
      box[0] = fetch();
      box[1] = fetch();
    }
    lgkm_wait0();
    __builtin_amdgcn_s_barrier();
    cur = __builtin_amdgcn_readfirstlane(box[0]);
    nxt = __builtin_amdgcn_readfirstlane(box[1]);
    lgkm_wait0();
    __builtin_amdgcn_s_barrier();
  }
  __device__ __forceinline__ uint32_t id(int t) const { return t == base ? cur : nxt; }
  __device__ __forceinline__ bool has(int t) const { return id(t) < total; }
  // ask for tile base + 2 (only while tiles remain): at tile 0's init, then
  // in every epilogue after rotate(), so that the atomic's round trip runs
  // beside the epilogue's stores and the next tile's multiplications
  __device__ __forceinline__ void ask() {
    if (threadIdx.x == 0 && nxt < total) asked = fetch();
  }
  // epilogue of tile `base`: tile base + 2's id to every wave, then advance
  __device__ __forceinline__ void rotate(char* scratch) {
    uint32_t* box = reinterpret_cast<uint32_t*>(scratch);
    if (threadIdx.x == 0) box[0] = nxt < total ? asked : total;
    lgkm_wait0();
    __builtin_amdgcn_s_barrier();
    const uint32_t n2 = __builtin_amdgcn_readfirstlane(box[0]);
    lgkm_wait0();
    __builtin_amdgcn_s_barrier();
    cur = nxt;
    nxt = n2;
    ++base;
  }
};

// Backward step 3: A = G read K-major (256 vocabulary columns, K = tokens),
// B = X^T rows of the block (256 hidden rows).  kQueue: persistent over the
// work queue above (grid = one workgroup per CU, K >= 2 stages); otherwise
// one workgroup per tile or a static persistent schedule (TileSeq).
template <bool kQueue, int kOut>
__device__ __forceinline__ void dw_bf16_body(char* lds, const DwArgs& a, uint32_t b, uint32_t nb) {
  const uint32_t total = (uint32_t)(a.tiles_m * a.tiles_n);
  const TileSeq seq(total, b, nb);
  DwQueue q;
  if constexpr (kQueue) q.start(a, total, lds);
  const EpiCoordsBf ec0;
  TrOp A;
  KcOp B;
  B.init_frag(ec0.wn * 128);
  auto logical = [&](int k) __attribute__((always_inline)) {
    if constexpr (kQueue) return q.id(k);
    else return seq.logical(k);
  };
  mainloop_bf16_seq<true, false, true>(
      lds, A, B, (a.kt_rows + kBKBf - 1) / kBKBf,
      [&](int k) __attribute__((always_inline)) {
        if constexpr (kQueue) return q.has(k);
        else return k < seq.count();
      },
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t m0 = (int32_t)tm * 256, h0 = (int32_t)tn * 256;
        A.init(make_rsrc(a.G, a.g_range), (uint32_t)m0 * 2u, (uint32_t)a.ldg_b, a.g_rows,
               a.g_cols - m0, ec0.wm * 128);
        B.set_rows(make_rsrc(a.XcT, a.xt_range), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t h = h0 + (int32_t)r;
          h = h < a.H ? h : a.H - 1;
          return (uint32_t)h * (uint32_t)a.ldxt_b;
        });
      },
      // epilogue: this tile's stores, the next tile's starting values
      [&](int k, f32x4_t(&acc)[8][8], char* scratch) __attribute__((always_inline)) {
        const EpiCoordsBf ec = fresh(ec0);
        uint32_t tm, tn;
        grouped_tile(logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        bool next;
        if constexpr (kQueue) {
          q.rotate(scratch);
          next = q.has(k + 1);
          q.ask();
        } else {
          next = k + 1 < seq.count();
        }
        if (next) {
          uint32_t ntm, ntn;
          grouped_tile(logical(k + 1), a.tiles_m, a.tiles_n, 4, ntm, ntn);
          dw_store_then_load<kOut>(acc, a, ec, (int32_t)tm * 256, (int32_t)tn * 256, scratch,
                                     (int32_t)ntm * 256, (int32_t)ntn * 256);
        } else {
          dw_store_acc<kOut>(acc, a, ec, (int32_t)tm * 256, (int32_t)tn * 256, scratch);
        }
      },
      // init: the first tile's starting values
      [&](int k, f32x4_t(&acc)[8][8]) __attribute__((always_inline)) {
        const EpiCoordsBf ec = fresh(ec0);
        uint32_t tm, tn;
        grouped_tile(logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        if constexpr (kQueue) q.ask();
        dw_load_acc<kOut>(acc, a, ec, (int32_t)tm * 256, (int32_t)tn * 256, a.accumulate != 0);
      });
}

template <bool kQueue, int kOut>
MT_GEMM_BF16_KERNEL void dw_bf16_kernel(DwArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBf];
  dw_bf16_body<kQueue, kOut>(lds, a, blockIdx.x, gridDim.x);
}

// dX and dW of one block in one launch: workgroups [0, dx_blocks) are dX's
// (dispatched first, so dX's long tiles start at once), the rest dW's (the
// CUs dX leaves free, then the others; the work queue's XCD shares follow
// the global workgroup index, which keeps the round-robin XCD placement).
// Both only read G and the X^T block.
template <int kMode, bool kQueue, int kOut>
MT_GEMM_BF16_KERNEL void dx_dw_bf16_kernel(DxArgs x, DwArgs w, uint32_t dx_blocks) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBf];
  if constexpr (kQueue && kOut == kDwTiles) {  // (the other outputs spill with this path in)
    if (x.xcds > 0) {
      // XCD-partitioned (DxArgs::xcds; one K slice, work-queue dW): the
      // hardware places workgroup b on XCD b % 8, so dX's tiles fill whole
      // XCDs while the dW workers take the rest and, as dX's workgroups end,
      // the later workgroups of the grid on those XCDs
      const uint32_t xcd = blockIdx.x & 7u, slot = blockIdx.x >> 3;
      const uint32_t t = xcd * (uint32_t)x.per_xcd + slot;
      if (xcd < (uint32_t)x.xcds && slot < (uint32_t)x.per_xcd && t < dx_blocks)
        dx_bf16_tile<kMode>(lds, x, t);
      else
        dw_bf16_body<kQueue, kOut>(lds, w, 0, 1);
      return;
    }
  }
  if (blockIdx.x < dx_blocks)
    dx_bf16_body<kMode>(lds, x, blockIdx.x, dx_blocks);
  else
    dw_bf16_body<kQueue, kOut>(lds, w, blockIdx.x - dx_blocks, gridDim.x - dx_blocks);
}

// Tiled fp32 dW (dw_bf16_kernel<*, true>: tile rows [0, lo_rows) from
// tiles_lo, the rest from tiles_hi) times *scale, narrowed to bf16 rows of
// pitch ldo_b bytes at `out` (V rows, H columns, H a multiple of 8): one
// workgroup per tile of tile rows tr0, tr0 + 1, ... (gridDim.x / tiles_n of
// them).  Each lane reads its fragment pairs (fn = 2p, 2p + 1) as contiguous
// KiB and, after one v_permlane16_swap per dword (the pairing the forward
// uses for its chunk of exponentials), writes 8 consecutive columns.  The
// output resource of a tile ends at its last element; lanes outside the
// tile (rows past V, columns past H) get an offset past that end.
__global__ __launch_bounds__(256) void narrow_tiles_kernel(const float* scale, const float* tiles_lo,
                                                           const float* tiles_hi, int32_t lo_rows,
                                                           int32_t tr0, int32_t tiles_n, int32_t V,
                                                           int32_t H, char* out, int64_t ldo_b) {
  const int32_t tile = tr0 * tiles_n + (int32_t)blockIdx.x;
  const int32_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const uint32_t rows = (uint32_t)min(256, V - tm * 256), cols = (uint32_t)min(256, H - tn * 256);
  const float sc = *scale;
  const EpiCoordsBf ec;
  const float* tsrc = tm < lo_rows ? tiles_lo + (int64_t)tile * 65536
                                   : tiles_hi + ((int64_t)(tm - lo_rows) * tiles_n + tn) * 65536;
  const rsrc_t src = make_rsrc(tsrc, 262144u);
  const rsrc_t dst = make_rsrc(out + (int64_t)tm * 256 * ldo_b + (int64_t)tn * 512,
                               (rows - 1u) * (uint32_t)ldo_b + cols * 2u);
  const uint32_t q = ec.lane >> 4;
  const uint32_t scol = ec.wn * 128u + 8u * (2u * (q & 1u) + (q >> 1));
  // the next fragment row's loads go out before this row's stores: loads and
  // stores share one in-order counter, so a load issued after a store would
  // wait for that store too
  f32x4_t cur[8], nxt[8];
#pragma unroll
  for (int fn = 0; fn < 8; ++fn)
    cur[fn] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(src, dw_tiled_off(ec, 0, fn), 0, kCpolNt));
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const uint32_t row = (uint32_t)ec.row(fm);
    if (fm < 7) {
#pragma unroll
      for (int fn = 0; fn < 8; ++fn)
        nxt[fn] = __builtin_bit_cast(
            f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(src, dw_tiled_off(ec, fm + 1, fn), 0, kCpolNt));
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const f32x4_t v0 = cur[2 * p], v1 = cur[2 * p + 1];
      const auto l2 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(v0[0] * sc, v0[1] * sc),
                                                       pack_bf16x2(v1[0] * sc, v1[1] * sc), false, false);
      const auto h2 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(v0[2] * sc, v0[3] * sc),
                                                       pack_bf16x2(v1[2] * sc, v1[3] * sc), false, false);
      u32x4_t o;
      o[0] = l2[0];
      o[1] = h2[0];
      o[2] = l2[1];
      o[3] = h2[1];
      const uint32_t col = scol + 32u * (uint32_t)p;
      const uint32_t off = row < rows && col < cols ? row * (uint32_t)ldo_b + col * 2u : kDwOut;
      __builtin_amdgcn_raw_buffer_store_b128(o, dst, off, 0, kCpolNt);
    }
#pragma unroll
    for (int fn = 0; fn < 8; ++fn) cur[fn] = nxt[fn];
  }
}

// Fused path, chunks whose exponentials would leave bf16's range: G = g_t
// (softmax(cap(S_t)) - onehot(y_t)) (1 - tanh^2), in place over one chunk of
// the bf16 logits S written by fwd_bf16_kernel<*, kStoreLogits>; nothing
// unless *run_if != 0 (run_if non-null).  One workgroup per row; rows >= cn
// and columns >= V become 0.  HBM-bound: one 16-byte read and one 16-byte
// write per 8 elements.
template <bool kCap>
__global__ __launch_bounds__(256) void softmax_grad_kernel(char* S, int64_t lds_b, int32_t cols,
                                                           int32_t cn, int32_t V,
                                                           const float* lse, const float* grad,
                                                           int64_t gstride,
                                                           const int32_t* row_index,
                                                           const int32_t* row_label,
                                                           float softcap,
                                                           const int32_t* run_if) {
  if (run_if && *run_if == 0) return;
  const int32_t row = blockIdx.x;
  const bool rv = row < cn;
  const float lse2 = rv ? lse[row] * kLog2e : 0.f;
  const float g = rv ? grad[(int64_t)row_index[row] * gstride] : 0.f;
  const int32_t y = rv ? row_label[row] : -1;
  const float inv_cap = kCap ? 1.0f / softcap : 0.f;
  u32x4_t* p = reinterpret_cast<u32x4_t*>(S + (int64_t)row * lds_b);
  // G of 8 consecutive columns starting at c
  auto grad8 = [&](u32x4_t v, int32_t c) __attribute__((always_inline)) {
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = v[j / 2];
      float x = __builtin_bit_cast(float, (j & 1) ? (w & 0xffff0000u) : (w << 16));
      float dcap = 1.f;
      if (kCap) {
        const float t = tanh_approx(x * inv_cap);
        x = softcap * t;
        dcap = 1.f - t * t;
      }
      float q = fast_exp2(fmaf(x, kLog2e, -lse2));
      q -= (c + j == y) ? 1.f : 0.f;
      o[j] = (rv && c + j < V) ? q * g * dcap : 0.f;
    }
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = pack_bf16x2(o[2 * j], o[2 * j + 1]);
    return r;
  };
  // four 16-byte loads in flight per thread before the first store (one at
  // a time left the pass at 5.5 TB/s)
  constexpr int32_t kStep = 256 * 8;
  int32_t c = threadIdx.x * 8;
  for (; c + 3 * kStep < cols; c += 4 * kStep) {
    u32x4_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = p[(c + k * kStep) / 8];
#pragma unroll
    for (int k = 0; k < 4; ++k) p[(c + k * kStep) / 8] = grad8(v[k], c + k * kStep);
  }
  for (; c < cols; c += kStep) p[c / 8] = grad8(p[c / 8], c);
}

}  // namespace mtf
