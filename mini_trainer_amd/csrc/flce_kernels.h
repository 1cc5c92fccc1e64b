// Kernels of the fused LM-head linear + per-token cross-entropy path.
//
//   fwd_kernel       logits tile = X_rows . W_tile^T (MFMA), fused online
//                    log-sum-exp over the vocabulary and label-logit capture;
//                    no logits are written to memory.
//   fwd_finalize     merge of the per-split (max, sum) partials -> lse, loss.
//   recompute_kernel logits tile recomputed and turned into
//                    G = g * (softmax - onehot) (bf16 / fp32) for one block.
//   dx_kernel        dX_block (+)= G . W_block    (W consumed K-major)
//   dw_kernel        dW_block (+)= G^T . X_block  (G consumed K-major)
//   small kernels    valid-row compaction, gather-transpose of X rows,
//                    zeroing of ignored rows, per-sample segment sums.
#pragma once

#include "flce_gemm.h"

namespace mtf {

#define MT_GEMM_KERNEL \
  __global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))

// Output coordinates of this lane's accumulators for a wave tile of
// 128 rows x (NFN * 16) columns, WC waves across the tile's columns (tile
// width NFN * 16 * WC: 8 x 16 x 2 for the four-wave fp32 kernels, 4 x 16 x 4
// for the eight-wave bf16 kernels).
template <int NFN, int WC = 2>
struct EpiCoordsT {
  static constexpr int kNF = NFN;
  static constexpr int kWC = WC;
  static constexpr int kTileN = NFN * 16 * WC;
  uint32_t lane, wm, wn;
  __device__ __forceinline__ EpiCoordsT() {
    lane = lane_id();
    uint32_t w = wave_id();
    wm = w / WC;
    wn = w % WC;
  }
  // Tile-local output row of fragment row fm held by this lane.
  __device__ __forceinline__ int row(int fm) const { return wm * 128 + fm * 16 + (lane & 15u); }
  // Tile-local output column of element 0 of fragment column fn.
  __device__ __forceinline__ int col(int fn) const {
    return wn * (NFN * 16) + fn * 16 + 4 * (lane >> 4);
  }
};
typedef EpiCoordsT<8> EpiCoords;

// Is column offset `rel` (label column minus this lane's column of fn = 0,
// r = 0) one of the NFN * 4 columns this lane holds?
template <int NFN>
__device__ __forceinline__ bool lane_holds(int rel) {
  return rel >= 0 && rel < NFN * 16 && (rel & 12) == 0;
}

// ===========================================================================
// Forward
// ===========================================================================
struct FwdArgs {
  const char* X;
  const char* W;  // vocabulary row vcol0 of the weight
  int64_t ldx_b, ldw_b;
  int32_t H, V, N;  // V: vocabulary rows from W on (this launch's block)
  int32_t vcol0;    // global vocabulary index of W's row 0 (a multiple of 256)
  uint32_t x_range, w_range, s_range;  // bytes addressable from X, W, S
  const int32_t* row_index;
  const int32_t* row_label;
  float softcap;
  int32_t tiles_m, splits, vt_total, vt_per_split;
  float* part;  // [N][splits][2] = (max in log2 units, scaled sum)
  float* xy;    // [N] label logit
  char* S;      // bf16 logits or exponentials [>= tiles_m * 256][lds_b / 2] (fused path only)
  int64_t lds_b;
  const int32_t* run_if = nullptr;  // non-null: the kernel does nothing unless *run_if != 0
  int32_t* guard_reset = nullptr;   // non-null: set to 0 by the launch (read only after it)
};

// Columns at or beyond V are masked with a select (no separate tail variant:
// one code path keeps the epilogue's register footprint small).
template <typename T, int NFN, bool kCap>
__device__ __forceinline__ void fwd_tile_epilogue(const f32x4_t (&acc)[8][NFN], float (&m2)[8],
                                                  float (&d)[8], const int32_t (&rel)[8],
                                                  const int32_t (&rglob)[8], int32_t ncol0,
                                                  const FwdArgs& a, bool any_hit) {
  const float cap = a.softcap, inv_cap = kCap ? 1.0f / a.softcap : 0.f;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    float v[NFN][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int fn = 0; fn < NFN; ++fn) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[fn][r] = acc[fm][fn][r];
      round_pair<T>(v[fn][0], v[fn][1]);
      round_pair<T>(v[fn][2], v[fn][3]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = v[fn][r];
        if (kCap) x = cap * tanh_approx(x * inv_cap);
        x = ncol0 + fn * 16 + r < a.V ? x : -INFINITY;
        v[fn][r] = x;
        tmax = fmaxf(tmax, x);
      }
    }
    const float mn = fmaxf(m2[fm], tmax * kLog2e);
    float s = 0.f;
#pragma unroll
    for (int fn = 0; fn < NFN; ++fn)
#pragma unroll
      for (int r = 0; r < 4; ++r) s += fast_exp2(fmaf(v[fn][r], kLog2e, -mn));
    d[fm] = fmaf(d[fm], fast_exp2(m2[fm] - mn), s);
    m2[fm] = mn;
    if (any_hit) {
      const int rl = rel[fm];
      if (lane_holds<NFN>(rl) && rglob[fm] < a.N) {
        float hitv = 0.f;
#pragma unroll
        for (int fn = 0; fn < NFN; ++fn)
#pragma unroll
          for (int r = 0; r < 4; ++r) hitv = (rl == fn * 16 + r) ? v[fn][r] : hitv;
        a.xy[rglob[fm]] = hitv;
      }
    }
  }
}

// Online-LSE update of one finished 256 x 256 logits tile (vocabulary rows
// vrow0 .. vrow0 + 255) plus label-logit capture.
template <typename T, bool kCap, int NFN, int WC>
__device__ __forceinline__ void fwd_tile_update(const f32x4_t (&acc)[8][NFN], float (&m2)[8],
                                                float (&d)[8], const int32_t (&lbl)[8],
                                                const int32_t (&rglob)[8], int32_t vrow0,
                                                const EpiCoordsT<NFN, WC>& ec, const FwdArgs& a) {
  const int32_t ncol0 = vrow0 + ec.col(0);
  int32_t rel[8];
  bool hit = false;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    rel[fm] = lbl[fm] - ncol0;
    hit |= lane_holds<NFN>(rel[fm]);
  }
  const bool any_hit = __builtin_amdgcn_ballot_w64(hit) != 0;
  fwd_tile_epilogue<T, NFN, kCap>(acc, m2, d, rel, rglob, ncol0, a, any_hit);
}

// x of lane l ^ 16 and of lane l ^ 32, from one lane swap and a select
// (v_permlane16_swap / v_permlane32_swap with x as both operands hand back
// rows (0, 0, 2, 2) and (1, 1, 3, 3) of 16 lanes, or halves (lo, lo) and
// (hi, hi)) instead of an LDS permute and its wait.
__device__ __forceinline__ float xor16(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (lane_id() & 16u) ? p[0] : p[1]);
}
__device__ __forceinline__ float xor32(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (lane_id() & 32u) ? p[0] : p[1]);
}

// Merge the four lanes that share a row, then the WC waves (wn = 0 .. WC - 1)
// that share the row through LDS, and write this split's (max, sum) partial
// of every row.
template <int NFN, int WC>
__device__ __forceinline__ void fwd_final_merge(char* lds, float (&m2)[8], float (&d)[8],
                                                const int32_t (&rglob)[8], uint32_t ts,
                                                const EpiCoordsT<NFN, WC>& ec, const FwdArgs& a) {
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    lse_merge(m2[fm], d[fm], xor16(m2[fm]), xor16(d[fm]));
    lse_merge(m2[fm], d[fm], xor32(m2[fm]), xor32(d[fm]));
  }
  float* red = reinterpret_cast<float*>(lds);  // [WC - 1][256 rows][2]
  __syncthreads();
  if (ec.wn != 0 && (ec.lane >> 4) == 0) {
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
      float* r = red + ((ec.wn - 1) * 256 + ec.row(fm)) * 2;
      r[0] = m2[fm];
      r[1] = d[fm];
    }
  }
  __syncthreads();
  if (ec.wn == 0 && (ec.lane >> 4) == 0) {
#pragma unroll
    for (int fm = 0; fm < 8; ++fm) {
#pragma unroll
      for (int w = 0; w < WC - 1; ++w) {
        const float* r = red + (w * 256 + ec.row(fm)) * 2;
        lse_merge(m2[fm], d[fm], r[0], r[1]);
      }
      if (rglob[fm] < a.N) {
        int64_t o = ((int64_t)rglob[fm] * a.splits + ts) * 2;
        a.part[o + 0] = m2[fm];
        a.part[o + 1] = d[fm];
      }
    }
  }
}

// kKTail: H is not a multiple of the K slab (the last slab is partial).
template <typename T, bool kKTail>
MT_GEMM_KERNEL void fwd_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  uint32_t tm, ts;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.splits, 4, tm, ts);
  const EpiCoords ec;
  FragOffsets fo;
  fo.init();

  const int32_t row0 = (int32_t)tm * 256;
  DirectLoader la;
  la.init([&](uint32_t r) __attribute__((always_inline)) {
    int32_t rr = row0 + (int32_t)r;
    rr = rr < a.N ? rr : a.N - 1;
    return a.X + (int64_t)a.row_index[rr] * a.ldx_b;
  });

  int32_t lbl[8], rglob[8];
  float m2[8], d[8];
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    rglob[fm] = row0 + ec.row(fm);
    lbl[fm] = rglob[fm] < a.N ? a.row_label[rglob[fm]] : -1;
    m2[fm] = kNegBig;
    d[fm] = 0.f;
  }

  const int KT = (a.H + Elt<T>::kBK - 1) / Elt<T>::kBK;
  const uint32_t c_lim = (uint32_t)(a.H - (KT - 1) * Elt<T>::kBK) / Elt<T>::kPerChunk;
  if constexpr (kKTail) la.set_tail(c_lim);
  const int vt0 = (int)ts * a.vt_per_split;
  const int vt1 = min(vt0 + a.vt_per_split, a.vt_total);
  f32x4_t acc[8][8];
  for (int vt = vt0; vt < vt1; ++vt) {
    const int32_t vrow0 = vt * 256;
    DirectLoader lb;
    lb.init([&](uint32_t r) __attribute__((always_inline)) {
      int32_t v = vrow0 + (int32_t)r;
      v = v < a.V ? v : a.V - 1;
      return a.W + (int64_t)v * a.ldw_b;
    });
    if constexpr (kKTail) lb.set_tail(c_lim);
    mainloop<T, kKTail>(lds, acc, la, lb, KT, fo, c_lim);

    if (a.softcap > 0.f) fwd_tile_update<T, true>(acc, m2, d, lbl, rglob, vrow0, ec, a);
    else fwd_tile_update<T, false>(acc, m2, d, lbl, rglob, vrow0, ec, a);
  }
  fwd_final_merge(lds, m2, d, rglob, ts, ec, a);
}

// lse and loss of each valid row from its `splits` (max, sum) partials: one
// wave per row, lanes merge strided partials, then a fixed shuffle tree
// (deterministic order).
// guard (non-null): set to 1 when some row's largest logit lies outside
// [kGuardLo, kGuardHi], the range in which the fused path keeps exp(logit)
// itself in bf16 (see fused_row_scale_kernel): at a row maximum of -48 the
// terms within 39 of it (relative weight e^-39 and more) stay normal numbers
// (e^-87 is about the smallest), and at +48, lse <= 48 + ln V keeps the row
// factor g exp(-lse) a normal fp32 number for g down to 1e-10 at V = 2^20.
constexpr float kGuardLo = -48.f, kGuardHi = 48.f;
__global__ __launch_bounds__(256) void fwd_finalize_kernel(const float* part, const float* xy,
                                                           int32_t N, int32_t splits,
                                                           const int32_t* row_index, float* loss,
                                                           float* lse, int32_t* guard) {
  const int32_t r = (int32_t)(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (r >= N) return;  // uniform per wave
  const int lane = (int)(threadIdx.x & 63u);
  const float* pr = part + (int64_t)r * splits * 2;
  float m = kNegBig, d = 0.f;
  for (int s = lane; s < splits; s += 64) lse_merge(m, d, pr[2 * s], pr[2 * s + 1]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lse_merge(m, d, __shfl_xor(m, off), __shfl_xor(d, off));
  if (lane == 0) {
    const float L = (m + fast_log2(d)) * kLn2;
    lse[r] = L;
    loss[row_index[r]] = L - xy[r];
    const float mx = m * kLn2;
    if (guard && !(mx >= kGuardLo && mx <= kGuardHi)) atomicOr(guard, 1);
  }
}

// Fused path, per row chunk, after the forward stored E = exp(z) (z the
// bf16-rounded, soft-capped logit; times the softcap derivative 1 - (z/cap)^2)
// instead of the logits: G = g (softmax - onehot) dz = s E - onehot g dz with
// the per-row factor s = g exp(-lse).  dX = G W and dW = G^T X then take s as
// a row scale of dX and of the gathered X^T (gather_t_kernel), and this
// kernel replaces the label's element by (exp(z_y) - exp(lse)) dz_y, formed
// in fp32 from the label logit (no cancellation against the rounded E).  When
// the guard is set the chunk holds G itself (the logits were stored and
// turned into G by softmax_grad_kernel): s = 1 and no element is touched.
// Rows cn .. cn_pad get s = 0.  One thread per row; the first n_zero threads
// also clear zero_words (the dW work queue of the chunk).
__global__ __launch_bounds__(256) void fused_row_scale_kernel(
    int32_t cn, int32_t cn_pad, const float* lse, const float* xy, const float* grad,
    int64_t gstride, const int32_t* row_index, const int32_t* row_label, const int32_t* guard,
    float softcap, char* E, int64_t lde_b, float* scale, uint32_t* zero_words, int32_t n_zero) {
  const int32_t t = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
  if (t < n_zero) zero_words[t] = 0u;
  if (t >= cn_pad) return;
  if (t >= cn) {
    scale[t] = 0.f;
    return;
  }
  if (*guard != 0) {
    scale[t] = 1.f;
    return;
  }
  const float L = lse[t], z = xy[t];
  const float g = grad[(int64_t)row_index[t] * gstride];
  float dz = 1.f;
  if (softcap > 0.f) {
    const float q = z / softcap;
    dz = fmaf(-q, q, 1.f);
  }
  const float e = (fast_exp2(z * kLog2e) - fast_exp2(L * kLog2e)) * dz;
  reinterpret_cast<__bf16*>(E + (int64_t)t * lde_b)[row_label[t]] = (__bf16)e;
  scale[t] = g * fast_exp2(-L * kLog2e);
}

// ===========================================================================
// Backward, step 1: G = g * (softmax(logits) - onehot) for one block.
// ===========================================================================
struct RecompArgs {
  const char* X;
  const char* W;  // vocabulary row v0 of the weight (the block's first row)
  int64_t ldx_b, ldw_b;
  int32_t H, V;
  uint32_t x_range, w_range, g_range;  // bytes addressable from X, W, G
  const int32_t* row_index;  // offset to the block's first valid row
  const int32_t* row_label;
  const float* lse;
  int32_t Cn;  // valid rows in the block
  const float* grad;
  int64_t gstride;
  float softcap;
  int32_t v0, cv;  // vocabulary range [v0, v0 + cv)
  char* G;         // [tiles_m * 256][>= tiles_n * 256], row pitch ldg_b
  int64_t ldg_b;
  int32_t tiles_m, tiles_n;
  uint32_t* zero_words = nullptr;  // cleared by the launch (dW's work queue, read after it)
  // non-null (bf16): the launch computes nothing unless *run_if != 0 (the
  // first vocabulary block, whose G a forward kept as exponentials, when
  // those left their range); zero_words is cleared either way
  const int32_t* run_if = nullptr;
};

// The first vocabulary block's G from the exponentials E = exp(z) that
// mt_flce_forward_keep left in the G block (columns [0, cols), softcap off):
// G = g (E exp(-lse) - onehot), in place, one workgroup per row of the block
// (rows >= cn become 0).  Nothing when *skip_if != 0: some row's largest
// logit left the range in which E holds its terms, and the block is
// recomputed instead (recompute_bf16_kernel with run_if = the same word).
// HBM-bound: one 16-byte read and one 16-byte write per 8 entries.
__global__ __launch_bounds__(256) void exp_to_grad_kernel(char* G, int64_t ldg_b, int32_t cols,
                                                          int32_t cn, const float* lse,
                                                          const float* grad, int64_t gstride,
                                                          const int32_t* row_index,
                                                          const int32_t* row_label,
                                                          const int32_t* skip_if) {
  if (*skip_if != 0) return;
  const int32_t row = (int32_t)blockIdx.x;
  const bool rv = row < cn;
  float s = 0.f, g = 0.f;
  int32_t y = -1;
  if (rv) {
    g = grad[(int64_t)row_index[row] * gstride];
    s = g * fast_exp2(-lse[row] * kLog2e);
    y = row_label[row];
  }
  char* p = G + (int64_t)row * ldg_b;
  for (int32_t c = (int32_t)threadIdx.x * 8; c < cols; c += 256 * 8) {
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(p + (int64_t)c * 2);
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float e0 = __builtin_bit_cast(float, v[j] << 16);
      const float e1 = __builtin_bit_cast(float, v[j] & 0xffff0000u);
      const int32_t c0 = c + 2 * j;
      const float g0 = fmaf(s, e0, c0 == y ? -g : 0.f);
      const float g1 = fmaf(s, e1, c0 + 1 == y ? -g : 0.f);
      o[j] = rv ? pack_bf16x2(g0, g1) : 0u;
    }
    *reinterpret_cast<u32x4_t*>(p + (int64_t)c * 2) = o;
  }
}

template <typename T>
__device__ __forceinline__ void store4(char* p, const float (&o)[4]);
template <>
__device__ __forceinline__ void store4<__bf16>(char* p, const float (&o)[4]) {
  u32x2_t w;
  w.x = pack_bf16x2(o[0], o[1]);
  w.y = pack_bf16x2(o[2], o[3]);
  *reinterpret_cast<u32x2_t*>(p) = w;
}
template <>
__device__ __forceinline__ void store4<float>(char* p, const float (&o)[4]) {
  *reinterpret_cast<f32x4_t*>(p) = f32x4_t{o[0], o[1], o[2], o[3]};
}

template <typename T, int NFN, bool kCap, int WC>
__device__ __forceinline__ void recompute_epilogue(const f32x4_t (&acc)[8][NFN], const RecompArgs& a,
                                                   const EpiCoordsT<NFN, WC>& ec, int32_t row0,
                                                   int32_t col0) {
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
    hit |= lane_holds<NFN>(rel[fm]);
  }
  const bool any_hit = __builtin_amdgcn_ballot_w64(hit) != 0;
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const bool rv = rowl[fm] < a.Cn;
    char* grow = a.G + (int64_t)rowl[fm] * a.ldg_b;
#pragma unroll
    for (int fn = 0; fn < NFN; ++fn) {
      float o[4];
      float xr[4] ={acc[fm][fn][0], acc[fm][fn][1], acc[fm][fn][2], acc[fm][fn][3]};
      round_pair<T>(xr[0], xr[1]);
      round_pair<T>(xr[2], xr[3]);
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
        const bool ok = rv && (ncol0 + fn * 16 + r < a.cv);
        o[r] = ok ? p * g[fm] * dcap : 0.f;
      }
      store4<T>(grow + (int64_t)(ncol0 + fn * 16) * Elt<T>::kBytes, o);
    }
  }
}

template <typename T, bool kKTail>
MT_GEMM_KERNEL void recompute_kernel(RecompArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  uint32_t tm, tn;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.tiles_n, 4, tm, tn);
  const EpiCoords ec;
  FragOffsets fo;
  fo.init();
  const int32_t row0 = (int32_t)tm * 256;
  DirectLoader la;
  la.init([&](uint32_t r) __attribute__((always_inline)) {
    int32_t rr = row0 + (int32_t)r;
    rr = rr < a.Cn ? rr : a.Cn - 1;
    return a.X + (int64_t)a.row_index[rr] * a.ldx_b;
  });
  const int32_t vloc0 = (int32_t)tn * 256;  // rows from the block's first (W's row 0)
  DirectLoader lb;
  lb.init([&](uint32_t r) __attribute__((always_inline)) {
    int32_t v = vloc0 + (int32_t)r;
    v = v < a.cv ? v : a.cv - 1;  // rows past the block repeat its last one
    return a.W + (int64_t)v * a.ldw_b;
  });
  f32x4_t acc[8][8];
  const int KT = (a.H + Elt<T>::kBK - 1) / Elt<T>::kBK;
  const uint32_t c_lim = (uint32_t)(a.H - (KT - 1) * Elt<T>::kBK) / Elt<T>::kPerChunk;
  if constexpr (kKTail) {
    la.set_tail(c_lim);
    lb.set_tail(c_lim);
  }
  mainloop<T, kKTail>(lds, acc, la, lb, KT, fo, c_lim);
  if (a.softcap > 0.f) recompute_epilogue<T, 8, true>(acc, a, ec, row0, (int32_t)tn * 256);
  else recompute_epilogue<T, 8, false>(acc, a, ec, row0, (int32_t)tn * 256);
}

// ===========================================================================
// Backward, step 2: dX rows of the block (+)= G . W[v0 : v0 + cv]
// ===========================================================================
enum DxMode : int32_t { kDxStore = 0, kDxAdd = 1, kDxAddEmit = 2, kDxEmit = 3 };
// bf16 only: kDxStore / kDxAdd / kDxAddEmit with the fp32 accumulator held as
// 256 x 256 tiles (accbuf + (tm * tiles_n + tn) * 65536 floats, each in the
// order of the wave's accumulators: one contiguous KiB per load and store)
constexpr int32_t kDxTiledAcc = 4;

struct DxArgs {
  const char* G;
  int64_t ldg_b;
  const char* W;  // vocabulary row v0 of the weight (the block's first row)
  int64_t ldw_b;
  uint32_t g_range, w_range;  // bytes addressable from G, W
  int32_t V, v0, kv;  // K = vocabulary entries v0 .. v0 + kv
  int32_t H, Cn;
  float* accbuf;  // fp32 [>= Cn][ld_acc] (modes >= kDxTiledAcc: tiles_m x tiles_n tiles)
  int64_t ld_acc;
  int32_t mode;
  char* dX;
  int64_t lddx_b;
  const int32_t* row_index;  // offset to the block's first valid row
  int32_t tiles_m, tiles_n;
  const float* row_scale = nullptr;  // non-null (bf16 kDxEmit): dX row r times row_scale[r]
  // split over K (bf16): nsplit slices of kslice vocabulary entries, slice z
  // stored (kDxStore) at accbuf + z * split_stride; the grid is
  // tiles_m * tiles_n * nsplit (dx_split_reduce_kernel sums the slices)
  int32_t nsplit = 1, kslice = 0;
  int64_t split_stride = 0;
  // dX beside a work-queue dW in one launch (dx_dw_bf16_kernel), XCD-
  // partitioned: xcds > 0 gives dX whole XCDs -- workgroup b (on XCD b % 8)
  // takes logical tile (b % 8) per_xcd + b / 8 when b % 8 < xcds and
  // b / 8 < per_xcd -- and every other workgroup is a dW worker, so that dX
  // and dW never share an XCD's L2 while dX runs; 0: workgroups [0, tiles)
  // are dX's (xcd_remap order)
  int32_t xcds = 0, per_xcd = 0;
};

// dX of a K-split fused chunk: row t < cn, columns h .. h + 3 of the sum of
// the nsplit fp32 slices (in slice order), times scale[t], to bf16 at dX row
// row_index[t].  One thread per 4 columns.
__global__ __launch_bounds__(256) void dx_split_reduce_kernel(const float* part, int64_t stride,
                                                              int32_t nsplit, int64_t ld, int32_t cn,
                                                              int32_t H, const float* scale,
                                                              const int32_t* row_index, char* dX,
                                                              int64_t lddx_b) {
  const int32_t t = (int32_t)blockIdx.y;
  const int32_t h = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (t >= cn || h >= H) return;
  const float* p = part + (int64_t)t * ld + h;
  f32x4_t v = *reinterpret_cast<const f32x4_t*>(p);
  for (int32_t z = 1; z < nsplit; ++z) v += *reinterpret_cast<const f32x4_t*>(p + z * stride);
  v *= scale[t];
  u32x2_t o;
  o[0] = pack_bf16x2(v[0], v[1]);
  o[1] = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<u32x2_t*>(dX + (int64_t)row_index[t] * lddx_b + (int64_t)h * 2) = o;
}

template <typename T, int NFN, int WC>
__device__ __forceinline__ void dx_epilogue(const f32x4_t (&acc)[8][NFN], const DxArgs& a,
                                            const EpiCoordsT<NFN, WC>& ec, int32_t row0, int32_t h0) {
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const int32_t rowl = row0 + ec.row(fm);
    if (rowl >= a.Cn) continue;
    float* arow = a.accbuf + (int64_t)rowl * a.ld_acc;
    char* xrow = a.dX + (int64_t)a.row_index[rowl] * a.lddx_b;
#pragma unroll
    for (int fn = 0; fn < NFN; ++fn) {
      const int32_t h = h0 + ec.col(fn);
      if (h >= a.H) continue;
      f32x4_t v = acc[fm][fn];
      if (a.mode == kDxStore) {
        *reinterpret_cast<f32x4_t*>(arow + h) = v;
      } else if (a.mode == kDxAdd) {
        v += *reinterpret_cast<const f32x4_t*>(arow + h);
        *reinterpret_cast<f32x4_t*>(arow + h) = v;
      } else {
        if (a.mode == kDxAddEmit) v += *reinterpret_cast<const f32x4_t*>(arow + h);
        const float o[4] = {v[0], v[1], v[2], v[3]};
        store4<T>(xrow + (int64_t)h * Elt<T>::kBytes, o);
      }
    }
  }
}

template <typename T>
MT_GEMM_KERNEL void dx_kernel(DxArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  uint32_t tm, tn;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.tiles_n, 4, tm, tn);
  const EpiCoords ec;
  FragOffsets fo;
  fo.init();
  const int32_t row0 = (int32_t)tm * 256;
  DirectLoader la;
  la.init([&](uint32_t r) __attribute__((always_inline)) { return a.G + (int64_t)(row0 + (int32_t)r) * a.ldg_b; });
  const int32_t h0 = (int32_t)tn * 256;
  TransLoader<T> lb;
  lb.init(a.W + (int64_t)h0 * Elt<T>::kBytes, a.ldw_b, a.V - a.v0, a.H - h0);
  f32x4_t acc[8][8];
  const int KT = (a.kv + Elt<T>::kBK - 1) / Elt<T>::kBK;
  mainloop<T>(lds, acc, la, lb, KT, fo);
  dx_epilogue<T, 8>(acc, a, ec, row0, h0);
}

// ===========================================================================
// Backward, step 3: dW[v0 : v0 + cv] (+)= G^T . X_block
// ===========================================================================
constexpr int kQueueWords = 8;
struct DwArgs {
  const char* G;  // [K = tokens][vocab], row pitch ldg_b
  int64_t ldg_b;
  int32_t g_rows;  // rows of G that exist (>= K rounded up to the K slab)
  int32_t g_cols;  // columns of G that exist
  const char* XcT;  // [H][K] gathered + transposed X rows of the block
  int64_t ldxt_b;
  uint32_t g_range, xt_range;  // bytes addressable from G, XcT
  int32_t kt_rows;  // K extent (valid rows of the block)
  int32_t H, cv, v0;
  float* dW;
  int64_t lddw;
  int32_t accumulate;
  int32_t tiles_m, tiles_n;
  // non-null: persistent schedule over a work queue (dw_bf16_kernel<true>):
  // kQueueWords counters, zero at launch, one per XCD's share of the tiles
  uint32_t* queue = nullptr;
  // tiled (bf16): dW in the library's tile order instead of rows of pitch
  // lddw, over two buffers: tile (tm, tn) at floats tile_pad + (tm tiles_n
  // + tn) 65536 from dW for tm < lo_rows, else at ((tm - lo_rows) tiles_n +
  // tn) 65536 from dW_hi; tm counted from vocabulary row 0 (the block's tile
  // rows start at v0 / 256, v0 a multiple of 256), wave w's fragment (fm,
  // fn) at ((w 64 + fm 8 + fn) 64 + lane) 4 within the tile
  int32_t tiled = 0;
  int64_t tile_pad = 0;
  float* dW_hi = nullptr;
  int32_t lo_rows = 0;
  // narrow (bf16, a dW every tile completes in one pass): dW is bf16 rows of
  // pitch lddw elements, each tile narrowed in its epilogue (kDwNarrow)
  int32_t narrow = 0;
};

// Where a bf16 dW kernel puts its tiles (template argument kOut): fp32 rows
// of pitch lddw, fp32 tiles (DwArgs::tiled), or -- for a dW that every tile
// completes in one pass (one row block, nothing added into) -- bf16 rows of
// pitch lddw (elements) at dW, narrowed in the epilogue.
constexpr int kDwRows = 0, kDwTiles = 1, kDwNarrow = 2;

template <int NFN, int WC>
__device__ __forceinline__ void dw_epilogue(const f32x4_t (&acc)[8][NFN], const DwArgs& a,
                                            const EpiCoordsT<NFN, WC>& ec, int32_t m0, int32_t h0) {
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    const int32_t vl = m0 + ec.row(fm);
    if (vl >= a.cv) continue;
    float* wrow = a.dW + (int64_t)(a.v0 + vl) * a.lddw;
#pragma unroll
    for (int fn = 0; fn < NFN; ++fn) {
      const int32_t h = h0 + ec.col(fn);
      if (h >= a.H) continue;
      f32x4_t v = acc[fm][fn];
      if (a.accumulate) v += *reinterpret_cast<const f32x4_t*>(wrow + h);
      *reinterpret_cast<f32x4_t*>(wrow + h) = v;
    }
  }
}

template <typename T>
MT_GEMM_KERNEL void dw_kernel(DwArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  uint32_t tm, tn;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.tiles_n, 4, tm, tn);
  const EpiCoords ec;
  FragOffsets fo;
  fo.init();
  const int32_t m0 = (int32_t)tm * 256;
  TransLoader<T> la;
  la.init(a.G + (int64_t)m0 * Elt<T>::kBytes, a.ldg_b, a.g_rows, a.g_cols - m0);
  const int32_t h0 = (int32_t)tn * 256;
  DirectLoader lb;
  lb.init([&](uint32_t r) __attribute__((always_inline)) {
    int32_t h = h0 + (int32_t)r;
    h = h < a.H ? h : a.H - 1;
    return a.XcT + (int64_t)h * a.ldxt_b;
  });
  f32x4_t acc[8][8];
  const int KT = (a.kt_rows + Elt<T>::kBK - 1) / Elt<T>::kBK;
  mainloop<T>(lds, acc, la, lb, KT, fo);
  dw_epilogue<8>(acc, a, ec, m0, h0);
}

// ===========================================================================
// Small kernels
// ===========================================================================

// XcT[h][t] = X[row_index[t]][h] for t < Cn, 0 for Cn <= t < t_pad.
// 64 x 64 element tiles; 16-byte loads along h, 16-byte stores along t.
// scale (non-null, bf16 only): row t is multiplied by scale[t] in fp32 and
// rounded to bf16 (the fused path's per-row factor of G, see
// fused_row_scale_kernel).
template <typename T>
__global__ __launch_bounds__(256) void gather_t_kernel(const char* X, int64_t ldx_b,
                                                       const int32_t* row_index, int32_t Cn,
                                                       int32_t H, char* XcT, int64_t ldxt_b,
                                                       const float* scale = nullptr) {
  constexpr int E = Elt<T>::kBytes;
  constexpr int PER = 16 / E;  // elements per 16-byte vector
  __shared__ T tile[64][64 + 1];
  const int32_t t0 = blockIdx.x * 64, hb = blockIdx.y * 64;
  // load 64 rows (t) x 64 h
  for (int v = threadIdx.x; v < 64 * 64 / PER; v += 256) {
    const int tr = v / (64 / PER), hc = (v % (64 / PER)) * PER;
    const int32_t t = t0 + tr;
    u32x4_t val = {0u, 0u, 0u, 0u};
    if (t < Cn && hb + hc < H)
      val = *reinterpret_cast<const u32x4_t*>(X + (int64_t)row_index[t] * ldx_b +
                                              (int64_t)(hb + hc) * E);
    if constexpr (sizeof(T) == 2) {
      if (scale && t < Cn) {
        const float sc = scale[t];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          val[j] = pack_bf16x2(__builtin_bit_cast(float, val[j] << 16) * sc,
                               __builtin_bit_cast(float, val[j] & 0xffff0000u) * sc);
      }
    }
    const T* e = reinterpret_cast<const T*>(&val);
#pragma unroll
    for (int j = 0; j < PER; ++j) tile[tr][hc + j] = e[j];
  }
  __syncthreads();
  for (int v = threadIdx.x; v < 64 * 64 / PER; v += 256) {
    const int hr = v / (64 / PER), tc = (v % (64 / PER)) * PER;
    if (hb + hr >= H) continue;
    u32x4_t val;
    T* e = reinterpret_cast<T*>(&val);
#pragma unroll
    for (int j = 0; j < PER; ++j) e[j] = tile[tc + j][hr];
    *reinterpret_cast<u32x4_t*>(XcT + (int64_t)(hb + hr) * ldxt_b + (int64_t)(t0 + tc) * E) = val;
  }
}

// Zero `nrows` rows (ids from rows[]) of a row-major matrix, row_bytes each
// (a multiple of 16).
__global__ __launch_bounds__(256) void zero_rows_kernel(char* base, int64_t ld_b,
                                                        const int32_t* rows, int64_t nrows,
                                                        int64_t row_bytes) {
  const int64_t nvec = row_bytes / 16;
  for (int64_t r = blockIdx.x; r < nrows; r += gridDim.x) {
    char* p = base + (int64_t)rows[r] * ld_b;
    for (int64_t v = threadIdx.x; v < nvec; v += blockDim.x)
      reinterpret_cast<u32x4_t*>(p)[v] = u32x4_t{0u, 0u, 0u, 0u};
  }
}

// Zero a dense [rows][cols] fp32 matrix with leading dimension ld.
__global__ __launch_bounds__(256) void zero_matrix_f32_kernel(float* p, int64_t rows, int64_t cols,
                                                              int64_t ld) {
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x)
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) p[r * ld + c] = 0.f;
}

__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }

// loss[rows[i]] = +0.0 for i < n.
__global__ __launch_bounds__(256) void zero_scatter_f32_kernel(float* loss, const int32_t* rows,
                                                               int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    loss[rows[i]] = 0.0f;
}

// Valid-row compaction in one workgroup of 1024 threads.
//   row_index[0 .. N)    positions t with a valid label, ascending
//   row_index[N .. T)    every other position (descending from the end)
//   row_label[0 .. N)    their labels
//   counts = {N, #labels outside [0, V), first such t or -1, 0}
__global__ __launch_bounds__(1024) void prepare_kernel(const int64_t* labels, int64_t T, int64_t V,
                                                       int64_t ignore, int shift, int32_t* row_index,
                                                       int32_t* row_label, int32_t* counts) {
  constexpr int kItems = 4;
  __shared__ int32_t wsum_v[16], wsum_m[16];
  __shared__ int32_t s_base_v, s_base_m, s_bad, s_first_bad;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) {
    s_base_v = 0;
    s_base_m = 0;
    s_bad = 0;
    s_first_bad = INT32_MAX;
  }
  __syncthreads();
  for (int64_t start = 0; start < T; start += 1024 * kItems) {
    int32_t y[kItems];
    uint32_t vmask = 0, mmask = 0;
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      const int64_t t = start + tid * kItems + j;
      y[j] = 0;
      if (t >= T) continue;
      int64_t lab;
      if (shift) lab = (t + 1 < T) ? labels[t + 1] : ignore;
      else lab = labels[t];
      if (lab == ignore) {
        mmask |= 1u << j;
      } else if (lab < 0 || lab >= V) {
        mmask |= 1u << j;
        atomicAdd(&s_bad, 1);
        atomicMin(&s_first_bad, (int32_t)t);
      } else {
        vmask |= 1u << j;
        y[j] = (int32_t)lab;
      }
    }
    const int cv = __builtin_popcount(vmask), cm = __builtin_popcount(mmask);
    // inclusive wave scans
    int sv = cv, sm = cm;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int tv = __shfl_up(sv, o), tmm = __shfl_up(sm, o);
      if (lane >= o) {
        sv += tv;
        sm += tmm;
      }
    }
    if (lane == 63) {
      wsum_v[wid] = sv;
      wsum_m[wid] = sm;
    }
    __syncthreads();
    int pv = 0, pm = 0, tv_all = 0, tm_all = 0;
    for (int w = 0; w < 16; ++w) {
      if (w < wid) {
        pv += wsum_v[w];
        pm += wsum_m[w];
      }
      tv_all += wsum_v[w];
      tm_all += wsum_m[w];
    }
    int ov = s_base_v + pv + sv - cv;
    int om = s_base_m + pm + sm - cm;
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      const int64_t t = start + tid * kItems + j;
      if (vmask & (1u << j)) {
        row_index[ov] = (int32_t)t;
        row_label[ov] = y[j];
        ++ov;
      } else if (mmask & (1u << j)) {
        row_index[T - 1 - om] = (int32_t)t;
        ++om;
      }
    }
    __syncthreads();
    if (tid == 0) {
      s_base_v += tv_all;
      s_base_m += tm_all;
    }
    __syncthreads();
  }
  if (tid == 0) {
    counts[0] = s_base_v;
    counts[1] = s_bad;
    counts[2] = s_bad ? s_first_bad : -1;
    counts[3] = 0;
  }
}

// status = 1 if cu_seqlens is not a valid partition of [0, T).
__global__ __launch_bounds__(256) void segment_check_kernel(const int32_t* cu, int64_t S, int64_t T,
                                                            int32_t* status) {
  __shared__ int32_t bad;
  if (threadIdx.x == 0) bad = (cu[0] != 0 || (int64_t)cu[S] != T) ? 1 : 0;
  __syncthreads();
  for (int64_t s = threadIdx.x; s < S; s += blockDim.x)
    if (cu[s + 1] < cu[s]) atomicOr(&bad, 1);
  __syncthreads();
  if (threadIdx.x == 0) *status = bad;
}

// One workgroup per sample: fixed-order tree sum of loss and count of valid
// targets over [cu[s], cu[s+1]).  With shift, the target of position t is
// labels[t + 1] (ignore_index at t = T - 1), as the causal shift forms it.
__global__ __launch_bounds__(256) void segment_sum_kernel(const float* loss, const int64_t* target,
                                                          int64_t T, int64_t ignore, int shift,
                                                          const int32_t* cu,
                                                          const int32_t* status, float* seg_loss,
                                                          int32_t* seg_count) {
  __shared__ float sl[256];
  __shared__ int32_t sc[256];
  const int64_t s = blockIdx.x;
  float acc = 0.f;
  int32_t cnt = 0;
  if (*status == 0) {
    for (int64_t t = cu[s] + threadIdx.x; t < cu[s + 1]; t += 256) {
      acc += loss[t];
      const int64_t src = t + (shift ? 1 : 0);
      cnt += (src < T && target[src] != ignore) ? 1 : 0;
    }
  }
  sl[threadIdx.x] = acc;
  sc[threadIdx.x] = cnt;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      sl[threadIdx.x] += sl[threadIdx.x + o];
      sc[threadIdx.x] += sc[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    seg_loss[s] = sl[0];
    seg_count[s] = sc[0];
  }
}

// ===========================================================================
// Gradients formed for a unit upstream gradient, rescaled once the real one
// is known: the reference's fused loss computes dX and dW in its forward and
// multiplies them by the scalar grad_output in its backward.  The scale is
// read from device memory (no host sync).  Rows are a grid-stride loop, 16
// bytes per thread and access; a column tail that is not a whole vector
// goes element by element.
// ===========================================================================

// dst[r, c] = scale * src[r, c] for an fp32 matrix; dst fp32 (may be src:
// every element is read and written by the same thread) or bf16 (round to
// nearest even).
template <bool kOutBf16>
__global__ __launch_bounds__(256) void scale_rows_f32_kernel(const float* src, int64_t ld_src,
                                                             void* dst, int64_t ld_dst,
                                                             int64_t rows, int64_t cols,
                                                             const float* scale) {
  const float c = *scale;
  const int64_t nv = cols / 4;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const float* s = src + r * ld_src;
    for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) {
      const f32x4_t x = reinterpret_cast<const f32x4_t*>(s)[v];
      const float y0 = x[0] * c, y1 = x[1] * c, y2 = x[2] * c, y3 = x[3] * c;
      if (kOutBf16) {
        u32x2_t o;
        o[0] = pack_bf16x2(y0, y1);
        o[1] = pack_bf16x2(y2, y3);
        reinterpret_cast<u32x2_t*>(static_cast<char*>(dst) + r * ld_dst * 2)[v] = o;
      } else {
        reinterpret_cast<f32x4_t*>(static_cast<float*>(dst) + r * ld_dst)[v] =
            f32x4_t{y0, y1, y2, y3};
      }
    }
    for (int64_t k = nv * 4 + threadIdx.x; k < cols; k += blockDim.x) {
      const float y = s[k] * c;
      if (kOutBf16)
        reinterpret_cast<__bf16*>(static_cast<char*>(dst) + r * ld_dst * 2)[k] = (__bf16)y;
      else
        (static_cast<float*>(dst) + r * ld_dst)[k] = y;
    }
  }
}

// In place: p[r, c] = bf16(scale * p[r, c]) for a bf16 matrix of row pitch
// ld_b bytes.
__global__ __launch_bounds__(256) void scale_rows_bf16_kernel(char* p, int64_t ld_b, int64_t rows,
                                                              int64_t cols, const float* scale) {
  const float c = *scale;
  const int64_t nv = cols / 8;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    u32x4_t* row = reinterpret_cast<u32x4_t*>(p + r * ld_b);
    for (int64_t v = threadIdx.x; v < nv; v += blockDim.x) {
      u32x4_t w = row[v];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = __builtin_bit_cast(float, w[j] << 16) * c;
        const float hi = __builtin_bit_cast(float, w[j] & 0xffff0000u) * c;
        w[j] = pack_bf16x2(lo, hi);
      }
      row[v] = w;
    }
    __bf16* e = reinterpret_cast<__bf16*>(p + r * ld_b);
    for (int64_t k = nv * 8 + threadIdx.x; k < cols; k += blockDim.x)
      e[k] = (__bf16)((float)e[k] * c);
  }
}

// In-place narrowing: bf16 row r = scale * fp32 row r, written to the first
// bytes of the same allocation (bf16 row r at element offset r * ld in bf16
// units, i.e. bytes [2 r ld, 2 r ld + 2 cols)), so the weight gradient in the
// weight's dtype needs no second buffer.  bf16 row r overlaps fp32 row
// floor(r / 2) only, so one launch per phase of rows -- {0}, {1}, [2, 4),
// [4, 8), ... -- overwrites only rows an earlier phase has consumed; within a
// row (row 0 overlaps itself) the workgroup reads the whole row before any of
// it is written.  kPer 16-byte vectors per thread cover cols <= 1024 kPer.
template <int kPer>
__global__ __launch_bounds__(256) void narrow_rows_inplace_kernel(float* base, int64_t ld,
                                                                  int64_t r0, int64_t r1,
                                                                  int64_t cols,
                                                                  const float* scale) {
  const float c = *scale;
  const int64_t nv = cols / 4, nt = cols - nv * 4;
  for (int64_t r = r0 + blockIdx.x; r < r1; r += gridDim.x) {
    const float* src = base + r * ld;
    f32x4_t v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t idx = threadIdx.x + (int64_t)i * 256;
      v[i] = idx < nv ? reinterpret_cast<const f32x4_t*>(src)[idx] : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    const float t = (int64_t)threadIdx.x < nt ? src[nv * 4 + threadIdx.x] : 0.f;
    __syncthreads();
    char* dst = reinterpret_cast<char*>(base) + r * ld * 2;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t idx = threadIdx.x + (int64_t)i * 256;
      if (idx < nv) {
        u32x2_t o;
        o[0] = pack_bf16x2(v[i][0] * c, v[i][1] * c);
        o[1] = pack_bf16x2(v[i][2] * c, v[i][3] * c);
        reinterpret_cast<u32x2_t*>(dst)[idx] = o;
      }
    }
    if ((int64_t)threadIdx.x < nt)
      reinterpret_cast<__bf16*>(dst)[nv * 4 + threadIdx.x] = (__bf16)(t * c);
    __syncthreads();
  }
}

// ===========================================================================
// Cross-entropy over materialised logits [T, V] (reduction 'none').
// One workgroup of 256 threads per row; 16-byte loads along V.
// ===========================================================================
template <typename T>
__device__ __forceinline__ void load_vec(const char* p, float (&x)[16 / sizeof(T)]);
template <>
__device__ __forceinline__ void load_vec<float>(const char* p, float (&x)[4]) {
  f32x4_t v = *reinterpret_cast<const f32x4_t*>(p);
  x[0] = v[0];
  x[1] = v[1];
  x[2] = v[2];
  x[3] = v[3];
}
template <>
__device__ __forceinline__ void load_vec<__bf16>(const char* p, float (&x)[8]) {
  u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = v[i];
    x[2 * i] = __builtin_bit_cast(float, w << 16);
    x[2 * i + 1] = __builtin_bit_cast(float, w & 0xffff0000u);
  }
}
template <typename T>
__device__ __forceinline__ float load_one(const char* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const float*>(p);
  } else {
    return __builtin_bit_cast(float, (uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
  }
}

// 16 bytes of T from floats (bf16: rounded to nearest even).
template <typename T>
__device__ __forceinline__ void store_vec(char* p, const float (&x)[16 / sizeof(T)]) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x4_t*>(p) = f32x4_t{x[0], x[1], x[2], x[3]};
  } else {
    u32x4_t v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    *reinterpret_cast<u32x4_t*>(p) = v;
  }
}

// Block-wide merge of per-thread (m, d) states; result valid in all threads.
__device__ __forceinline__ void block_lse_merge(float& m, float& d, float* sm) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) lse_merge(m, d, __shfl_xor(m, o), __shfl_xor(d, o));
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    sm[2 * w] = m;
    sm[2 * w + 1] = d;
  }
  __syncthreads();
  m = kNegBig;
  d = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) lse_merge(m, d, sm[2 * i], sm[2 * i + 1]);
}

template <typename T>
__global__ __launch_bounds__(256) void ce_forward_kernel(const char* logits, int64_t V, int64_t ld_b,
                                                         const int64_t* target, int64_t ignore,
                                                         float* loss, float* lse, int32_t* status) {
  constexpr int E = sizeof(T), VEC = 16 / E;
  __shared__ float sm[16];
  const int64_t t = blockIdx.x;
  const int64_t y = target[t];
  if (y == ignore) {
    if (threadIdx.x == 0) {
      loss[t] = 0.0f;
      lse[t] = 0.0f;
    }
    return;
  }
  if (y < 0 || y >= V) {
    if (threadIdx.x == 0) {
      atomicOr(status, 1);
      loss[t] = 0.0f;
      lse[t] = 0.0f;
    }
    return;
  }
  const char* row = logits + t * ld_b;
  float m = kNegBig, d = 0.f;
  // scalar head up to 16-byte alignment, 16-byte vectors, scalar tail
  const int64_t mis = (int64_t)(reinterpret_cast<uintptr_t>(row) & 15u) / E;
  const int64_t head = mis ? min<int64_t>(VEC - mis, V) : 0;
  const int64_t nvec = (V - head) / VEC;
  const char* vrow = row + head * E;
  auto merge_vec = [&](const float (&x)[VEC]) __attribute__((always_inline)) {
    float mx = x[0];
#pragma unroll
    for (int j = 1; j < VEC; ++j) mx = fmaxf(mx, x[j]);
    const float mn = fmaxf(m, mx * kLog2e);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) s += fast_exp2(fmaf(x[j], kLog2e, -mn));
    d = fmaf(d, fast_exp2(m - mn), s);
    m = mn;
  };
  // four 16-byte loads in flight per thread
  int64_t i = threadIdx.x;
  for (; i + 3 * 256 < nvec; i += 4 * 256) {
    float x[4][VEC];
#pragma unroll
    for (int k = 0; k < 4; ++k) load_vec<T>(vrow + (i + k * 256) * 16, x[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) merge_vec(x[k]);
  }
  for (; i < nvec; i += 256) {
    float x[VEC];
    load_vec<T>(vrow + i * 16, x);
    merge_vec(x);
  }
  for (int64_t v = threadIdx.x; v < head; v += 256) lse_merge(m, d, load_one<T>(row + v * E) * kLog2e, 1.0f);
  for (int64_t v = head + nvec * VEC + threadIdx.x; v < V; v += 256)
    lse_merge(m, d, load_one<T>(row + v * E) * kLog2e, 1.0f);
  block_lse_merge(m, d, sm);
  if (threadIdx.x == 0) {
    const float L = (m + fast_log2(d)) * kLn2;
    lse[t] = L;
    loss[t] = L - load_one<T>(row + y * E);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ce_backward_kernel(const char* logits, int64_t V, int64_t ld_b,
                                                          const int64_t* target, int64_t ignore,
                                                          const float* lse, const float* grad,
                                                          int64_t gstride, char* dlogits,
                                                          int64_t ldd_b) {
  constexpr int E = sizeof(T);
  const int64_t t = blockIdx.x;
  const int64_t y = target[t];
  const bool valid = y != ignore && y >= 0 && y < V;
  const float g = valid ? grad[t * gstride] : 0.f;
  const float l2 = valid ? lse[t] * kLog2e : 0.f;
  const char* row = logits + t * ld_b;
  char* drow = dlogits + t * ldd_b;
  constexpr int VEC = 16 / E;
  if (((reinterpret_cast<uintptr_t>(row) | reinterpret_cast<uintptr_t>(drow)) & 15u) == 0) {
    // 16-byte rows (the usual case): whole vectors, four loads in flight per
    // thread, then the scalar tail of V mod VEC
    const int64_t nvec = V / VEC;
    auto grad_vec = [&](float (&x)[VEC], int64_t c0) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float p = fast_exp2(fmaf(x[j], kLog2e, -l2));
        x[j] = valid ? g * (p - (c0 + j == y ? 1.f : 0.f)) : 0.f;
      }
    };
    int64_t i = threadIdx.x;
    for (; i + 3 * 256 < nvec; i += 4 * 256) {
      float x[4][VEC];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (valid) load_vec<T>(row + (i + k * 256) * 16, x[k]);
        else
#pragma unroll
          for (int j = 0; j < VEC; ++j) x[k][j] = 0.f;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        grad_vec(x[k], (i + k * 256) * VEC);
        store_vec<T>(drow + (i + k * 256) * 16, x[k]);
      }
    }
    for (; i < nvec; i += 256) {
      float x[VEC];
      if (valid) load_vec<T>(row + i * 16, x);
      else
#pragma unroll
        for (int j = 0; j < VEC; ++j) x[j] = 0.f;
      grad_vec(x, i * VEC);
      store_vec<T>(drow + i * 16, x);
    }
    for (int64_t c = nvec * VEC + threadIdx.x; c < V; c += 256) {
      float r = 0.f;
      if (valid) r = g * (fast_exp2(fmaf(load_one<T>(row + c * E), kLog2e, -l2)) - (c == y ? 1.f : 0.f));
      if constexpr (E == 4)
        reinterpret_cast<float*>(drow)[c] = r;
      else
        *reinterpret_cast<uint16_t*>(drow + c * 2) = (uint16_t)(pack_bf16x2(r, 0.f) & 0xffffu);
    }
    return;
  }
  // any alignment: pairs of elements so bf16 rows are written 4 bytes at a time
  for (int64_t v = 2 * threadIdx.x; v < V; v += 512) {
    float o[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t c = v + j;
      float r = 0.f;
      if (valid && c < V) {
        const float p = fast_exp2(fmaf(load_one<T>(row + c * E), kLog2e, -l2));
        r = g * (p - (c == y ? 1.f : 0.f));
      }
      o[j] = r;
    }
    if constexpr (E == 4) {
      reinterpret_cast<float*>(drow)[v] = o[0];
      if (v + 1 < V) reinterpret_cast<float*>(drow)[v + 1] = o[1];
    } else {
      const uint32_t pk = pack_bf16x2(o[0], o[1]);
      char* p = drow + v * 2;
      if (v + 1 < V && (reinterpret_cast<uintptr_t>(p) & 3u) == 0) {
        *reinterpret_cast<uint32_t*>(p) = pk;
      } else {
        *reinterpret_cast<uint16_t*>(p) = (uint16_t)(pk & 0xffffu);
        if (v + 1 < V) *reinterpret_cast<uint16_t*>(p + 2) = (uint16_t)(pk >> 16);
      }
    }
  }
}

}  // namespace mtf
