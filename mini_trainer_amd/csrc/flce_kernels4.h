// bf16 kernels on the eight-wave main loop (flce_gemm4.h): output tiles of
// 256 x 256, wave tiles 128 x 64.  Arguments, accumulation order and
// epilogues are those of the generic kernels in flce_kernels.h (the fp32
// path).
#pragma once

#include "flce_gemm4.h"
#include "flce_kernels.h"

namespace mtf {

#define MT_GEMM4_KERNEL \
  __global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))

typedef EpiCoordsT<4, 4> EpiCoords4;

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
  __device__ __forceinline__ int count() const {
    return first < total ? (int)((total - first + stride - 1) / stride) : 0;
  }
  __device__ __forceinline__ uint32_t logical(int k) const { return first + (uint32_t)k * stride; }
};

// Forward: one 256 x 256 logits tile per work unit (A = gathered X rows, B =
// W rows), persistent over the (row tile, vocabulary tile) grid.  The
// epilogue reduces the tile to a (max, sum) partial per row -- lanes that
// share a row through shuffles, the four wave columns through a 6 KiB LDS
// region beside the stage buffers -- and writes it to part[vocab tile][row];
// the lane that holds a row's label logit writes it to xy[row].  Nothing is
// carried in registers from one tile to the next.
// With kStoreS the tile's bf16-rounded logits (before the softcap) are also
// written to S, row = compacted row of the chunk, column = vocabulary index:
// the fused path forms G from them in place once the row's lse is known.
constexpr int kFwdRed4 = 3 * 256 * 2 * (int)sizeof(float);
// Row tiles per group of the forward's tile walk: W (the larger operand) is
// streamed once per group, so wider groups cut its re-reads (8: 2% faster
// than 4 at config 3; 16 is no better and costs L2 hits).
constexpr uint32_t kFwdGroup4 = 8;

template <bool kCap, bool kStoreS>
MT_GEMM4_KERNEL void fwd4_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds4 + kFwdRed4];
  const TileSeq seq((uint32_t)(a.tiles_m * a.vt_total));
  const EpiCoords4 ec;
  Kc4 A, B;
  A.init_frag(ec.wm * 128);
  B.init_frag(ec.wn * 64);
  mainloop4(
      lds, A, B, a.H / kBK4, seq.count(),
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tv;
        grouped_tile(seq.logical(k), a.tiles_m, a.vt_total, kFwdGroup4, tm, tv);
        const int32_t row0 = (int32_t)tm * 256, vrow0 = (int32_t)tv * 256;
        A.set_rows(make_rsrc(a.X, kWholeRange), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t rr = row0 + (int32_t)r;
          rr = rr < a.N ? rr : a.N - 1;
          return (uint32_t)a.row_index[rr] * (uint32_t)a.ldx_b;
        });
        B.set_rows(make_rsrc(a.W, kWholeRange), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t v = vrow0 + (int32_t)r;
          v = v < a.V ? v : a.V - 1;
          return (uint32_t)v * (uint32_t)a.ldw_b;
        });
      },
      [&](int k, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
        uint32_t tm, tv;
        grouped_tile(seq.logical(k), a.tiles_m, a.vt_total, kFwdGroup4, tm, tv);
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
        fwd_tile_update<__bf16, kCap>(acc, m2, d, lbl, rglob, (int32_t)tv * 256, ec, a);
        if (kStoreS) {
#pragma unroll
          for (int fm = 0; fm < 8; ++fm) {
            char* srow = a.S + (int64_t)rglob[fm] * a.lds_b;
#pragma unroll
            for (int fn = 0; fn < 4; ++fn) {
              const float o[4] = {acc[fm][fn][0], acc[fm][fn][1], acc[fm][fn][2], acc[fm][fn][3]};
              store4<__bf16>(srow + (int64_t)((int32_t)tv * 256 + ec.col(fn)) * 2, o);
            }
          }
        }
        fwd_final_merge(lds + kLds4, m2, d, rglob, tv, ec, a);
      });
}

// Backward step 1: A = X rows of the block (256 tokens), B = W rows (256
// vocabulary entries); the epilogue writes G.
template <bool kCap>
MT_GEMM4_KERNEL void recompute4_kernel(RecompArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds4];
  const TileSeq seq((uint32_t)(a.tiles_m * a.tiles_n));
  const EpiCoords4 ec;
  Kc4 A, B;
  A.init_frag(ec.wm * 128);
  B.init_frag(ec.wn * 64);
  mainloop4(
      lds, A, B, a.H / kBK4, seq.count(),
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t row0 = (int32_t)tm * 256, vrow0 = a.v0 + (int32_t)tn * 256;
        A.set_rows(make_rsrc(a.X, kWholeRange), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t rr = row0 + (int32_t)r;
          rr = rr < a.Cn ? rr : a.Cn - 1;
          return (uint32_t)a.row_index[rr] * (uint32_t)a.ldx_b;
        });
        B.set_rows(make_rsrc(a.W, kWholeRange), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t v = vrow0 + (int32_t)r;
          v = v < a.V ? v : a.V - 1;
          return (uint32_t)v * (uint32_t)a.ldw_b;
        });
      },
      [&](int k, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t row0 = (int32_t)tm * 256, col0 = (int32_t)tn * 256;
        recompute_epilogue<__bf16, 4, kCap>(acc, a, ec, row0, col0);
      });
}

// Backward step 2: A = G rows (256 tokens, K = vocabulary), B = W read
// K-major (256 hidden columns).
MT_GEMM4_KERNEL void dx4_kernel(DxArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds4];
  const TileSeq seq((uint32_t)(a.tiles_m * a.tiles_n));
  const EpiCoords4 ec;
  Kc4 A;
  Tr4 B;
  A.init_frag(ec.wm * 128);
  mainloop4(
      lds, A, B, (a.kv + kBK4 - 1) / kBK4, seq.count(),
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t row0 = (int32_t)tm * 256, h0 = (int32_t)tn * 256;
        A.set_rows(make_rsrc(a.G, kWholeRange), [&](uint32_t r) __attribute__((always_inline)) {
          return (uint32_t)(row0 + (int32_t)r) * (uint32_t)a.ldg_b;
        });
        B.init(make_rsrc(a.W, kWholeRange), (uint32_t)a.v0 * (uint32_t)a.ldw_b + (uint32_t)h0 * 2u,
               (uint32_t)a.ldw_b, a.V - a.v0, a.H - h0, ec.wn * 64);
      },
      [&](int k, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        dx_epilogue<__bf16>(acc, a, ec, (int32_t)tm * 256, (int32_t)tn * 256);
      });
}

// Backward step 3: A = G read K-major (256 vocabulary columns, K = tokens),
// B = X^T rows of the block (256 hidden rows).
MT_GEMM4_KERNEL void dw4_kernel(DwArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds4];
  const TileSeq seq((uint32_t)(a.tiles_m * a.tiles_n));
  const EpiCoords4 ec;
  Tr4 A;
  Kc4 B;
  B.init_frag(ec.wn * 64);
  mainloop4(
      lds, A, B, (a.kt_rows + kBK4 - 1) / kBK4, seq.count(),
      [&](int k) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        const int32_t m0 = (int32_t)tm * 256, h0 = (int32_t)tn * 256;
        A.init(make_rsrc(a.G, kWholeRange), (uint32_t)m0 * 2u, (uint32_t)a.ldg_b, a.g_rows,
               a.g_cols - m0, ec.wm * 128);
        B.set_rows(make_rsrc(a.XcT, kWholeRange), [&](uint32_t r) __attribute__((always_inline)) {
          int32_t h = h0 + (int32_t)r;
          h = h < a.H ? h : a.H - 1;
          return (uint32_t)h * (uint32_t)a.ldxt_b;
        });
      },
      [&](int k, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
        uint32_t tm, tn;
        grouped_tile(seq.logical(k), a.tiles_m, a.tiles_n, 4, tm, tn);
        dw_epilogue(acc, a, ec, (int32_t)tm * 256, (int32_t)tn * 256);
      });
}

// Fused path: G = g_t (softmax(cap(S_t)) - onehot(y_t)) (1 - tanh^2), in place
// over one chunk of the bf16 logits S written by fwd4_kernel<*, true>.  One
// workgroup per row; rows >= cn and columns >= V become 0.  HBM-bound: one
// 16-byte read and one 16-byte write per 8 elements.
__global__ __launch_bounds__(256) void softmax_grad_kernel(char* S, int64_t lds_b, int32_t cols,
                                                           int32_t cn, int32_t V,
                                                           const float* lse, const float* grad,
                                                           int64_t gstride,
                                                           const int32_t* row_index,
                                                           const int32_t* row_label,
                                                           float softcap) {
  const int32_t row = blockIdx.x;
  const bool rv = row < cn;
  const float lse2 = rv ? lse[row] * kLog2e : 0.f;
  const float g = rv ? grad[(int64_t)row_index[row] * gstride] : 0.f;
  const int32_t y = rv ? row_label[row] : -1;
  const bool cap = softcap > 0.f;
  const float inv_cap = cap ? 1.0f / softcap : 0.f;
  u32x4_t* p = reinterpret_cast<u32x4_t*>(S + (int64_t)row * lds_b);
  for (int32_t c = threadIdx.x * 8; c < cols; c += 256 * 8) {
    u32x4_t v = p[c / 8];
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = v[j / 2];
      float x = __builtin_bit_cast(float, (j & 1) ? (w & 0xffff0000u) : (w << 16));
      float dcap = 1.f;
      if (cap) {
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
    p[c / 8] = r;
  }
}

}  // namespace mtf
