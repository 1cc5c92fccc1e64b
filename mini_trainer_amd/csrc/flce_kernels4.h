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
constexpr int kFwdRed4 = 3 * 256 * 2 * (int)sizeof(float);

template <bool kCap>
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
        grouped_tile(seq.logical(k), a.tiles_m, a.vt_total, 4, tm, tv);
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
        grouped_tile(seq.logical(k), a.tiles_m, a.vt_total, 4, tm, tv);
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

}  // namespace mtf
