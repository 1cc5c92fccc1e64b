// bf16 kernels on the two-workgroups-per-CU main loop (flce_gemm3.h): output
// tiles of 256 x 128, wave tiles 128 x 64.  Arguments, accumulation order and
// epilogues are those of the generic kernels in flce_kernels.h (the fp32 path).
#pragma once

#include "flce_gemm3.h"
#include "flce_kernels.h"

namespace mtf {

#define MT_GEMM3_KERNEL \
  __global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2, 2)))

typedef EpiCoordsT<4> EpiCoords3;

// Forward: A = gathered X rows (256 tokens), B = W rows (128 vocabulary
// entries per tile), streaming over this workgroup's vocabulary tiles.
MT_GEMM3_KERNEL void fwd3_kernel(FwdArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds3];
  uint32_t tm, ts;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.splits, 4, tm, ts);
  const EpiCoords3 ec;
  const int32_t row0 = (int32_t)tm * kRowsA3;
  KcOp<kRowsA3> A;
  KcOp<kRowsB3> B;
  A.set_rows([&](uint32_t r) __attribute__((always_inline)) {
    int32_t rr = row0 + (int32_t)r;
    rr = rr < a.N ? rr : a.N - 1;
    return a.X + (int64_t)a.row_index[rr] * a.ldx_b;
  });
  A.init_frag(ec.wm * 128);
  B.init_frag(ec.wn * 64);

  int32_t lbl[8], rglob[8];
  float m2[8], d[8];
#pragma unroll
  for (int fm = 0; fm < 8; ++fm) {
    rglob[fm] = row0 + ec.row(fm);
    lbl[fm] = rglob[fm] < a.N ? a.row_label[rglob[fm]] : -1;
    m2[fm] = kNegBig;
    d[fm] = 0.f;
  }
  const int vt0 = (int)ts * a.vt_per_split;
  const int ntiles = min(vt0 + a.vt_per_split, a.vt_total) - vt0;
  mainloop3(
      lds, A, B, a.H / kBK3, ntiles,
      [&](int tile) __attribute__((always_inline)) {
        const int32_t vrow0 = (vt0 + tile) * kRowsB3;
        B.set_rows([&](uint32_t r) __attribute__((always_inline)) {
          int32_t v = vrow0 + (int32_t)r;
          v = v < a.V ? v : a.V - 1;
          return a.W + (int64_t)v * a.ldw_b;
        });
      },
      [&](int tile, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
        fwd_tile_update<__bf16, 4>(acc, m2, d, lbl, rglob, (vt0 + tile) * kRowsB3, ec, a);
      });
  fwd_final_merge<4>(lds, m2, d, rglob, ts, ec, a);
}

// Backward step 1: A = X rows of the block (256 tokens), B = W rows (128
// vocabulary entries); epilogue writes G.
MT_GEMM3_KERNEL void recompute3_kernel(RecompArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds3];
  uint32_t tm, tn;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.tiles_n, 4, tm, tn);
  const EpiCoords3 ec;
  const int32_t row0 = (int32_t)tm * kRowsA3, col0 = (int32_t)tn * kRowsB3;
  const int32_t vrow0 = a.v0 + col0;
  KcOp<kRowsA3> A;
  KcOp<kRowsB3> B;
  A.set_rows([&](uint32_t r) __attribute__((always_inline)) {
    int32_t rr = row0 + (int32_t)r;
    rr = rr < a.Cn ? rr : a.Cn - 1;
    return a.X + (int64_t)a.row_index[rr] * a.ldx_b;
  });
  B.set_rows([&](uint32_t r) __attribute__((always_inline)) {
    int32_t v = vrow0 + (int32_t)r;
    v = v < a.V ? v : a.V - 1;
    return a.W + (int64_t)v * a.ldw_b;
  });
  A.init_frag(ec.wm * 128);
  B.init_frag(ec.wn * 64);
  mainloop3(lds, A, B, a.H / kBK3, 1, [](int) __attribute__((always_inline)) {},
            [&](int, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
              if (a.softcap > 0.f) recompute_epilogue<__bf16, 4, true>(acc, a, ec, row0, col0);
              else recompute_epilogue<__bf16, 4, false>(acc, a, ec, row0, col0);
            });
}

// Backward step 2: A = G rows (256 tokens, K = vocabulary), B = W read
// K-major (128 hidden columns).
MT_GEMM3_KERNEL void dx3_kernel(DxArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds3];
  uint32_t tm, tn;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.tiles_n, 4, tm, tn);
  const EpiCoords3 ec;
  const int32_t row0 = (int32_t)tm * kRowsA3, h0 = (int32_t)tn * kRowsB3;
  KcOp<kRowsA3> A;
  A.set_rows([&](uint32_t r) __attribute__((always_inline)) {
    return a.G + (int64_t)(row0 + (int32_t)r) * a.ldg_b;
  });
  A.init_frag(ec.wm * 128);
  TrOp<kRowsB3> B;
  B.init(a.W + (int64_t)a.v0 * a.ldw_b + (int64_t)h0 * 2, a.ldw_b, a.V - a.v0, a.H - h0,
         ec.wn * 64);
  mainloop3(lds, A, B, (a.kv + kBK3 - 1) / kBK3, 1, [](int) __attribute__((always_inline)) {},
            [&](int, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
              dx_epilogue<__bf16, 4>(acc, a, ec, row0, h0);
            });
}

// Backward step 3: A = G read K-major (256 vocabulary columns, K = tokens),
// B = X^T rows of the block (128 hidden rows).
MT_GEMM3_KERNEL void dw3_kernel(DwArgs a) {
  __shared__ __attribute__((aligned(1024))) char lds[kLds3];
  uint32_t tm, tn;
  grouped_tile(xcd_remap(blockIdx.x, gridDim.x), a.tiles_m, a.tiles_n, 4, tm, tn);
  const EpiCoords3 ec;
  const int32_t m0 = (int32_t)tm * kRowsA3, h0 = (int32_t)tn * kRowsB3;
  TrOp<kRowsA3> A;
  A.init(a.G + (int64_t)m0 * 2, a.ldg_b, a.g_rows, a.g_cols - m0, ec.wm * 128);
  KcOp<kRowsB3> B;
  B.set_rows([&](uint32_t r) __attribute__((always_inline)) {
    int32_t h = h0 + (int32_t)r;
    h = h < a.H ? h : a.H - 1;
    return a.XcT + (int64_t)h * a.ldxt_b;
  });
  B.init_frag(ec.wn * 64);
  mainloop3(lds, A, B, (a.kt_rows + kBK3 - 1) / kBK3, 1, [](int) __attribute__((always_inline)) {},
            [&](int, f32x4_t(&acc)[8][4]) __attribute__((always_inline)) {
              dw_epilogue<4>(acc, a, ec, m0, h0);
            });
}

}  // namespace mtf
