// Measurement kernel (no counterpart in the reference): a register-only
// stream of bf16 MFMAs, the ceiling that the GEMM kernels' main loops are
// measured against.  One four-wave workgroup per CU (the 160 KiB of LDS it
// reserves keep a second one off the CU), every wave a GEMM-shaped grid of
// independent accumulators over operand registers loaded once from
// `operands` (caller-chosen values, e.g. random bf16): kShape 0 = 8 x 8
// v_mfma_f32_16x16x32_bf16 per iteration (the GEMM kernels' instruction),
// 1 = 4 x 4 v_mfma_f32_32x32x16_bf16.  No memory traffic inside the loop;
// each thread writes the sum of its accumulators to out[] at the end.
#pragma once

#include "flce_device.h"

namespace mtf {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int kShape>
__global__ __launch_bounds__(256) void mfma_probe_kernel(const u32x4_t* operands, float* out,
                                                         int32_t iters, int32_t touch_lds) {
  __shared__ char reserve[160 * 1024];
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  float s = 0.f;
  if constexpr (kShape == 0) {
    bf16x8_t a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = __builtin_bit_cast(bf16x8_t, operands[gid * 16 + i]);
      b[i] = __builtin_bit_cast(bf16x8_t, operands[gid * 16 + 8 + i]);
    }
    f32x4_t acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int32_t it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) s += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  } else {
    bf16x8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = __builtin_bit_cast(bf16x8_t, operands[gid * 16 + i]);
      b[i] = __builtin_bit_cast(bf16x8_t, operands[gid * 16 + 8 + i]);
    }
    f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    for (int32_t it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][j][r];
  }
  if (touch_lds) {  // never set by the library: keeps the reservation in the kernel
    reserve[threadIdx.x] = (char)s;
    __syncthreads();
    s += reserve[(threadIdx.x + 1) & 255];
  }
  out[gid] = s;
}

}  // namespace mtf
