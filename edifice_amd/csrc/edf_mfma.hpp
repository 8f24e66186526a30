// MFMA fragment types and the lane layout of v_mfma_f32_32x32x16_bf16 (gfx950).
//
// For D[32x32] += A[32x16] * B[16x32] executed by one wave (lane l, g = l / 32):
//   A operand  lane l holds A[l % 32][8 g .. 8 g + 7]           (8 bf16)
//   B operand  lane l holds B[8 g .. 8 g + 7][l % 32]           (8 bf16)
//   D          lane l, register r holds D[8 (r / 4) + 4 g + (r % 4)][l % 32]
// i.e. a lane owns one column of the result.  The layout is checked on the GPU by
// tests/test_gpu_mfma_layout.py through edf_debug_mfma_32x32x16_bf16().
#pragma once

#include "edf_common.hpp"

namespace edf {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;

EDF_DEVICE f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

EDF_DEVICE bf16x8 cat4(bf16x4 lo, bf16x4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

EDF_DEVICE f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Row (within the 32-row tile) held by register r of a lane in half g.
EDF_DEVICE constexpr int d_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

}  // namespace edf
