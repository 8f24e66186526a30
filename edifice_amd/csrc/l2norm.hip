// L2 normalisation of rows, forward and backward: the DeltaNet / GatedDeltaNet key norm
// k / sqrt(sum k^2 + eps) (lib/edifice/recurrent/delta_net.ex:291,
// gated_delta_net.ex:387, eps inside the square root), block glue in front of the delta rule.
//   y = x r,  r = 1 / sqrt(sum_j x_j^2 + eps);   dx = r (dy - y <y, dy>)
// x, y, dy, dx [rows, d] in the io dtype, f32 inside.  A 16-lane DPP row holds one row of x
// (16-byte accesses: 8 bf16 or 4 f32 per lane and step, d up to 16 vectors per lane's share),
// its sums by a row butterfly; rows whose length is not a multiple of the vector, or
// misaligned tensors, take one element per lane and step.  The backward recomputes r from x.
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int L2_NT = 256;      // 16 rows per workgroup (a 16-lane group per row)
constexpr int L2_MAX_D = 1024;

template <typename T> struct L2Vec;
template <> struct L2Vec<bf16> {
  static constexpr int W = 8;
  static EDF_DEVICE void ld(const bf16* p, float* v) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const unsigned w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __builtin_bit_cast(float, w4[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, w4[i] & 0xffff0000u);
    }
  }
  static EDF_DEVICE void st(bf16* p, const float* v) {
    unsigned w4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w4[i] = (unsigned)__builtin_bit_cast(unsigned short, (bf16)v[2 * i]) |
              ((unsigned)__builtin_bit_cast(unsigned short, (bf16)v[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
};
template <> struct L2Vec<float> {
  static constexpr int W = 4;
  static EDF_DEVICE void ld(const float* p, float* v) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  static EDF_DEVICE void st(float* p, const float* v) { *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]); }
};

// NV vectors per lane (row length <= 16 NV W); NV = 0: one element per lane and step
template <typename T, bool BWD, int NV>
__global__ __launch_bounds__(L2_NT) void l2_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                  T* __restrict__ out, long rows, int d, float eps) {
  constexpr int W = L2Vec<T>::W;
  const int i16 = threadIdx.x & 15;
  const long r = (long)blockIdx.x * (L2_NT / 16) + (threadIdx.x >> 4);
  // rows past the end compute on row rows - 1 (every lane of a DPP row takes part in its
  // butterfly) and store nothing
  const bool live = r < rows;
  const long rr = live ? r : rows - 1;
  const T* xr = x + rr * d;
  if constexpr (NV > 0) {
    float v[NV][W], g[NV][W];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 16 + i16) * W;
      if (c0 < d) {
        L2Vec<T>::ld(xr + c0, v[k]);
        if constexpr (BWD) L2Vec<T>::ld(dy + rr * d + c0, g[k]);
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) v[k][i] = g[k][i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) ss = fmaf(v[k][i], v[k][i], ss);
    }
    const float rn = 1.0f / sqrtf(row16_sum(ss) + eps);
    float dot = 0.0f;
    if constexpr (BWD) {
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int i = 0; i < W; ++i) dot = fmaf(v[k][i] * rn, g[k][i], dot);
      dot = row16_sum(dot);
    }
    if (!live) return;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 16 + i16) * W;
      if (c0 >= d) continue;
      float o[W];
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const float y = v[k][i] * rn;
        o[i] = BWD ? rn * fmaf(-y, dot, g[k][i]) : y;
      }
      L2Vec<T>::st(out + rr * d + c0, o);
    }
  } else {
    float ss = 0.0f;
    for (int c = i16; c < d; c += 16) {
      const float a = to_f32(xr[c]);
      ss = fmaf(a, a, ss);
    }
    const float rn = 1.0f / sqrtf(row16_sum(ss) + eps);
    float dot = 0.0f;
    if constexpr (BWD) {
      for (int c = i16; c < d; c += 16) dot = fmaf(to_f32(xr[c]) * rn, to_f32(dy[rr * d + c]), dot);
      dot = row16_sum(dot);
    }
    if (!live) return;
    for (int c = i16; c < d; c += 16) {
      const float y = to_f32(xr[c]) * rn;
      out[rr * d + c] = from_f32<T>(BWD ? rn * fmaf(-y, dot, to_f32(dy[rr * d + c])) : y);
    }
  }
}

template <typename T, bool BWD>
int l2_run(hipStream_t s, const void* x, const void* dy, void* out, long rows, int d, float eps) {
  constexpr int W = L2Vec<T>::W;
  const unsigned grid = (unsigned)((rows + L2_NT / 16 - 1) / (L2_NT / 16));
  const bool al = !(((uintptr_t)x | (uintptr_t)out | (BWD ? (uintptr_t)dy : 0)) & 15);
  const int nvec = d / W;
  int nv = 0;
  if (al && d % W == 0)
    for (int c : {1, 2, 4, 8})
      if (nvec <= 16 * c) {
        nv = c;
        break;
      }
  const T* xp = (const T*)x;
  const T* gp = (const T*)dy;
  T* op = (T*)out;
  switch (nv) {
    case 1: l2_kernel<T, BWD, 1><<<grid, L2_NT, 0, s>>>(xp, gp, op, rows, d, eps); break;
    case 2: l2_kernel<T, BWD, 2><<<grid, L2_NT, 0, s>>>(xp, gp, op, rows, d, eps); break;
    case 4: l2_kernel<T, BWD, 4><<<grid, L2_NT, 0, s>>>(xp, gp, op, rows, d, eps); break;
    case 8: l2_kernel<T, BWD, 8><<<grid, L2_NT, 0, s>>>(xp, gp, op, rows, d, eps); break;
    default: l2_kernel<T, BWD, 0><<<grid, L2_NT, 0, s>>>(xp, gp, op, rows, d, eps);
  }
  return check_launch(BWD ? "l2 normalize backward" : "l2 normalize");
}

int l2_check(long rows, int d, int dtype, float eps) {
  EDF_REQUIRE(rows > 0 && d > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(d <= L2_MAX_D, EDF_ERR_UNSUPPORTED, "rows of at most %d elements", L2_MAX_D);
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(eps >= 0.0f, EDF_ERR_INVALID_ARG, "eps must be non-negative");
  return EDF_OK;
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_l2_normalize(void* stream, const void* x, void* y, long rows, int d, float eps, int dtype) {
  using namespace edf;
  int rc = l2_check(rows, d, dtype, eps);
  if (rc) return rc;
  EDF_REQUIRE(x && y, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? l2_run<bf16, false>(s, x, nullptr, y, rows, d, eps)
                           : l2_run<float, false>(s, x, nullptr, y, rows, d, eps);
}

int edf_l2_normalize_backward(void* stream, const void* x, const void* grad_y, void* grad_x, long rows, int d,
                              float eps, int dtype) {
  using namespace edf;
  int rc = l2_check(rows, d, dtype, eps);
  if (rc) return rc;
  EDF_REQUIRE(x && grad_y && grad_x, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? l2_run<bf16, true>(s, x, grad_y, grad_x, rows, d, eps)
                           : l2_run<float, true>(s, x, grad_y, grad_x, rows, d, eps);
}

}  // extern "C"
