// Softplus, forward and backward: the Mamba block's dt activation (Axon.activation(:softplus),
// lib/edifice/ssm/common.ex:366), block glue in front of the selective scan.
//   y = max(x, 0) + log1p(exp(-|x|))   (= log(1 + e^x) without overflow for large x)
//   dx = dy sigmoid(x)
// Elementwise over n values in the io dtype, f32 inside: 16-byte accesses (8 bf16 or 4 f32
// per thread and step) when the pointers allow, grid-stride, scalar tail.
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int SP_NT = 256;
constexpr int SP_MAX_WG = 4096;

template <typename T> struct SpVec;
template <> struct SpVec<bf16> {
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
template <> struct SpVec<float> {
  static constexpr int W = 4;
  static EDF_DEVICE void ld(const float* p, float* v) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  static EDF_DEVICE void st(float* p, const float* v) { *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]); }
};

// softplus_f (edf_common.hpp): log1p(e^-|x|) from the hardware exp2 / log2; an IEEE log1pf
// made the pass compute-bound (101 us per 16.8 M values).
EDF_DEVICE float sigmoid_f(float x) { return sigmoid_rcp(x); }

// BWD: out = dy sigmoid(x), else out = softplus(x); VEC: 16-byte accesses over n / W vectors
template <typename T, bool BWD, bool VEC>
__global__ __launch_bounds__(SP_NT) void sp_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                  T* __restrict__ out, long n) {
  const long stride = (long)gridDim.x * SP_NT;
  const long t0 = (long)blockIdx.x * SP_NT + threadIdx.x;
  if constexpr (VEC) {
    constexpr int W = SpVec<T>::W;
    const long nv = n / W;
    for (long v = t0; v < nv; v += stride) {
      float a[W], o[W];
      SpVec<T>::ld(x + v * W, a);
      if constexpr (BWD) {
        float g[W];
        SpVec<T>::ld(dy + v * W, g);
#pragma unroll
        for (int i = 0; i < W; ++i) o[i] = g[i] * sigmoid_f(a[i]);
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) o[i] = softplus_f(a[i]);
      }
      SpVec<T>::st(out + v * W, o);
    }
    for (long i = nv * W + t0; i < n; i += stride)  // tail
      out[i] = from_f32<T>(BWD ? to_f32(dy[i]) * sigmoid_f(to_f32(x[i])) : softplus_f(to_f32(x[i])));
  } else {
    for (long i = t0; i < n; i += stride)
      out[i] = from_f32<T>(BWD ? to_f32(dy[i]) * sigmoid_f(to_f32(x[i])) : softplus_f(to_f32(x[i])));
  }
}

template <typename T, bool BWD>
int sp_run(hipStream_t s, const void* x, const void* dy, void* out, long n) {
  constexpr int W = SpVec<T>::W;
  const bool vec = !(((uintptr_t)x | (uintptr_t)out | (BWD ? (uintptr_t)dy : 0)) & 15);
  const long units = vec ? std::max(n / W, 1L) : n;
  const unsigned grid = (unsigned)std::min((units + SP_NT - 1) / SP_NT, (long)SP_MAX_WG);
  if (vec)
    sp_kernel<T, BWD, true><<<grid, SP_NT, 0, s>>>((const T*)x, (const T*)dy, (T*)out, n);
  else
    sp_kernel<T, BWD, false><<<grid, SP_NT, 0, s>>>((const T*)x, (const T*)dy, (T*)out, n);
  return check_launch(BWD ? "softplus backward" : "softplus");
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_softplus(void* stream, const void* x, void* y, long n, int dtype) {
  using namespace edf;
  EDF_REQUIRE(n > 0, EDF_ERR_INVALID_ARG, "n must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(x && y, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? sp_run<bf16, false>(s, x, nullptr, y, n) : sp_run<float, false>(s, x, nullptr, y, n);
}

int edf_softplus_backward(void* stream, const void* x, const void* grad_y, void* grad_x, long n, int dtype) {
  using namespace edf;
  EDF_REQUIRE(n > 0, EDF_ERR_INVALID_ARG, "n must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(x && grad_y && grad_x, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? sp_run<bf16, true>(s, x, grad_y, grad_x, n)
                           : sp_run<float, true>(s, x, grad_y, grad_x, n);
}

}  // extern "C"
