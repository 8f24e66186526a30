// Mean next-token cross entropy over logits, forward and backward: the loss the block
// models train with (the LM head's softmax cross entropy of the config-5 hybrid decoder).
// The logits stay in their storage dtype; every reduction runs in f32.
//   lse[n] = log sum_v exp(x[n, v]);  loss[n] = lse[n] - x[n, target[n]]
//   d x[n, v] = scale (exp(x[n, v] - lse[n]) - [v == target[n]]),  scale = *grad * inv_n
// A row whose target lies outside [0, V) contributes loss 0 and gradient 0.
// One workgroup per row: 16-byte loads over the row (8 bf16 or 4 f32 per thread and
// step), an online max / sum-of-exponentials per thread, one LDS reduction.  The forward
// stores lse for the backward, which reads the row once more and writes the gradient in
// the logits' dtype (no float32 copy of the logits, no float32 gradient).
#include <stdint.h>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int CE_NT = 256;

template <typename T> struct CEVec;
template <> struct CEVec<bf16> {
  static constexpr int N = 8;
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
template <> struct CEVec<float> {
  static constexpr int N = 4;
  static EDF_DEVICE void ld(const float* p, float* v) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  static EDF_DEVICE void st(float* p, const float* v) { *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]); }
};

// (max, sum exp(x - max)) of two partial sets
EDF_DEVICE void ce_merge(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  s = (m == -__builtin_huge_valf() ? 0.0f : s * __expf(m - mm)) + (m2 == -__builtin_huge_valf() ? 0.0f : s2 * __expf(m2 - mm));
  m = mm;
}

// VEC: 16-byte accesses (the row length is a multiple of the vector and the rows aligned)
template <typename T, bool VEC>
__global__ __launch_bounds__(CE_NT) void ce_fwd_kernel(const T* __restrict__ x, const int64_t* __restrict__ tgt,
                                                      float* __restrict__ loss, float* __restrict__ lse, int V) {
  constexpr int W = VEC ? CEVec<T>::N : 1;
  __shared__ float sm[CE_NT / 64], ss[CE_NT / 64];
  const long n = blockIdx.x;
  const T* row = x + n * V;
  float m = -__builtin_huge_valf(), s = 0.0f;
  for (int v0 = threadIdx.x * W; v0 < V; v0 += CE_NT * W) {
    float f[W];
    if constexpr (VEC) CEVec<T>::ld(row + v0, f);
    else f[0] = to_f32(row[v0]);
    float mb = f[0];
#pragma unroll
    for (int i = 1; i < W; ++i) mb = fmaxf(mb, f[i]);
    float sb = 0.0f;
#pragma unroll
    for (int i = 0; i < W; ++i) sb += __expf(f[i] - mb);
    ce_merge(m, s, mb, sb);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ce_merge(m, s, __shfl_xor(m, o), __shfl_xor(s, o));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm[w] = m;
    ss[w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
#pragma unroll
    for (int i = 1; i < CE_NT / 64; ++i) ce_merge(M, S, sm[i], ss[i]);
    const float l = M + __logf(S);
    const long t = tgt[n];
    lse[n] = l;
    loss[n] = (t >= 0 && t < V) ? l - to_f32(row[t]) : 0.0f;
  }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(CE_NT) void ce_bwd_kernel(const T* __restrict__ x, const int64_t* __restrict__ tgt,
                                                      const float* __restrict__ lse, const float* __restrict__ grad,
                                                      float inv_n, T* __restrict__ dx, int V) {
  constexpr int W = VEC ? CEVec<T>::N : 1;
  const long n = blockIdx.x;
  const T* row = x + n * V;
  T* drow = dx + n * V;
  const long t = tgt[n];
  const bool live = t >= 0 && t < V;
  const float scale = live ? grad[0] * inv_n : 0.0f;
  const float l = lse[n];
  for (int v0 = threadIdx.x * W; v0 < V; v0 += CE_NT * W) {
    float f[W];
    if constexpr (VEC) CEVec<T>::ld(row + v0, f);
    else f[0] = to_f32(row[v0]);
#pragma unroll
    for (int i = 0; i < W; ++i) f[i] = scale * (__expf(f[i] - l) - (v0 + i == t ? 1.0f : 0.0f));
    if constexpr (VEC) CEVec<T>::st(drow + v0, f);
    else drow[v0] = (T)f[0];
  }
}

bool ce_vec(const void* a, const void* b, int V, int dtype) {
  const int w = dtype == EDF_BF16 ? 8 : 4;
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; };
  return V % w == 0 && al(a) && al(b);
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_cross_entropy(void* stream, const void* logits, const int64_t* targets, float* loss_rows, float* lse, int rows,
                      int vocab, int dtype) {
  using namespace edf;
  EDF_REQUIRE(rows > 0 && vocab > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(logits && targets && loss_rows && lse, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  const bool vec = ce_vec(logits, nullptr, vocab, dtype);
  if (dtype == EDF_BF16) {
    if (vec) ce_fwd_kernel<bf16, true><<<rows, CE_NT, 0, s>>>((const bf16*)logits, targets, loss_rows, lse, vocab);
    else ce_fwd_kernel<bf16, false><<<rows, CE_NT, 0, s>>>((const bf16*)logits, targets, loss_rows, lse, vocab);
  } else {
    if (vec) ce_fwd_kernel<float, true><<<rows, CE_NT, 0, s>>>((const float*)logits, targets, loss_rows, lse, vocab);
    else ce_fwd_kernel<float, false><<<rows, CE_NT, 0, s>>>((const float*)logits, targets, loss_rows, lse, vocab);
  }
  return check_launch("cross entropy");
}

int edf_cross_entropy_backward(void* stream, const void* logits, const int64_t* targets, const float* lse,
                               const float* grad_loss, float inv_rows, void* grad_logits, int rows, int vocab,
                               int dtype) {
  using namespace edf;
  EDF_REQUIRE(rows > 0 && vocab > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(logits && targets && lse && grad_loss && grad_logits, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  const bool vec = ce_vec(logits, grad_logits, vocab, dtype);
  if (dtype == EDF_BF16) {
    if (vec)
      ce_bwd_kernel<bf16, true><<<rows, CE_NT, 0, s>>>((const bf16*)logits, targets, lse, grad_loss, inv_rows,
                                                       (bf16*)grad_logits, vocab);
    else
      ce_bwd_kernel<bf16, false><<<rows, CE_NT, 0, s>>>((const bf16*)logits, targets, lse, grad_loss, inv_rows,
                                                        (bf16*)grad_logits, vocab);
  } else {
    if (vec)
      ce_bwd_kernel<float, true><<<rows, CE_NT, 0, s>>>((const float*)logits, targets, lse, grad_loss, inv_rows,
                                                        (float*)grad_logits, vocab);
    else
      ce_bwd_kernel<float, false><<<rows, CE_NT, 0, s>>>((const float*)logits, targets, lse, grad_loss, inv_rows,
                                                         (float*)grad_logits, vocab);
  }
  return check_launch("cross entropy backward");
}

}  // extern "C"
