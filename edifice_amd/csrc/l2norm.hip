// L2 normalisation of rows, forward and backward: the DeltaNet / GatedDeltaNet key norm
// k / sqrt(sum k^2 + eps) (lib/edifice/recurrent/delta_net.ex:291,
// gated_delta_net.ex:387, eps inside the square root), block glue in front of the delta rule.
//   y = x r,  r = 1 / sqrt(sum_j x_j^2 + eps);   dx = r (dy - y <y, dy>)
// x, y, dy, dx [rows, d] in the io dtype, f32 inside.  A 16-lane DPP row holds one row of x
// (16-byte accesses: 8 bf16 or 4 f32 per lane and step, d up to 16 vectors per lane's share),
// its sums by a row butterfly; rows whose length is not a multiple of the vector, or
// misaligned tensors, take one element per lane and step.  The backward recomputes r from x.
//
// DeltaNet input split (delta_net.ex:274-300): the layer's projection [rows, 4 H d] holds
// q | k | v | beta_pre per row; one pass writes q, the per-head L2-normalised k, v and
// sigmoid(beta_pre) as [rows, H, d] tensors (the scan's layout), and the backward writes the
// projection's gradient [rows, 4 H d] from dq, dk, dv, dbeta in one pass (k's norm and the
// sigmoid recomputed from the projection), in place of head-layout copies, a separate norm,
// a sigmoid and a concatenation.  One 16-lane row per (row, head).
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

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

// 16 bytes copied unchanged
EDF_DEVICE void cp16(const void* src, void* dst) {
  *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
}

// units = rows H (row, head) pairs, HD = H d; NV as l2_kernel (d <= 16 NV W), NV = 0: one
// element per lane and step.  Forward: out[0..3] = q, k / |k|, v, sigmoid(beta_pre) [units, d].
template <typename T, int NV>
__global__ __launch_bounds__(L2_NT) void dnp_fwd_kernel(const T* __restrict__ proj, T* __restrict__ oq,
                                                       T* __restrict__ ok, T* __restrict__ ov, T* __restrict__ ob,
                                                       long units, int H, int d, float eps) {
  constexpr int W = L2Vec<T>::W;
  const int i16 = threadIdx.x & 15;
  const long u = (long)blockIdx.x * (L2_NT / 16) + (threadIdx.x >> 4);
  const bool live = u < units;  // dead rows compute on the last unit and store nothing
  const long uu = live ? u : units - 1;
  const long HD = (long)H * d;
  const T* pr = proj + (uu / H) * 4 * HD + (uu % H) * d;  // this unit's q; k, v, beta_pre at +HD, +2HD, +3HD
  const long ou = uu * d;
  if constexpr (NV > 0) {
    float kv[NV][W];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 16 + i16) * W;
      if (c0 < d) {
        L2Vec<T>::ld(pr + HD + c0, kv[k]);
        if (live) {
          cp16(pr + c0, oq + ou + c0);
          cp16(pr + 2 * HD + c0, ov + ou + c0);
          float bv[W];
          L2Vec<T>::ld(pr + 3 * HD + c0, bv);
#pragma unroll
          for (int i = 0; i < W; ++i) bv[i] = sigmoid_rcp(bv[i]);
          L2Vec<T>::st(ob + ou + c0, bv);
        }
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) kv[k][i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) ss = fmaf(kv[k][i], kv[k][i], ss);
    }
    const float rn = 1.0f / sqrtf(row16_sum(ss) + eps);
    if (!live) return;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 16 + i16) * W;
      if (c0 >= d) continue;
      float o[W];
#pragma unroll
      for (int i = 0; i < W; ++i) o[i] = kv[k][i] * rn;
      L2Vec<T>::st(ok + ou + c0, o);
    }
  } else {
    float ss = 0.0f;
    for (int c = i16; c < d; c += 16) {
      const float a = to_f32(pr[HD + c]);
      ss = fmaf(a, a, ss);
    }
    const float rn = 1.0f / sqrtf(row16_sum(ss) + eps);
    if (!live) return;
    for (int c = i16; c < d; c += 16) {
      oq[ou + c] = pr[c];
      ok[ou + c] = from_f32<T>(to_f32(pr[HD + c]) * rn);
      ov[ou + c] = pr[2 * HD + c];
      ob[ou + c] = from_f32<T>(sigmoid_rcp(to_f32(pr[3 * HD + c])));
    }
  }
}

// Backward: dproj [rows, 4 HD] from dq, dk, dv, dbeta [units, d]; dk through the norm
// (dk_pre = r (dk - y <y, dk>), y = k r), dbeta through the sigmoid (dbeta s (1 - s)).
template <typename T, int NV>
__global__ __launch_bounds__(L2_NT) void dnp_bwd_kernel(const T* __restrict__ proj, const T* __restrict__ gq,
                                                       const T* __restrict__ gk, const T* __restrict__ gv,
                                                       const T* __restrict__ gb, T* __restrict__ dproj, long units,
                                                       int H, int d, float eps) {
  constexpr int W = L2Vec<T>::W;
  const int i16 = threadIdx.x & 15;
  const long u = (long)blockIdx.x * (L2_NT / 16) + (threadIdx.x >> 4);
  const bool live = u < units;
  const long uu = live ? u : units - 1;
  const long HD = (long)H * d;
  const long po = (uu / H) * 4 * HD + (uu % H) * d;
  const T* pr = proj + po;
  T* dr = dproj + po;
  const long ou = uu * d;
  if constexpr (NV > 0) {
    float kv[NV][W], g[NV][W];
    float ss = 0.0f, dot = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 16 + i16) * W;
      if (c0 < d) {
        L2Vec<T>::ld(pr + HD + c0, kv[k]);
        L2Vec<T>::ld(gk + ou + c0, g[k]);
        if (live) {
          cp16(gq + ou + c0, dr + c0);
          cp16(gv + ou + c0, dr + 2 * HD + c0);
          float bv[W], bg[W];
          L2Vec<T>::ld(pr + 3 * HD + c0, bv);
          L2Vec<T>::ld(gb + ou + c0, bg);
#pragma unroll
          for (int i = 0; i < W; ++i) {
            const float sg = sigmoid_rcp(bv[i]);
            bv[i] = bg[i] * sg * (1.0f - sg);
          }
          L2Vec<T>::st(dr + 3 * HD + c0, bv);
        }
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) kv[k][i] = g[k][i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) {
        ss = fmaf(kv[k][i], kv[k][i], ss);
        dot = fmaf(kv[k][i], g[k][i], dot);
      }
    }
    const float rn = 1.0f / sqrtf(row16_sum(ss) + eps);
    dot = row16_sum(dot) * rn;  // <y, dk>
    if (!live) return;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 16 + i16) * W;
      if (c0 >= d) continue;
      float o[W];
#pragma unroll
      for (int i = 0; i < W; ++i) o[i] = rn * fmaf(-kv[k][i] * rn, dot, g[k][i]);
      L2Vec<T>::st(dr + HD + c0, o);
    }
  } else {
    float ss = 0.0f, dot = 0.0f;
    for (int c = i16; c < d; c += 16) {
      const float a = to_f32(pr[HD + c]);
      ss = fmaf(a, a, ss);
      dot = fmaf(a, to_f32(gk[ou + c]), dot);
    }
    const float rn = 1.0f / sqrtf(row16_sum(ss) + eps);
    dot = row16_sum(dot) * rn;
    if (!live) return;
    for (int c = i16; c < d; c += 16) {
      dr[c] = gq[ou + c];
      dr[HD + c] = from_f32<T>(rn * fmaf(-to_f32(pr[HD + c]) * rn, dot, to_f32(gk[ou + c])));
      dr[2 * HD + c] = gv[ou + c];
      const float sg = sigmoid_rcp(to_f32(pr[3 * HD + c]));
      dr[3 * HD + c] = from_f32<T>(to_f32(gb[ou + c]) * sg * (1.0f - sg));
    }
  }
}

// vectors per lane for a d-element row (0: one element per lane and step)
template <typename T>
int l2_nv(uintptr_t ptrs, int d) {
  constexpr int W = L2Vec<T>::W;
  if ((ptrs & 15) || d % W) return 0;
  for (int c : {1, 2, 4, 8})
    if (d / W <= 16 * c) return c;
  return 0;
}

template <typename T>
int dnp_run(hipStream_t s, bool bwd, const void* proj, const void* a0, const void* a1, const void* a2,
            const void* a3, void* o0, void* o1, void* o2, void* o3, long rows, int H, int d, float eps) {
  const long units = rows * H;
  const unsigned grid = (unsigned)((units + L2_NT / 16 - 1) / (L2_NT / 16));
  const uintptr_t ptrs = (uintptr_t)proj | (uintptr_t)a0 | (uintptr_t)a1 | (uintptr_t)a2 | (uintptr_t)a3 |
                         (uintptr_t)o0 | (uintptr_t)o1 | (uintptr_t)o2 | (uintptr_t)o3;
  const T* p = (const T*)proj;
  auto launch = [&](auto nvc) {
    constexpr int NV = decltype(nvc)::value;
    if (bwd)
      dnp_bwd_kernel<T, NV><<<grid, L2_NT, 0, s>>>(p, (const T*)a0, (const T*)a1, (const T*)a2, (const T*)a3,
                                                   (T*)o0, units, H, d, eps);
    else
      dnp_fwd_kernel<T, NV><<<grid, L2_NT, 0, s>>>(p, (T*)o0, (T*)o1, (T*)o2, (T*)o3, units, H, d, eps);
  };
  switch (l2_nv<T>(ptrs, d)) {
    case 1: launch(std::integral_constant<int, 1>{}); break;
    case 2: launch(std::integral_constant<int, 2>{}); break;
    case 4: launch(std::integral_constant<int, 4>{}); break;
    case 8: launch(std::integral_constant<int, 8>{}); break;
    default: launch(std::integral_constant<int, 0>{});
  }
  return check_launch(bwd ? "delta net split backward" : "delta net split");
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

int edf_delta_net_split(void* stream, const void* proj, void* q, void* k, void* v, void* beta, long rows,
                        int num_heads, int head_dim, float eps, int dtype) {
  using namespace edf;
  EDF_REQUIRE(num_heads > 0, EDF_ERR_INVALID_ARG, "num_heads must be positive");
  int rc = l2_check(rows, head_dim, dtype, eps);
  if (rc) return rc;
  EDF_REQUIRE(proj && q && k && v && beta, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16
             ? dnp_run<bf16>(s, false, proj, nullptr, nullptr, nullptr, nullptr, q, k, v, beta, rows, num_heads,
                             head_dim, eps)
             : dnp_run<float>(s, false, proj, nullptr, nullptr, nullptr, nullptr, q, k, v, beta, rows, num_heads,
                              head_dim, eps);
}

int edf_delta_net_split_backward(void* stream, const void* proj, const void* grad_q, const void* grad_k,
                                 const void* grad_v, const void* grad_beta, void* grad_proj, long rows,
                                 int num_heads, int head_dim, float eps, int dtype) {
  using namespace edf;
  EDF_REQUIRE(num_heads > 0, EDF_ERR_INVALID_ARG, "num_heads must be positive");
  int rc = l2_check(rows, head_dim, dtype, eps);
  if (rc) return rc;
  EDF_REQUIRE(proj && grad_q && grad_k && grad_v && grad_beta && grad_proj, EDF_ERR_INVALID_ARG,
              "null tensor pointer");
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? dnp_run<bf16>(s, true, proj, grad_q, grad_k, grad_v, grad_beta, grad_proj, nullptr,
                                           nullptr, nullptr, rows, num_heads, head_dim, eps)
                           : dnp_run<float>(s, true, proj, grad_q, grad_k, grad_v, grad_beta, grad_proj, nullptr,
                                            nullptr, nullptr, rows, num_heads, head_dim, eps);
}

}  // extern "C"
