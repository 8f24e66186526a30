// Layer normalisation over the last dimension, forward and backward: the pre-norms and final
// norms of the block models (Axon.layer_norm: lib/edifice/ssm/common.ex:224,
// lib/edifice/recurrent/delta_net.ex:159,199, lib/edifice/blocks/model_builder.ex:111,165,
// transformer_block.ex:251; biased variance, epsilon inside the square root).  In the
// reference these are Axon layers; here they are the block callers' glue around the fused
// scans, one pass over the activations each way.
//
//   y[r, c] = (x[r, c] - mu_r) rstd_r gamma[c] + beta[c],   rstd_r = 1 / sqrt(var_r + eps)
// backward, with xh = (x - mu) rstd and g = dy gamma:
//   dx = rstd (g - mean_c(g) - xh mean_c(g xh)),  dgamma = sum_r dy xh,  dbeta = sum_r dy
//
// x, y, dy, dx [rows, cols] in the io dtype, gamma / beta (and their gradients) [cols] in the
// parameter dtype, mean / rstd [rows] float32 (the forward keeps them for the backward); all
// arithmetic in f32.  One wave per row at a time: when cols is a multiple of the 16-byte
// vector and at most 2048, each lane holds its NV vectors of the row in registers (the mean,
// then the variance about it, from registers) and each wave takes a stride of rows with
// gamma / beta of its columns in registers; otherwise the row is read from memory once per
// pass.  The backward's waves keep per-column dgamma / dbeta sums in registers, summed over
// the four waves of a workgroup in LDS into one partial per workgroup and over the
// workgroups, in order, by two small kernels (deterministic, no atomics).
//
// Residual form (a pre-norm block stack's h' = h + f(norm h) followed by the next norm): the
// forward takes the sum s = x + res rounded to the io dtype (what a separate add stores),
// writes it and normalises it; the backward adds the gradient arriving at s from the residual
// path to dx before its store (dx = LN'(dy) + grad_add, rounded once), so neither add is a pass
// of its own.
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int LN_NT = 256;       // four waves per workgroup, one row per wave
constexpr int LN_BWD_WG = 512;   // backward workgroups (rows strided over their waves)
constexpr int LN_FWD_WG = 1024;  // forward workgroups of the register path
constexpr int LN_MAX_COLS = 8192;

template <typename T> struct LnVec;
template <> struct LnVec<bf16> {
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
template <> struct LnVec<float> {
  static constexpr int W = 4;
  static EDF_DEVICE void ld(const float* p, float* v) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  static EDF_DEVICE void st(float* p, const float* v) { *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]); }
};

EDF_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// gamma / beta element c (1 / 0 when the parameter is absent)
template <typename TP> EDF_DEVICE float pget(const TP* p, int c, float dflt) { return p ? to_f32(p[c]) : dflt; }

// W consecutive parameters from c0 (a 16-byte aligned parameter array, c0 a multiple of W) as
// f32, or dflt for an absent parameter: one or two vector loads instead of W scalar ones
template <typename TP, int W> EDF_DEVICE void pvec(const TP* p, int c0, float* o, float dflt) {
  if (!p) {
#pragma unroll
    for (int i = 0; i < W; ++i) o[i] = dflt;
    return;
  }
  if constexpr (sizeof(TP) == 2) {
    if constexpr (W == 8) {
      LnVec<bf16>::ld(reinterpret_cast<const bf16*>(p) + c0, o);
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(p + c0);
      o[0] = __builtin_bit_cast(float, u.x << 16), o[1] = __builtin_bit_cast(float, u.x & 0xffff0000u);
      o[2] = __builtin_bit_cast(float, u.y << 16), o[3] = __builtin_bit_cast(float, u.y & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < W; j += 4) LnVec<float>::ld(reinterpret_cast<const float*>(p) + c0 + j, o + j);
  }
}

// a + b rounded to T (the value a separate add in T stores), as f32
template <typename T> EDF_DEVICE float add_rnd(float a, float b) { return to_f32(from_f32<T>(a + b)); }

// ---- forward, row in registers: NV vectors of W elements per lane --------------------------
// Each wave takes a stride of rows with gamma / beta of its columns in registers.
// RES: the row is x + res (rounded to T), also stored to sum
template <typename T, typename TP, int NV, bool RES>
__global__ __launch_bounds__(LN_NT) void ln_fwd_kernel(const T* __restrict__ x, const T* __restrict__ res,
                                                      T* __restrict__ sum, const TP* __restrict__ gamma,
                                                      const TP* __restrict__ beta, T* __restrict__ y,
                                                      float* __restrict__ mean, float* __restrict__ rstd, int rows,
                                                      int cols, float eps) {
  constexpr int W = LnVec<T>::W;
  constexpr int NW = LN_NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float gm[NV][W], bt[NV][W];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c0 = (k * 64 + lane) * W;
    if (c0 < cols) {
      pvec<TP, W>(gamma, c0, gm[k], 1.0f);
      pvec<TP, W>(beta, c0, bt[k], 0.0f);
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) gm[k][i] = bt[k][i] = 0.0f;
    }
  }
  const float inv_c = 1.0f / (float)cols;
  for (long r = (long)blockIdx.x * NW + w; r < rows; r += (long)gridDim.x * NW) {
    const T* xr = x + r * cols;
    float v[NV][W];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 64 + lane) * W;
      if (c0 < cols) {
        LnVec<T>::ld(xr + c0, v[k]);
        if constexpr (RES) {
          float rv[W];
          LnVec<T>::ld(res + r * cols + c0, rv);
#pragma unroll
          for (int i = 0; i < W; ++i) v[k][i] = add_rnd<T>(v[k][i], rv[i]);
          LnVec<T>::st(sum + r * cols + c0, v[k]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) v[k][i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) s += v[k][i];
    }
    const float mu = wave_sum(s) * inv_c;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if ((k * 64 + lane) * W >= cols) continue;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        const float d = v[k][i] - mu;
        q = fmaf(d, d, q);
      }
    }
    const float rs = 1.0f / sqrtf(wave_sum(q) * inv_c + eps);
    T* yr = y + r * cols;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 64 + lane) * W;
      if (c0 >= cols) continue;
      float o[W];
#pragma unroll
      for (int i = 0; i < W; ++i) o[i] = fmaf((v[k][i] - mu) * rs, gm[k][i], bt[k][i]);
      LnVec<T>::st(yr + c0, o);
    }
    if (lane == 0) {
      mean[r] = mu;
      rstd[r] = rs;
    }
  }
}

// ---- forward, any shape: one pass over memory per statistic --------------------------------
// RES: the sum x + res is formed and stored by the first pass, which the later passes read
template <typename T, typename TP, bool RES>
__global__ __launch_bounds__(LN_NT) void ln_fwd_any_kernel(const T* __restrict__ x, const T* __restrict__ res,
                                                          T* __restrict__ sum, const TP* __restrict__ gamma,
                                                          const TP* __restrict__ beta, T* __restrict__ y,
                                                          float* __restrict__ mean, float* __restrict__ rstd, int rows,
                                                          int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const long r = (long)blockIdx.x * (LN_NT / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const T* xr = x + r * cols;
  float s = 0.0f;
  if constexpr (RES) {
    T* sr = sum + r * cols;
    for (int c = lane; c < cols; c += 64) {
      const T v = from_f32<T>(to_f32(xr[c]) + to_f32(res[r * cols + c]));
      sr[c] = v;
      s += to_f32(v);
    }
    xr = sr;  // each lane re-reads only the elements it wrote
  } else {
    for (int c = lane; c < cols; c += 64) s += to_f32(xr[c]);
  }
  const float mu = wave_sum(s) / (float)cols;
  float q = 0.0f;
  for (int c = lane; c < cols; c += 64) {
    const float d = to_f32(xr[c]) - mu;
    q = fmaf(d, d, q);
  }
  const float rs = 1.0f / sqrtf(wave_sum(q) / (float)cols + eps);
  T* yr = y + r * cols;
  for (int c = lane; c < cols; c += 64)
    yr[c] = from_f32<T>(fmaf((to_f32(xr[c]) - mu) * rs, pget(gamma, c, 1.0f), pget(beta, c, 0.0f)));
  if (lane == 0) {
    mean[r] = mu;
    rstd[r] = rs;
  }
}

// ---- backward, row in registers -----------------------------------------------------------
// part [LN_BWD_WG][2][cols]: this workgroup's dgamma (0) and dbeta (1) column sums
// GADD: dx = LN'(dy) + ga
template <typename T, typename TP, int NV, bool GADD>
__global__ __launch_bounds__(LN_NT) void ln_bwd_kernel(const T* __restrict__ x, const TP* __restrict__ gamma,
                                                      const float* __restrict__ mean, const float* __restrict__ rstd,
                                                      const T* __restrict__ dy, const T* __restrict__ ga,
                                                      T* __restrict__ dx, float* __restrict__ part, int rows,
                                                      int cols) {
  constexpr int W = LnVec<T>::W;
  constexpr int NW = LN_NT / 64;
  __shared__ float s_acc[NW][2][NV * 64 * W];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float gm[NV][W], ag[NV][W], ab[NV][W];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c0 = (k * 64 + lane) * W;
    if (c0 < cols) {
      pvec<TP, W>(gamma, c0, gm[k], 1.0f);
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) gm[k][i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < W; ++i) ag[k][i] = ab[k][i] = 0.0f;
  }
  const float inv_c = 1.0f / (float)cols;
  for (long r = (long)blockIdx.x * NW + w; r < rows; r += (long)gridDim.x * NW) {
    const T* xr = x + r * cols;
    const T* gr = dy + r * cols;
    const float mu = mean[r], rs = rstd[r];
    float xh[NV][W], g[NV][W];
    float s1 = 0.0f, s2 = 0.0f;  // sum g, sum g xh
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 64 + lane) * W;
      float xv[W], dv[W];
      if (c0 < cols) {
        LnVec<T>::ld(xr + c0, xv);
        LnVec<T>::ld(gr + c0, dv);
      } else {
#pragma unroll
        for (int i = 0; i < W; ++i) xv[i] = dv[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) {
        xh[k][i] = c0 < cols ? (xv[i] - mu) * rs : 0.0f;
        g[k][i] = dv[i] * gm[k][i];
        ag[k][i] = fmaf(dv[i], xh[k][i], ag[k][i]);
        ab[k][i] += dv[i];
        s1 += g[k][i];
        s2 = fmaf(g[k][i], xh[k][i], s2);
      }
    }
    const float m1 = wave_sum(s1) * inv_c, m2 = wave_sum(s2) * inv_c;
    T* dr = dx + r * cols;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int c0 = (k * 64 + lane) * W;
      if (c0 >= cols) continue;
      float o[W];
#pragma unroll
      for (int i = 0; i < W; ++i) o[i] = rs * (g[k][i] - fmaf(xh[k][i], m2, m1));
      if constexpr (GADD) {
        float av[W];
        LnVec<T>::ld(ga + r * cols + c0, av);
#pragma unroll
        for (int i = 0; i < W; ++i) o[i] += av[i];
      }
      LnVec<T>::st(dr + c0, o);
    }
  }
  // this workgroup's column sums, the four waves added in wave order
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int i = 0; i < W; ++i) {
      s_acc[w][0][(k * 64 + lane) * W + i] = ag[k][i];
      s_acc[w][1][(k * 64 + lane) * W + i] = ab[k][i];
    }
  __syncthreads();
  float* pw = part + (long)blockIdx.x * 2 * cols;
  for (int e = threadIdx.x; e < 2 * cols; e += LN_NT) {
    const int q = e / cols, c = e % cols;
    float a = s_acc[0][q][c];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) a += s_acc[ww][q][c];
    pw[e] = a;
  }
}

// ---- backward, any shape ------------------------------------------------------------------
template <typename T, typename TP, bool GADD>
__global__ __launch_bounds__(LN_NT) void ln_bwd_any_kernel(const T* __restrict__ x, const TP* __restrict__ gamma,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ rstd, const T* __restrict__ dy,
                                                          const T* __restrict__ ga, T* __restrict__ dx,
                                                          float* __restrict__ part, int rows, int cols) {
  constexpr int NW = LN_NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const float inv_c = 1.0f / (float)cols;
  for (long r = (long)blockIdx.x * NW + w; r < rows; r += (long)gridDim.x * NW) {
    const T* xr = x + r * cols;
    const T* gr = dy + r * cols;
    const float mu = mean[r], rs = rstd[r];
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = lane; c < cols; c += 64) {
      const float g = to_f32(gr[c]) * pget(gamma, c, 1.0f);
      s1 += g;
      s2 = fmaf(g, (to_f32(xr[c]) - mu) * rs, s2);
    }
    const float m1 = wave_sum(s1) * inv_c, m2 = wave_sum(s2) * inv_c;
    T* dr = dx + r * cols;
    for (int c = lane; c < cols; c += 64) {
      const float g = to_f32(gr[c]) * pget(gamma, c, 1.0f);
      const float o = rs * (g - fmaf((to_f32(xr[c]) - mu) * rs, m2, m1));
      dr[c] = from_f32<T>(GADD ? o + to_f32(ga[r * cols + c]) : o);
    }
  }
  // column sums of this workgroup's rows (in row order per column)
  float* pw = part + (long)blockIdx.x * 2 * cols;
  for (int c = threadIdx.x; c < cols; c += LN_NT) {
    float a = 0.0f, b = 0.0f;
    for (long r = (long)blockIdx.x * NW; r < rows; r += (long)gridDim.x * NW)
      for (int ww = 0; ww < NW && r + ww < rows; ++ww) {
        const float d = to_f32(dy[(r + ww) * cols + c]);
        a = fmaf(d, (to_f32(x[(r + ww) * cols + c]) - mean[r + ww]) * rstd[r + ww], a);
        b += d;
      }
    pw[c] = a;
    pw[cols + c] = b;
  }
}

// dgamma / dbeta from the workgroup partials, in workgroup order, in two stages: slice ps
// (LN_RS consecutive partials) per thread and column, then the slices per column.
constexpr int LN_RS = 16;
inline int ln_slices(int nwg) { return (nwg + LN_RS - 1) / LN_RS; }

__global__ __launch_bounds__(256) void ln_reduce1_kernel(const float* __restrict__ part, float* __restrict__ part2,
                                                        int nwg, int cols) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= 2 * cols) return;
  const int k0 = blockIdx.y * LN_RS, k1 = min(nwg, k0 + LN_RS);
  float a = 0.0f;
#pragma unroll 8
  for (int k = k0; k < k1; ++k) a += part[(long)k * 2 * cols + e];
  part2[(long)blockIdx.y * 2 * cols + e] = a;
}

template <typename TP>
__global__ __launch_bounds__(256) void ln_reduce2_kernel(const float* __restrict__ part2, TP* __restrict__ dgamma,
                                                        TP* __restrict__ dbeta, int nslice, int cols) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= 2 * cols) return;
  float a = 0.0f;
#pragma unroll 8
  for (int k = 0; k < nslice; ++k) a += part2[(long)k * 2 * cols + e];
  TP* dst = e < cols ? dgamma : dbeta;
  if (dst) dst[e < cols ? e : e - cols] = from_f32<TP>(a);
}

// vectors per lane for a row held in registers (at most 32 values per lane and array; 0:
// the any-shape kernels); ptrs: every pointer the vector kernels read or write, OR-ed
template <typename T>
int ln_nv(uintptr_t ptrs, int cols) {
  constexpr int W = LnVec<T>::W;
  if (cols % W != 0 || (ptrs & 15)) return 0;
  const int nvec = cols / W;
  for (int nv : {1, 2, 4, 8})
    if (nv * W <= 32 && nvec <= 64 * nv) return nv;
  return 0;
}

inline int ln_bwd_groups(int rows) { return std::min((rows + LN_NT / 64 - 1) / (LN_NT / 64), LN_BWD_WG); }

template <typename T, typename TP, bool RES>
int ln_fwd(hipStream_t s, const void* x, const void* res, void* sum, const void* gamma, const void* beta, void* y,
           float* mean, float* rstd, int rows, int cols, float eps) {
  const unsigned grid = (unsigned)((rows + LN_NT / 64 - 1) / (LN_NT / 64));
  const unsigned gridr = std::min(grid, (unsigned)LN_FWD_WG);
  const T* xp = (const T*)x;
  const T* rp = (const T*)res;
  T* sp = (T*)sum;
  const TP* gp = (const TP*)gamma;
  const TP* bp = (const TP*)beta;
  T* yp = (T*)y;
  const int nv = ln_nv<T>((uintptr_t)x | (uintptr_t)y | (uintptr_t)res | (uintptr_t)sum | (uintptr_t)gamma |
                             (uintptr_t)beta, cols);
  switch (nv) {
    case 1: ln_fwd_kernel<T, TP, 1, RES><<<gridr, LN_NT, 0, s>>>(xp, rp, sp, gp, bp, yp, mean, rstd, rows, cols, eps); break;
    case 2: ln_fwd_kernel<T, TP, 2, RES><<<gridr, LN_NT, 0, s>>>(xp, rp, sp, gp, bp, yp, mean, rstd, rows, cols, eps); break;
    case 4: ln_fwd_kernel<T, TP, 4, RES><<<gridr, LN_NT, 0, s>>>(xp, rp, sp, gp, bp, yp, mean, rstd, rows, cols, eps); break;
    case 8:
      if constexpr (8 * LnVec<T>::W <= 32)
        ln_fwd_kernel<T, TP, 8, RES><<<gridr, LN_NT, 0, s>>>(xp, rp, sp, gp, bp, yp, mean, rstd, rows, cols, eps);
      break;
    default: ln_fwd_any_kernel<T, TP, RES><<<grid, LN_NT, 0, s>>>(xp, rp, sp, gp, bp, yp, mean, rstd, rows, cols, eps);
  }
  return check_launch(RES ? "add + layer norm" : "layer norm");
}

template <typename T, typename TP, bool GADD>
int ln_bwd(hipStream_t s, const void* x, const void* gamma, const float* mean, const float* rstd, const void* dy,
           const void* ga, void* dx, void* dgamma, void* dbeta, float* part, int rows, int cols) {
  const int nwg = ln_bwd_groups(rows);
  const T* xp = (const T*)x;
  const TP* gp = (const TP*)gamma;
  const T* dyp = (const T*)dy;
  const T* gap = (const T*)ga;
  T* dxp = (T*)dx;
  const int nv = ln_nv<T>((uintptr_t)x | (uintptr_t)dx | (uintptr_t)dy | (uintptr_t)ga | (uintptr_t)gamma, cols);
  switch (nv) {
    case 1: ln_bwd_kernel<T, TP, 1, GADD><<<nwg, LN_NT, 0, s>>>(xp, gp, mean, rstd, dyp, gap, dxp, part, rows, cols); break;
    case 2: ln_bwd_kernel<T, TP, 2, GADD><<<nwg, LN_NT, 0, s>>>(xp, gp, mean, rstd, dyp, gap, dxp, part, rows, cols); break;
    case 4: ln_bwd_kernel<T, TP, 4, GADD><<<nwg, LN_NT, 0, s>>>(xp, gp, mean, rstd, dyp, gap, dxp, part, rows, cols); break;
    case 8:
      if constexpr (8 * LnVec<T>::W <= 32)
        ln_bwd_kernel<T, TP, 8, GADD><<<nwg, LN_NT, 0, s>>>(xp, gp, mean, rstd, dyp, gap, dxp, part, rows, cols);
      break;
    default: ln_bwd_any_kernel<T, TP, GADD><<<nwg, LN_NT, 0, s>>>(xp, gp, mean, rstd, dyp, gap, dxp, part, rows, cols);
  }
  int rc = check_launch("layer norm backward");
  if (rc || (!dgamma && !dbeta)) return rc;
  const int nsl = ln_slices(nwg);
  float* part2 = part + (long)nwg * 2 * cols;
  ln_reduce1_kernel<<<dim3((2 * cols + 255) / 256, nsl), 256, 0, s>>>(part, part2, nwg, cols);
  ln_reduce2_kernel<TP><<<(2 * cols + 255) / 256, 256, 0, s>>>(part2, (TP*)dgamma, (TP*)dbeta, nsl, cols);
  return check_launch("layer norm parameter gradients");
}

template <typename F>
int ln_dtypes(int io, int par, F&& f) {
  if (io == EDF_BF16 && par == EDF_BF16) return f((bf16*)nullptr, (bf16*)nullptr);
  if (io == EDF_BF16 && par == EDF_F32) return f((bf16*)nullptr, (float*)nullptr);
  if (io == EDF_F32 && par == EDF_BF16) return f((float*)nullptr, (bf16*)nullptr);
  return f((float*)nullptr, (float*)nullptr);
}

int ln_check(int rows, int cols, int io, int par) {
  EDF_REQUIRE(rows > 0 && cols > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(cols <= LN_MAX_COLS, EDF_ERR_UNSUPPORTED, "at most %d columns", LN_MAX_COLS);
  EDF_REQUIRE(valid_dtype(io) && valid_dtype(par), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  return EDF_OK;
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_layer_norm(void* stream, const void* x, const void* gamma, const void* beta, void* y, float* mean,
                   float* rstd, int rows, int cols, float eps, int dtype, int param_dtype) {
  using namespace edf;
  int rc = ln_check(rows, cols, dtype, param_dtype);
  if (rc) return rc;
  EDF_REQUIRE(x && y && mean && rstd, EDF_ERR_INVALID_ARG, "null tensor pointer");
  EDF_REQUIRE(eps >= 0.0f, EDF_ERR_INVALID_ARG, "eps must be non-negative");
  hipStream_t s = as_stream(stream);
  return ln_dtypes(dtype, param_dtype, [&](auto* ti, auto* tp) {
    using T = std::remove_pointer_t<decltype(ti)>;
    using TP = std::remove_pointer_t<decltype(tp)>;
    return ln_fwd<T, TP, false>(s, x, nullptr, nullptr, gamma, beta, y, mean, rstd, rows, cols, eps);
  });
}

int edf_add_layer_norm(void* stream, const void* x, const void* res, void* sum, const void* gamma, const void* beta,
                       void* y, float* mean, float* rstd, int rows, int cols, float eps, int dtype, int param_dtype) {
  using namespace edf;
  int rc = ln_check(rows, cols, dtype, param_dtype);
  if (rc) return rc;
  EDF_REQUIRE(x && res && sum && y && mean && rstd, EDF_ERR_INVALID_ARG, "null tensor pointer");
  EDF_REQUIRE(eps >= 0.0f, EDF_ERR_INVALID_ARG, "eps must be non-negative");
  hipStream_t s = as_stream(stream);
  return ln_dtypes(dtype, param_dtype, [&](auto* ti, auto* tp) {
    using T = std::remove_pointer_t<decltype(ti)>;
    using TP = std::remove_pointer_t<decltype(tp)>;
    return ln_fwd<T, TP, true>(s, x, res, sum, gamma, beta, y, mean, rstd, rows, cols, eps);
  });
}

size_t edf_layer_norm_backward_workspace_bytes(int rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  const int nwg = edf::ln_bwd_groups(rows);
  return (size_t)(nwg + edf::ln_slices(nwg)) * 2 * cols * sizeof(float);
}

int edf_layer_norm_backward(void* stream, const void* x, const void* gamma, const float* mean, const float* rstd,
                            const void* grad_y, void* grad_x, void* grad_gamma, void* grad_beta, void* workspace,
                            size_t workspace_bytes, int rows, int cols, int dtype, int param_dtype) {
  return edf_layer_norm_backward_add(stream, x, gamma, mean, rstd, grad_y, nullptr, grad_x, grad_gamma, grad_beta,
                                     workspace, workspace_bytes, rows, cols, dtype, param_dtype);
}

int edf_layer_norm_backward_add(void* stream, const void* x, const void* gamma, const float* mean, const float* rstd,
                                const void* grad_y, const void* grad_add, void* grad_x, void* grad_gamma,
                                void* grad_beta, void* workspace, size_t workspace_bytes, int rows, int cols,
                                int dtype, int param_dtype) {
  using namespace edf;
  int rc = ln_check(rows, cols, dtype, param_dtype);
  if (rc) return rc;
  EDF_REQUIRE(x && mean && rstd && grad_y && grad_x, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf_layer_norm_backward_workspace_bytes(rows, cols);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  return ln_dtypes(dtype, param_dtype, [&](auto* ti, auto* tp) {
    using T = std::remove_pointer_t<decltype(ti)>;
    using TP = std::remove_pointer_t<decltype(tp)>;
    return grad_add ? ln_bwd<T, TP, true>(s, x, gamma, mean, rstd, grad_y, grad_add, grad_x, grad_gamma, grad_beta,
                                          (float*)workspace, rows, cols)
                    : ln_bwd<T, TP, false>(s, x, gamma, mean, rstd, grad_y, nullptr, grad_x, grad_gamma, grad_beta,
                                           (float*)workspace, rows, cols);
  });
}

}  // extern "C"
