// Causal depthwise conv1d + bias + SiLU, forward and backward: the convolution the Mamba
// block applies to its x branch (lib/edifice/ssm/common.ex:251-252 around
// build_depthwise_conv1d, common.ex:298-309: kernel K, K - 1 steps of left padding, one
// group per channel) and the GatedDeltaNet short convolution
// (lib/edifice/recurrent/gated_delta_net.ex:239-245).  In the reference these are Axon
// layers; here they are the block callers' glue around the fused scans, one pass over
// the activations instead of K shifted multiply-adds in float32 plus their casts.
//
//   pre[b, t, c] = bias[c] + sum_{j < K} w[c, j] x[b, t - (K - 1) + j, c]   (x = 0 for t < 0)
//   y = pre sigmoid(pre)
// backward, g = dy s (1 + pre (1 - s)) with s = sigmoid(pre):
//   dx[t] = sum_j w[j] g[t + K - 1 - j];  dw[j] = sum_{b, t} g[t] x[t - (K - 1) + j];  dbias = sum g
//
// Layout: x [B, T, C] with any row stride (a column slice of a wider projection needs no
// copy), y / dy / dx [B, T, C] contiguous, w [C, K], bias [C].  A thread owns VEC adjacent
// channels (one 16-byte access per step: 8 bf16 or 4 f32; 1 when C or the pointers do not
// allow it) over a run of CC_L steps, keeping the K - 1 previous inputs in registers; the
// threads of a wave cover consecutive channel groups of one step (coalesced rows).  All
// arithmetic in f32.  The backward recomputes pre, forms g for its run plus the K - 1
// steps after it, and reduces dw / dbias over the CC_RW runs of a workgroup in LDS (in run
// order) into one partial per workgroup, which a second kernel adds in workgroup order
// (deterministic, no atomics).
#include <stdint.h>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int CC_L = 32;    // steps per thread run
constexpr int CC_CGW = 64;  // channel groups per workgroup
constexpr int CC_RW = 4;    // runs per workgroup (256 threads)
constexpr int CC_KMAX = 8;

struct CCArgs {
  const void* x;
  const void* w;
  const void* bias;
  const void* dy;
  void* y;   // forward output / backward dx
  float* part;  // [P][C][K + 1] backward partials (dw, dbias)
  long xs;      // row stride of x (elements)
  int B, T, C, nrun, nrb;
};

template <typename T, int VEC> struct Vec;
template <> struct Vec<float, 1> {
  static EDF_DEVICE void ld(const float* p, float* v) { v[0] = *p; }
  static EDF_DEVICE void st(float* p, const float* v) { *p = v[0]; }
};
template <> struct Vec<float, 4> {
  static EDF_DEVICE void ld(const float* p, float* v) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  static EDF_DEVICE void st(float* p, const float* v) { *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]); }
};
template <> struct Vec<bf16, 1> {
  static EDF_DEVICE void ld(const bf16* p, float* v) { v[0] = (float)*p; }
  static EDF_DEVICE void st(bf16* p, const float* v) { *p = (bf16)v[0]; }
};
template <> struct Vec<bf16, 8> {
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

EDF_DEVICE float cc_sigmoid(float v) { return 1.0f / (1.0f + __expf(-v)); }

// this thread's (batch, run, channel group); run and channel group may lie past the end
// (padding threads of the last workgroups: they load nothing and store nothing)
struct CCPos {
  int b, run, cg, rl, cgl;
  bool ok;
};
template <int VEC>
EDF_DEVICE CCPos cc_pos(const CCArgs& a) {
  CCPos q;
  q.cgl = threadIdx.x % CC_CGW;
  q.rl = threadIdx.x / CC_CGW;
  q.cg = blockIdx.x * CC_CGW + q.cgl;
  q.run = blockIdx.y * CC_RW + q.rl;
  q.b = blockIdx.z;
  q.ok = q.cg * VEC < a.C && q.run < a.nrun;
  return q;
}

template <typename T, int VEC, int K>
__global__ __launch_bounds__(256) void cc_fwd_kernel(const CCArgs a) {
  const CCPos q = cc_pos<VEC>(a);
  if (!q.ok) return;
  const int c0 = q.cg * VEC, t0 = q.run * CC_L;
  const T* x = (const T*)a.x + (long)q.b * a.T * a.xs + c0;
  T* y = (T*)a.y + (long)q.b * a.T * a.C + c0;
  float w[K][VEC], bs[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
#pragma unroll
    for (int j = 0; j < K; ++j) w[j][v] = ld((const T*)a.w, (long)(c0 + v) * K + j);
    bs[v] = a.bias ? ld((const T*)a.bias, c0 + v) : 0.0f;
  }
  float win[K][VEC];  // win[j] = x[t - (K - 1) + j] for the current step t (win[K - 1] loaded at t)
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int t = t0 - (K - 1) + j;
    if (t >= 0) Vec<T, VEC>::ld(x + (long)t * a.xs, win[j]);
    else
#pragma unroll
      for (int v = 0; v < VEC; ++v) win[j][v] = 0.0f;
  }
  const int n = min(CC_L, a.T - t0);
#pragma unroll 4
  for (int tt = 0; tt < n; ++tt) {
    const int t = t0 + tt;
    Vec<T, VEC>::ld(x + (long)t * a.xs, win[K - 1]);
    float o[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float pre = bs[v];
#pragma unroll
      for (int j = 0; j < K; ++j) pre = fmaf(w[j][v], win[j][v], pre);
      o[v] = pre * cc_sigmoid(pre);
    }
    Vec<T, VEC>::st(y + (long)t * a.C, o);
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int v = 0; v < VEC; ++v) win[j][v] = win[j + 1][v];
  }
}

template <typename T, int VEC, int K>
__global__ __launch_bounds__(256) void cc_bwd_kernel(const CCArgs a) {
  constexpr int NQ = VEC * (K + 1);  // dw[v][j] and dbias[v] of this thread's channels
  __shared__ float s_red[CC_RW][CC_CGW][NQ + 1];
  const CCPos q = cc_pos<VEC>(a);
  float acc[VEC][K + 1];
#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int j = 0; j <= K; ++j) acc[v][j] = 0.0f;
  if (q.ok) {
    const int c0 = q.cg * VEC, t0 = q.run * CC_L;
    const T* x = (const T*)a.x + (long)q.b * a.T * a.xs + c0;
    const T* dy = (const T*)a.dy + (long)q.b * a.T * a.C + c0;
    T* dx = (T*)a.y + (long)q.b * a.T * a.C + c0;
    float w[K][VEC], bs[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
#pragma unroll
      for (int j = 0; j < K; ++j) w[j][v] = ld((const T*)a.w, (long)(c0 + v) * K + j);
      bs[v] = a.bias ? ld((const T*)a.bias, c0 + v) : 0.0f;
    }
    // walk t = t0 .. t0 + n + K - 2 forming g[t]; xw holds x[t - (K - 1) .. t], gw the last
    // K values of g (gw[K - 1] = g[t]); dx[t - (K - 1)] = sum_j w[j] g[t - j] once t - (K - 1) >= t0
    float xw[K][VEC], gw[K][VEC];
#pragma unroll
    for (int j = 0; j < K; ++j)
#pragma unroll
      for (int v = 0; v < VEC; ++v) gw[j][v] = 0.0f;
#pragma unroll
    for (int j = 0; j < K - 1; ++j) {
      const int t = t0 - (K - 1) + j;
      if (t >= 0) Vec<T, VEC>::ld(x + (long)t * a.xs, xw[j]);
      else
#pragma unroll
        for (int v = 0; v < VEC; ++v) xw[j][v] = 0.0f;
    }
    const int n = min(CC_L, a.T - t0);
    const int tend = min(t0 + n + K - 1, a.T);  // g needed up to t0 + n + K - 2, zero past T
#pragma unroll 2
    for (int t = t0; t < t0 + n + K - 1; ++t) {
      float g[VEC];
      if (t < tend) {
        Vec<T, VEC>::ld(x + (long)t * a.xs, xw[K - 1]);
        float d[VEC];
        Vec<T, VEC>::ld(dy + (long)t * a.C, d);
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          float pre = bs[v];
#pragma unroll
          for (int j = 0; j < K; ++j) pre = fmaf(w[j][v], xw[j][v], pre);
          const float s = cc_sigmoid(pre);
          g[v] = d[v] * s * fmaf(pre, 1.0f - s, 1.0f);
        }
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) g[v] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < K - 1; ++j)
#pragma unroll
        for (int v = 0; v < VEC; ++v) gw[j][v] = gw[j + 1][v];
#pragma unroll
      for (int v = 0; v < VEC; ++v) gw[K - 1][v] = g[v];
      if (t < t0 + n) {  // this run's own step: dw, dbias
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
#pragma unroll
          for (int j = 0; j < K; ++j) acc[v][j] = fmaf(g[v], xw[j][v], acc[v][j]);
          acc[v][K] += g[v];
        }
      }
      const int ts = t - (K - 1);  // dx of step ts needs g[ts .. ts + K - 1] = gw[0 .. K - 1]
      if (ts >= t0) {
        float o[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          float s = 0.0f;
#pragma unroll
          for (int j = 0; j < K; ++j) s = fmaf(w[j][v], gw[K - 1 - j][v], s);
          o[v] = s;
        }
        Vec<T, VEC>::st(dx + (long)ts * a.C, o);
      }
#pragma unroll
      for (int j = 0; j < K - 1; ++j)
#pragma unroll
        for (int v = 0; v < VEC; ++v) xw[j][v] = xw[j + 1][v];
    }
  }
  // dw / dbias over the workgroup's runs, in run order, into this workgroup's partial
#pragma unroll
  for (int v = 0; v < VEC; ++v)
#pragma unroll
    for (int j = 0; j <= K; ++j) s_red[q.rl][q.cgl][v * (K + 1) + j] = acc[v][j];
  __syncthreads();
  const long P = (long)q.b * a.nrb + blockIdx.y;
  for (int e = threadIdx.x; e < CC_CGW * NQ; e += 256) {
    const int cgl = e / NQ, r = e % NQ;
    const int c = (blockIdx.x * CC_CGW + cgl) * VEC + r / (K + 1);
    if (c >= a.C) continue;
    float s = 0.0f;
#pragma unroll
    for (int rl = 0; rl < CC_RW; ++rl) s += s_red[rl][cgl][r];
    a.part[(P * a.C + c) * (K + 1) + r % (K + 1)] = s;
  }
}

// dw [C][K] and dbias [C] = the P workgroup partials: 8 lanes per output each add a
// contiguous eighth of them in order, then the eight sums are combined in a fixed tree
// (deterministic; one thread per output would leave most of the chip idle)
template <typename T, int K>
__global__ __launch_bounds__(256) void cc_reduce_kernel(const float* __restrict__ part, T* dw, T* dbias, int C, long P) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) >> 3;  // over C (K + 1)
  const int sub = threadIdx.x & 7;
  const long n = (long)C * (K + 1);
  const long p0 = (P * sub) / 8, p1 = (P * (sub + 1)) / 8;
  float s = 0.0f;
  if (i < n)
    for (long p = p0; p < p1; ++p) s += part[p * n + i];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  if (i >= n || sub != 0) return;
  const int c = (int)(i / (K + 1)), j = (int)(i % (K + 1));
  if (j < K) {
    if (dw) dw[(long)c * K + j] = (T)s;
  } else if (dbias) {
    dbias[c] = (T)s;
  }
}

template <typename T, int K>
int cc_launch(hipStream_t s, CCArgs& a, bool bwd, int vec, void* dw, void* dbias) {
  const int ncg = (a.C + vec - 1) / vec;
  const dim3 grid((ncg + CC_CGW - 1) / CC_CGW, a.nrb, a.B);
  if (!bwd) {
    if (vec > 1)
      cc_fwd_kernel<T, (sizeof(T) == 2 ? 8 : 4), K><<<grid, 256, 0, s>>>(a);
    else
      cc_fwd_kernel<T, 1, K><<<grid, 256, 0, s>>>(a);
    return check_launch("causal conv");
  }
  if (vec > 1)
    cc_bwd_kernel<T, (sizeof(T) == 2 ? 8 : 4), K><<<grid, 256, 0, s>>>(a);
  else
    cc_bwd_kernel<T, 1, K><<<grid, 256, 0, s>>>(a);
  if (int rc = check_launch("causal conv backward")) return rc;
  if (dw || dbias) {
    const long n = (long)a.C * (K + 1);
    cc_reduce_kernel<T, K><<<(unsigned)((8 * n + 255) / 256), 256, 0, s>>>(a.part, (T*)dw, (T*)dbias, a.C,
                                                                       (long)a.B * a.nrb);
    return check_launch("causal conv dw reduction");
  }
  return EDF_OK;
}

template <typename T>
int cc_dispatch(hipStream_t s, CCArgs& a, int K, bool bwd, int vec, void* dw, void* dbias) {
  switch (K) {
    case 1: return cc_launch<T, 1>(s, a, bwd, vec, dw, dbias);
    case 2: return cc_launch<T, 2>(s, a, bwd, vec, dw, dbias);
    case 3: return cc_launch<T, 3>(s, a, bwd, vec, dw, dbias);
    case 4: return cc_launch<T, 4>(s, a, bwd, vec, dw, dbias);
    case 5: return cc_launch<T, 5>(s, a, bwd, vec, dw, dbias);
    case 6: return cc_launch<T, 6>(s, a, bwd, vec, dw, dbias);
    case 7: return cc_launch<T, 7>(s, a, bwd, vec, dw, dbias);
    default: return cc_launch<T, 8>(s, a, bwd, vec, dw, dbias);
  }
}

// 16-byte accesses when every row start of x, y / dy / dx is 16-byte aligned
int cc_vec(const CCArgs& a, int dtype, const void* out2) {
  const int vec = dtype == EDF_BF16 ? 8 : 4;
  const size_t es = dtype == EDF_BF16 ? 2 : 4;
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; };
  const bool ok = a.C % vec == 0 && a.xs % vec == 0 && al(a.x) && al(a.y) && al(a.dy) && al(out2) &&
                  (a.xs * es) % 16 == 0;
  return ok ? vec : 1;
}

int cc_common(CCArgs& a, const void* x, int x_row_stride, const void* w, const void* bias, int batch, int seq_len,
              int channels, int kernel_size, int dtype) {
  EDF_REQUIRE(batch > 0 && seq_len > 0 && channels > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(kernel_size >= 1 && kernel_size <= CC_KMAX, EDF_ERR_UNSUPPORTED, "kernel_size must be 1..%d", CC_KMAX);
  EDF_REQUIRE(x_row_stride >= channels, EDF_ERR_INVALID_ARG, "x_row_stride (%d) < channels (%d)", x_row_stride,
              channels);
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(x && w, EDF_ERR_INVALID_ARG, "null tensor pointer");
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.xs = x_row_stride;
  a.B = batch;
  a.T = seq_len;
  a.C = channels;
  a.nrun = (seq_len + CC_L - 1) / CC_L;
  a.nrb = (a.nrun + CC_RW - 1) / CC_RW;
  return EDF_OK;
}

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace
}  // namespace edf

extern "C" {

int edf_causal_conv1d_silu(void* stream, const void* x, int x_row_stride, const void* weight, const void* bias,
                           void* out, int batch, int seq_len, int channels, int kernel_size, int dtype) {
  using namespace edf;
  CCArgs a{};
  if (int rc = cc_common(a, x, x_row_stride, weight, bias, batch, seq_len, channels, kernel_size, dtype)) return rc;
  EDF_REQUIRE(out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  a.y = out;
  const int vec = cc_vec(a, dtype, nullptr);
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? cc_dispatch<bf16>(s, a, kernel_size, false, vec, nullptr, nullptr)
                           : cc_dispatch<float>(s, a, kernel_size, false, vec, nullptr, nullptr);
}

size_t edf_causal_conv1d_silu_backward_workspace_bytes(int batch, int seq_len, int channels, int kernel_size) {
  if (batch <= 0 || seq_len <= 0 || channels <= 0 || kernel_size < 1 || kernel_size > edf::CC_KMAX) return 0;
  const long nrb = ((seq_len + edf::CC_L - 1) / edf::CC_L + edf::CC_RW - 1) / edf::CC_RW;
  return edf::align256((size_t)batch * nrb * channels * (kernel_size + 1) * sizeof(float));
}

int edf_causal_conv1d_silu_backward(void* stream, const void* x, int x_row_stride, const void* weight,
                                    const void* bias, const void* grad_out, void* grad_x, void* grad_weight,
                                    void* grad_bias, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                    int channels, int kernel_size, int dtype) {
  using namespace edf;
  CCArgs a{};
  if (int rc = cc_common(a, x, x_row_stride, weight, bias, batch, seq_len, channels, kernel_size, dtype)) return rc;
  EDF_REQUIRE(grad_out && grad_x, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf_causal_conv1d_silu_backward_workspace_bytes(batch, seq_len, channels, kernel_size);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  a.dy = grad_out;
  a.y = grad_x;
  a.part = (float*)workspace;
  const int vec = cc_vec(a, dtype, nullptr);
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? cc_dispatch<bf16>(s, a, kernel_size, true, vec, grad_weight, grad_bias)
                           : cc_dispatch<float>(s, a, kernel_size, true, vec, grad_weight, grad_bias);
}

}  // extern "C"
