// Flash attention forward for gfx950: O = softmax(Q K^T / sqrt(d) [+ causal -inf]) V.
//
// Semantics (reference): lib/edifice/cuda/fused_scan.ex:3476-3508 (flash_attention_fallback),
// native/cuda/fused_flash_attention.cu:52-154; layout [B, H, T, d]; causal keeps keys
// j <= i.  Additionally emits the natural-log row log-sum-exp (float32 [B, H, T]) used
// by the backward.
//
// bf16 path (the performance path), per workgroup of 4 waves and 128 queries:
//   * each wave owns 32 queries; Q^T stays in registers as MFMA B fragments;
//   * K and V tiles of 64 keys are staged in LDS (K row-major, V transposed to
//     [dim][key] so the MFMA A operand of V^T is a contiguous LDS read), rows padded
//     against bank conflicts;
//   * S^T = K Q^T with v_mfma_f32_32x32x16_bf16: every lane owns one query column,
//     so the online-softmax max/sum are lane-local plus one exchange between the two
//     wave halves;
//   * O^T += V^T P^T reuses the S^T result registers directly as the B operand
//     (keys permuted consistently in the V^T reads), so P never goes through LDS;
//   * causal: key tiles above the diagonal are skipped, only diagonal tiles are
//     masked, and query blocks are issued heaviest-first.
// f32 (or odd head_dim) path: one wave per query, lanes over head_dim, for parity.
#include "edf_abi.hpp"
#include "edf_common.hpp"
#include "edf_mfma.hpp"

namespace edf {
namespace {

constexpr float LN2 = 0.6931471805599453f;

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fa_fwd_mfma_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                             const bf16* __restrict__ V, bf16* __restrict__ O,
                                                             float* __restrict__ LSE, int T, float scale_log2) {
  constexpr int BM = 128, BN = 64;
  constexpr int KS = HD + 8;  // sK row stride (elements)
  constexpr int VS = BN + 4;  // sVt row stride (elements)
  constexpr int NKK = HD / 16, NDT = HD / 32;
  __shared__ __attribute__((aligned(16))) bf16 sK[BN * KS];
  __shared__ __attribute__((aligned(16))) bf16 sVt[HD * VS];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const long bh = blockIdx.y;
  const int qb = CAUSAL ? (gridDim.x - 1 - blockIdx.x) : blockIdx.x;
  const int q0 = qb * BM;
  const int qw = q0 + 32 * w;
  const int myq = qw + li;
  const bf16* Qh = Q + bh * T * HD;
  const bf16* Kh = K + bh * T * HD;
  const bf16* Vh = V + bh * T * HD;

  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    if (myq < T)
      qf[kk] = *(const bf16x8*)(Qh + (long)myq * HD + kk * 16 + 8 * g);
    else
      qf[kk] = bf16x8{};
  }
  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = zero16();
  float m = -INFINITY, lsum = 0.0f;

  const int kend = CAUSAL ? min(T, q0 + BM) : T;
  const int nkt = (kend + BN - 1) / BN;
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * BN;
    __syncthreads();
    for (int c = tid; c < BN * HD / 8; c += 256) {
      const int row = c / (HD / 8), col = (c % (HD / 8)) * 8;
      const int key = k0 + row;
      bf16x8 v = key < T ? *(const bf16x8*)(Kh + (long)key * HD + col) : bf16x8{};
      *(bf16x8*)(sK + row * KS + col) = v;
    }
    for (int c = tid; c < (BN / 2) * (HD / 8); c += 256) {
      const int kp = c / (HD / 8), col = (c % (HD / 8)) * 8;
      const int key = k0 + 2 * kp;
      bf16x8 v0 = key < T ? *(const bf16x8*)(Vh + (long)key * HD + col) : bf16x8{};
      bf16x8 v1 = key + 1 < T ? *(const bf16x8*)(Vh + (long)(key + 1) * HD + col) : bf16x8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
        bf16x2 pr = {v0[e], v1[e]};
        *(bf16x2*)(sVt + (col + e) * VS + 2 * kp) = pr;
      }
    }
    __syncthreads();

    f32x16 s[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      s[h2] = zero16();
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const bf16x8 a = *(const bf16x8*)(sK + (h2 * 32 + li) * KS + kk * 16 + 8 * g);
        s[h2] = mfma32(a, qf[kk], s[h2]);
      }
    }
    const bool need_mask = (k0 + BN > T) || (CAUSAL && k0 + BN - 1 > qw);
    float mx = -INFINITY;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[h2][r] * scale_log2;
        if (need_mask) {
          const int key = k0 + h2 * 32 + d_row(r, g);
          if (key >= T || (CAUSAL && key > myq)) v = -INFINITY;
        }
        s[h2][r] = v;
        mx = fmaxf(mx, v);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(m, mx);
    const float alpha = fast_exp2(m - mnew);
    float rs = 0.0f;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(s[h2][r] - mnew);
        s[h2][r] = p;
        rs += p;
      }
    }
    rs += __shfl_xor(rs, 32);
    lsum = lsum * alpha + rs;
    m = mnew;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;

    bf16x8 pf[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int it = 0; it < 8; ++it) pf[kc][it] = (bf16)s[kc >> 1][8 * (kc & 1) + it];

#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const bf16* vrow = sVt + (dt * 32 + li) * VS + 4 * g;
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const bf16x8 a = cat4(*(const bf16x4*)(vrow + kc * 16), *(const bf16x4*)(vrow + kc * 16 + 8));
        o[dt] = mfma32(a, pf[kc], o[dt]);
      }
    }
  }

  if (myq < T) {
    const float inv = 1.0f / lsum;
    bf16* orow = O + bh * T * HD + (long)myq * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(o[dt][rb * 4 + e] * inv);
        *(bf16x4*)(orow + dt * 32 + 8 * rb + 4 * g) = v;
      }
    if (g == 0 && LSE != nullptr) LSE[bh * T + myq] = (m + __log2f(lsum)) * LN2;
  }
}

// Generic path: one wave per query row, lanes over head_dim (any dtype, any head_dim <= 256).
template <typename TT, int DPL>
__global__ __launch_bounds__(256) void fa_fwd_wave_kernel(const TT* __restrict__ Q, const TT* __restrict__ K,
                                                          const TT* __restrict__ V, TT* __restrict__ O,
                                                          float* __restrict__ LSE, int BH, int T, int HD,
                                                          float scale_log2, int causal) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= BH * T) return;
  const long bh = row / T;
  const int i = row % T;
  float q[DPL], o[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    q[e] = d < HD ? ld(Q, (bh * T + i) * HD + d) : 0.0f;
    o[e] = 0.0f;
  }
  float m = -INFINITY, lsum = 0.0f;
  const int jend = causal ? i + 1 : T;
  for (int j = 0; j < jend; ++j) {
    const long kb = (bh * T + j) * HD;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) s = fmaf(q[e], ld(K, kb + d), s);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    s *= scale_log2;
    const float mnew = fmaxf(m, s);
    const float alpha = fast_exp2(m - mnew);
    const float p = fast_exp2(s - mnew);
    lsum = lsum * alpha + p;
    m = mnew;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      o[e] = o[e] * alpha + (d < HD ? p * ld(V, kb + d) : 0.0f);
    }
  }
  const float inv = 1.0f / lsum;
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) st(O, (bh * T + i) * HD + d, o[e] * inv);
  }
  if (lane == 0 && LSE != nullptr) LSE[bh * T + i] = (m + __log2f(lsum)) * LN2;
}

__global__ void debug_mfma_kernel(const bf16* A, const bf16* B, float* C) {
  const int l = threadIdx.x, g = l >> 5, li = l & 31;
  bf16x8 a, b;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    a[it] = A[li * 16 + 8 * g + it];   // A row-major [32][16]
    b[it] = B[(8 * g + it) * 32 + li]; // B row-major [16][32]
  }
  f32x16 d = mfma32(a, b, zero16());
#pragma unroll
  for (int r = 0; r < 16; ++r) C[d_row(r, g) * 32 + li] = d[r];
}

template <int HD>
void launch_mfma_fwd(hipStream_t s, const void* q, const void* k, const void* v, void* o, float* lse, int BH, int T,
                     int causal, float scale_log2) {
  const dim3 grid((T + 127) / 128, BH);
  if (causal)
    fa_fwd_mfma_kernel<HD, true><<<grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, (bf16*)o, lse,
                                                      T, scale_log2);
  else
    fa_fwd_mfma_kernel<HD, false><<<grid, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, (bf16*)o, lse,
                                                       T, scale_log2);
}

template <typename TT>
void launch_wave_fwd(hipStream_t s, const void* q, const void* k, const void* v, void* o, float* lse, int BH, int T,
                     int HD, int causal, float scale_log2) {
  const long rows = (long)BH * T;
  const unsigned grid = (unsigned)((rows + 3) / 4);
  if (HD <= 64)
    fa_fwd_wave_kernel<TT, 1><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (TT*)o, lse, BH, T, HD,
                                                   scale_log2, causal);
  else if (HD <= 128)
    fa_fwd_wave_kernel<TT, 2><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (TT*)o, lse, BH, T, HD,
                                                   scale_log2, causal);
  else
    fa_fwd_wave_kernel<TT, 4><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (TT*)o, lse, BH, T, HD,
                                                   scale_log2, causal);
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_debug_mfma_32x32x16_bf16(void* stream, const void* A, const void* B, float* C) {
  EDF_REQUIRE(A && B && C, EDF_ERR_INVALID_ARG, "null tensor pointer");
  edf::debug_mfma_kernel<<<1, 64, 0, edf::as_stream(stream)>>>((const edf::bf16*)A, (const edf::bf16*)B, C);
  return edf::check_launch("debug mfma");
}

int edf_fused_flash_attention(void* stream, const void* q, const void* k, const void* v, void* out, float* lse,
                              int batch, int num_heads, int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(head_dim <= 256, EDF_ERR_UNSUPPORTED, "head_dim %d > 256 unsupported", head_dim);
  EDF_REQUIRE(q && k && v && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
  const float scale_log2 = LOG2E / sqrtf((float)head_dim);
  if (dtype == EDF_BF16 && (head_dim == 32 || head_dim == 64 || head_dim == 128)) {
    if (head_dim == 128)
      launch_mfma_fwd<128>(s, q, k, v, out, lse, BH, seq_len, causal, scale_log2);
    else if (head_dim == 64)
      launch_mfma_fwd<64>(s, q, k, v, out, lse, BH, seq_len, causal, scale_log2);
    else
      launch_mfma_fwd<32>(s, q, k, v, out, lse, BH, seq_len, causal, scale_log2);
  } else if (dtype == EDF_BF16) {
    launch_wave_fwd<bf16>(s, q, k, v, out, lse, BH, seq_len, head_dim, causal, scale_log2);
  } else {
    launch_wave_fwd<float>(s, q, k, v, out, lse, BH, seq_len, head_dim, causal, scale_log2);
  }
  return check_launch("flash attention");
}

}  // extern "C"
