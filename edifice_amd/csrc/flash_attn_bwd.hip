// Flash attention backward for gfx950.
//
// Semantics (reference): lib/edifice/cuda/fused_scan.ex:3527-3570
// (flash_attention_backward_fallback): P = softmax(S), dV = P^T dO, dP = dO V^T,
// dS = P (dP - rowsum(dP P)) / sqrt(d), dQ = dS K, dK = dS^T Q; and
// native/cuda/fused_flash_attention_backward.cu:256-340 for D = rowsum(dO * O).
// The softmax is recomputed from the forward's log-sum-exp (natural log).
//
// bf16 / head_dim in {32, 64, 128} runs three kernels, none of which allocates or
// uses atomics:
//   1. D = rowsum(dO * O) (float32, one 16-lane group per row);
//   2. dK/dV: a workgroup owns 128 keys (32 per wave, K and V kept in registers as
//      MFMA B fragments) and walks the query tiles; S = Q K^T puts one key per lane
//      column, so P and dS feed dV += P^T dO and dK += dS^T Q directly from
//      registers (Q and dO are staged in LDS both row-major and transposed);
//   3. dQ: a workgroup owns 128 queries (32 per wave, Q and dO in registers) and
//      walks the key tiles; S^T = K Q^T puts one query per lane, so dS feeds
//      dQ += dS K from registers (K staged transposed in LDS).
//   Causal: only tiles on or below the diagonal are visited.
// float32 or other head_dim: wave-per-row kernels (parity path).
#include "edf_abi.hpp"
#include "edf_common.hpp"
#include "edf_mfma.hpp"

namespace edf {
namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// ---- D = rowsum(dO * O) ------------------------------------------------------
template <typename TT>
__global__ __launch_bounds__(256) void fa_bwd_dot_kernel(const TT* __restrict__ O, const TT* __restrict__ dO,
                                                         float* __restrict__ Dv, long rows, int HD) {
  const long row = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  float acc = 0.0f;
  if (row < rows)
    for (int d = sub; d < HD; d += 16) acc = fmaf(ld(O, row * HD + d), ld(dO, row * HD + d), acc);
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (row < rows && sub == 0) Dv[row] = acc;
}

// ---- dK / dV -------------------------------------------------------------------
template <int HD, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fa_bwd_dkdv_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                             const bf16* __restrict__ V, const bf16* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             const float* __restrict__ Dd, bf16* __restrict__ dK,
                                                             bf16* __restrict__ dV, int T, float scale_log2,
                                                             float scale) {
  constexpr int BKEY = 128, BQ = 32;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  constexpr int RS = HD + 8;  // row-major tile stride
  constexpr int TS = BQ + 4;  // transposed tile stride
  __shared__ __attribute__((aligned(16))) bf16 sQ[BQ * RS];
  __shared__ __attribute__((aligned(16))) bf16 sdO[BQ * RS];
  __shared__ __attribute__((aligned(16))) bf16 sQt[HD * TS];
  __shared__ __attribute__((aligned(16))) bf16 sdOt[HD * TS];
  __shared__ __attribute__((aligned(16))) float sL[BQ];
  __shared__ __attribute__((aligned(16))) float sD[BQ];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const long bh = blockIdx.y;
  const int kb0 = blockIdx.x * BKEY;
  const int kw = kb0 + 32 * w;
  const int mykey = kw + li;
  const long base = bh * T * HD;

  // K, V as B fragments: B[k = dim][j = key] -> lane holds row `mykey`, 8 dims
  bf16x8 kf[NKK], vf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    if (mykey < T) {
      kf[kk] = *(const bf16x8*)(K + base + (long)mykey * HD + kk * 16 + 8 * g);
      vf[kk] = *(const bf16x8*)(V + base + (long)mykey * HD + kk * 16 + 8 * g);
    } else {
      kf[kk] = bf16x8{};
      vf[kk] = bf16x8{};
    }
  }
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dk[dt] = zero16();
    dv[dt] = zero16();
  }

  const int qstart = CAUSAL ? (kb0 / BQ) * BQ : 0;
  for (int q0 = qstart; q0 < T; q0 += BQ) {
    __syncthreads();
    for (int c = tid; c < BQ * HD / 8; c += 256) {
      const int row = c / (HD / 8), col = (c % (HD / 8)) * 8;
      const int q = q0 + row;
      bf16x8 a = q < T ? *(const bf16x8*)(Q + base + (long)q * HD + col) : bf16x8{};
      bf16x8 b = q < T ? *(const bf16x8*)(dO + base + (long)q * HD + col) : bf16x8{};
      *(bf16x8*)(sQ + row * RS + col) = a;
      *(bf16x8*)(sdO + row * RS + col) = b;
    }
    for (int c = tid; c < (BQ / 2) * (HD / 8); c += 256) {
      const int qp = c / (HD / 8), col = (c % (HD / 8)) * 8;
      const int q = q0 + 2 * qp;
      const bf16x8 a0 = q < T ? *(const bf16x8*)(Q + base + (long)q * HD + col) : bf16x8{};
      const bf16x8 a1 = q + 1 < T ? *(const bf16x8*)(Q + base + (long)(q + 1) * HD + col) : bf16x8{};
      const bf16x8 b0 = q < T ? *(const bf16x8*)(dO + base + (long)q * HD + col) : bf16x8{};
      const bf16x8 b1 = q + 1 < T ? *(const bf16x8*)(dO + base + (long)(q + 1) * HD + col) : bf16x8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        *(bf16x2*)(sQt + (col + e) * TS + 2 * qp) = bf16x2{a0[e], a1[e]};
        *(bf16x2*)(sdOt + (col + e) * TS + 2 * qp) = bf16x2{b0[e], b1[e]};
      }
    }
    if (tid < BQ) {
      const int q = q0 + tid;
      sL[tid] = q < T ? LSE[bh * T + q] * LOG2E : 0.0f;
      sD[tid] = q < T ? Dd[bh * T + q] : 0.0f;
    }
    __syncthreads();
    if (CAUSAL && q0 + BQ - 1 < kw) continue;  // every query of the tile precedes this wave's keys

    // S = Q K^T and dP = dO V^T (32 queries x 32 keys); lane owns key column
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const bf16x8 aq = *(const bf16x8*)(sQ + li * RS + kk * 16 + 8 * g);
      const bf16x8 ao = *(const bf16x8*)(sdO + li * RS + kk * 16 + 8 * g);
      s = mfma32(aq, kf[kk], s);
      dp = mfma32(ao, vf[kk], dp);
    }
    const bool mask = (q0 + BQ > T) || (mykey >= T) || (CAUSAL && q0 < kw + 31);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const f32x4 lv = *(const f32x4*)(sL + 8 * rb + 4 * g);
      const f32x4 dv4 = *(const f32x4*)(sD + 8 * rb + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = rb * 4 + e;
        float p = fast_exp2(s[r] * scale_log2 - lv[e]);
        if (mask) {
          const int q = q0 + 8 * rb + 4 * g + e;
          if (q >= T || mykey >= T || (CAUSAL && mykey > q)) p = 0.0f;
        }
        s[r] = p;
        dp[r] = p * (dp[r] - dv4[e]) * scale;
      }
    }
    // A fragments of P^T and dS^T (rows = keys, k = queries in the permuted order)
    bf16x8 pa[2], da[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        pa[kc][it] = (bf16)s[8 * kc + it];
        da[kc][it] = (bf16)dp[8 * kc + it];
      }
    // dV += P^T dO ; dK += dS^T Q   (B = dO / Q rows for 8 permuted queries, one dim)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const bf16* orow = sdOt + (dt * 32 + li) * TS + 4 * g;
      const bf16* qrow = sQt + (dt * 32 + li) * TS + 4 * g;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const bf16x8 bo = cat4(*(const bf16x4*)(orow + kc * 16), *(const bf16x4*)(orow + kc * 16 + 8));
        const bf16x8 bq = cat4(*(const bf16x4*)(qrow + kc * 16), *(const bf16x4*)(qrow + kc * 16 + 8));
        dv[dt] = mfma32(pa[kc], bo, dv[dt]);
        dk[dt] = mfma32(da[kc], bq, dk[dt]);
      }
    }
  }
  // dK, dV: D[i = key][j = dim] -> lane owns dim column li of tile dt, rows = keys
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kw + d_row(r, g);
      if (key < T) {
        dK[base + (long)key * HD + dt * 32 + li] = (bf16)dk[dt][r];
        dV[base + (long)key * HD + dt * 32 + li] = (bf16)dv[dt][r];
      }
    }
}

// ---- dQ -----------------------------------------------------------------------------
template <int HD, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fa_bwd_dq_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                           const bf16* __restrict__ V, const bf16* __restrict__ dO,
                                                           const float* __restrict__ LSE, const float* __restrict__ Dd,
                                                           bf16* __restrict__ dQ, int T, float scale_log2,
                                                           float scale) {
  constexpr int BM = 128, BN = 64;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  constexpr int RS = HD + 8;
  constexpr int TS = BN + 4;
  __shared__ __attribute__((aligned(16))) bf16 sK[BN * RS];
  __shared__ __attribute__((aligned(16))) bf16 sV[BN * RS];
  __shared__ __attribute__((aligned(16))) bf16 sKt[HD * TS];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const long bh = blockIdx.y;
  const int qb = CAUSAL ? (gridDim.x - 1 - blockIdx.x) : blockIdx.x;
  const int q0 = qb * BM;
  const int qw = q0 + 32 * w;
  const int myq = qw + li;
  const long base = bh * T * HD;

  bf16x8 qf[NKK], of[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    if (myq < T) {
      qf[kk] = *(const bf16x8*)(Q + base + (long)myq * HD + kk * 16 + 8 * g);
      of[kk] = *(const bf16x8*)(dO + base + (long)myq * HD + kk * 16 + 8 * g);
    } else {
      qf[kk] = bf16x8{};
      of[kk] = bf16x8{};
    }
  }
  const float myl = myq < T ? LSE[bh * T + myq] * LOG2E : 0.0f;
  const float myd = myq < T ? Dd[bh * T + myq] : 0.0f;
  f32x16 dq[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dq[dt] = zero16();

  const int kend = CAUSAL ? min(T, q0 + BM) : T;
  for (int k0 = 0; k0 < kend; k0 += BN) {
    __syncthreads();
    for (int c = tid; c < BN * HD / 8; c += 256) {
      const int row = c / (HD / 8), col = (c % (HD / 8)) * 8;
      const int key = k0 + row;
      *(bf16x8*)(sK + row * RS + col) = key < T ? *(const bf16x8*)(K + base + (long)key * HD + col) : bf16x8{};
      *(bf16x8*)(sV + row * RS + col) = key < T ? *(const bf16x8*)(V + base + (long)key * HD + col) : bf16x8{};
    }
    for (int c = tid; c < (BN / 2) * (HD / 8); c += 256) {
      const int kp = c / (HD / 8), col = (c % (HD / 8)) * 8;
      const int key = k0 + 2 * kp;
      const bf16x8 a0 = key < T ? *(const bf16x8*)(K + base + (long)key * HD + col) : bf16x8{};
      const bf16x8 a1 = key + 1 < T ? *(const bf16x8*)(K + base + (long)(key + 1) * HD + col) : bf16x8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) *(bf16x2*)(sKt + (col + e) * TS + 2 * kp) = bf16x2{a0[e], a1[e]};
    }
    __syncthreads();
    if (CAUSAL && k0 > qw + 31) continue;

    f32x16 s[2], dp[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      s[h2] = zero16();
      dp[h2] = zero16();
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const bf16x8 ak = *(const bf16x8*)(sK + (h2 * 32 + li) * RS + kk * 16 + 8 * g);
        const bf16x8 av = *(const bf16x8*)(sV + (h2 * 32 + li) * RS + kk * 16 + 8 * g);
        s[h2] = mfma32(ak, qf[kk], s[h2]);
        dp[h2] = mfma32(av, of[kk], dp[h2]);
      }
    }
    const bool mask = (k0 + BN > T) || (myq >= T) || (CAUSAL && k0 + BN - 1 > qw);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(s[h2][r] * scale_log2 - myl);
        if (mask) {
          const int key = k0 + h2 * 32 + d_row(r, g);
          if (key >= T || myq >= T || (CAUSAL && key > myq)) p = 0.0f;
        }
        s[h2][r] = p * (dp[h2][r] - myd) * scale;  // dS^T
      }
    bf16x8 da[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int it = 0; it < 8; ++it) da[kc][it] = (bf16)s[kc >> 1][8 * (kc & 1) + it];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const bf16* krow = sKt + (dt * 32 + li) * TS + 4 * g;
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const bf16x8 b = cat4(*(const bf16x4*)(krow + kc * 16), *(const bf16x4*)(krow + kc * 16 + 8));
        dq[dt] = mfma32(da[kc], b, dq[dt]);
      }
    }
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = qw + d_row(r, g);
      if (q < T) dQ[base + (long)q * HD + dt * 32 + li] = (bf16)dq[dt][r];
    }
}

// ---- generic wave-per-row kernels (float32 / any head_dim) ------------------------
template <typename TT, int DPL>
__global__ __launch_bounds__(256) void fa_bwd_dq_wave_kernel(const TT* __restrict__ Q, const TT* __restrict__ K,
                                                             const TT* __restrict__ V, const TT* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             const float* __restrict__ Dd, TT* __restrict__ dQ, int BH,
                                                             int T, int HD, float scale_log2, float scale,
                                                             int causal) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (long)BH * T) return;
  const long bh = row / T;
  const int i = (int)(row % T);
  float q[DPL], go[DPL], acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    q[e] = d < HD ? ld(Q, row * HD + d) : 0.0f;
    go[e] = d < HD ? ld(dO, row * HD + d) : 0.0f;
    acc[e] = 0.0f;
  }
  const float lse2 = LSE[row] * LOG2E, Di = Dd[row];
  const int jend = causal ? i + 1 : T;
  for (int j = 0; j < jend; ++j) {
    const long kb = (bh * T + j) * HD;
    float s = 0.0f, dp = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) {
        s = fmaf(q[e], ld(K, kb + d), s);
        dp = fmaf(go[e], ld(V, kb + d), dp);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s += __shfl_xor(s, off);
      dp += __shfl_xor(dp, off);
    }
    const float ds = fast_exp2(s * scale_log2 - lse2) * (dp - Di) * scale;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) acc[e] = fmaf(ds, ld(K, kb + d), acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) st(dQ, row * HD + d, acc[e]);
  }
}

template <typename TT, int DPL>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_wave_kernel(const TT* __restrict__ Q, const TT* __restrict__ K,
                                                               const TT* __restrict__ V, const TT* __restrict__ dO,
                                                               const float* __restrict__ LSE,
                                                               const float* __restrict__ Dd, TT* __restrict__ dK,
                                                               TT* __restrict__ dV, int BH, int T, int HD,
                                                               float scale_log2, float scale, int causal) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (long)BH * T) return;
  const long bh = row / T;
  const int j = (int)(row % T);
  float kk[DPL], vv[DPL], ak[DPL], av[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    kk[e] = d < HD ? ld(K, row * HD + d) : 0.0f;
    vv[e] = d < HD ? ld(V, row * HD + d) : 0.0f;
    ak[e] = av[e] = 0.0f;
  }
  for (int i = causal ? j : 0; i < T; ++i) {
    const long qb = (bh * T + i) * HD;
    float s = 0.0f, dp = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) {
        s = fmaf(ld(Q, qb + d), kk[e], s);
        dp = fmaf(ld(dO, qb + d), vv[e], dp);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s += __shfl_xor(s, off);
      dp += __shfl_xor(dp, off);
    }
    const float p = fast_exp2(s * scale_log2 - LSE[bh * T + i] * LOG2E);
    const float ds = p * (dp - Dd[bh * T + i]) * scale;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) {
        av[e] = fmaf(p, ld(dO, qb + d), av[e]);
        ak[e] = fmaf(ds, ld(Q, qb + d), ak[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) {
      st(dK, row * HD + d, ak[e]);
      st(dV, row * HD + d, av[e]);
    }
  }
}

template <int HD>
void launch_mfma_bwd(hipStream_t s, const void* q, const void* k, const void* v, const void* go, const float* lse,
                     const float* Dd, void* dq, void* dk, void* dv, int BH, int T, int causal, float scale_log2,
                     float scale) {
  const dim3 g1((T + 127) / 128, BH);
  if (causal) {
    fa_bwd_dkdv_kernel<HD, true><<<g1, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, (const bf16*)go,
                                                    lse, Dd, (bf16*)dk, (bf16*)dv, T, scale_log2, scale);
    fa_bwd_dq_kernel<HD, true><<<g1, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, (const bf16*)go,
                                                  lse, Dd, (bf16*)dq, T, scale_log2, scale);
  } else {
    fa_bwd_dkdv_kernel<HD, false><<<g1, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v,
                                                     (const bf16*)go, lse, Dd, (bf16*)dk, (bf16*)dv, T, scale_log2,
                                                     scale);
    fa_bwd_dq_kernel<HD, false><<<g1, 256, 0, s>>>((const bf16*)q, (const bf16*)k, (const bf16*)v, (const bf16*)go,
                                                   lse, Dd, (bf16*)dq, T, scale_log2, scale);
  }
}

template <typename TT>
void launch_wave_bwd(hipStream_t s, const void* q, const void* k, const void* v, const void* go, const float* lse,
                     const float* Dd, void* dq, void* dk, void* dv, int BH, int T, int HD, int causal,
                     float scale_log2, float scale) {
  const long rows = (long)BH * T;
  const unsigned grid = (unsigned)((rows + 3) / 4);
#define EDF_FA_WAVE_BWD(DPL)                                                                                      \
  fa_bwd_dq_wave_kernel<TT, DPL><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (const TT*)go, lse, \
                                                      Dd, (TT*)dq, BH, T, HD, scale_log2, scale, causal);          \
  fa_bwd_dkdv_wave_kernel<TT, DPL><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (const TT*)go,    \
                                                        lse, Dd, (TT*)dk, (TT*)dv, BH, T, HD, scale_log2, scale,   \
                                                        causal)
  if (HD <= 64) {
    EDF_FA_WAVE_BWD(1);
  } else if (HD <= 128) {
    EDF_FA_WAVE_BWD(2);
  } else {
    EDF_FA_WAVE_BWD(4);
  }
#undef EDF_FA_WAVE_BWD
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_flash_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim) {
  if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  return (size_t)batch * num_heads * seq_len * sizeof(float);
}

int edf_fused_flash_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* out,
                                       const void* grad_out, const float* lse, void* grad_q, void* grad_k,
                                       void* grad_v, void* workspace, size_t workspace_bytes, int batch,
                                       int num_heads, int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(head_dim <= 256, EDF_ERR_UNSUPPORTED, "head_dim %d > 256 unsupported", head_dim);
  EDF_REQUIRE(q && k && v && out && grad_out && lse && grad_q && grad_k && grad_v, EDF_ERR_INVALID_ARG,
              "null tensor pointer (the forward's lse is required)");
  const size_t need = edf_flash_attention_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
  const long rows = (long)BH * seq_len;
  float* Dd = (float*)workspace;
  const unsigned gd = (unsigned)((rows + 15) / 16);
  if (dtype == EDF_BF16)
    fa_bwd_dot_kernel<bf16><<<gd, 256, 0, s>>>((const bf16*)out, (const bf16*)grad_out, Dd, rows, head_dim);
  else
    fa_bwd_dot_kernel<float><<<gd, 256, 0, s>>>((const float*)out, (const float*)grad_out, Dd, rows, head_dim);
  int rc = check_launch("flash attention backward rowsum");
  if (rc) return rc;
  const float scale = 1.0f / sqrtf((float)head_dim);
  const float scale_log2 = scale * LOG2E;
  if (dtype == EDF_BF16 && (head_dim == 32 || head_dim == 64 || head_dim == 128)) {
    if (head_dim == 128)
      launch_mfma_bwd<128>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, causal, scale_log2,
                           scale);
    else if (head_dim == 64)
      launch_mfma_bwd<64>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, causal, scale_log2,
                          scale);
    else
      launch_mfma_bwd<32>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, causal, scale_log2,
                          scale);
  } else if (dtype == EDF_BF16) {
    launch_wave_bwd<bf16>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, head_dim, causal,
                          scale_log2, scale);
  } else {
    launch_wave_bwd<float>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, head_dim, causal,
                           scale_log2, scale);
  }
  return check_launch("flash attention backward");
}

}  // extern "C"
