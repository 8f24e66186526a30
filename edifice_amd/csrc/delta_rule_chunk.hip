// Chunked (WY / UT-transform) gated delta rule forward on bf16 MFMA, per-head beta.
//
// Same recurrence as the step path (delta_rule_seq.hip; reference
// lib/edifice/recurrent/gated_delta_net.ex:300-353 with beta broadcast along the value
// rows), rewritten per chunk of C = 64 steps with M = S^T [d_k x d_v], gamma_t the
// cumulative decay inside the chunk and M0 the state entering it:
//   A  = strict_lower(diag(beta) (Gamma o K K^T)),   Gamma_ts = gamma_t / gamma_s
//   T  = (I + A)^-1
//   R  = diag(beta) (V - diag(gamma) K M0)
//   E  = T R                         (the per-step delta-rule corrections)
//   O  = diag(gamma) Q M0 + (Q K^T o Gamma o tril) E
//   M1 = gamma_C M0 + K^T diag(gamma_C / gamma) E
// The R form folds the usual W = T diag(beta gamma) K into K M0, so the value-sliced
// phase never needs a d_k-wide W.
//
// Phase 1 (one workgroup per (b, h, chunk), fully parallel): K K^T and Q K^T on MFMA,
//   the decays, and T by blocked inversion (16x16 diagonal blocks by forward
//   substitution, off-diagonal blocks by small products); T, the masked Q K^T and the
//   log-decays go to the workspace (bf16 / f32).
// Phase 2 (one workgroup per (b, h, 32-wide d_v slice), sequential over chunks): the
//   f32 state slice lives in registers (one 32x32 MFMA tile per wave); K M0, Q M0, T R,
//   P E and K^T E-tilde are 32x32x16 bf16 MFMAs with operands staged in LDS.
#include "edf_abi.hpp"
#include "edf_common.hpp"
#include "edf_mfma.hpp"

namespace edf {
namespace {

constexpr int CH = 64;   // chunk length
constexpr int DK = 128;  // head dim handled by this path
constexpr int VS = 32;   // d_v slice per phase-2 workgroup

struct ChunkArgs {
  const bf16 *q, *k, *v, *beta, *alpha;
  bf16* out;
  bf16* tbuf;   // [BH][nch][CH][CH]  T
  bf16* pbuf;   // [BH][nch][CH][CH]  masked Q K^T o Gamma
  float* lbuf;  // [BH][nch][CH]      inclusive log-decay inside the chunk
  int H, T, nch;
};

EDF_DEVICE long row_off(const ChunkArgs& p, int b, int h, int t) { return (((long)b * p.T + t) * p.H + h) * DK; }

// ---------------------------------------------------------------------------
// phase 1
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dr_chunk_prep_kernel(const ChunkArgs p) {
  constexpr int KS = DK + 8;
  constexpr int AS = CH + 1;
  __shared__ __attribute__((aligned(16))) bf16 sK[CH * KS];
  __shared__ __attribute__((aligned(16))) bf16 sQ[CH * KS];
  __shared__ float sA[CH * AS];
  __shared__ float sT[CH * AS];
  __shared__ float sX[16 * 17];
  __shared__ float lg[CH], bt[CH];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int c = blockIdx.x;
  const long bh = blockIdx.y;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int t0 = c * CH;

  for (int e = tid; e < CH * DK / 8; e += 256) {
    const int row = e / (DK / 8), col = (e % (DK / 8)) * 8;
    const int t = t0 + row;
    const bool ok = t < p.T;
    *(bf16x8*)(sK + row * KS + col) = ok ? *(const bf16x8*)(p.k + row_off(p, b, h, t) + col) : bf16x8{};
    *(bf16x8*)(sQ + row * KS + col) = ok ? *(const bf16x8*)(p.q + row_off(p, b, h, t) + col) : bf16x8{};
  }
  if (w == 0) {
    const int t = t0 + l;
    const bool ok = t < p.T;
    const long hi = ((long)b * p.T + t) * p.H + h;
    float la = (ok && p.alpha != nullptr) ? __logf(to_f32(p.alpha[hi])) : 0.0f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(la, off);
      if (l >= off) la += y;
    }
    lg[l] = la;
    bt[l] = ok ? to_f32(p.beta[hi]) : 0.0f;
  }
  __syncthreads();

  // K K^T and Q K^T tiles (I, J) of 32x32; the upper tile (0, 1) is all zero after masking
  if (w != 1) {
    const int I = w >= 2 ? 1 : 0, J = (w == 3) ? 1 : 0;
    f32x16 G = zero16(), QK = zero16();
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk) {
      const bf16x8 bk = *(const bf16x8*)(sK + (J * 32 + li) * KS + kk * 16 + 8 * g);
      const bf16x8 ak = *(const bf16x8*)(sK + (I * 32 + li) * KS + kk * 16 + 8 * g);
      const bf16x8 aq = *(const bf16x8*)(sQ + (I * 32 + li) * KS + kk * 16 + 8 * g);
      G = mfma32(ak, bk, G);
      QK = mfma32(aq, bk, QK);
    }
    const int s = J * 32 + li;
    bf16* prow = p.pbuf + (((long)bh * p.nch + c) * CH) * CH;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = I * 32 + d_row(r, g);
      const float dec = __expf(lg[t] - lg[s]);
      sA[t * AS + s] = s < t ? bt[t] * dec * G[r] : 0.0f;
      prow[t * CH + s] = (bf16)(s <= t ? dec * QK[r] : 0.0f);
    }
  } else {
    // the zero upper tile of P and A
    const int s = 32 + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = d_row(r, g);
      sA[t * AS + s] = 0.0f;
      p.pbuf[(((long)bh * p.nch + c) * CH + t) * CH + s] = (bf16)0.0f;
    }
  }
  __syncthreads();

  // diagonal 16x16 blocks of T = (I + A)^-1: wave w, lane j < 16 -> column 16w + j
  if (l < 16) {
    const int o = 16 * w;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float v = (i == l) ? 1.0f : 0.0f;
#pragma unroll
      for (int s = 0; s < i; ++s) v = fmaf(-sA[(o + i) * AS + o + s], x[s], v);
      x[i] = v;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sT[(o + i) * AS + o + l] = x[i];
  }
  // zero the strict upper part of T
  for (int e = tid; e < CH * CH; e += 256) {
    const int i = e / CH, j = e % CH;
    if ((j >> 4) > (i >> 4)) sT[i * AS + j] = 0.0f;
  }
  __syncthreads();
  // off-diagonal blocks, by distance from the diagonal: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj
  const int ri = tid >> 4, cj = tid & 15;
  for (int dist = 1; dist < 4; ++dist) {
    for (int bj = 0; bj + dist < 4; ++bj) {
      const int bi = bj + dist;
      float xs = 0.0f;
      for (int kb = bj; kb < bi; ++kb)
#pragma unroll
        for (int m = 0; m < 16; ++m) xs = fmaf(sA[(16 * bi + ri) * AS + 16 * kb + m], sT[(16 * kb + m) * AS + 16 * bj + cj], xs);
      sX[ri * 17 + cj] = xs;
      __syncthreads();
      float y = 0.0f;
#pragma unroll
      for (int m = 0; m < 16; ++m) y = fmaf(sT[(16 * bi + ri) * AS + 16 * bi + m], sX[m * 17 + cj], y);
      sT[(16 * bi + ri) * AS + 16 * bj + cj] = -y;
      __syncthreads();
    }
  }
  bf16* tout = p.tbuf + (((long)bh * p.nch + c) * CH) * CH;
  for (int e = tid; e < CH * CH; e += 256) tout[e] = (bf16)sT[(e / CH) * AS + (e % CH)];
  if (tid < CH) p.lbuf[((long)bh * p.nch + c) * CH + tid] = lg[tid];
}

// ---------------------------------------------------------------------------
// phase 2
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dr_chunk_state_kernel(const ChunkArgs p) {
  constexpr int KS = DK + 8;  // [t][dk]
  constexpr int TS = CH + 8;  // [*][t]
  __shared__ __attribute__((aligned(16))) bf16 sK[CH * KS];
  __shared__ __attribute__((aligned(16))) bf16 sQ[CH * KS];
  __shared__ __attribute__((aligned(16))) bf16 sKt[DK * TS];
  __shared__ __attribute__((aligned(16))) bf16 sT[CH * TS];
  __shared__ __attribute__((aligned(16))) bf16 sP[CH * TS];
  __shared__ __attribute__((aligned(16))) bf16 sMt[VS * KS];  // M0^T [dv][dk]
  __shared__ __attribute__((aligned(16))) bf16 sRt[VS * TS];  // R^T  [dv][t]
  __shared__ __attribute__((aligned(16))) bf16 sEt[VS * TS];  // E^T
  __shared__ __attribute__((aligned(16))) bf16 sEs[VS * TS];  // (gamma_C / gamma) E, transposed
  __shared__ float sV[CH * (VS + 1)];
  __shared__ float lg[CH], bt[CH];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int nsl = DK / VS;
  const long bh = blockIdx.x / nsl;
  const int sl = blockIdx.x % nsl;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int v0 = sl * VS;

  f32x16 M = zero16();  // rows dk = 32 w + d_row(r, g), column dv = li (within the slice)
  for (int c = 0; c < p.nch; ++c) {
    const int t0 = c * CH;
    __syncthreads();
    for (int e = tid; e < CH * DK / 8; e += 256) {
      const int row = e / (DK / 8), col = (e % (DK / 8)) * 8;
      const int t = t0 + row;
      const bool ok = t < p.T;
      const bf16x8 kv = ok ? *(const bf16x8*)(p.k + row_off(p, b, h, t) + col) : bf16x8{};
      *(bf16x8*)(sK + row * KS + col) = kv;
      *(bf16x8*)(sQ + row * KS + col) = ok ? *(const bf16x8*)(p.q + row_off(p, b, h, t) + col) : bf16x8{};
#pragma unroll
      for (int e2 = 0; e2 < 8; ++e2) sKt[(col + e2) * TS + row] = kv[e2];
    }
    {
      const bf16* tsrc = p.tbuf + (((long)bh * p.nch + c) * CH) * CH;
      const bf16* psrc = p.pbuf + (((long)bh * p.nch + c) * CH) * CH;
      for (int e = tid; e < CH * CH / 8; e += 256) {
        const int row = e / (CH / 8), col = (e % (CH / 8)) * 8;
        *(bf16x8*)(sT + row * TS + col) = *(const bf16x8*)(tsrc + row * CH + col);
        *(bf16x8*)(sP + row * TS + col) = *(const bf16x8*)(psrc + row * CH + col);
      }
    }
    for (int e = tid; e < CH * VS; e += 256) {
      const int row = e / VS, col = e % VS;
      const int t = t0 + row;
      sV[row * (VS + 1) + col] = t < p.T ? to_f32(p.v[row_off(p, b, h, t) + v0 + col]) : 0.0f;
    }
    if (tid < CH) {
      const int t = t0 + tid;
      lg[tid] = p.lbuf[((long)bh * p.nch + c) * CH + tid];
      bt[tid] = t < p.T ? to_f32(p.beta[((long)b * p.T + t) * p.H + h]) : 0.0f;
    }
    // M0^T tile of this wave -> LDS (bf16)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      bf16x4 m4;
#pragma unroll
      for (int e = 0; e < 4; ++e) m4[e] = (bf16)M[rb * 4 + e];
      *(bf16x4*)(sMt + li * KS + 32 * w + 8 * rb + 4 * g) = m4;
    }
    __syncthreads();

    // K M0 (waves 0, 1) and Q M0 (waves 2, 3): rows t = 32 (w & 1) + d_row, column dv = li
    const int tb = 32 * (w & 1);
    const bf16* src = (w < 2) ? sK : sQ;
    f32x16 X = zero16();
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk) {
      const bf16x8 a = *(const bf16x8*)(src + (tb + li) * KS + kk * 16 + 8 * g);
      const bf16x8 bm = *(const bf16x8*)(sMt + li * KS + kk * 16 + 8 * g);
      X = mfma32(a, bm, X);
    }
    if (w < 2) {  // R = beta (V - gamma K M0), stored transposed
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 r4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = tb + 8 * rb + 4 * g + e;
          r4[e] = (bf16)(bt[t] * (sV[t * (VS + 1) + li] - __expf(lg[t]) * X[rb * 4 + e]));
        }
        *(bf16x4*)(sRt + li * TS + tb + 8 * rb + 4 * g) = r4;
      }
    }
    __syncthreads();
    if (w < 2) {  // E = T R (T lower triangular: s < 32 (w + 1))
      f32x16 E = zero16();
      const int send = 32 * (w + 1);
      for (int s0 = 0; s0 < send; s0 += 16) {
        const bf16x8 a = *(const bf16x8*)(sT + (tb + li) * TS + s0 + 8 * g);
        const bf16x8 br = *(const bf16x8*)(sRt + li * TS + s0 + 8 * g);
        E = mfma32(a, br, E);
      }
      const float lgC = lg[CH - 1];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 e4, s4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = tb + 8 * rb + 4 * g + e;
          e4[e] = (bf16)E[rb * 4 + e];
          s4[e] = (bf16)(__expf(lgC - lg[t]) * E[rb * 4 + e]);
        }
        *(bf16x4*)(sEt + li * TS + tb + 8 * rb + 4 * g) = e4;
        *(bf16x4*)(sEs + li * TS + tb + 8 * rb + 4 * g) = s4;
      }
    }
    __syncthreads();
    if (w >= 2) {  // O = gamma Q M0 + P E
      f32x16 O = zero16();
      const int send = 32 * ((w & 1) + 1);
      for (int s0 = 0; s0 < send; s0 += 16) {
        const bf16x8 a = *(const bf16x8*)(sP + (tb + li) * TS + s0 + 8 * g);
        const bf16x8 be = *(const bf16x8*)(sEt + li * TS + s0 + 8 * g);
        O = mfma32(a, be, O);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = tb + d_row(r, g);
        if (t0 + t < p.T) p.out[row_off(p, b, h, t0 + t) + v0 + li] = (bf16)fmaf(__expf(lg[t]), X[r], O[r]);
      }
    }
    // M1 = gamma_C M0 + K^T E-tilde  (this wave's 32 rows of d_k)
    const float gC = __expf(lg[CH - 1]);
#pragma unroll
    for (int r = 0; r < 16; ++r) M[r] *= gC;
#pragma unroll
    for (int s0 = 0; s0 < CH; s0 += 16) {
      const bf16x8 a = *(const bf16x8*)(sKt + (32 * w + li) * TS + s0 + 8 * g);
      const bf16x8 be = *(const bf16x8*)(sEs + li * TS + s0 + 8 * g);
      M = mfma32(a, be, M);
    }
  }
}

}  // namespace

bool dr_chunk_eligible(int seq, int d, int dtype, int beta_per_head) {
  return dtype == EDF_BF16 && beta_per_head && d == DK && seq >= CH;
}

size_t dr_chunk_workspace_bytes(int batch, int seq, int heads, int d) {
  const size_t nch = (seq + CH - 1) / CH;
  const size_t bh = (size_t)batch * heads;
  return bh * nch * (2 * CH * CH * sizeof(bf16) + CH * sizeof(float));
}

int dr_chunk_run(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
                 void* out, void* workspace, int batch, int seq, int heads, int d) {
  (void)d;
  ChunkArgs a{};
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.beta = (const bf16*)beta; a.alpha = (const bf16*)alpha; a.out = (bf16*)out;
  a.H = heads; a.T = seq; a.nch = (seq + CH - 1) / CH;
  const size_t bh = (size_t)batch * heads;
  char* ws = (char*)workspace;
  a.tbuf = (bf16*)ws;
  a.pbuf = (bf16*)(ws + bh * a.nch * CH * CH * sizeof(bf16));
  a.lbuf = (float*)(ws + 2 * bh * a.nch * CH * CH * sizeof(bf16));
  hipStream_t s = as_stream(stream);
  dr_chunk_prep_kernel<<<dim3(a.nch, (unsigned)bh), 256, 0, s>>>(a);
  int rc = check_launch("delta rule chunk prep");
  if (rc) return rc;
  dr_chunk_state_kernel<<<(unsigned)(bh * (DK / VS)), 256, 0, s>>>(a);
  return check_launch("delta rule chunk state");
}

}  // namespace edf
