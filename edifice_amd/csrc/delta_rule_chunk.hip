// Chunked (WY / UT-transform) gated delta rule on bf16 MFMA, per-head beta, head_dim 128
// (64 .. 128 in steps of 8, zero-padded to 128): forward and backward.
//
// Same recurrence as the step path (delta_rule_seq.hip; reference
// lib/edifice/recurrent/gated_delta_net.ex:300-353 with beta broadcast along the value
// rows).  With M = S^T [d_k x d_v], rows of Q, K, V the C = 64 steps of a chunk,
// gamma_t the cumulative decay inside the chunk (lg = log gamma) and h the state
// entering it:
//   A     = strict_lower(diag(beta) (Gamma o K K^T)),  Gamma_ts = gamma_t / gamma_s
//   T     = (I + A)^-1
//   W     = T diag(beta gamma) K,   U = T diag(beta) V
//   v_new = U - W h                               (the per-step delta-rule corrections)
//   O     = diag(gamma) Q h + P v_new,            P = Q K^T o Gamma o tril
//   h'    = gamma_C h + Kd^T v_new,               Kd = diag(gamma_C / gamma) K
//
// Forward:  prep (parallel over chunks: T, W, U, Kd^T)  ->  scan (sequential over
//   chunks, one workgroup per (b, h, 32-wide d_v slice): h and v_new per chunk)  ->
//   out (parallel over chunks: O).
// Backward: prep, scan (recompute h, v_new)  ->  dlocal (parallel: P^T dO and
//   Q^T diag(gamma) dO)  ->  reverse scan (dh per chunk, dv_new)  ->  grad (parallel:
//   dQ, dK, dV, dbeta, dalpha).  With dR = T^T dv_new:
//   dh_prev = gamma_C dh + Q^T diag(gamma) dO - W^T dv_new,  dv_new = P^T dO + Kd dh
//   dQ = diag(gamma) dO h^T + dS K
//   dK = diag(gamma_C/gamma) v_new dh^T - diag(beta gamma) dR h^T + dS^T Q + (dG + dG^T) K
//   dV = diag(beta) dR,  dA = -dR v_new^T,  dS = dP o Gamma o tril,  dP = dO v_new^T,
//   dG = diag(beta) dA o Gamma (strict lower),
//   dbeta_t = <dR_t, V_t - gamma_t (K h)_t> + sum_s dA_ts (Gamma o K K^T)_ts,
//   dlg collects every gamma above; dalpha_s = (sum_{t >= s} dlg_t) / alpha_s.
//
// Every product is a 32x32x16 bf16 MFMA with f32 accumulation.  Operands contract over
// their contiguous dimension; results are stored with rows contiguous (store_rows) or
// reused in registers through acc_kfrag, which is why the workspace keeps some tensors
// in both orientations.
#include "edf_abi.hpp"
#include "edf_common.hpp"
#include "edf_mfma.hpp"

namespace edf {
namespace {

constexpr int CH = 64;      // chunk length
constexpr int DK = 128;     // head dim handled by this path
constexpr int VS = 32;      // d_v slice per scan workgroup
constexpr int KS = DK + 8;  // LDS row stride (bf16) of [*][DK] tiles
constexpr int TS = CH + 8;  // LDS row stride (bf16) of [*][CH] tiles

struct CkArgs {
  const bf16 *q, *k, *v, *beta, *alpha, *dout;
  bf16* out;
  bf16 *dq, *dk, *dv, *dbeta, *dalpha;
  float* lg;  // [ci][CH]       inclusive log-decay inside the chunk (ci = bh * nch + c)
  bf16* W;    // [ci][CH][DK]   W = T diag(beta gamma) K
  bf16* Wt;   // [ci][DK][CH]   W^T
  bf16* Ut;   // [ci][DK][CH]   U^T
  bf16* Kdt;  // [ci][DK][CH]   Kd^T
  bf16* Tt;   // [ci][CH][CH]   T^T
  bf16* P;    // [ci][CH][CH]   P = Q K^T o Gamma o tril, [t][s] (forward with fused output)
  bf16* hN;   // [ci][DK][DK]   same, [d_k][d_v]
  bf16* vN;   // [ci][CH][DK]   v_new
  bf16* dvl;  // [ci][DK][CH]   (P^T dO)^T
  bf16* dhl;  // [ci][DK][DK]   (Q^T diag(gamma) dO)^T, [d_v][d_k]
  bf16* dmN;  // [ci][DK][DK]   dL/d(state leaving the chunk), [d_k][d_v]
  bf16* dvT;  // [ci][DK][CH]   (dL/dv_new)^T
  int H, T, nch;
  int D;  // head_dim of the [B,T,H,D] tensors, a multiple of 8 up to DK
};

// A head_dim D < DK is zero-padded to DK inside the kernels: the [B,T,H,D] tensors are read
// through ld_row8 (zeros at columns >= D) and written only at columns < D.  Zero columns of
// q, k and v stay zero through K K^T, T, W, U, the state and the outputs, so the first D
// columns are the D-dimensional recurrence itself (at the cost of DK-wide tiles).
EDF_DEVICE long row_off(const CkArgs& p, int b, int h, int t) { return (((long)b * p.T + t) * p.H + h) * p.D; }
EDF_DEVICE long head_off(const CkArgs& p, int b, int h, int t) { return ((long)b * p.T + t) * p.H + h; }

// 8 bf16 of row t, columns col .. col + 7 (zeros beyond the sequence or the head dim,
// col a multiple of 8); the load itself is always in bounds.
EDF_DEVICE bf16x8 ld_row8(const bf16* base, const CkArgs& p, int b, int h, int t, int col) {
  const bool ok = t < p.T && col < p.D;
  const bf16x8 v = *(const bf16x8*)(base + row_off(p, b, h, t < p.T ? t : p.T - 1) + (col < p.D ? col : 0));
  return ok ? v : bf16x8{};
}

// Transposed staging of a chunk of a [B,T,H,DK] tensor: dst[d * TS + t] = scale_t * src[t][d].
// Lanes run along t so that the 2-byte LDS writes of a wave fill consecutive words.
template <int NT>
EDF_DEVICE void stage_t(bf16* dst, const bf16* src, const CkArgs& p, int b, int h, int t0, const float* scale) {
  for (int e = threadIdx.x; e < CH * DK / 8; e += NT) {
    const int t = e & (CH - 1), cb = (e >> 6) * 8;
    const bf16x8 x = ld_row8(src, p, b, h, t0 + t, cb);
    const float sc = scale != nullptr ? scale[t] : 1.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[(cb + i) * TS + t] = (bf16)((float)x[i] * sc);
  }
}

// ---------------------------------------------------------------------------
// prep: decays, T = (I + A)^-1, W (and W^T), U^T, Kd^T (and T^T).
// LDS is reused across phases (A then K^T, T then V^T) so three workgroups share a CU.
// ---------------------------------------------------------------------------
// BWD: also store T^T and W^T (the backward's context); OUT_P: also store P for the
// scan's fused output.
template <bool BWD, bool OUT_P>
__global__ __launch_bounds__(256) void dr_ck_prep_kernel(const CkArgs p) {
  constexpr int AS = CH + 1;
  __shared__ __attribute__((aligned(16))) char u1[DK * TS * sizeof(bf16)];
  __shared__ __attribute__((aligned(16))) char u2[DK * TS * sizeof(bf16)];
  __shared__ __attribute__((aligned(16))) bf16 sTb[CH * TS];  // T
  __shared__ float lg[CH], bt[CH], kbs[CH], kds[CH];
  float* sA = (float*)u1;      // [CH][AS]   A, during the inversion
  float* sX = sA + CH * AS;    // [16][17]   substitution scratch
  bf16* sKb = (bf16*)u1;       // [DK][TS]   (diag(beta gamma) K)^T, afterwards
  float* sT = (float*)u2;      // [CH][AS]   T in f32, during the inversion
  bf16* sVb = (bf16*)u2;       // [DK][TS]   (diag(beta) V)^T, afterwards

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int c = blockIdx.x;
  const long bh = blockIdx.y;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int t0 = c * CH;
  const long ci = bh * p.nch + c;

  if (w == 0) {
    const int t = t0 + l;
    const bool ok = t < p.T;
    const long hi = head_off(p, b, h, ok ? t : p.T - 1);
    float la = (ok && p.alpha != nullptr) ? __logf(to_f32(p.alpha[hi])) : 0.0f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(la, off);
      if (l >= off) la += y;
    }
    const float lC = __shfl(la, 63);
    const float bv = ok ? to_f32(p.beta[hi]) : 0.0f;
    lg[l] = la;
    bt[l] = bv;
    kbs[l] = bv * __expf(la);
    kds[l] = __expf(lC - la);
  }
  __syncthreads();

  if constexpr (OUT_P) {
    // P tiles X[s][t] = K Q^T (rows s = 32 I, columns t = 32 J, s <= t), staged as [t][s]
    // in the T buffer (free until the inversion ends) and written as whole 128-byte rows
    const int I = w == 3 ? 1 : 0, J = w >= 2 ? 1 : 0;
    f32x16 X = zero16();
    if (w != 1) {
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk)
        X = mfma32(ld_row8(p.k, p, b, h, t0 + 32 * I + li, 16 * kk + 8 * g),
                   ld_row8(p.q, p, b, h, t0 + 32 * J + li, 16 * kk + 8 * g), X);
      const int t = 32 * J + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int sidx = 32 * I + d_row(r, g);
        X[r] = sidx <= t ? X[r] * __expf(lg[t] - lg[sidx]) : 0.0f;
      }
    }
    // w == 1 stores the zero tile s >= 32, t < 32
    store_rows(sTb + (32 * (w == 1 ? 0 : J)) * TS + 32 * (w == 1 ? 1 : I), TS, X, li, g);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i, row = e >> 3, ch = e & 7;  // 64 rows of 128 bytes
      *(bf16x8*)(p.P + ci * CH * CH + row * CH + 8 * ch) = *(const bf16x8*)(sTb + row * TS + 8 * ch);
    }
  }

  // A from the K K^T tiles (I, J), operands straight from global; the tile above the diagonal is zero
  if (w != 1) {
    const int I = w >= 2 ? 1 : 0, J = (w == 3) ? 1 : 0;
    f32x16 G = zero16();
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
      G = mfma32(ld_row8(p.k, p, b, h, t0 + 32 * I + li, 16 * kk + 8 * g),
                 ld_row8(p.k, p, b, h, t0 + 32 * J + li, 16 * kk + 8 * g), G);
    const int s = J * 32 + li;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = I * 32 + d_row(r, g);
      sA[t * AS + s] = s < t ? bt[t] * __expf(lg[t] - lg[s]) * G[r] : 0.0f;
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) sA[d_row(r, g) * AS + 32 + li] = 0.0f;
  }
  __syncthreads();

  // diagonal 16x16 blocks of T by forward substitution: wave w, lane j < 16 -> column 16w + j
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
  for (int e = tid; e < CH * CH; e += 256) {
    const int i = e / CH, j = e % CH;
    if ((j >> 4) > (i >> 4)) sT[i * AS + j] = 0.0f;
  }
  __syncthreads();
  // off-diagonal blocks by distance from the diagonal: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj
  {
    const int ri = tid >> 4, cj = tid & 15;
    for (int dist = 1; dist < 4; ++dist) {
      for (int bj = 0; bj + dist < 4; ++bj) {
        const int bi = bj + dist;
        float xs = 0.0f;
        for (int kb = bj; kb < bi; ++kb)
#pragma unroll
          for (int m = 0; m < 16; ++m)
            xs = fmaf(sA[(16 * bi + ri) * AS + 16 * kb + m], sT[(16 * kb + m) * AS + 16 * bj + cj], xs);
        sX[ri * 17 + cj] = xs;
        __syncthreads();
        float y = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) y = fmaf(sT[(16 * bi + ri) * AS + 16 * bi + m], sX[m * 17 + cj], y);
        sT[(16 * bi + ri) * AS + 16 * bj + cj] = -y;
        __syncthreads();
      }
    }
  }

  // T -> bf16 (and T^T to the workspace); then sA and sT are free
  for (int e = tid; e < CH * CH / 8; e += 256) {
    const int row = e >> 3, cb = (e & 7) * 8;
    bf16x8 tv;
#pragma unroll
    for (int i = 0; i < 8; ++i) tv[i] = (bf16)sT[row * AS + cb + i];
    *(bf16x8*)(sTb + row * TS + cb) = tv;
    if (BWD) {
      bf16x8 tt;
#pragma unroll
      for (int i = 0; i < 8; ++i) tt[i] = (bf16)sT[(cb + i) * AS + row];
      *(bf16x8*)(p.Tt + ci * CH * CH + row * CH + cb) = tt;
    }
  }
  if (tid < CH) p.lg[ci * CH + tid] = lg[tid];
  __syncthreads();
  stage_t<256>(sKb, p.k, p, b, h, t0, nullptr);
  stage_t<256>(sVb, p.v, p, b, h, t0, bt);
  __syncthreads();
  // K^T -> Kd^T (workspace) and (diag(beta gamma) K)^T (in place)
  for (int e = tid; e < DK * CH / 8; e += 256) {
    const int d = e >> 3, tb = (e & 7) * 8;
    const bf16x8 kv = *(const bf16x8*)(sKb + d * TS + tb);
    bf16x8 kb, kd;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float kf = (float)kv[i];
      kb[i] = (bf16)(kbs[tb + i] * kf);
      kd[i] = (bf16)(kds[tb + i] * kf);
    }
    *(bf16x8*)(sKb + d * TS + tb) = kb;
    *(bf16x8*)(p.Kdt + ci * DK * CH + d * CH + tb) = kd;
  }
  __syncthreads();

  // T is lower triangular, so row tile 0 only reaches s < 32 (k-steps 0, 1).
  // W^T tile: rows d_k = 32 w + .., columns t = 32 J + li  ->  W stored [t][d_k]
  // U tile:   rows t = 32 J + .., columns d_v = 32 w + li  ->  U^T stored [d_v][t]
  // W tile:   rows t = 32 J + .., columns d_k = 32 w + li  ->  W^T stored [d_k][t] (backward)
  auto product = [&](const bf16* A, const bf16* Bm, int J) {
    f32x16 X = zero16();
#pragma unroll
    for (int kk = 0; kk < 2 * (J + 1); ++kk)
      X = mfma32(*(const bf16x8*)(A + li * TS + 16 * kk + 8 * g), *(const bf16x8*)(Bm + li * TS + 16 * kk + 8 * g), X);
    return X;
  };
  f32x16 XW[2], XU[2];
#pragma unroll
  for (int J = 0; J < 2; ++J) {
    XW[J] = product(sKb + (32 * w) * TS, sTb + (32 * J) * TS, J);
    XU[J] = product(sTb + (32 * J) * TS, sVb + (32 * w) * TS, J);
  }
  // The results of the chunk are contiguous 16 KB blocks of the workspace: they are staged
  // in operand tiles that are no longer read and written as whole rows, 16 bytes per lane
  // (stores straight from the accumulator layout scatter each instruction over 32 rows).
  bf16* sW = (bf16*)u1;  // [t][d_k], row stride KS (over K^T once that is consumed)
  bf16* sU = (bf16*)u2;  // [d_v][t] or [d_k][t], row stride TS (over V^T)
  auto copy_w = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, row = e >> 4, ch = e & 15;  // 64 rows of 256 bytes
      *(bf16x8*)(p.W + ci * CH * DK + row * DK + 8 * ch) = *(const bf16x8*)(sW + row * KS + 8 * ch);
    }
  };
  auto copy_u = [&](bf16* dst) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, row = e >> 3, ch = e & 7;  // 128 rows of 128 bytes
      *(bf16x8*)(dst + ci * DK * CH + row * CH + 8 * ch) = *(const bf16x8*)(sU + row * TS + 8 * ch);
    }
  };
  __syncthreads();  // V^T consumed
#pragma unroll
  for (int J = 0; J < 2; ++J) store_rows(sU + (32 * w) * TS + 32 * J, TS, XU[J], li, g);
  if constexpr (!BWD) {
#pragma unroll
    for (int J = 0; J < 2; ++J) store_rows(sW + (32 * J) * KS + 32 * w, KS, XW[J], li, g);
    __syncthreads();
    copy_u(p.Ut);
    copy_w();
  } else {
    f32x16 XWt[2];
#pragma unroll
    for (int J = 0; J < 2; ++J) XWt[J] = product(sTb + (32 * J) * TS, sKb + (32 * w) * TS, J);
    __syncthreads();  // U^T staged, K^T consumed
    copy_u(p.Ut);
#pragma unroll
    for (int J = 0; J < 2; ++J) store_rows(sW + (32 * J) * KS + 32 * w, KS, XW[J], li, g);
    __syncthreads();  // W staged, U^T copied
    copy_w();
#pragma unroll
    for (int J = 0; J < 2; ++J) store_rows(sU + (32 * w) * TS + 32 * J, TS, XWt[J], li, g);
    __syncthreads();
    copy_u(p.Wt);
  }
}

// ---------------------------------------------------------------------------
// scan over chunks, one workgroup per (b, h, d_v slice); wave w owns state rows
// d_k = 32 w .. 32 w + 31 of the slice as one f32 accumulator tile.  Per chunk, waves 0
// and 1 compute the two 32-step tiles of v (reading A1 and the published state from
// LDS) and publish v; after a second barrier every wave updates its state rows with v
// read from LDS.  (Each wave computing all of v itself reads four times the LDS bytes.)
//   MODE 1 / 3 (forward states):  v = U - W h;          h = gamma_C h + Kd^T v
//   MODE 2 (reverse, gradients):   v = dvl + Kd dh;      dh = gamma_C dh + dhl - W^T v
// MODE 1 stores h as [d_k][d_v] and v (the backward's context); MODE 3 stores the same
// and also forms the output of the slice, O = diag(gamma) Q h + P v: waves 2 and 3 (idle
// while waves 0 and 1 form v) take one 32-step tile each, the Q h part before the v
// barrier and the P v part after it, and write their O rows themselves;
// MODE 2 stores dh (the gradient of the state leaving each chunk) as [d_k][d_v] and v^T.
// Every stored tile is first staged in LDS in its global layout and then written by all
// threads as contiguous 16-byte rows (the slice of one chunk is one 8 KB / 4 KB block, or
// 64-byte row segments): storing straight from the accumulator layout scatters each
// instruction over 32 rows, and those stores alone took half of the scan's time.  The v
// tile of a step is written out at the end of the step.
// ---------------------------------------------------------------------------
constexpr int NS = VS + 8;  // LDS row stride (bf16) of [*][VS] tiles

template <int MODE>
__global__ __launch_bounds__(256) void dr_ck_scan_kernel(const CkArgs p) {
  static_assert(MODE >= 1 && MODE <= 3, "scan mode");
  constexpr bool REV = MODE == 2;
  constexpr bool OUT = MODE == 3;
  constexpr bool FWD_CTX = MODE == 1 || MODE == 3;  // store h as [d_k][d_v] and v as [t][d_v]
  __shared__ __attribute__((aligned(16))) bf16 sA1[2][CH * KS];  // W, or Kd in the reverse pass: [t][d_k]
  __shared__ __attribute__((aligned(16))) bf16 sSt[2][VS * KS];  // state slice, [d_v][d_k]
  // the state slice as [d_k][d_v], v as [d_v][t] and (forward) as [t][d_v]
  __shared__ __attribute__((aligned(16))) bf16 sN[2][DK * NS];
  __shared__ __attribute__((aligned(16))) bf16 sV[2][VS * TS];
  __shared__ __attribute__((aligned(16))) bf16 sV2[FWD_CTX ? 2 : 1][FWD_CTX ? CH * NS : 8];
  // the output rows of waves 2 and 3 ([t][d_v], 32 rows each), written out by the wave
  __shared__ __attribute__((aligned(16))) bf16 sO[OUT ? 2 : 1][OUT ? 32 * NS : 8];

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, g = l >> 5, li = l & 31;
  constexpr int NSL = DK / VS;
  const int logical = remap_xcd(blockIdx.x, gridDim.x);  // the slices of one head share an XCD
  const long bh = logical / NSL;
  const int v0 = (logical % NSL) * VS;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  auto chunk_of_ = [&](int it) { return REV ? p.nch - 1 - it : it; };

  f32x16 S = zero16();  // rows d_k = 32 w + d_row(r, g), column d_v = v0 + li

  // output regions of this head (buffer resources: a dropped store needs no branch)
  const long hbytes = (long)p.nch * DK * DK * 2, vbytes = (long)p.nch * DK * CH * 2;
  const rsrc_t rH = make_rsrc((FWD_CTX ? p.hN : p.dmN) + bh * p.nch * DK * DK, (unsigned)hbytes);
  const rsrc_t rV = make_rsrc((FWD_CTX ? p.vN : p.dvT) + bh * p.nch * DK * CH, (unsigned)vbytes);
  auto st16 = [&](const rsrc_t& r, unsigned off, const bf16* src) {
    __builtin_amdgcn_raw_buffer_store_b128(*(const u32x4*)src, r, (int)off, 0, 0);
  };
  // the v tile of step it (chunk c)
  auto copy_v = [&](int it, int c) {
    if constexpr (FWD_CTX) {  // v as [t][d_v]: 64 rows of 64 bytes
      const int row = tid >> 2, ch = tid & 3;
      st16(rV, (unsigned)(((c * CH + row) * DK + v0 + 8 * ch) * 2), sV2[it & 1] + row * NS + 8 * ch);
    } else {  // v^T as [d_v][t]: 32 rows of 128 bytes
      const int row = tid >> 3, ch = tid & 7;
      st16(rV, (unsigned)(((c * DK + v0 + row) * CH + 8 * ch) * 2), sV[it & 1] + row * TS + 8 * ch);
    }
  };

  // operands of the next two chunks, loaded ahead into two register sets (the loop is
  // unrolled by two so that each set is addressed statically)
  struct Pre {
    bf16x8 a1[4];
    float l1[4];
    bf16x8 a2[4];
    bf16x4 x0[4];  // this wave's t tile (w & 1) of U^T or dvl
    bf16x4 y0[4];
    float lgC;
    // output (waves 2, 3): this lane's row t = 32 (w - 2) + li of Q and of P, log-decay at t
    bf16x8 qo[OUT ? DK / 16 : 1];
    bf16x8 po[OUT ? CH / 16 : 1];
    float lgo;
  };
  Pre pre0, pre1;
  // A1 rows of chunk c (consumed first, into LDS)
  auto fetch_a1 = [&](Pre& P, int c) {
    const long ci = bh * p.nch + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i;
      const int row = e >> 4, col = (e & 15) * 8;
      if (!REV) {
        P.a1[i] = *(const bf16x8*)(p.W + ci * CH * DK + row * DK + col);
      } else {
        P.a1[i] = ld_row8(p.k, p, b, h, c * CH + row, col);
        P.l1[i] = p.lg[ci * CH + row];
      }
    }
  };
  // the rest of chunk c (consumed at the end of its step)
  auto fetch_rest = [&](Pre& P, int c) {
    const long ci = bh * p.nch + c;
    const bf16* a2 = (REV ? p.Wt : p.Kdt) + ci * DK * CH + (32 * w + li) * CH + 8 * g;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) P.a2[kk] = *(const bf16x8*)(a2 + 16 * kk);
    const bf16* x0 = (REV ? p.dvl : p.Ut) + ci * DK * CH + (v0 + li) * CH + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) P.x0[q] = *(const bf16x4*)(x0 + 32 * (w & 1) + 8 * q);
    if (REV) {
      const bf16* y0 = p.dhl + ci * DK * DK + (v0 + li) * DK + 32 * w + 4 * g;
#pragma unroll
      for (int q = 0; q < 4; ++q) P.y0[q] = *(const bf16x4*)(y0 + 8 * q);
    }
    P.lgC = p.lg[ci * CH + CH - 1];
    if constexpr (OUT) {
      // every wave loads (waves 0, 1 a valid row they do not use): no wave-dependent branch
      // around the loads
      const int t = 32 * (w & 1) + li;
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk) P.qo[kk] = ld_row8(p.q, p, b, h, c * CH + t, 16 * kk + 8 * g);
#pragma unroll
      for (int kk = 0; kk < CH / 16; ++kk) P.po[kk] = *(const bf16x8*)(p.P + ci * CH * CH + t * CH + 16 * kk + 8 * g);
      P.lgo = p.lg[ci * CH + t];
    }
  };
  auto chunk_of = chunk_of_;
  fetch_a1(pre0, chunk_of(0));
  fetch_rest(pre0, chunk_of(0));
  if (p.nch > 1) {
    fetch_a1(pre1, chunk_of(1));
    fetch_rest(pre1, chunk_of(1));
  }

  // Each register set is consumed in place and refilled (for the chunk two steps
  // ahead) right after its last use, so no copy of an in-flight load is needed.
  auto body = [&](int it, Pre& P) {
    const int c = chunk_of(it);
    bf16* sa = sA1[it & 1];
    bf16* ss = sSt[it & 1];
    // publish the state entering (forward) / leaving (reverse) chunk c
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)S[4 * q + e];
      *(bf16x4*)(ss + li * KS + 32 * w + 8 * q + 4 * g) = v;
    }
    {
      bf16* sn = sN[it & 1];
#pragma unroll
      for (int r = 0; r < 16; ++r) sn[(32 * w + d_row(r, g)) * NS + li] = (bf16)S[r];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i;
      const int row = e >> 4, col = (e & 15) * 8;
      bf16x8 a = P.a1[i];
      if (REV) {
        const float sc = __expf(P.lgC - P.l1[i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = (bf16)((float)a[j] * sc);
      }
      *(bf16x8*)(sa + row * KS + col) = a;
    }
    const float gC = __expf(P.lgC);
    // Prefetches are unconditional (past the last chunk they reload it): a conditional
    // one makes the compiler copy the loaded registers at the loop latch behind a full
    // vmcnt(0) drain, which serialises every step on an HBM round trip.
    fetch_a1(P, chunk_of(min(it + 2, p.nch - 1)));
    __syncthreads();

    // v for the t tile w = 0, 1: X = A1 * state (rows t, column d_v), published as [d_v][t]
    bf16* sv = sV[it & 1];
    f32x16 XO = zero16();  // output tile of waves 2, 3: O^T rows d_v, column t = 32 (w - 2) + li
    if (OUT && w >= 2) {
      // diag(gamma) Q h while waves 0 and 1 form v
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk) XO = mfma32(*(const bf16x8*)(ss + li * KS + 16 * kk + 8 * g), P.qo[kk], XO);
      const float gt = __expf(P.lgo);
#pragma unroll
      for (int r = 0; r < 16; ++r) XO[r] *= gt;
    }
    if (w < 2) {
      f32x16 X = zero16();
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk) {
        const bf16x8 a = *(const bf16x8*)(sa + (32 * w + li) * KS + 16 * kk + 8 * g);
        const bf16x8 bb = *(const bf16x8*)(ss + li * KS + 16 * kk + 8 * g);
        X = mfma32(a, bb, X);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x0v = (float)P.x0[r >> 2][r & 3];
        X[r] = REV ? x0v + X[r] : x0v - X[r];
      }
      store_rows(sv + 32 * w, TS, X, li, g);
      if constexpr (FWD_CTX) {  // and as [t][d_v] for the store of v
        bf16* dst = sV2[it & 1] + (32 * w) * NS + li;
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[d_row(r, g) * NS] = (bf16)X[r];
      }
    }
    __syncthreads();
    // state update: Y = A2 * v, contracting over t
    f32x16 Y = zero16();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) Y = mfma32(P.a2[kk], *(const bf16x8*)(sv + li * TS + 16 * kk + 8 * g), Y);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      S[r] = REV ? fmaf(gC, S[r], (float)P.y0[r >> 2][r & 3] - Y[r]) : fmaf(gC, S[r], Y[r]);
    if (OUT && w >= 2) {
      // + P v (P[t][s] = 0 for s > t: the first tile needs s < 32 only), staged as [t][d_v]
      // rows of this wave and written out as 64-byte row segments
      const int J = w - 2;
#pragma unroll
      for (int kk = 0; kk < CH / 16; ++kk) {
        if (kk >= 2 * (J + 1)) continue;
        XO = mfma32(*(const bf16x8*)(sv + li * TS + 16 * kk + 8 * g), P.po[kk], XO);
      }
      bf16* so = sO[J];
#pragma unroll
      for (int r = 0; r < 16; ++r) so[li * NS + d_row(r, g)] = (bf16)XO[r];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = l + 64 * i, row = e >> 2, ch = e & 3;  // 32 rows x 64 bytes
        const int t = c * CH + 32 * J + row;
        if (t < p.T && v0 + 8 * ch < p.D)
          *(bf16x8*)(p.out + row_off(p, b, h, t) + v0 + 8 * ch) = *(const bf16x8*)(so + row * NS + 8 * ch);
      }
      __builtin_amdgcn_wave_barrier();
    }
    // coalesced stores, off the step's dependency chain: the state this step started
    // from and its v
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 256 * i;
      // [d_k][d_v]: 128 rows of 64 bytes
      const int row = e >> 2, ch = e & 3;
      st16(rH, (unsigned)(((c * DK + row) * DK + v0 + 8 * ch) * 2), sN[it & 1] + row * NS + 8 * ch);
    }
    copy_v(it, c);
    fetch_rest(P, chunk_of(min(it + 2, p.nch - 1)));
  };
  // both bodies of the unrolled pair run unconditionally inside the loop (an odd last
  // chunk is peeled), for the same reason as the unconditional prefetches
  int it = 0;
  for (; it + 1 < p.nch; it += 2) {
    body(it, pre0);
    body(it + 1, pre1);
  }
  if (it < p.nch) body(it, pre0);
}

// ---------------------------------------------------------------------------
// out: O = diag(gamma) Q h + P v_new per chunk, from the state h ([d_k][d_v]) and v_new
// ([t][d_v]) the forward scan stores for the backward.  Computed as O^T tiles (rows d_v,
// column t per lane) so that O rows store contiguously; the h^T and v_new^T A fragments
// come from transposed reads of the row-major tiles (ds_read_b64_tr_b16), which hand each
// lane rows 4g..4g+3 and 8+4g..8+4g+3 of a 16-row step, so the B fragments (Q rows, P rows)
// are read in that same order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dr_ck_out_kernel(const CkArgs p) {
  __shared__ __attribute__((aligned(16))) bf16 sH[DK * DK];  // h [d_k][d_v], swizzled rows
  __shared__ __attribute__((aligned(16))) bf16 sVn[CH * DK];  // v_new [t][d_v], swizzled rows
  __shared__ __attribute__((aligned(16))) bf16 sQ[CH * KS];   // Q [t][d_k]
  __shared__ __attribute__((aligned(16))) bf16 sP[CH * TS];   // P [t][s]
  __shared__ float lg[CH];
  bf16* sO = sH;  // O rows [t][d] (KS stride), over h once that is consumed

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int c = blockIdx.x;
  const long bh = blockIdx.y;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int t0 = c * CH;
  const long ci = bh * p.nch + c;
  if (tid < CH) lg[tid] = p.lg[ci * CH + tid];
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // h: 128 rows x 16 chunks
    const int e = tid + 256 * i, row = e >> 4, col = (e & 15) * 8;
    *(bf16x8*)(sH + lds_off<DK>(row, col)) = *(const bf16x8*)(p.hN + ci * DK * DK + row * DK + col);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // v_new and Q: 64 rows x 16 chunks
    const int e = tid + 256 * i, row = e >> 4, col = (e & 15) * 8;
    *(bf16x8*)(sVn + lds_off<DK>(row, col)) = *(const bf16x8*)(p.vN + ci * CH * DK + row * DK + col);
    *(bf16x8*)(sQ + row * KS + col) = ld_row8(p.q, p, b, h, t0 + row, col);
  }
  __syncthreads();

  // P^T tiles X[s][t] = K Q^T (rows s = 32 I, columns t = 32 J, s <= t) -> sP [t][s]
  {
    const int I = w == 3 ? 1 : 0, J = w >= 2 ? 1 : 0;
    f32x16 X = zero16();
    if (w != 1) {
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk)
        X = mfma32(ld_row8(p.k, p, b, h, t0 + 32 * I + li, 16 * kk + 8 * g),
                   *(const bf16x8*)(sQ + (32 * J + li) * KS + 16 * kk + 8 * g), X);
      const int t = 32 * J + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int sidx = 32 * I + d_row(r, g);
        X[r] = sidx <= t ? X[r] * __expf(lg[t] - lg[sidx]) : 0.0f;
      }
    }
    store_rows(sP + (32 * (w == 1 ? 0 : J)) * TS + 32 * (w == 1 ? 1 : I), TS, X, li, g);
  }
  __syncthreads();

  // transposed-read addressing: lane i of each 16-lane group reads row base + i / 4,
  // columns 32 w + d0 .. + 3 and receives column 32 w + li of rows 4 g .. 4 g + 3
  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
  const int kr = 4 * (grp >> 1) + (i16 >> 2);
  f32x16 XO[2];
#pragma unroll
  for (int J = 0; J < 2; ++J) {
    const int t = 32 * J + li;
    f32x16 X = zero16();
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk) {
      const int row = 16 * kk + kr, col = 32 * w + d0;
      const bf16x8 a = cat4(lds_read_tr16(sH + lds_off<DK>(row, col)), lds_read_tr16(sH + lds_off<DK>(row + 8, col)));
      const bf16* qr = sQ + t * KS + 16 * kk + 4 * g;
      X = mfma32(a, cat4(*(const bf16x4*)qr, *(const bf16x4*)(qr + 8)), X);
    }
    const float gm = __expf(lg[t]);
#pragma unroll
    for (int r = 0; r < 16; ++r) X[r] *= gm;
#pragma unroll
    for (int kc = 0; kc < CH / 16; ++kc) {
      if (kc >= 2 * (J + 1)) continue;  // P[t][s] = 0 for s > t
      const int row = 16 * kc + kr, col = 32 * w + d0;
      const bf16x8 a = cat4(lds_read_tr16(sVn + lds_off<DK>(row, col)), lds_read_tr16(sVn + lds_off<DK>(row + 8, col)));
      const bf16* pr = sP + t * TS + 16 * kc + 4 * g;
      X = mfma32(a, cat4(*(const bf16x4*)pr, *(const bf16x4*)(pr + 8)), X);
    }
    XO[J] = X;
  }
  __syncthreads();  // h consumed: O goes over it
#pragma unroll
  for (int J = 0; J < 2; ++J) store_rows(sO + (32 * J) * KS + 32 * w, KS, XO[J], li, g);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid + 256 * i, row = e >> 4, ch = e & 15;
    if (t0 + row < p.T && 8 * ch < p.D)
      *(bf16x8*)(p.out + row_off(p, b, h, t0 + row) + 8 * ch) = *(const bf16x8*)(sO + row * KS + 8 * ch);
  }
}

// ---------------------------------------------------------------------------
// dlocal: dvl = (P^T dO)^T and dhl = (Q^T diag(gamma) dO)^T per chunk
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dr_ck_dlocal_kernel(const CkArgs p) {
  __shared__ __attribute__((aligned(16))) bf16 sPt[CH * TS];  // P^T [s][t]
  __shared__ __attribute__((aligned(16))) bf16 sdOt[DK * TS];  // dO^T [d_v][t]
  __shared__ __attribute__((aligned(16))) bf16 sQg[DK * TS];  // (diag(gamma) Q)^T [d_k][t]
  __shared__ float lg[CH], gm[CH];
  // each wave's 32 output rows (d_v = 32 w + ..) staged whole: dvl rows of 64 t, then dhl
  // rows of 128 d_k, written as full rows (128 / 256 contiguous bytes)
  __shared__ __attribute__((aligned(16))) bf16 sRow[4][32 * KS];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int c = blockIdx.x;
  const long bh = blockIdx.y;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int t0 = c * CH;
  const long ci = bh * p.nch + c;
  if (tid < CH) {
    lg[tid] = p.lg[ci * CH + tid];
    gm[tid] = __expf(lg[tid]);
  }
  __syncthreads();
  stage_t<256>(sdOt, p.dout, p, b, h, t0, nullptr);
  stage_t<256>(sQg, p.q, p, b, h, t0, gm);

  // S = Q K^T tile (rows t = 32 I, columns s = 32 J) -> P^T [s][t]
  {
    const int I = w >> 1, J = w & 1;
    f32x16 X = zero16();
    if (w != 1) {
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk)
        X = mfma32(ld_row8(p.q, p, b, h, t0 + 32 * I + li, 16 * kk + 8 * g),
                   ld_row8(p.k, p, b, h, t0 + 32 * J + li, 16 * kk + 8 * g), X);
      const int s = 32 * J + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * I + d_row(r, g);
        X[r] = s <= t ? X[r] * __expf(lg[t] - lg[s]) : 0.0f;
      }
    }
    store_rows(sPt + (32 * J) * TS + 32 * I, TS, X, li, g);
  }
  __syncthreads();

  // P^T dO: rows s (tile I), columns d_v = 32 w + li; P^T[s][t] = 0 for t < s
#pragma unroll
  for (int I = 0; I < 2; ++I) {
    f32x16 X = zero16();
#pragma unroll
    for (int kk = 2 * I; kk < 4; ++kk)
      X = mfma32(*(const bf16x8*)(sPt + (32 * I + li) * TS + 16 * kk + 8 * g),
                 *(const bf16x8*)(sdOt + (32 * w + li) * TS + 16 * kk + 8 * g), X);
    store_rows(sRow[w] + 32 * I, TS, X, li, g);
  }
  // this wave's rows are private: no workgroup barrier, the rows are a contiguous block
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // 32 rows x 128 bytes
    const int e = l + 64 * i, row = e >> 3, ch = e & 7;
    *(bf16x8*)(p.dvl + ci * DK * CH + (long)(32 * w + row) * CH + 8 * ch) = *(const bf16x8*)(sRow[w] + row * TS + 8 * ch);
  }
  __builtin_amdgcn_wave_barrier();
  // Q^T diag(gamma) dO: rows d_k (tile I), columns d_v = 32 w + li
#pragma unroll
  for (int I = 0; I < 4; ++I) {
    f32x16 X = zero16();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      X = mfma32(*(const bf16x8*)(sQg + (32 * I + li) * TS + 16 * kk + 8 * g),
                 *(const bf16x8*)(sdOt + (32 * w + li) * TS + 16 * kk + 8 * g), X);
    store_rows(sRow[w] + 32 * I, KS, X, li, g);
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < 8; ++i) {  // 32 rows x 256 bytes
    const int e = l + 64 * i, row = e >> 4, ch = e & 15;
    *(bf16x8*)(p.dhl + ci * DK * DK + (long)(32 * w + row) * DK + 8 * ch) = *(const bf16x8*)(sRow[w] + row * KS + 8 * ch);
  }
}

// ---------------------------------------------------------------------------
// grad: dQ, dK, dV, dbeta, dalpha of one chunk.  Four waves, two workgroups per CU: the
// phases are short and separated by barriers and global loads, so while one workgroup
// waits the other computes (one 8-wave workgroup per CU spent most of its time waiting).
// Wave w owns the 32-wide d tile w of the [d][t] products (dR^T, dQ^T, dK^T) over both
// 32-step tiles, and one or two of the six 32x32 (t, s) tiles of S | dP and G | dA.
// LDS (67 KB): Q, K and dR as unpadded swizzled rows (lds_off); the transposed operands
// K^T, Q^T and dS^T come from transposed reads (lds_read_tr16) of those rows and of the
// dS tile; the row and column sums behind dlog-gamma and dbeta are formed in registers;
// dV, dQ and dK are staged over tiles that are dead by then.
// ---------------------------------------------------------------------------

// Sum over the 32 lanes of each half-wave of an accumulator tile's rows: afterwards lanes li
// and li ^ 16 hold the sum of register r = li & 15.  A reduce-scatter inside each 16-lane
// row (each exchange halves the number of registers still to be summed) on DPP lane
// exchanges - row_mirror (li ^ 15) and row_half_mirror (li ^ 7), valid pairings because
// they come before the exchanges of the lower bits, then quad permutes (li ^ 2, li ^ 1) -
// and one exchange between the two rows of the half-wave at the end.
template <int CTRL>
EDF_DEVICE float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
EDF_DEVICE float rowsum32(const f32x16& x, int li) {
  float a[8], b[4], c[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool hi = li & 8;
    a[j] = (hi ? x[j + 8] : x[j]) + dpp<0x140>(hi ? x[j] : x[j + 8]);  // row_mirror
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool hi = li & 4;
    b[j] = (hi ? a[j + 4] : a[j]) + dpp<0x141>(hi ? a[j] : a[j + 4]);  // row_half_mirror
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bool hi = li & 2;
    c[j] = (hi ? b[j + 2] : b[j]) + dpp<0x4E>(hi ? b[j] : b[j + 2]);  // quad_perm [2, 3, 0, 1]
  }
  const bool hi = li & 1;
  const float d = (hi ? c[1] : c[0]) + dpp<0xB1>(hi ? c[0] : c[1]);  // quad_perm [1, 0, 3, 2]
  return d + __shfl_xor(d, 16);
}

__global__ __launch_bounds__(256, 2) void dr_ck_grad_kernel(const CkArgs p) {
  __shared__ __attribute__((aligned(16))) bf16 sQ[CH * DK];         // Q [t][d_k]  (lds_off rows)
  __shared__ __attribute__((aligned(16))) bf16 sK[CH * DK];         // K [s][d_k]
  __shared__ __attribute__((aligned(16))) bf16 sdR[CH * DK];        // dR [s][d_v]
  __shared__ __attribute__((aligned(16))) bf16 sdSF[2 * CH * TS];   // dS [t][s], dF = dG + dG^T [t][s]
  __shared__ float lg[CH], bt[CH], dlg[CH], dbt[CH];
  bf16* sdS = sdSF;
  bf16* sdF = sdSF + CH * TS;
  bf16* sV = sdSF;  // dV [s][d_v] (lds_off rows), staged before dS and dF are formed

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int c = blockIdx.x;
  const long bh = blockIdx.y;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int t0 = c * CH;
  const long ci = bh * p.nch + c;
  const bf16* hN = p.hN + ci * DK * DK;
  const bf16* vN = p.vN + ci * CH * DK;
  // transposed reads: lane i of each 16-lane group reads row r0 + kr, columns c0 + d0 .. + 3
  // and receives column c0 + li of rows r0 + 4 g .. + 3 (twice, at r0 and r0 + 8, gives the
  // 16-step operand in the order 4 g .. 4 g + 3, 8 + 4 g .. 8 + 4 g + 3)
  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
  const int kr = 4 * (grp >> 1) + (i16 >> 2);
  auto tr_frag = [&](const bf16* tile, int r0, int c0) {
    return cat4(lds_read_tr16(tile + lds_off<DK>(r0 + kr, c0 + d0)), lds_read_tr16(tile + lds_off<DK>(r0 + kr + 8, c0 + d0)));
  };
  auto tr_frag_ts = [&](const bf16* tile, int r0, int c0) {  // [*][TS] tiles
    return cat4(lds_read_tr16(tile + (r0 + kr) * TS + c0 + d0), lds_read_tr16(tile + (r0 + kr + 8) * TS + c0 + d0));
  };
  // row t of a [*][TS] tile in the transposed-read order (B operand beside tr_frag)
  auto row_frag_ts = [&](const bf16* tile, int t, int kk) {
    const bf16* r = tile + t * TS + 16 * kk + 4 * g;
    return cat4(*(const bf16x4*)r, *(const bf16x4*)(r + 8));
  };
  // staged [t][d] tile -> whole 256-byte rows of a [B,T,H,D] tensor
  auto copy_rows = [&](bf16* dst, const bf16* src) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, row = e >> 4, ch = e & 15;
      if (t0 + row < p.T && 8 * ch < p.D)
        *(bf16x8*)(dst + row_off(p, b, h, t0 + row) + 8 * ch) = *(const bf16x8*)(src + lds_off<DK>(row, 8 * ch));
    }
  };
  // accumulator tile (rows d = 32 w + d_row(r, g), column j0 + li) -> row j0 + li of dst
  auto put_rows = [&](bf16* dst, int j0, const f32x16& x, float scale) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)(x[4 * q + e] * scale);
      *(bf16x4*)(dst + lds_off<DK>(j0 + li, 32 * w + 8 * q + 4 * g)) = v;
    }
  };

  // ---- stage Q and K; the dR^T operands and V rows load meanwhile ----
  const float lg0 = p.lg[ci * CH + (tid & (CH - 1))];
  const bf16 bt0 = p.beta[head_off(p, b, h, min(t0 + (tid & (CH - 1)), p.T - 1))];
  bf16x8 rq[4], rk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid + 256 * i, row = e >> 4, col = (e & 15) * 8;
    rq[i] = ld_row8(p.q, p, b, h, t0 + row, col);
    rk[i] = ld_row8(p.k, p, b, h, t0 + row, col);
  }
  bf16x8 aD[4], aT[2][4];  // rows d_v = 32 w + li of dv_new^T; rows s of T^T (kk < 2 j multiply zeros of T)
  bf16x4 vA[2][4];         // V rows s (dbeta), columns >= D masked at use
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) aD[kk] = *(const bf16x8*)(p.dvT + ci * DK * CH + (long)(32 * w + li) * CH + 16 * kk + 8 * g);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      aT[j][kk] = *(const bf16x8*)(p.Tt + ci * CH * CH + (long)(32 * j + li) * CH + 16 * kk + 8 * g);
    const long ro = row_off(p, b, h, min(t0 + 32 * j + li, p.T - 1));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = 32 * w + 8 * q + 4 * g;
      vA[j][q] = *(const bf16x4*)(p.v + ro + (col < p.D ? col : 0));
    }
  }
  if (tid < CH) {
    lg[tid] = lg0;
    bt[tid] = t0 + tid < p.T ? to_f32(bt0) : 0.0f;
    dlg[tid] = 0.0f;
    dbt[tid] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = tid + 256 * i, row = e >> 4, col = (e & 15) * 8;
    *(bf16x8*)(sQ + lds_off<DK>(row, col)) = rq[i];
    *(bf16x8*)(sK + lds_off<DK>(row, col)) = rk[i];
  }
  __syncthreads();
  const float lgC = lg[CH - 1];

  // ---- dR^T = dv_new^T T (rows d_v = 32 w + .., columns s): dR rows, dV = beta dR, dbeta ----
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int s = 32 * j + li;
    f32x16 X = zero16();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk < 2 * j) continue;
      X = mfma32(aD[kk], aT[j][kk], X);
    }
    put_rows(sdR, 32 * j, X, 1.0f);
    put_rows(sV, 32 * j, X, bt[s]);
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool okc = 32 * w + 8 * q + 4 * g < p.D;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fmaf(X[4 * q + e], okc ? (float)vA[j][q][e] : 0.0f, acc);
    }
    acc += __shfl_xor(acc, 32);
    if (g == 0) atomicAdd(&dbt[s], t0 + s < p.T ? acc : 0.0f);
  }
  __syncthreads();  // dR rows and the dV tile complete
  copy_rows(p.dv, sV);

  // ---- the six (t, s) tiles: items 0-2 are S | dP, items 3-5 G | dA on tiles
  // (0, 0), (1, 0), (1, 1); wave w takes items w and w + 4 ----
  const int nit = w < 2 ? 2 : 1;
  f32x16 SG[2], DD[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if (u >= nit) break;
    const int it = w + 4 * u, kind = it >= 3, tile = it % 3;
    const int I = tile >= 1, J = tile == 2;
    f32x16 A = zero16(), D = zero16();
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk) {
      const bf16x8 vb = *(const bf16x8*)(vN + (long)(32 * J + li) * DK + 16 * kk + 8 * g);
      const bf16x8 da = kind ? *(const bf16x8*)(sdR + lds_off<DK>(32 * I + li, 16 * kk + 8 * g))
                             : ld_row8(p.dout, p, b, h, t0 + 32 * I + li, 16 * kk + 8 * g);
      D = mfma32(da, vb, D);
      A = mfma32(*(const bf16x8*)((kind ? sK : sQ) + lds_off<DK>(32 * I + li, 16 * kk + 8 * g)),
                 *(const bf16x8*)(sK + lds_off<DK>(32 * J + li, 16 * kk + 8 * g)), A);
    }
    SG[u] = A;
    DD[u] = D;
  }
  __syncthreads();  // dV copied out: dS and dF go over it
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    if (u >= nit) break;
    const int it = w + 4 * u, kind = it >= 3, tile = it % 3;
    const int I = tile >= 1, J = tile == 2;
    const int s = 32 * J + li;
    const f32x16& S = SG[u];
    const f32x16& D = DD[u];
    f32x16 z, sb;
    if (!kind) {  // dS = dP o Gamma o tril;  z = dP o S o Gamma (dlog-gamma)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * I + d_row(r, g);
        const float gam = __expf(lg[t] - lg[s]);
        const bool m = s <= t;
        sdS[t * TS + s] = (bf16)(m ? D[r] * gam : 0.0f);
        z[r] = m ? D[r] * S[r] * gam : 0.0f;
      }
    } else {  // dA = -dR v_new^T;  dG = beta dA o Gamma (strict lower), dF = dG + dG^T
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = 32 * I + d_row(r, g);
        const float gam = __expf(lg[t] - lg[s]);
        const bool m = s < t;
        const float GG = m ? gam * S[r] : 0.0f;
        const float dAv = -D[r];
        z[r] = dAv * bt[t] * GG;
        sb[r] = dAv * GG;
        const float dG = m ? bt[t] * dAv * gam : 0.0f;
        if (m) {
          sdF[t * TS + s] = (bf16)dG;
          sdF[s * TS + t] = (bf16)dG;
        } else if (s == t) {
          sdF[t * TS + t] = (bf16)0.0f;
        }
      }
    }
    // dlog-gamma_t += sum_s z[t][s] - sum_s z[s][t];  dbeta_t += sum_s (dA o Gamma o G)[t][s]
    float cs = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) cs += z[r];
    cs += __shfl_xor(cs, 32);
    if (g == 0) atomicAdd(&dlg[s], -cs);
    const int tr = 32 * I + d_row(li & 15, g);
    const float rs = rowsum32(z, li);
    if (li < 16) atomicAdd(&dlg[tr], rs);
    if (kind) {
      const float rb = rowsum32(sb, li);
      if (li < 16) atomicAdd(&dbt[tr], rb);
    }
  }
  // dh rows d_k = 32 w + li
  bf16x8 fm[DK / 16];
#pragma unroll
  for (int kk = 0; kk < DK / 16; ++kk)
    fm[kk] = *(const bf16x8*)(p.dmN + ci * DK * DK + (long)(32 * w + li) * DK + 16 * kk + 8 * g);
  __syncthreads();  // dS, dF and the sums complete

  // ---- dQ^T and dK^T: rows d_k = 32 w + .., columns t = 32 j + li, in three passes so that
  // few operands are live at once ----
  // (1) X1 = dh v_new^T
  f32x16 X1[2], X2[2], XQ[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    X1[j] = zero16();
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
      X1[j] = mfma32(fm[kk], *(const bf16x8*)(vN + (long)(32 * j + li) * DK + 16 * kk + 8 * g), X1[j]);
  }
  // (2) h dO^T and h dR^T (h rows d_k = 32 w + li); <dh, h> over this wave's rows (the four
  // waves cover the matrix once)
  float hdh = 0.0f;
  {
    bf16x8 hf[DK / 16];
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk) hf[kk] = *(const bf16x8*)(hN + (long)(32 * w + li) * DK + 16 * kk + 8 * g);
#pragma unroll
    for (int kk = 0; kk < DK / 16; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) hdh = fmaf((float)fm[kk][e], (float)hf[kk][e], hdh);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = 32 * j + li;
      XQ[j] = zero16();
      X2[j] = zero16();
#pragma unroll
      for (int kk = 0; kk < DK / 16; ++kk) {
        XQ[j] = mfma32(hf[kk], ld_row8(p.dout, p, b, h, t0 + t, 16 * kk + 8 * g), XQ[j]);
        X2[j] = mfma32(hf[kk], *(const bf16x8*)(sdR + lds_off<DK>(t, 16 * kk + 8 * g)), X2[j]);
      }
    }
  }
  // (3) dQ^T = gamma (h dO^T) + K^T dS^T;
  //     dK^T = (gamma_C / gamma) dh v_new^T - (beta gamma) h dR^T + Q^T dS + K^T dF
  float dlgC = 0.0f;
  f32x16 XK[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = 32 * j + li;
    f32x16 X = XQ[j];
    const float gmt = __expf(lg[t]);
    float qx = 0.0f, k1 = 0.0f, k2 = 0.0f;
    bf16x4 qv[4], kv[4];  // Q[t][d], K[t][d] at this lane's rows d = 32 w + 8 q + 4 g + e
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      qv[q] = *(const bf16x4*)(sQ + lds_off<DK>(t, 32 * w + 8 * q + 4 * g));
      kv[q] = *(const bf16x4*)(sK + lds_off<DK>(t, 32 * w + 8 * q + 4 * g));
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      qx = fmaf((float)qv[r >> 2][r & 3], X[r], qx);
      X[r] *= gmt;
    }
    qx += __shfl_xor(qx, 32);
    if (g == 0) atomicAdd(&dlg[t], gmt * qx);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk >= 2 * (j + 1)) continue;  // dS[t][s] = 0 for s > t
      X = mfma32(tr_frag(sK, 16 * kk, 32 * w), row_frag_ts(sdS, t, kk), X);
    }
    XQ[j] = X;

    f32x16 X3 = zero16();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk < 2 * j) continue;  // dS[t'][s] = 0 for t' < s
      X3 = mfma32(tr_frag(sQ, 16 * kk, 32 * w), tr_frag_ts(sdS, 16 * kk, 32 * j), X3);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) X3 = mfma32(tr_frag(sK, 16 * kk, 32 * w), row_frag_ts(sdF, t, kk), X3);
    const float sc1 = __expf(lgC - lg[t]);
    const float sc2 = bt[t] * gmt;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float kvr = (float)kv[r >> 2][r & 3];
      k1 = fmaf(kvr, X1[j][r], k1);
      k2 = fmaf(kvr, X2[j][r], k2);
      X3[r] += sc1 * X1[j][r] - sc2 * X2[j][r];
    }
    k1 += __shfl_xor(k1, 32);
    k2 += __shfl_xor(k2, 32);
    if (g == 0) {
      atomicAdd(&dlg[t], -sc1 * k1 - sc2 * k2);
      atomicAdd(&dbt[t], -gmt * k2);
      dlgC += sc1 * k1;
    }
    XK[j] = X3;
  }
  {  // gamma_C <dh, h> and the Kd terms enter the decay of the last step
    float acc = hdh * __expf(lgC) + dlgC;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (l == 0) atomicAdd(&dlg[CH - 1], acc);
  }
  __syncthreads();  // every read of sQ and sK done: dQ and dK go over them
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    put_rows(sQ, 32 * j, XQ[j], 1.0f);
    put_rows(sK, 32 * j, XK[j], 1.0f);
  }
  __syncthreads();
  copy_rows(p.dq, sQ);
  copy_rows(p.dk, sK);

  if (w == 0) {
    // dlog(alpha_s) = sum_{t >= s} dlg_t
    float x = dlg[l];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_down(x, off);
      if (l + off < 64) x += y;
    }
    const int t = t0 + l;
    if (t < p.T) {
      const long hi = head_off(p, b, h, t);
      p.dbeta[hi] = (bf16)dbt[l];
      if (p.dalpha != nullptr) p.dalpha[hi] = (bf16)(x / to_f32(p.alpha[hi]));
    }
  }
}

__global__ void dr_ck_debug_kfrag_kernel(const float* x, bf16* out) {
  const int l = threadIdx.x, g = l >> 5, li = l & 31;
  f32x16 t0, t1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    t0[r] = x[d_row(r, g) * 32 + li];
    t1[r] = x[(32 + d_row(r, g)) * 32 + li];
  }
  *(bf16x8*)(out + (l * 4 + 0) * 8) = acc_kfrag(t0, 0);
  *(bf16x8*)(out + (l * 4 + 1) * 8) = acc_kfrag(t0, 1);
  *(bf16x8*)(out + (l * 4 + 2) * 8) = acc_kfrag(t1, 0);
  *(bf16x8*)(out + (l * 4 + 3) * 8) = acc_kfrag(t1, 1);
}

struct Layout {
  size_t lg, W, Wt, Ut, Kdt, Tt, P, hN, vN, dvl, dhl, dmN, dvT, total;
};

inline size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace regions.  The forward's (FWD) hold, on return, the per-chunk context the
// backward reads (lg, W, W^T, U^T, Kd^T, T^T, h, v_new; P only for the fused output); the
// backward's own (BWD) hold its reverse-pass tiles.  The recomputing backward takes both in
// one workspace (ALL).
enum LayoutKind { FWD, BWD, ALL };

Layout layout(int batch, int seq, int heads, LayoutKind kind) {
  const size_t nci = (size_t)batch * heads * ((seq + CH - 1) / CH);
  const size_t tile_ck = nci * CH * DK * sizeof(bf16), tile_kk = nci * DK * DK * sizeof(bf16);
  const bool ctx = kind != BWD, rev = kind != FWD;
  Layout L{};
  size_t off = 0;
  auto take = [&](size_t& slot, size_t bytes, bool use) {
    slot = use ? off : 0;
    if (use) off += a256(bytes);
  };
  take(L.lg, nci * CH * sizeof(float), ctx);
  take(L.W, tile_ck, ctx);
  take(L.Wt, tile_ck, ctx);
  take(L.Ut, tile_ck, ctx);
  take(L.Kdt, tile_ck, ctx);
  take(L.Tt, nci * CH * CH * sizeof(bf16), ctx);
  take(L.P, nci * CH * CH * sizeof(bf16), false);
  take(L.hN, tile_kk, ctx);
  take(L.vN, tile_ck, ctx);
  take(L.dvl, tile_ck, rev);
  take(L.dhl, tile_kk, rev);
  take(L.dmN, tile_kk, rev);
  take(L.dvT, tile_ck, rev);
  L.total = off;
  return L;
}

// pointers into the context workspace (forward regions) and the reverse-pass workspace
CkArgs make_args(const Layout& Lc, void* ctx_ws, const Layout& Lr, void* rev_ws, int seq, int heads, int d) {
  CkArgs a{};
  char* wc = (char*)ctx_ws;
  char* wr = (char*)rev_ws;
  a.lg = (float*)(wc + Lc.lg);
  a.W = (bf16*)(wc + Lc.W);
  a.Wt = (bf16*)(wc + Lc.Wt);
  a.Ut = (bf16*)(wc + Lc.Ut);
  a.Kdt = (bf16*)(wc + Lc.Kdt);
  a.Tt = (bf16*)(wc + Lc.Tt);
  a.P = Lc.P ? (bf16*)(wc + Lc.P) : nullptr;
  a.hN = (bf16*)(wc + Lc.hN);
  a.vN = (bf16*)(wc + Lc.vN);
  if (rev_ws != nullptr) {
    a.dvl = (bf16*)(wr + Lr.dvl);
    a.dhl = (bf16*)(wr + Lr.dhl);
    a.dmN = (bf16*)(wr + Lr.dmN);
    a.dvT = (bf16*)(wr + Lr.dvT);
  }
  a.H = heads;
  a.T = seq;
  a.nch = (seq + CH - 1) / CH;
  a.D = d;
  return a;
}

}  // namespace

bool dr_chunk_eligible(int seq, int d, int dtype, int beta_per_head) {
  // seq bound: the scan addresses one head's per-chunk tiles with 32-bit byte offsets.
  // head_dim 64 .. 128 (a multiple of 8) runs zero-padded to 128; below 64 the padding
  // would cost more than the exact per-step kernels.
  return dtype == EDF_BF16 && beta_per_head && d >= 64 && d <= DK && d % 8 == 0 && seq >= CH &&
         seq <= (1 << 21);
}

size_t dr_chunk_workspace_bytes(int batch, int seq, int heads, int d) {
  (void)d;
  return layout(batch, seq, heads, FWD).total;
}

size_t dr_chunk_backward_workspace_bytes(int batch, int seq, int heads, int d) {
  (void)d;
  return layout(batch, seq, heads, ALL).total;
}

size_t dr_chunk_saved_backward_workspace_bytes(int batch, int seq, int heads, int d) {
  (void)d;
  return layout(batch, seq, heads, BWD).total;
}

// forward: prep (T, W, U, Kd and the backward's context), the scan (states, v_new), the
// output; the workspace keeps the context for dr_chunk_saved_backward_run
int dr_chunk_run(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
                 void* out, void* workspace, int batch, int seq, int heads, int d) {
  const Layout L = layout(batch, seq, heads, FWD);
  CkArgs a = make_args(L, workspace, L, nullptr, seq, heads, d);
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.beta = (const bf16*)beta; a.alpha = (const bf16*)alpha; a.out = (bf16*)out;
  const unsigned bh = (unsigned)batch * heads;
  hipStream_t s = as_stream(stream);
  dr_ck_prep_kernel<true, false><<<dim3(a.nch, bh), 256, 0, s>>>(a);
  int rc = check_launch("delta rule chunk prep");
  if (rc) return rc;
  dr_ck_scan_kernel<1><<<bh * (DK / VS), 256, 0, s>>>(a);
  rc = check_launch("delta rule chunk scan");
  if (rc) return rc;
  dr_ck_out_kernel<<<dim3(a.nch, bh), 256, 0, s>>>(a);
  return check_launch("delta rule chunk output");
}

// the reverse pass from a complete context: dlocal, reverse scan, gradients
int reverse_pass(hipStream_t s, CkArgs& a, unsigned bh, const void* grad_out, void* dq, void* dk, void* dv,
                 void* dbeta, void* dalpha) {
  a.dout = (const bf16*)grad_out;
  a.dq = (bf16*)dq; a.dk = (bf16*)dk; a.dv = (bf16*)dv; a.dbeta = (bf16*)dbeta; a.dalpha = (bf16*)dalpha;
  dr_ck_dlocal_kernel<<<dim3(a.nch, bh), 256, 0, s>>>(a);
  int rc = check_launch("delta rule chunk dlocal");
  if (rc) return rc;
  dr_ck_scan_kernel<2><<<bh * (DK / VS), 256, 0, s>>>(a);
  rc = check_launch("delta rule chunk reverse scan");
  if (rc) return rc;
  dr_ck_grad_kernel<<<dim3(a.nch, bh), 256, 0, s>>>(a);
  return check_launch("delta rule chunk grad");
}

// backward that recomputes the context (prep, forward scan) into its own workspace
int dr_chunk_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                          const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                          void* dalpha, void* workspace, int batch, int seq, int heads, int d) {
  const Layout L = layout(batch, seq, heads, ALL);
  CkArgs a = make_args(L, workspace, L, workspace, seq, heads, d);
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.beta = (const bf16*)beta; a.alpha = (const bf16*)alpha;
  const unsigned bh = (unsigned)batch * heads;
  hipStream_t s = as_stream(stream);
  dr_ck_prep_kernel<true, false><<<dim3(a.nch, bh), 256, 0, s>>>(a);
  int rc = check_launch("delta rule chunk prep");
  if (rc) return rc;
  dr_ck_scan_kernel<1><<<bh * (DK / VS), 256, 0, s>>>(a);
  rc = check_launch("delta rule chunk scan");
  if (rc) return rc;
  return reverse_pass(s, a, bh, grad_out, dq, dk, dv, dbeta, dalpha);
}

// backward from the context a forward call left in its workspace (same inputs)
int dr_chunk_saved_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                                void* dalpha, const void* fwd_workspace, void* workspace, int batch, int seq,
                                int heads, int d) {
  (void)d;
  const Layout Lc = layout(batch, seq, heads, FWD), Lr = layout(batch, seq, heads, BWD);
  CkArgs a = make_args(Lc, const_cast<void*>(fwd_workspace), Lr, workspace, seq, heads, d);
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.beta = (const bf16*)beta; a.alpha = (const bf16*)alpha;
  return reverse_pass(as_stream(stream), a, (unsigned)batch * heads, grad_out, dq, dk, dv, dbeta, dalpha);
}

}  // namespace edf

extern "C" int edf_debug_acc_kfrag_bf16(void* stream, const float* x, void* out) {
  using namespace edf;
  clear_error();
  EDF_REQUIRE(x != nullptr && out != nullptr, EDF_ERR_INVALID_ARG, "null pointer");
  dr_ck_debug_kfrag_kernel<<<1, 64, 0, as_stream(stream)>>>(x, (bf16*)out);
  return check_launch("acc_kfrag probe");
}
