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
constexpr int VS = 32;      // d_v slice per scan wave
constexpr int KS = DK + 8;  // LDS row stride (bf16) of [*][DK] tiles
constexpr int TS = CH + 8;  // LDS row stride (bf16) of [*][CH] tiles

// W, W^T and Kd^T are stored for the scan with the contraction axis permuted within every
// group of 16: stored position s holds logical position kperm(s) (elements 4..7 and 8..11
// swapped), the order in which an MFMA accumulator tile holds the rows it hands on as an
// operand (see the scan).
EDF_DEVICE constexpr int kperm(int s) { return (s & ~12) | ((s & 4) << 1) | ((s & 8) >> 1); }

struct CkArgs {
  const bf16 *q, *k, *v, *beta, *alpha, *dout;
  bf16* out;
  bf16 *dq, *dk, *dv, *dbeta, *dalpha;
  float* lg;  // [ci][CH]       inclusive log-decay inside the chunk (ci = bh * nch + c)
  bf16* W;    // [ci][CH][DK]   -W, W = T diag(beta gamma) K (d_k in kperm order)
  bf16* Wt;   // [ci][DK][CH]   -W^T                         (t in kperm order)
  bf16* Ut;   // [ci][DK][CH]   U^T
  bf16* Kdt;  // [ci][DK][CH]   Kd^T                         (t in kperm order)
  bf16* Kd;   // [ci][CH][DK]   Kd                           (d_k in kperm order)
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

  // Kd = diag(gamma_C / gamma) K as rows [t][d_k] in the scan's kperm order along d_k (the
  // reverse scan's operand): stored chunk ch of row t holds logical columns 16 (ch / 2) +
  // 4 (ch % 2) + 0..3 and 8 more on
  if constexpr (BWD) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // 64 rows x 8 groups of 16 columns
      const int e = tid + 256 * i, row = e >> 3, q = e & 7;
      const bf16x8 lo = ld_row8(p.k, p, b, h, t0 + row, 16 * q), hi = ld_row8(p.k, p, b, h, t0 + row, 16 * q + 8);
      const float sc = kds[row];
      bf16x8 k0, k1;  // stored chunks 2 q (columns 0..3, 8..11 of the group) and 2 q + 1 (4..7, 12..15)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        k0[j] = (bf16)(sc * (float)lo[j]);
        k0[4 + j] = (bf16)(sc * (float)hi[j]);
        k1[j] = (bf16)(sc * (float)lo[4 + j]);
        k1[4 + j] = (bf16)(sc * (float)hi[4 + j]);
      }
      bf16* dst = p.Kd + ci * CH * DK + row * DK + 16 * q;
      *(bf16x8*)dst = k0;
      *(bf16x8*)(dst + 8) = k1;
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
  // K^T -> Kd^T (workspace, t in the scan's kperm order: logical t .. t + 3 of this chunk at
  // stored kperm(t % 16), t + 4 .. t + 7 at kperm(t % 16 + 4)) and (diag(beta gamma) K)^T
  // (in place)
  for (int e = tid; e < DK * CH / 8; e += 256) {
    const int d = e >> 3, tb = (e & 7) * 8;
    const bf16x8 kv = *(const bf16x8*)(sKb + d * TS + tb);
    bf16x8 kb;
    bf16x4 kd0, kd1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float kf = (float)kv[i];
      kb[i] = (bf16)(kbs[tb + i] * kf);
      if (i < 4) kd0[i] = (bf16)(kds[tb + i] * kf);
      else kd1[i - 4] = (bf16)(kds[tb + i] * kf);
    }
    *(bf16x8*)(sKb + d * TS + tb) = kb;
    bf16* kdr = p.Kdt + ci * DK * CH + d * CH + (tb & ~15);
    *(bf16x4*)(kdr + kperm(tb & 15)) = kd0;
    *(bf16x4*)(kdr + kperm((tb & 15) + 4)) = kd1;
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
  // stored 16-byte chunk ch of a kperm-ordered row: logical elements 16 (ch / 2) + 4 (ch % 2)
  // + 0..3 and 8 more on
  auto perm_chunk = [&](const bf16* row, int ch) {
    const bf16* src = row + 16 * (ch >> 1) + 4 * (ch & 1);
    return cat4(*(const bf16x4*)src, *(const bf16x4*)(src + 8));
  };
  auto copy_w = [&]() {  // -W in the scan's kperm order along d_k
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, row = e >> 4, ch = e & 15;  // 64 rows of 256 bytes
      *(bf16x8*)(p.W + ci * CH * DK + row * DK + 8 * ch) = -perm_chunk(sW + row * KS, ch);
    }
  };
  // perm: -W^T, in the scan's kperm order along t; else U^T as staged
  auto copy_u = [&](bf16* dst, bool perm) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + 256 * i, row = e >> 3, ch = e & 7;  // 128 rows of 128 bytes
      *(bf16x8*)(dst + ci * DK * CH + row * CH + 8 * ch) =
          perm ? -perm_chunk(sU + row * TS, ch) : *(const bf16x8*)(sU + row * TS + 8 * ch);
    }
  };
  __syncthreads();  // V^T consumed
#pragma unroll
  for (int J = 0; J < 2; ++J) store_rows(sU + (32 * w) * TS + 32 * J, TS, XU[J], li, g);
  if constexpr (!BWD) {
#pragma unroll
    for (int J = 0; J < 2; ++J) store_rows(sW + (32 * J) * KS + 32 * w, KS, XW[J], li, g);
    __syncthreads();
    copy_u(p.Ut, false);
    copy_w();
  } else {
    f32x16 XWt[2];
#pragma unroll
    for (int J = 0; J < 2; ++J) XWt[J] = product(sTb + (32 * J) * TS, sKb + (32 * w) * TS, J);
    __syncthreads();  // U^T staged, K^T consumed
    copy_u(p.Ut, false);
#pragma unroll
    for (int J = 0; J < 2; ++J) store_rows(sW + (32 * J) * KS + 32 * w, KS, XW[J], li, g);
    __syncthreads();  // W staged, U^T copied
    copy_w();
#pragma unroll
    for (int J = 0; J < 2; ++J) store_rows(sU + (32 * w) * TS + 32 * J, TS, XWt[J], li, g);
    __syncthreads();
    copy_u(p.Wt, true);
  }
}

// ---------------------------------------------------------------------------
// scan over chunks, one wave per (b, h, 32-wide d_v slice), the state in registers.
//   forward:  v = U - W h;           h = gamma_C h + Kd^T v         (stores h, v)
//   reverse:  v = dvl + Kd dh;       dh = gamma_C dh + dhl - W^T v  (stores dh, v^T)
// The d_v columns of the state evolve independently, so a wave owns its slice's whole
// chain: the state is four 32x32 f32 accumulator tiles (rows d_k, lane = d_v column) and
// v two (rows t); neither leaves the registers between the two products of a step.  An
// accumulator tile is itself the B operand of a product that contracts over its rows,
// with the contraction index in the order the accumulator holds it: lane half g of k-step
// kk holds rows 16 kk + 4 g + 0..3 and 16 kk + 8 + 4 g + 0..3 (registers 8 kk' .. 8 kk' + 7).
// The A operands read from memory use the same order: prep stores W, Kd^T and W^T in kperm
// order along the contraction axis, so each A fragment is one 16-byte read; the reverse
// pass's K rows come from k's own layout as two 8-byte reads.  Per chunk the operand tiles
// (W or K, Kd^T or W^T: 32 KB; U^T or dvl's slice; the decays; in reverse dhl's slice) are
// copied global -> LDS by DMA (no registers) one chunk ahead into the other of two buffers.
// The stored h / dh ([d_k][d_v]) and v ([t][d_v]) leave through transposed LDS tiles: each
// lane writes its accumulator column as 8-byte pieces of four consecutive rows, and
// transposed reads (ds_read_b64_tr_b16) hand every lane 8 consecutive d_v of one row, one
// 16-byte store; v^T ([d_v][t], reverse) is read back as plain rows.
// ---------------------------------------------------------------------------
// 16-byte chunk slots of the scan's LDS tiles: 256-byte rows (16 chunks) XOR the row mod
// 16, 128-byte rows (8 chunks) XOR (row / 2) mod 8.  A 16-lane read of one chunk of 16
// consecutive rows then covers the 64 banks once.
EDF_DEVICE int slot_k(int row, int c) { return row * 16 + (c ^ (row & 15)); }
EDF_DEVICE int slot_t(int row, int c) { return row * 8 + (c ^ ((row >> 1) & 7)); }
typedef __attribute__((address_space(3))) bf16 lbf16;
typedef __attribute__((address_space(3))) float lf32;
template <typename T> EDF_DEVICE T lds_ld(const lbf16* p) { return *(const __attribute__((address_space(3))) T*)p; }
template <typename T> EDF_DEVICE void lds_st(lbf16* p, T v) { *(__attribute__((address_space(3))) T*)p = v; }
EDF_DEVICE bf16x4 lds_tr16(const lbf16* p) {
  typedef __attribute__((ext_vector_type(4))) short s16x4;
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}

template <bool REV>
__global__ __launch_bounds__(64) void dr_ck_scanw_kernel(const CkArgs p) {
  // three buffers per chunk operand: chunk it + 2 is copied in while chunk it is used
  __shared__ __attribute__((aligned(16))) bf16 sA1a[CH * DK];  // W (fwd) or K (rev) [t][d_k]
  __shared__ __attribute__((aligned(16))) bf16 sA1b[CH * DK];
  __shared__ __attribute__((aligned(16))) bf16 sA1c[CH * DK];
  __shared__ __attribute__((aligned(16))) bf16 sA2a[DK * CH];  // Kd^T (fwd) or W^T (rev) [d_k][t]
  __shared__ __attribute__((aligned(16))) bf16 sA2b[DK * CH];
  __shared__ __attribute__((aligned(16))) bf16 sA2c[DK * CH];
  __shared__ __attribute__((aligned(16))) bf16 sDa[REV ? 32 * DK : 8];  // dhl slice [32 d_v][d_k] (rev)
  __shared__ __attribute__((aligned(16))) bf16 sDb[REV ? 32 * DK : 8];
  __shared__ __attribute__((aligned(16))) bf16 sDc[REV ? 32 * DK : 8];
  __shared__ __attribute__((aligned(16))) bf16 sXa[32 * CH];  // U^T (fwd) or dvl (rev) slice [32 d_v][t]
  __shared__ __attribute__((aligned(16))) bf16 sXb[32 * CH];
  __shared__ __attribute__((aligned(16))) bf16 sXc[32 * CH];
  __shared__ __attribute__((aligned(16))) float sLa[CH];      // log-decays of the chunk
  __shared__ __attribute__((aligned(16))) float sLb[CH];
  __shared__ __attribute__((aligned(16))) float sLc[CH];
  __shared__ __attribute__((aligned(16))) bf16 sHT[32 * DK];  // state slice transposed [32 d_v][d_k]
  __shared__ __attribute__((aligned(16))) bf16 sVT[32 * CH];  // v slice transposed [32 d_v][t]
  struct Buf {
    lbf16 *a1, *a2, *dh, *xs;
    lf32* lg;
  };
  const Buf B0{(lbf16*)sA1a, (lbf16*)sA2a, (lbf16*)sDa, (lbf16*)sXa, (lf32*)sLa};
  const Buf B1{(lbf16*)sA1b, (lbf16*)sA2b, (lbf16*)sDb, (lbf16*)sXb, (lf32*)sLb};
  const Buf B2{(lbf16*)sA1c, (lbf16*)sA2c, (lbf16*)sDc, (lbf16*)sXc, (lf32*)sLc};
  lbf16 *const HT = (lbf16*)sHT, *const VT = (lbf16*)sVT;

  const int l = threadIdx.x, g = l >> 5, li = l & 31;
  constexpr int NSL = DK / 32;
  const int logical = remap_xcd(blockIdx.x, gridDim.x);  // the slices of one head share an XCD
  const long bh = logical / NSL;
  const int v0 = (logical % NSL) * 32;
  auto chunk_of = [&](int it) { return REV ? p.nch - 1 - it : it; };

  // Buffer resources over this head's regions; a DMA load's lane offset depends only on the
  // lane and on j modulo the swizzle period (4 for 256-byte rows, 2 for 128-byte rows), the
  // rest of every offset is scalar.
  const long nchl = p.nch;
  const rsrc_t rA1 = make_rsrc((REV ? p.Kd : p.W) + bh * nchl * CH * DK, (unsigned)(nchl * CH * DK * 2));
  const rsrc_t rW = make_rsrc((REV ? p.Wt : p.W) + bh * nchl * CH * DK, (unsigned)(nchl * CH * DK * 2));
  const rsrc_t rKd = make_rsrc(p.Kdt + bh * nchl * CH * DK, (unsigned)(nchl * CH * DK * 2));
  const rsrc_t rDh = make_rsrc(REV ? p.dhl + bh * nchl * DK * DK : p.W, REV ? (unsigned)(nchl * DK * DK * 2) : 0u);
  const rsrc_t rLg = make_rsrc(p.lg + bh * nchl * CH, (unsigned)(nchl * CH * 4));
  const rsrc_t rX = make_rsrc((REV ? p.dvl : p.Ut) + bh * nchl * DK * CH, (unsigned)(nchl * DK * CH * 2));
  const rsrc_t rH = make_rsrc((REV ? p.dmN : p.hN) + bh * nchl * DK * DK, (unsigned)(nchl * DK * DK * 2));
  const rsrc_t rV = make_rsrc((REV ? p.dvT : p.vN) + bh * nchl * DK * CH, (unsigned)(nchl * DK * CH * 2));
  unsigned o256[4], o128[2];  // DMA lane offsets (bytes) of the 256- and 128-byte-row tiles
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 4 * j + (l >> 4), lc = (l & 15) ^ (row & 15);
    o256[j] = (unsigned)((row * DK + 8 * lc) * 2);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 8 * j + (l >> 3), lc = (l & 7) ^ ((row >> 1) & 7);
    o128[j] = (unsigned)((row * CH + 8 * lc) * 2);
  }
  auto dma = [&](int c, const Buf& bf) {
    lbf16 *a1 = bf.a1, *a2 = bf.a2, *dh = bf.dh, *xs = bf.xs;
    lf32* lgs = bf.lg;
#pragma unroll
    for (int j = 0; j < 16; ++j)  // -W (fwd) or Kd (rev): 4 rows of 256 bytes per load
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rA1, (lds_void*)(a1 + 512 * j), 16, (int)o256[j & 3],
                                               c * CH * DK * 2 + (j >> 2) * 4096, 0, 0);
    if constexpr (REV) {
#pragma unroll
      for (int j = 0; j < 8; ++j)  // dhl rows d_v = v0 .. v0 + 31 ([d_v][d_k], 256-byte rows)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rDh, (lds_void*)(dh + 512 * j), 16, (int)o256[j & 3],
                                                 (c * DK + v0) * DK * 2 + (j >> 2) * 4096, 0, 0);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rLg, (lds_void*)lgs, 4, 4 * l, c * CH * 4, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)  // U^T (fwd) or dvl (rev) rows d_v = v0 .. v0 + 31 (128-byte rows)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rX, (lds_void*)(xs + 512 * j), 16, (int)o128[j & 1],
                                               (c * DK + v0) * CH * 2 + (j >> 1) * 2048, 0, 0);
#pragma unroll
    for (int j = 0; j < 16; ++j)  // Kd^T (fwd) or W^T (rev): 8 rows of 128 bytes per load
      __builtin_amdgcn_raw_ptr_buffer_load_lds(REV ? rW : rKd, (lds_void*)(a2 + 512 * j), 16, (int)o128[j & 1],
                                               c * DK * CH * 2 + (j >> 1) * 2048, 0, 0);
  };

  f32x16 S[4];  // state slice: rows d_k = 32 m + d_row(r, g), column d_v = v0 + li
#pragma unroll
  for (int m = 0; m < 4; ++m) S[m] = zero16();

  // transposed reads of the staging tiles: lane i of a 16-lane group G reads row (d_v)
  // 8 G + 4 hf + i / 4, columns c0 + 4 (i % 4) .. + 3 and receives column c0 + i of rows
  // 8 G + 4 hf .. + 3; two reads give 8 consecutive d_v of one row, stored at (row c0 + i,
  // d_v v0 + 8 G ..)
  const int G = l >> 4, i16 = l & 15;
  const unsigned so = (unsigned)((i16 * DK + 8 * G) * 2);  // store offset in [rows][DK] layouts
  const unsigned sor = (unsigned)(((l >> 3) * CH + 8 * (l & 7)) * 2);  // v^T rows (reverse)
  auto tr_pair = [&](const lbf16* tile, bool k256, int c0) {
    bf16x4 r[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = 8 * G + 4 * hf + (i16 >> 2), c = (c0 >> 3) + ((i16 & 3) >> 1);
      r[hf] = lds_tr16(tile + 8 * (k256 ? slot_k(row, c) : slot_t(row, c)) + 4 * (i16 & 1));
    }
    return __builtin_bit_cast(u32x4, cat4(r[0], r[1]));
  };

  // Identity A fragments in the accumulator's contraction order: element e of lane (li, g) for
  // k-step kk of a 32-row tile is 1 where its row 16 kk + 4 g + e (e < 4) or 16 kk + 8 + 4 g +
  // e - 4 equals li.  A product with them adds a [rows][d_v] tile held as B fragments.
  bf16x8 Id[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) Id[kk][e] = (bf16)((16 * kk + (e < 4 ? 4 * g + e : 8 + 4 * g + e - 4)) == li ? 1.0f : 0.0f);
  // B fragment of rows 32 tb + 16 kk + (accumulator order) of column li from a [32][cols]
  // LDS tile holding the transpose (row li = column li of the operand)
  auto bfrag_t = [&](const lbf16* tile, bool k256, int c0) {
    const int c = c0 >> 3;
    return k256 ? cat4(lds_ld<bf16x4>(tile + 8 * slot_k(li, c) + 4 * g), lds_ld<bf16x4>(tile + 8 * slot_k(li, c + 1) + 4 * g))
                : cat4(lds_ld<bf16x4>(tile + 8 * slot_t(li, c) + 4 * g), lds_ld<bf16x4>(tile + 8 * slot_t(li, c + 1) + 4 * g));
  };

  auto body = [&](int it, const Buf& bf) {
    const lbf16 *a1 = bf.a1, *a2 = bf.a2, *dh = bf.dh, *xs = bf.xs;
    const lf32* lgs = bf.lg;
    const int c = chunk_of(it);
    // A fragments of the first product (rows t = 32 tb + li, 8 k-steps over d_k), all issued
    // before the first MFMA so that their LDS latency overlaps
    bf16x8 AX[2][8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) AX[tb][kk] = lds_ld<bf16x8>(a1 + 8 * slot_k(32 * tb + li, 2 * kk + g));
    const float lgC = lgs[CH - 1];
    // v = U + (-W) h (forward) or dvl + Kd dh (reverse): rows t = 32 tb + .., column d_v; the
    // U / dvl tile enters through identity products
    f32x16 V[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      V[tb] = zero16();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) V[tb] = mfma32(Id[kk], bfrag_t(xs, false, 32 * tb + 16 * kk), V[tb]);
    }
    // B fragments of the state (k = d_k) in bf16, staged transposed (four rows d_k of column
    // li per 8-byte write)
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      bf16x8 bs;
#pragma unroll
      for (int e = 0; e < 8; ++e) bs[e] = (bf16)S[kk >> 1][8 * (kk & 1) + e];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) V[tb] = mfma32(AX[tb][kk], bs, V[tb]);
      // rows 16 kk + 4 g .. + 3 and 16 kk + 8 + 4 g .. + 3 of column li
      lds_st(HT + 8 * slot_k(li, 2 * kk) + 4 * g, __builtin_shufflevector(bs, bs, 0, 1, 2, 3));
      lds_st(HT + 8 * slot_k(li, 2 * kk + 1) + 4 * g, __builtin_shufflevector(bs, bs, 4, 5, 6, 7));
    }
    __builtin_amdgcn_sched_barrier(0);
    // A fragments of the state update (rows d_k = 32 m + li, 4 k-steps over t)
    bf16x8 AU[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) AU[m][kk] = lds_ld<bf16x8>(a2 + 8 * slot_t(32 * m + li, 2 * kk + g));
    const float gC = __expf(lgC);
    // B fragments of v (k = t); v itself is staged transposed ([d_v][t]: four rows t of
    // column li per 8-byte write)
    bf16x8 Bv[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int e = 0; e < 8; ++e) Bv[kk][e] = (bf16)V[kk >> 1][8 * (kk & 1) + e];
      lds_st(VT + 8 * slot_t(li, 2 * kk) + 4 * g, __builtin_shufflevector(Bv[kk], Bv[kk], 0, 1, 2, 3));
      lds_st(VT + 8 * slot_t(li, 2 * kk + 1) + 4 * g, __builtin_shufflevector(Bv[kk], Bv[kk], 4, 5, 6, 7));
    }
    // state update over t: forward h = gamma_C h + Kd^T v; reverse dh = gamma_C dh + dhl +
    // (-W^T) v, the dhl tile through identity products
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int r = 0; r < 16; ++r) S[m][r] *= gC;
      if constexpr (REV) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) S[m] = mfma32(Id[kk], bfrag_t(dh, true, 32 * m + 16 * kk), S[m]);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) S[m] = mfma32(AU[m][kk], Bv[kk], S[m]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // stored rows, 16 bytes per lane: the state [d_k][v0 .. v0 + 31] (eight transposed read
    // pairs), then v [t][v0 ..] (forward, four pairs) or v^T [v0 .. v0 + 31][t] (reverse, rows)
#pragma unroll
    for (int s = 0; s < 8; ++s)
      __builtin_amdgcn_raw_buffer_store_b128(tr_pair(HT, true, 16 * s), rH, (int)so,
                                             (c * DK * DK + 16 * s * DK + v0) * 2, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if constexpr (!REV) {
        __builtin_amdgcn_raw_buffer_store_b128(tr_pair(VT, false, 16 * s), rV, (int)so,
                                               (c * CH * DK + 16 * s * DK + v0) * 2, 0);
      } else {  // rows d_v = 8 s + (l >> 3), chunk l & 7
        const u32x4 d = lds_ld<u32x4>(VT + 8 * slot_t(8 * s + (l >> 3), l & 7));
        __builtin_amdgcn_raw_buffer_store_b128(d, rV, (int)sor, (c * DK * CH + (v0 + 8 * s) * CH) * 2, 0);
      }
    }
  };

  dma(chunk_of(0), B0);
  dma(chunk_of(min(1, p.nch - 1)), B1);
  // Step it reads buffer it % 3 after issuing chunk it + 2's copies into buffer (it + 2) % 3
  // (unconditional: past the last chunk they reload it).  First it waits until its own
  // copies have landed: issued after them are the stores of steps it - 2 and it - 1 (NST
  // each) and chunk it + 1's copies (NDMA), more than the counter's 63 in reverse, where
  // vmcnt(63) is the closest bound; and until every LDS access of step it - 1 has completed
  // (the DMA overwrites what step it - 1 read).
  constexpr int NST = 12;               // global stores per step (8 state rows + 4 v rows per lane)
  constexpr int NDMA = REV ? 45 : 37;   // DMA loads per chunk
  constexpr int WAITV = 2 * NST + NDMA < 63 ? 2 * NST + NDMA : 63;
  auto step = [&](int it, const Buf& cur, const Buf& nxt2) {
    __builtin_amdgcn_s_waitcnt(0x0070 | (WAITV & 15) | ((WAITV >> 4) << 14));  // vmcnt(WAITV) lgkmcnt(0)
    dma(chunk_of(min(it + 2, p.nch - 1)), nxt2);
    body(it, cur);
  };
  int it = 0;
  for (; it + 2 < p.nch; it += 3) {
    step(it, B0, B2);
    step(it + 1, B1, B0);
    step(it + 2, B2, B1);
  }
  if (it < p.nch) step(it, B0, B2);
  if (it + 1 < p.nch) step(it + 1, B1, B0);
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
  __shared__ float lg[CH], bt[CH];
  // d log-gamma and dbeta per step: one row per wave, added to only by its own wave, so its LDS
  // atomic adds (no return value, no wait) land in program order; the rows are summed over the
  // waves in a fixed order at the end, so the result is the same on every run (one row shared
  // by the four waves added in arrival order)
  __shared__ float dlgw[4][CH], dbtw[4][CH];
  bf16* sdS = sdSF;
  bf16* sdF = sdSF + CH * TS;
  bf16* sV = sdSF;  // dV [s][d_v] (lds_off rows), staged before dS and dF are formed

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  // this wave's row of dlgw / dbtw, chosen by a wave-uniform branch so that each add's LDS
  // address keeps a constant row base (a per-wave row pointer cost registers and spills)
  const int wrow = __builtin_amdgcn_readfirstlane(w);
  auto add_row = [&](float (*rows)[CH], int i, float v) {
    if (wrow == 0) atomicAdd(&rows[0][i], v);
    else if (wrow == 1) atomicAdd(&rows[1][i], v);
    else if (wrow == 2) atomicAdd(&rows[2][i], v);
    else atomicAdd(&rows[3][i], v);
  };
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
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      dlgw[ww][tid] = 0.0f;
      dbtw[ww][tid] = 0.0f;
    }
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
    if (g == 0) add_row(dbtw, s, t0 + s < p.T ? acc : 0.0f);
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
    if (g == 0) add_row(dlgw, s, -cs);
    const int tr = 32 * I + d_row(li & 15, g);
    const float rs = rowsum32(z, li);
    if (li < 16) add_row(dlgw, tr, rs);
    if (kind) {
      const float rb = rowsum32(sb, li);
      if (li < 16) add_row(dbtw, tr, rb);
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
    if (g == 0) add_row(dlgw, t, gmt * qx);
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
      add_row(dlgw, t, -sc1 * k1 - sc2 * k2);
      add_row(dbtw, t, -gmt * k2);
      dlgC += sc1 * k1;
    }
    XK[j] = X3;
  }
  {  // gamma_C <dh, h> and the Kd terms enter the decay of the last step
    float acc = hdh * __expf(lgC) + dlgC;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (l == 0) add_row(dlgw, CH - 1, acc);
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
    float x = (dlgw[0][l] + dlgw[1][l]) + (dlgw[2][l] + dlgw[3][l]);
    const float dbl = (dbtw[0][l] + dbtw[1][l]) + (dbtw[2][l] + dbtw[3][l]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_down(x, off);
      if (l + off < 64) x += y;
    }
    const int t = t0 + l;
    if (t < p.T) {
      const long hi = head_off(p, b, h, t);
      p.dbeta[hi] = (bf16)dbl;
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
  size_t lg, W, Wt, Ut, Kdt, Kd, Tt, P, hN, vN, dvl, dhl, dmN, dvT, total;
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
  take(L.Kd, tile_ck, ctx);
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
  a.Kd = (bf16*)(wc + Lc.Kd);
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
  dr_ck_scanw_kernel<false><<<bh * (DK / VS), 64, 0, s>>>(a);
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
  dr_ck_scanw_kernel<true><<<bh * (DK / VS), 64, 0, s>>>(a);
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
  dr_ck_scanw_kernel<false><<<bh * (DK / VS), 64, 0, s>>>(a);
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
