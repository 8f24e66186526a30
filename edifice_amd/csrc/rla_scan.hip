// RLA / RDN (residual linear attention): a base state S and a residual state R, forward and
// backward (native/cuda/fused_rla_scan.cu, fused_rla_scan_backward.cu).
//
// Semantics (S, R [d_v x d_k] per (batch, head); alpha, beta, gamma per head and step):
//   e = v - S k,  re = clip(e, -c, c)              (retrieval from the state BEFORE the step)
//   RLA (variant 0): S = a S + b v k^T,       R = a R + g re k^T
//   RDN (variant 1): S = a S + b e k^T,       R = a R + g (re - R k) k^T
//   o = (S + R) q
// (fused_rla_scan.cu:1-20 and 114-180; fallback fused_scan.ex:2692-2768.)
//
// Every row of S and R evolves on its own given k and the gates, so the work is laid out
// as in the per-step delta kernels: a workgroup owns RB = 16 value rows of both states of
// one head, lane (tr, tc) holds columns tc + 16 c of row 16 rb + tr of each, and row sums
// are 16-lane DPP reductions.  The forward is row-local end to end.  The backward's sums
// over rows (dq, dk and the three per-head gate gradients) are formed per row block (a
// per-step LDS tile of the block's 16 rows, summed in row order behind a barrier) and
// added across blocks in a fixed order by a small kernel.  The forward states are
// checkpointed every CK = 8 steps and recomputed per chunk (two states per lane, so half
// the delta kernels' chunk keeps them in registers).
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int RLA_RB = 16;  // state rows per workgroup
constexpr int RLA_CKF = 16;  // forward staging chunk
constexpr int RLA_CK = 8;    // backward chunk / checkpoint interval
static_assert(RLA_CKF % RLA_CK == 0, "a forward chunk holds whole checkpoint intervals");

struct RLAArgs {
  const void *q, *k, *v, *alpha, *beta, *gamma, *dout;
  void *out, *dq, *dk, *dv, *dalpha, *dbeta, *dgamma;
  float* ckpt;    // [BH][nck][2][DP*DP]  (S, R) after each chunk
  float* part_q;  // [nrb][B*T*H][d]
  float* part_k;  // [nrb][B*T*H][d]
  float* part_s;  // [3][nrb][B*T*H]      dalpha, dbeta, dgamma
  int H, T, d, nck;
  float clip;
};

template <int CK, int DP>
struct RStage {
  float k[CK][DP], q[CK][DP];
  float v[CK][RLA_RB], go[CK][RLA_RB];
  float a[CK], b[CK], g[CK];
};

// A chunk's inputs loaded a chunk ahead into registers (raw values from clamped addresses:
// no branch around a load, whose join would wait for it), then masked - zero beyond T and
// d; beyond T the gates are a = 1, b = g = 0, so a padding step is the identity of the
// recurrence and of its adjoint - and written to the other of two LDS stages once the
// current chunk is done, so their latency hides under the chunk's steps (one barrier per
// chunk).
template <typename TT, int CK, int DP>
struct RRegs {
  static constexpr int EK = (CK * DP + 255) / 256;
  static constexpr int EV = (CK * RLA_RB + 255) / 256;
  TT k[EK], q[EK], v[EV], go[EV], a, b, g;
};

template <typename TT, int CK, int DP>
EDF_DEVICE void rla_load(RRegs<TT, CK, DP>& R, const RLAArgs& p, long bh, int rb, int t0, bool grad) {
  const int b = (int)(bh / p.H), h = (int)(bh % p.H), d = p.d, tid = threadIdx.x;
#pragma unroll
  for (int n = 0; n < RRegs<TT, CK, DP>::EK; ++n) {
    const int e = min(tid + 256 * n, CK * DP - 1), tt = e / DP, j = e % DP;
    const long idx = (((long)b * p.T + min(t0 + tt, p.T - 1)) * p.H + h) * d + min(j, d - 1);
    R.k[n] = ((const TT*)p.k)[idx];
    R.q[n] = ((const TT*)p.q)[idx];
  }
#pragma unroll
  for (int n = 0; n < RRegs<TT, CK, DP>::EV; ++n) {
    const int e = min(tid + 256 * n, CK * RLA_RB - 1), tt = e / RLA_RB, i = rb * RLA_RB + e % RLA_RB;
    const long idx = (((long)b * p.T + min(t0 + tt, p.T - 1)) * p.H + h) * d + min(i, d - 1);
    R.v[n] = ((const TT*)p.v)[idx];
    if (grad) R.go[n] = ((const TT*)p.dout)[idx];
  }
  const long gi = ((long)b * p.T + min(t0 + tid % CK, p.T - 1)) * p.H + h;
  R.a = ((const TT*)p.alpha)[gi];
  R.b = ((const TT*)p.beta)[gi];
  R.g = ((const TT*)p.gamma)[gi];
}

template <typename TT, int CK, int DP>
EDF_DEVICE void rla_store(RStage<CK, DP>& sm, const RRegs<TT, CK, DP>& R, const RLAArgs& p, int rb, int t0,
                          bool grad) {
  const int d = p.d, tid = threadIdx.x;
#pragma unroll
  for (int n = 0; n < RRegs<TT, CK, DP>::EK; ++n) {
    const int e = tid + 256 * n, tt = e / DP, j = e % DP;
    if (e < CK * DP) {
      const bool ok = t0 + tt < p.T && j < d;
      sm.k[tt][j] = ok ? to_f32(R.k[n]) : 0.0f;
      sm.q[tt][j] = ok ? to_f32(R.q[n]) : 0.0f;
    }
  }
#pragma unroll
  for (int n = 0; n < RRegs<TT, CK, DP>::EV; ++n) {
    const int e = tid + 256 * n, tt = e / RLA_RB, ii = e % RLA_RB, i = rb * RLA_RB + ii;
    if (e < CK * RLA_RB) {
      const bool ok = t0 + tt < p.T && i < d;
      sm.v[tt][ii] = ok ? to_f32(R.v[n]) : 0.0f;
      if (grad) sm.go[tt][ii] = ok ? to_f32(R.go[n]) : 0.0f;
    }
  }
  if (tid < CK) {
    const bool ok = t0 + tid < p.T;
    sm.a[tid] = ok ? to_f32(R.a) : 1.0f;
    sm.b[tid] = ok ? to_f32(R.b) : 0.0f;
    sm.g[tid] = ok ? to_f32(R.g) : 0.0f;
  }
}

// The row coefficients of k^T in the two updates, from the pre-step retrievals.
template <int VAR>
EDF_DEVICE void rla_coefs(float vi, float rs, float rr, float b, float g, float clip, float& e, float& re,
                          float& cs, float& cr) {
  e = vi - rs;
  re = fminf(fmaxf(e, -clip), clip);
  if (VAR == 0) {
    cs = b * vi;
    cr = g * re;
  } else {
    cs = b * e;
    cr = g * (re - rr);
  }
}

template <int CK, int DP, int VAR>
EDF_DEVICE void rla_step(float (&S)[DP / 16], float (&R)[DP / 16], const RStage<CK, DP>& sm, int tt, int tr, int tc,
                         float clip) {
  constexpr int NC = DP / 16;
  float rs = 0.0f, rr = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    rs = fmaf(S[c], sm.k[tt][tc + 16 * c], rs);
    if (VAR == 1) rr = fmaf(R[c], sm.k[tt][tc + 16 * c], rr);
  }
  rs = row16_sum(rs);
  if (VAR == 1) rr = row16_sum(rr);
  float e, re, cs, cr;
  rla_coefs<VAR>(sm.v[tt][tr], rs, rr, sm.b[tt], sm.g[tt], clip, e, re, cs, cr);
  const float a = sm.a[tt];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float kj = sm.k[tt][tc + 16 * c];
    S[c] = fmaf(cs, kj, a * S[c]);
    R[c] = fmaf(cr, kj, a * R[c]);
  }
}

// OB: p.out is set and stored through a buffer resource over the batch row by every lane (an
// out-of-bounds offset where the lane stores nothing, steps past T past the row), so the
// unrolled steps hold no branch around the store.
template <typename TT, int DP, int VAR, int CK, bool OB>
__global__ __launch_bounds__(256) void rla_fwd_kernel(const RLAArgs p) {
  constexpr int NC = DP / 16;
  __shared__ RStage<CK, DP> sms[2];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long bh = blockIdx.x;
  const int rb = blockIdx.y, i = rb * RLA_RB + tr;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int nch = (p.T + CK - 1) / CK;
  const long rowel = (long)p.T * p.H * p.d;
  const rsrc_t r_out = make_rsrc(OB ? (const TT*)p.out + (long)b * rowel : (const TT*)p.k,
                                 OB ? (unsigned)(rowel * sizeof(TT)) : 0u);
  const unsigned obase = (tc == 0 && i < p.d) ? (unsigned)(((long)h * p.d + i) * sizeof(TT)) : OOB_OFF;
  const unsigned ostep = (unsigned)((long)p.H * p.d * sizeof(TT));
  float S[NC], R[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) S[c] = R[c] = 0.0f;
  RRegs<TT, CK, DP> G;
  rla_load<TT, CK, DP>(G, p, bh, rb, 0, false);
  rla_store<TT, CK, DP>(sms[0], G, p, rb, 0, false);
  __syncthreads();
  for (int chn = 0; chn < nch; ++chn) {
    const int t0 = chn * CK;
    const RStage<CK, DP>& sm = sms[chn & 1];
    rla_load<TT, CK, DP>(G, p, bh, rb, min(t0 + CK, (nch - 1) * CK), false);  // next chunk (past the last: a reload)
#pragma unroll
    for (int tt = 0; tt < CK; ++tt) {  // padding past T: identity steps (a = 1, b = g = 0, k = 0)
      rla_step<CK, DP, VAR>(S, R, sm, tt, tr, tc, p.clip);
      if (OB || p.out != nullptr) {
        float o = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) o = fmaf(S[c] + R[c], sm.q[tt][tc + 16 * c], o);
        o = row16_sum(o);
        if constexpr (OB) bstore<TT>(r_out, obase + (unsigned)(t0 + tt) * ostep, o);
        else if (tc == 0 && i < p.d && t0 + tt < p.T) st((TT*)p.out, (((long)b * p.T + t0 + tt) * p.H + h) * p.d + i, o);
      }
      // both states after every RLA_CK steps (a 16-step chunk writes two; none past the last)
      const int ck = (t0 + tt) / RLA_CK;
      if (tt % RLA_CK == RLA_CK - 1 && p.ckpt != nullptr && ck < p.nck) {
        float* cp = p.ckpt + (((long)bh * p.nck + ck) * 2) * DP * DP + (long)i * DP + tc;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          cp[16 * c] = S[c];
          cp[DP * DP + 16 * c] = R[c];
        }
      }
    }
    // the other stage was last read in the previous chunk, before the barrier below it
    rla_store<TT, CK, DP>(sms[(chn + 1) & 1], G, p, rb, t0 + CK, false);
    __syncthreads();
  }
}

// Backward over chunks in reverse.  Per step (S_p, R_p before it; dS, dR the adjoints after):
//   dS_t = dS + do q^T, dR_t = dR + do q^T, dq = (S_n + R_n)^T do, ds_k = dS_t k, dr_k = dR_t k,
//   m = [|e| <= c], dE_S = g dr_k m (RLA) | b ds_k + g dr_k m (RDN), dE_R = 0 | g dr_k,
//   dv = b ds_k + g dr_k m, dk = dS_t^T cS + dR_t^T cR - S_p^T dE_S - R_p^T dE_R,
//   dalpha = <dS_t, S_p> + <dR_t, R_p>, dbeta = ds_k . (v | e), dgamma = dr_k . (re | re - R_p k),
//   dS <- a dS_t - dE_S k^T, dR <- a dR_t - dE_R k^T.
template <typename TT, int DP, int VAR>
__global__ __launch_bounds__(256) void rla_bwd_kernel(const RLAArgs p) {
  constexpr int NC = DP / 16, CK = RLA_CK;
  __shared__ RStage<CK, DP> sms[2];
  __shared__ float red[2][RLA_RB][row16_stride(DP)];  // this step's per-row dq and dk terms
  __shared__ float reds[3][RLA_RB];         // and dalpha, dbeta, dgamma terms
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long bh = blockIdx.x;
  const int rb = blockIdx.y, i = rb * RLA_RB + tr;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const long nbth = (long)gridDim.x * p.T;
  const float clip = p.clip;
  float dS[NC], dR[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dS[c] = dR[c] = 0.0f;

  // chunk inputs and the checkpoints each chunk starts from, loaded a chunk ahead
  RRegs<TT, CK, DP> G;
  float cS[NC], cR[NC];
  auto load_ck = [&](int ck) {
    // chunk 0 starts from zero; its (unused) load address stays in bounds
    const float* cp = p.ckpt + (((long)bh * p.nck + max(ck - 1, 0)) * 2) * DP * DP + (long)i * DP + tc;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      cS[c] = cp[16 * c];
      cR[c] = cp[DP * DP + 16 * c];
    }
  };
  rla_load<TT, CK, DP>(G, p, bh, rb, (p.nck - 1) * CK, true);
  load_ck(p.nck - 1);
  rla_store<TT, CK, DP>(sms[(p.nck - 1) & 1], G, p, rb, (p.nck - 1) * CK, true);
  __syncthreads();
  for (int ck = p.nck - 1; ck >= 0; --ck) {
    const int t0 = ck * CK;
    const RStage<CK, DP>& sm = sms[ck & 1];
    float Sl[CK][NC], Rl[CK][NC];
    {
      float S[NC], R[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        S[c] = ck > 0 ? cS[c] : 0.0f;
        R[c] = ck > 0 ? cR[c] : 0.0f;
      }
      // the previous chunk's inputs and checkpoints load under this chunk's work
      rla_load<TT, CK, DP>(G, p, bh, rb, max(ck - 1, 0) * CK, true);
      load_ck(max(ck - 1, 0));
#pragma unroll
      for (int tt = 0; tt < CK; ++tt) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          Sl[tt][c] = S[c];
          Rl[tt][c] = R[c];
        }
        rla_step<CK, DP, VAR>(S, R, sm, tt, tr, tc, clip);
      }
    }
#pragma unroll
    for (int tt = CK - 1; tt >= 0; --tt) {
      const int t = t0 + tt;
      const float goi = sm.go[tt][tr], vi = sm.v[tt][tr];
      const float a = sm.a[tt], bb = sm.b[tt], gg = sm.g[tt];
      float rs = 0.0f, rr = 0.0f, dsk = 0.0f, drk = 0.0f, dts[NC], dtr[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float kj = sm.k[tt][tc + 16 * c], qj = sm.q[tt][tc + 16 * c];
        dts[c] = fmaf(goi, qj, dS[c]);
        dtr[c] = fmaf(goi, qj, dR[c]);
        rs = fmaf(Sl[tt][c], kj, rs);
        if (VAR == 1) rr = fmaf(Rl[tt][c], kj, rr);
        dsk = fmaf(dts[c], kj, dsk);
        drk = fmaf(dtr[c], kj, drk);
      }
      rs = row16_sum(rs);
      if (VAR == 1) rr = row16_sum(rr);
      dsk = row16_sum(dsk);
      drk = row16_sum(drk);
      float e, re, cs, cr;
      rla_coefs<VAR>(vi, rs, rr, bb, gg, clip, e, re, cs, cr);
      const float gm = fabsf(e) <= clip ? gg * drk : 0.0f;
      const float des = VAR == 0 ? gm : fmaf(bb, dsk, gm);
      const float der = VAR == 0 ? 0.0f : gg * drk;
      float pa = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float kj = sm.k[tt][tc + 16 * c];
        const float sn = fmaf(cs, kj, a * Sl[tt][c]), rn = fmaf(cr, kj, a * Rl[tt][c]);
        red[0][tr][tc + 16 * c] = (sn + rn) * goi;
        red[1][tr][tc + 16 * c] = fmaf(dts[c], cs, dtr[c] * cr) - fmaf(Sl[tt][c], des, Rl[tt][c] * der);
        pa = fmaf(dts[c], Sl[tt][c], fmaf(dtr[c], Rl[tt][c], pa));
        dS[c] = fmaf(-des, kj, a * dts[c]);
        dR[c] = fmaf(-der, kj, a * dtr[c]);
      }
      pa = row16_sum(pa);
      const bool row = tc == 0 && i < p.d;
      if (tc == 0) {
        reds[0][tr] = row ? pa : 0.0f;
        reds[1][tr] = row ? dsk * (VAR == 0 ? vi : e) : 0.0f;
        reds[2][tr] = row ? drk * (VAR == 0 ? re : re - rr) : 0.0f;
      }
      if (t < p.T && row) st((TT*)p.dv, (((long)b * p.T + t) * p.H + h) * p.d + i, fmaf(bb, dsk, gm));
      // the block's sums over its 16 rows, in row order, through LDS
      __syncthreads();
      if (t < p.T) {
        const long bth = ((long)b * p.T + t) * p.H + h;
        for (int e2 = tid; e2 < 2 * DP; e2 += 256) {
          const int qty = e2 / DP, j = e2 % DP;
          float acc = 0.0f;
#pragma unroll
          for (int m = 0; m < RLA_RB; ++m) acc += red[qty][m][j];
          if (j < p.d) (qty == 0 ? p.part_q : p.part_k)[((long)rb * nbth + bth) * p.d + j] = acc;
        }
        if (tid >= 253) {
          const int qty = tid - 253, nrb = gridDim.y;
          float acc = 0.0f;
#pragma unroll
          for (int m = 0; m < RLA_RB; ++m) acc += reds[qty][m];
          p.part_s[((long)qty * nrb + rb) * nbth + bth] = acc;
        }
      }
      __syncthreads();
    }
    // the other stage was last read in the previous chunk, before this chunk's barriers
    rla_store<TT, CK, DP>(sms[(ck + 1) & 1], G, p, rb, (ck - 1) * CK, true);
    __syncthreads();
  }
}

// dq, dk and the per-head gate gradients: row-block partials added in block order.
template <typename TT>
__global__ __launch_bounds__(256) void rla_reduce_kernel(const RLAArgs p, long nbth, int nrb) {
  long e = (long)blockIdx.x * 256 + threadIdx.x;
  const long nvec = nbth * p.d;
  // with d a multiple of 4, the dq / dk sums go four at a time (16-byte loads, the row blocks
  // added in the same order as one at a time) and the items after them continue below
  const long n4 = p.d % 4 == 0 ? 2 * nvec / 4 : 0;
  if (e < n4) {
    const long e4 = 4 * e;
    const int qty = e4 >= nvec;
    const long o = e4 - qty * nvec;
    const float4* part = reinterpret_cast<const float4*>((qty ? p.part_k : p.part_q) + o);
    float4 acc = part[0];
    for (int r = 1; r < nrb; ++r) {
      const float4 v = part[(long)r * (nvec / 4)];
      acc.x += v.x, acc.y += v.y, acc.z += v.z, acc.w += v.w;
    }
    TT* dst = (TT*)(qty ? p.dk : p.dq) + o;
    st(dst, 0, acc.x), st(dst, 1, acc.y), st(dst, 2, acc.z), st(dst, 3, acc.w);
    return;
  }
  e += 4 * n4 - n4;  // the items before e - n4 were the 4 n4 vector elements
  if (e < 2 * nvec) {
    const int qty = e >= nvec;
    const long o = e - qty * nvec;
    const float* part = qty ? p.part_k : p.part_q;
    float acc = 0.0f;
    for (int r = 0; r < nrb; ++r) acc += part[r * nvec + o];
    st((TT*)(qty ? p.dk : p.dq), o, acc);
  } else if (e < 2 * nvec + 3 * nbth) {
    const long f = e - 2 * nvec;
    const int qty = (int)(f / nbth);
    const long o = f - qty * nbth;
    float acc = 0.0f;
    for (int r = 0; r < nrb; ++r) acc += p.part_s[((long)qty * nrb + r) * nbth + o];
    st((TT*)(qty == 0 ? p.dalpha : qty == 1 ? p.dbeta : p.dgamma), o, acc);
  }
}

inline int rla_pad(int d) { return d <= 16 ? 16 : d <= 32 ? 32 : d <= 64 ? 64 : 128; }
inline size_t rla_align(size_t v) { return (v + 255) & ~(size_t)255; }

struct RLAWs {
  size_t ckpt, part_q, part_k, part_s, total;
};

inline RLAWs rla_ws(int batch, int seq, int heads, int d) {
  const size_t dp = rla_pad(d), nrb = dp / RLA_RB, nck = (seq + RLA_CK - 1) / RLA_CK;
  const size_t bh = (size_t)batch * heads, nbth = bh * seq;
  RLAWs w{};
  size_t off = 0;
  w.ckpt = off;
  off += rla_align(bh * nck * 2 * dp * dp * 4);
  w.part_q = off;
  off += rla_align(nrb * nbth * d * 4);
  w.part_k = off;
  off += rla_align(nrb * nbth * d * 4);
  w.part_s = off;
  off += rla_align(3 * nrb * nbth * 4);
  w.total = off;
  return w;
}

template <typename TT, int VAR>
int rla_launch(hipStream_t s, const RLAArgs& a, int mode, int BH) {
  // mode 0: forward; 1: forward writing checkpoints every RLA_CK steps; 2: backward
  const int d = a.d;
  const bool ob = a.out != nullptr && (long)(a.T + RLA_CKF) * a.H * a.d * (long)sizeof(TT) < (1L << 31);
#define EDF_RLA_LAUNCH(DP)                                               \
  do {                                                                   \
    const dim3 grid(BH, DP / RLA_RB);                                    \
    if (mode == 2)                                                       \
      rla_bwd_kernel<TT, DP, VAR><<<grid, 256, 0, s>>>(a);               \
    else if (mode == 1 && ob)                                            \
      rla_fwd_kernel<TT, DP, VAR, RLA_CK, true><<<grid, 256, 0, s>>>(a); \
    else if (mode == 1)                                                  \
      rla_fwd_kernel<TT, DP, VAR, RLA_CK, false><<<grid, 256, 0, s>>>(a); \
    else if (ob)                                                         \
      rla_fwd_kernel<TT, DP, VAR, RLA_CKF, true><<<grid, 256, 0, s>>>(a); \
    else                                                                 \
      rla_fwd_kernel<TT, DP, VAR, RLA_CKF, false><<<grid, 256, 0, s>>>(a); \
  } while (0)
  if (d <= 16)
    EDF_RLA_LAUNCH(16);
  else if (d <= 32)
    EDF_RLA_LAUNCH(32);
  else if (d <= 64)
    EDF_RLA_LAUNCH(64);
  else
    EDF_RLA_LAUNCH(128);
#undef EDF_RLA_LAUNCH
  return check_launch(mode == 2 ? "rla backward" : "rla");
}

template <typename TT>
int rla_launch_v(hipStream_t s, const RLAArgs& a, int mode, int BH, int variant) {
  return variant == 0 ? rla_launch<TT, 0>(s, a, mode, BH) : rla_launch<TT, 1>(s, a, mode, BH);
}

int check_rla(int batch, int seq, int heads, int d, int variant, float clip, int dtype) {
  EDF_REQUIRE(batch > 0 && seq > 0 && heads > 0 && d > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(d <= 128, EDF_ERR_UNSUPPORTED, "head_dim %d > 128 unsupported", d);
  EDF_REQUIRE(variant == 0 || variant == 1, EDF_ERR_INVALID_ARG, "variant must be 0 (RLA) or 1 (RDN)");
  EDF_REQUIRE(clip >= 0.0f, EDF_ERR_INVALID_ARG, "clip threshold must be >= 0");
  return EDF_OK;
}

RLAArgs rla_args(const void* q, const void* k, const void* v, const void* alpha, const void* beta, const void* gamma,
                 int seq, int heads, int d, float clip) {
  RLAArgs a{};
  a.q = q; a.k = k; a.v = v; a.alpha = alpha; a.beta = beta; a.gamma = gamma;
  a.H = heads; a.T = seq; a.d = d; a.clip = clip;
  a.nck = (seq + RLA_CK - 1) / RLA_CK;
  return a;
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_fused_rla_scan(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                       const void* beta, const void* gamma, void* out, int batch, int seq_len, int num_heads,
                       int head_dim, int variant, float clip_threshold, int dtype) {
  using namespace edf;
  int rc = check_rla(batch, seq_len, num_heads, head_dim, variant, clip_threshold, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && gamma && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  RLAArgs a = rla_args(q, k, v, alpha, beta, gamma, seq_len, num_heads, head_dim, clip_threshold);
  a.out = out;
  hipStream_t s = as_stream(stream);
  const int bh = batch * num_heads;
  return dtype == EDF_BF16 ? rla_launch_v<bf16>(s, a, 0, bh, variant) : rla_launch_v<float>(s, a, 0, bh, variant);
}

size_t edf_rla_scan_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return edf::rla_ws(batch, seq_len, num_heads, head_dim).total;
}

// the backward proper; `context` (nullable) holds the states every RLA_CK steps a recording
// forward left, else a checkpointing forward pass writes them first
static int rla_backward(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                        const void* beta, const void* gamma, const void* grad_out, void* grad_q, void* grad_k,
                        void* grad_v, void* grad_alpha, void* grad_beta, void* grad_gamma, const void* context,
                        void* workspace, size_t workspace_bytes, int batch, int seq_len, int num_heads, int head_dim,
                        int variant, float clip_threshold, int dtype) {
  using namespace edf;
  int rc = check_rla(batch, seq_len, num_heads, head_dim, variant, clip_threshold, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && gamma && grad_out && grad_q && grad_k && grad_v && grad_alpha &&
                  grad_beta && grad_gamma,
              EDF_ERR_INVALID_ARG, "null tensor pointer");
  const RLAWs w = rla_ws(batch, seq_len, num_heads, head_dim);
  EDF_REQUIRE(workspace && workspace_bytes >= w.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              w.total);
  char* ws = (char*)workspace;
  RLAArgs a = rla_args(q, k, v, alpha, beta, gamma, seq_len, num_heads, head_dim, clip_threshold);
  a.dout = grad_out;
  a.dq = grad_q; a.dk = grad_k; a.dv = grad_v;
  a.dalpha = grad_alpha; a.dbeta = grad_beta; a.dgamma = grad_gamma;
  a.ckpt = context ? (float*)const_cast<void*>(context) : (float*)(ws + w.ckpt);
  a.part_q = (float*)(ws + w.part_q);
  a.part_k = (float*)(ws + w.part_k);
  a.part_s = (float*)(ws + w.part_s);
  const int bh = batch * num_heads, nrb = rla_pad(head_dim) / RLA_RB;
  const long nbth = (long)bh * seq_len;
  const long n4 = head_dim % 4 == 0 ? 2 * nbth * head_dim / 4 : 0;  // vector items of the reduction
  const unsigned gred = (unsigned)((2 * nbth * head_dim + 3 * nbth - 3 * n4 + 255) / 256);
  hipStream_t s = as_stream(stream);
  if (dtype == EDF_BF16) {
    if (!context && (rc = rla_launch_v<bf16>(s, a, 1, bh, variant))) return rc;
    if ((rc = rla_launch_v<bf16>(s, a, 2, bh, variant))) return rc;
    rla_reduce_kernel<bf16><<<gred, 256, 0, s>>>(a, nbth, nrb);
  } else {
    if (!context && (rc = rla_launch_v<float>(s, a, 1, bh, variant))) return rc;
    if ((rc = rla_launch_v<float>(s, a, 2, bh, variant))) return rc;
    rla_reduce_kernel<float><<<gred, 256, 0, s>>>(a, nbth, nrb);
  }
  return check_launch("rla backward reduction");
}

int edf_fused_rla_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                const void* beta, const void* gamma, const void* forward_out, const void* grad_out,
                                void* grad_q, void* grad_k, void* grad_v, void* grad_alpha, void* grad_beta,
                                void* grad_gamma, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                int num_heads, int head_dim, int variant, float clip_threshold, int dtype) {
  (void)forward_out;  // states are recomputed from the inputs
  return rla_backward(stream, q, k, v, alpha, beta, gamma, grad_out, grad_q, grad_k, grad_v, grad_alpha, grad_beta,
                      grad_gamma, nullptr, workspace, workspace_bytes, batch, seq_len, num_heads, head_dim, variant,
                      clip_threshold, dtype);
}

size_t edf_rla_scan_context_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return edf::rla_ws(batch, seq_len, num_heads, head_dim).part_q;
}

int edf_fused_rla_scan_with_context(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                    const void* beta, const void* gamma, void* out, void* context,
                                    size_t context_bytes, int batch, int seq_len, int num_heads, int head_dim,
                                    int variant, float clip_threshold, int dtype) {
  using namespace edf;
  int rc = check_rla(batch, seq_len, num_heads, head_dim, variant, clip_threshold, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && gamma && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = rla_ws(batch, seq_len, num_heads, head_dim).part_q;
  EDF_REQUIRE(context && context_bytes >= need, EDF_ERR_WORKSPACE, "context too small: need %zu bytes", need);
  RLAArgs a = rla_args(q, k, v, alpha, beta, gamma, seq_len, num_heads, head_dim, clip_threshold);
  a.out = out;
  a.ckpt = (float*)context;  // the output kernel also writes the states every RLA_CK steps
  hipStream_t s = as_stream(stream);
  const int bh = batch * num_heads;
  return dtype == EDF_BF16 ? rla_launch_v<bf16>(s, a, 0, bh, variant) : rla_launch_v<float>(s, a, 0, bh, variant);
}

int edf_fused_rla_scan_backward_saved(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                      const void* beta, const void* gamma, const void* grad_out, void* grad_q,
                                      void* grad_k, void* grad_v, void* grad_alpha, void* grad_beta,
                                      void* grad_gamma, const void* context, size_t context_bytes, void* workspace,
                                      size_t workspace_bytes, int batch, int seq_len, int num_heads, int head_dim,
                                      int variant, float clip_threshold, int dtype) {
  const size_t need = edf_rla_scan_context_bytes(batch, seq_len, num_heads, head_dim, dtype);
  EDF_REQUIRE(context && context_bytes >= need, EDF_ERR_WORKSPACE,
              "context too small: need the %zu bytes the forward filled", need);
  return rla_backward(stream, q, k, v, alpha, beta, gamma, grad_out, grad_q, grad_k, grad_v, grad_alpha, grad_beta,
                      grad_gamma, context, workspace, workspace_bytes, batch, seq_len, num_heads, head_dim, variant,
                      clip_threshold, dtype);
}

}  // extern "C"
