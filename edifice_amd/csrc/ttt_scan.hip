// TTT-Linear (test-time training) scan, forward and backward
// (native/cuda/fused_ttt_scan.cu, fused_ttt_scan_backward.cu).
//
// Semantics: an inner linear model W [D x D] per batch element (initial w0), per step
//   pred = W k;  x_hat = (pred - mean) / sqrt(var + 1e-6)  (population variance over D)
//   err = ln_g x_hat + ln_b - v;  W = W - (eta err) k^T;  o = W q
// (fused_ttt_scan.cu:1-30 and 85-150; fallback ttt.ex:369-404.)
//
// The LayerNorm couples all D rows of W at every step, so one workgroup owns one batch
// element's whole W (the chip holds B workgroups, as the reference's one block per batch).
// 256 lanes = 16 groups of 16; group g owns rows g RPG .. g RPG + RPG - 1 (RPG = D/16) and
// lane tc of a group holds columns tc + 16 c of each of them, so pred and o are 16-lane DPP
// row sums and the LayerNorm statistics combine the groups' (count, mean, M2) through LDS
// (Chan's pairwise formula: one barrier per step, no E[x^2] - mean^2 cancellation).
// Backward: the forward re-run checkpoints W every CK steps and stores x_hat, err and
// 1/std per step; each chunk restarts from its exact end-of-chunk checkpoint and walks back
// with W_prev = W + (eta err) k^T (at most CK steps of rounding drift, where the reference
// undoes the whole sequence from W_T).  dq and dk sum over rows: each group sums its rows in
// registers, the 16 group partials meet in LDS (double-buffered by step parity, so two
// barriers per step in all).  dln_g / dln_b are per-batch partials added by a small kernel.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int TTT_CK = 8;  // staged steps / checkpoint interval
constexpr float TTT_EPS = 1.0e-6f;  // fused_ttt_scan.cu:35

struct TArgs {
  const void *q, *k, *v, *eta, *w0, *ln_g, *ln_b, *dout;
  void *out, *dq, *dk, *dv, *deta, *dw0, *dln_g, *dln_b;
  float* ckpt;    // [B][nck][DP*DP]  W after each chunk
  float* xh;      // [B][T][D]
  float* err;     // [B][T][D]
  float* rstd;    // [B][T]
  float* part_g;  // [B][D]
  float* part_b;  // [B][D]
  int T, D, nck;
};

// Chunks of NA [B, T, D] inputs loaded a chunk ahead into registers (raw values from
// clamped addresses: no branch around a load, whose join would wait for it), masked (zero
// beyond T and D) and written to the other of two LDS stages once the current chunk is
// done: their latency hides under the chunk's steps instead of sitting between two
// barriers at its start.
template <typename ST, int DP, int NA>
struct TRegs {
  static constexpr int E = (TTT_CK * DP + 255) / 256;
  ST v[NA][E];
};

template <typename ST, int DP, int NA>
EDF_DEVICE void ttt_load(TRegs<ST, DP, NA>& R, const void* const (&src)[NA], const TArgs& p, int b, int t0) {
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int n = 0; n < TRegs<ST, DP, NA>::E; ++n) {
      const int e = min((int)threadIdx.x + 256 * n, TTT_CK * DP - 1), tt = e / DP, j = min(e % DP, p.D - 1);
      R.v[a][n] = ((const ST*)src[a])[((long)b * p.T + min(t0 + tt, p.T - 1)) * p.D + j];
    }
}

template <typename ST, int DP, int NA>
EDF_DEVICE void ttt_store(float (*const (&dst)[NA])[DP], const TRegs<ST, DP, NA>& R, const TArgs& p, int t0) {
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int n = 0; n < TRegs<ST, DP, NA>::E; ++n) {
      const int e = threadIdx.x + 256 * n, tt = e / DP, j = e % DP;
      if (e < TTT_CK * DP) dst[a][tt][j] = t0 + tt < p.T && j < p.D ? to_f32(R.v[a][n]) : 0.0f;
    }
}

template <typename TT, int DP>
__global__ __launch_bounds__(256) void ttt_fwd_kernel(const TArgs p) {
  constexpr int NC = DP / 16, RPG = DP / 16;
  __shared__ float stg[2][4][TTT_CK][DP];  // two stages of k, q, v, eta
  __shared__ float sg[DP], sb[DP];
  __shared__ float stat[2][16][3];  // per group: valid rows, mean, M2
  const int tid = threadIdx.x, g = tid >> 4, tc = tid & 15, b = blockIdx.x, D = p.D;
  const int ng = max(0, min(RPG, D - g * RPG));
  float W[RPG][NC];
#pragma unroll
  for (int rr = 0; rr < RPG; ++rr) {
    const int r = g * RPG + rr;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int j = tc + 16 * c;
      W[rr][c] = r < D && j < D ? ld((const TT*)p.w0, ((long)b * D + r) * D + j) : 0.0f;
    }
  }
  for (int j = tid; j < DP; j += 256) {
    sg[j] = j < D ? ld((const TT*)p.ln_g, j) : 0.0f;
    sb[j] = j < D ? ld((const TT*)p.ln_b, j) : 0.0f;
  }
  const void* const srcs[4] = {p.k, p.q, p.v, p.eta};
  TRegs<TT, DP, 4> R;
  const int nch = (p.T + TTT_CK - 1) / TTT_CK;
  {
    float(*const d0[4])[DP] = {stg[0][0], stg[0][1], stg[0][2], stg[0][3]};
    ttt_load<TT, DP, 4>(R, srcs, p, b, 0);
    ttt_store<TT, DP, 4>(d0, R, p, 0);
  }
  __syncthreads();
  for (int chn = 0; chn < nch; ++chn) {
    const int t0 = chn * TTT_CK, cb = chn & 1;
    float(*const sk)[DP] = stg[cb][0];
    float(*const sq)[DP] = stg[cb][1];
    float(*const sv)[DP] = stg[cb][2];
    float(*const se)[DP] = stg[cb][3];
    ttt_load<TT, DP, 4>(R, srcs, p, b, min(t0 + TTT_CK, (nch - 1) * TTT_CK));  // next chunk (past the last: a reload)
    for (int tt = 0; tt < TTT_CK && t0 + tt < p.T; ++tt) {
      const int t = t0 + tt, par = t & 1;
      float pred[RPG];
      float s1 = 0.0f;
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) a = fmaf(W[rr][c], sk[tt][tc + 16 * c], a);
        pred[rr] = row16_sum(a);
        if (rr < ng) s1 += pred[rr];
      }
      const float mg = ng > 0 ? s1 / (float)ng : 0.0f;
      float m2 = 0.0f;
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr)
        if (rr < ng) m2 = fmaf(pred[rr] - mg, pred[rr] - mg, m2);
      if (tc == 0) {
        stat[par][g][0] = (float)ng;
        stat[par][g][1] = mg;
        stat[par][g][2] = m2;
      }
      __syncthreads();
      float mu = 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) mu = fmaf(stat[par][u][0], stat[par][u][1], mu);
      mu /= (float)D;
      float M2 = 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float dm = stat[par][u][1] - mu;
        M2 += stat[par][u][2] + stat[par][u][0] * dm * dm;
      }
      const float rs = 1.0f / sqrtf(M2 / (float)D + TTT_EPS);
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr) {
        const int r = g * RPG + rr;
        const float x = (pred[rr] - mu) * rs;
        const float er = fmaf(sg[r], x, sb[r]) - sv[tt][r];
        const float s = se[tt][r] * er;  // 0 on padded rows (eta staged as 0)
#pragma unroll
        for (int c = 0; c < NC; ++c) W[rr][c] = fmaf(-s, sk[tt][tc + 16 * c], W[rr][c]);
        if (p.xh != nullptr && tc == 0 && r < D) {
          p.xh[((long)b * p.T + t) * D + r] = x;
          p.err[((long)b * p.T + t) * D + r] = er;
        }
      }
      if (p.rstd != nullptr && tid == 0) p.rstd[(long)b * p.T + t] = rs;
      if (p.out != nullptr) {
#pragma unroll
        for (int rr = 0; rr < RPG; ++rr) {
          float o = 0.0f;
#pragma unroll
          for (int c = 0; c < NC; ++c) o = fmaf(W[rr][c], sq[tt][tc + 16 * c], o);
          o = row16_sum(o);
          const int r = g * RPG + rr;
          if (tc == 0 && r < D) st((TT*)p.out, ((long)b * p.T + t) * D + r, o);
        }
      }
    }
    if (p.ckpt != nullptr) {
      float* cp = p.ckpt + ((long)b * p.nck + t0 / TTT_CK) * DP * DP;
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr)
#pragma unroll
        for (int c = 0; c < NC; ++c) cp[(g * RPG + rr) * DP + tc + 16 * c] = W[rr][c];
    }
    // the other stage was last read in the previous chunk, before its steps' barriers
    {
      const int nb = cb ^ 1;
      float(*const dn[4])[DP] = {stg[nb][0], stg[nb][1], stg[nb][2], stg[nb][3]};
      ttt_store<TT, DP, 4>(dn, R, p, t0 + TTT_CK);
    }
    __syncthreads();
  }
}

// Backward over chunks in reverse; per step (W_t after it, W_p before, dW the adjoint after):
//   dW_t = dW + do q^T, dq = W_t^T do, d se = -dW_t k, deta = d se err, d err = d se eta,
//   dv = -d err, dln_g += d err x_hat, dln_b += d err, dx = ln_g d err,
//   d pred = rstd (dx - mean(dx) - x_hat mean(dx x_hat)), W_p = W_t + se k^T,
//   dk = -dW_t^T se + W_p^T d pred, dW <- dW_t + d pred k^T.
template <typename TT, int DP>
__global__ __launch_bounds__(256) void ttt_bwd_kernel(const TArgs p) {
  constexpr int NC = DP / 16, RPG = DP / 16;
  __shared__ float stg[2][6][TTT_CK][DP];  // two stages of k, q, eta, dout, x_hat, err
  __shared__ float srss[2][TTT_CK];
  __shared__ float sg[DP];
  __shared__ float stat[2][16][2];      // per group: sum dx, sum dx x_hat
  __shared__ float red[2][16][2][DP];   // per group: dq, dk partials
  const int tid = threadIdx.x, g = tid >> 4, tc = tid & 15, b = blockIdx.x, D = p.D;
  float W[RPG][NC], dW[RPG][NC], agg[RPG], agb[RPG];
#pragma unroll
  for (int rr = 0; rr < RPG; ++rr) {
    agg[rr] = agb[rr] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) dW[rr][c] = 0.0f;
  }
  for (int j = tid; j < DP; j += 256) sg[j] = j < D ? ld((const TT*)p.ln_g, j) : 0.0f;
  // each chunk's inputs, per-step rstd and (DP <= 64: the registers allow it) the W it ends
  // with load a chunk ahead
  constexpr bool PRE_W = DP <= 64;
  const void* const srct[4] = {p.k, p.q, p.eta, p.dout};
  const void* const srcf[2] = {p.xh, p.err};
  TRegs<TT, DP, 4> RT;
  TRegs<float, DP, 2> RF;
  float rsn = 0.0f, Wn[PRE_W ? RPG : 1][PRE_W ? NC : 1];
  auto load_next = [&](int ck) {
    ttt_load<TT, DP, 4>(RT, srct, p, b, ck * TTT_CK);
    ttt_load<float, DP, 2>(RF, srcf, p, b, ck * TTT_CK);
    rsn = p.rstd[(long)b * p.T + min(ck * TTT_CK + (int)(tid % TTT_CK), p.T - 1)];
    if constexpr (PRE_W) {
      const float* cp = p.ckpt + ((long)b * p.nck + ck) * DP * DP;
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr)
#pragma unroll
        for (int c = 0; c < NC; ++c) Wn[rr][c] = cp[(g * RPG + rr) * DP + tc + 16 * c];
    }
  };
  auto store_next = [&](int ck, int sb) {
    const int t0n = ck * TTT_CK;
    float(*const dt[4])[DP] = {stg[sb][0], stg[sb][1], stg[sb][2], stg[sb][3]};
    float(*const df[2])[DP] = {stg[sb][4], stg[sb][5]};
    ttt_store<TT, DP, 4>(dt, RT, p, t0n);
    ttt_store<float, DP, 2>(df, RF, p, t0n);
    if (tid < TTT_CK) srss[sb][tid] = t0n + tid < p.T ? rsn : 0.0f;
  };
  load_next(p.nck - 1);
  store_next(p.nck - 1, (p.nck - 1) & 1);
  __syncthreads();
  for (int ck = p.nck - 1; ck >= 0; --ck) {
    const int t0 = ck * TTT_CK, cb = ck & 1;
    float(*const sk)[DP] = stg[cb][0];
    float(*const sq)[DP] = stg[cb][1];
    float(*const se)[DP] = stg[cb][2];
    float(*const sdo)[DP] = stg[cb][3];
    float(*const sx)[DP] = stg[cb][4];
    float(*const sr)[DP] = stg[cb][5];
    const float* const srs = srss[cb];
    if constexpr (PRE_W) {
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr)
#pragma unroll
        for (int c = 0; c < NC; ++c) W[rr][c] = Wn[rr][c];
    } else {
      const float* cp = p.ckpt + ((long)b * p.nck + ck) * DP * DP;
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr)
#pragma unroll
        for (int c = 0; c < NC; ++c) W[rr][c] = cp[(g * RPG + rr) * DP + tc + 16 * c];
    }
    load_next(max(ck - 1, 0));  // the previous chunk (for chunk 0, a reload)
    for (int tt = min(TTT_CK, p.T - t0) - 1; tt >= 0; --tt) {
      const int t = t0 + tt, par = t & 1;
      const long row0 = ((long)b * p.T + t) * D;
      float pq[NC], pk[NC], dse[RPG], sv[RPG];
#pragma unroll
      for (int c = 0; c < NC; ++c) pq[c] = pk[c] = 0.0f;
      float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr) {
        const int r = g * RPG + rr;
        const float dor = sdo[tt][r];
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int j = tc + 16 * c;
          dW[rr][c] = fmaf(dor, sq[tt][j], dW[rr][c]);
          pq[c] = fmaf(W[rr][c], dor, pq[c]);
          a = fmaf(dW[rr][c], sk[tt][j], a);
        }
        dse[rr] = -row16_sum(a);
        const float er = sr[tt][r], et = se[tt][r], x = sx[tt][r];
        const float derr = dse[rr] * et;
        if (tc == 0 && r < D) {
          st((TT*)p.deta, row0 + r, dse[rr] * er);
          st((TT*)p.dv, row0 + r, -derr);
        }
        agg[rr] = fmaf(derr, x, agg[rr]);
        agb[rr] += derr;
        const float dx = sg[r] * derr;
        s1 += dx;
        s2 = fmaf(dx, x, s2);
        dse[rr] = dx;  // keep dx for the LayerNorm backward below
        sv[rr] = et * er;
#pragma unroll
        for (int c = 0; c < NC; ++c) W[rr][c] = fmaf(sv[rr], sk[tt][tc + 16 * c], W[rr][c]);
      }
      if (tc == 0) {
        stat[par][g][0] = s1;
        stat[par][g][1] = s2;
      }
      __syncthreads();
      float m1 = 0.0f, m2 = 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        m1 += stat[par][u][0];
        m2 += stat[par][u][1];
      }
      m1 /= (float)D;
      m2 /= (float)D;
      const float rs = srs[tt];
#pragma unroll
      for (int rr = 0; rr < RPG; ++rr) {
        const int r = g * RPG + rr;
        const float dp = r < D ? rs * (dse[rr] - m1 - sx[tt][r] * m2) : 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const float kj = sk[tt][tc + 16 * c];
          pk[c] = fmaf(-dW[rr][c], sv[rr], fmaf(W[rr][c], dp, pk[c]));
          dW[rr][c] = fmaf(dp, kj, dW[rr][c]);
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        red[par][g][0][tc + 16 * c] = pq[c];
        red[par][g][1][tc + 16 * c] = pk[c];
      }
      __syncthreads();
      if (tid < 2 * DP) {
        const int qty = tid / DP, j = tid % DP;
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < 16; ++u) acc += red[par][u][qty][j];
        if (j < D) st((TT*)(qty == 0 ? p.dq : p.dk), row0 + j, acc);
      }
    }
    // the other stage was last read in the previous chunk, before the barrier that ended it
    store_next(max(ck - 1, 0), cb ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int rr = 0; rr < RPG; ++rr) {
    const int r = g * RPG + rr;
    if (r >= D) continue;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int j = tc + 16 * c;
      if (j < D) st((TT*)p.dw0, ((long)b * D + r) * D + j, dW[rr][c]);
    }
    if (tc == 0) {
      p.part_g[(long)b * D + r] = agg[rr];
      p.part_b[(long)b * D + r] = agb[rr];
    }
  }
}

// dln_g, dln_b: the per-batch partials added in batch order.
template <typename TT>
__global__ __launch_bounds__(256) void ttt_ln_reduce_kernel(const TArgs p, int batch) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= 2 * p.D) return;
  const int qty = e / p.D, j = e % p.D;
  const float* part = qty ? p.part_b : p.part_g;
  float acc = 0.0f;
  for (int b = 0; b < batch; ++b) acc += part[(long)b * p.D + j];
  st((TT*)(qty ? p.dln_b : p.dln_g), j, acc);
}

inline int ttt_pad(int d) { return d <= 16 ? 16 : d <= 32 ? 32 : d <= 64 ? 64 : 128; }
inline size_t ttt_align(size_t v) { return (v + 255) & ~(size_t)255; }

struct TWs {
  size_t ckpt, xh, err, rstd, part_g, part_b, total;
};

inline TWs ttt_ws(int batch, int seq, int d) {
  const size_t dp = ttt_pad(d), nck = (seq + TTT_CK - 1) / TTT_CK, bt = (size_t)batch * seq;
  TWs w{};
  size_t off = 0;
  w.ckpt = off;
  off += ttt_align((size_t)batch * nck * dp * dp * 4);
  w.xh = off;
  off += ttt_align(bt * d * 4);
  w.err = off;
  off += ttt_align(bt * d * 4);
  w.rstd = off;
  off += ttt_align(bt * 4);
  w.part_g = off;
  off += ttt_align((size_t)batch * d * 4);
  w.part_b = off;
  off += ttt_align((size_t)batch * d * 4);
  w.total = off;
  return w;
}

template <typename TT>
int ttt_launch(hipStream_t s, const TArgs& a, bool bwd, int batch) {
#define EDF_TTT_LAUNCH(DP)                                        \
  do {                                                            \
    if (bwd)                                                      \
      ttt_bwd_kernel<TT, DP><<<batch, 256, 0, s>>>(a);            \
    else                                                          \
      ttt_fwd_kernel<TT, DP><<<batch, 256, 0, s>>>(a);            \
  } while (0)
  if (a.D <= 16)
    EDF_TTT_LAUNCH(16);
  else if (a.D <= 32)
    EDF_TTT_LAUNCH(32);
  else if (a.D <= 64)
    EDF_TTT_LAUNCH(64);
  else
    EDF_TTT_LAUNCH(128);
#undef EDF_TTT_LAUNCH
  return check_launch(bwd ? "ttt backward" : "ttt");
}

int check_ttt(int batch, int seq, int inner, int dtype) {
  EDF_REQUIRE(batch > 0 && seq > 0 && inner > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(inner <= 128, EDF_ERR_UNSUPPORTED, "inner_size %d > 128 unsupported (reference TTT_MAX_INNER)", inner);
  return EDF_OK;
}

TArgs ttt_args(const void* q, const void* k, const void* v, const void* eta, const void* w0, const void* ln_g,
               const void* ln_b, int seq, int inner) {
  TArgs a{};
  a.q = q; a.k = k; a.v = v; a.eta = eta; a.w0 = w0; a.ln_g = ln_g; a.ln_b = ln_b;
  a.T = seq; a.D = inner; a.nck = (seq + TTT_CK - 1) / TTT_CK;
  return a;
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_fused_ttt_scan(void* stream, const void* q, const void* k, const void* v, const void* eta, const void* w0,
                       const void* ln_g, const void* ln_b, void* out, int batch, int seq_len, int inner_size,
                       int dtype) {
  using namespace edf;
  int rc = check_ttt(batch, seq_len, inner_size, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && eta && w0 && ln_g && ln_b && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  TArgs a = ttt_args(q, k, v, eta, w0, ln_g, ln_b, seq_len, inner_size);
  a.out = out;
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? ttt_launch<bf16>(s, a, false, batch) : ttt_launch<float>(s, a, false, batch);
}

size_t edf_ttt_scan_backward_workspace_bytes(int batch, int seq_len, int inner_size, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || inner_size <= 0) return 0;
  return edf::ttt_ws(batch, seq_len, inner_size).total;
}

// the backward proper; `context` (nullable) holds what a recording forward stored (W every
// TTT_CK steps, x_hat, err and 1/sigma per step), else a forward pass records it first
static int ttt_backward(void* stream, const void* q, const void* k, const void* v, const void* eta, const void* w0,
                        const void* ln_g, const void* ln_b, const void* grad_out, void* grad_q, void* grad_k,
                        void* grad_v, void* grad_eta, void* grad_w0, void* grad_ln_g, void* grad_ln_b,
                        const void* context, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                        int inner_size, int dtype) {
  using namespace edf;
  int rc = check_ttt(batch, seq_len, inner_size, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && eta && w0 && ln_g && ln_b && grad_out && grad_q && grad_k && grad_v && grad_eta &&
                  grad_w0 && grad_ln_g && grad_ln_b,
              EDF_ERR_INVALID_ARG, "null tensor pointer");
  const TWs w = ttt_ws(batch, seq_len, inner_size);
  EDF_REQUIRE(workspace && workspace_bytes >= w.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              w.total);
  char* ws = (char*)workspace;
  char* rec = context ? (char*)const_cast<void*>(context) : ws;  // the records: same layout either way
  TArgs a = ttt_args(q, k, v, eta, w0, ln_g, ln_b, seq_len, inner_size);
  a.ckpt = (float*)(rec + w.ckpt);
  a.xh = (float*)(rec + w.xh);
  a.err = (float*)(rec + w.err);
  a.rstd = (float*)(rec + w.rstd);
  a.part_g = (float*)(ws + w.part_g);
  a.part_b = (float*)(ws + w.part_b);
  TArgs f = a;  // forward re-run: checkpoints and per-step LayerNorm values, no output
  a.dout = grad_out;
  a.dq = grad_q; a.dk = grad_k; a.dv = grad_v; a.deta = grad_eta; a.dw0 = grad_w0;
  a.dln_g = grad_ln_g; a.dln_b = grad_ln_b;
  hipStream_t s = as_stream(stream);
  const unsigned gred = (unsigned)((2 * inner_size + 255) / 256);
  if (dtype == EDF_BF16) {
    if (!context && (rc = ttt_launch<bf16>(s, f, false, batch))) return rc;
    if ((rc = ttt_launch<bf16>(s, a, true, batch))) return rc;
    ttt_ln_reduce_kernel<bf16><<<gred, 256, 0, s>>>(a, batch);
  } else {
    if (!context && (rc = ttt_launch<float>(s, f, false, batch))) return rc;
    if ((rc = ttt_launch<float>(s, a, true, batch))) return rc;
    ttt_ln_reduce_kernel<float><<<gred, 256, 0, s>>>(a, batch);
  }
  return check_launch("ttt backward reduction");
}

int edf_fused_ttt_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* eta,
                                const void* w0, const void* ln_g, const void* ln_b, const void* grad_out,
                                void* grad_q, void* grad_k, void* grad_v, void* grad_eta, void* grad_w0,
                                void* grad_ln_g, void* grad_ln_b, void* workspace, size_t workspace_bytes,
                                int batch, int seq_len, int inner_size, int dtype) {
  return ttt_backward(stream, q, k, v, eta, w0, ln_g, ln_b, grad_out, grad_q, grad_k, grad_v, grad_eta, grad_w0,
                      grad_ln_g, grad_ln_b, nullptr, workspace, workspace_bytes, batch, seq_len, inner_size, dtype);
}

size_t edf_ttt_scan_context_bytes(int batch, int seq_len, int inner_size, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || inner_size <= 0) return 0;
  return edf::ttt_ws(batch, seq_len, inner_size).part_g;
}

int edf_fused_ttt_scan_with_context(void* stream, const void* q, const void* k, const void* v, const void* eta,
                                    const void* w0, const void* ln_g, const void* ln_b, void* out, void* context,
                                    size_t context_bytes, int batch, int seq_len, int inner_size, int dtype) {
  using namespace edf;
  int rc = check_ttt(batch, seq_len, inner_size, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && eta && w0 && ln_g && ln_b && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const TWs w = ttt_ws(batch, seq_len, inner_size);
  EDF_REQUIRE(context && context_bytes >= w.part_g, EDF_ERR_WORKSPACE, "context too small: need %zu bytes",
              w.part_g);
  char* rec = (char*)context;
  TArgs a = ttt_args(q, k, v, eta, w0, ln_g, ln_b, seq_len, inner_size);
  a.out = out;
  a.ckpt = (float*)(rec + w.ckpt);
  a.xh = (float*)(rec + w.xh);
  a.err = (float*)(rec + w.err);
  a.rstd = (float*)(rec + w.rstd);
  hipStream_t s = as_stream(stream);
  return dtype == EDF_BF16 ? ttt_launch<bf16>(s, a, false, batch) : ttt_launch<float>(s, a, false, batch);
}

int edf_fused_ttt_scan_backward_saved(void* stream, const void* q, const void* k, const void* v, const void* eta,
                                      const void* w0, const void* ln_g, const void* ln_b, const void* grad_out,
                                      void* grad_q, void* grad_k, void* grad_v, void* grad_eta, void* grad_w0,
                                      void* grad_ln_g, void* grad_ln_b, const void* context, size_t context_bytes,
                                      void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                      int inner_size, int dtype) {
  const size_t need = edf_ttt_scan_context_bytes(batch, seq_len, inner_size, dtype);
  EDF_REQUIRE(context && context_bytes >= need, EDF_ERR_WORKSPACE,
              "context too small: need the %zu bytes the forward filled", need);
  return ttt_backward(stream, q, k, v, eta, w0, ln_g, ln_b, grad_out, grad_q, grad_k, grad_v, grad_eta, grad_w0,
                      grad_ln_g, grad_ln_b, context, workspace, workspace_bytes, batch, seq_len, inner_size, dtype);
}

}  // extern "C"
