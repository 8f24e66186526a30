// DeltaProduct: n_h generalized-Householder delta-rule sub-steps per token, forward and
// backward (native/cuda/fused_delta_product_scan.cu, fused_delta_product_scan_backward.cu).
//
// Semantics, with S [d_v x d_k] per (batch, head) as in the delta rule kernels (the
// reference keeps the transpose, S_ref[key][value]):
//   per token t, for j in 0..n_h-1:  kn = k_tj / sqrt(|k_tj|^2 + 1e-6)
//                                    S  = S + beta_tj (v_tj - S kn) kn^T
//   o_raw[j] = sum_i S[i][j] q_t[i]  (the reference's S_ref q_t, a sum over value rows)
//   o_t = o_raw / sqrt(mean(o_raw^2) + 1e-6)
// k and v are [B, T, n_h, H, d], i.e. [B, T*n_h, H, d]: the sub-steps form one delta-rule
// sequence of T*n_h steps whose every n_h-th step emits an output.
//
// Layout of the work: as in the per-step delta kernels, a workgroup owns RB = 16 value
// rows of one head's state (lane (tr, tc) holds S[16 rb + tr][tc + 16 c]); the update
// and the retrieval S kn are row-local.  The output sums over ALL rows, so each row
// block writes a partial o_raw (its 16 rows summed in row order through an LDS tile) and
// a small kernel adds the d/16 partials in block order and applies the RMS norm.
// Backward: dO (the gradient at o_raw) is computed from the re-run forward's partials;
// dq_t = S_t dO and dv are row-local, the key and beta gradients sum over rows (per step
// through an LDS tile of the block's 16 rows, then row-block partials reduced in order and
// taken through the key normalization).  The forward
// states are checkpointed every CK sub-steps and recomputed per chunk, never inverted.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int DPR_CK = 16;  // sub-steps per staged chunk / checkpoint interval
constexpr int DPR_RB = 16;  // state rows per workgroup
constexpr float DPR_EPS = 1.0e-6f;  // fused_delta_product_scan.cu:38

struct DPArgs {
  const void *q, *k, *v, *beta, *dout;
  void *out, *dq, *dk, *dv, *dbeta;
  float* dO;      // [B*T*H][d]        gradient at the raw output (backward)
  float* ckpt;    // [BH][nck][DP*DP]  state after each chunk of sub-steps
  float* part_o;  // [nrb][B*T*H][d]   per-row-block partial raw output
  float* part_k;  // [nrb][B*TS*H][d]  per-row-block partial gradient of the normalized key
  float* part_b;  // [nrb][B*TS*H]     per-row-block partial dbeta
  int H, T, NH, TS, d, nck;  // TS = T * NH sub-steps
};

template <int DP>
struct DPStage {
  float k[DPR_CK][DP];          // normalized key per sub-step (0 beyond TS and d)
  float g[DPR_CK][DP];          // backward: dO of the token a sub-step closes, else 0
  float v[DPR_CK][DPR_RB];      // this block's value rows
  float q[DPR_CK][DPR_RB];      // q rows of the token a sub-step closes, else 0
  float b[DPR_CK];              // beta per sub-step
};

// The sub-steps of the chunk starting at t0 that close a token, as a bit mask over the
// chunk (bit tt = sub-step t0 + tt), and the token index of the chunk's first closing
// sub-step: one division per chunk (wave-uniform) instead of one per element or step.
struct Closing {
  unsigned mask;
  int tok0;
  EDF_DEVICE bool at(int tt) const { return (mask >> tt) & 1u; }
  EDF_DEVICE int tok(int tt) const { return tok0 + __builtin_popcount(mask & ((1u << tt) - 1u)); }
};

EDF_DEVICE Closing closing(const DPArgs& p, int t0) {
  Closing c;
  c.tok0 = t0 / p.NH;
  c.mask = 0u;
  int r = t0 - c.tok0 * p.NH;
  for (int tt = 0; tt < DPR_CK; ++tt) {
    if (r == p.NH - 1 && t0 + tt < p.TS) c.mask |= 1u << tt;
    r = r == p.NH - 1 ? 0 : r + 1;
  }
  return c;
}

EDF_DEVICE float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
  return x;
}

// A chunk's inputs are loaded a chunk ahead into registers (raw values from clamped
// addresses: no branch around a load, whose join would wait for it), then masked - zero
// beyond TS and d, q and dO only on sub-steps that close a token - and written to the
// other of two LDS stages once the current chunk is done; after a barrier each key row is
// normalized in place (16 lanes per sub-step, each over its own columns).  The loads'
// latency hides under the current chunk's sub-steps (forward: 2.39 -> 1.92 ms at
// 8x2048x2x8x128).
template <typename TT, int DP>
struct DPRegs {
  static constexpr int EK = DPR_CK * DP / 256;
  TT k[EK], v, q, b;
  float g[EK];
};

template <typename TT, int DP>
EDF_DEVICE void dp_load(DPRegs<TT, DP>& R, const DPArgs& p, long bh, int rb, int t0, bool grad) {
  const int b = (int)(bh / p.H), h = (int)(bh % p.H), d = p.d, tid = threadIdx.x;
  const Closing cl = closing(p, t0);
#pragma unroll
  for (int n = 0; n < DPRegs<TT, DP>::EK; ++n) {
    const int e = tid + 256 * n, tt = e / DP, j = min(e % DP, d - 1);
    R.k[n] = ((const TT*)p.k)[(((long)b * p.TS + min(t0 + tt, p.TS - 1)) * p.H + h) * d + j];
    if (grad) R.g[n] = p.dO[(((long)b * p.T + min(cl.tok(tt), p.T - 1)) * p.H + h) * d + j];
  }
  const int tt = tid / DPR_RB, i = min(rb * DPR_RB + tid % DPR_RB, d - 1);
  R.v = ((const TT*)p.v)[(((long)b * p.TS + min(t0 + tt, p.TS - 1)) * p.H + h) * d + i];
  R.q = ((const TT*)p.q)[(((long)b * p.T + min(cl.tok(tt), p.T - 1)) * p.H + h) * d + i];
  R.b = ((const TT*)p.beta)[((long)b * p.TS + min(t0 + tid % DPR_CK, p.TS - 1)) * p.H + h];
}

template <typename TT, int DP>
EDF_DEVICE void dp_store(DPStage<DP>& sm, const DPRegs<TT, DP>& R, const DPArgs& p, int rb, int t0, bool grad) {
  const int d = p.d, tid = threadIdx.x;
  const Closing cl = closing(p, t0);
#pragma unroll
  for (int n = 0; n < DPRegs<TT, DP>::EK; ++n) {
    const int e = tid + 256 * n, tt = e / DP, j = e % DP;
    sm.k[tt][j] = t0 + tt < p.TS && j < d ? to_f32(R.k[n]) : 0.0f;
    if (grad) sm.g[tt][j] = cl.at(tt) && j < d ? R.g[n] : 0.0f;
  }
  const int tt = tid / DPR_RB, ii = tid % DPR_RB, i = rb * DPR_RB + ii;
  sm.v[tt][ii] = t0 + tt < p.TS && i < d ? to_f32(R.v) : 0.0f;
  sm.q[tt][ii] = cl.at(tt) && i < d ? to_f32(R.q) : 0.0f;
  if (tid < DPR_CK) sm.b[tid] = t0 + tid < p.TS ? to_f32(R.b) : 0.0f;
}

template <int DP>
EDF_DEVICE void dp_normalize(DPStage<DP>& sm) {
  constexpr int NC = DP / 16;
  const int tt = threadIdx.x >> 4, l = threadIdx.x & 15;
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) ss = fmaf(sm.k[tt][l + 16 * c], sm.k[tt][l + 16 * c], ss);
  const float inv = 1.0f / sqrtf(row16_sum(ss) + DPR_EPS);
#pragma unroll
  for (int c = 0; c < NC; ++c) sm.k[tt][l + 16 * c] *= inv;
}

// The backward stages each chunk at its start. Its recomputed states hold too many
// registers for the forward's loads a chunk ahead: at D = 128 they cost it an occupancy
// level, and capped at two waves per SIMD (256 VGPRs, no spills) they gained nothing
// (backward call 6.67 ms either way at 8x2048x2x8x128).
template <typename TT, int DP>
EDF_DEVICE void stage(DPStage<DP>& sm, const DPArgs& p, long bh, int rb, int t0, bool grad) {
  constexpr int NC = DP / 16;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H), d = p.d;
  const int tid = threadIdx.x;
  const Closing cl = closing(p, t0);
  for (int e = tid; e < DPR_CK * DP; e += 256) {
    const int tt = e / DP, j = e % DP, s = t0 + tt;
    const bool ok = s < p.TS && j < d;
    sm.k[tt][j] = ok ? ld((const TT*)p.k, (((long)b * p.TS + s) * p.H + h) * d + j) : 0.0f;
    if (grad) {
      sm.g[tt][j] = cl.at(tt) && j < d ? p.dO[(((long)b * p.T + cl.tok(tt)) * p.H + h) * d + j] : 0.0f;
    }
  }
  for (int e = tid; e < DPR_CK * DPR_RB; e += 256) {
    const int tt = e / DPR_RB, ii = e % DPR_RB, i = rb * DPR_RB + ii, s = t0 + tt;
    const bool ok = s < p.TS && i < d;
    sm.v[tt][ii] = ok ? ld((const TT*)p.v, (((long)b * p.TS + s) * p.H + h) * d + i) : 0.0f;
    sm.q[tt][ii] = cl.at(tt) && i < d ? ld((const TT*)p.q, (((long)b * p.T + cl.tok(tt)) * p.H + h) * d + i) : 0.0f;
  }
  if (tid < DPR_CK) {
    const int s = t0 + tid;
    sm.b[tid] = s < p.TS ? ld((const TT*)p.beta, ((long)b * p.TS + s) * p.H + h) : 0.0f;
  }
  __syncthreads();
  // key normalization: 16 lanes per sub-step, each over its own columns
  {
    const int tt = tid >> 4, l = tid & 15;
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) ss = fmaf(sm.k[tt][l + 16 * c], sm.k[tt][l + 16 * c], ss);
    const float inv = 1.0f / sqrtf(row16_sum(ss) + DPR_EPS);
#pragma unroll
    for (int c = 0; c < NC; ++c) sm.k[tt][l + 16 * c] *= inv;
  }
}

// One sub-step of the lane's row segment: S = S + beta (v - S kn) kn^T.
template <int DP>
EDF_DEVICE void sub_step(float (&S)[DP / 16], const DPStage<DP>& sm, int tt, int tr, int tc) {
  constexpr int NC = DP / 16;
  float r = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) r = fmaf(S[c], sm.k[tt][tc + 16 * c], r);
  const float e = sm.b[tt] * (sm.v[tt][tr] - row16_sum(r));
#pragma unroll
  for (int c = 0; c < NC; ++c) S[c] = fmaf(e, sm.k[tt][tc + 16 * c], S[c]);
}

template <typename TT, int DP>
__global__ __launch_bounds__(256) void dp_fwd_kernel(const DPArgs p) {
  constexpr int NC = DP / 16;
  __shared__ DPStage<DP> sms[2];
  __shared__ float redo[DPR_RB][row16_stride(DP)];  // a closing sub-step's per-row output terms
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long bh = blockIdx.x;
  const int rb = blockIdx.y, i = rb * DPR_RB + tr;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const long nbth = (long)gridDim.x * p.T;
  const int nch = (p.TS + DPR_CK - 1) / DPR_CK;
  float S[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) S[c] = 0.0f;
  DPRegs<TT, DP> G;
  dp_load<TT, DP>(G, p, bh, rb, 0, false);
  dp_store<TT, DP>(sms[0], G, p, rb, 0, false);
  __syncthreads();
  dp_normalize<DP>(sms[0]);
  __syncthreads();
  for (int chn = 0; chn < nch; ++chn) {
    const int t0 = chn * DPR_CK;
    const DPStage<DP>& sm = sms[chn & 1];
    // the next chunk's inputs load under this chunk's sub-steps (past the last: a reload)
    dp_load<TT, DP>(G, p, bh, rb, min(t0 + DPR_CK, (nch - 1) * DPR_CK), false);
    const Closing cl = closing(p, t0);
#pragma unroll
    for (int tt = 0; tt < DPR_CK; ++tt) {  // padding past TS: identity sub-steps, never closing
      sub_step<DP>(S, sm, tt, tr, tc);
      if (p.part_o != nullptr && cl.at(tt)) {  // the block's 16 rows summed in row order
        const float qi = sm.q[tt][tr];
#pragma unroll
        for (int c = 0; c < NC; ++c) redo[tr][tc + 16 * c] = S[c] * qi;
        __syncthreads();
        const long bth = ((long)b * p.T + cl.tok(tt)) * p.H + h;
        for (int j = tid; j < p.d; j += 256) {
          float acc = 0.0f;
#pragma unroll
          for (int m = 0; m < DPR_RB; ++m) acc += redo[m][j];
          p.part_o[((long)rb * nbth + bth) * p.d + j] = acc;
        }
        __syncthreads();
      }
    }
    if (p.ckpt != nullptr) {
      float* cp = p.ckpt + ((long)bh * p.nck + t0 / DPR_CK) * DP * DP + (long)i * DP + tc;
#pragma unroll
      for (int c = 0; c < NC; ++c) cp[16 * c] = S[c];
    }
    // the other stage was last read in the previous chunk, before the barriers below it
    dp_store<TT, DP>(sms[(chn + 1) & 1], G, p, rb, t0 + DPR_CK, false);
    __syncthreads();
    dp_normalize<DP>(sms[(chn + 1) & 1]);
    __syncthreads();
  }
}

// o_raw = the row-block partials added in block order; forward: out = RMS_norm(o_raw);
// backward: dO = dout / r - o_raw (dout . o_raw) / (d r^3).  One wave per (b, t, h).
template <typename TT>
__global__ __launch_bounds__(256) void dp_finish_kernel(const DPArgs p, long nbth, int nrb, int backward) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nbth) return;
  const int lane = threadIdx.x & 63, d = p.d;
  // column of element u of this lane: 2 lane + u when d is even (8-byte loads of the
  // partials), lane + 64 u otherwise; the row blocks are added in the same order either way
  const bool pair = d % 2 == 0;
  auto col = [&](int u) { return pair ? 2 * lane + u : lane + 64 * u; };
  float o[2], g[2];
  if (pair) {
    float2 acc = make_float2(0.0f, 0.0f);
    if (2 * lane < d)
      for (int r = 0; r < nrb; ++r) {
        const float2 v = *reinterpret_cast<const float2*>(p.part_o + ((long)r * nbth + row) * d + 2 * lane);
        acc.x += v.x, acc.y += v.y;
      }
    o[0] = acc.x, o[1] = acc.y;
  } else {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float acc = 0.0f;
      if (col(u) < d)
        for (int r = 0; r < nrb; ++r) acc += p.part_o[((long)r * nbth + row) * d + col(u)];
      o[u] = acc;
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) g[u] = backward && col(u) < d ? ld((const TT*)p.dout, row * d + col(u)) : 0.0f;
  const float ms = wave_sum(o[0] * o[0] + o[1] * o[1]) / (float)d;
  const float rinv = 1.0f / sqrtf(ms + DPR_EPS);
  if (!backward) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      if (col(u) < d) st((TT*)p.out, row * d + col(u), o[u] * rinv);
    return;
  }
  const float dot = wave_sum(g[0] * o[0] + g[1] * o[1]);
  const float c = dot * rinv * rinv * rinv / (float)d;
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (col(u) < d) p.dO[row * d + col(u)] = g[u] * rinv - o[u] * c;
}

// Backward over chunks of sub-steps in reverse.  Per sub-step (S_p the state before it,
// S_n = S_p + be kn^T, dtot = dS + q dO^T on a token's last sub-step):
//   dq = S_n dO (token's last sub-step), ds_k = dtot kn, dv = beta ds_k, dbeta = err . ds_k,
//   dkn = dtot^T be - S_p^T (beta ds_k), dS <- dtot - beta ds_k kn^T, err = v - S_p kn, be = beta err.
//
// The sums over the block's rows (the key-gradient terms, one per column, and the per-head
// dbeta term, one per row) leave the sub-steps' dependency chain as in the delta rule's
// per-step backward: each wave adds its four rows' terms in registers (rows4_scatter) into a
// per-sub-step slot of an LDS tile, and every FS sub-steps one barrier pair adds the four
// waves' slots in wave order and stores the partials.
// BUF: dv and dq go through buffer resources over the batch row, every lane storing at an
// offset with bit 31 set where the lane or the sub-step stores nothing (OR, not add: no
// offset wraps back into range), so the unrolled sub-steps hold no branch.
template <typename TT, int DP, bool BUF>
__global__ __launch_bounds__(256) void dp_bwd_kernel(const DPArgs p) {
  constexpr int NC = DP / 16;
  constexpr int FS = 8;                 // sub-steps per flush of the row sums
  constexpr int NG = (NC + 3) / 4;      // rows4_scatter groups of the lane's NC column terms
  static_assert(DPR_CK % FS == 0, "flushes split the chunk");
  __shared__ DPStage<DP> sm;
  __shared__ float wsum[FS][4][NG][64];  // [slot][wave][group][lane]: four-row sums
  __shared__ float redb[FS][DPR_RB];     // [slot][row]: dbeta terms
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int w = tid >> 6, lane = tid & 63;
  const long bh = blockIdx.x;
  const int rb = blockIdx.y, i = rb * DPR_RB + tr;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const long nbts = (long)gridDim.x * p.TS;
  const long vrow = (long)p.TS * p.H * p.d, qrow = (long)p.T * p.H * p.d;  // elements per batch row
  const rsrc_t r_dv = make_rsrc(BUF ? (const TT*)p.dv + (long)b * vrow : (const TT*)p.k,
                                BUF ? (unsigned)(vrow * sizeof(TT)) : 0u);
  const rsrc_t r_dq = make_rsrc(BUF ? (const TT*)p.dq + (long)b * qrow : (const TT*)p.k,
                                BUF ? (unsigned)(qrow * sizeof(TT)) : 0u);
  const unsigned lbase = (unsigned)(((long)h * p.d + i) * sizeof(TT));
  const unsigned lpoison = (tc == 0 && i < p.d) ? 0u : OOB_OFF;
  const unsigned ostep = (unsigned)((long)p.H * p.d * sizeof(TT));
  float dS[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dS[c] = 0.0f;

  for (int ck = p.nck - 1; ck >= 0; --ck) {
    const int t0 = ck * DPR_CK;
    __syncthreads();
    stage<TT, DP>(sm, p, bh, rb, t0, true);
    __syncthreads();
    const Closing cl = closing(p, t0);
    float Sl[DPR_CK][NC];  // Sl[tt] = state before sub-step t0 + tt
    {
      float S[NC];
      const float* cp = p.ckpt + ((long)bh * p.nck + max(ck - 1, 0)) * DP * DP + (long)i * DP + tc;
#pragma unroll
      for (int c = 0; c < NC; ++c) S[c] = ck > 0 ? cp[16 * c] : 0.0f;
#pragma unroll
      for (int tt = 0; tt < DPR_CK; ++tt) {
#pragma unroll
        for (int c = 0; c < NC; ++c) Sl[tt][c] = S[c];
        sub_step<DP>(S, sm, tt, tr, tc);
      }
    }
#pragma unroll
    for (int tt = DPR_CK - 1; tt >= 0; --tt) {
      const int s = t0 + tt;
      const float qi = sm.q[tt][tr], bi = sm.b[tt];
      float r = 0.0f, sk = 0.0f, dtot[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float kj = sm.k[tt][tc + 16 * c];
        dtot[c] = fmaf(qi, sm.g[tt][tc + 16 * c], dS[c]);
        r = fmaf(Sl[tt][c], kj, r);
        sk = fmaf(dtot[c], kj, sk);
      }
      r = row16_sum(r);
      sk = row16_sum(sk);
      const float err = sm.v[tt][tr] - r;
      const float be = bi * err, bdk = bi * sk;
      float pq = 0.0f, vals[4 * NG];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float kj = sm.k[tt][tc + 16 * c];
        pq = fmaf(fmaf(be, kj, Sl[tt][c]), sm.g[tt][tc + 16 * c], pq);
        vals[c] = fmaf(dtot[c], be, -Sl[tt][c] * bdk);
        dS[c] = fmaf(-bdk, kj, dtot[c]);
      }
#pragma unroll
      for (int k = NC; k < 4 * NG; ++k) vals[k] = 0.0f;
      const int slot = tt % FS;
#pragma unroll
      for (int g = 0; g < NG; ++g)
        wsum[slot][w][g][lane] = rows4_scatter(vals[4 * g], vals[4 * g + 1], vals[4 * g + 2], vals[4 * g + 3]);
      pq = row16_sum(pq);
      if constexpr (BUF) {
        redb[slot][tr] = i < p.d ? err * sk : 0.0f;  // the row's 16 lanes hold the same value
        // sub-steps past TS land past the batch row
        bstore<TT>(r_dv, (lbase + (unsigned)s * ostep) | lpoison, bdk);
        bstore<TT>(r_dq, (lbase + (unsigned)cl.tok(tt) * ostep) | lpoison | (cl.at(tt) ? 0u : OOB_OFF), pq);
      } else {
        if (tc == 0) redb[slot][tr] = i < p.d ? err * sk : 0.0f;
        if (s < p.TS && tc == 0 && i < p.d) {
          st((TT*)p.dv, (((long)b * p.TS + s) * p.H + h) * p.d + i, bdk);
          if (cl.at(tt)) st((TT*)p.dq, (((long)b * p.T + cl.tok(tt)) * p.H + h) * p.d + i, pq);
        }
      }
      if (slot == 0) {  // sub-steps s .. s + FS - 1 are in the slots: sum the waves, store
        __syncthreads();
        for (int e = tid; e < FS * DP; e += 256) {
          const int sl = e / DP, j = e % DP;
          const int g = (j >> 4) >> 2, src = 16 * rows4_item((j >> 4) & 3) + (j & 15);
          const float acc = ((wsum[sl][0][g][src] + wsum[sl][1][g][src]) + wsum[sl][2][g][src]) + wsum[sl][3][g][src];
          if (s + sl < p.TS && j < p.d) p.part_k[((long)rb * nbts + ((long)b * p.TS + s + sl) * p.H + h) * p.d + j] = acc;
        }
        if (tid < FS) {
          float acc = 0.0f;
#pragma unroll
          for (int m = 0; m < DPR_RB; ++m) acc += redb[tid][m];
          if (s + tid < p.TS) p.part_b[(long)rb * nbts + ((long)b * p.TS + s + tid) * p.H + h] = acc;
        }
        __syncthreads();
      }
    }
  }
}

// dk = the row-block partials of dkn added in block order, through the key normalization
// dk = (dkn - kn (dkn . kn)) / sqrt(|k|^2 + 1e-6); dbeta likewise summed.  One wave per
// (b, sub-step, h).
template <typename TT>
__global__ __launch_bounds__(256) void dp_reduce_kernel(const DPArgs p, long nbts, int nrb) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nbts) return;
  const int lane = threadIdx.x & 63, d = p.d;
  float g[2], kv[2];
  if (d % 2 == 0) {  // lane owns columns 2 lane, 2 lane + 1: 8-byte loads, the same order of sums
    const int j = 2 * lane;
    float2 acc = make_float2(0.0f, 0.0f);
    if (j < d)
      for (int r = 0; r < nrb; ++r) {
        const float2 v = *reinterpret_cast<const float2*>(p.part_k + ((long)r * nbts + row) * d + j);
        acc.x += v.x, acc.y += v.y;
      }
    g[0] = acc.x, g[1] = acc.y;
    kv[0] = j < d ? ld((const TT*)p.k, row * d + j) : 0.0f;
    kv[1] = j < d ? ld((const TT*)p.k, row * d + j + 1) : 0.0f;
  } else {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = lane + 64 * u;
      float acc = 0.0f;
      if (j < d)
        for (int r = 0; r < nrb; ++r) acc += p.part_k[((long)r * nbts + row) * d + j];
      g[u] = acc;
      kv[u] = j < d ? ld((const TT*)p.k, row * d + j) : 0.0f;
    }
  }
  const float inv = 1.0f / sqrtf(wave_sum(kv[0] * kv[0] + kv[1] * kv[1]) + DPR_EPS);
  const float dot = wave_sum(g[0] * kv[0] + g[1] * kv[1]) * inv;  // dkn . kn
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int j = d % 2 == 0 ? 2 * lane + u : lane + 64 * u;
    if (j < d) st((TT*)p.dk, row * d + j, (g[u] - kv[u] * inv * dot) * inv);
  }
  if (lane == 0) {
    float acc = 0.0f;
    for (int r = 0; r < nrb; ++r) acc += p.part_b[(long)r * nbts + row];
    st((TT*)p.dbeta, row, acc);
  }
}

inline int dp_pad(int d) { return d <= 16 ? 16 : d <= 32 ? 32 : d <= 64 ? 64 : 128; }
inline size_t dp_align(size_t v) { return (v + 255) & ~(size_t)255; }

struct DPWs {
  size_t part_o, ckpt, dO, part_k, part_b, total;
};

inline DPWs dp_ws(int batch, int seq, int nh, int heads, int d, bool backward) {
  const size_t dp = dp_pad(d), nrb = dp / DPR_RB, ts = (size_t)seq * nh;
  const size_t bh = (size_t)batch * heads, nbth = bh * seq, nbts = bh * ts;
  const size_t nck = (ts + DPR_CK - 1) / DPR_CK;
  DPWs w{};
  size_t off = 0;
  w.part_o = off;
  off += dp_align(nrb * nbth * d * 4);
  if (backward) {
    w.ckpt = off;
    off += dp_align(bh * nck * dp * dp * 4);
    w.dO = off;
    off += dp_align(nbth * d * 4);
    w.part_k = off;
    off += dp_align(nrb * nbts * d * 4);
    w.part_b = off;
    off += dp_align(nrb * nbts * 4);
  }
  w.total = off;
  return w;
}

template <typename TT>
int dp_launch(hipStream_t s, const DPArgs& a, bool bwd, int BH) {
  const int d = a.d;
#define EDF_DP_LAUNCH(DP)                                       \
  do {                                                          \
    const dim3 grid(BH, DP / DPR_RB);                           \
    if (bwd && (long)(a.TS + DPR_CK) * a.H * a.d * (long)sizeof(TT) < (1L << 31)) \
      dp_bwd_kernel<TT, DP, true><<<grid, 256, 0, s>>>(a);      \
    else if (bwd)                                               \
      dp_bwd_kernel<TT, DP, false><<<grid, 256, 0, s>>>(a);     \
    else                                                        \
      dp_fwd_kernel<TT, DP><<<grid, 256, 0, s>>>(a);            \
  } while (0)
  if (d <= 16)
    EDF_DP_LAUNCH(16);
  else if (d <= 32)
    EDF_DP_LAUNCH(32);
  else if (d <= 64)
    EDF_DP_LAUNCH(64);
  else
    EDF_DP_LAUNCH(128);
#undef EDF_DP_LAUNCH
  return check_launch(bwd ? "delta product backward" : "delta product");
}

int check_dp(int batch, int seq, int nh, int heads, int d, int dtype) {
  EDF_REQUIRE(batch > 0 && seq > 0 && nh > 0 && heads > 0 && d > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(d <= 128, EDF_ERR_UNSUPPORTED, "head_dim %d > 128 unsupported", d);
  EDF_REQUIRE((long)seq * nh < (1L << 30), EDF_ERR_UNSUPPORTED, "seq_len * num_householder too large");
  return EDF_OK;
}

DPArgs dp_args(const void* q, const void* k, const void* v, const void* beta, int seq, int nh, int heads, int d) {
  DPArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta;
  a.H = heads; a.T = seq; a.NH = nh; a.TS = seq * nh; a.d = d;
  a.nck = (a.TS + DPR_CK - 1) / DPR_CK;
  return a;
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_delta_product_workspace_bytes(int batch, int seq_len, int num_householder, int num_heads, int head_dim,
                                         int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_householder <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return edf::dp_ws(batch, seq_len, num_householder, num_heads, head_dim, false).total;
}

size_t edf_delta_product_backward_workspace_bytes(int batch, int seq_len, int num_householder, int num_heads,
                                                  int head_dim, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_householder <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return edf::dp_ws(batch, seq_len, num_householder, num_heads, head_dim, true).total;
}

int edf_fused_delta_product_scan(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                 void* out, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                 int num_householder, int num_heads, int head_dim, int dtype) {
  using namespace edf;
  int rc = check_dp(batch, seq_len, num_householder, num_heads, head_dim, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && beta && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const DPWs w = dp_ws(batch, seq_len, num_householder, num_heads, head_dim, false);
  EDF_REQUIRE(workspace && workspace_bytes >= w.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              w.total);
  DPArgs a = dp_args(q, k, v, beta, seq_len, num_householder, num_heads, head_dim);
  a.out = out;
  a.part_o = (float*)((char*)workspace + w.part_o);
  const int bh = batch * num_heads, nrb = dp_pad(head_dim) / DPR_RB;
  const long nbth = (long)bh * seq_len;
  hipStream_t s = as_stream(stream);
  const unsigned grows = (unsigned)((nbth + 3) / 4);
  if (dtype == EDF_BF16) {
    rc = dp_launch<bf16>(s, a, false, bh);
    if (rc) return rc;
    dp_finish_kernel<bf16><<<grows, 256, 0, s>>>(a, nbth, nrb, 0);
  } else {
    rc = dp_launch<float>(s, a, false, bh);
    if (rc) return rc;
    dp_finish_kernel<float><<<grows, 256, 0, s>>>(a, nbth, nrb, 0);
  }
  return check_launch("delta product output norm");
}

// the backward proper; `context` (nullable) holds the row-block output partials and the
// state checkpoints a recording forward left, else a forward pass recomputes them
static int dp_backward(void* stream, const void* q, const void* k, const void* v, const void* beta,
                       const void* grad_out, void* grad_q, void* grad_k, void* grad_v, void* grad_beta,
                       const void* context, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                       int num_householder, int num_heads, int head_dim, int dtype) {
  using namespace edf;
  int rc = check_dp(batch, seq_len, num_householder, num_heads, head_dim, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && beta && grad_out && grad_q && grad_k && grad_v && grad_beta, EDF_ERR_INVALID_ARG,
              "null tensor pointer");
  const DPWs w = dp_ws(batch, seq_len, num_householder, num_heads, head_dim, true);
  EDF_REQUIRE(workspace && workspace_bytes >= w.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              w.total);
  char* ws = (char*)workspace;
  char* rec = context ? (char*)const_cast<void*>(context) : ws;  // partials and checkpoints: same layout
  DPArgs a = dp_args(q, k, v, beta, seq_len, num_householder, num_heads, head_dim);
  a.dout = grad_out;
  a.dq = grad_q; a.dk = grad_k; a.dv = grad_v; a.dbeta = grad_beta;
  a.part_o = (float*)(rec + w.part_o);
  a.ckpt = (float*)(rec + w.ckpt);
  a.dO = (float*)(ws + w.dO);
  a.part_k = (float*)(ws + w.part_k);
  a.part_b = (float*)(ws + w.part_b);
  const int bh = batch * num_heads, nrb = dp_pad(head_dim) / DPR_RB;
  const long nbth = (long)bh * seq_len, nbts = nbth * num_householder;
  hipStream_t s = as_stream(stream);
  const unsigned grows = (unsigned)((nbth + 3) / 4), gsub = (unsigned)((nbts + 3) / 4);
  if (dtype == EDF_BF16) {
    if (!context && (rc = dp_launch<bf16>(s, a, false, bh))) return rc;
    dp_finish_kernel<bf16><<<grows, 256, 0, s>>>(a, nbth, nrb, 1);
    if ((rc = dp_launch<bf16>(s, a, true, bh))) return rc;
    dp_reduce_kernel<bf16><<<gsub, 256, 0, s>>>(a, nbts, nrb);
  } else {
    if (!context && (rc = dp_launch<float>(s, a, false, bh))) return rc;
    dp_finish_kernel<float><<<grows, 256, 0, s>>>(a, nbth, nrb, 1);
    if ((rc = dp_launch<float>(s, a, true, bh))) return rc;
    dp_reduce_kernel<float><<<gsub, 256, 0, s>>>(a, nbts, nrb);
  }
  return check_launch("delta product backward reduction");
}

int edf_fused_delta_product_scan_backward(void* stream, const void* q, const void* k, const void* v,
                                          const void* beta, const void* forward_out, const void* grad_out,
                                          void* grad_q, void* grad_k, void* grad_v, void* grad_beta, void* workspace,
                                          size_t workspace_bytes, int batch, int seq_len, int num_householder,
                                          int num_heads, int head_dim, int dtype) {
  (void)forward_out;  // the raw output and its norm are recomputed from the inputs
  return dp_backward(stream, q, k, v, beta, grad_out, grad_q, grad_k, grad_v, grad_beta, nullptr, workspace,
                     workspace_bytes, batch, seq_len, num_householder, num_heads, head_dim, dtype);
}

size_t edf_delta_product_context_bytes(int batch, int seq_len, int num_householder, int num_heads, int head_dim,
                                       int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_householder <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return edf::dp_ws(batch, seq_len, num_householder, num_heads, head_dim, true).dO;
}

int edf_fused_delta_product_scan_with_context(void* stream, const void* q, const void* k, const void* v,
                                              const void* beta, void* out, void* context, size_t context_bytes,
                                              int batch, int seq_len, int num_householder, int num_heads,
                                              int head_dim, int dtype) {
  using namespace edf;
  int rc = check_dp(batch, seq_len, num_householder, num_heads, head_dim, dtype);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && beta && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const DPWs w = dp_ws(batch, seq_len, num_householder, num_heads, head_dim, true);
  EDF_REQUIRE(context && context_bytes >= w.dO, EDF_ERR_WORKSPACE, "context too small: need %zu bytes", w.dO);
  DPArgs a = dp_args(q, k, v, beta, seq_len, num_householder, num_heads, head_dim);
  a.out = out;
  a.part_o = (float*)((char*)context + w.part_o);
  a.ckpt = (float*)((char*)context + w.ckpt);
  const int bh = batch * num_heads, nrb = dp_pad(head_dim) / DPR_RB;
  const long nbth = (long)bh * seq_len;
  hipStream_t s = as_stream(stream);
  const unsigned grows = (unsigned)((nbth + 3) / 4);
  if (dtype == EDF_BF16) {
    if ((rc = dp_launch<bf16>(s, a, false, bh))) return rc;
    dp_finish_kernel<bf16><<<grows, 256, 0, s>>>(a, nbth, nrb, 0);
  } else {
    if ((rc = dp_launch<float>(s, a, false, bh))) return rc;
    dp_finish_kernel<float><<<grows, 256, 0, s>>>(a, nbth, nrb, 0);
  }
  return check_launch("delta product output norm");
}

int edf_fused_delta_product_scan_backward_saved(void* stream, const void* q, const void* k, const void* v,
                                                const void* beta, const void* grad_out, void* grad_q, void* grad_k,
                                                void* grad_v, void* grad_beta, const void* context,
                                                size_t context_bytes, void* workspace, size_t workspace_bytes,
                                                int batch, int seq_len, int num_householder, int num_heads,
                                                int head_dim, int dtype) {
  const size_t need = edf_delta_product_context_bytes(batch, seq_len, num_householder, num_heads, head_dim, dtype);
  EDF_REQUIRE(context && context_bytes >= need, EDF_ERR_WORKSPACE,
              "context too small: need the %zu bytes the forward filled", need);
  return dp_backward(stream, q, k, v, beta, grad_out, grad_q, grad_k, grad_v, grad_beta, context, workspace,
                     workspace_bytes, batch, seq_len, num_householder, num_heads, head_dim, dtype);
}

}  // extern "C"
