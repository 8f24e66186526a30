// Delta rule (DeltaNet / GatedDeltaNet), step-by-step recurrence, forward and backward.
//
// Semantics (reference):
//   S_g = alpha_t S;  r = S_g k_t;  S = S_g + diag(beta_t)(v_t - r) k_t^T;  o_t = S q_t
//   S is [d_v x d_k] per (batch, head); beta per element [B,T,H,d] (one gate per value
//   row, lib/edifice/recurrent/delta_net.ex:231-273, native/cuda/fused_delta_rule_scan.cu:146-154)
//   or per head [B,T,H]; alpha per head [B,T,H] or absent
//   (lib/edifice/recurrent/gated_delta_net.ex:300-353), or (KDA) a log-space decay per
//   value row [B,T,H,d], S_g = diag(exp(alpha_t)) S (native/cuda/fused_kda_scan.cu:1-24,
//   lib/edifice/cuda/fused_scan.ex:2632-2665; d alpha_i = exp(alpha_i) sum_j dS_g S_p).
//   Backward: lib/edifice/cuda/fused_scan.ex:1257-1431 (dq = S_t^T do, ds_k = dS_tot k,
//   dv = beta ds_k, dbeta = err ds_k, dk = dS_tot^T (beta err) - S_g^T (beta ds_k),
//   dalpha = sum(dS_to_decayed * S_prev), dS_prev = alpha dS_to_decayed).
//
// This is the exact per-step path: it supports per-element beta (where each row of S
// has its own gate, so the chunked UT form of the per-head path does not apply),
// float32 I/O and any head_dim <= 128.
//
// Rows of S evolve independently given k, q, alpha and the row's beta, so a workgroup
// owns one block of RB = 16 rows of one (batch, head) state (DP / 16 workgroups per
// head): lane (tr, tc) holds S[16 rb + tr][tc + 16 c], row sums are reductions inside a
// 16-lane DPP row, and only the backward's sums over rows (dq, dk, dalpha and a per-head
// dbeta) cross workgroups: each row block writes its partial sums and a small kernel adds
// the DP / 16 partials in a fixed order (deterministic, no atomics).
// The backward does not invert the update (the reference divides by alpha): the
// forward states are checkpointed every CK steps and each chunk's CK states are
// recomputed into registers (16 x DP/16 floats per lane) before its reverse sweep.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int CK = 16;  // steps per staged chunk / checkpoint interval
constexpr int RB = 16;  // state rows per workgroup

struct DRArgs {
  const void *q, *k, *v, *beta, *alpha, *dout;
  void *out, *dq, *dk, *dv, *dbeta, *dalpha;
  float* ckpt;    // [BH][nck][DP*DP] state after each chunk
  float* part_q;  // [nrb][B*T*H][d]   per-row-block partial dq
  float* part_k;  // [nrb][B*T*H][d]   per-row-block partial dk
  float* part_a;  // [nrb][B*T*H]      per-row-block partial dalpha
  float* part_b;  // [nrb][B*T*H]      per-row-block partial per-head dbeta
  int H, T, d, beta_per_head, nck;
  int alpha_per_row;  // KDA: alpha [B,T,H,d] in log space, one decay per value row
};

// One chunk of inputs: k and q over all DP columns, v, beta, the decay (and dout) for this
// workgroup's RB rows; zero beyond T and beyond d, decay 1 beyond T, so padding steps are
// identities of the recurrence and of its adjoint.
template <int DP>
struct Stage {
  float k[CK][DP], q[CK][DP], v[CK][RB], b[CK][RB], go[CK][RB];
  float a[CK][RB];
};

// A chunk's inputs are loaded a chunk ahead into registers (raw values from clamped
// addresses: no branch around a load, whose join would wait for it), then masked (zero
// beyond T and beyond d, decay 1 beyond T), converted and written to the other of two LDS
// stages once the current chunk's steps are done: one barrier per chunk, and the loads'
// latency hides under 16 steps (staging the chunk at its start, between two barriers,
// exposed it: forward 883 -> 494 us, backward 2843 -> 2180 us at 8x2048x8x128).
template <typename TT, int DP>
struct StageRegs {
  static constexpr int EK = CK * DP / 256;
  TT k[EK], q[EK], v, b, go, a;
};

template <typename TT, int DP>
EDF_DEVICE void load_chunk(StageRegs<TT, DP>& R, const DRArgs& p, long bh, int rb, int t0, bool with_dout) {
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int d = p.d;
#pragma unroll
  for (int n = 0; n < StageRegs<TT, DP>::EK; ++n) {
    const int e = threadIdx.x + 256 * n, tt = e / DP, j = e % DP;
    const long idx = (((long)b * p.T + min(t0 + tt, p.T - 1)) * p.H + h) * d + min(j, d - 1);
    R.k[n] = ((const TT*)p.k)[idx];
    R.q[n] = ((const TT*)p.q)[idx];
  }
  const int tt = threadIdx.x / RB, i = rb * RB + threadIdx.x % RB;
  const long bth = ((long)b * p.T + min(t0 + tt, p.T - 1)) * p.H + h;
  const long idx = bth * d + min(i, d - 1);
  R.v = ((const TT*)p.v)[idx];
  R.b = ((const TT*)p.beta)[p.beta_per_head ? bth : idx];
  if (with_dout) R.go = ((const TT*)p.dout)[idx];
  if (p.alpha != nullptr) R.a = ((const TT*)p.alpha)[p.alpha_per_row ? idx : bth];
}

template <typename TT, int DP>
EDF_DEVICE void store_chunk(Stage<DP>& sm, const StageRegs<TT, DP>& R, const DRArgs& p, int rb, int t0,
                            bool with_dout) {
  const int d = p.d;
#pragma unroll
  for (int n = 0; n < StageRegs<TT, DP>::EK; ++n) {
    const int e = threadIdx.x + 256 * n, tt = e / DP, j = e % DP;
    const bool ok = t0 + tt < p.T && j < d;
    sm.k[tt][j] = ok ? to_f32(R.k[n]) : 0.0f;
    sm.q[tt][j] = ok ? to_f32(R.q[n]) : 0.0f;
  }
  const int tt = threadIdx.x / RB, ii = threadIdx.x % RB, i = rb * RB + ii;
  const bool ok = t0 + tt < p.T && i < d;
  sm.v[tt][ii] = ok ? to_f32(R.v) : 0.0f;
  sm.b[tt][ii] = ok ? to_f32(R.b) : 0.0f;
  if (with_dout) sm.go[tt][ii] = ok ? to_f32(R.go) : 0.0f;
  float av = 1.0f;
  if (p.alpha != nullptr && ok) av = p.alpha_per_row ? __expf(to_f32(R.a)) : to_f32(R.a);
  sm.a[tt][ii] = av;
}

// One forward step of the lane's row segment: S = a S + beta (v - a S k) k^T.  DECAY = false
// (DeltaNet: no alpha, a = 1) compiles the decay multiplies out.
template <int DP, bool DECAY>
EDF_DEVICE void fwd_step(float (&S)[DP / 16], const Stage<DP>& sm, int tt, int tr, int tc) {
  constexpr int NC = DP / 16;
  const float at = DECAY ? sm.a[tt][tr] : 1.0f;
  float r = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) r = fmaf(S[c], sm.k[tt][tc + 16 * c], r);
  r = row16_sum(r) * at;
  const float e = sm.b[tt][tr] * (sm.v[tt][tr] - r);
#pragma unroll
  for (int c = 0; c < NC; ++c) S[c] = fmaf(e, sm.k[tt][tc + 16 * c], at * S[c]);
}

// OUTM: 0 no output (p.out null), 1 output stored by the row's lane 0 (tensors of 2 GiB per
// batch row and more), 2 output through a buffer resource over the batch row, every lane
// storing (lanes other than the row's lane 0, rows past d and steps past T at an offset the
// hardware drops): no branch in the unrolled steps, which a per-step branch splits into
// basic blocks, each waiting for its own LDS reads.
template <typename TT, int DP, bool DECAY, int OUTM>
__global__ __launch_bounds__(256) void dr_seq_fwd_kernel(const DRArgs p) {
  constexpr int NC = DP / 16;
  __shared__ Stage<DP> sms[2];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long bh = blockIdx.x;
  const int rb = blockIdx.y, i = rb * RB + tr;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int nch = (p.T + CK - 1) / CK;
  const long rowel = (long)p.T * p.H * p.d;  // output elements of one batch row
  const rsrc_t r_out = make_rsrc(OUTM == 2 ? (const TT*)p.out + (long)b * rowel : (const TT*)p.k,
                                 OUTM == 2 ? (unsigned)(rowel * sizeof(TT)) : 0u);
  const bool orow = tc == 0 && i < p.d;
  // OUTM 2: the lane's byte offset at step 0, out of bounds for lanes that store nothing; a
  // step past T lands past the batch row (the host keeps (T + CK) H d elements under 2 GiB,
  // so no offset wraps)
  const unsigned obase = orow ? (unsigned)(((long)h * p.d + i) * sizeof(TT)) : OOB_OFF;
  const unsigned ostep = (unsigned)((long)p.H * p.d * sizeof(TT));
  float S[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) S[c] = 0.0f;
  StageRegs<TT, DP> R;
  load_chunk<TT, DP>(R, p, bh, rb, 0, false);
  store_chunk<TT, DP>(sms[0], R, p, rb, 0, false);
  __syncthreads();
  for (int ch = 0; ch < nch; ++ch) {
    const int t0 = ch * CK;
    const Stage<DP>& sm = sms[ch & 1];
    // the next chunk's inputs load under this chunk's steps (past the last chunk, a reload)
    load_chunk<TT, DP>(R, p, bh, rb, min(t0 + CK, (nch - 1) * CK), false);
    // all CK steps unrolled (the staged padding past T makes the extra steps identities), so
    // the next step's LDS reads can be issued under the current step's arithmetic
#pragma unroll
    for (int tt = 0; tt < CK; ++tt) {
      fwd_step<DP, DECAY>(S, sm, tt, tr, tc);
      if constexpr (OUTM != 0) {  // o_i = sum_j S[i][j] q_j
        float o = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) o = fmaf(S[c], sm.q[tt][tc + 16 * c], o);
        o = row16_sum(o);
        if constexpr (OUTM == 2) {
          bstore<TT>(r_out, obase + (unsigned)(t0 + tt) * ostep, o);
        } else if (orow && t0 + tt < p.T) {
          st((TT*)p.out, (((long)b * p.T + t0 + tt) * p.H + h) * p.d + i, o);
        }
      }
    }
    if (p.ckpt != nullptr) {
      float* cp = p.ckpt + ((long)bh * p.nck + t0 / CK) * DP * DP + (long)i * DP + tc;
#pragma unroll
      for (int c = 0; c < NC; ++c) cp[16 * c] = S[c];
    }
    // the other buffer was last read in the previous chunk, before the barrier below it
    store_chunk<TT, DP>(sms[(ch + 1) & 1], R, p, rb, t0 + CK, false);
    __syncthreads();
  }
}

// Backward over chunks in reverse.  Per step t (S_p the state before it, S_g = a S_p,
// S_t = S_g + be k^T, dtot = dS + do q^T):  dq = S_t^T do, dv = beta ds_k,
// dbeta = err ds_k, dk = dtot^T be - S_g^T (beta ds_k), dalpha = sum((dtot - beta ds_k k^T) o S_p),
// dS <- a (dtot - beta ds_k k^T), with err = v - S_g k, be = beta err, ds_k = dtot k.
//
// The sums over the block's rows (dq, dk: one value per column; dalpha and a per-head
// dbeta: one per row) leave the dependency chain of the steps: each wave sums its four
// rows in registers (rows4_scatter: the lane of row r keeps the column sums of one value
// in four) into a per-step slot of an LDS buffer, and every FS steps one barrier pair adds
// the four waves' slots (in wave order) and stores the partials of those steps.
// BUF: the per-row outputs (dv, per-element dbeta, KDA's dalpha) go through buffer resources
// over the batch row, every lane storing at an offset the hardware drops where the lane
// stores nothing (as the forward's OUTM 2), so the unrolled steps hold no branch.
template <typename TT, int DP, bool DECAY, bool BUF>
__global__ __launch_bounds__(256) void dr_seq_bwd_kernel(const DRArgs p) {
  constexpr int NC = DP / 16;
  constexpr int FS = 8;                 // steps per flush of the row sums
  constexpr int NG = (2 * NC + 3) / 4;  // rows4_scatter groups of the lane's 2 NC column values
  static_assert(CK % FS == 0, "flushes split the chunk");
  __shared__ Stage<DP> sms[2];
  __shared__ float wsum[FS][4][NG][64];  // [step slot][wave][group][lane]: four-row sums
  __shared__ float rsum[FS][2][RB];      // [step slot][dalpha | dbeta][row]
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int w = tid >> 6, lane = tid & 63;
  const long bh = blockIdx.x;
  const int rb = blockIdx.y, i = rb * RB + tr;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const long nbth = (long)gridDim.x * p.T;  // B * T * H
  const long rowel = (long)p.T * p.H * p.d;  // per-row output elements of one batch row
  const unsigned rbytes = (unsigned)(BUF ? rowel * sizeof(TT) : 0);
  const rsrc_t r_dv = make_rsrc(BUF ? (const TT*)p.dv + (long)b * rowel : (const TT*)p.k, rbytes);
  const rsrc_t r_db = make_rsrc(BUF && !p.beta_per_head ? (const TT*)p.dbeta + (long)b * rowel : (const TT*)p.k,
                                BUF && !p.beta_per_head ? rbytes : 0u);
  const rsrc_t r_da = make_rsrc(BUF && p.alpha_per_row ? (const TT*)p.dalpha + (long)b * rowel : (const TT*)p.k,
                                BUF && p.alpha_per_row ? rbytes : 0u);
  const unsigned obase = (tc == 0 && i < p.d) ? (unsigned)(((long)h * p.d + i) * sizeof(TT)) : OOB_OFF;
  const unsigned ostep = (unsigned)((long)p.H * p.d * sizeof(TT));
  float dS[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) dS[c] = 0.0f;

  // chunk inputs and the checkpoint each chunk starts from, loaded a chunk ahead
  StageRegs<TT, DP> R;
  float cpn[NC];
  auto load_ck = [&](int ck) {
    // chunk 0 starts from zero; its (unused) load address stays in bounds
    const float* cp = p.ckpt + ((long)bh * p.nck + max(ck - 1, 0)) * DP * DP + (long)i * DP + tc;
#pragma unroll
    for (int c = 0; c < NC; ++c) cpn[c] = cp[16 * c];
  };
  load_chunk<TT, DP>(R, p, bh, rb, (p.nck - 1) * CK, true);
  load_ck(p.nck - 1);
  store_chunk<TT, DP>(sms[(p.nck - 1) & 1], R, p, rb, (p.nck - 1) * CK, true);
  __syncthreads();
  for (int ck = p.nck - 1; ck >= 0; --ck) {
    const int t0 = ck * CK;
    const Stage<DP>& sm = sms[ck & 1];
    float S[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) S[c] = ck > 0 ? cpn[c] : 0.0f;
    // the previous chunk's inputs and checkpoint load under this chunk's work (for chunk
    // 0, a reload)
    load_chunk<TT, DP>(R, p, bh, rb, max(ck - 1, 0) * CK, true);
    load_ck(max(ck - 1, 0));
    // recompute the chunk's states into registers: Sl[tt] = state before step t0 + tt
    float Sl[CK][NC];
    {
#pragma unroll
      for (int tt = 0; tt < CK; ++tt) {
#pragma unroll
        for (int c = 0; c < NC; ++c) Sl[tt][c] = S[c];
        fwd_step<DP, DECAY>(S, sm, tt, tr, tc);
      }
    }
#pragma unroll
    for (int tt = CK - 1; tt >= 0; --tt) {
      const int t = t0 + tt;
      const float at = DECAY ? sm.a[tt][tr] : 1.0f;
      const float goi = sm.go[tt][tr], bi = sm.b[tt][tr];
      float r = 0.0f, sk = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float kj = sm.k[tt][tc + 16 * c];
        r = fmaf(Sl[tt][c], kj, r);
        sk = fmaf(fmaf(goi, sm.q[tt][tc + 16 * c], dS[c]), kj, sk);
      }
      r = row16_sum(r) * at;
      sk = row16_sum(sk);
      const float err = sm.v[tt][tr] - r;
      const float be = bi * err, bdk = bi * sk;
      float pq[NC], pk[NC], pa = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float kj = sm.k[tt][tc + 16 * c], qj = sm.q[tt][tc + 16 * c];
        const float sg = at * Sl[tt][c];
        const float snew = fmaf(be, kj, sg);
        const float dtot = fmaf(goi, qj, dS[c]);
        pq[c] = snew * goi;
        pk[c] = fmaf(dtot, be, -sg * bdk);
        const float ddec = fmaf(-bdk, kj, dtot);
        if (DECAY) pa = fmaf(ddec, Sl[tt][c], pa);  // dalpha: no decay, no gradient
        dS[c] = at * ddec;
      }
      const bool live = t < p.T;
      const long bth = ((long)b * p.T + t) * p.H + h;
      if constexpr (BUF) {  // per-row outputs: dv, per-element dbeta (steps past T land past the row)
        const unsigned off = obase + (unsigned)t * ostep;
        bstore<TT>(r_dv, off, bdk);
        bstore<TT>(r_db, off, err * sk);
      } else if (live && tc == 0 && i < p.d) {
        st((TT*)p.dv, bth * p.d + i, bdk);
        if (!p.beta_per_head) st((TT*)p.dbeta, bth * p.d + i, err * sk);
      }
      // this wave's four rows summed per column: value k = qty NC + c (pq then pk), group
      // k / 4; the lane of row r keeps item rows4_item(r) of each group
      const int slot = tt % FS;
      float vals[4 * NG];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        vals[c] = pq[c];
        vals[NC + c] = pk[c];
      }
#pragma unroll
      for (int k = 2 * NC; k < 4 * NG; ++k) vals[k] = 0.0f;
#pragma unroll
      for (int g = 0; g < NG; ++g)
        wsum[slot][w][g][lane] = rows4_scatter(vals[4 * g], vals[4 * g + 1], vals[4 * g + 2], vals[4 * g + 3]);
      if (DECAY) pa = row16_sum(pa);
      if constexpr (BUF) {
        // every lane of the row holds the row sums: the 16 equal writes need no branch
        rsum[slot][0][tr] = pa;
        rsum[slot][1][tr] = i < p.d ? err * sk : 0.0f;
        // KDA: the row's own decay gradient, in log space
        if constexpr (DECAY) bstore<TT>(r_da, obase + (unsigned)t * ostep, pa * at);
      } else if (tc == 0) {
        rsum[slot][0][tr] = pa;
        rsum[slot][1][tr] = i < p.d ? err * sk : 0.0f;
        if (p.alpha_per_row && live && i < p.d) st((TT*)p.dalpha, bth * p.d + i, pa * at);
      }
      if (slot == 0) {  // steps t .. t + FS - 1 are in the slots: sum the waves, store
        __syncthreads();
        for (int e = tid; e < FS * 2 * DP; e += 256) {
          const int sl = e / (2 * DP), qty = (e / DP) & 1, j = e % DP;
          const int k = qty * NC + (j >> 4), g = k >> 2, src = 16 * rows4_item(k & 3) + (j & 15);
          const float acc = ((wsum[sl][0][g][src] + wsum[sl][1][g][src]) + wsum[sl][2][g][src]) + wsum[sl][3][g][src];
          const int ts = t + sl;
          if (ts < p.T && j < p.d)
            (qty == 0 ? p.part_q : p.part_k)[((long)rb * nbth + ((long)b * p.T + ts) * p.H + h) * p.d + j] = acc;
        }
        if (tid < 2 * FS) {
          const int sl = tid >> 1, qty = tid & 1, ts = t + sl;
          float acc = 0.0f;
#pragma unroll
          for (int m = 0; m < RB; ++m) acc += rsum[sl][qty][m];
          if (ts < p.T) (qty == 0 ? p.part_a : p.part_b)[(long)rb * nbth + ((long)b * p.T + ts) * p.H + h] = acc;
        }
        __syncthreads();
      }
    }
    // the other buffer was last read in the previous chunk, before this chunk's barriers
    store_chunk<TT, DP>(sms[(ck + 1) & 1], R, p, rb, (ck - 1) * CK, true);
    __syncthreads();
  }
}

// dq, dk (and dalpha, per-head dbeta) = the row-block partials added in block order.
template <typename TT>
__global__ __launch_bounds__(256) void dr_seq_reduce_kernel(const DRArgs p, long nbth, int nrb) {
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
  } else if (e < 2 * nvec + 2 * nbth) {
    const int qty = e >= 2 * nvec + nbth;
    const long o = e - 2 * nvec - qty * nbth;
    const float* part = qty ? p.part_b : p.part_a;
    float acc = 0.0f;
    for (int r = 0; r < nrb; ++r) acc += part[r * nbth + o];
    if (qty == 0 && p.dalpha != nullptr && !p.alpha_per_row) st((TT*)p.dalpha, o, acc);
    if (qty == 1 && p.beta_per_head) st((TT*)p.dbeta, o, acc);
  }
}

template <typename TT, int DP, bool DECAY>
void fwd_out(hipStream_t s, dim3 grid, const DRArgs& a) {
  if (a.out == nullptr)
    dr_seq_fwd_kernel<TT, DP, DECAY, 0><<<grid, 256, 0, s>>>(a);
  else if ((long)(a.T + CK) * a.H * a.d * (long)sizeof(TT) < (1L << 31))
    dr_seq_fwd_kernel<TT, DP, DECAY, 2><<<grid, 256, 0, s>>>(a);
  else
    dr_seq_fwd_kernel<TT, DP, DECAY, 1><<<grid, 256, 0, s>>>(a);
}

template <typename TT, int DP, bool DECAY>
void bwd_out(hipStream_t s, dim3 grid, const DRArgs& a) {
  if ((long)(a.T + CK) * a.H * a.d * (long)sizeof(TT) < (1L << 31))
    dr_seq_bwd_kernel<TT, DP, DECAY, true><<<grid, 256, 0, s>>>(a);
  else
    dr_seq_bwd_kernel<TT, DP, DECAY, false><<<grid, 256, 0, s>>>(a);
}

template <typename TT>
int launch_seq(hipStream_t s, const DRArgs& a, bool bwd, int BH) {
  const int d = a.d;
#define EDF_DR_LAUNCH(DP)                                              \
  do {                                                                 \
    const dim3 grid(BH, DP / RB);                                      \
    if (bwd && a.alpha != nullptr)                                     \
      bwd_out<TT, DP, true>(s, grid, a);                               \
    else if (bwd)                                                      \
      bwd_out<TT, DP, false>(s, grid, a);                              \
    else if (a.alpha != nullptr)                                       \
      fwd_out<TT, DP, true>(s, grid, a);                               \
    else                                                               \
      fwd_out<TT, DP, false>(s, grid, a);                              \
  } while (0)
  if (d <= 16)
    EDF_DR_LAUNCH(16);
  else if (d <= 32)
    EDF_DR_LAUNCH(32);
  else if (d <= 64)
    EDF_DR_LAUNCH(64);
  else
    EDF_DR_LAUNCH(128);
#undef EDF_DR_LAUNCH
  return check_launch(bwd ? "delta rule backward" : "delta rule");
}

inline int pad_dim(int d) { return d <= 16 ? 16 : d <= 32 ? 32 : d <= 64 ? 64 : 128; }

struct SeqWs {
  size_t ckpt, part_q, part_k, part_a, part_b, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline SeqWs seq_ws(int batch, int heads, int seq, int d) {
  const size_t dp = pad_dim(d), nrb = dp / RB;
  const size_t nck = (seq + CK - 1) / CK;
  const size_t bh = (size_t)batch * heads, nbth = bh * seq;
  SeqWs w{};
  size_t off = 0;
  w.ckpt = off;
  off += align256(bh * nck * dp * dp * 4);
  w.part_q = off;
  off += align256(nrb * nbth * d * 4);
  w.part_k = off;
  off += align256(nrb * nbth * d * 4);
  w.part_a = off;
  off += align256(nrb * nbth * 4);
  w.part_b = off;
  off += align256(nrb * nbth * 4);
  w.total = off;
  return w;
}

}  // namespace

size_t dr_seq_backward_workspace_bytes(int batch, int heads, int seq, int d) {
  return seq_ws(batch, heads, seq, d).total;
}

// the states the per-step forward can store for a later backward (the checkpoints the
// backward would otherwise recompute with a forward pass of its own)
size_t dr_seq_context_bytes(int batch, int heads, int seq, int d) {
  const SeqWs w = seq_ws(batch, heads, seq, d);
  return w.part_q - w.ckpt;
}

int dr_seq_run(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
               void* out, int batch, int seq, int heads, int d, int dtype, int beta_per_head, int alpha_per_row,
               float* context) {
  DRArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.alpha = alpha; a.out = out;
  a.ckpt = context;  // also store the checkpoints (one pass writes both)
  a.H = heads; a.T = seq; a.d = d; a.beta_per_head = beta_per_head; a.alpha_per_row = alpha_per_row;
  a.nck = (seq + CK - 1) / CK;
  hipStream_t s = as_stream(stream);
  if (dtype == EDF_BF16) return launch_seq<bf16>(s, a, false, batch * heads);
  return launch_seq<float>(s, a, false, batch * heads);
}

int dr_seq_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                        const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                        void* dalpha, void* workspace, int batch, int seq, int heads, int d, int dtype,
                        int beta_per_head, int alpha_per_row, const float* context) {
  DRArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.alpha = alpha; a.dout = grad_out;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dbeta = dbeta; a.dalpha = dalpha;
  a.H = heads; a.T = seq; a.d = d; a.beta_per_head = beta_per_head; a.alpha_per_row = alpha_per_row;
  a.nck = (seq + CK - 1) / CK;
  const SeqWs w = seq_ws(batch, heads, seq, d);
  char* ws = (char*)workspace;
  a.ckpt = context ? const_cast<float*>(context) : (float*)(ws + w.ckpt);
  a.part_q = (float*)(ws + w.part_q);
  a.part_k = (float*)(ws + w.part_k);
  a.part_a = (float*)(ws + w.part_a);
  a.part_b = (float*)(ws + w.part_b);
  const int bh = batch * heads;
  const long nbth = (long)bh * seq;
  const int nrb = pad_dim(d) / RB;
  hipStream_t s = as_stream(stream);
  // forward pass that only writes the checkpoints
  DRArgs f = a;
  f.out = nullptr;
  const long n4 = d % 4 == 0 ? 2 * nbth * d / 4 : 0;  // vector items of the reduction (see the kernel)
  const long nred = 2 * nbth * d + 2 * nbth - 3 * n4;
  const unsigned gred = (unsigned)((nred + 255) / 256);
  int rc;
  if (dtype == EDF_BF16) {
    if (!context) {  // the forward's stored checkpoints, or a pass that writes only them
      rc = launch_seq<bf16>(s, f, false, bh);
      if (rc) return rc;
    }
    rc = launch_seq<bf16>(s, a, true, bh);
    if (rc) return rc;
    dr_seq_reduce_kernel<bf16><<<gred, 256, 0, s>>>(a, nbth, nrb);
  } else {
    if (!context) {
      rc = launch_seq<float>(s, f, false, bh);
      if (rc) return rc;
    }
    rc = launch_seq<float>(s, a, true, bh);
    if (rc) return rc;
    dr_seq_reduce_kernel<float><<<gred, 256, 0, s>>>(a, nbth, nrb);
  }
  return check_launch("delta rule backward reduction");
}

}  // namespace edf
