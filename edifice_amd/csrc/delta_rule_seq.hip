// Delta rule (DeltaNet / GatedDeltaNet), step-by-step recurrence, forward and backward.
//
// Semantics (reference):
//   S_g = alpha_t S;  r = S_g k_t;  S = S_g + diag(beta_t)(v_t - r) k_t^T;  o_t = S q_t
//   S is [d_v x d_k] per (batch, head); beta per element [B,T,H,d] (one gate per value
//   row, lib/edifice/recurrent/delta_net.ex:231-273, native/cuda/fused_delta_rule_scan.cu:146-154)
//   or per head [B,T,H]; alpha per head [B,T,H] or absent
//   (lib/edifice/recurrent/gated_delta_net.ex:300-353).
//   Backward: lib/edifice/cuda/fused_scan.ex:1257-1431 (dq = S_t^T do, ds_k = dS_tot k,
//   dv = beta ds_k, dbeta = err ds_k, dk = dS_tot^T (beta err) - S_g^T (beta ds_k),
//   dalpha = sum(dS_to_decayed * S_prev), dS_prev = alpha dS_to_decayed).
//
// This is the exact per-step path: it supports per-element beta (where each row of S
// has its own gate, so the chunked UT form of the per-head path does not apply),
// float32 I/O and any head_dim <= 128.  One workgroup of 256 lanes owns one
// (batch, head) state; lane (tr, tc) holds S[tr + 16 a][tc + 16 c], so row sums are
// reductions inside a 16-lane DPP row and column sums go through LDS.
// The backward does not invert the update (the reference divides by alpha): the
// forward states are checkpointed every CK steps into the workspace and each chunk's
// CK states are recomputed into a per-(batch, head) workspace slab.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int CK = 16;  // steps per staged chunk / checkpoint interval

struct DRArgs {
  const void *q, *k, *v, *beta, *alpha, *dout;
  void *out, *dq, *dk, *dv, *dbeta, *dalpha;
  float* ckpt;  // [BH][nck][DP*DP]
  float* slab;  // [BH][CK][DP*DP]
  int H, T, d, beta_per_head, nck;
};

EDF_DEVICE float row16_sum(float x) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) x += __shfl_xor(x, off, 16);
  return x;
}

template <typename TT, int DP>
struct Stage {
  float k[CK][DP], q[CK][DP], v[CK][DP], b[CK][DP], go[CK][DP];
  float a[CK];
};

// Stage CK steps of the per-(b,h) inputs (zero-padded beyond T and beyond d).
template <typename TT, int DP>
EDF_DEVICE void stage_chunk(Stage<TT, DP>& sm, const DRArgs& p, long bh, int t0, bool with_dout) {
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  const int d = p.d;
  for (int e = threadIdx.x; e < CK * DP; e += 256) {
    const int tt = e / DP, j = e % DP;
    const int t = t0 + tt;
    const bool ok = t < p.T && j < d;
    const long idx = (((long)b * p.T + t) * p.H + h) * d + j;
    sm.k[tt][j] = ok ? ld((const TT*)p.k, idx) : 0.0f;
    sm.q[tt][j] = ok ? ld((const TT*)p.q, idx) : 0.0f;
    sm.v[tt][j] = ok ? ld((const TT*)p.v, idx) : 0.0f;
    float bv = 0.0f;
    if (ok) bv = p.beta_per_head ? ld((const TT*)p.beta, ((long)b * p.T + t) * p.H + h) : ld((const TT*)p.beta, idx);
    sm.b[tt][j] = bv;
    if (with_dout) sm.go[tt][j] = ok ? ld((const TT*)p.dout, idx) : 0.0f;
  }
  for (int tt = threadIdx.x; tt < CK; tt += 256) {
    const int t = t0 + tt;
    sm.a[tt] = (p.alpha != nullptr && t < p.T) ? ld((const TT*)p.alpha, ((long)b * p.T + t) * p.H + h) : 1.0f;
  }
}

// One forward step on the lane's tile; returns nothing, updates S in place.
template <int DP>
EDF_DEVICE void fwd_step(float (&S)[DP / 16][DP / 16], const float* kt, const float* vt, const float* bt, float at,
                         int tr, int tc, float* r_out) {
  constexpr int NA = DP / 16;
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    float r = 0.0f;
#pragma unroll
    for (int c = 0; c < NA; ++c) r = fmaf(S[a][c], kt[tc + 16 * c], r);
    r = row16_sum(r) * at;
    const int i = tr + 16 * a;
    const float e = bt[i] * (vt[i] - r);
    if (r_out) r_out[a] = r;
#pragma unroll
    for (int c = 0; c < NA; ++c) S[a][c] = fmaf(e, kt[tc + 16 * c], at * S[a][c]);
  }
}

template <typename TT, int DP>
__global__ __launch_bounds__(256) void dr_seq_fwd_kernel(const DRArgs p) {
  constexpr int NA = DP / 16;
  __shared__ Stage<TT, DP> sm;
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long bh = blockIdx.x;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  float S[NA][NA];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int c = 0; c < NA; ++c) S[a][c] = 0.0f;
  for (int t0 = 0; t0 < p.T; t0 += CK) {
    __syncthreads();
    stage_chunk<TT, DP>(sm, p, bh, t0, false);
    __syncthreads();
    for (int tt = 0; tt < CK && t0 + tt < p.T; ++tt) {
      fwd_step<DP>(S, sm.k[tt], sm.v[tt], sm.b[tt], sm.a[tt], tr, tc, nullptr);
      // o_i = sum_j S[i][j] q_j
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        float o = 0.0f;
#pragma unroll
        for (int c = 0; c < NA; ++c) o = fmaf(S[a][c], sm.q[tt][tc + 16 * c], o);
        o = row16_sum(o);
        const int i = tr + 16 * a;
        if (p.out != nullptr && tc == a && i < p.d) st((TT*)p.out, (((long)b * p.T + t0 + tt) * p.H + h) * p.d + i, o);
      }
    }
    if (p.ckpt != nullptr) {
      float* cp = p.ckpt + ((long)bh * p.nck + t0 / CK) * DP * DP;
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int c = 0; c < NA; ++c) cp[(tr + 16 * a) * DP + tc + 16 * c] = S[a][c];
    }
  }
}

template <typename TT, int DP>
__global__ __launch_bounds__(256) void dr_seq_bwd_kernel(const DRArgs p) {
  constexpr int NA = DP / 16;
  __shared__ Stage<TT, DP> sm;
  __shared__ float red[2][16][DP + 1];  // column partials: [qty][tr][j]
  __shared__ float reda[16 * 16];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const long bh = blockIdx.x;
  const int b = (int)(bh / p.H), h = (int)(bh % p.H);
  float* slab = p.slab + bh * CK * DP * DP;
  float dS[NA][NA];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int c = 0; c < NA; ++c) dS[a][c] = 0.0f;

  for (int ck = p.nck - 1; ck >= 0; --ck) {
    const int t0 = ck * CK;
    __syncthreads();
    stage_chunk<TT, DP>(sm, p, bh, t0, true);
    __syncthreads();
    // recompute the chunk: slab[tt] = state before step t0 + tt
    {
      float S[NA][NA];
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int c = 0; c < NA; ++c)
          S[a][c] = ck > 0 ? p.ckpt[((long)bh * p.nck + (ck - 1)) * DP * DP + (tr + 16 * a) * DP + tc + 16 * c] : 0.0f;
      for (int tt = 0; tt < CK; ++tt) {
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int c = 0; c < NA; ++c) slab[(long)tt * DP * DP + (tr + 16 * a) * DP + tc + 16 * c] = S[a][c];
        fwd_step<DP>(S, sm.k[tt], sm.v[tt], sm.b[tt], sm.a[tt], tr, tc, nullptr);
      }
    }
    for (int tt = CK - 1; tt >= 0; --tt) {
      const int t = t0 + tt;
      if (t >= p.T) continue;
      const float at = sm.a[tt];
      const float* kt = sm.k[tt];
      const float* qt = sm.q[tt];
      const float* bt = sm.b[tt];
      const float* got = sm.go[tt];
      float Sp[NA][NA];
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int c = 0; c < NA; ++c) Sp[a][c] = slab[(long)tt * DP * DP + (tr + 16 * a) * DP + tc + 16 * c];
      float err[NA], be[NA], bdk[NA], dsk[NA];
      float pq[NA], pk[NA], pa = 0.0f;
#pragma unroll
      for (int c = 0; c < NA; ++c) {
        pq[c] = 0.0f;
        pk[c] = 0.0f;
      }
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int i = tr + 16 * a;
        float r = 0.0f, sk = 0.0f;
#pragma unroll
        for (int c = 0; c < NA; ++c) {
          r = fmaf(Sp[a][c], kt[tc + 16 * c], r);
          sk = fmaf(fmaf(got[i], qt[tc + 16 * c], dS[a][c]), kt[tc + 16 * c], sk);
        }
        r = row16_sum(r) * at;
        sk = row16_sum(sk);
        err[a] = sm.v[tt][i] - r;
        be[a] = bt[i] * err[a];
        dsk[a] = sk;
        bdk[a] = bt[i] * sk;
      }
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int i = tr + 16 * a;
#pragma unroll
        for (int c = 0; c < NA; ++c) {
          const int j = tc + 16 * c;
          const float sg = at * Sp[a][c];
          const float snew = fmaf(be[a], kt[j], sg);
          const float dtot = fmaf(got[i], qt[j], dS[a][c]);
          pq[c] = fmaf(snew, got[i], pq[c]);
          pk[c] = fmaf(dtot, be[a], fmaf(-sg, bdk[a], pk[c]));
          const float ddec = fmaf(-bdk[a], kt[j], dtot);
          pa = fmaf(ddec, Sp[a][c], pa);
          dS[a][c] = at * ddec;
        }
      }
      // per-row outputs: dv, dbeta
      const long rowbase = (((long)b * p.T + t) * p.H + h) * p.d;
      float dbh = 0.0f;
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int i = tr + 16 * a;
        if (tc == 0 && i < p.d) {
          st((TT*)p.dv, rowbase + i, bdk[a]);
          if (!p.beta_per_head) st((TT*)p.dbeta, rowbase + i, err[a] * dsk[a]);
        }
        dbh += (i < p.d) ? err[a] * dsk[a] : 0.0f;
      }
      // column sums (dq, dk) and the full sums (dalpha, per-head dbeta) through LDS
#pragma unroll
      for (int c = 0; c < NA; ++c) {
        red[0][tr][tc + 16 * c] = pq[c];
        red[1][tr][tc + 16 * c] = pk[c];
      }
      pa = row16_sum(pa);
      if (tc == 0) {
        reda[tr] = pa;
        reda[16 + tr] = dbh;
      }
      __syncthreads();
      for (int e = tid; e < 2 * DP; e += 256) {
        const int qty = e / DP, j = e % DP;
        float s = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) s += red[qty][m][j];
        if (j < p.d) st((TT*)(qty == 0 ? p.dq : p.dk), rowbase + j, s);
      }
      if (tid == 0) {
        float sa = 0.0f, sb = 0.0f;
        for (int m = 0; m < 16; ++m) {
          sa += reda[m];
          sb += reda[16 + m];
        }
        const long hidx = ((long)b * p.T + t) * p.H + h;
        if (p.dalpha != nullptr) st((TT*)p.dalpha, hidx, sa);
        if (p.beta_per_head) st((TT*)p.dbeta, hidx, sb);
      }
      __syncthreads();
    }
  }
}

template <typename TT>
int launch_seq(hipStream_t s, const DRArgs& a, bool bwd, int BH) {
  const int d = a.d;
#define EDF_DR_LAUNCH(DP)                                              \
  do {                                                                 \
    if (bwd)                                                           \
      dr_seq_bwd_kernel<TT, DP><<<BH, 256, 0, s>>>(a);                 \
    else                                                               \
      dr_seq_fwd_kernel<TT, DP><<<BH, 256, 0, s>>>(a);                 \
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

}  // namespace

size_t dr_seq_backward_workspace_bytes(int batch, int heads, int seq, int d) {
  const size_t dp = pad_dim(d);
  const size_t nck = (seq + CK - 1) / CK;
  const size_t bh = (size_t)batch * heads;
  return bh * nck * dp * dp * 4 + bh * CK * dp * dp * 4;
}

int dr_seq_run(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
               void* out, int batch, int seq, int heads, int d, int dtype, int beta_per_head) {
  DRArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.alpha = alpha; a.out = out;
  a.H = heads; a.T = seq; a.d = d; a.beta_per_head = beta_per_head;
  a.nck = (seq + CK - 1) / CK;
  hipStream_t s = as_stream(stream);
  if (dtype == EDF_BF16) return launch_seq<bf16>(s, a, false, batch * heads);
  return launch_seq<float>(s, a, false, batch * heads);
}

int dr_seq_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                        const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                        void* dalpha, void* workspace, int batch, int seq, int heads, int d, int dtype,
                        int beta_per_head) {
  DRArgs a{};
  a.q = q; a.k = k; a.v = v; a.beta = beta; a.alpha = alpha; a.dout = grad_out;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dbeta = dbeta; a.dalpha = dalpha;
  a.H = heads; a.T = seq; a.d = d; a.beta_per_head = beta_per_head;
  a.nck = (seq + CK - 1) / CK;
  const size_t dp = pad_dim(d);
  const size_t bh = (size_t)batch * heads;
  a.ckpt = (float*)workspace;
  a.slab = (float*)((char*)workspace + bh * a.nck * dp * dp * 4);
  hipStream_t s = as_stream(stream);
  // forward pass that only writes the checkpoints (output goes to the slab area, unused)
  DRArgs f = a;
  f.out = nullptr;
  int rc;
  if (dtype == EDF_BF16) {
    rc = launch_seq<bf16>(s, f, false, (int)bh);
    if (rc) return rc;
    return launch_seq<bf16>(s, a, true, (int)bh);
  }
  rc = launch_seq<float>(s, f, false, (int)bh);
  if (rc) return rc;
  return launch_seq<float>(s, a, true, (int)bh);
}

}  // namespace edf
