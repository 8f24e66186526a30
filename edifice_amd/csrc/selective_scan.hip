// Mamba selective scan, forward and backward, for gfx950.
//
// Semantics (reference):
//   dt_c = clip(dt, 1e-3, 0.1); h[d,n] = exp(dt_c A[d,n]) h[d,n] + dt_b B[n] x[d];
//   y[d] = sum_n C[n] h[d,n]
//     native/cuda/fused_selective_scan.cu:30-31,41-91 (kernel semantics, dt_b = dt_c)
//     lib/edifice/ssm/common.ex:402-445 (block semantics, dt_b = mean_d dt_c: "mean" mode)
//   backward lib/edifice/cuda/fused_scan.ex:1453-1533 (dx, ddt masked to the unclipped
//   range, dB, dC), extended with dA, dD and the silu(z) gate, which have no reference
//   kernel counterpart (the Mamba block applies them outside the scan,
//   common.ex:270-278).
//   Optional extensions: y += D[d] x, then y *= silu(z).
//
// Design (see the repository design notes for the roofline discussion):
//   * lane = (channel d, state n); LPC = min(N,16) lanes per channel, SPL = N/LPC
//     states per lane, so a channel's states live in one 16-lane DPP row and the
//     grid has B*D*N/SPL lanes (3072 waves at B=8, D=1536, N=16) without splitting T;
//   * inputs are staged per block of timesteps through LDS with coalesced row loads
//     (x, dt, z: [t][channel] rows; B, C: [t][n] rows shared by the whole workgroup);
//     clip(dt) and dt*x are computed once per (t, d) at staging time;
//   * per (t, n) the lane does one v_exp_f32 and four VALU ops;
//   * y = sum_n C h is a transpose-reduce through LDS (one add per (t, n));
//   * workgroup ids are remapped so that tiles sharing 128 B lines share an XCD;
//   * backward: the forward writes the state every CK timesteps ("checkpoints");
//     backward walks chunks in reverse, recomputes the chunk's states and decays
//     into registers, then runs the reverse recurrence.  Sums over channels
//     (dB, dC) are reduced in LDS per workgroup and then across workgroups by a
//     small deterministic reduction kernel; sums over states (dx, ddt) use the
//     LDS transpose-reduce.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr float DT_MIN = 1.0e-3f;
constexpr float DT_MAX = 0.1f;

struct SSArgs {
  const void* x;
  const void* dt;
  const void* A;
  const void* B;
  const void* C;
  const void* D;
  const void* z;
  const float* dtmean;  // [batch, seq] or null (per-channel dt_b)
  void* out;
  float* ckpt;  // [batch, dim, nck, N] state after each chunk of ck timesteps
  // backward only
  const void* dout;
  void* dx;
  void* ddt;
  void* dz;
  float* part_bc;  // [ntile, batch, seq, 2, N]
  float* part_a;   // [batch, dim, N]
  float* part_d;   // [batch, dim]
  float* part_m;   // [ntile, batch, seq] (mean mode)
  int batch, seq, dim, ck, nck, ntile;
};

template <int N, int NT>
struct Geo {
  static constexpr int LPC = N < 16 ? N : 16;
  static constexpr int SPL = N / LPC;
  static constexpr int CPW = NT / LPC;  // channels per workgroup
};

// ---------------------------------------------------------------------------
// dt mean over channels (block semantics), one wave per (b, t)
// ---------------------------------------------------------------------------
template <typename TI>
__global__ __launch_bounds__(256) void ss_dtmean_kernel(const TI* __restrict__ dt, float* __restrict__ dtm, int rows,
                                                        int dim) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const TI* p = dt + (long)row * dim;
  float s = 0.0f;
  for (int d = lane; d < dim; d += 64) s += clampf(ld(p, d), DT_MIN, DT_MAX);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) dtm[row] = s / (float)dim;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename TI, typename TP, int N, int NT, bool MEAN, bool HAS_Z>
__global__ __launch_bounds__(NT) void ss_fwd_kernel(const SSArgs p) {
  using G = Geo<N, NT>;
  constexpr int LPC = G::LPC, SPL = G::SPL, CPW = G::CPW;
  constexpr int TS = 16;
  constexpr int PT = TS + 1;  // odd row stride: row writes and column reads hit distinct banks
  constexpr int EPT = CPW * TS / NT;              // staged (t, channel) elements per thread
  constexpr int BPT = (N * TS + NT - 1) / NT;     // staged (t, n) elements per thread
  __shared__ float s_x[CPW][PT], s_dtc[CPW][PT], s_dtx[CPW][PT], s_z[CPW][PT];
  __shared__ float s_B[N][TS + 1], s_C[N][TS + 1];
  __shared__ float s_p[NT][PT];
  __shared__ float s_y[TS][CPW + 1];

  const TI* x = (const TI*)p.x;
  const TI* dt = (const TI*)p.dt;
  const TI* z = (const TI*)p.z;
  const TP* Am = (const TP*)p.A;
  const TP* Bm = (const TP*)p.B;
  const TP* Cm = (const TP*)p.C;
  const TP* Dv = (const TP*)p.D;
  TI* out = (TI*)p.out;
  const int seq = p.seq, dim = p.dim;

  const int tid = threadIdx.x;
  const int n = tid % LPC, cl = tid / LPC;
  const int logical = remap_xcd(blockIdx.x, gridDim.x);
  const int b = logical / p.ntile, tile = logical % p.ntile;
  const int c0 = tile * CPW, c = c0 + cl;
  const bool cvalid = c < dim;

  float A2[SPL], h[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    A2[s] = cvalid ? ld(Am, (long)c * N + n * SPL + s) * LOG2E : 0.0f;
    h[s] = 0.0f;
  }
  const float Dc = (Dv != nullptr && cvalid) ? ld(Dv, c) : 0.0f;
  const long rowbase = (long)b * seq * dim;

  // Raw values of the next block, loaded one block ahead from clamped (in-bounds)
  // indices so no load sits behind a divergent branch.
  // Kept in the storage type: converting at load time would force a wait on the load.
  TI px[EPT], pdt[EPT], pz[EPT];
  TP pb[BPT], pc[BPT];
  float pm[EPT];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * NT;
      const int t = min(t0 + e / CPW, seq - 1), cc = min(c0 + e % CPW, dim - 1);
      const long idx = rowbase + (long)t * dim + cc;
      px[k] = x[idx];
      pdt[k] = dt[idx];
      if (HAS_Z) pz[k] = z[idx];
      pm[k] = MEAN ? p.dtmean[(long)b * seq + t] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      const int e = min(tid + k * NT, N * TS - 1);
      const long idx = ((long)b * seq + min(t0 + e / N, seq - 1)) * N + e % N;
      pb[k] = Bm[idx];
      pc[k] = Cm[idx];
    }
  };
  fetch(0);

  const int nblk = (seq + TS - 1) / TS;
  for (int blk = 0; blk < nblk; ++blk) {
    const int t0 = blk * TS;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * NT;
      const int tt = e / CPW, ch = e % CPW;
      const bool ok = (t0 + tt < seq) && (c0 + ch < dim);
      const float xv = to_f32(px[k]);
      const float dtc = ok ? clampf(to_f32(pdt[k]), DT_MIN, DT_MAX) : 0.0f;
      s_x[ch][tt] = ok ? xv : 0.0f;
      s_dtc[ch][tt] = dtc;
      s_dtx[ch][tt] = ok ? (MEAN ? pm[k] : dtc) * xv : 0.0f;
      s_z[ch][tt] = (ok && HAS_Z) ? to_f32(pz[k]) : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      const int e = tid + k * NT;
      if (e < N * TS) {
        const int tt = e / N, nn = e % N;
        const bool ok = t0 + tt < seq;
        s_B[nn][tt] = ok ? to_f32(pb[k]) : 0.0f;
        s_C[nn][tt] = ok ? to_f32(pc[k]) : 0.0f;
      }
    }
    if (t0 + TS < seq) fetch(t0 + TS);
    __syncthreads();

    float pr[TS];
#pragma unroll
    for (int tt = 0; tt < TS; ++tt) {
      const float dtc = s_dtc[cl][tt];
      const float dtx = s_dtx[cl][tt];
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        const int nn = n * SPL + s;
        const float a = fast_exp2(dtc * A2[s]);
        h[s] = fmaf(a, h[s], dtx * s_B[nn][tt]);
        acc = fmaf(s_C[nn][tt], h[s], acc);
      }
      pr[tt] = acc;
    }
    if (p.ckpt != nullptr && cvalid && (((t0 + TS) % p.ck) == 0 || t0 + TS >= seq)) {
      const int k = (min(t0 + TS, seq) - 1) / p.ck;
#pragma unroll
      for (int s = 0; s < SPL; ++s) p.ckpt[(((long)b * dim + c) * p.nck + k) * N + n * SPL + s] = h[s];
    }
#pragma unroll
    for (int tt = 0; tt < TS; ++tt) s_p[tid][tt] = pr[tt];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < TS / LPC; ++q) {
      const int tt = n + q * LPC;
      float y = 0.0f;
#pragma unroll
      for (int m = 0; m < LPC; ++m) y += s_p[cl * LPC + m][tt];
      y = fmaf(Dc, s_x[cl][tt], y);
      if (HAS_Z) {
        const float zv = s_z[cl][tt];
        y *= zv * sigmoidf(zv);
      }
      s_y[tt][cl] = y;
    }
    __syncthreads();
    if (out != nullptr) {
      for (int e = tid; e < CPW * TS; e += NT) {
        const int tt = e / CPW, ch = e % CPW;
        const int t = t0 + tt, cc = c0 + ch;
        if (t < seq && cc < dim) st(out, rowbase + (long)t * dim + cc, s_y[tt][ch]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
template <typename TI, typename TP, int N, int NT, int CK>
__global__ __launch_bounds__(NT) void ss_bwd_kernel(const SSArgs p) {
  using G = Geo<N, NT>;
  constexpr int LPC = G::LPC, SPL = G::SPL, CPW = G::CPW;
  static_assert(SPL == 1, "backward keeps one state per lane");
  constexpr int TS = 8;  // reduction block (timesteps)
  constexpr int PC = CK + 1;  // odd row stride: conflict-free staging writes
  // chunk tiles [channel][t]
  __shared__ float s_x[CPW][PC], s_dtc[CPW][PC], s_dtb[CPW][PC], s_rng[CPW][PC], s_dy[CPW][PC];
  __shared__ float s_B[N][CK + 1], s_C[N][CK + 1];
  // reduction scratch: [qty][lane][t]
  __shared__ float s_r[4][NT][TS + 1];
  __shared__ float s_o[2][CK][CPW + 1];  // staged dx / ddt (and dz) rows

  const TI* x = (const TI*)p.x;
  const TI* dt = (const TI*)p.dt;
  const TI* z = (const TI*)p.z;
  const TI* dout = (const TI*)p.dout;
  const TP* Am = (const TP*)p.A;
  const TP* Bm = (const TP*)p.B;
  const TP* Cm = (const TP*)p.C;
  const TP* Dv = (const TP*)p.D;
  const int seq = p.seq, dim = p.dim;
  const bool mean_mode = p.dtmean != nullptr;

  const int tid = threadIdx.x;
  const int n = tid % LPC, cl = tid / LPC;
  const int logical = remap_xcd(blockIdx.x, gridDim.x);
  const int b = logical / p.ntile, tile = logical % p.ntile;
  const int c0 = tile * CPW, c = c0 + cl;
  const bool cvalid = c < dim;

  float A1[SPL], A2[SPL], dh[SPL], dA[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    A1[s] = cvalid ? ld(Am, (long)c * N + n * SPL + s) : 0.0f;
    A2[s] = A1[s] * LOG2E;
    dh[s] = 0.0f;
    dA[s] = 0.0f;
  }
  const float Dc = (Dv != nullptr && cvalid) ? ld(Dv, c) : 0.0f;
  float dD = 0.0f;
  const long rowbase = (long)b * seq * dim;

  // Raw values of the next chunk (in reverse order), fetched one chunk ahead from
  // clamped in-bounds indices so the loads are never behind a divergent branch.
  constexpr int EPT = CPW * CK / NT;
  constexpr int BPT = (N * CK + NT - 1) / NT;
  TI px[EPT], pdt[EPT], pgo[EPT], pz[EPT];
  TP pb[BPT], pc[BPT];
  float pm[EPT];
  auto fetch = [&](int ts) {
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int e = tid + q * NT;
      const int t = min(ts + e / CPW, seq - 1), cc = min(c0 + e % CPW, dim - 1);
      const long idx = rowbase + (long)t * dim + cc;
      px[q] = x[idx];
      pdt[q] = dt[idx];
      pgo[q] = dout[idx];
      pz[q] = z != nullptr ? z[idx] : px[q];
      pm[q] = mean_mode ? p.dtmean[(long)b * seq + t] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const int e = min(tid + q * NT, N * CK - 1);
      const long idx = ((long)b * seq + min(ts + e / N, seq - 1)) * N + e % N;
      pb[q] = Bm[idx];
      pc[q] = Cm[idx];
    }
  };
  fetch((p.nck - 1) * CK);

  for (int k = p.nck - 1; k >= 0; --k) {
    const int ts = k * CK;
    // ---- stage the chunk ------------------------------------------------
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int e = tid + q * NT;
      const int tt = e / CPW, ch = e % CPW;
      const bool ok = (ts + tt < seq) && (c0 + ch < dim);
      const float dtr = to_f32(pdt[q]);
      const float dtc = ok ? clampf(dtr, DT_MIN, DT_MAX) : 0.0f;
      s_x[ch][tt] = ok ? to_f32(px[q]) : 0.0f;
      s_dtc[ch][tt] = dtc;
      s_dtb[ch][tt] = ok ? (mean_mode ? pm[q] : dtc) : 0.0f;
      s_rng[ch][tt] = (ok && dtr >= DT_MIN && dtr <= DT_MAX) ? 1.0f : 0.0f;
      s_dy[ch][tt] = ok ? to_f32(pgo[q]) : 0.0f;  // raw upstream gradient; gated below if z is present
      s_o[0][tt][ch] = ok ? to_f32(pz[q]) : 0.0f;  // raw z, consumed by the recompute epilogue
    }
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const int e = tid + q * NT;
      if (e < N * CK) {
        const int tt = e / N, nn = e % N;
        const bool ok = ts + tt < seq;
        s_B[nn][tt] = ok ? to_f32(pb[q]) : 0.0f;
        s_C[nn][tt] = ok ? to_f32(pc[q]) : 0.0f;
      }
    }
    if (k > 0) fetch((k - 1) * CK);
    __syncthreads();

    // ---- recompute the chunk's states ------------------------------------
    float h0[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      h0[s] = (k > 0 && cvalid) ? p.ckpt[(((long)b * dim + c) * p.nck + (k - 1)) * N + n * SPL + s] : 0.0f;
    float hs[CK][SPL], as[CK][SPL];
    {
      float hh[SPL];
#pragma unroll
      for (int s = 0; s < SPL; ++s) hh[s] = h0[s];
#pragma unroll
      for (int j = 0; j < CK; ++j) {
        const float dtc = s_dtc[cl][j];
        const float dtx = s_dtb[cl][j] * s_x[cl][j];
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          const int nn = n * SPL + s;
          const float a = fast_exp2(dtc * A2[s]);
          hh[s] = fmaf(a, hh[s], dtx * s_B[nn][j]);
          as[j][s] = a;
          hs[j][s] = hh[s];
        }
      }
    }

    // ---- gate: dy = dout * silu(z); dz = dout * y * silu'(z) ---------------
    if (z != nullptr) {
#pragma unroll
      for (int jb = 0; jb < CK; jb += TS) {
#pragma unroll
        for (int j = 0; j < TS; ++j) {
          float acc = 0.0f;
#pragma unroll
          for (int s = 0; s < SPL; ++s) acc = fmaf(s_C[n * SPL + s][jb + j], hs[jb + j][s], acc);
          s_r[0][tid][j] = acc;
        }
        __syncthreads();
        for (int q = n; q < TS; q += LPC) {
          float y = 0.0f;
#pragma unroll
          for (int m = 0; m < LPC; ++m) y += s_r[0][cl * LPC + m][q];
          const int j = jb + q;
          y = fmaf(Dc, s_x[cl][j], y);
          const float zv = s_o[0][j][cl];
          const float sg = sigmoidf(zv);
          const float go = s_dy[cl][j];
          s_dy[cl][j] = go * zv * sg;
          s_o[1][j][cl] = go * y * sg * (1.0f + zv * (1.0f - sg));
        }
        __syncthreads();
      }
      if (p.dz != nullptr) {
        for (int e = tid; e < CPW * CK; e += NT) {
          const int tt = e / CPW, ch = e % CPW;
          const int t = ts + tt, cc = c0 + ch;
          if (t < seq && cc < dim) st((TI*)p.dz, rowbase + (long)t * dim + cc, s_o[1][tt][ch]);
        }
      }
      __syncthreads();
    }

    // ---- reverse recurrence over the chunk ---------------------------------
#pragma unroll
    for (int jb = CK - TS; jb >= 0; jb -= TS) {
#pragma unroll
      for (int j = TS - 1; j >= 0; --j) {
        const int jj = jb + j;
        const float dyv = s_dy[cl][jj];
        const float dtc = s_dtc[cl][jj];
        const float dtx = s_dtb[cl][jj] * s_x[cl][jj];
        float px = 0.0f, pa = 0.0f, gC = 0.0f, gB = 0.0f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          const int nn = n * SPL + s;
          const float Bv = s_B[nn][jj];
          const float Cv = s_C[nn][jj];
          dh[s] = fmaf(dyv, Cv, dh[s]);
          const float hp = jj > 0 ? hs[jj - 1][s] : h0[s];
          gC = dyv * hs[jj][s];
          gB = dh[s] * dtx;
          px = fmaf(dh[s], Bv, px);
          const float ga = dh[s] * hp * as[jj][s];
          dA[s] = fmaf(ga, dtc, dA[s]);
          pa = fmaf(ga, A1[s], pa);
          dh[s] *= as[jj][s];
        }
        s_r[0][tid][j] = px;
        s_r[1][tid][j] = pa;
        s_r[2][tid][j] = gC;
        s_r[3][tid][j] = gB;
      }
      __syncthreads();
      // sums over states: dx, ddt per (t, channel)
      for (int q = n; q < TS; q += LPC) {
        float px = 0.0f, pa = 0.0f;
#pragma unroll
        for (int m = 0; m < LPC; ++m) {
          px += s_r[0][cl * LPC + m][q];
          pa += s_r[1][cl * LPC + m][q];
        }
        const int jj = jb + q;
        const float xv = s_x[cl][jj];
        const float dyv = s_dy[cl][jj];
        dD = fmaf(dyv, xv, dD);
        s_o[0][jj][cl] = fmaf(px, s_dtb[cl][jj], dyv * Dc);
        const float g = mean_mode ? pa : pa + px * xv;
        s_o[1][jj][cl] = s_rng[cl][jj] * g;
        if (mean_mode) s_r[0][cl * LPC + n][q] = px * xv;  // reused below for the dt-mean coupling
      }
      // sums over channels: dC (qty 0) and dB (qty 1) per (t, n) for this workgroup's tile
      for (int e = tid; e < 2 * N * TS; e += NT) {
        const int qty = e / (N * TS);
        const int r = e % (N * TS);
        const int nn = r / TS, q = r % TS;
        float acc = 0.0f;
        for (int ch = 0; ch < CPW; ++ch) acc += s_r[2 + qty][ch * LPC + nn][q];
        const int t = ts + jb + q;
        if (t < seq) p.part_bc[((((long)tile * p.batch + b) * seq + t) * 2 + qty) * N + nn] = acc;
      }
      __syncthreads();
      if (mean_mode) {
        for (int q = tid; q < TS; q += NT) {
          float acc = 0.0f;
          for (int ch = 0; ch < CPW; ++ch) acc += s_r[0][ch * LPC + (q % LPC)][q];
          const int t = ts + jb + q;
          if (t < seq) p.part_m[((long)tile * p.batch + b) * seq + t] = acc;
        }
        __syncthreads();
      }
    }
    // ---- write dx, ddt rows for the chunk ------------------------------------
    for (int e = tid; e < CPW * CK; e += NT) {
      const int tt = e / CPW, ch = e % CPW;
      const int t = ts + tt, cc = c0 + ch;
      if (t < seq && cc < dim) {
        const long idx = rowbase + (long)t * dim + cc;
        st((TI*)p.dx, idx, s_o[0][tt][ch]);
        st((TI*)p.ddt, idx, s_o[1][tt][ch]);
      }
    }
    __syncthreads();
  }
  // dA partial per (b, d, n); dD partial per (b, d)
  if (cvalid) {
#pragma unroll
    for (int s = 0; s < SPL; ++s) p.part_a[((long)b * dim + c) * N + n * SPL + s] = dA[s];
  }
  // dD: lanes of a channel hold disjoint timesteps; reduce over the LPC lanes
  s_r[0][tid][0] = dD;
  __syncthreads();
  if (n == 0 && cvalid) {
    float acc = 0.0f;
    for (int m = 0; m < LPC; ++m) acc += s_r[0][cl * LPC + m][0];
    p.part_d[(long)b * dim + c] = acc;
  }
}

// dB, dC = sum over channel tiles
__global__ __launch_bounds__(256) void ss_reduce_bc_kernel(const float* __restrict__ part, float* __restrict__ dB,
                                                           float* __restrict__ dC, int ntile, long rows, int N) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // over rows * 2N
  const long total = rows * 2 * N;
  if (i >= total) return;
  float acc = 0.0f;
  for (int tl = 0; tl < ntile; ++tl) acc += part[(long)tl * total + i];
  const long row = i / (2 * N);
  const int r = (int)(i % (2 * N));
  const int qty = r / N, nn = r % N;
  if (qty == 0) {
    if (dC) dC[row * N + nn] = acc;
  } else {
    if (dB) dB[row * N + nn] = acc;
  }
}

// dA[d, n] = sum_b part_a; dD[d] = sum_b part_d
__global__ __launch_bounds__(256) void ss_reduce_ad_kernel(const float* __restrict__ part_a,
                                                           const float* __restrict__ part_d, float* __restrict__ dA,
                                                           float* __restrict__ dD, int batch, int dim, int N) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const long na = (long)dim * N;
  if (i < na) {
    float acc = 0.0f;
    for (int bb = 0; bb < batch; ++bb) acc += part_a[(long)bb * na + i];
    if (dA) dA[i] = acc;
  } else if (i < na + dim) {
    const long d = i - na;
    float acc = 0.0f;
    for (int bb = 0; bb < batch; ++bb) acc += part_d[(long)bb * dim + d];
    if (dD) dD[d] = acc;
  }
}

// mean mode: ddt[b,t,d] += in_range * (sum over tiles part_m[b,t]) / dim
template <typename TI>
__global__ __launch_bounds__(256) void ss_mean_fixup_kernel(const float* __restrict__ part_m,
                                                            const TI* __restrict__ dt, TI* __restrict__ ddt,
                                                            int ntile, long rows, int dim) {
  const long row = blockIdx.x;
  if (row >= rows) return;
  float tot = 0.0f;
  for (int tl = 0; tl < ntile; ++tl) tot += part_m[(long)tl * rows + row];
  tot /= (float)dim;
  for (int d = threadIdx.x; d < dim; d += 256) {
    const long idx = row * dim + d;
    const float dtr = ld(dt, idx);
    if (dtr >= DT_MIN && dtr <= DT_MAX) st(ddt, idx, ld(ddt, idx) + tot);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr int FWD_NT = 256;
constexpr int BWD_NT = 256;

inline int ss_ck(int N) { return N <= 16 ? 32 : 16; }

inline bool pow2_state(int N) { return N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32; }

inline int ntiles(int dim, int N, int nt) {
  const int lpc = N < 16 ? N : 16;
  const int cpw = nt / lpc;
  return (dim + cpw - 1) / cpw;
}

struct WsLayout {
  size_t ckpt, dtmean, part_bc, part_a, part_d, part_m, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline WsLayout bwd_layout(int batch, int seq, int dim, int N, bool need_ckpt, bool mean_mode) {
  WsLayout w{};
  const int ck = ss_ck(N);
  const long nck = (seq + ck - 1) / ck;
  const int nt = ntiles(dim, N, BWD_NT);
  size_t off = 0;
  w.ckpt = off;
  if (need_ckpt) off += align256((size_t)batch * dim * nck * N * 4);
  w.dtmean = off;
  if (mean_mode) off += align256((size_t)batch * seq * 4);
  w.part_bc = off;
  off += align256((size_t)nt * batch * seq * 2 * N * 4);
  w.part_a = off;
  off += align256((size_t)batch * dim * N * 4);
  w.part_d = off;
  off += align256((size_t)batch * dim * 4);
  w.part_m = off;
  if (mean_mode) off += align256((size_t)nt * batch * seq * 4);
  w.total = off;
  return w;
}

template <typename TI, typename TP, int N>
void launch_fwd_t(hipStream_t s, const SSArgs& a) {
  const int grid = a.batch * a.ntile;
  const bool mean = a.dtmean != nullptr, hz = a.z != nullptr;
  if (mean && hz) ss_fwd_kernel<TI, TP, N, FWD_NT, true, true><<<grid, FWD_NT, 0, s>>>(a);
  else if (mean) ss_fwd_kernel<TI, TP, N, FWD_NT, true, false><<<grid, FWD_NT, 0, s>>>(a);
  else if (hz) ss_fwd_kernel<TI, TP, N, FWD_NT, false, true><<<grid, FWD_NT, 0, s>>>(a);
  else ss_fwd_kernel<TI, TP, N, FWD_NT, false, false><<<grid, FWD_NT, 0, s>>>(a);
}

template <typename TI, typename TP>
int launch_fwd_n(hipStream_t s, const SSArgs& a, int N) {
  switch (N) {
    case 1: launch_fwd_t<TI, TP, 1>(s, a); break;
    case 2: launch_fwd_t<TI, TP, 2>(s, a); break;
    case 4: launch_fwd_t<TI, TP, 4>(s, a); break;
    case 8: launch_fwd_t<TI, TP, 8>(s, a); break;
    case 16: launch_fwd_t<TI, TP, 16>(s, a); break;
    case 32: launch_fwd_t<TI, TP, 32>(s, a); break;
    default: return set_error(EDF_ERR_UNSUPPORTED, "state size %d unsupported (1, 2, 4, 8, 16 or 32)", N);
  }
  return check_launch("selective scan");
}

template <typename TI, typename TP, int N>
void launch_bwd_t(hipStream_t s, const SSArgs& a) {
  const int grid = a.batch * a.ntile;
  ss_bwd_kernel<TI, TP, N, BWD_NT, 32><<<grid, BWD_NT, 0, s>>>(a);
}

template <typename TI, typename TP>
int launch_bwd_n(hipStream_t s, const SSArgs& a, int N) {
  switch (N) {
    case 4: launch_bwd_t<TI, TP, 4>(s, a); break;
    case 8: launch_bwd_t<TI, TP, 8>(s, a); break;
    case 16: launch_bwd_t<TI, TP, 16>(s, a); break;
    default: return set_error(EDF_ERR_UNSUPPORTED, "backward state size %d unsupported (4, 8 or 16)", N);
  }
  return check_launch("selective scan backward");
}

template <typename F>
int by_dtypes(int io, int par, F&& f) {
  if (io == EDF_BF16 && par == EDF_BF16) return f((bf16*)nullptr, (bf16*)nullptr);
  if (io == EDF_BF16 && par == EDF_F32) return f((bf16*)nullptr, (float*)nullptr);
  if (io == EDF_F32 && par == EDF_BF16) return f((float*)nullptr, (bf16*)nullptr);
  return f((float*)nullptr, (float*)nullptr);
}

int check_common(int batch, int seq, int dim, int N, int io, int par, int mode) {
  EDF_REQUIRE(batch > 0 && seq > 0 && dim > 0 && N > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(io) && valid_dtype(par), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(pow2_state(N), EDF_ERR_UNSUPPORTED, "state size %d unsupported (1, 2, 4, 8, 16 or 32)", N);
  EDF_REQUIRE(mode == EDF_SS_DT_PER_CHANNEL || mode == EDF_SS_DT_MEAN, EDF_ERR_INVALID_ARG, "unknown dt mode %d",
              mode);
  return EDF_OK;
}

int run_dtmean(hipStream_t s, const void* dt, float* dtm, int batch, int seq, int dim, int io) {
  const int rows = batch * seq;
  const int grid = (rows + 3) / 4;
  if (io == EDF_BF16)
    ss_dtmean_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)dt, dtm, rows, dim);
  else
    ss_dtmean_kernel<float><<<grid, 256, 0, s>>>((const float*)dt, dtm, rows, dim);
  return check_launch("selective scan dt mean");
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_selective_scan_states_bytes(int batch, int seq_len, int hidden, int state) {
  if (batch <= 0 || seq_len <= 0 || hidden <= 0 || state <= 0) return 0;
  const int ck = edf::ss_ck(state);
  const size_t nck = (size_t)(seq_len + ck - 1) / ck;
  return (size_t)batch * hidden * nck * state * sizeof(float);
}

size_t edf_selective_scan_workspace_bytes(int batch, int seq_len, int hidden, int state, int mode) {
  if (batch <= 0 || seq_len <= 0) return 0;
  return mode == EDF_SS_DT_MEAN ? edf::align256((size_t)batch * seq_len * 4) : 0;
}

size_t edf_selective_scan_backward_workspace_bytes(int batch, int seq_len, int hidden, int state, int mode,
                                                   int have_states) {
  if (batch <= 0 || seq_len <= 0 || hidden <= 0 || state <= 0) return 0;
  return edf::bwd_layout(batch, seq_len, hidden, state, !have_states, mode == EDF_SS_DT_MEAN).total;
}

int edf_fused_selective_scan(void* stream, const void* x, const void* dt, const void* A, const void* B, const void* C,
                             const void* D, const void* z, void* out, void* states, void* workspace,
                             size_t workspace_bytes, int batch, int seq_len, int hidden, int state, int io_dtype,
                             int param_dtype, int mode) {
  using namespace edf;
  int rc = check_common(batch, seq_len, hidden, state, io_dtype, param_dtype, mode);
  if (rc) return rc;
  EDF_REQUIRE(x && dt && A && B && C && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf_selective_scan_workspace_bytes(batch, seq_len, hidden, state, mode);
  EDF_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), EDF_ERR_WORKSPACE,
              "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  SSArgs a{};
  a.x = x; a.dt = dt; a.A = A; a.B = B; a.C = C; a.D = D; a.z = z; a.out = out;
  a.ckpt = (float*)states;
  a.batch = batch; a.seq = seq_len; a.dim = hidden;
  a.ck = ss_ck(state);
  a.nck = (seq_len + a.ck - 1) / a.ck;
  a.ntile = ntiles(hidden, state, FWD_NT);
  if (mode == EDF_SS_DT_MEAN) {
    a.dtmean = (float*)workspace;
    rc = run_dtmean(s, dt, (float*)workspace, batch, seq_len, hidden, io_dtype);
    if (rc) return rc;
  }
  return by_dtypes(io_dtype, param_dtype, [&](auto* ti, auto* tp) {
    using TI = std::remove_pointer_t<decltype(ti)>;
    using TP = std::remove_pointer_t<decltype(tp)>;
    return launch_fwd_n<TI, TP>(s, a, state);
  });
}

int edf_fused_selective_scan_backward(void* stream, const void* x, const void* dt, const void* A, const void* B,
                                      const void* C, const void* D, const void* z, const void* grad_out,
                                      const void* states, void* grad_x, void* grad_dt, void* grad_A, void* grad_B,
                                      void* grad_C, void* grad_D, void* grad_z, void* workspace,
                                      size_t workspace_bytes, int batch, int seq_len, int hidden, int state,
                                      int io_dtype, int param_dtype, int mode) {
  using namespace edf;
  int rc = check_common(batch, seq_len, hidden, state, io_dtype, param_dtype, mode);
  if (rc) return rc;
  EDF_REQUIRE(state == 4 || state == 8 || state == 16, EDF_ERR_UNSUPPORTED,
              "backward state size %d unsupported (4, 8 or 16)", state);
  EDF_REQUIRE(x && dt && A && B && C && grad_out && grad_x && grad_dt, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const bool mean_mode = mode == EDF_SS_DT_MEAN;
  const WsLayout L = bwd_layout(batch, seq_len, hidden, state, states == nullptr, mean_mode);
  EDF_REQUIRE(workspace && workspace_bytes >= L.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              L.total);
  hipStream_t s = as_stream(stream);
  char* ws = (char*)workspace;
  SSArgs a{};
  a.x = x; a.dt = dt; a.A = A; a.B = B; a.C = C; a.D = D; a.z = z;
  a.batch = batch; a.seq = seq_len; a.dim = hidden;
  a.ck = ss_ck(state);
  a.nck = (seq_len + a.ck - 1) / a.ck;
  if (mean_mode) {
    a.dtmean = (float*)(ws + L.dtmean);
    rc = run_dtmean(s, dt, (float*)(ws + L.dtmean), batch, seq_len, hidden, io_dtype);
    if (rc) return rc;
  }
  a.ckpt = states ? (float*)states : (float*)(ws + L.ckpt);
  if (states == nullptr) {  // recompute checkpoints with a forward pass that writes no output
    SSArgs f = a;
    f.out = nullptr;
    f.ntile = ntiles(hidden, state, FWD_NT);
    rc = by_dtypes(io_dtype, param_dtype, [&](auto* ti, auto* tp) {
      using TI = std::remove_pointer_t<decltype(ti)>;
      using TP = std::remove_pointer_t<decltype(tp)>;
      return launch_fwd_n<TI, TP>(s, f, state);
    });
    if (rc) return rc;
  }
  a.dout = grad_out;
  a.dx = grad_x;
  a.ddt = grad_dt;
  a.dz = grad_z;
  a.part_bc = (float*)(ws + L.part_bc);
  a.part_a = (float*)(ws + L.part_a);
  a.part_d = (float*)(ws + L.part_d);
  a.part_m = mean_mode ? (float*)(ws + L.part_m) : nullptr;
  a.ntile = ntiles(hidden, state, BWD_NT);
  rc = by_dtypes(io_dtype, param_dtype, [&](auto* ti, auto* tp) {
    using TI = std::remove_pointer_t<decltype(ti)>;
    using TP = std::remove_pointer_t<decltype(tp)>;
    return launch_bwd_n<TI, TP>(s, a, state);
  });
  if (rc) return rc;
  const long rows = (long)batch * seq_len;
  if (grad_B || grad_C) {
    const long total = rows * 2 * state;
    ss_reduce_bc_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(a.part_bc, (float*)grad_B, (float*)grad_C,
                                                                        a.ntile, rows, state);
    rc = check_launch("selective scan dB/dC reduction");
    if (rc) return rc;
  }
  if (grad_A || grad_D) {
    const long total = (long)hidden * state + hidden;
    ss_reduce_ad_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(a.part_a, a.part_d, (float*)grad_A,
                                                                        (float*)grad_D, batch, hidden, state);
    rc = check_launch("selective scan dA/dD reduction");
    if (rc) return rc;
  }
  if (mean_mode) {
    if (io_dtype == EDF_BF16)
      ss_mean_fixup_kernel<bf16><<<(unsigned)rows, 256, 0, s>>>(a.part_m, (const bf16*)dt, (bf16*)grad_dt, a.ntile,
                                                                rows, hidden);
    else
      ss_mean_fixup_kernel<float><<<(unsigned)rows, 256, 0, s>>>(a.part_m, (const float*)dt, (float*)grad_dt,
                                                                 a.ntile, rows, hidden);
    rc = check_launch("selective scan dt-mean coupling");
    if (rc) return rc;
  }
  return EDF_OK;
}

}  // extern "C"
