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
//   Optional extensions: y += D[d] x, then y *= silu(z); in dt-mean mode, dt given before its
//   softplus (the EDF_SS_DT_SOFTPLUS mode flag: softplus(dt) wherever dt is read, grad_dt
//   with respect to the pre-activation).
//
// Design.  The op is VALU-bound: per (b, t, d, n) element the forward needs one
// v_exp_f32 and four other VALU ops, several times the HBM time at config-2 size, so the
// layout is chosen to keep every SIMD busy and to spend little else per element:
//   * one state per lane.  A wave holds SW = 4 states (one per 16-lane DPP row) of
//     CW = 16 channels (fewer states, more channels when N < 4); a workgroup holds G
//     such channel groups and all N states of them (G N / SW waves).  At config 2
//     (B = 8, D = 1536, N = 16) G = 3 gives 256 workgroups of 12 waves: every CU gets one,
//     3 waves per SIMD.  (One workgroup per (b, 64-channel tile) gave 192 workgroups: 64
//     CUs idle.)  The host picks G from the grid it would produce;
//   * B[b, t, n] and C[b, t, n] are the same for the 16 lanes of a row: a block of 16
//     timesteps sits in one VGPR (lane i of the row holds step i of the row's state) and
//     reaches the row through DPP row_newbcast, folded into v_mul_f32_dpp: no LDS traffic;
//   * x, dt (and z) are staged per block of 16 timesteps through LDS from coalesced rows,
//     clip(dt) and dt_b x computed once per (t, d); the recurrence reads them as 16-byte
//     vectors (the four rows of a wave read the same addresses);
//   * y = sum_n C h: every lane writes C h for its (state, t, d) to an LDS tile and the
//     thread that staged (t, d) adds the N values, applies the D skip and the gate and
//     stores y; double-buffered tiles need one barrier per block; raw inputs are
//     prefetched four blocks ahead;
//   * the forward writes the state every CK = 16 timesteps ("checkpoints", layout
//     [b][chunk][n][d], coalesced over d) and, with a gate, the pre-gate y (for dz) into
//     the same caller buffer, so the backward recomputes neither;
//   * any state size 1..32 (the reference's limit): the kernels are compiled for the next
//     power of two NP >= N and the states past N are padding, with A = B = C = 0 loaded
//     for them, so they stay 0 and add nothing; A, B, C, dA, dB and dC keep the caller's
//     stride N, checkpoints and partial sums the padded NP;
//   * backward: chunks of 16 steps in reverse, each chunk's states and decays recomputed
//     from its checkpoint into registers, then the reverse recurrence in two halves of 8
//     steps.  Every lane writes its four per-element terms (dx and ddt terms summed over
//     states, dC and dB terms summed over channels) to LDS tiles; after a barrier all
//     threads reduce them: (t, d, quantity) sums over the N states -> dx, ddt; (t, n,
//     quantity, channel group) sums over 16 channels, added over the G groups one half
//     later into one partial per workgroup, summed over the workgroups by a small
//     deterministic kernel (no atomics).
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr float DT_MIN = 1.0e-3f;
constexpr float DT_MAX = 0.1f;
constexpr int SS_CK = 16;  // checkpoint interval (timesteps) = recompute chunk = lanes per DPP row

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
  float* ckpt;  // [batch, nck, N, dim] state after each chunk of SS_CK timesteps
  void* ypre;   // [batch, seq, dim] y before the gate (io type), written with a gate
  // backward only
  const void* dout;
  void* dx;
  void* ddt;
  void* dz;
  float* part_bc;  // [ntile, batch, seq, 2, N]  (qty 0 = dC, 1 = dB)
  float* part_a;   // [batch, dim, N]
  float* part_d;   // [batch, dim]
  float* part_m;   // [ntile, batch, seq] (mean mode)
  int batch, seq, dim, nck, ntile;
  int nst;    // the caller's state count N (<= the kernel's padded NP): stride of A, B, C rows
  int dt_sp;  // dt holds the pre-activation: softplus(dt) is read, grad_dt is with respect to dt
};

// Lane layout: one state per lane; a wave holds SW states (each on 64 / SW lanes, whole
// 16-lane DPP rows) of CW channels; a workgroup holds G channel groups x all N states.
template <int N, int G>
struct RGeo {
  static constexpr int SW = N < 4 ? N : 4;  // states per wave
  static constexpr int CW = 64 / SW;        // channels per wave
  static constexpr int NSG = N / SW;        // state groups
  static constexpr int NW = G * NSG;        // waves per workgroup
  static constexpr int NT = 64 * NW;
  static constexpr int CT = G * CW;         // channels per workgroup
  static_assert(NW <= 16, "at most 16 waves per workgroup");
};

// the wide channel-group count compiled per state size (the narrow one is G = 1)
template <int N> constexpr int ss_gwide() { return N >= 32 ? 1 : (N == 16 ? 3 : (N >= 4 ? 4 : 1)); }

EDF_DEVICE int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// DPP quad_perm [1, 0, 3, 2]: the value of the neighbouring lane of a lane pair
EDF_DEVICE float pair_swap(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}

// ---------------------------------------------------------------------------
// dt mean over channels (block semantics), one wave per (b, t)
// ---------------------------------------------------------------------------
template <typename TI>
__global__ __launch_bounds__(256) void ss_dtmean_kernel(const TI* __restrict__ dt, float* __restrict__ dtm, int rows,
                                                        int dim, int sp) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const TI* p = dt + (long)row * dim;
  float s = 0.0f;
  constexpr int V = 16 / sizeof(TI);  // one 16-byte load per lane and step when the row allows it
  if (dim % V == 0 && ((uintptr_t)dt & 15) == 0) {
    for (int d0 = lane * V; d0 < dim; d0 += 64 * V) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + d0);
      const TI* e = reinterpret_cast<const TI*>(&u);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float v = to_f32(e[i]);
        s += clampf(sp ? softplus_f(v) : v, DT_MIN, DT_MAX);
      }
    }
  } else {
    for (int d = lane; d < dim; d += 64) {
      const float v = ld(p, d);
      s += clampf(sp ? softplus_f(v) : v, DT_MIN, DT_MAX);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) dtm[row] = s / (float)dim;
}

// Padded length of an LDS row holding the N states of one (t, channel): 16-byte reads of
// the rows of 16 consecutive channels are conflict-free (PN / 4 odd), and so are one
// wave's writes (16 channels x 4 states) with the slot swizzle below.
template <int N> constexpr int ss_pn() { return N == 4 ? 12 : N + 4; }
// A 32-lane half of a ds_write_b32 spreads over 32 banks (word address mod 32); the rows of
// one wave's state-term writes (16 channels x states r, r + 1 per half) lie PN words apart,
// and PN * 8 = 0 mod 32 for every PN above, so channels j and j + 8 would share a bank.
// Channels with bit 3 set keep their states in the row at s ^ 2 (rows hold N >= 4 states;
// sums over a whole row are unchanged).  16-byte reads of whole rows are untouched.
template <int N> EDF_DEVICE int ss_swz(int cl) { return N >= 4 ? (cl & 8) >> 2 : 0; }
constexpr int mod64_to(int v, int r) { return v + ((r - v % 64) % 64 + 64) % 64; }  // smallest >= v, = r mod 64
// Row stride of the dC / dB tile's state rows: a 16-channel row pair of one 32-lane write
// needs rows 16 apart mod 32 words; 2 SSR is then 32 mod 64, which the paired channel-sum
// reads rely on.  Wider rows (N < 4) keep a 64-word residue of their channel count.
constexpr int ss_ssr(int v, int cw) { return cw == 16 ? v + ((16 - v % 32) % 32 + 32) % 32 : mod64_to(v, cw % 64); }

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// WRITE_Y: store the gated output.  With a gate, y before the gate is stored into p.ypre
// (through a zero-length resource, i.e. dropped, when p.ypre is null); without WRITE_Y
// and without a gate only the checkpoints are written.
template <typename TI, typename TP, int N, int G, bool MEAN, bool HAS_Z, bool WRITE_Y>
__global__ __launch_bounds__((RGeo<N, G>::NT)) void ss_fwd_kernel(const SSArgs p, const TP* __restrict__ Bm,
                                                                const TP* __restrict__ Cm) {
  using Geo = RGeo<N, G>;
  constexpr int SW = Geo::SW, CW = Geo::CW, NT = Geo::NT, CT = Geo::CT;
  constexpr int TS = SS_CK;                 // timesteps per block (one checkpoint per block)
  constexpr int PS = TS + 4;                // [channel][t] row stride: 16-byte reads are conflict-free
  constexpr int NE = TS * CT;               // staged (t, channel) elements per block
  constexpr int EPT = (NE + NT - 1) / NT;   // per thread
  constexpr bool SAVE_YP = HAS_Z;
  constexpr bool YSUM = WRITE_Y || SAVE_YP;
  constexpr int PN = ss_pn<N>();            // C h tile [t][channel][state], rows of PN floats
  constexpr int PD = N >= 8 ? 4 : 2;        // prefetch distance (blocks)
  static_assert(PD % 2 == 0, "the LDS buffer parity follows the ring slot");
  __shared__ __align__(16) float s_dtc[2][CT][PS];
  __shared__ __align__(16) float s_dtx[2][CT][PS];
  __shared__ __align__(16) float s_yp[YSUM ? 2 : 1][YSUM ? TS * CT * PN : 1];

  const TI* __restrict__ x = (const TI*)p.x;
  const TI* __restrict__ dt = (const TI*)p.dt;
  const TI* __restrict__ z = (const TI*)p.z;
  const TP* __restrict__ Am = (const TP*)p.A;
  const TP* __restrict__ Dv = (const TP*)p.D;
  const int seq = p.seq, dim = p.dim;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int g = w % G, sg = w / G;          // this wave's channel group and state group
  const int s = sg * SW + lane / CW;        // this lane's state
  const int cl = g * CW + lane % CW;        // this lane's channel within the tile
  const int sx = s ^ ss_swz<N>(cl);         // its slot in a C h row
  const int logical = remap_xcd(blockIdx.x, gridDim.x);
  const int b = logical / p.ntile, tile = logical % p.ntile;
  const int c = tile * CT + cl;
  const bool cvalid = c < dim;

  const int ns = p.nst;
  const float A2 = (cvalid && s < ns) ? ld(Am, (long)c * ns + s) * LOG2E : 0.0f;
  float h = 0.0f;

  // the (t, channel) elements this thread stages and finishes: e = tid + i NT
  int et[EPT], ec[EPT];
  bool ev[EPT];
  float eD[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = tid + i * NT;
    et[i] = e / CT;
    ec[i] = e % CT;
    ev[i] = e < NE && tile * CT + ec[i] < dim;
    eD[i] = (Dv != nullptr && ev[i]) ? ld(Dv, tile * CT + ec[i]) : 0.0f;
  }
  const long rowbase = (long)b * seq * dim;
  // every global access goes through a buffer resource on this batch row: SGPR base plus a
  // 32-bit offset (no 64-bit address VALU), out-of-range offsets load 0 / drop the store
  typedef typename Bits<TI>::type RI;
  typedef typename Bits<TP>::type RP;
  const unsigned rowbytes = (unsigned)((long)seq * dim * sizeof(TI));
  const rsrc_t r_x = make_rsrc(x + rowbase, rowbytes), r_dt = make_rsrc(dt + rowbase, rowbytes);
  const rsrc_t r_z = make_rsrc(HAS_Z ? z + rowbase : x + rowbase, rowbytes);
  const rsrc_t r_y = make_rsrc(WRITE_Y ? (TI*)p.out + rowbase : x + rowbase, WRITE_Y ? rowbytes : 0u);
  const rsrc_t r_yp = make_rsrc(SAVE_YP && p.ypre != nullptr ? (TI*)p.ypre + rowbase : x + rowbase,
                                SAVE_YP && p.ypre != nullptr ? rowbytes : 0u);
  const unsigned bcbytes = (unsigned)((long)seq * ns * sizeof(TP));
  const rsrc_t r_B = make_rsrc(Bm + (long)b * seq * ns, bcbytes), r_C = make_rsrc(Cm + (long)b * seq * ns, bcbytes);
  const rsrc_t r_m =
      make_rsrc(MEAN ? (const void*)(p.dtmean + (long)b * seq) : (const void*)x, (unsigned)(seq * sizeof(float)));
  const unsigned ckbytes = (unsigned)((long)p.nck * N * dim * sizeof(float));
  const rsrc_t r_ck = make_rsrc(p.ckpt != nullptr ? (const void*)(p.ckpt + (long)b * p.nck * N * dim) : (const void*)x,
                                p.ckpt != nullptr ? ckbytes : 0u);

  // Raw values of the blocks ahead, loaded PD blocks early from clamped (in-bounds)
  // indices so no load sits behind a divergent branch; kept in the storage type until
  // staged.  B/C: lane i of each 16-lane row loads step t0 + i of the row's state.
  RI rx[PD][EPT], rdt[PD][EPT], rz[PD][EPT];
  RP rB[PD], rC[PD];
  float rm[PD][EPT];
  float cx[EPT], cz[EPT], nx[EPT], nz[EPT];
  auto fetch = [&](int slot, int t0) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int t = min(t0 + et[i], seq - 1);
      const unsigned off = ev[i] ? ((unsigned)t * dim + tile * CT + ec[i]) * (unsigned)sizeof(TI) : OOB_OFF;
      rx[slot][i] = bload<TI>(r_x, off);
      rdt[slot][i] = bload<TI>(r_dt, off);
      if (HAS_Z) rz[slot][i] = bload<TI>(r_z, off);
      rm[slot][i] = MEAN ? bits_f32(bload<float>(r_m, (unsigned)t * 4u)) : 0.0f;
    }
    // padding states (s >= ns) read 0 through an out-of-range offset
    const unsigned off = s < ns ? ((unsigned)(t0 + min(lane & 15, seq - 1 - t0)) * ns + s) * (unsigned)sizeof(TP)
                                : OOB_OFF;
    rB[slot] = bload<TP>(r_B, off);
    rC[slot] = bload<TP>(r_C, off);
  };
  auto stage = [&](int slot, int t0, int buf, float* xs, float* zs) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const bool ok = ev[i] && t0 + et[i] < seq;
      const float xv = bits_f32(rx[slot][i]);
      float dtr = bits_f32(rdt[slot][i]);
      if constexpr (MEAN) {  // the softplus flag exists in dt-mean mode only: C2's kernels stay as they were
        if (p.dt_sp) dtr = softplus_f(dtr);
      }
      const float dtc = ok ? clampf(dtr, DT_MIN, DT_MAX) : 0.0f;
      if (NE % NT == 0 || tid + i * NT < NE) {
        s_dtc[buf][ec[i]][et[i]] = dtc;
        s_dtx[buf][ec[i]][et[i]] = ok ? (MEAN ? rm[slot][i] : dtc) * xv : 0.0f;
      }
      xs[i] = xv;
      zs[i] = HAS_Z ? bits_f32(rz[slot][i]) : 0.0f;
    }
  };

  // Pipeline: raw slot j holds block j mod PD.  Block blk is computed from LDS buffer
  // blk & 1 and from its B/C values in slot blk % PD; then block blk + 1 is staged into
  // the other LDS buffer and block blk + PD is fetched into slot blk % PD, which block
  // blk no longer needs.
  // Every fetch and stage is unconditional (block indices clamped to the last block, and
  // the block count padded to a multiple of PD with empty blocks whose staged dt is 0,
  // i.e. identity steps): a conditional refill makes the compiler drain the whole ring
  // (vmcnt(0)) at the loop head.  Only stores are guarded.
  const int nblk = (seq + TS - 1) / TS;
  const int npad = (nblk + PD - 1) / PD * PD;
#pragma unroll
  for (int jb = 0; jb < PD; ++jb) fetch(jb, min(jb, nblk - 1) * TS);
  stage(0, 0, 0, cx, cz);
  __syncthreads();

  for (int blk0 = 0; blk0 < npad; blk0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int blk = blk0 + u;
      const int t0 = blk * TS, buf = u & 1;  // PD is even, so u & 1 == blk & 1
      // ---- recurrence over the block ----
      const float rb = bits_f32(rB[u]), rc = bits_f32(rC[u]);
      static_for<TS / 4>([&](auto qi) {
        constexpr int q = decltype(qi)::value;
        const float4 dc4 = *reinterpret_cast<const float4*>(&s_dtc[buf][cl][4 * q]);
        const float4 dx4 = *reinterpret_cast<const float4*>(&s_dtx[buf][cl][4 * q]);
        const float dcv[4] = {dc4.x, dc4.y, dc4.z, dc4.w};
        const float dxv[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
        static_for<4>([&](auto vi) {
          constexpr int v = decltype(vi)::value, tt = 4 * q + v;
          const float a = fast_exp2(dcv[v] * A2);
          h = fmaf(a, h, row_bcast<tt>(rb) * dxv[v]);
          if (YSUM) s_yp[buf][(tt * CT + cl) * PN + sx] = row_bcast<tt>(rc) * h;
        });
      });
      if (p.ckpt != nullptr)
        bstore<float>(r_ck, (cvalid && blk < nblk) ? (((unsigned)blk * N + s) * dim + c) * 4u : OOB_OFF, h);
      stage((u + 1) % PD, t0 + TS, buf ^ 1, nx, nz);
      fetch(u, min(blk + PD, nblk - 1) * TS);
      __syncthreads();
      // ---- y for the (t, d) this thread staged: sum over the states, D skip, gate ----
      if (YSUM) {
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          if (NE % NT != 0 && tid + i * NT >= NE) continue;
          const float* src = &s_yp[buf][(et[i] * CT + ec[i]) * PN];
          float y;
          if constexpr (PN % 4 == 0) {
            const float4 f0 = *reinterpret_cast<const float4*>(src);
            y = (f0.x + f0.y) + (f0.z + f0.w);
#pragma unroll
            for (int v = 4; v < N; v += 4) {
              const float4 f = *reinterpret_cast<const float4*>(src + v);
              y += (f.x + f.y) + (f.z + f.w);
            }
          } else {
            y = src[0];
#pragma unroll
            for (int v = 1; v < N; ++v) y += src[v];
          }
          y = fmaf(eD[i], cx[i], y);
          const unsigned off =
              (ev[i] && t0 + et[i] < seq) ? ((unsigned)(t0 + et[i]) * dim + tile * CT + ec[i]) * (unsigned)sizeof(TI)
                                          : OOB_OFF;
          if (SAVE_YP) bstore<TI>(r_yp, off, y);
          if (HAS_Z) y *= cz[i] * sigmoid_rcp(cz[i]);
          if (WRITE_Y) bstore<TI>(r_y, off, y);
        }
      }
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        cx[i] = nx[i];
        cz[i] = nz[i];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
template <typename TI, typename TP, int N, int G, bool MEAN, bool HAS_Z>
__global__ __launch_bounds__((RGeo<N, G>::NT)) void ss_bwd_kernel(const SSArgs p, const TP* __restrict__ Bm,
                                                                  const TP* __restrict__ Cm) {
  using Geo = RGeo<N, G>;
  constexpr int SW = Geo::SW, CW = Geo::CW, NT = Geo::NT, CT = Geo::CT;
  constexpr int CK = SS_CK;                 // recompute chunk (= checkpoint interval)
  constexpr int TS = N >= 32 ? 4 : 8;       // reverse steps per reduction round
  constexpr int NSB = CK / TS;
  constexpr int PS = CK + 4;                // [channel][t] row stride of the staged values
  constexpr int NE = CK * CT;               // staged (t, channel) elements per chunk
  constexpr int EPT = (NE + NT - 1) / NT;
  // px / pa tile [qty][t][channel][state]: a lane's state-sum item reads one contiguous row;
  // PN and the slot swizzle make one wave's writes and the 16-byte reads of consecutive
  // channels conflict-free, QP puts the two quantities of one (t, channel) on different banks
  constexpr int PN = ss_pn<N>();
  constexpr int QP = mod64_to(TS * CT * PN, 32);
  // dC / dB tile [qty][state][t][group][CW + 4]: a channel-group item reads one contiguous
  // run of CW values; SSR puts a wave's state rows on different banks
  constexpr int CWP = CW + 4, CTP = G * CWP;
  constexpr int SSR = ss_ssr(TS * CTP, CW);
  constexpr int NA = 2 * TS * CT;           // state sums per round: (t, channel, dx | ddt term)
  constexpr int NB = 2 * TS * N * G;        // channel-group sums per round: (qty, t, state, group)
  constexpr int NC = 2 * TS * N;            // partials per round: (qty, t, state)
  // A 16-lane group of 16-byte reads spreads over 64 banks; the runs of one row are CWP
  // (= 4 mod 8) words apart, so 16 consecutive runs are conflict-free, but a group that
  // crosses from one row into the next (SSR = 16 mod 32 words on, for the writes) is not
  // when a row holds IPB = 8 mod 16 runs: those pair rows A and A + 2 instead.
  constexpr int IPB = TS * G;
  constexpr bool BC_PAIR = CW == 16 && IPB % 16 == 8 && N % 2 == 0;
  static_assert(NT % CT == 0, "a thread's staged elements share one channel");
  // staged per chunk, double-buffered: clip(dt) with the sign bit set where the raw dt lies
  // outside [DT_MIN, DT_MAX] (no gradient), dt_b x, dy (after the gate)
  __shared__ __align__(16) float s_st[2][3][CT][PS];
  __shared__ float s_dtm[MEAN ? 2 : 1][CK];
  __shared__ __align__(16) float s_pq[2 * QP];
  __shared__ __align__(16) float s_bc[2 * N * SSR];
  __shared__ float s_red[2][2][N][TS][G];
  __shared__ float s_m[MEAN ? 2 : 1][MEAN ? TS : 1][CT];
  __shared__ float s_Dv[CT];

  const TI* __restrict__ x = (const TI*)p.x;
  const TI* __restrict__ dt = (const TI*)p.dt;
  const TI* __restrict__ z = (const TI*)p.z;
  const TI* __restrict__ dout = (const TI*)p.dout;
  const TP* __restrict__ Am = (const TP*)p.A;
  const TP* __restrict__ Dv = (const TP*)p.D;
  const int seq = p.seq, dim = p.dim;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int g = w % G, sg = w / G;
  const int s = sg * SW + lane / CW;
  const int cl = g * CW + lane % CW;
  const int sx = s ^ ss_swz<N>(cl);  // this lane's slot in a px / ga row
  const int logical = remap_xcd(blockIdx.x, gridDim.x);
  const int b = logical / p.ntile, tile = logical % p.ntile;
  const int c = tile * CT + cl;
  const bool cvalid = c < dim;

  const int ns = p.nst;
  const float A1 = (cvalid && s < ns) ? ld(Am, (long)c * ns + s) : 0.0f;
  const float A2 = A1 * LOG2E;
  float dh = 0.0f, dA = 0.0f;

  // staged elements (t, channel): e = tid + i NT
  int et[EPT], ec[EPT];
  bool ev[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const int e = tid + i * NT;
    et[i] = e / CT;
    ec[i] = e % CT;
    ev[i] = e < NE && tile * CT + ec[i] < dim;
  }
  // D per channel of the tile; dD accumulates over the elements this thread stages (all
  // of one channel, since NT is a multiple of CT)
  if (tid < CT) s_Dv[tid] = (Dv != nullptr && tile * CT + tid < dim) ? ld(Dv, tile * CT + tid) : 0.0f;
  const int aq = tid & 1;  // the quantity of this thread's state-sum items (NT is even)
  float dD = 0.0f;
  // The ddt term sums A[d, n] ga over the states.  For N >= 2 a thread's state-sum items
  // share one channel (NT is a multiple of 2 CT), so the multiply by A moves out of the
  // per-element reverse pass into the sum: weights A[d, :] for quantity 1, ones for 0.
  constexpr bool AW = N >= 2 && N <= 16;
  float aw[AW ? N : 1];
  if constexpr (AW) {
    static_assert(NT % (2 * CT) == 0, "state-sum items of a thread share one channel");
    const int wl = (tid >> 1) % CT, wc = tile * CT + wl, wx = ss_swz<N>(wl);
#pragma unroll
    for (int sn = 0; sn < N; ++sn)  // slot sn of the channel's row holds state sn ^ wx
      aw[sn] = aq == 0 ? 1.0f : ((wc < dim && (sn ^ wx) < ns) ? ld(Am, (long)wc * ns + (sn ^ wx)) : 0.0f);
  }

  const long rowbase = (long)b * seq * dim;
  typedef typename Bits<TI>::type RI;
  typedef typename Bits<TP>::type RP;
  const unsigned rowbytes = (unsigned)((long)seq * dim * sizeof(TI));
  const rsrc_t r_x = make_rsrc(x + rowbase, rowbytes), r_dt = make_rsrc(dt + rowbase, rowbytes);
  const rsrc_t r_do = make_rsrc(dout + rowbase, rowbytes);
  const rsrc_t r_z = make_rsrc(HAS_Z ? z + rowbase : x + rowbase, rowbytes);
  const rsrc_t r_yp = make_rsrc(HAS_Z ? (const TI*)p.ypre + rowbase : x + rowbase, rowbytes);
  const unsigned bcbytes = (unsigned)((long)seq * ns * sizeof(TP));
  const rsrc_t r_B = make_rsrc(Bm + (long)b * seq * ns, bcbytes), r_C = make_rsrc(Cm + (long)b * seq * ns, bcbytes);
  const rsrc_t r_m =
      make_rsrc(MEAN ? (const void*)(p.dtmean + (long)b * seq) : (const void*)x, (unsigned)(seq * sizeof(float)));
  const rsrc_t r_dx = make_rsrc((TI*)p.dx + rowbase, rowbytes), r_ddt = make_rsrc((TI*)p.ddt + rowbase, rowbytes);
  const rsrc_t r_dz = make_rsrc(p.dz != nullptr ? (TI*)p.dz + rowbase : (TI*)p.dx + rowbase,
                                p.dz != nullptr ? rowbytes : 0u);
  const rsrc_t r_ck = make_rsrc(p.ckpt + (long)b * p.nck * N * dim, (unsigned)((long)p.nck * N * dim * 4));

  // raw values of the next chunk (in reverse order), loaded a chunk ahead
  RI rx[EPT], rdt[EPT], rdo[EPT], rz[EPT], ryp[EPT];
  float rm[EPT];
  RP rB, rC;
  float rck;  // the state the fetched chunk starts from (its predecessor's checkpoint)
  // B/C values and starting state of the staged chunk, moved from the fetch registers
  float cB, cC, cck;
  auto fetch = [&](int ts) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int t = min(ts + et[i], seq - 1);
      const unsigned off = ev[i] ? ((unsigned)t * dim + tile * CT + ec[i]) * (unsigned)sizeof(TI) : OOB_OFF;
      rx[i] = bload<TI>(r_x, off);
      rdt[i] = bload<TI>(r_dt, off);
      rdo[i] = bload<TI>(r_do, off);
      if (HAS_Z) {
        rz[i] = bload<TI>(r_z, off);
        ryp[i] = bload<TI>(r_yp, off);
      }
      rm[i] = MEAN ? bits_f32(bload<float>(r_m, (unsigned)t * 4u)) : 0.0f;
    }
    const unsigned off = s < ns ? ((unsigned)(ts + min(lane & 15, seq - 1 - ts)) * ns + s) * (unsigned)sizeof(TP)
                                : OOB_OFF;
    rB = bload<TP>(r_B, off);
    rC = bload<TP>(r_C, off);
    // chunk 0 starts from zero (selected at use); the load stays unconditional
    const int kp = max(ts / CK - 1, 0);
    rck = bits_f32(bload<float>(r_ck, cvalid ? (((unsigned)kp * N + s) * dim + c) * 4u : OOB_OFF));
  };
  // stage the fetched chunk (first step ts) into buffer sb; the gate's dz is stored here;
  // wgt = 0 when the chunk was staged before (dD counts each element once)
  auto stage = [&](int ts, int sb, float wgt) {
    cB = bits_f32(rB);
    cC = bits_f32(rC);
    cck = rck;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      if (NE % NT != 0 && tid + i * NT >= NE) continue;
      const bool ok = ev[i] && ts + et[i] < seq;
      float dtr = bits_f32(rdt[i]);
      if constexpr (MEAN) {
        if (p.dt_sp) dtr = softplus_f(dtr);
      }
      const float dtc = ok ? clampf(dtr, DT_MIN, DT_MAX) : 0.0f;
      const float dtb = ok ? (MEAN ? rm[i] : dtc) : 0.0f;
      const float xv = ok ? bits_f32(rx[i]) : 0.0f;
      const float go = ok ? bits_f32(rdo[i]) : 0.0f;
      float dyp = go;
      if (HAS_Z) {
        const float zv = bits_f32(rz[i]);
        const float sgm = sigmoid_rcp(zv);
        dyp = go * zv * sgm;
        const unsigned off = ok ? ((unsigned)(ts + et[i]) * dim + tile * CT + ec[i]) * (unsigned)sizeof(TI) : OOB_OFF;
        bstore<TI>(r_dz, off, go * bits_f32(ryp[i]) * sgm * (1.0f + zv * (1.0f - sgm)));
      }
      dD = fmaf(wgt * dyp, xv, dD);
      s_st[sb][0][ec[i]][et[i]] = (dtr >= DT_MIN && dtr <= DT_MAX) ? dtc : -dtc;
      s_st[sb][1][ec[i]][et[i]] = dtb * xv;
      s_st[sb][2][ec[i]][et[i]] = dyp;
      if (MEAN && ec[i] == 0) s_dtm[sb][et[i]] = ok ? rm[i] : 0.0f;
    }
  };

  // channel-group sums of the previous round -> this workgroup's dC/dB partial; dt-mean
  // coupling of the previous round -> its partial
  auto finish_round = [&](int par, int ts0) {
#pragma unroll 1
    for (int it = tid; it < NC + (MEAN ? TS : 0); it += NT) {
      if (it < NC) {
        const int sn = it % N, tl = (it / N) % TS, q = it / (N * TS);
        float v = s_red[par][q][sn][tl][0];
#pragma unroll
        for (int gg = 1; gg < G; ++gg) v += s_red[par][q][sn][tl][gg];
        const int t = ts0 + tl;
        if (t < seq) p.part_bc[((((long)tile * p.batch + b) * seq + t) * 2 + q) * N + sn] = v;
      } else if (MEAN) {
        const int tl = it - NC;
        float v = 0.0f;
        for (int cc = 0; cc < CT; ++cc) v += s_m[MEAN ? par : 0][MEAN ? tl : 0][cc];
        const int t = ts0 + tl;
        if (t < seq) p.part_m[((long)tile * p.batch + b) * seq + t] = v;
      }
    }
  };

  fetch((p.nck - 1) * CK);
  stage((p.nck - 1) * CK, (p.nck - 1) & 1, 1.0f);
  fetch(max(p.nck - 2, 0) * CK);
  __syncthreads();
  int prev_par = -1, prev_ts = 0, par = 0;

  for (int k = p.nck - 1; k >= 0; --k) {
    const int ts = k * CK, sb = k & 1;
    // the chunk's B/C values and starting state (moved out of the fetch registers when the
    // chunk was staged).  The reverse pass broadcasts B from a separate copy: the
    // compiler would otherwise share one broadcast between the two passes and fold it into
    // neither multiply.
    const float rb = cB, rc = cC;
    float rb2;
    asm volatile("v_mov_b32 %0, %1" : "=v"(rb2) : "v"(rb));
    const float h0 = (k > 0 && cvalid) ? cck : 0.0f;
    // ---- recompute the chunk's states and decays from its checkpoint; the chunk's staged
    // dt values stay in registers for the reverse pass ---------------------------------
    float hs[CK], as[CK], dcs[CK], dxs[CK];
    {
      float hh = h0;
      static_for<CK / 4>([&](auto qi) {
        constexpr int q = decltype(qi)::value;
        const float4 dc4 = *reinterpret_cast<const float4*>(&s_st[sb][0][cl][4 * q]);
        const float4 dx4 = *reinterpret_cast<const float4*>(&s_st[sb][1][cl][4 * q]);
        dcs[4 * q] = dc4.x; dcs[4 * q + 1] = dc4.y; dcs[4 * q + 2] = dc4.z; dcs[4 * q + 3] = dc4.w;
        dxs[4 * q] = dx4.x; dxs[4 * q + 1] = dx4.y; dxs[4 * q + 2] = dx4.z; dxs[4 * q + 3] = dx4.w;
        static_for<4>([&](auto vi) {
          constexpr int tt = 4 * q + decltype(vi)::value;
          const float a = fast_exp2(fabsf(dcs[tt]) * A2);
          hh = fmaf(a, hh, row_bcast<tt>(rb) * dxs[tt]);
          as[tt] = a;
          hs[tt] = hh;
        });
      });
    }
    // ---- reverse recurrence in rounds of TS steps --------------------------------
    static_for<NSB>([&](auto ui) {
      constexpr int u = NSB - 1 - decltype(ui)::value;  // round u covers steps u TS .. u TS + TS - 1
      static_for<TS / 4>([&](auto qi) {
        constexpr int q = TS / 4 - 1 - decltype(qi)::value;
        constexpr int tq = u * TS + 4 * q;
        const float4 dy4 = *reinterpret_cast<const float4*>(&s_st[sb][2][cl][tq]);
        const float dyv[4] = {dy4.x, dy4.y, dy4.z, dy4.w};
        static_for<4>([&](auto vi) {
          constexpr int v = 3 - decltype(vi)::value, tt = tq + v, tl = tt - u * TS;
          dh = fmaf(dyv[v], row_bcast<tt>(rc), dh);
          const float gC = dyv[v] * hs[tt];
          const float gB = dh * dxs[tt];
          const float px = dh * row_bcast<tt>(rb2);
          dh *= as[tt];
          const float ga = dh * (tt > 0 ? hs[tt > 0 ? tt - 1 : 0] : h0);
          dA = fmaf(ga, fabsf(dcs[tt]), dA);
          s_pq[(tl * CT + cl) * PN + sx] = px;
          s_pq[QP + (tl * CT + cl) * PN + sx] = AW ? ga : ga * A1;
          s_bc[s * SSR + tl * CTP + g * CWP + lane % CW] = gC;
          s_bc[N * SSR + s * SSR + tl * CTP + g * CWP + lane % CW] = gB;
        });
      });
      if (u == 0) {
        // the next chunk's inputs into the other staging buffer (last read by the chunk
        // before this one), and the chunk after it into the registers; unconditional
        // (chunk 0 stages itself again, counted with weight 0): a conditional fetch makes
        // the compiler drain every outstanding load
        stage(max(k - 1, 0) * CK, sb ^ 1, k > 0 ? 1.0f : 0.0f);
        fetch(max(k - 2, 0) * CK);
      }
      __syncthreads();
      // ---- state sums -> dx, ddt; channel-group sums -> s_red ----------------------
#pragma unroll 1
      for (int it = tid; it < NA; it += NT) {
        const int tl = (it >> 1) / CT, tt = u * TS + tl, ac = (it >> 1) % CT;
        const float* src = &s_pq[aq * QP + (tl * CT + ac) * PN];
        float v;
        if constexpr (AW && PN % 4 == 0) {
          const float4 f0 = *reinterpret_cast<const float4*>(src);
          v = fmaf(f0.w, aw[3], fmaf(f0.z, aw[2], fmaf(f0.y, aw[1], f0.x * aw[0])));
#pragma unroll
          for (int sn = 4; sn < N; sn += 4) {
            const float4 f = *reinterpret_cast<const float4*>(src + sn);
            v = fmaf(f.w, aw[sn + 3], fmaf(f.z, aw[sn + 2], fmaf(f.y, aw[sn + 1], fmaf(f.x, aw[sn], v))));
          }
        } else if constexpr (AW) {
          v = src[0] * aw[0];
#pragma unroll
          for (int sn = 1; sn < N; ++sn) v = fmaf(src[sn], aw[sn], v);
        } else if constexpr (PN % 4 == 0) {
          const float4 f0 = *reinterpret_cast<const float4*>(src);
          v = (f0.x + f0.y) + (f0.z + f0.w);
#pragma unroll
          for (int sn = 4; sn < N; sn += 4) {
            const float4 f = *reinterpret_cast<const float4*>(src + sn);
            v += (f.x + f.y) + (f.z + f.w);
          }
        } else {
          v = src[0];
#pragma unroll
          for (int sn = 1; sn < N; ++sn) v += src[sn];
        }
        const float other = pair_swap(v);
        const float pxs = aq ? other : v, pas = aq ? v : other;
        const float dcr = s_st[sb][0][ac][tt], dtx = s_st[sb][1][ac][tt], dyp = s_st[sb][2][ac][tt];
        const float dtb = MEAN ? s_dtm[MEAN ? sb : 0][tt] : fabsf(dcr);
        // x = dt_b x / dt_b (dt_b >= DT_MIN wherever the element is inside the tensor)
        const float xv = dtb > 0.0f ? dtx * fast_rcp(dtb) : 0.0f;
        const bool ok = tile * CT + ac < dim && ts + tt < seq;
        const unsigned off = ok ? ((unsigned)(ts + tt) * dim + tile * CT + ac) * (unsigned)sizeof(TI) : OOB_OFF;
        if (aq == 0) {
          bstore<TI>(r_dx, off, fmaf(pxs, dtb, dyp * s_Dv[ac]));
          if (MEAN) s_m[MEAN ? par : 0][MEAN ? tl : 0][ac] = pxs * xv;
        } else {
          // with the softplus flag (mean mode) the fixup kernel adds the coupling term and
          // applies the chain factor sigmoid(pre) to the sum
          const float mk = dcr > 0.0f ? 1.0f : 0.0f;
          bstore<TI, BUF_NT>(r_ddt, off, mk * (MEAN ? pas : fmaf(pxs, xv, pas)));
        }
      }
#pragma unroll 1
      for (int it = tid; it < NB; it += NT) {
        int blk, i;  // item (blk = (qty, state) row of the tile, i = (t, group) run in it)
        if constexpr (BC_PAIR) {
          // 16-lane groups: rows A and A + 2 (2 SSR = 32 mod 64 words apart) each fill
          // IPB / 16 whole groups, and their last 8 runs share one group
          constexpr int F = IPB / 16;
          const int pi = it / (2 * IPB), u = it % (2 * IPB);
          const int A = 4 * (pi >> 1) + (pi & 1);
          if (u < 16 * F) {
            blk = A;
            i = u;
          } else if (u < 32 * F) {
            blk = A + 2;
            i = u - 16 * F;
          } else {
            blk = u - 32 * F < 8 ? A : A + 2;
            i = 16 * F + (u & 7);
          }
        } else {
          blk = it / IPB;
          i = it % IPB;
        }
        const int q = blk / N, sn = blk % N, tl = i / G, gg = i % G;
        const float* src = &s_bc[blk * SSR + tl * CTP + gg * CWP];
        const float4 f0 = *reinterpret_cast<const float4*>(src);
        float v = (f0.x + f0.y) + (f0.z + f0.w);
#pragma unroll
        for (int cc = 4; cc < CW; cc += 4) {
          const float4 f = *reinterpret_cast<const float4*>(src + cc);
          v += (f.x + f.y) + (f.z + f.w);
        }
        s_red[par][q][sn][tl][gg] = v;
      }
      if (prev_par >= 0) finish_round(prev_par, prev_ts);
      prev_par = par;
      prev_ts = ts + u * TS;
      par ^= 1;
      __syncthreads();  // the tiles are rewritten by the next round
    });
  }
  finish_round(prev_par, prev_ts);
  // dA partial per (b, d, n); dD partial per (b, d): threads with the same channel hold
  // disjoint timesteps
  if (cvalid) p.part_a[((long)b * dim + c) * N + s] = dA;
  float* s_dd = s_pq;
  s_dd[tid] = dD;
  __syncthreads();
  if (tid < CT && tile * CT + tid < dim) {
    float acc = 0.0f;
#pragma unroll 1
    for (int kk = 0; kk < NT / CT; ++kk) acc += s_dd[kk * CT + tid];
    p.part_d[(long)b * dim + tile * CT + tid] = acc;
  }
}

// dB, dC = sum over channel tiles, in tile order; partials carry NP (padded) states, outputs
// ns.  VEC = 4 (NP >= 2, so 2 NP and the partial stride are multiples of 4): a thread sums
// four consecutive (row, qty, n) entries with 16-byte loads, eight tiles' loads in flight.
template <int VEC>
__global__ __launch_bounds__(256) void ss_reduce_bc_kernel(const float* __restrict__ part, float* __restrict__ dB,
                                                           float* __restrict__ dC, int ntile, long rows, int NP,
                                                           int ns) {
  typedef float vec_t __attribute__((ext_vector_type(VEC)));
  const long total = rows * 2 * NP;
  const long i0 = ((long)blockIdx.x * 256 + threadIdx.x) * VEC;  // over rows * 2NP
  if (i0 >= total) return;
  const vec_t* p = reinterpret_cast<const vec_t*>(part + i0);
  const long stride = total / VEC;
  vec_t acc = (vec_t)0.0f;
  int tl = 0;
  for (; tl + 8 <= ntile; tl += 8) {
    vec_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[(long)(tl + k) * stride];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += v[k];
  }
  for (; tl < ntile; ++tl) acc += p[(long)tl * stride];
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
    const long i = i0 + k;
    const long row = i / (2 * NP);
    const int r = (int)(i % (2 * NP));
    const int qty = r / NP, nn = r % NP;
    if (nn >= ns) continue;
    float* dst = qty == 0 ? dC : dB;
    if (dst) dst[row * ns + nn] = acc[k];
  }
}

// dA[d, n] = sum_b part_a (NP padded states per channel); dD[d] = sum_b part_d
__global__ __launch_bounds__(256) void ss_reduce_ad_kernel(const float* __restrict__ part_a,
                                                           const float* __restrict__ part_d, float* __restrict__ dA,
                                                           float* __restrict__ dD, int batch, int dim, int NP,
                                                           int ns) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const long na = (long)dim * NP;
  if (i < na) {
    const long d = i / NP;
    const int n = (int)(i % NP);
    if (n >= ns) return;
    float acc = 0.0f;
    for (int bb = 0; bb < batch; ++bb) acc += part_a[(long)bb * na + i];
    if (dA) dA[d * ns + n] = acc;
  } else if (i < na + dim) {
    const long d = i - na;
    float acc = 0.0f;
    for (int bb = 0; bb < batch; ++bb) acc += part_d[(long)bb * dim + d];
    if (dD) dD[d] = acc;
  }
}

// mean mode: ddt[b,t,d] += in_range * (sum over tiles part_m[b,t]) / dim.  One workgroup per
// row: its threads split the tile partials (in tile order within each thread, then a fixed
// tree), so the row total is formed once, not by every thread.  sp: dt holds the
// pre-activation, in_range tests softplus(dt) and the sum is scaled by sigmoid(dt).
template <typename TI>
__global__ __launch_bounds__(256) void ss_mean_fixup_kernel(const float* __restrict__ part_m,
                                                            const TI* __restrict__ dt, TI* __restrict__ ddt,
                                                            int ntile, long rows, int dim, int sp) {
  // 16 rows per workgroup.  The tile partials of a row sit `rows` apart (one per channel
  // tile): 16 lanes take 16 consecutive rows and the 16 lane groups a sixteenth of the tiles
  // each, combined in a fixed order; then each wave updates whole rows, 16-byte accesses.
  constexpr int RW = 16;
  __shared__ float s_part[RW][RW + 1];
  __shared__ float s_tot[RW];
  const long r0 = (long)blockIdx.x * RW;
  const int rl = threadIdx.x & (RW - 1), grp = threadIdx.x / RW;
  float tot = 0.0f;
  if (r0 + rl < rows)
    for (int tl = grp; tl < ntile; tl += 256 / RW) tot += part_m[(long)tl * rows + r0 + rl];
  s_part[rl][grp] = tot;
  __syncthreads();
  if (threadIdx.x < RW) {
    float t = 0.0f;
#pragma unroll
    for (int g = 0; g < RW; ++g) t += s_part[threadIdx.x][g];
    s_tot[threadIdx.x] = t / (float)dim;
  }
  __syncthreads();
  constexpr int V = 16 / sizeof(TI);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nrow = (int)min((long)RW, rows - r0);
  const bool vec = dim % V == 0 && ((uintptr_t)dt & 15) == 0 && ((uintptr_t)ddt & 15) == 0;
  for (int r = w; r < nrow; r += 4) {
    const float t = s_tot[r];
    const long base = (r0 + r) * dim;
    if (vec) {
      for (int d0 = lane * V; d0 < dim; d0 += 64 * V) {
        const uint4 ud = *reinterpret_cast<const uint4*>(dt + base + d0);
        uint4 ug = *reinterpret_cast<const uint4*>(ddt + base + d0);
        const TI* vd = reinterpret_cast<const TI*>(&ud);
        TI* vg = reinterpret_cast<TI*>(&ug);
#pragma unroll
        for (int i = 0; i < V; ++i) {
          const float raw = to_f32(vd[i]);
          const float dtr = sp ? softplus_f(raw) : raw;
          if (dtr >= DT_MIN && dtr <= DT_MAX) vg[i] = (TI)((to_f32(vg[i]) + t) * (sp ? sigmoid_rcp(raw) : 1.0f));
        }
        *reinterpret_cast<uint4*>(ddt + base + d0) = ug;
      }
    } else {
      for (int d = lane; d < dim; d += 64) {
        const float raw = ld(dt, base + d);
        const float dtr = sp ? softplus_f(raw) : raw;
        if (dtr >= DT_MIN && dtr <= DT_MAX)
          st(ddt, base + d, (ld(ddt, base + d) + t) * (sp ? sigmoid_rcp(raw) : 1.0f));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr int SS_MAX_STATE = 32;  // the reference's limit (fused_selective_scan.cu:57-76, _backward.cu:59)

// the power of two the kernels are compiled for: NP >= N, the states past N are padding
inline int padded_state(int N) {
  int np = 1;
  while (np < N) np *= 2;
  return np;
}

inline long num_chunks(int seq) { return (seq + SS_CK - 1) / SS_CK; }

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Channel groups per workgroup.  The kernels are compiled for G = 1 and for a wide G per
// state size; the host takes the one whose grid loads the busiest CU with the fewest
// waves (workgroups spread evenly over 256 CUs, at most as many per CU as LDS and the
// 32 waves per CU allow), the wide one on a tie (fewer dC/dB partials, longer rows).
struct SSPlan {
  int G, CT, ntile;
};

inline int wide_groups(int NP) { return NP >= 32 ? 1 : (NP == 16 ? 3 : (NP >= 4 ? 4 : 1)); }

// LDS bytes of one workgroup (mirrors the kernels' __shared__ declarations)
inline size_t fwd_lds(int NP, int G) {
  const int SW = NP < 4 ? NP : 4, CW = 64 / SW, CT = G * CW, PN = NP == 4 ? 12 : NP + 4;
  return (size_t)2 * 2 * CT * (SS_CK + 4) * 4 + (size_t)2 * SS_CK * CT * PN * 4;
}
inline int mod64_up(int v, int r) { return v + ((r - v % 64) % 64 + 64) % 64; }
inline size_t bwd_lds(int NP, int G) {
  const int SW = NP < 4 ? NP : 4, CW = 64 / SW, CT = G * CW, TS = NP >= 32 ? 4 : 8;
  const int PN = NP == 4 ? 12 : NP + 4, QP = mod64_up(TS * CT * PN, 32), SSR = ss_ssr(TS * G * (CW + 4), CW);
  return (size_t)2 * 3 * CT * (SS_CK + 4) * 4 + 2 * SS_CK * 4 + (size_t)2 * QP * 4 + (size_t)2 * NP * SSR * 4 +
         (size_t)2 * 2 * TS * NP * G * 4 + (size_t)2 * TS * CT * 4 + CT * 4;
}

// EDF_SS_PLAN=narrow | wide forces one of the two compiled plans (every call reads it, so
// the workspace query and the launch that follows agree while it is unchanged); anything
// else, or unset, lets the host choose.  Tests use it to run both plans at every state size.
inline int forced_plan() {
  const char* f = getenv("EDF_SS_PLAN");
  if (!f) return 0;
  if (!strcmp(f, "narrow")) return 1;
  if (!strcmp(f, "wide")) return 2;
  return 0;
}

inline SSPlan choose_plan(int batch, int dim, int NP, bool bwd) {
  const int SW = NP < 4 ? NP : 4, CW = 64 / SW, NSG = NP / SW;
  const int gw = wide_groups(NP);
  SSPlan best{gw, gw * CW, (dim + gw * CW - 1) / (gw * CW)};
  const int force = forced_plan();
  if (force == 1) return SSPlan{1, CW, (dim + CW - 1) / CW};
  if (force == 2) return best;
  double best_score = 1e30;
  const int cands[2] = {gw, 1};
  for (int G : cands) {
    const int CT = G * CW, nt = (dim + CT - 1) / CT, nw = G * NSG;
    const long nwg = (long)batch * nt;
    const size_t lds = bwd ? bwd_lds(NP, G) : fwd_lds(NP, G);
    const long occ = std::max(1L, std::min((long)(163840 / lds), (long)(32 / nw)));
    const long per_cu = (nwg + 255) / 256;
    // the channel work the busiest CU holds, slowed where its resident waves cannot fill 12
    // slots (three per SIMD); a tie goes to the wide plan (fewer dB / dC partials)
    const double waves = (double)std::min(per_cu, occ) * nw;
    const double score = (double)per_cu * CT / std::min(1.0, waves / 12.0);
    if (score < best_score) {
      best_score = score;
      best = SSPlan{G, CT, nt};
    }
  }
  return best;
}

// caller-owned "states" buffer: checkpoints [batch][nck][NP][dim] float32, then y before the
// gate [batch][seq][dim] (io type, written when the gate z is given)
inline size_t ckpt_bytes(int batch, int seq, int dim, int nst) {
  return align256((size_t)batch * num_chunks(seq) * padded_state(nst) * dim * sizeof(float));
}

struct WsLayout {
  size_t ckpt, ypre, dtmean, part_bc, part_a, part_d, part_m, total;
};

inline WsLayout bwd_layout(int batch, int seq, int dim, int nst, bool need_ckpt, bool mean_mode) {
  const int N = padded_state(nst);
  WsLayout w{};
  const int nt = choose_plan(batch, dim, N, true).ntile;
  size_t off = 0;
  w.ckpt = off;
  if (need_ckpt) off += ckpt_bytes(batch, seq, dim, nst);
  w.ypre = off;
  if (need_ckpt) off += align256((size_t)batch * seq * dim * sizeof(float));
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

template <typename TI, typename TP, int N, int G>
void launch_fwd_g(hipStream_t s, const SSArgs& a) {
  constexpr int NT = RGeo<N, G>::NT;
  const int grid = a.batch * a.ntile;
  const bool mean = a.dtmean != nullptr, hz = a.z != nullptr, wy = a.out != nullptr;
  const TP* Bp = (const TP*)a.B;
  const TP* Cp = (const TP*)a.C;
#define EDF_SS_FWD(M, Z, Y) ss_fwd_kernel<TI, TP, N, G, M, Z, Y><<<grid, NT, 0, s>>>(a, Bp, Cp)
  if (wy) {
    if (mean && hz) EDF_SS_FWD(true, true, true);
    else if (mean) EDF_SS_FWD(true, false, true);
    else if (hz) EDF_SS_FWD(false, true, true);
    else EDF_SS_FWD(false, false, true);
  } else {  // checkpoints (and y before the gate) only: the backward without saved states
    if (mean && hz) EDF_SS_FWD(true, true, false);
    else if (mean) EDF_SS_FWD(true, false, false);
    else if (hz) EDF_SS_FWD(false, true, false);
    else EDF_SS_FWD(false, false, false);
  }
#undef EDF_SS_FWD
}

template <typename TI, typename TP, int N>
void launch_fwd_t(hipStream_t s, SSArgs a) {
  const SSPlan pl = choose_plan(a.batch, a.dim, N, false);
  a.ntile = pl.ntile;
  constexpr int GW = ss_gwide<N>();
  if constexpr (GW != 1) {
    if (pl.G == GW) return launch_fwd_g<TI, TP, N, GW>(s, a);
  }
  launch_fwd_g<TI, TP, N, 1>(s, a);
}

template <typename TI, typename TP>
int launch_fwd_n(hipStream_t s, const SSArgs& a, int nst) {
  switch (padded_state(nst)) {
    case 1: launch_fwd_t<TI, TP, 1>(s, a); break;
    case 2: launch_fwd_t<TI, TP, 2>(s, a); break;
    case 4: launch_fwd_t<TI, TP, 4>(s, a); break;
    case 8: launch_fwd_t<TI, TP, 8>(s, a); break;
    case 16: launch_fwd_t<TI, TP, 16>(s, a); break;
    case 32: launch_fwd_t<TI, TP, 32>(s, a); break;
    default: return set_error(EDF_ERR_UNSUPPORTED, "state size %d unsupported (1..32)", nst);
  }
  return check_launch("selective scan");
}

template <typename TI, typename TP, int N, int G>
void launch_bwd_g(hipStream_t s, const SSArgs& a) {
  constexpr int NT = RGeo<N, G>::NT;
  const int grid = a.batch * a.ntile;
  const bool mean = a.dtmean != nullptr, hz = a.z != nullptr;
  const TP* Bp = (const TP*)a.B;
  const TP* Cp = (const TP*)a.C;
  if (mean && hz) ss_bwd_kernel<TI, TP, N, G, true, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  else if (mean) ss_bwd_kernel<TI, TP, N, G, true, false><<<grid, NT, 0, s>>>(a, Bp, Cp);
  else if (hz) ss_bwd_kernel<TI, TP, N, G, false, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  else ss_bwd_kernel<TI, TP, N, G, false, false><<<grid, NT, 0, s>>>(a, Bp, Cp);
}

template <typename TI, typename TP, int N>
void launch_bwd_t(hipStream_t s, const SSArgs& a) {
  // a.ntile (and the partial buffers sized from it) come from the same plan
  constexpr int GW = ss_gwide<N>();
  if constexpr (GW != 1) {
    if (choose_plan(a.batch, a.dim, N, true).G == GW) return launch_bwd_g<TI, TP, N, GW>(s, a);
  }
  launch_bwd_g<TI, TP, N, 1>(s, a);
}

template <typename TI, typename TP>
int launch_bwd_n(hipStream_t s, const SSArgs& a, int nst) {
  switch (padded_state(nst)) {
    case 1: launch_bwd_t<TI, TP, 1>(s, a); break;
    case 2: launch_bwd_t<TI, TP, 2>(s, a); break;
    case 4: launch_bwd_t<TI, TP, 4>(s, a); break;
    case 8: launch_bwd_t<TI, TP, 8>(s, a); break;
    case 16: launch_bwd_t<TI, TP, 16>(s, a); break;
    case 32: launch_bwd_t<TI, TP, 32>(s, a); break;
    default: return set_error(EDF_ERR_UNSUPPORTED, "state size %d unsupported (1..32)", nst);
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
  EDF_REQUIRE(N <= SS_MAX_STATE, EDF_ERR_UNSUPPORTED, "state size %d unsupported (1..%d)", N, SS_MAX_STATE);
  const int base_mode = mode & ~EDF_SS_DT_SOFTPLUS;
  EDF_REQUIRE(base_mode == EDF_SS_DT_PER_CHANNEL || base_mode == EDF_SS_DT_MEAN, EDF_ERR_INVALID_ARG,
              "unknown dt mode %d", mode);
  EDF_REQUIRE(!(mode & EDF_SS_DT_SOFTPLUS) || base_mode == EDF_SS_DT_MEAN, EDF_ERR_UNSUPPORTED,
              "the dt softplus flag is built for dt-mean mode (the Mamba block's form) only");
  // the kernels address one batch row of x, dt, z, y, dy, dx, ddt, dz (and of B, C and the
  // checkpoints) through buffer resources with 32-bit byte offsets
  EDF_REQUIRE((long)seq * dim * 4 < (1L << 31) && num_chunks(seq) * padded_state(N) * dim * 4 < (1L << 31) &&
                  (long)seq * N * 4 < (1L << 31),
              EDF_ERR_UNSUPPORTED,
              "one batch row of seq_len * hidden elements (and its checkpoints) must stay below 2 GiB");
  return EDF_OK;
}

int run_dtmean(hipStream_t s, const void* dt, float* dtm, int batch, int seq, int dim, int io, int sp) {
  const int rows = batch * seq;
  const int grid = (rows + 3) / 4;
  if (io == EDF_BF16)
    ss_dtmean_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)dt, dtm, rows, dim, sp);
  else
    ss_dtmean_kernel<float><<<grid, 256, 0, s>>>((const float*)dt, dtm, rows, dim, sp);
  return check_launch("selective scan dt mean");
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_selective_scan_states_bytes(int batch, int seq_len, int hidden, int state) {
  if (batch <= 0 || seq_len <= 0 || hidden <= 0 || state <= 0) return 0;
  return edf::ckpt_bytes(batch, seq_len, hidden, state) + (size_t)batch * seq_len * hidden * sizeof(float);
}

size_t edf_selective_scan_workspace_bytes(int batch, int seq_len, int hidden, int state, int mode) {
  if (batch <= 0 || seq_len <= 0) return 0;
  return (mode & EDF_SS_DT_MEAN) ? edf::align256((size_t)batch * seq_len * 4) : 0;
}

size_t edf_selective_scan_backward_workspace_bytes(int batch, int seq_len, int hidden, int state, int mode,
                                                   int have_states) {
  if (batch <= 0 || seq_len <= 0 || hidden <= 0 || state <= 0 || state > edf::SS_MAX_STATE) return 0;
  return edf::bwd_layout(batch, seq_len, hidden, state, !have_states, (mode & EDF_SS_DT_MEAN) != 0).total;
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
  a.ypre = states != nullptr ? (char*)states + ckpt_bytes(batch, seq_len, hidden, state) : nullptr;
  a.batch = batch; a.seq = seq_len; a.dim = hidden; a.nst = state;
  a.nck = (int)num_chunks(seq_len);
  a.dt_sp = (mode & EDF_SS_DT_SOFTPLUS) != 0;
  if (mode & EDF_SS_DT_MEAN) {
    a.dtmean = (float*)workspace;
    rc = run_dtmean(s, dt, (float*)workspace, batch, seq_len, hidden, io_dtype, a.dt_sp);
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
  EDF_REQUIRE(x && dt && A && B && C && grad_out && grad_x && grad_dt, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const bool mean_mode = (mode & EDF_SS_DT_MEAN) != 0;
  const WsLayout L = bwd_layout(batch, seq_len, hidden, state, states == nullptr, mean_mode);
  EDF_REQUIRE(workspace && workspace_bytes >= L.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              L.total);
  hipStream_t s = as_stream(stream);
  char* ws = (char*)workspace;
  SSArgs a{};
  a.x = x; a.dt = dt; a.A = A; a.B = B; a.C = C; a.D = D; a.z = z;
  a.batch = batch; a.seq = seq_len; a.dim = hidden; a.nst = state;
  a.nck = (int)num_chunks(seq_len);
  a.dt_sp = (mode & EDF_SS_DT_SOFTPLUS) != 0;
  if (mean_mode) {
    a.dtmean = (float*)(ws + L.dtmean);
    rc = run_dtmean(s, dt, (float*)(ws + L.dtmean), batch, seq_len, hidden, io_dtype, a.dt_sp);
    if (rc) return rc;
  }
  if (states != nullptr) {
    a.ckpt = (float*)states;
    a.ypre = (char*)states + ckpt_bytes(batch, seq_len, hidden, state);
  } else {  // recompute checkpoints (and y before the gate) with a forward pass that writes no output
    a.ckpt = (float*)(ws + L.ckpt);
    a.ypre = ws + L.ypre;
    SSArgs f = a;
    f.out = nullptr;
    rc = by_dtypes(io_dtype, param_dtype, [&](auto* ti, auto* tp) {
      using TI = std::remove_pointer_t<decltype(ti)>;
      using TP = std::remove_pointer_t<decltype(tp)>;
      return launch_fwd_n<TI, TP>(s, f, state);
    });
    if (rc) return rc;
  }
  a.ntile = choose_plan(batch, hidden, padded_state(state), true).ntile;
  a.dout = grad_out;
  a.dx = grad_x;
  a.ddt = grad_dt;
  a.dz = grad_z;
  a.part_bc = (float*)(ws + L.part_bc);
  a.part_a = (float*)(ws + L.part_a);
  a.part_d = (float*)(ws + L.part_d);
  a.part_m = mean_mode ? (float*)(ws + L.part_m) : nullptr;
  rc = by_dtypes(io_dtype, param_dtype, [&](auto* ti, auto* tp) {
    using TI = std::remove_pointer_t<decltype(ti)>;
    using TP = std::remove_pointer_t<decltype(tp)>;
    return launch_bwd_n<TI, TP>(s, a, state);
  });
  if (rc) return rc;
  const long rows = (long)batch * seq_len;
  const int np = padded_state(state);
  if (grad_B || grad_C) {
    const long total = rows * 2 * np;
    if (np >= 2 && ((uintptr_t)a.part_bc & 15) == 0)  // the caller's workspace may sit at any offset
      ss_reduce_bc_kernel<4><<<(unsigned)((total / 4 + 255) / 256), 256, 0, s>>>(a.part_bc, (float*)grad_B,
                                                                               (float*)grad_C, a.ntile, rows, np, state);
    else
      ss_reduce_bc_kernel<1><<<(unsigned)((total + 255) / 256), 256, 0, s>>>(a.part_bc, (float*)grad_B,
                                                                             (float*)grad_C, a.ntile, rows, np, state);
    rc = check_launch("selective scan dB/dC reduction");
    if (rc) return rc;
  }
  if (grad_A || grad_D) {
    const long total = (long)hidden * np + hidden;
    ss_reduce_ad_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(a.part_a, a.part_d, (float*)grad_A,
                                                                        (float*)grad_D, batch, hidden, np, state);
    rc = check_launch("selective scan dA/dD reduction");
    if (rc) return rc;
  }
  if (mean_mode) {
    if (io_dtype == EDF_BF16)
      ss_mean_fixup_kernel<bf16><<<(unsigned)((rows + 15) / 16), 256, 0, s>>>(
          a.part_m, (const bf16*)dt, (bf16*)grad_dt, a.ntile, rows, hidden, a.dt_sp);
    else
      ss_mean_fixup_kernel<float><<<(unsigned)((rows + 15) / 16), 256, 0, s>>>(
          a.part_m, (const float*)dt, (float*)grad_dt, a.ntile, rows, hidden, a.dt_sp);
    rc = check_launch("selective scan dt-mean coupling");
    if (rc) return rc;
  }
  return EDF_OK;
}

}  // extern "C"
