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
// Design.  The op is VALU-bound: per (b, t, d, n) element the forward needs one
// v_exp_f32 (about 10 cycles per wave on MI355X, measured) and four VALU ops, several
// times the HBM time at config-2 size.  The layout minimises everything else:
//   * lane = channel d (64 channels per wave) holding K states in registers (one in the
//     forward, two in the backward); NW = N / K waves per workgroup cover one 64-channel
//     tile's N states (16 or 8 waves at N = 16: 4 or 2 waves per SIMD hide the LDS and
//     transcendental latency, which four states per lane at 1 wave per SIMD did not);
//   * the B[b, t, :] and C[b, t, :] values a wave needs are the same for all its lanes.
//     Forward: a block's values are loaded into a few VGPRs (16 values per register,
//     replicated over the four 16-lane rows) and broadcast with DPP row_newbcast, folded
//     into v_mul_f32_dpp: no LDS traffic.  Backward: staged through LDS once per chunk
//     and read as broadcasts.  (Scalar loads into SGPR operands were tried and are
//     slower: every timestep waits on the scalar cache.)
//   * x, dt (and z) are staged per block of timesteps through LDS from coalesced rows,
//     clip(dt) and dt_b * x computed once per (t, d); the recurrence reads them as
//     16-byte vectors;
//   * y = sum_n C h: each lane sums its K states, the NW wave partials are added
//     through LDS by the thread that staged that (t, d), which still holds x and z in
//     registers for the D skip and the gate; double-buffered tiles need one barrier
//     per block, and the raw inputs are prefetched four blocks ahead;
//   * the forward writes the state every CK = 16 timesteps ("checkpoints", layout
//     [b][chunk][n][d], coalesced over d);
//   * any state size 1..32 (the reference's limit): the kernels are compiled for the next
//     power of two NP >= N and the states past N are padding, with A = B = C = 0 loaded
//     for them, so they stay 0 and add nothing; A, B, C, dA, dB and dC keep the caller's
//     stride N, checkpoints and partial sums the padded NP;
//   * backward: chunks are walked in reverse; each chunk's states and decays are
//     recomputed from its checkpoint into registers, then the reverse recurrence runs
//     with the same lane layout.  Sums over states (dx, ddt) are in-lane plus an LDS
//     add over the NW waves; sums over channels (dB, dC) go through an LDS tile per
//     block of 8 timesteps (conflict-free strides) into per-tile partials, summed over
//     the tiles by a small deterministic kernel (no atomics).
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr float DT_MIN = 1.0e-3f;
constexpr float DT_MAX = 0.1f;
constexpr int SS_CK = 16;  // checkpoint interval (timesteps) = backward recompute chunk

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
  int nst;  // the caller's state count N (<= the kernel's padded NP): stride of A, B, C rows
};

// lane = channel; K = min(N, KMAX) states per lane (at least N / 16, so a workgroup
// has at most 16 waves); NW waves per workgroup cover the N states.
template <int N, int KMAX = 4>
struct SSGeo {
  static constexpr int KLO = KMAX > N / 16 ? KMAX : N / 16;
  static constexpr int K = N < KLO ? N : KLO;
  static constexpr int NW = N / K;
  static constexpr int NT = 64 * NW;
};

EDF_DEVICE int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

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
template <typename TI, typename TP, int N, int KMAX, bool MEAN, bool HAS_Z, bool WRITE_Y>
__global__ __launch_bounds__((SSGeo<N, KMAX>::NT)) void ss_fwd_kernel(const SSArgs p, const TP* __restrict__ Bm,
                                                                    const TP* __restrict__ Cm) {
  using G = SSGeo<N, KMAX>;
  constexpr int K = G::K, NW = G::NW, NT = G::NT;
  constexpr int TS = SS_CK;          // timesteps per staged block (one checkpoint per block)
  constexpr int PS = TS + 4;         // [channel][t] row stride: 16-byte reads are conflict-free
  constexpr int EPT = TS * 64 / NT;  // staged (t, channel) elements per thread
  constexpr int R = TS * 2 * K / 16;  // VGPRs holding a block's B/C values (16 per row)
  constexpr int PD = 4;                // prefetch distance (blocks)
  static_assert(TS % 4 == 0 && EPT * NW == TS && PD % 2 == 0 && (TS * K) % 16 == 0, "staging layout");
  __shared__ __align__(16) float s_dtc[2][64][PS];
  __shared__ __align__(16) float s_dtx[2][64][PS];
  __shared__ float s_yp[2][NW][TS][64];

  const TI* __restrict__ x = (const TI*)p.x;
  const TI* __restrict__ dt = (const TI*)p.dt;
  const TI* __restrict__ z = (const TI*)p.z;
  const TP* __restrict__ Am = (const TP*)p.A;
  const TP* __restrict__ Dv = (const TP*)p.D;
  TI* __restrict__ out = (TI*)p.out;
  const int seq = p.seq, dim = p.dim;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);  // this wave's state group
  const int logical = remap_xcd(blockIdx.x, gridDim.x);
  const int b = logical / p.ntile, tile = logical % p.ntile;
  const int c = tile * 64 + lane;
  const bool cvalid = c < dim;
  const int cc = min(c, dim - 1);

  const int ns = p.nst;
  float A2[K], h[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    A2[s] = (cvalid && w * K + s < ns) ? ld(Am, (long)c * ns + w * K + s) * LOG2E : 0.0f;
    h[s] = 0.0f;
  }
  const float Dc = (Dv != nullptr && cvalid) ? ld(Dv, c) : 0.0f;
  const long rowbase = (long)b * seq * dim;
  // every global access goes through a buffer resource on this batch row: SGPR base plus a
  // 32-bit offset (no 64-bit address VALU), out-of-range offsets load 0 / drop the store
  typedef typename Bits<TI>::type RI;
  typedef typename Bits<TP>::type RP;
  const unsigned rowbytes = (unsigned)((long)seq * dim * sizeof(TI));
  const rsrc_t r_x = make_rsrc(x + rowbase, rowbytes), r_dt = make_rsrc(dt + rowbase, rowbytes);
  const rsrc_t r_z = make_rsrc(HAS_Z ? z + rowbase : x + rowbase, rowbytes);
  const rsrc_t r_y = make_rsrc(WRITE_Y ? out + rowbase : x + rowbase, WRITE_Y ? rowbytes : 0u);
  const unsigned bcbytes = (unsigned)((long)seq * ns * sizeof(TP));
  const rsrc_t r_B = make_rsrc(Bm + (long)b * seq * ns, bcbytes), r_C = make_rsrc(Cm + (long)b * seq * ns, bcbytes);
  const rsrc_t r_m =
      make_rsrc(MEAN ? (const void*)(p.dtmean + (long)b * seq) : (const void*)x, (unsigned)(seq * sizeof(float)));
  const unsigned ckbytes = (unsigned)((long)p.nck * N * dim * sizeof(float));
  const rsrc_t r_ck = make_rsrc(p.ckpt != nullptr ? (const void*)(p.ckpt + (long)b * p.nck * N * dim) : (const void*)x,
                                p.ckpt != nullptr ? ckbytes : 0u);

  // Raw values of the blocks ahead, loaded PD blocks early from clamped (in-bounds)
  // indices so no load sits behind a divergent branch and the HBM latency is covered by
  // PD blocks of compute; kept in the storage type until staged.
  // B/C: the wave needs B[t, wK..wK+K) and C[t, wK..wK+K) for the TS steps of a block,
  // the same for every lane.  Value v = t K + s of B sits in lane v % 16 of every
  // 16-lane row of register v / 16 (C likewise in registers R/2..R-1) and reaches all
  // lanes through a DPP row broadcast (folded into v_mul_f32_dpp for B): no LDS traffic.
  // Scalar loads into SGPR operands were tried and are slower: the scalar-cache latency
  // and the 64-bit scalar address arithmetic are not hidden.
  RI rx[PD][EPT], rdt[PD][EPT], rz[PD][EPT];
  RP rbc[PD][R];
  float rm[PD][EPT];
  float cx[EPT], cz[EPT], nx[EPT], nz[EPT];
  auto fetch = [&](int slot, int t0) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int t = min(t0 + w + i * NW, seq - 1);
      const unsigned off = ((unsigned)t * dim + cc) * (unsigned)sizeof(TI);
      rx[slot][i] = bload<TI>(r_x, off);
      rdt[slot][i] = bload<TI>(r_dt, off);
      if (HAS_Z) rz[slot][i] = bload<TI>(r_z, off);
      rm[slot][i] = MEAN ? bits_f32(bload<float>(r_m, (unsigned)t * 4u)) : 0.0f;
    }
    const int tmax = seq - 1 - t0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int v = (16 * r + (lane & 15)) % (TS * K);
      const int st = w * K + v % K;  // padding states (st >= ns) read 0 through an out-of-range offset
      const unsigned off =
          st < ns ? ((unsigned)(t0 + min(v / K, tmax)) * ns + st) * (unsigned)sizeof(TP) : OOB_OFF;
      rbc[slot][r] = bload<TP>(r < R / 2 ? r_B : r_C, off);
    }
  };
  auto stage = [&](int slot, int t0, int buf, float* xs, float* zs) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int tt = w + i * NW;
      const bool ok = (t0 + tt < seq) && cvalid;
      const float xv = bits_f32(rx[slot][i]);
      const float dtc = ok ? clampf(bits_f32(rdt[slot][i]), DT_MIN, DT_MAX) : 0.0f;
      s_dtc[buf][lane][tt] = dtc;
      s_dtx[buf][lane][tt] = ok ? (MEAN ? rm[slot][i] : dtc) * xv : 0.0f;
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
  for (int j = 0; j < PD; ++j) fetch(j, min(j, nblk - 1) * TS);
  stage(0, 0, 0, cx, cz);
  __syncthreads();

  for (int blk0 = 0; blk0 < npad; blk0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int blk = blk0 + u;
      const int t0 = blk * TS, buf = u & 1;  // PD is even, so u & 1 == blk & 1
      // ---- recurrence over the block ----
      float bcr[R];  // this block's B/C values (slot blk % PD == u)
#pragma unroll
      for (int r = 0; r < R; ++r) bcr[r] = bits_f32(rbc[u][r]);
      static_for<TS / 4>([&](auto qi) {
        constexpr int q = decltype(qi)::value;
        const float4 dc4 = *reinterpret_cast<const float4*>(&s_dtc[buf][lane][4 * q]);
        const float4 dx4 = *reinterpret_cast<const float4*>(&s_dtx[buf][lane][4 * q]);
        const float dcv[4] = {dc4.x, dc4.y, dc4.z, dc4.w};
        const float dxv[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
        static_for<4>([&](auto vi) {
          constexpr int v = decltype(vi)::value, tt = 4 * q + v;
          float acc = 0.0f;
          static_for<K>([&](auto si) {
            constexpr int s = decltype(si)::value;
            constexpr int vb = tt * K + s, vc = vb + TS * K;  // B and C value indices
            const float a = fast_exp2(dcv[v] * A2[s]);
            h[s] = fmaf(a, h[s], row_bcast<vb % 16>(bcr[vb / 16]) * dxv[v]);
            // the first state's C h is a DPP-folded multiply, not a broadcast + fma with 0
            if (WRITE_Y) acc = s == 0 ? row_bcast<vc % 16>(bcr[vc / 16]) * h[s]
                                      : fmaf(row_bcast<vc % 16>(bcr[vc / 16]), h[s], acc);
          });
          if (WRITE_Y) s_yp[buf][w][tt][lane] = acc;
        });
      });
      if (p.ckpt != nullptr) {
        const bool ok = cvalid && blk < nblk;
#pragma unroll
        for (int s = 0; s < K; ++s)
          bstore<float>(r_ck, ok ? (((unsigned)blk * N + w * K + s) * dim + c) * 4u : OOB_OFF, h[s]);
      }
      stage((u + 1) % PD, t0 + TS, buf ^ 1, nx, nz);
      fetch(u, min(blk + PD, nblk - 1) * TS);
      __syncthreads();
      // ---- y for the (t, d) this thread staged: sum the wave partials, D skip, gate ----
      if (WRITE_Y) {
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const int tt = w + i * NW;
          float y = 0.0f;
#pragma unroll
          for (int v = 0; v < NW; ++v) y += s_yp[buf][v][tt][lane];
          y = fmaf(Dc, cx[i], y);
          if (HAS_Z) y *= cz[i] * sigmoid_rcp(cz[i]);
          bstore<TI>(r_y, (t0 + tt < seq && cvalid) ? ((unsigned)(t0 + tt) * dim + c) * (unsigned)sizeof(TI) : OOB_OFF,
                     y);
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
template <typename TI, typename TP, int N, int KMAX, bool MEAN, bool HAS_Z>
__global__ __launch_bounds__((SSGeo<N, KMAX>::NT)) void ss_bwd_kernel(const SSArgs p, const TP* __restrict__ Bm,
                                                                      const TP* __restrict__ Cm) {
  using G = SSGeo<N, KMAX>;
  constexpr int K = G::K, NW = G::NW, NT = G::NT;
  static_assert(K == 1 || K == 2 || K == 4, "backward keeps one, two or four states per lane");
  constexpr int CK = SS_CK;          // recompute chunk (= checkpoint interval)
  constexpr int TS = 16 / K;         // reduction block (timesteps): 2 K TS = 32 outputs per wave
  constexpr bool BC_REG = K <= 2;    // the chunk's B/C values held in registers (else read from LDS)
  constexpr int PS = CK + 4;         // [channel][t] row stride (16-byte reads conflict-free)
  constexpr int EPT = CK * 64 / NT;  // staged (t, channel) elements per thread
  constexpr int GS = 2 * K * TS + 4;  // per-lane stride of a wave's dC/dB tile: b128 writes conflict-free
  constexpr int OPW = 2 * K * TS;     // dC/dB outputs per wave per block
  constexpr int LPO = 64 / OPW;       // lanes per output (each sums 64 / LPO channels)
  static_assert(EPT * NW == CK && CK % TS == 0 && LPO == 2, "staging layout");
  constexpr int BCN = CK * 2 * N;               // B/C values staged per chunk
  constexpr int BCT = (BCN + NT - 1) / NT;      // per thread (the last round partly idle)
  __shared__ __align__(16) float s_bc[CK][2 * N];  // per t: B[0..N), C[0..N)
  __shared__ __align__(16) float s_dtc[64][PS];
  __shared__ __align__(16) float s_dtx[64][PS];
  __shared__ __align__(16) float s_dy[64][PS];
  // each wave's private dC/dB tile: [lane][t][qty][state], reduced by the wave itself
  __shared__ __align__(16) float s_g[NW][64 * GS];
  // per-(t, d) partial sums over each wave's states for the chunk, px and pa
  // ([2][NW][CK][64]); the same memory first holds the gate's y partials ([NW][CK][64])
  __shared__ float s_pp[2 * NW * CK * 64];
  __shared__ float s_m[MEAN ? CK : 1][64];

  const TI* __restrict__ x = (const TI*)p.x;
  const TI* __restrict__ dt = (const TI*)p.dt;
  const TI* __restrict__ z = (const TI*)p.z;
  const TI* __restrict__ dout = (const TI*)p.dout;
  const TP* __restrict__ Am = (const TP*)p.A;
  const TP* __restrict__ Dv = (const TP*)p.D;
  const int seq = p.seq, dim = p.dim;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int logical = remap_xcd(blockIdx.x, gridDim.x);
  const int b = logical / p.ntile, tile = logical % p.ntile;
  const int c = tile * 64 + lane;
  const bool cvalid = c < dim;
  const int cc = min(c, dim - 1);
  auto pp = [&](int q, int v, int t) -> float& { return s_pp[((q * NW + v) * CK + t) * 64 + lane]; };

  const int ns = p.nst;
  float A1[K], A2[K], dh[K], dA[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    A1[s] = (cvalid && w * K + s < ns) ? ld(Am, (long)c * ns + w * K + s) : 0.0f;
    A2[s] = A1[s] * LOG2E;
    dh[s] = 0.0f;
    dA[s] = 0.0f;
  }
  const float Dc = (Dv != nullptr && cvalid) ? ld(Dv, c) : 0.0f;
  float dD = 0.0f;
  const long rowbase = (long)b * seq * dim;

  // raw values of the next chunk (in reverse order), loaded a chunk ahead through buffer
  // resources on this batch row (SGPR base, 32-bit offsets: no 64-bit address VALU)
  typedef typename Bits<TI>::type RI;
  typedef typename Bits<TP>::type RP;
  const unsigned rowbytes = (unsigned)((long)seq * dim * sizeof(TI));
  const rsrc_t r_x = make_rsrc(x + rowbase, rowbytes), r_dt = make_rsrc(dt + rowbase, rowbytes);
  const rsrc_t r_do = make_rsrc(dout + rowbase, rowbytes);
  const rsrc_t r_z = make_rsrc(HAS_Z ? z + rowbase : x + rowbase, rowbytes);
  const unsigned bcbytes = (unsigned)((long)seq * ns * sizeof(TP));
  const rsrc_t r_B = make_rsrc(Bm + (long)b * seq * ns, bcbytes), r_C = make_rsrc(Cm + (long)b * seq * ns, bcbytes);
  const rsrc_t r_m =
      make_rsrc(MEAN ? (const void*)(p.dtmean + (long)b * seq) : (const void*)x, (unsigned)(seq * sizeof(float)));
  const rsrc_t r_dx = make_rsrc((TI*)p.dx + rowbase, rowbytes), r_ddt = make_rsrc((TI*)p.ddt + rowbase, rowbytes);
  const rsrc_t r_dz = make_rsrc(p.dz != nullptr ? (TI*)p.dz + rowbase : (TI*)p.dx + rowbase, rowbytes);
  RI rx[EPT], rdt[EPT], rdo[EPT], rz[EPT];
  RP rbc[BCT];
  float rm[EPT];
  float rck[K];  // the checkpoint the fetched chunk starts from (its predecessor's state)
  // this thread's staged (t, d) values, kept for the per-(t, d) epilogues
  float ex[EPT], edtb[EPT], emask[EPT], edy[EPT], ego[EPT], ez[EPT];
  auto fetch = [&](int ts) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int t = min(ts + w + i * NW, seq - 1);
      const unsigned off = ((unsigned)t * dim + cc) * (unsigned)sizeof(TI);
      rx[i] = bload<TI>(r_x, off);
      rdt[i] = bload<TI>(r_dt, off);
      rdo[i] = bload<TI>(r_do, off);
      if (HAS_Z) rz[i] = bload<TI>(r_z, off);
      rm[i] = MEAN ? bits_f32(bload<float>(r_m, (unsigned)t * 4u)) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < BCT; ++i) {
      const int e = min(tid + i * NT, BCN - 1);  // clamped: the load stays unconditional
      const int r = e % (2 * N);
      // padding states (r % N >= ns) read 0 through an out-of-range offset
      const unsigned off = r % N < ns ? ((unsigned)min(ts + e / (2 * N), seq - 1) * ns + (r % N)) * (unsigned)sizeof(TP)
                                      : OOB_OFF;
      // lanes split between B and C: both loads issue, the other one out of bounds reads 0
      rbc[i] = bload<TP>(r_B, r < N ? off : OOB_OFF) | bload<TP>(r_C, r < N ? OOB_OFF : off);
    }
    const int kp = max(ts / CK - 1, 0);  // chunk 0 starts from zero (selected at use)
#pragma unroll
    for (int s = 0; s < K; ++s) rck[s] = p.ckpt[(((long)b * p.nck + kp) * N + w * K + s) * dim + cc];
  };

  // The next chunk's inputs and checkpoint are fetched one chunk ahead, unconditionally
  // (chunk 0 fetches itself again): a conditional fetch makes the compiler drain every
  // outstanding load at the loop latch.
  fetch((p.nck - 1) * CK);
  for (int k = p.nck - 1; k >= 0; --k) {
    const int ts = k * CK;
    // ---- stage the chunk ---------------------------------------------------------
#pragma unroll
    for (int i = 0; i < BCT; ++i) {
      const int e = tid + i * NT;
      if (BCN % NT == 0 || e < BCN) s_bc[e / (2 * N)][e % (2 * N)] = bits_f32(rbc[i]);
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int tt = w + i * NW;
      const bool ok = (ts + tt < seq) && cvalid;
      const float dtr = bits_f32(rdt[i]);
      const float dtc = ok ? clampf(dtr, DT_MIN, DT_MAX) : 0.0f;
      const float dtb = ok ? (MEAN ? rm[i] : dtc) : 0.0f;
      const float xv = ok ? bits_f32(rx[i]) : 0.0f;
      ex[i] = xv;
      edtb[i] = dtb;
      emask[i] = (ok && dtr >= DT_MIN && dtr <= DT_MAX) ? 1.0f : 0.0f;
      ego[i] = ok ? bits_f32(rdo[i]) : 0.0f;
      ez[i] = (HAS_Z && ok) ? bits_f32(rz[i]) : 0.0f;
      s_dtc[lane][tt] = dtc;
      s_dtx[lane][tt] = dtb * xv;
      if (!HAS_Z) {
        edy[i] = ego[i];
        s_dy[lane][tt] = ego[i];
      }
    }
    float ck0[K];
#pragma unroll
    for (int s = 0; s < K; ++s) ck0[s] = rck[s];
    fetch(max(k - 1, 0) * CK);
    __syncthreads();

    // ---- recompute the chunk's states and decays from its checkpoint ---------------
    // states, decays and this wave's B/C values of the chunk, kept in registers for the
    // reverse pass (reading B/C from LDS once per chunk halves that LDS traffic)
    float h0[K], hs[CK][K], as[CK][K], bB[BC_REG ? CK : 1][K], bC[BC_REG ? CK : 1][K];
#pragma unroll
    for (int s = 0; s < K; ++s)
      h0[s] = (k > 0 && cvalid) ? ck0[s] : 0.0f;
    {
      float hh[K];
#pragma unroll
      for (int s = 0; s < K; ++s) hh[s] = h0[s];
#pragma unroll
      for (int q = 0; q < CK / 4; ++q) {
        const float4 dc4 = *reinterpret_cast<const float4*>(&s_dtc[lane][4 * q]);
        const float4 dx4 = *reinterpret_cast<const float4*>(&s_dtx[lane][4 * q]);
        const float dcv[4] = {dc4.x, dc4.y, dc4.z, dc4.w};
        const float dxv[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = 4 * q + u;
          const float* bc = &s_bc[j][w * K];
          float acc = 0.0f;
#pragma unroll
          for (int s = 0; s < K; ++s) {
            if constexpr (BC_REG) {
              bB[j][s] = bc[s];
              bC[j][s] = bc[N + s];
            }
            const float a = fast_exp2(dcv[u] * A2[s]);
            hh[s] = fmaf(a, hh[s], dxv[u] * bc[s]);
            as[j][s] = a;
            hs[j][s] = hh[s];
            if (HAS_Z) acc = fmaf(bc[N + s], hh[s], acc);
          }
          if (HAS_Z) pp(0, w, j) = acc;
        }
      }
    }

    // ---- gate: dy = dout silu(z); dz = dout y silu'(z) (y before the gate) -----------
    if (HAS_Z) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        const int tt = w + i * NW;
        float y = 0.0f;
#pragma unroll
        for (int v = 0; v < NW; ++v) y += pp(0, v, tt);
        y = fmaf(Dc, ex[i], y);
        const float sg = sigmoid_rcp(ez[i]);
        edy[i] = ego[i] * ez[i] * sg;
        s_dy[lane][tt] = edy[i];
        if (p.dz != nullptr)
          bstore<TI>(r_dz, (ts + tt < seq && cvalid) ? ((unsigned)(ts + tt) * dim + c) * (unsigned)sizeof(TI) : OOB_OFF,
                     ego[i] * y * sg * (1.0f + ez[i] * (1.0f - sg)));
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < EPT; ++i) dD = fmaf(edy[i], ex[i], dD);

    // ---- reverse recurrence, in blocks of TS timesteps ------------------------------
#pragma unroll
    for (int jb = CK - TS; jb >= 0; jb -= TS) {
      float dyv[TS], dcv[TS], dxv[TS];
#pragma unroll
      for (int q = 0; q < TS / 4; ++q) {
        const float4 a4 = *reinterpret_cast<const float4*>(&s_dy[lane][jb + 4 * q]);
        const float4 b4 = *reinterpret_cast<const float4*>(&s_dtc[lane][jb + 4 * q]);
        const float4 c4 = *reinterpret_cast<const float4*>(&s_dtx[lane][jb + 4 * q]);
        dyv[4 * q] = a4.x; dyv[4 * q + 1] = a4.y; dyv[4 * q + 2] = a4.z; dyv[4 * q + 3] = a4.w;
        dcv[4 * q] = b4.x; dcv[4 * q + 1] = b4.y; dcv[4 * q + 2] = b4.z; dcv[4 * q + 3] = b4.w;
        dxv[4 * q] = c4.x; dxv[4 * q + 1] = c4.y; dxv[4 * q + 2] = c4.z; dxv[4 * q + 3] = c4.w;
      }
      float* g = &s_g[w][lane * GS];
#pragma unroll
      for (int j = TS - 1; j >= 0; --j) {
        const int jj = jb + j;
        float px = 0.0f, pa = 0.0f, gC[K], gB[K];
#pragma unroll
        for (int s = 0; s < K; ++s) {
          const float Bv = BC_REG ? bB[BC_REG ? jj : 0][s] : s_bc[jj][w * K + s];
          const float Cv = BC_REG ? bC[BC_REG ? jj : 0][s] : s_bc[jj][N + w * K + s];
          dh[s] = fmaf(dyv[j], Cv, dh[s]);
          gC[s] = dyv[j] * hs[jj][s];
          gB[s] = dh[s] * dxv[j];
          px = fmaf(dh[s], Bv, px);
          dh[s] *= as[jj][s];
          const float ga = dh[s] * (jj > 0 ? hs[jj - 1][s] : h0[s]);
          dA[s] = fmaf(ga, dcv[j], dA[s]);
          pa = fmaf(ga, A1[s], pa);
        }
        if constexpr (K == 4) {
          *reinterpret_cast<float4*>(g + j * 2 * K) = make_float4(gC[0], gC[1], gC[2], gC[3]);
          *reinterpret_cast<float4*>(g + j * 2 * K + K) = make_float4(gB[0], gB[1], gB[2], gB[3]);
        } else if constexpr (K == 2) {
          *reinterpret_cast<float4*>(g + j * 2 * K) = make_float4(gC[0], gC[1], gB[0], gB[1]);
        } else {
          *reinterpret_cast<float2*>(g + j * 2 * K) = make_float2(gC[0], gB[0]);
        }
        pp(0, w, jj) = px;
        pp(1, w, jj) = pa;
      }
      // sums over the 64 channels of this wave's dC (qty 0) and dB (qty 1) per (t, n):
      // the tile is the wave's own, so LDS ordering within the wave replaces a barrier
      // and other waves keep computing meanwhile.  Output o = (t, qty, state) is the
      // o-th float of every lane row; LPO = 2 lanes share it (channels 0..31 / 32..63).
      {
        __builtin_amdgcn_wave_barrier();  // keep the tile writes before the column reads
        const int o = lane % OPW, hf = lane / OPW;
        const float* src = &s_g[w][hf * (64 / LPO) * GS + o];
        float acc = 0.0f;
#pragma unroll 16
        for (int l = 0; l < 64 / LPO; ++l) acc += src[l * GS];
        __builtin_amdgcn_wave_barrier();  // and the reads before the next block's writes
        acc += __shfl_xor(acc, 32);
        const int j = o / (2 * K), qty = (o / K) % 2, n = w * K + o % K;
        const int t = ts + jb + j;
        if (hf == 0 && t < seq) p.part_bc[((((long)tile * p.batch + b) * seq + t) * 2 + qty) * N + n] = acc;
      }
    }
    // ---- sums over the states: dx, ddt for the (t, d) this thread staged --------------
    __syncthreads();
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int tt = w + i * NW;
      float pxs = 0.0f, pas = 0.0f;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        pxs += pp(0, v, tt);
        pas += pp(1, v, tt);
      }
      {
        const unsigned off = (ts + tt < seq && cvalid) ? ((unsigned)(ts + tt) * dim + c) * (unsigned)sizeof(TI) : OOB_OFF;
        bstore<TI>(r_dx, off, fmaf(pxs, edtb[i], edy[i] * Dc));
        bstore<TI>(r_ddt, off, emask[i] * (MEAN ? pas : fmaf(pxs, ex[i], pas)));
      }
      if (MEAN) s_m[tt][lane] = pxs * ex[i];  // dt-mean coupling, summed over channels below
    }
    if (MEAN) {
      __syncthreads();
      if (tid < CK) {
        float acc = 0.0f;
        for (int l = 0; l < 64; ++l) acc += s_m[tid][l];
        const int t = ts + tid;
        if (t < seq) p.part_m[((long)tile * p.batch + b) * seq + t] = acc;
      }
    }
  }
  // dA partial per (b, d, n); dD partial per (b, d): the lanes of one channel in the
  // NW waves hold disjoint timesteps
  if (cvalid) {
#pragma unroll
    for (int s = 0; s < K; ++s) p.part_a[((long)b * dim + c) * N + w * K + s] = dA[s];
  }
  __syncthreads();  // the last chunk's epilogue has read s_pp
  pp(0, w, 0) = dD;
  __syncthreads();
  if (w == 0 && cvalid) {
    float acc = 0.0f;
#pragma unroll
    for (int v = 0; v < NW; ++v) acc += pp(0, v, 0);
    p.part_d[(long)b * dim + c] = acc;
  }
}

// dB, dC = sum over channel tiles; partials carry NP (padded) states, outputs ns
__global__ __launch_bounds__(256) void ss_reduce_bc_kernel(const float* __restrict__ part, float* __restrict__ dB,
                                                           float* __restrict__ dC, int ntile, long rows, int NP,
                                                           int ns) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // over rows * 2NP
  const long total = rows * 2 * NP;
  if (i >= total) return;
  const long row = i / (2 * NP);
  const int r = (int)(i % (2 * NP));
  const int qty = r / NP, nn = r % NP;
  if (nn >= ns) return;
  float acc = 0.0f;
  for (int tl = 0; tl < ntile; ++tl) acc += part[(long)tl * total + i];
  if (qty == 0) {
    if (dC) dC[row * ns + nn] = acc;
  } else {
    if (dB) dB[row * ns + nn] = acc;
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
constexpr int SS_MAX_STATE = 32;  // the reference's limit (fused_selective_scan.cu:57-76, _backward.cu:59)

// the power of two the kernels are compiled for: NP >= N, the states past N are padding
inline int padded_state(int N) {
  int np = 1;
  while (np < N) np *= 2;
  return np;
}

// one workgroup per (batch, 64-channel tile)
inline int ntiles(int dim) { return (dim + 63) / 64; }

inline long num_chunks(int seq) { return (seq + SS_CK - 1) / SS_CK; }

struct WsLayout {
  size_t ckpt, dtmean, part_bc, part_a, part_d, part_m, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline WsLayout bwd_layout(int batch, int seq, int dim, int nst, bool need_ckpt, bool mean_mode) {
  const int N = padded_state(nst);
  WsLayout w{};
  const long nck = num_chunks(seq);
  const int nt = ntiles(dim);
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

template <typename TI, typename TP, int N, int KMAX>
void launch_fwd_k(hipStream_t s, const SSArgs& a) {
  constexpr int NT = SSGeo<N, KMAX>::NT;
  const int grid = a.batch * a.ntile;
  const bool mean = a.dtmean != nullptr, hz = a.z != nullptr;
  const TP* Bp = (const TP*)a.B;
  const TP* Cp = (const TP*)a.C;
  if (a.out == nullptr) {  // checkpoints only (backward without saved states)
    if (mean) ss_fwd_kernel<TI, TP, N, KMAX, true, false, false><<<grid, NT, 0, s>>>(a, Bp, Cp);
    else ss_fwd_kernel<TI, TP, N, KMAX, false, false, false><<<grid, NT, 0, s>>>(a, Bp, Cp);
  } else if (mean && hz) {
    ss_fwd_kernel<TI, TP, N, KMAX, true, true, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  } else if (mean) {
    ss_fwd_kernel<TI, TP, N, KMAX, true, false, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  } else if (hz) {
    ss_fwd_kernel<TI, TP, N, KMAX, false, true, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  } else {
    ss_fwd_kernel<TI, TP, N, KMAX, false, false, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  }
}

// States per lane.  Backward: two (2 waves per SIMD at config-2 size, 192 workgroups of 8
// waves), which hides the LDS and exp latencies better than four states per lane at 1 wave
// per SIMD (measured on MI355X: 722 vs 811 us); at NP = 32 four (8 waves), since 16 waves'
// dC/dB tiles and state-sum partials do not fit the 160 KB of LDS.  Forward: one (16 waves
// per workgroup, 4 per SIMD; 190 vs 200 us with two states per lane, interleaved A/B).
template <int N> constexpr int ss_kmax_bwd() { return N >= 32 ? 4 : 2; }
constexpr int SS_KMAX_FWD = 1;

template <typename TI, typename TP, int N>
void launch_fwd_t(hipStream_t s, const SSArgs& a) {
  launch_fwd_k<TI, TP, N, SS_KMAX_FWD>(s, a);
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

template <typename TI, typename TP, int N, int KMAX>
void launch_bwd_k(hipStream_t s, const SSArgs& a) {
  constexpr int NT = SSGeo<N, KMAX>::NT;
  const int grid = a.batch * a.ntile;
  const bool mean = a.dtmean != nullptr, hz = a.z != nullptr;
  const TP* Bp = (const TP*)a.B;
  const TP* Cp = (const TP*)a.C;
  if (mean && hz) ss_bwd_kernel<TI, TP, N, KMAX, true, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  else if (mean) ss_bwd_kernel<TI, TP, N, KMAX, true, false><<<grid, NT, 0, s>>>(a, Bp, Cp);
  else if (hz) ss_bwd_kernel<TI, TP, N, KMAX, false, true><<<grid, NT, 0, s>>>(a, Bp, Cp);
  else ss_bwd_kernel<TI, TP, N, KMAX, false, false><<<grid, NT, 0, s>>>(a, Bp, Cp);
}

template <typename TI, typename TP, int N>
void launch_bwd_t(hipStream_t s, const SSArgs& a) {
  launch_bwd_k<TI, TP, N, ss_kmax_bwd<N>()>(s, a);
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
  return (size_t)batch * edf::num_chunks(seq_len) * edf::padded_state(state) * hidden * sizeof(float);
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
  // the kernels address one batch row of x, dt, z, y (and of B, C and the checkpoints)
  // through buffer resources with 32-bit byte offsets
  EDF_REQUIRE((long)seq_len * hidden * (io_dtype == EDF_BF16 ? 2 : 4) < (1L << 31) &&
                  num_chunks(seq_len) * padded_state(state) * hidden * 4 < (1L << 31),
              EDF_ERR_UNSUPPORTED, "one batch row of seq_len * hidden elements (and its checkpoints) must stay below 2 GiB");
  const size_t need = edf_selective_scan_workspace_bytes(batch, seq_len, hidden, state, mode);
  EDF_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), EDF_ERR_WORKSPACE,
              "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  SSArgs a{};
  a.x = x; a.dt = dt; a.A = A; a.B = B; a.C = C; a.D = D; a.z = z; a.out = out;
  a.ckpt = (float*)states;
  a.batch = batch; a.seq = seq_len; a.dim = hidden; a.nst = state;
  a.nck = (int)num_chunks(seq_len);
  a.ntile = ntiles(hidden);
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
  EDF_REQUIRE(x && dt && A && B && C && grad_out && grad_x && grad_dt, EDF_ERR_INVALID_ARG, "null tensor pointer");
  // the backward kernel addresses one batch row of x, dt, dy, z, dx, ddt, dz (and of B, C)
  // through a buffer resource with 32-bit byte offsets
  EDF_REQUIRE((long)seq_len * hidden * (io_dtype == EDF_BF16 ? 2 : 4) < (1L << 31) &&
                  (long)seq_len * (state > 1 ? state : 1) * 4 < (1L << 31),
              EDF_ERR_UNSUPPORTED, "backward needs seq_len * hidden elements of one batch row below 2 GiB");
  const bool mean_mode = mode == EDF_SS_DT_MEAN;
  const WsLayout L = bwd_layout(batch, seq_len, hidden, state, states == nullptr, mean_mode);
  EDF_REQUIRE(workspace && workspace_bytes >= L.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              L.total);
  hipStream_t s = as_stream(stream);
  char* ws = (char*)workspace;
  SSArgs a{};
  a.x = x; a.dt = dt; a.A = A; a.B = B; a.C = C; a.D = D; a.z = z;
  a.batch = batch; a.seq = seq_len; a.dim = hidden; a.nst = state;
  a.nck = (int)num_chunks(seq_len);
  a.ntile = ntiles(hidden);
  if (mean_mode) {
    a.dtmean = (float*)(ws + L.dtmean);
    rc = run_dtmean(s, dt, (float*)(ws + L.dtmean), batch, seq_len, hidden, io_dtype);
    if (rc) return rc;
  }
  a.ckpt = states ? (float*)states : (float*)(ws + L.ckpt);
  if (states == nullptr) {  // recompute checkpoints with a forward pass that writes no output
    SSArgs f = a;
    f.out = nullptr;
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
    ss_reduce_bc_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(a.part_bc, (float*)grad_B, (float*)grad_C,
                                                                        a.ntile, rows, np, state);
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
