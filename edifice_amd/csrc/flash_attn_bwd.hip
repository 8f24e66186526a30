// Flash attention backward for gfx950.
//
// Semantics (reference): lib/edifice/cuda/fused_scan.ex:3527-3570
// (flash_attention_backward_fallback): P = softmax(S), dV = P^T dO, dP = dO V^T,
// dS = P (dP - rowsum(dP P)) / sqrt(d), dQ = dS K, dK = dS^T Q; and
// native/cuda/fused_flash_attention_backward.cu:256-340 for D = rowsum(dO * O).
// The softmax is recomputed from the forward's log-sum-exp (natural log).
//
// bf16 / head_dim in {32, 64, 128} runs three kernels, none of which allocates or
// uses atomics:
//   1. D = rowsum(dO * O) (float32, one 16-lane group per row);
//   2. dK/dV: a workgroup owns 128 keys (32 per wave, K and V kept in registers as
//      MFMA B fragments) and walks 64-query tiles; S = Q K^T puts one key per lane
//      column, so P and dS feed dV^T += dO^T P and dK^T += Q^T dS directly from
//      registers, and dO^T, Q^T come from the row-major LDS tiles through
//      ds_read_b64_tr_b16 (no transposed staging);
//   3. dQ: a workgroup owns 128 queries (32 per wave, Q and dO in registers) and
//      walks 64-key tiles; S^T = K Q^T puts one query per lane, so dS^T feeds
//      dQ^T += K^T dS^T from registers (K^T by transposed reads).
//   Tiles are double-buffered in LDS (one barrier per tile).
//   Causal: only tiles on or below the diagonal are visited.
// float32 or other head_dim: wave-per-row kernels (parity path).
#include "edf_abi.hpp"
#include "edf_common.hpp"
#include "edf_mfma.hpp"

#include <mutex>
#include <type_traits>

namespace edf {
namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// ---- D = rowsum(dO * O) ------------------------------------------------------
template <typename TT>
__global__ __launch_bounds__(256) void fa_bwd_dot_kernel(const TT* __restrict__ O, const TT* __restrict__ dO,
                                                         float* __restrict__ Dv, long rows, int HD) {
  const long row = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  float acc = 0.0f;
  if (row < rows)
    for (int d = sub; d < HD; d += 16) acc = fmaf(ld(O, row * HD + d), ld(dO, row * HD + d), acc);
  acc = row16_sum(acc);  // the 16 lanes of a row group are one DPP row
  if (row < rows && sub == 0) Dv[row] = acc;
}

// ---- dK / dV -------------------------------------------------------------------
// A workgroup owns 128 keys (32 per wave: K and V stay in registers as the B fragments
// of S = Q K^T and dP = dO V^T, so a lane owns one key column) and walks 64-query tiles
// of Q, dO, LSE and D staged in a double-buffered LDS ring (one barrier per tile).
// dV^T += dO^T P and dK^T += Q^T dS take P and dS straight from the accumulator
// registers as B fragments (query order as the accumulator rows hold it) and the
// transposed A operands from the row-major tiles with ds_read_b64_tr_b16.
// FOX (forgetting attention, causal): scores carry + (cs_q - cs_k) sqrt(d) (sqd); this
// kernel also writes -sum_q dS_qk, the key side of d cs, to DCSK (f32 [BH][T]).
template <int HD, bool CAUSAL, bool FOX = false>
__global__ __launch_bounds__(256, 1) void fa_bwd_dkdv_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                             const bf16* __restrict__ V, const bf16* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             const float* __restrict__ Dd, bf16* __restrict__ dK,
                                                             bf16* __restrict__ dV, int T, float scale_log2,
                                                             float scale, const bf16* __restrict__ CS,
                                                             float* __restrict__ DCSK, float sqd) {
  constexpr int BKEY = 128, BQ = 64;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  constexpr int CPR = HD / 8;          // 16-byte chunks per row
  constexpr int CPT = BQ * CPR / 256;  // chunks per thread per tile and tensor
  static_assert(CPT >= 1 && BQ * CPR % 256 == 0, "tile staging");
  __shared__ __attribute__((aligned(16))) bf16 sQ[2][lds_tile_elems<HD>(BQ)];
  __shared__ __attribute__((aligned(16))) bf16 sdO[2][lds_tile_elems<HD>(BQ)];
  __shared__ __attribute__((aligned(16))) float sL[2][BQ];
  __shared__ __attribute__((aligned(16))) float sD[2][BQ];
  __shared__ __attribute__((aligned(16))) float sC[FOX ? 2 : 1][FOX ? BQ : 4];  // cs of the tile's queries

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  int xb;
  long bh;
  head_block(xb, bh);
  const int kb0 = xb * BKEY;  // causal: low key blocks see the most queries and run first
  const int kw = kb0 + 32 * w;
  const int mykey = kw + li;
  const long base = bh * T * HD;

  bf16x8 kf[NKK], vf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    kf[kk] = mykey < T ? *(const bf16x8*)(K + base + (long)mykey * HD + kk * 16 + 8 * g) : bf16x8{};
    vf[kk] = mykey < T ? *(const bf16x8*)(V + base + (long)mykey * HD + kk * 16 + 8 * g) : bf16x8{};
  }
  f32x16 dkt[NDT], dvt[NDT];  // dK^T, dV^T: rows = dims, column = this lane's key
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dkt[dt] = zero16();
    dvt[dt] = zero16();
  }

  bf16x8 rq[CPT], ro[CPT];
  float rl = 0.0f, rd = 0.0f, rc = 0.0f;
  const float csk = FOX && mykey < T ? to_f32(CS[bh * T + mykey]) * sqd : 0.0f;
  float colacc = 0.0f;  // FOX: sum over queries of this lane's key's dS
  auto gload = [&](int q0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
      // rows past the end are clamped, not branched around: their P and dS are 0
      const long q = min(q0 + row, T - 1);
      rq[i] = *(const bf16x8*)(Q + base + q * HD + col);
      ro[i] = *(const bf16x8*)(dO + base + q * HD + col);
    }
    if (tid < BQ) {
      const long q = min(q0 + tid, T - 1);
      const float lv = LSE[bh * T + q];
      // a query past the end gets an infinite LSE, so its P and dS are 0 in every body
      rl = q0 + tid < T ? lv * LOG2E : INFINITY;
      rd = Dd[bh * T + q];
      if constexpr (FOX) rc = to_f32(CS[bh * T + q]);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
      *(bf16x8*)(&sQ[buf][lds_off<HD>(row, col)]) = rq[i];
      *(bf16x8*)(&sdO[buf][lds_off<HD>(row, col)]) = ro[i];
    }
    if (tid < BQ) {
      sL[buf][tid] = rl;
      sD[buf][tid] = rd;
      if constexpr (FOX) sC[buf][tid] = rc;
    }
  };

  const int qstart = CAUSAL ? kb0 : 0;  // causal: queries before kb0 see none of these keys
  const int ntile = qstart < T ? (T - qstart + BQ - 1) / BQ : 0;
  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);  // transposed-read column within a 32-dim tile
  const int kr = 4 * (grp >> 1) + (i16 >> 2);     // and row within a 16-query chunk
  if (ntile > 0) {
    gload(qstart);
    sstore(0);
    if (ntile > 1) gload(qstart + BQ);
  }
  __syncthreads();
  for (int it = 0; it < ntile; ++it) {
    const int q0 = qstart + it * BQ, buf = it & 1;
#pragma unroll
    for (int sub = 0; sub < BQ / 32; ++sub) {
      const int qs = q0 + 32 * sub;
      if (CAUSAL && qs + 31 < kw) continue;  // every query of the sub-tile precedes this wave's keys
      auto subtile = [&](auto masked) {
      constexpr bool MASK = decltype(masked)::value;
      // S = Q K^T and dP = dO V^T (32 queries x 32 keys); lane owns key column
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const int off = lds_off<HD>(32 * sub + li, kk * 16 + 8 * g);
        const bf16x8 aq = *(const bf16x8*)(&sQ[buf][off]);
        const bf16x8 ao = *(const bf16x8*)(&sdO[buf][off]);
        s = mfma32(aq, kf[kk], s);
        dp = mfma32(ao, vf[kk], dp);
      }
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const f32x4 lv = *(const f32x4*)(&sL[buf][32 * sub + 8 * rb + 4 * g]);
        const f32x4 dv4 = *(const f32x4*)(&sD[buf][32 * sub + 8 * rb + 4 * g]);
        f32x4 cq4 = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (FOX) cq4 = *(const f32x4*)(&sC[buf][32 * sub + 8 * rb + 4 * g]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rb * 4 + e;
          if constexpr (FOX) s[r] += fmaf(cq4[e], sqd, -csk);
          float p = fast_exp2(fmaf(s[r], scale_log2, -lv[e]));
          if constexpr (MASK) {
            const int q = qs + 8 * rb + 4 * g + e;
            p = (q >= T || mykey >= T || (CAUSAL && mykey > q)) ? 0.0f : p;
          }
          s[r] = p;
          dp[r] = p * (dp[r] - dv4[e]);  // dS / scale: 1/sqrt(d) is applied to dK once at the end
          if constexpr (FOX) colacc += dp[r];
        }
      }
      // B fragments: queries 16 kc + 4 g + {0..3} and 16 kc + 8 + 4 g + {0..3}
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pb[kc][e] = (bf16)s[8 * kc + e];
          db[kc][e] = (bf16)dp[8 * kc + e];
        }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const int row = 32 * sub + 16 * kc + kr, col = dt * 32 + d0;
          const int o0 = lds_off<HD>(row, col), o1 = lds_off<HD>(row + 8, col);
          const bf16x8 ao = cat4(lds_read_tr16(&sdO[buf][o0]), lds_read_tr16(&sdO[buf][o1]));
          const bf16x8 aq = cat4(lds_read_tr16(&sQ[buf][o0]), lds_read_tr16(&sQ[buf][o1]));
          dvt[dt] = mfma32(ao, pb[kc], dvt[dt]);
          dkt[dt] = mfma32(aq, db[kc], dkt[dt]);
        }
      }
      };
      // Only sub-tiles on the causal diagonal need the masked body: queries past the end
      // have P = 0 by their LSE, and keys past the end only feed their own (unstored) dK,
      // dV columns.  The non-causal kernel thus has a single body.
      if (CAUSAL && qs < kw + 31) subtile(std::true_type{});
      else subtile(std::false_type{});
    }
    if (it + 1 < ntile) {
      sstore(buf ^ 1);
      if (it + 2 < ntile) gload(q0 + 2 * BQ);
    }
    __syncthreads();
  }
  if constexpr (FOX) {
    colacc += __shfl_xor(colacc, 32);  // the two lane halves hold the key's other queries
    if (g == 0 && mykey < T) DCSK[bh * T + mykey] = -colacc;
  }
  // lane li owns key mykey; register r of tile dt holds dim dt * 32 + d_row(r, g)
  if (mykey < T) {
    bf16* krow = dK + base + (long)mykey * HD;
    bf16* vrow = dV + base + (long)mykey * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 a, b;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[e] = (bf16)(dkt[dt][rb * 4 + e] * scale);
          b[e] = (bf16)dvt[dt][rb * 4 + e];
        }
        *(bf16x4*)(krow + dt * 32 + 8 * rb + 4 * g) = a;
        *(bf16x4*)(vrow + dt * 32 + 8 * rb + 4 * g) = b;
      }
  }
}

// ---- dQ -----------------------------------------------------------------------------
// A workgroup owns 128 queries (32 per wave: Q and dO in registers as B fragments of
// S^T = K Q^T and dP^T = V dO^T, so a lane owns one query column) and walks 64-key tiles
// of K and V in a double-buffered LDS ring.  dQ^T += K^T dS^T takes dS^T from the
// accumulator registers and K^T from the row-major K tile with transposed reads.
// FOX: as the dK/dV kernel; writes d cs = sum_k dS_qk plus the key side DCSK to DCS.
template <int HD, bool CAUSAL, bool FOX = false>
__global__ __launch_bounds__(256, 1) void fa_bwd_dq_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                           const bf16* __restrict__ V, const bf16* __restrict__ dO,
                                                           const float* __restrict__ LSE, const float* __restrict__ Dd,
                                                           bf16* __restrict__ dQ, int T, float scale_log2,
                                                           float scale, const bf16* __restrict__ CS,
                                                           const float* __restrict__ DCSK, bf16* __restrict__ DCS,
                                                           float sqd) {
  constexpr int BM = 128, BN = 64;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  constexpr int CPR = HD / 8;
  constexpr int CPT = BN * CPR / 256;
  static_assert(CPT >= 1 && BN * CPR % 256 == 0, "tile staging");
  __shared__ __attribute__((aligned(16))) bf16 sK[2][lds_tile_elems<HD>(BN)];
  __shared__ __attribute__((aligned(16))) bf16 sV[2][lds_tile_elems<HD>(BN)];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  int xb;
  long bh;
  head_block(xb, bh);
  const int qb = CAUSAL ? (gridDim.x - 1 - xb) : xb;  // heaviest blocks first
  const int q0 = qb * BM;
  const int qw = q0 + 32 * w;
  const int myq = qw + li;
  const long base = bh * T * HD;

  bf16x8 qf[NKK], of[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    qf[kk] = myq < T ? *(const bf16x8*)(Q + base + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
    of[kk] = myq < T ? *(const bf16x8*)(dO + base + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
  }
  const float myl = myq < T ? LSE[bh * T + myq] * LOG2E : 0.0f;
  const float myd = myq < T ? Dd[bh * T + myq] : 0.0f;
  __shared__ __attribute__((aligned(16))) float sCS[FOX ? 2 : 1][FOX ? BN : 4];  // cs of the tile's keys
  const float csq = FOX && myq < T ? to_f32(CS[bh * T + myq]) * sqd : 0.0f;
  float rowacc = 0.0f, rcs = 0.0f;  // FOX: sum over keys of this lane's query's dS
  f32x16 dqt[NDT];  // dQ^T: rows = dims, column = this lane's query
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dqt[dt] = zero16();

  bf16x8 rk[CPT], rv[CPT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
      // rows past the end are clamped, not branched around: their P is masked to 0
      const long key = min(k0 + row, T - 1);
      rk[i] = *(const bf16x8*)(K + base + key * HD + col);
      rv[i] = *(const bf16x8*)(V + base + key * HD + col);
    }
    if constexpr (FOX) {
      if (tid < BN) rcs = to_f32(CS[bh * T + min(k0 + tid, T - 1)]);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
      *(bf16x8*)(&sK[buf][lds_off<HD>(row, col)]) = rk[i];
      *(bf16x8*)(&sV[buf][lds_off<HD>(row, col)]) = rv[i];
    }
    if constexpr (FOX) {
      if (tid < BN) sCS[buf][tid] = rcs;
    }
  };

  const int kend = CAUSAL ? min(T, q0 + BM) : T;
  const int nkt = (kend + BN - 1) / BN;
  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
  const int kr = 4 * (grp >> 1) + (i16 >> 2);
  gload(0);
  sstore(0);
  if (nkt > 1) gload(BN);
  __syncthreads();
  auto tile = [&](int kt, auto masked) {
      constexpr bool MASK = decltype(masked)::value;
      const int k0 = kt * BN, buf = kt & 1;
      f32x16 s[2], dp[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        s[h2] = zero16();
        dp[h2] = zero16();
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          const int off = lds_off<HD>(h2 * 32 + li, kk * 16 + 8 * g);
          const bf16x8 ak = *(const bf16x8*)(&sK[buf][off]);
          const bf16x8 av = *(const bf16x8*)(&sV[buf][off]);
          s[h2] = mfma32(ak, qf[kk], s[h2]);
          dp[h2] = mfma32(av, of[kk], dp[h2]);
        }
      }
      if constexpr (FOX) {  // + (cs_q - cs_key) sqrt(d); key h2 * 32 + 8 rb + 4 g + e
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) {
            const f32x4 ck = *(const f32x4*)(&sCS[buf][h2 * 32 + 8 * rb + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e) s[h2][4 * rb + e] += fmaf(-ck[e], sqd, csq);
          }
      }
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(fmaf(s[h2][r], scale_log2, -myl));
          if constexpr (MASK) {
            const int key = k0 + h2 * 32 + d_row(r, g);
            p = (key >= T || myq >= T || (CAUSAL && key > myq)) ? 0.0f : p;
          }
          s[h2][r] = p * (dp[h2][r] - myd);  // dS^T / scale: 1/sqrt(d) is applied to dQ at the end
          if constexpr (FOX) rowacc += s[h2][r];
        }
      bf16x8 db[4];
#pragma unroll
      for (int kc = 0; kc < 4; ++kc)
#pragma unroll
        for (int e = 0; e < 8; ++e) db[kc][e] = (bf16)s[kc >> 1][8 * (kc & 1) + e];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          const int row = 16 * kc + kr, col = dt * 32 + d0;
          const bf16x8 a = cat4(lds_read_tr16(&sK[buf][lds_off<HD>(row, col)]),
                                lds_read_tr16(&sK[buf][lds_off<HD>(row + 8, col)]));
          dqt[dt] = mfma32(a, db[kc], dqt[dt]);
        }
      }
  };
  auto advance = [&](int kt) {
    if (kt + 1 < nkt) {
      sstore((kt & 1) ^ 1);
      if (kt + 2 < nkt) gload((kt + 2) * BN);
    }
    __syncthreads();
  };
  // A wave's unmasked tiles (inside the sequence for its keys and queries and, causal,
  // wholly at or below its queries' diagonal) come first: two loops with one tile body
  // each (a branch between the bodies inside one loop costs registers).  ksplit is
  // wave-uniform and every wave runs nkt steps, so the barriers stay matched.
  const int ksplit = qw + 31 >= T ? 0 : min(min(T / BN, nkt), CAUSAL ? (qw + 1) / BN : nkt);
  int kt = 0;
  for (; kt < ksplit; ++kt) {
    tile(kt, std::false_type{});
    advance(kt);
  }
  for (; kt < nkt; ++kt) {
    if (!(CAUSAL && kt * BN > qw + 31)) tile(kt, std::true_type{});  // some key visible to the wave
    advance(kt);
  }
  if constexpr (FOX) {
    rowacc += __shfl_xor(rowacc, 32);  // the two lane halves hold the query's other keys
    if (g == 0 && myq < T) DCS[bh * T + myq] = (bf16)(rowacc + DCSK[bh * T + myq]);
  }
  if (myq < T) {
    bf16* qrow = dQ + base + (long)myq * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(dqt[dt][rb * 4 + e] * scale);
        *(bf16x4*)(qrow + dt * 32 + 8 * rb + 4 * g) = v;
      }
  }
}

// ---- head_dim 128: two workgroups per CU, tiles by direct global->LDS loads ----------
// The kernels above keep their next tile in registers on its way to LDS and, at 320+
// registers, run one wave per SIMD: each MFMA waits on the LDS read issued just before
// it and the matrix core idles through the softmax.  These variants move the tiles with
// 16-byte DMA loads (global_load_lds_dwordx4, no registers in flight), fit 256 registers
// and run two workgroups (8 waves) per CU, so one wave's softmax and LDS waits overlap the
// other's MFMAs.  Each ring buffer is its own __shared__ array and the loop is unrolled
// over the two, so the compiler's wait for a DMA into one buffer never lands before the
// reads of the other; every wave waits for its own DMA before the barrier that publishes
// the tile.
// dK / dV, head_dim 128: 128 keys per workgroup, 32 per wave as in fa_bwd_dkdv_kernel,
// with K as register B fragments but V read from an LDS copy of the workgroup's 128 x 128
// tile (its fragments would not fit 256 registers beside the dK^T, dV^T accumulators) and
// 32-query tiles of Q and dO (two workgroups' rings and V tiles fit the 160 KB LDS).
// FULL (non-causal, T a multiple of the query tile): no tile needs the mask, and only the
// unmasked body is compiled (with both bodies the non-causal instance spills its K
// fragments).  Keys past the end then get nonzero P and dS in their own columns, which are
// never stored.
template <bool CAUSAL, bool FOX, bool FULL = false>
__global__ __launch_bounds__(256, 2) void fa_bwd_dkdv128_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                                const bf16* __restrict__ V,
                                                                const bf16* __restrict__ dO,
                                                                const float* __restrict__ LSE,
                                                                const float* __restrict__ Dd, bf16* __restrict__ dK,
                                                                bf16* __restrict__ dV, int T, float scale_log2,
                                                                float scale, const bf16* __restrict__ CS,
                                                                float* __restrict__ DCSK, float sqd) {
  constexpr int HD = 128, BKEY = 128, BQ = 32;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  static_assert(!(FULL && (CAUSAL || FOX)), "FULL is the unmasked non-causal instance");
  __shared__ __attribute__((aligned(16))) bf16 sV[BKEY * HD];
  // ring slot b: Q then dO (one array per slot: the compiler's fixed array addresses are
  // not folded into the LDS offset field, so each array costs address registers)
  __shared__ __attribute__((aligned(16))) bf16 sR0[2 * BQ * HD];
  __shared__ __attribute__((aligned(16))) bf16 sR1[2 * BQ * HD];
  __shared__ __attribute__((aligned(16))) float sL0[BQ], sL1[BQ], sD0[BQ], sD1[BQ];
  __shared__ __attribute__((aligned(16))) float sC0[FOX ? BQ : 4], sC1[FOX ? BQ : 4];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  int xb;
  long bh;
  head_block(xb, bh);
  const int kb0 = xb * BKEY;
  const int kw = kb0 + 32 * w;
  const int mykey = kw + li;
  const long base = bh * T * HD;

  // per-head buffer resources: DMA rows past the end read as zeros
  const rsrc_t rQ = make_rsrc(Q + base, (unsigned)T * HD * 2), rdO = make_rsrc(dO + base, (unsigned)T * HD * 2);
  // keys past the end read zero rows of V: they only feed their own dK, dV columns, never stored
  stage_hb<BKEY>(make_rsrc(V + base, (unsigned)T * HD * 2), sV, kb0, wu, l);
  bf16x8 kf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)
    kf[kk] = mykey < T ? *(const bf16x8*)(K + base + (long)mykey * HD + kk * 16 + 8 * g) : bf16x8{};
  f32x16 dkt[NDT], dvt[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dkt[dt] = zero16();
    dvt[dt] = zero16();
  }
  const float csk = FOX && mykey < T ? to_f32(CS[bh * T + mykey]) * sqd : 0.0f;
  float colacc = 0.0f;
  float rl = 0.0f, rd = 0.0f;
  bf16 rc = {};

  // Tile q0 into ring buffer B: Q and dO by DMA, the LSE, D and cs of its queries into
  // registers of the first wave, which publish() converts (LSE to log2 units, +inf past
  // the end) and writes to LDS once the tile's work is done; converting them here would
  // wait for the DMA loads issued before them.
  auto issue = [&](auto bt, int q0) {
    constexpr int B = decltype(bt)::value;
    stage_hb<BQ>(rQ, B ? sR1 : sR0, q0, wu, l);
    stage_hb<BQ>(rdO, (B ? sR1 : sR0) + BQ * HD, q0, wu, l);
    if (tid < BQ) {
      const long q = min(q0 + tid, T - 1);
      rl = LSE[bh * T + q];
      rd = Dd[bh * T + q];
      if constexpr (FOX) rc = CS[bh * T + q];
    }
  };
  auto publish = [&](auto bt, int q0) {
    constexpr int B = decltype(bt)::value;
    wait_vm();
    if (tid < BQ) {
      (B ? sL1 : sL0)[tid] = q0 + tid < T ? rl * LOG2E : INFINITY;
      (B ? sD1 : sD0)[tid] = rd;
      if constexpr (FOX) (B ? sC1 : sC0)[tid] = to_f32(rc);
    }
  };

  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
  const int kr = 4 * (grp >> 1) + (i16 >> 2);
  const int qrow[2] = {hb_row_base(li, g, 0), hb_row_base(li, g, 1)};
  const int vrow[2] = {hb_row_base(li, g, 0) + hb_row_off<BKEY>(0, 32 * w),
                       hb_row_base(li, g, 1) + hb_row_off<BKEY>(0, 32 * w)};
  const int qtr[2] = {hb_tr_base(kr, d0, 0), hb_tr_base(kr, d0, 1)};

  auto subtile = [&](auto bt, int q0, int sub, auto masked) {
    constexpr int B = decltype(bt)::value;
    constexpr bool MASK = decltype(masked)::value;
    const bf16* sQ = B ? sR1 : sR0;
    const bf16* sO = sQ + BQ * HD;
    const float* sL = B ? sL1 : sL0;
    const float* sD = B ? sD1 : sD0;
    const float* sC = B ? sC1 : sC0;
    const int qs = q0 + 32 * sub;
    // The two bodies begin with the same LDS reads; distinct scheduling barriers keep the
    // compiler from hoisting all 24 fragments above the branch (96 live registers, spills).
    __builtin_amdgcn_sched_barrier(MASK ? 1 : 2);
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const int off = qrow[kk & 1] + hb_row_off<BQ>(kk, 32 * sub);
      const bf16x8 vf = *(const bf16x8*)(&sV[vrow[kk & 1] + hb_row_off<BKEY>(kk, 0)]);
      s = mfma32(*(const bf16x8*)(&sQ[off]), kf[kk], s);
      dp = mfma32(*(const bf16x8*)(&sO[off]), vf, dp);
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const f32x4 lv = *(const f32x4*)(&sL[32 * sub + 8 * rb + 4 * g]);
      const f32x4 dv4 = *(const f32x4*)(&sD[32 * sub + 8 * rb + 4 * g]);
      f32x4 cq4 = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (FOX) cq4 = *(const f32x4*)(&sC[32 * sub + 8 * rb + 4 * g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = rb * 4 + e;
        if constexpr (FOX) s[r] += fmaf(cq4[e], sqd, -csk);
        float p = fast_exp2(fmaf(s[r], scale_log2, -lv[e]));
        if constexpr (MASK) {
          const int q = qs + 8 * rb + 4 * g + e;
          p = (q >= T || mykey >= T || (CAUSAL && mykey > q)) ? 0.0f : p;
        }
        s[r] = p;
        dp[r] = p * (dp[r] - dv4[e]);
        if constexpr (FOX) colacc += dp[r];
      }
    }
    bf16x8 pb[2], db[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pb[kc][e] = (bf16)s[8 * kc + e];
        db[kc][e] = (bf16)dp[8 * kc + e];
      }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int o0 = qtr[0] + hb_tr_off<BQ>(dt, kc, 32 * sub);
        const int o1 = qtr[1] + hb_tr_off<BQ>(dt, kc, 32 * sub);
        dvt[dt] = mfma32(cat4(lds_read_tr16(&sO[o0]), lds_read_tr16(&sO[o1])), pb[kc], dvt[dt]);
        dkt[dt] = mfma32(cat4(lds_read_tr16(&sQ[o0]), lds_read_tr16(&sQ[o1])), db[kc], dkt[dt]);
      }
  };
  // FULL: a skip test the compiler cannot resolve (opaque_lo is -1, no tile is skipped).
  // With an unconditional tile body the register allocator spilled 129 registers (the K
  // fragments among them, reloaded inside the loop); with the causal instance's shape of
  // control flow it needs 250 and spills none.
  int opaque_lo = -1;
  if constexpr (FULL) asm volatile("" : "+s"(opaque_lo));
  auto tile = [&](auto bt, int q0) {
#pragma unroll
    for (int sub = 0; sub < BQ / 32; ++sub) {
      const int qs = q0 + 32 * sub;
      if (CAUSAL && qs + 31 < kw) continue;  // every query of the sub-tile precedes this wave's keys
      if (FULL && qs < opaque_lo) continue;
      // masked body on the causal diagonal and in a tile that runs past the end
      if constexpr (FULL) subtile(bt, q0, sub, std::false_type{});
      else if ((CAUSAL && qs < kw + 31) || q0 + BQ > T) subtile(bt, q0, sub, std::true_type{});
      else subtile(bt, q0, sub, std::false_type{});
    }
  };

  const int qstart = CAUSAL ? kb0 : 0;
  const int ntile = qstart < T ? (T - qstart + BQ - 1) / BQ : 0;
  const std::integral_constant<int, 0> b0{};
  const std::integral_constant<int, 1> b1{};
  if (ntile > 0) {
    issue(b0, qstart);
    publish(b0, qstart);
  }
  __syncthreads();
  for (int it = 0; it < ntile; it += 2) {
    const int q0 = qstart + it * BQ;
    if (it + 1 < ntile) issue(b1, q0 + BQ);
    tile(b0, q0);
    if (it + 1 < ntile) publish(b1, q0 + BQ);
    __syncthreads();
    if (it + 1 >= ntile) break;
    if (it + 2 < ntile) issue(b0, q0 + 2 * BQ);
    tile(b1, q0 + BQ);
    if (it + 2 < ntile) publish(b0, q0 + 2 * BQ);
    __syncthreads();
  }
  if constexpr (FOX) {
    colacc += __shfl_xor(colacc, 32);
    if (g == 0 && mykey < T) DCSK[bh * T + mykey] = -colacc;
  }
  if (mykey < T) {
    bf16* krow = dK + base + (long)mykey * HD;
    bf16* vrow = dV + base + (long)mykey * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 a, b;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[e] = (bf16)(dkt[dt][rb * 4 + e] * scale);
          b[e] = (bf16)dvt[dt][rb * 4 + e];
        }
        *(bf16x4*)(krow + dt * 32 + 8 * rb + 4 * g) = a;
        *(bf16x4*)(vrow + dt * 32 + 8 * rb + 4 * g) = b;
      }
  }
}

// dQ, head_dim 128 (same decomposition as fa_bwd_dq_kernel: 128 queries per workgroup,
// 32 per wave with Q and dO as register B fragments, 64-key tiles, each processed as two
// 32-key halves so only one half's S^T / dP^T is live).  OWN_D: the kernel forms
// D = rowsum(dO o O) of its queries itself (O read in dO's fragment layout) and writes it
// to Dw for the dK/dV kernel that runs after it; otherwise it reads D from Dd.
template <bool CAUSAL, bool FOX, bool OWN_D = false>
__global__ __launch_bounds__(256, 2) void fa_bwd_dq128_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                              const bf16* __restrict__ V, const bf16* __restrict__ dO,
                                                              const float* __restrict__ LSE,
                                                              const float* __restrict__ Dd, bf16* __restrict__ dQ,
                                                              int T, float scale_log2, float scale,
                                                              const bf16* __restrict__ CS,
                                                              const float* __restrict__ DCSK, bf16* __restrict__ DCS,
                                                              float sqd, const bf16* __restrict__ O = nullptr,
                                                              float* __restrict__ Dw = nullptr) {
  constexpr int HD = 128, BM = 128, BN = 64;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  __shared__ __attribute__((aligned(16))) bf16 sR0[2 * BN * HD];  // ring slot: K then V
  __shared__ __attribute__((aligned(16))) bf16 sR1[2 * BN * HD];
  __shared__ __attribute__((aligned(16))) float sCS0[FOX ? BN : 4], sCS1[FOX ? BN : 4];

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  int xb;
  long bh;
  head_block(xb, bh);
  const int qb = CAUSAL ? (gridDim.x - 1 - xb) : xb;  // heaviest blocks first
  const int q0 = qb * BM;
  const int qw = q0 + 32 * w;
  const int myq = qw + li;
  const long base = bh * T * HD;
  const rsrc_t rK = make_rsrc(K + base, (unsigned)T * HD * 2), rV = make_rsrc(V + base, (unsigned)T * HD * 2);

  bf16x8 qf[NKK], of[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    qf[kk] = myq < T ? *(const bf16x8*)(Q + base + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
    of[kk] = myq < T ? *(const bf16x8*)(dO + base + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
  }
  const float myl = myq < T ? LSE[bh * T + myq] * LOG2E : 0.0f;
  float myd = 0.0f;
  if constexpr (OWN_D) {  // the lane's 64 dims, then the other half's through the lane 32 apart
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      const bf16x8 ov = myq < T ? *(const bf16x8*)(O + base + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) myd = fmaf((float)of[kk][e], (float)ov[e], myd);
    }
    myd += __shfl_xor(myd, 32);
    if (g == 0 && myq < T) Dw[bh * T + myq] = myd;
  } else {
    myd = myq < T ? Dd[bh * T + myq] : 0.0f;
  }
  const float csq = FOX && myq < T ? to_f32(CS[bh * T + myq]) * sqd : 0.0f;
  float rowacc = 0.0f;
  bf16 rcs = {};
  f32x16 dqt[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dqt[dt] = zero16();

  auto issue = [&](auto bt, int k0) {
    constexpr int B = decltype(bt)::value;
    stage_hb<BN>(rK, B ? sR1 : sR0, k0, wu, l);
    stage_hb<BN>(rV, (B ? sR1 : sR0) + BN * HD, k0, wu, l);
    if constexpr (FOX) {
      if (tid < BN) rcs = CS[bh * T + min(k0 + tid, T - 1)];  // converted by publish()
    }
  };
  auto publish = [&](auto bt) {
    constexpr int B = decltype(bt)::value;
    wait_vm();
    if constexpr (FOX) {
      if (tid < BN) (B ? sCS1 : sCS0)[tid] = to_f32(rcs);
    }
  };

  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
  const int kr = 4 * (grp >> 1) + (i16 >> 2);
  const int krow[2] = {hb_row_base(li, g, 0), hb_row_base(li, g, 1)};
  const int ktr[2] = {hb_tr_base(kr, d0, 0), hb_tr_base(kr, d0, 1)};
  auto tile = [&](auto bt, int kt, auto masked) {
    constexpr int B = decltype(bt)::value;
    constexpr bool MASK = decltype(masked)::value;
    const bf16* sK = B ? sR1 : sR0;
    const bf16* sV = sK + BN * HD;
    const float* sCS = B ? sCS1 : sCS0;
    const int k0 = kt * BN;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      if (MASK && CAUSAL && k0 + 32 * h2 > qw + 31) continue;  // the half is above the wave's diagonal
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const int off = krow[kk & 1] + hb_row_off<BN>(kk, 32 * h2);
        s = mfma32(*(const bf16x8*)(&sK[off]), qf[kk], s);
        dp = mfma32(*(const bf16x8*)(&sV[off]), of[kk], dp);
      }
      if constexpr (FOX) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const f32x4 ck = *(const f32x4*)(&sCS[h2 * 32 + 8 * rb + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) s[4 * rb + e] += fmaf(-ck[e], sqd, csq);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], scale_log2, -myl));
        if constexpr (MASK) {
          const int key = k0 + h2 * 32 + d_row(r, g);
          p = (key >= T || myq >= T || (CAUSAL && key > myq)) ? 0.0f : p;
        }
        s[r] = p * (dp[r] - myd);
        if constexpr (FOX) rowacc += s[r];
      }
      bf16x8 db[2];
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int e = 0; e < 8; ++e) db[kc][e] = (bf16)s[8 * kc + e];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const int o = hb_tr_off<BN>(dt, kc, 32 * h2);
          const bf16x8 a = cat4(lds_read_tr16(&sK[ktr[0] + o]), lds_read_tr16(&sK[ktr[1] + o]));
          dqt[dt] = mfma32(a, db[kc], dqt[dt]);
        }
    }
  };

  const int kend = CAUSAL ? min(T, q0 + BM) : T;
  const int nkt = (kend + BN - 1) / BN;
  // unmasked tiles: inside the sequence for the wave's keys and queries and, causal, wholly
  // at or below its queries' diagonal (wave-uniform)
  const int ksplit = qw + 31 >= T ? 0 : min(min(T / BN, nkt), CAUSAL ? (qw + 1) / BN : nkt);
  auto step = [&](auto bt, int kt) {
    constexpr int B = decltype(bt)::value;
    const std::integral_constant<int, 1 - B> other{};
    if (kt + 1 < nkt) issue(other, (kt + 1) * BN);
    if (kt < ksplit) tile(bt, kt, std::false_type{});
    else if (!(CAUSAL && kt * BN > qw + 31)) tile(bt, kt, std::true_type{});
    if (kt + 1 < nkt) publish(other);
    __syncthreads();
  };
  const std::integral_constant<int, 0> b0{};
  const std::integral_constant<int, 1> b1{};
  issue(b0, 0);
  publish(b0);
  __syncthreads();
  for (int kt = 0; kt < nkt; kt += 2) {
    step(b0, kt);
    if (kt + 1 < nkt) step(b1, kt + 1);
  }
  if constexpr (FOX) {
    rowacc += __shfl_xor(rowacc, 32);
    if (g == 0 && myq < T) DCS[bh * T + myq] = (bf16)(rowacc + DCSK[bh * T + myq]);
  }
  if (myq < T) {
    bf16* qrow = dQ + base + (long)myq * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(dqt[dt][rb * 4 + e] * scale);
        *(bf16x4*)(qrow + dt * 32 + 8 * rb + 4 * g) = v;
      }
  }
}

// ---- generic wave-per-row kernels (float32 / any head_dim) ------------------------
template <typename TT, int DPL>
__global__ __launch_bounds__(256) void fa_bwd_dq_wave_kernel(const TT* __restrict__ Q, const TT* __restrict__ K,
                                                             const TT* __restrict__ V, const TT* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             const float* __restrict__ Dd, TT* __restrict__ dQ, int BH,
                                                             int T, int HD, float scale_log2, float scale,
                                                             int causal, const TT* __restrict__ CS,
                                                             const float* __restrict__ DCSK, TT* __restrict__ DCS,
                                                             float sqd) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (long)BH * T) return;
  const long bh = row / T;
  const int i = (int)(row % T);
  float q[DPL], go[DPL], acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    q[e] = d < HD ? ld(Q, row * HD + d) : 0.0f;
    go[e] = d < HD ? ld(dO, row * HD + d) : 0.0f;
    acc[e] = 0.0f;
  }
  const float lse2 = LSE[row] * LOG2E, Di = Dd[row];
  const float csi = CS != nullptr ? ld(CS, row) * sqd : 0.0f;
  float rowacc = 0.0f;  // FoX: sum over keys of dS
  const int jend = causal ? i + 1 : T;
  for (int j = 0; j < jend; ++j) {
    const long kb = (bh * T + j) * HD;
    float s = 0.0f, dp = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) {
        s = fmaf(q[e], ld(K, kb + d), s);
        dp = fmaf(go[e], ld(V, kb + d), dp);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s += __shfl_xor(s, off);
      dp += __shfl_xor(dp, off);
    }
    if (CS != nullptr) s += fmaf(-ld(CS, bh * T + j), sqd, csi);  // FoX bias (cs_i - cs_j) sqrt(d)
    const float g = fast_exp2(s * scale_log2 - lse2) * (dp - Di);
    rowacc += g;
    const float ds = g * scale;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) acc[e] = fmaf(ds, ld(K, kb + d), acc[e]);
    }
  }
  if (CS != nullptr && lane == 0) st(DCS, row, rowacc + DCSK[row]);
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) st(dQ, row * HD + d, acc[e]);
  }
}

template <typename TT, int DPL>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_wave_kernel(const TT* __restrict__ Q, const TT* __restrict__ K,
                                                               const TT* __restrict__ V, const TT* __restrict__ dO,
                                                               const float* __restrict__ LSE,
                                                               const float* __restrict__ Dd, TT* __restrict__ dK,
                                                               TT* __restrict__ dV, int BH, int T, int HD,
                                                               float scale_log2, float scale, int causal,
                                                               const TT* __restrict__ CS, float* __restrict__ DCSK,
                                                               float sqd) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (long)BH * T) return;
  const long bh = row / T;
  const int j = (int)(row % T);
  float kk[DPL], vv[DPL], ak[DPL], av[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    kk[e] = d < HD ? ld(K, row * HD + d) : 0.0f;
    vv[e] = d < HD ? ld(V, row * HD + d) : 0.0f;
    ak[e] = av[e] = 0.0f;
  }
  const float csj = CS != nullptr ? ld(CS, row) * sqd : 0.0f;
  float colacc = 0.0f;  // FoX: sum over queries of dS
  for (int i = causal ? j : 0; i < T; ++i) {
    const long qb = (bh * T + i) * HD;
    float s = 0.0f, dp = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) {
        s = fmaf(ld(Q, qb + d), kk[e], s);
        dp = fmaf(ld(dO, qb + d), vv[e], dp);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s += __shfl_xor(s, off);
      dp += __shfl_xor(dp, off);
    }
    if (CS != nullptr) s += fmaf(ld(CS, bh * T + i), sqd, -csj);  // FoX bias (cs_i - cs_j) sqrt(d)
    const float p = fast_exp2(s * scale_log2 - LSE[bh * T + i] * LOG2E);
    const float gq = p * (dp - Dd[bh * T + i]);
    colacc += gq;
    const float ds = gq * scale;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) {
        av[e] = fmaf(p, ld(dO, qb + d), av[e]);
        ak[e] = fmaf(ds, ld(Q, qb + d), ak[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) {
      st(dK, row * HD + d, ak[e]);
      st(dV, row * HD + d, av[e]);
    }
  }
  if (CS != nullptr && lane == 0) DCSK[row] = -colacc;
}

// head_dim 128: the two-workgroups-per-CU kernels.  FoX (CS != nullptr, causal, D already
// in Dd): dK/dV first, since dQ adds its key-side d cs.  Otherwise (O given, Dd not yet
// written): dQ first, forming D of its queries into Dd, then dK/dV reading it.
void launch_mfma_bwd128(hipStream_t s, const bf16* Q, const bf16* K, const bf16* V, const bf16* G, const float* lse,
                        float* Dd, bf16* dq, bf16* dk, bf16* dv, int BH, int T, int causal, float scale_log2,
                        float scale, const bf16* CS, float* dcsk, bf16* dcs, float sqd, const bf16* O) {
  const dim3 g1((T + 127) / 128, BH);
  if (CS != nullptr) {
    fa_bwd_dkdv128_kernel<true, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, dk, dv, T, scale_log2, scale, CS, dcsk,
                                                         sqd);
    fa_bwd_dq128_kernel<true, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, dq, T, scale_log2, scale, CS, dcsk, dcs,
                                                       sqd);
  } else if (causal) {
    fa_bwd_dq128_kernel<true, false, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, nullptr, dq, T, scale_log2, scale,
                                                              nullptr, nullptr, nullptr, 0.0f, O, Dd);
    fa_bwd_dkdv128_kernel<true, false><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, dk, dv, T, scale_log2, scale, nullptr,
                                                          nullptr, 0.0f);
  } else {
    fa_bwd_dq128_kernel<false, false, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, nullptr, dq, T, scale_log2, scale,
                                                               nullptr, nullptr, nullptr, 0.0f, O, Dd);
    // non-causal dK/dV: the two-workgroup kernel's unmasked instance when every query tile
    // is whole; otherwise the one-wave-per-SIMD kernel (the two-workgroup variant spills its
    // K fragments when compiled with the masked body but without the causal branches)
    if (T % 32 == 0)
      fa_bwd_dkdv128_kernel<false, false, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, dk, dv, T, scale_log2, scale,
                                                                   nullptr, nullptr, 0.0f);
    else
      fa_bwd_dkdv_kernel<128, false><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, dk, dv, T, scale_log2, scale, nullptr,
                                                        nullptr, 0.0f);
  }
}

template <int HD>
void launch_mfma_bwd(hipStream_t s, const void* q, const void* k, const void* v, const void* go, const float* lse,
                     const float* Dd, void* dq, void* dk, void* dv, int BH, int T, int causal, float scale_log2,
                     float scale, const void* cs = nullptr, float* dcsk = nullptr, void* dcs = nullptr,
                     float sqd = 0.0f) {
  const dim3 g1((T + 127) / 128, BH);
  const bf16 *Q = (const bf16*)q, *K = (const bf16*)k, *V = (const bf16*)v, *G = (const bf16*)go;
  const bf16* CS = (const bf16*)cs;
  if constexpr (HD == 128) {  // FoX only: plain attention goes through launch_mfma_bwd128 with O
    launch_mfma_bwd128(s, Q, K, V, G, lse, (float*)Dd, (bf16*)dq, (bf16*)dk, (bf16*)dv, BH, T, causal, scale_log2,
                       scale, CS, dcsk, (bf16*)dcs, sqd, nullptr);
    return;
  }
  if (cs != nullptr) {  // FoX attention is causal; dK/dV first: dQ adds its key-side d cs
    fa_bwd_dkdv_kernel<HD, true, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, (bf16*)dk, (bf16*)dv, T, scale_log2,
                                                          scale, CS, dcsk, sqd);
    fa_bwd_dq_kernel<HD, true, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, (bf16*)dq, T, scale_log2, scale, CS, dcsk,
                                                        (bf16*)dcs, sqd);
  } else if (causal) {
    fa_bwd_dkdv_kernel<HD, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, (bf16*)dk, (bf16*)dv, T, scale_log2, scale,
                                                    nullptr, nullptr, 0.0f);
    fa_bwd_dq_kernel<HD, true><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, (bf16*)dq, T, scale_log2, scale, nullptr,
                                                  nullptr, nullptr, 0.0f);
  } else {
    fa_bwd_dkdv_kernel<HD, false><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, (bf16*)dk, (bf16*)dv, T, scale_log2, scale,
                                                     nullptr, nullptr, 0.0f);
    fa_bwd_dq_kernel<HD, false><<<g1, 256, 0, s>>>(Q, K, V, G, lse, Dd, (bf16*)dq, T, scale_log2, scale, nullptr,
                                                   nullptr, nullptr, 0.0f);
  }
}

template <typename TT>
void launch_wave_bwd(hipStream_t s, const void* q, const void* k, const void* v, const void* go, const float* lse,
                     const float* Dd, void* dq, void* dk, void* dv, int BH, int T, int HD, int causal,
                     float scale_log2, float scale, const void* cs = nullptr, float* dcsk = nullptr,
                     void* dcs = nullptr, float sqd = 0.0f) {
  const long rows = (long)BH * T;
  const unsigned grid = (unsigned)((rows + 3) / 4);
  const TT *Q = (const TT*)q, *K = (const TT*)k, *V = (const TT*)v, *G = (const TT*)go, *CS = (const TT*)cs;
  // dK/dV first: with FoX the dQ kernel adds the key side of d cs that it writes
#define EDF_FA_WAVE_BWD(DPL)                                                                                        \
  fa_bwd_dkdv_wave_kernel<TT, DPL><<<grid, 256, 0, s>>>(Q, K, V, G, lse, Dd, (TT*)dk, (TT*)dv, BH, T, HD, scale_log2, \
                                                        scale, causal, CS, dcsk, sqd);                               \
  fa_bwd_dq_wave_kernel<TT, DPL><<<grid, 256, 0, s>>>(Q, K, V, G, lse, Dd, (TT*)dq, BH, T, HD, scale_log2, scale,     \
                                                      causal, CS, dcsk, (TT*)dcs, sqd)
  if (HD <= 64) {
    EDF_FA_WAVE_BWD(1);
  } else if (HD <= 128) {
    EDF_FA_WAVE_BWD(2);
  } else {
    EDF_FA_WAVE_BWD(4);
  }
#undef EDF_FA_WAVE_BWD
}

// ---------------------------------------------------------------------------
// host side: argument checks and the launch sequence shared by the entry points
// ---------------------------------------------------------------------------
int fa_bwd_check(const void* q, const void* k, const void* v, const void* out, const void* grad_out, const float* lse,
                 const void* grad_q, const void* grad_k, const void* grad_v, int batch, int num_heads, int seq_len,
                 int head_dim, int dtype) {
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(head_dim <= 256, EDF_ERR_UNSUPPORTED, "head_dim %d > 256 unsupported", head_dim);
  EDF_REQUIRE(q && k && v && out && grad_out && lse && grad_q && grad_k && grad_v, EDF_ERR_INVALID_ARG,
              "null tensor pointer (the forward's lse is required)");
  return EDF_OK;
}

// D = rowsum(dO o O) into Dd [B*H*T] (every entry written before it is read), then the dK/dV
// and dQ kernels; bf16 head_dim 128 forms D inside its dQ kernel.
int fa_bwd_run(hipStream_t s, const void* q, const void* k, const void* v, const void* out, const void* grad_out,
               const float* lse, void* grad_q, void* grad_k, void* grad_v, float* Dd, int batch, int num_heads,
               int seq_len, int head_dim, int causal, int dtype) {
  const int BH = batch * num_heads;
  const long rows = (long)BH * seq_len;
  const unsigned gd = (unsigned)((rows + 15) / 16);
  if (dtype == EDF_BF16 && head_dim == 128) {
    const float scale = 1.0f / sqrtf(128.0f);
    launch_mfma_bwd128(s, (const bf16*)q, (const bf16*)k, (const bf16*)v, (const bf16*)grad_out, lse, Dd,
                       (bf16*)grad_q, (bf16*)grad_k, (bf16*)grad_v, BH, seq_len, causal, scale * LOG2E, scale,
                       nullptr, nullptr, nullptr, 0.0f, (const bf16*)out);
    return check_launch("flash attention backward");
  }
  if (dtype == EDF_BF16)
    fa_bwd_dot_kernel<bf16><<<gd, 256, 0, s>>>((const bf16*)out, (const bf16*)grad_out, Dd, rows, head_dim);
  else
    fa_bwd_dot_kernel<float><<<gd, 256, 0, s>>>((const float*)out, (const float*)grad_out, Dd, rows, head_dim);
  int rc = check_launch("flash attention backward rowsum");
  if (rc) return rc;
  const float scale = 1.0f / sqrtf((float)head_dim);
  const float scale_log2 = scale * LOG2E;
  if (dtype == EDF_BF16 && (head_dim == 32 || head_dim == 64)) {
    if (head_dim == 64)
      launch_mfma_bwd<64>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, causal, scale_log2,
                          scale);
    else
      launch_mfma_bwd<32>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, causal, scale_log2,
                          scale);
  } else if (dtype == EDF_BF16) {
    launch_wave_bwd<bf16>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, head_dim, causal,
                          scale_log2, scale);
  } else {
    launch_wave_bwd<float>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, head_dim, causal,
                           scale_log2, scale);
  }
  return check_launch("flash attention backward");
}

// ---------------------------------------------------------------------------
// Scratch for the allocation-free backward: D lives in a file-scope device array of
// EDF_FA_NOALLOC_SCRATCH_BYTES, of which each GPU holds its own copy (from module load until
// the process ends).  In host code `scratch` names a host-side stand-in, not a device address,
// so kernels get the device address that hipGetSymbolAddress returns, looked up once per
// device with that device current and cached.  Calls on one GPU share its copy: calls that
// overlap in time on one GPU (two streams) race on it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[EDF_FA_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int FA_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[FA_MAX_DEVICES] = {};

int scratch_address(hipStream_t s, float** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return set_error(EDF_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  int dev = cur;
  if (s != nullptr) {  // the stream's device (the kernels run there), not only the current one
    e = hipStreamGetDevice(s, &dev);
    if (e != hipSuccess) return set_error(EDF_ERR_LAUNCH, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
  }
  EDF_REQUIRE(dev >= 0 && dev < FA_MAX_DEVICES, EDF_ERR_UNSUPPORTED, "device %d beyond %d", dev, FA_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return set_error(EDF_ERR_LAUNCH, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess && back != hipSuccess)
        return set_error(EDF_ERR_LAUNCH, "hipSetDevice(%d) failed: %s", cur, hipGetErrorString(back));
    }
    if (e != hipSuccess || p == nullptr)
      return set_error(EDF_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = (float*)p;
  }
  *out = g_scratch_ptr[dev];
  return EDF_OK;
}

}  // namespace
}  // namespace edf

extern "C" {


size_t edf_flash_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim) {
  if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  return (size_t)batch * num_heads * seq_len * sizeof(float);
}

int edf_fused_flash_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* out,
                                       const void* grad_out, const float* lse, void* grad_q, void* grad_k,
                                       void* grad_v, void* workspace, size_t workspace_bytes, int batch,
                                       int num_heads, int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  int rc = fa_bwd_check(q, k, v, out, grad_out, lse, grad_q, grad_k, grad_v, batch, num_heads, seq_len, head_dim,
                        dtype);
  if (rc) return rc;
  const size_t need = edf_flash_attention_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  return fa_bwd_run(as_stream(stream), q, k, v, out, grad_out, lse, grad_q, grad_k, grad_v, (float*)workspace, batch,
                    num_heads, seq_len, head_dim, causal, dtype);
}

int edf_fused_flash_attention_backward_noalloc(void* stream, const void* q, const void* k, const void* v,
                                               const void* out, const void* grad_out, const float* lse,
                                               void* grad_q, void* grad_k, void* grad_v, int batch, int num_heads,
                                               int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  int rc = fa_bwd_check(q, k, v, out, grad_out, lse, grad_q, grad_k, grad_v, batch, num_heads, seq_len, head_dim,
                        dtype);
  if (rc) return rc;
  const size_t need = edf_flash_attention_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(need <= EDF_FA_NOALLOC_SCRATCH_BYTES, EDF_ERR_UNSUPPORTED,
              "batch * heads * seq_len = %zu exceeds the no-alloc scratch (%zu rows, %d MiB)", need / sizeof(float),
              (size_t)EDF_FA_NOALLOC_SCRATCH_BYTES / sizeof(float), (int)(EDF_FA_NOALLOC_SCRATCH_BYTES >> 20));
  hipStream_t s = as_stream(stream);
  float* Dd = nullptr;
  rc = scratch_address(s, &Dd);
  if (rc) return rc;
  return fa_bwd_run(s, q, k, v, out, grad_out, lse, grad_q, grad_k, grad_v, Dd, batch, num_heads, seq_len, head_dim,
                    causal, dtype);
}

size_t edf_fox_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim) {
  if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  const size_t rows = (size_t)batch * num_heads * seq_len;
  return ((rows * sizeof(float) + 255) & ~(size_t)255) + rows * sizeof(float);  // D, then the key side of d cs
}

int edf_fused_fox_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* cs,
                                     const void* out, const void* grad_out, const float* lse, void* grad_q,
                                     void* grad_k, void* grad_v, void* grad_cs, void* workspace,
                                     size_t workspace_bytes, int batch, int num_heads, int seq_len, int head_dim,
                                     int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(head_dim <= 256, EDF_ERR_UNSUPPORTED, "head_dim %d > 256 unsupported", head_dim);
  EDF_REQUIRE(q && k && v && cs && out && grad_out && lse && grad_q && grad_k && grad_v && grad_cs,
              EDF_ERR_INVALID_ARG, "null tensor pointer (the forward's lse is required)");
  const size_t need = edf_fox_attention_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
  const long rows = (long)BH * seq_len;
  float* Dd = (float*)workspace;
  float* dcsk = (float*)((char*)workspace + ((rows * sizeof(float) + 255) & ~(size_t)255));
  const unsigned gd = (unsigned)((rows + 15) / 16);
  if (dtype == EDF_BF16)
    fa_bwd_dot_kernel<bf16><<<gd, 256, 0, s>>>((const bf16*)out, (const bf16*)grad_out, Dd, rows, head_dim);
  else
    fa_bwd_dot_kernel<float><<<gd, 256, 0, s>>>((const float*)out, (const float*)grad_out, Dd, rows, head_dim);
  int rc = check_launch("fox attention backward rowsum");
  if (rc) return rc;
  const float scale = 1.0f / sqrtf((float)head_dim);
  const float scale_log2 = scale * LOG2E;
  const float sqd = sqrtf((float)head_dim);
  if (dtype == EDF_BF16 && (head_dim == 32 || head_dim == 64 || head_dim == 128)) {
    if (head_dim == 128)
      launch_mfma_bwd<128>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, 1, scale_log2, scale,
                           cs, dcsk, grad_cs, sqd);
    else if (head_dim == 64)
      launch_mfma_bwd<64>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, 1, scale_log2, scale,
                          cs, dcsk, grad_cs, sqd);
    else
      launch_mfma_bwd<32>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, 1, scale_log2, scale,
                          cs, dcsk, grad_cs, sqd);
  } else if (dtype == EDF_BF16) {
    launch_wave_bwd<bf16>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, head_dim, 1,
                          scale_log2, scale, cs, dcsk, grad_cs, sqd);
  } else {
    launch_wave_bwd<float>(s, q, k, v, grad_out, lse, Dd, grad_q, grad_k, grad_v, BH, seq_len, head_dim, 1,
                           scale_log2, scale, cs, dcsk, grad_cs, sqd);
  }
  return check_launch("fox attention backward");
}

}  // extern "C"
