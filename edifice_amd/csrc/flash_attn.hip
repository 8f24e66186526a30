// Flash attention forward for gfx950: O = softmax(Q K^T / sqrt(d) [+ causal -inf]) V.
//
// Semantics (reference): lib/edifice/cuda/fused_scan.ex:3476-3508 (flash_attention_fallback),
// native/cuda/fused_flash_attention.cu:52-154; layout [B, H, T, d]; causal keeps keys
// j <= i.  Additionally emits the natural-log row log-sum-exp (float32 [B, H, T]) used
// by the backward.
//
// bf16 path (the performance path), per workgroup of 4 waves and 128 queries:
//   * each wave owns 32 queries; Q^T stays in registers as MFMA B fragments;
//   * K and V tiles of 64 keys are staged in LDS (K row-major, V transposed to
//     [dim][key] so the MFMA A operand of V^T is a contiguous LDS read), rows padded
//     against bank conflicts;
//   * S^T = K Q^T with v_mfma_f32_32x32x16_bf16: every lane owns one query column,
//     so the online-softmax max/sum are lane-local plus one exchange between the two
//     wave halves;
//   * O^T += V^T P^T reuses the S^T result registers directly as the B operand
//     (keys permuted consistently in the V^T reads), so P never goes through LDS;
//   * causal: key tiles above the diagonal are skipped, only diagonal tiles are
//     masked, and query blocks are issued heaviest-first.
// f32 (or odd head_dim) path: one wave per query, lanes over head_dim, for parity.
#include "edf_abi.hpp"
#include "edf_common.hpp"
#include "edf_mfma.hpp"

#include <type_traits>

namespace edf {
namespace {

constexpr float LN2 = 0.6931471805599453f;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// FOX: the forgetting-attention bias cs_q - cs_k (CS [BH][T], cumulative log forget
// gates; reference native/cuda/fused_fox_attention.cu:1-14, fused_scan.ex:3860-3905) is
// added to every score; scores are kept unscaled, so the bias enters as
// (cs_q - cs_k) sqrt(d) (sqd).
template <int HD, bool CAUSAL, bool FOX = false>
__global__ __launch_bounds__(256, 2) void fa_fwd_mfma_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                             const bf16* __restrict__ V, bf16* __restrict__ O,
                                                             float* __restrict__ LSE, int T, float scale_log2,
                                                             const bf16* __restrict__ CS, float sqd) {
  constexpr int BM = 128, BN = 64;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  constexpr int CPR = HD / 8;             // 16-byte chunks per row
  constexpr int CPT = BN * CPR / 256;     // chunks per thread per tile (K and V each)
  static_assert(CPT >= 1 && BN * CPR % 256 == 0, "tile staging");
  __shared__ __attribute__((aligned(16))) bf16 sK[2][lds_tile_elems<HD>(BN)];
  __shared__ __attribute__((aligned(16))) bf16 sV[2][lds_tile_elems<HD>(BN)];
  __shared__ __attribute__((aligned(16))) float sCS[FOX ? 2 : 1][FOX ? BN : 4];  // cs of the tile's keys

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 5, li = l & 31;
  int xb;
  long bh;
  head_block(xb, bh);
  const int qb = CAUSAL ? (gridDim.x - 1 - xb) : xb;  // heaviest blocks first
  const int q0 = qb * BM;
  const int qw = q0 + 32 * w;
  const int myq = qw + li;
  const bf16* Qh = Q + bh * T * HD;
  const bf16* Kh = K + bh * T * HD;
  const bf16* Vh = V + bh * T * HD;

  // Q^T as MFMA B fragments, kept in registers
  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)
    qf[kk] = myq < T ? *(const bf16x8*)(Qh + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = zero16();
  float m = -INFINITY, lsum = 0.0f;  // running max (unscaled score units) and sum

  // K / V tiles: global -> registers one tile ahead, registers -> LDS double buffer
  bf16x8 rk[CPT], rv[CPT];
  float rcs = 0.0f;
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
      // rows past the end are clamped, not branched around: their scores are masked
      const long key = min(k0 + row, T - 1);
      rk[i] = *(const bf16x8*)(Kh + key * HD + col);
      rv[i] = *(const bf16x8*)(Vh + key * HD + col);
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
  const float csq = FOX && myq < T ? to_f32(CS[bh * T + myq]) * sqd : 0.0f;

  const int kend = CAUSAL ? min(T, q0 + BM) : T;
  const int nkt = (kend + BN - 1) / BN;
  gload(0);
  sstore(0);
  if (nkt > 1) gload(BN);
  __syncthreads();
  // One key tile; the masked body selects -inf per score without branching.
  auto tile = [&](int kt, auto masked) {
    constexpr bool MASK = decltype(masked)::value;
    const int k0 = kt * BN, buf = kt & 1;
    const bf16* sk = sK[buf];
    const bf16* sv = sV[buf];
    // S^T = K Q^T: lane owns query column li, rows are keys
    f32x16 s[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      s[h2] = zero16();
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        const bf16x8 a = *(const bf16x8*)(sk + lds_off<HD>(h2 * 32 + li, kk * 16 + 8 * g));
        s[h2] = mfma32(a, qf[kk], s[h2]);
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
    float mx = -INFINITY;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (MASK) {
          const int key = k0 + h2 * 32 + d_row(r, g);
          s[h2][r] = (key >= T || (CAUSAL && key > myq)) ? -INFINITY : s[h2][r];
        }
        mx = fmaxf(mx, s[h2][r]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(m, mx);
    // scale folded into the exponent: p = 2^(s c - m c)
    const float mns = mnew == -INFINITY ? 0.0f : mnew * scale_log2;
    if (__any(mnew > m)) {  // rescale only when some row maximum grew
      const float alpha = fast_exp2(m * scale_log2 - mns);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    }
    m = mnew;
    float rs = 0.0f;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = fast_exp2(fmaf(s[h2][r], scale_log2, -mns));
        s[h2][r] = pv;
        rs += pv;
      }
    }
    lsum += rs + __shfl_xor(rs, 32);

    // P^T straight from the S^T registers: B fragment kc holds keys
    // 16 kc + 4 g + {0..3} and 16 kc + 8 + 4 g + {0..3}
    bf16x8 pf[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int it = 0; it < 8; ++it) pf[kc][it] = (bf16)s[kc >> 1][8 * (kc & 1) + it];

    // O^T += V^T P^T; the V^T A fragment (same key order) comes from two transposed
    // reads of the row-major V tile: lane i of each 16-lane group addresses key row
    // base + i / 4, columns d0 + 4 (i % 4)
    {
      const int grp = l >> 4, i16 = l & 15;
      const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
      const int kr = 4 * (grp >> 1) + (i16 >> 2);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          const int row = 16 * kc + kr, col = dt * 32 + d0;
          const bf16x8 a = cat4(lds_read_tr16(sv + lds_off<HD>(row, col)), lds_read_tr16(sv + lds_off<HD>(row + 8, col)));
          o[dt] = mfma32(a, pf[kc], o[dt]);
        }
      }
    }
  };
  // the next tile into the other LDS buffer, the one after it into registers
  auto advance = [&](int kt) {
    if (kt + 1 < nkt) {
      sstore((kt & 1) ^ 1);
      if (kt + 2 < nkt) gload((kt + 2) * BN);
    }
    __syncthreads();
  };
  // A wave's unmasked tiles (inside the sequence and, causal, wholly at or below its
  // queries' diagonal) come first: two loops with one tile body each (both bodies behind
  // a branch in one loop spilled registers).  ksplit is wave-uniform; every wave runs nkt
  // steps, so the barriers stay matched.
  const int ksplit = min(min(T / BN, nkt), CAUSAL ? (qw + 1) / BN : nkt);
  int kt = 0;
  for (; kt < ksplit; ++kt) {
    tile(kt, std::false_type{});
    advance(kt);
  }
  for (; kt < nkt; ++kt) {
    tile(kt, std::true_type{});
    advance(kt);
  }

  // O goes through the (now free) K tiles, each wave's 32 rows privately, and is written as
  // whole rows: a lane holds one query row, so storing from registers would touch 32 rows
  // per instruction in 16-byte pieces.
  bf16* so = &sK[0][0];
  static_assert(2 * lds_tile_elems<HD>(BN) >= lds_tile_elems<HD>(BM), "O staging");
  const float inv = myq < T ? 1.0f / lsum : 0.0f;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)(o[dt][rb * 4 + e] * inv);
      *(bf16x4*)(so + lds_off<HD>(32 * w + li, dt * 32 + 8 * rb + 4 * g)) = v;
    }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < 32 * CPR / 64; ++i) {
    const int e = l + 64 * i, row = e / CPR, ch = e % CPR;
    if (qw + row < T)
      *(bf16x8*)(O + bh * T * HD + (long)(qw + row) * HD + 8 * ch) = *(const bf16x8*)(so + lds_off<HD>(32 * w + row, 8 * ch));
  }
  if (myq < T && g == 0 && LSE != nullptr) LSE[bh * T + myq] = (m * scale_log2 + __log2f(lsum)) * LN2;
}

// head_dim 128: the same decomposition (128 queries per workgroup, 32 per wave with Q^T as
// register B fragments, 64-key tiles), with K and V moved by 16-byte DMA loads into
// half-row-block LDS tiles (stage_hb: fragment addresses are bases plus immediates, no
// staging registers), and K one tile ahead of V: iteration t issues the MFMAs of S(t + 1) before
// the softmax of S(t), so the matrix core works on the next scores while the VALU turns
// the current ones into P (the two rings stay two-deep: K(t) was consumed in iteration
// t - 1).  Two workgroups per CU.  FULL (non-causal, T a multiple of the key tile): every
// tile is inside the sequence and unmasked, so the masked body is not compiled (with it,
// the non-causal instance spilled 49 registers).
template <bool CAUSAL, bool FOX = false, bool FULL = false>
__global__ __launch_bounds__(256, 2) void fa_fwd128_kernel(const bf16* __restrict__ Q, const bf16* __restrict__ K,
                                                           const bf16* __restrict__ V, bf16* __restrict__ O,
                                                           float* __restrict__ LSE, int T, float scale_log2,
                                                           const bf16* __restrict__ CS, float sqd) {
  constexpr int HD = 128, BM = 128, BN = 64;
  constexpr int NKK = HD / 16, NDT = HD / 32;
  static_assert(!(FULL && (CAUSAL || FOX)), "FULL is the unmasked non-causal instance");
  // Two arrays, X0 = {K buffer 0, V buffer 1} and X1 = {K buffer 1, V buffer 0}: iteration t
  // (parity B) writes only X_B and reads only X_(1-B), and each array's fixed address costs
  // address registers (it is not folded into the LDS offset field).
  __shared__ __attribute__((aligned(16))) bf16 sX0[2 * BN * HD];
  __shared__ __attribute__((aligned(16))) bf16 sX1[2 * BN * HD];
  __shared__ __attribute__((aligned(16))) float sC0[FOX ? BN : 4], sC1[FOX ? BN : 4];  // cs of a K tile's keys

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
  // per-head buffer resources: DMA rows past the end read as zeros (their scores are masked)
  const rsrc_t rK = make_rsrc(K + base, (unsigned)T * HD * 2), rV = make_rsrc(V + base, (unsigned)T * HD * 2);

  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)
    qf[kk] = myq < T ? *(const bf16x8*)(Q + base + (long)myq * HD + kk * 16 + 8 * g) : bf16x8{};
  f32x16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = zero16();
  float m = -INFINITY, lsum = 0.0f;
  const float csq = FOX && myq < T ? to_f32(CS[bh * T + myq]) * sqd : 0.0f;
  bf16 rcs = {};

  const int grp = l >> 4, i16 = l & 15;
  const int d0 = 16 * (grp & 1) + 4 * (i16 & 3);
  const int kr = 4 * (grp >> 1) + (i16 >> 2);
  const int krow[2] = {hb_row_base(li, g, 0), hb_row_base(li, g, 1)};
  const int vtr[2] = {hb_tr_base(kr, d0, 0), hb_tr_base(kr, d0, 1)};

  const int kend = CAUSAL ? min(T, q0 + BM) : T;
  const int nkt = (kend + BN - 1) / BN;
  // unmasked tiles of this wave: inside the sequence and, causal, at or below its diagonal
  const int ksplit = min(min(T / BN, nkt), CAUSAL ? (qw + 1) / BN : nkt);
  auto visible = [&](int t) __attribute__((always_inline)) { return !(CAUSAL && t * BN > qw + 31); };

  auto issue_k = [&](auto bt, int t) __attribute__((always_inline)) {  // K tile t (and its cs) into K buffer B
    constexpr int B = decltype(bt)::value;
    stage_hb<BN>(rK, B ? sX1 : sX0, t * BN, wu, l);
    if constexpr (FOX) {
      if (tid < BN) rcs = CS[bh * T + min(t * BN + tid, T - 1)];  // converted by publish_k()
    }
  };
  auto issue_v = [&](auto bt, int t) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value;
    stage_hb<BN>(rV, (B ? sX0 : sX1) + BN * HD, t * BN, wu, l);
  };
  auto publish_k = [&](auto bt) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value;
    if constexpr (FOX) {
      if (tid < BN) (B ? sC1 : sC0)[tid] = to_f32(rcs);
    }
  };
  // S^T of the K tile in buffer B: lane owns query column li, rows are the tile's keys
  auto scores = [&](auto bt, f32x16* s) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value;
    const bf16* sk = B ? sX1 : sX0;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      s[h2] = zero16();
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk)
        s[h2] = mfma32(*(const bf16x8*)(&sk[krow[kk & 1] + hb_row_off<BN>(kk, 32 * h2)]), qf[kk], s[h2]);
    }
    if constexpr (FOX) {  // + (cs_q - cs_key) sqrt(d); key h2 * 32 + 8 rb + 4 g + e
      const float* sc = B ? sC1 : sC0;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const f32x4 ck = *(const f32x4*)(&sc[h2 * 32 + 8 * rb + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) s[h2][4 * rb + e] += fmaf(-ck[e], sqd, csq);
        }
    }
  };
  f32x16 sc[2], sn[2];  // scores of the current and the next tile
  // Online softmax of tile t's scores, first half: mask, row maximum, rescale of O and the
  // sum when a maximum grew; returns the new maximum in scaled log2 units.
  auto softmax_max = [&](f32x16* s, int t, auto masked) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(masked)::value;
    const int k0 = t * BN;
    float mx = -INFINITY;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (MASK) {
          const int key = k0 + h2 * 32 + d_row(r, g);
          s[h2][r] = (key >= T || (CAUSAL && key > myq)) ? -INFINITY : s[h2][r];
        }
        mx = fmaxf(mx, s[h2][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // The exponentials are taken against a reference maximum m that is moved (and O and
    // the sum rescaled) only when a score exceeds it by more than 2^8: p <= 256 is exact
    // enough in float32 and bf16, and O, the sum and the LSE all refer to the same m.
    if (__any(mx * scale_log2 > m * scale_log2 + 8.0f)) {
      const float mnew = fmaxf(m, mx);
      const float alpha = fast_exp2(m * scale_log2 - (mnew == -INFINITY ? 0.0f : mnew * scale_log2));
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      m = mnew;
    }
    return m == -INFINITY ? 0.0f : m * scale_log2;
  };
  // Second half for elements 2 j, 2 j + 1 of the 32: p = 2^(s c - m c) into the row sum and
  // the bf16 B fragments of P^T (fragment kc holds keys 16 kc + 4 g + {0..3} and
  // 16 kc + 8 + 4 g + {0..3}, the S^T registers' own order).
  // pin: an empty volatile asm takes the pair and the sum, so the compiler cannot sink this
  // arithmetic below the scheduling barrier of the step that issued it.
  auto softmax_pair = [&](f32x16* s, int j, float mns, float& rs, bf16x8* pf, auto pin) __attribute__((always_inline)) {
    const int h2 = j >> 3, r = (2 * j) & 15;
    const float p0 = fast_exp2(fmaf(s[h2][r], scale_log2, -mns));
    const float p1 = fast_exp2(fmaf(s[h2][r + 1], scale_log2, -mns));
    unsigned pk = pack_bf16x2(p0, p1);
    // the row sum of the bf16 P that the MFMA consumes, one dot2 per pair
    rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), bf16x2{(bf16)1.0f, (bf16)1.0f}, rs, false);
    if constexpr (decltype(pin)::value) asm volatile("" : "+v"(pk), "+v"(rs));
    const int kc = 2 * h2 + (r >> 3), it = r & 7;
    const bf16x2 pp = __builtin_bit_cast(bf16x2, pk);
    pf[kc][it] = pp[0];
    pf[kc][it + 1] = pp[1];
  };
  // O^T += V^T P^T with V from buffer B (transposed reads in the P^T key order)
  // (step j: keys 16 (j / 4) .. of dims 32 (j % 4) ..; consecutive MFMAs go to different
  // accumulators, and the transposed V fragments are read three steps ahead)
  auto pv_mma = [&](auto bt, const bf16x8* pf) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value;
    const bf16* sv = (B ? sX0 : sX1) + BN * HD;
    auto vfrag = [&](int j) __attribute__((always_inline)) {
      const int o16 = hb_tr_off<BN>(j & 3, j >> 2, 0);
      return cat4(lds_read_tr16(&sv[vtr[0] + o16]), lds_read_tr16(&sv[vtr[1] + o16]));
    };
    bf16x8 a[3] = {vfrag(0), vfrag(1), vfrag(2)};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      o[j & 3] = mfma32(a[j % 3], pf[j >> 2], o[j & 3]);
      if (j + 3 < 16) a[j % 3] = vfrag(j + 3);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Generic tile: softmax of s, then O with V buffer B.
  auto consume = [&](auto bt, f32x16* s, int t, auto masked) __attribute__((always_inline)) {
    const float mns = softmax_max(s, t, masked);
    float rs = 0.0f;
    bf16x8 pf[4];
#pragma unroll
    for (int j = 0; j < 16; ++j) softmax_pair(s, j, mns, rs, pf, std::false_type{});
    lsum += rs + __shfl_xor(rs, 32);
    pv_mma(bt, pf);
  };
  // Unmasked tile t with a visible successor: the 16 MFMAs of S(t + 1) (K buffer 1 - B, its
  // fragments read four steps ahead) alternate with the exponentials of S(t), two per MFMA,
  // pinned by scheduling barriers so the matrix core and the VALU work at the same time.
  auto fused = [&](auto bt, int t) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value;
    const bf16* sk = B ? sX0 : sX1;  // K(t + 1) is in K buffer 1 - B
    const float mns = softmax_max(sc, t, std::false_type{});
    auto kfrag = [&](int i) __attribute__((always_inline)) {  // step i: keys 32 (i % 2) + li, dims of kk = i / 2
      const int kk = i >> 1, h2 = i & 1;
      return *(const bf16x8*)(&sk[krow[kk & 1] + hb_row_off<BN>(kk, 32 * h2)]);
    };
    bf16x8 fr[4] = {kfrag(0), kfrag(1), kfrag(2), kfrag(3)};
    sn[0] = zero16();
    sn[1] = zero16();
    float rs = 0.0f;
    bf16x8 pf[4];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sn[i & 1] = mfma32(fr[i & 3], qf[i >> 1], sn[i & 1]);
      if (i + 4 < 16) fr[i & 3] = kfrag(i + 4);
      softmax_pair(sc, i, mns, rs, pf, std::true_type{});
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FOX) {  // + (cs_q - cs_key) sqrt(d) for the next tile's scores
      const float* scs = B ? sC0 : sC1;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
          const f32x4 ck = *(const f32x4*)(&scs[h2 * 32 + 8 * rb + 4 * g]);
#pragma unroll
          for (int e = 0; e < 4; ++e) sn[h2][4 * rb + e] += fmaf(-ck[e], sqd, csq);
        }
    }
    lsum += rs + __shfl_xor(rs, 32);
    pv_mma(bt, pf);
  };

  const std::integral_constant<int, 0> b0{};
  const std::integral_constant<int, 1> b1{};
  // prologue: K(0), V(0), K(1) in; S(0); a barrier before iteration 0 reloads K buffer 0
  issue_k(b0, 0);
  issue_v(b0, 0);
  wait_vm();
  publish_k(b0);
  if (nkt > 1) issue_k(b1, 1);
  __syncthreads();  // K(0), its cs and V(0) visible
  if (visible(0)) scores(b0, sc);
  wait_vm();
  if (nkt > 1) publish_k(b1);
  __syncthreads();  // K(1) visible, K buffer 0 free
  // iteration t (buffer parity B = t % 2): K(t + 2) into K buffer B, V(t + 1) into V buffer
  // 1 - B; S(t + 1) from K buffer 1 - B; softmax of S(t) and O with V buffer B
  auto step = [&](auto bt, int t) __attribute__((always_inline)) {
    constexpr int B = decltype(bt)::value;
    const std::integral_constant<int, 1 - B> ot{};
    if (t + 2 < nkt) issue_k(bt, t + 2);
    if (t + 1 < nkt) issue_v(ot, t + 1);
    const bool nvis = t + 1 < nkt && visible(t + 1);
    if constexpr (FULL) {
      if (nvis) fused(bt, t);
      else consume(bt, sc, t, std::false_type{});
    } else if (visible(t)) {
      if (t < ksplit && nvis) {
        fused(bt, t);
      } else {
        if (nvis) scores(ot, sn);
        if (t < ksplit) consume(bt, sc, t, std::false_type{});
        else consume(bt, sc, t, std::true_type{});
      }
    }
    wait_vm();
    if (t + 2 < nkt) publish_k(bt);
    __syncthreads();
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) sc[h2] = sn[h2];
  };
  for (int t = 0; t < nkt; t += 2) {
    step(b0, t);
    if (t + 1 < nkt) step(b1, t + 1);
  }

  // O through the free array X0 (each wave its 32 rows, row-major swizzled), written as
  // whole rows: a lane holds one query row, so storing from registers would touch 32 rows
  // per instruction in 16-byte pieces.
  bf16* so = sX0 + w * 32 * HD;
  const float inv = myq < T ? 1.0f / lsum : 0.0f;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)(o[dt][rb * 4 + e] * inv);
      *(bf16x4*)(so + lds_off<HD>(li, dt * 32 + 8 * rb + 4 * g)) = v;
    }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int i = 0; i < 32 * 16 / 64; ++i) {
    const int e = l + 64 * i, row = e / 16, ch = e % 16;
    if (qw + row < T)
      *(bf16x8*)(O + base + (long)(qw + row) * HD + 8 * ch) = *(const bf16x8*)(so + lds_off<HD>(row, 8 * ch));
  }
  if (myq < T && g == 0 && LSE != nullptr) LSE[bh * T + myq] = (m * scale_log2 + __log2f(lsum)) * LN2;
}

// Generic path: one wave per query row, lanes over head_dim (any dtype, any head_dim <= 256).
template <typename TT, int DPL>
__global__ __launch_bounds__(256) void fa_fwd_wave_kernel(const TT* __restrict__ Q, const TT* __restrict__ K,
                                                          const TT* __restrict__ V, TT* __restrict__ O,
                                                          float* __restrict__ LSE, int BH, int T, int HD,
                                                          float scale_log2, int causal, const TT* __restrict__ CS,
                                                          float sqd) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= BH * T) return;
  const long bh = row / T;
  const int i = row % T;
  float q[DPL], o[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    q[e] = d < HD ? ld(Q, (bh * T + i) * HD + d) : 0.0f;
    o[e] = 0.0f;
  }
  float m = -INFINITY, lsum = 0.0f;
  const float csi = CS != nullptr ? ld(CS, bh * T + i) * sqd : 0.0f;
  const int jend = causal ? i + 1 : T;
  for (int j = 0; j < jend; ++j) {
    const long kb = (bh * T + j) * HD;
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      if (d < HD) s = fmaf(q[e], ld(K, kb + d), s);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (CS != nullptr) s += fmaf(-ld(CS, bh * T + j), sqd, csi);  // FoX bias (cs_i - cs_j) sqrt(d)
    s *= scale_log2;
    const float mnew = fmaxf(m, s);
    const float alpha = fast_exp2(m - mnew);
    const float p = fast_exp2(s - mnew);
    lsum = lsum * alpha + p;
    m = mnew;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      const int d = lane + 64 * e;
      o[e] = o[e] * alpha + (d < HD ? p * ld(V, kb + d) : 0.0f);
    }
  }
  const float inv = 1.0f / lsum;
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = lane + 64 * e;
    if (d < HD) st(O, (bh * T + i) * HD + d, o[e] * inv);
  }
  if (lane == 0 && LSE != nullptr) LSE[bh * T + i] = (m + __log2f(lsum)) * LN2;
}

__global__ void debug_mfma_kernel(const bf16* A, const bf16* B, float* C) {
  const int l = threadIdx.x, g = l >> 5, li = l & 31;
  bf16x8 a, b;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    a[it] = A[li * 16 + 8 * g + it];   // A row-major [32][16]
    b[it] = B[(8 * g + it) * 32 + li]; // B row-major [16][32]
  }
  f32x16 d = mfma32(a, b, zero16());
#pragma unroll
  for (int r = 0; r < 16; ++r) C[d_row(r, g) * 32 + li] = d[r];
}

__global__ void debug_tr16_kernel(const bf16* x, bf16* out) {
  __shared__ __attribute__((aligned(16))) bf16 t[64 * 64];
  const int l = threadIdx.x;
  for (int i = l; i < 64 * 64; i += 64) t[i] = x[i];
  __syncthreads();
  const int grp = l >> 4, i16 = l & 15;
  const int row = 4 * (grp >> 1) + (i16 >> 2), col = 16 * (grp & 1) + 4 * (i16 & 3);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) *(bf16x4*)(out + (l * 2 + rb) * 4) = lds_read_tr16(t + (8 * rb + row) * 64 + col);
}

template <int HD>
void launch_mfma_fwd(hipStream_t s, const void* q, const void* k, const void* v, void* o, float* lse, int BH, int T,
                     int causal, float scale_log2, const void* cs = nullptr, float sqd = 0.0f) {
  const dim3 grid((T + 127) / 128, BH);
  const bf16 *Q = (const bf16*)q, *K = (const bf16*)k, *V = (const bf16*)v, *CS = (const bf16*)cs;
  if constexpr (HD == 128) {
    if (cs != nullptr)  // FoX attention is causal
      fa_fwd128_kernel<true, true><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, CS, sqd);
    else if (causal)
      fa_fwd128_kernel<true><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, nullptr, 0.0f);
    else if (T % 64 == 0)
      fa_fwd128_kernel<false, false, true><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, nullptr, 0.0f);
    else
      fa_fwd128_kernel<false><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, nullptr, 0.0f);
    return;
  }
  if (cs != nullptr)  // FoX attention is causal
    fa_fwd_mfma_kernel<HD, true, true><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, CS, sqd);
  else if (causal)
    fa_fwd_mfma_kernel<HD, true><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, nullptr, 0.0f);
  else
    fa_fwd_mfma_kernel<HD, false><<<grid, 256, 0, s>>>(Q, K, V, (bf16*)o, lse, T, scale_log2, nullptr, 0.0f);
}

template <typename TT>
void launch_wave_fwd(hipStream_t s, const void* q, const void* k, const void* v, void* o, float* lse, int BH, int T,
                     int HD, int causal, float scale_log2, const void* cs = nullptr, float sqd = 0.0f) {
  const long rows = (long)BH * T;
  const unsigned grid = (unsigned)((rows + 3) / 4);
  if (HD <= 64)
    fa_fwd_wave_kernel<TT, 1><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (TT*)o, lse, BH, T, HD,
                                                   scale_log2, causal, (const TT*)cs, sqd);
  else if (HD <= 128)
    fa_fwd_wave_kernel<TT, 2><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (TT*)o, lse, BH, T, HD,
                                                   scale_log2, causal, (const TT*)cs, sqd);
  else
    fa_fwd_wave_kernel<TT, 4><<<grid, 256, 0, s>>>((const TT*)q, (const TT*)k, (const TT*)v, (TT*)o, lse, BH, T, HD,
                                                   scale_log2, causal, (const TT*)cs, sqd);
}

}  // namespace
}  // namespace edf

extern "C" {

int edf_debug_mfma_32x32x16_bf16(void* stream, const void* A, const void* B, float* C) {
  EDF_REQUIRE(A && B && C, EDF_ERR_INVALID_ARG, "null tensor pointer");
  edf::debug_mfma_kernel<<<1, 64, 0, edf::as_stream(stream)>>>((const edf::bf16*)A, (const edf::bf16*)B, C);
  return edf::check_launch("debug mfma");
}

int edf_debug_lds_read_tr16(void* stream, const void* x, void* out) {
  EDF_REQUIRE(x && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  edf::debug_tr16_kernel<<<1, 64, 0, edf::as_stream(stream)>>>((const edf::bf16*)x, (edf::bf16*)out);
  return edf::check_launch("debug lds transposed read");
}

int edf_fused_flash_attention(void* stream, const void* q, const void* k, const void* v, void* out, float* lse,
                              int batch, int num_heads, int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(head_dim <= 256, EDF_ERR_UNSUPPORTED, "head_dim %d > 256 unsupported", head_dim);
  EDF_REQUIRE(q && k && v && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
  const float scale_log2 = LOG2E / sqrtf((float)head_dim);
  if (dtype == EDF_BF16 && (head_dim == 32 || head_dim == 64 || head_dim == 128)) {
    if (head_dim == 128)
      launch_mfma_fwd<128>(s, q, k, v, out, lse, BH, seq_len, causal, scale_log2);
    else if (head_dim == 64)
      launch_mfma_fwd<64>(s, q, k, v, out, lse, BH, seq_len, causal, scale_log2);
    else
      launch_mfma_fwd<32>(s, q, k, v, out, lse, BH, seq_len, causal, scale_log2);
  } else if (dtype == EDF_BF16) {
    launch_wave_fwd<bf16>(s, q, k, v, out, lse, BH, seq_len, head_dim, causal, scale_log2);
  } else {
    launch_wave_fwd<float>(s, q, k, v, out, lse, BH, seq_len, head_dim, causal, scale_log2);
  }
  return check_launch("flash attention");
}

int edf_fused_fox_attention(void* stream, const void* q, const void* k, const void* v, const void* cs, void* out,
                            float* lse, int batch, int num_heads, int seq_len, int head_dim, int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(head_dim <= 256, EDF_ERR_UNSUPPORTED, "head_dim %d > 256 unsupported", head_dim);
  EDF_REQUIRE(q && k && v && cs && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  hipStream_t s = as_stream(stream);
  const int BH = batch * num_heads;
  const float scale_log2 = LOG2E / sqrtf((float)head_dim);
  const float sqd = sqrtf((float)head_dim);
  if (dtype == EDF_BF16 && (head_dim == 32 || head_dim == 64 || head_dim == 128)) {
    if (head_dim == 128)
      launch_mfma_fwd<128>(s, q, k, v, out, lse, BH, seq_len, 1, scale_log2, cs, sqd);
    else if (head_dim == 64)
      launch_mfma_fwd<64>(s, q, k, v, out, lse, BH, seq_len, 1, scale_log2, cs, sqd);
    else
      launch_mfma_fwd<32>(s, q, k, v, out, lse, BH, seq_len, 1, scale_log2, cs, sqd);
  } else if (dtype == EDF_BF16) {
    launch_wave_fwd<bf16>(s, q, k, v, out, lse, BH, seq_len, head_dim, 1, scale_log2, cs, sqd);
  } else {
    launch_wave_fwd<float>(s, q, k, v, out, lse, BH, seq_len, head_dim, 1, scale_log2, cs, sqd);
  }
  return check_launch("fox attention");
}

}  // extern "C"
