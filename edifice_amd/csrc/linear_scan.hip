// MinGRU / MinLSTM and generic linear scans, forward and backward, for gfx950.
//
// Semantics (reference):
//   linear  h_t = a_t h_{t-1} + b_t   (a, b given; Griffin, MEGA, GSS, MambaVision, ...)
//           native/cuda/fused_linear_scan.cu:42-64, fused_scan.ex:171-185, 4429-4443
//           backward fused_linear_scan_backward.cu:42-80, fused_scan.ex:884-910
//           (da = dh h_{t-1}, db = dh, dh0 = a_0 dh_0)
//   MinGRU  h_t = (1 - z_t) h_{t-1} + z_t c_t
//           native/cuda/fused_mingru_scan.cu:38-65, lib/edifice/cuda/fused_scan.ex:516-528
//           backward fused_scan.ex:548-581 (dz = dh (c - h_{t-1}), dc = dh z, dh0)
//   MinLSTM c_t = f'_t c_{t-1} + i'_t c~_t,  f' = f/(f+i+1e-6), i' = i/(f+i+1e-6)
//           native/cuda/fused_minlstm_scan.cu:27,37-68, fused_scan.ex:583-602
//           backward fused_scan.ex:623-677 (quotient rule)
//   Gate-logit variants apply the sigmoid inside the kernel and return the
//   gradient w.r.t. the logits, i.e. the chain rule dz z (1 - z) of
//   fused_scan.ex:474-480 / :505-510 fused into the same pass.
//
// Design (HBM-bound; every input element is read once, every output written once):
//   * one lane per channel, 64 consecutive channels per wave -> each load/store
//     instruction moves one contiguous 128 B (bf16) / 256 B (f32) row segment;
//   * the W waves of a workgroup split time: per macro-step of W*L timesteps,
//     wave w owns L consecutive timesteps held in registers;
//   * each wave folds its L steps into an affine map h -> A h + B, publishes
//     (A, B) in LDS, and after one barrier composes the maps of the earlier waves
//     with the carry of the previous macro-step (a carry-propagating scan over W
//     waves; no second read of the inputs);
//   * backward runs the same scan in reverse time on u_t = a_t (g_t + u_{t+1});
//   * the raw inputs of the next macro-step are loaded into a register ring while the
//     current one is composed and stored; every global access is a raw buffer access
//     whose out-of-range offsets (padding steps, channels past hid) the hardware turns
//     into zero loads and dropped stores, so the steady-state loop has no branch.
#include "edf_abi.hpp"
#include "edf_common.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

namespace edf {
namespace {

constexpr float MINLSTM_EPS = 1.0e-6f;
// Long-sequence geometry (16 waves per workgroup), measured on MI355X at 8x2048x1536:
// timesteps per wave per macro-step (L) and register-ring depth in macro-steps (P).
// Deeper rings (P = 3, 4) were slower for both directions.
constexpr int LIN_LF = 8, LIN_PF = 2;  // forward
constexpr int LIN_LB = 4, LIN_PB = 2;  // backward (five inputs per step)
// two channels per lane (bf16): 8 waves = 16 virtual waves of L steps (more waves spill)
constexpr int LIN2_LF = 8, LIN2_LB = 4, LIN2_W = 8;

enum { OP_MINGRU = 0, OP_MINLSTM = 1, OP_LINEAR = 2 };  // OP_LINEAR: a, b given directly

// Coefficients of step t: h_t = a h_{t-1} + b.
template <int OP, bool LOGITS>
struct Step {
  float a, b;
  EDF_DEVICE void make(float g1, float g2, float c) {
    if (OP == OP_LINEAR) {
      a = g1;
      b = c;
    } else if (OP == OP_MINGRU) {
      const float z = LOGITS ? sigmoid_rcp(g1) : g1;
      a = 1.0f - z;
      b = z * c;
    } else {
      const float f = LOGITS ? sigmoid_rcp(g1) : g1;
      const float i = LOGITS ? sigmoid_rcp(g2) : g2;
      const float r = fast_rcp(f + (i + MINLSTM_EPS));
      a = f * r;
      b = (i * r) * c;
    }
  }
};

// Raw inputs of P macro-steps are kept in a register ring: the slot of macro-step ms is
// refilled with macro-step ms + P as soon as its values are consumed, so P - 1 macro-steps
// of loads are in flight while the barrier, the composition and the stores of the current
// one run.  All global accesses are raw buffer accesses (per-batch resources): steps past
// the sequence and channels past hid use an out-of-range offset, so the loads return 0 and
// the stores are dropped by the hardware, and the loop body has no branch around a memory
// access (which would make the compiler drain the whole ring at the loop head).  The
// macro-step count is padded to a multiple of P with such empty steps.
template <typename T, int OP, bool LOGITS, int L, int W, int P, bool PAD>
__global__ __launch_bounds__(64 * W) void linscan_fwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                             const T* __restrict__ cand, const T* __restrict__ h0,
                                                             T* __restrict__ out, int seq, int hid) {
  typedef typename Bits<T>::type RB;
  constexpr unsigned ES = sizeof(T);
  __shared__ float sA[2][W][64];
  __shared__ float sB[2][W][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool valid = c < hid;
  const long slab = (long)b * seq * hid;
  const unsigned bytes = (unsigned)((long)seq * hid * ES);
  const rsrc_t R1 = make_rsrc(g1 + slab, bytes);
  const rsrc_t R2 = make_rsrc((OP == OP_MINLSTM ? g2 : g1) + slab, bytes);
  const rsrc_t RC = make_rsrc(cand + slab, bytes);
  const rsrc_t RO = make_rsrc(out + slab, bytes);
  // a channel's base offset plus t rows: rows at and past seq lie beyond the resource (the
  // hardware returns 0 / drops the store), channels past hid start out of range
  const unsigned cb = valid ? (unsigned)c * ES : OOB_OFF, rowb = (unsigned)hid * ES;
  auto off = [&](int t) -> unsigned { return cb + (unsigned)t * rowb; };

  RB r1[P][L], r2[P][L], rc[P][L];
  auto fetch = [&](int slot, int ms) {
    const int t0 = (ms * W + w) * L;
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const unsigned o = off(t0 + j);
      r1[slot][j] = bload<T>(R1, o);
      if (OP == OP_MINLSTM) r2[slot][j] = bload<T>(R2, o);
      rc[slot][j] = bload<T>(RC, o);
    }
  };

  float h = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c) : 0.0f;
  const int steps = (seq + W * L - 1) / (W * L);
  const int npad = (steps + P - 1) / P * P;
#pragma unroll
  for (int j = 0; j < P; ++j) fetch(j, j);
  for (int ms0 = 0; ms0 < npad; ms0 += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const int ms = ms0 + u;
      const int t0 = (ms * W + w) * L;
      float a[L], bb[L];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        Step<OP, LOGITS> s;
        s.make(bits_f32(r1[u][j]), OP == OP_MINLSTM ? bits_f32(r2[u][j]) : 0.0f, bits_f32(rc[u][j]));
        const bool ok = !PAD || (valid && t0 + j < seq);  // padding steps are the identity map
        a[j] = ok ? s.a : 1.0f;
        bb[j] = ok ? s.b : 0.0f;
      }
      fetch(u, ms + P);
      float A = 1.0f, B = 0.0f;
#pragma unroll
      for (int j = 0; j < L; ++j) {
        B = fmaf(a[j], B, bb[j]);
        A *= a[j];
      }
      const int buf = ms & 1;
      sA[buf][w][lane] = A;
      sB[buf][w][lane] = B;
      __syncthreads();
      // compose the W wave maps in time order (all 2W LDS reads issued together; a loop
      // over the preceding waves only is a chain of dependent reads and measured slower);
      // this wave starts from the prefix before it
      float x = h, hh = h;
#pragma unroll
      for (int v = 0; v < W; ++v) {
        if (v == w) hh = x;
        x = fmaf(sA[buf][v][lane], x, sB[buf][v][lane]);
      }
      h = x;
#pragma unroll
      for (int j = 0; j < L; ++j) {
        hh = fmaf(a[j], hh, bb[j]);
        bstore<T>(RO, off(t0 + j), hh);
      }
    }
  }
}

// Backward: reverse scan u_t = a_t (g_t + u_{t+1}), dh_t = g_t + u_{t+1}, dh0 = u_0.
// Same register ring and buffer addressing as the forward, walking macro-steps from the
// end of the (padded) sequence.
template <typename T, int OP, bool LOGITS, int L, int W, int P, bool PAD>
__global__ __launch_bounds__(64 * W) void linscan_bwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                             const T* __restrict__ cand, const T* __restrict__ h0,
                                                             const T* __restrict__ fwd, const T* __restrict__ dy,
                                                             T* __restrict__ d1, T* __restrict__ d2,
                                                             T* __restrict__ dcand, T* __restrict__ dh0, int seq,
                                                             int hid) {
  typedef typename Bits<T>::type RB;
  constexpr unsigned ES = sizeof(T);
  __shared__ float sA[2][W][64];
  __shared__ float sB[2][W][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool valid = c < hid;
  const long slab = (long)b * seq * hid;
  const unsigned bytes = (unsigned)((long)seq * hid * ES);
  const rsrc_t R1 = make_rsrc(g1 + slab, bytes);
  const rsrc_t R2 = make_rsrc((OP == OP_MINLSTM ? g2 : g1) + slab, bytes);
  const rsrc_t RC = make_rsrc((OP == OP_LINEAR ? g1 : cand) + slab, bytes);  // b is not needed
  const rsrc_t RH = make_rsrc(fwd + slab, bytes);
  const rsrc_t RY = make_rsrc(dy + slab, bytes);
  const rsrc_t W1 = make_rsrc(d1 + slab, bytes);
  const rsrc_t W2 = make_rsrc((OP == OP_MINLSTM ? d2 : d1) + slab, bytes);
  const rsrc_t WC = make_rsrc(dcand + slab, bytes);
  // a channel's base offset plus t rows: rows at and past seq lie beyond the resource (the
  // hardware returns 0 / drops the store), channels past hid start out of range
  const unsigned cb = valid ? (unsigned)c * ES : OOB_OFF, rowb = (unsigned)hid * ES;
  auto off = [&](int t) -> unsigned { return cb + (unsigned)t * rowb; };
  // h_{t-1}: the forward output one row up; t = 0 reads out of range (0) and takes h0
  // h_{t-1}: t = 0 wraps below zero, out of range (0), and takes h0
  auto offp = [&](int t) -> unsigned { return cb + (unsigned)(t - 1) * rowb; };
  const float h0v = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c) : 0.0f;

  const int steps = (seq + W * L - 1) / (W * L);
  const int npad = (steps + P - 1) / P * P;
  const int tpad = npad * W * L;
  // wave 0 owns the latest L timesteps of each macro-step
  auto first_t = [&](int ms) { return tpad - (ms + 1) * W * L + (W - 1 - w) * L; };
  RB r1[P][L], r2[P][L], rc[P][L], rh[P][L], ry[P][L];
  auto fetch = [&](int slot, int ms) {
    const int t0 = first_t(ms);
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const unsigned o = off(t0 + j);
      r1[slot][j] = bload<T>(R1, o);
      if (OP == OP_MINLSTM) r2[slot][j] = bload<T>(R2, o);
      if (OP != OP_LINEAR) rc[slot][j] = bload<T>(RC, o);
      rh[slot][j] = bload<T>(RH, offp(t0 + j));
      ry[slot][j] = bload<T>(RY, o);
    }
  };

  float u = 0.0f;  // u_{t+1} entering the macro-step from the right
#pragma unroll
  for (int j = 0; j < P; ++j) fetch(j, j);
  for (int ms0 = 0; ms0 < npad; ms0 += P) {
#pragma unroll
    for (int sl = 0; sl < P; ++sl) {
      const int ms = ms0 + sl;
      const int t0 = first_t(ms);
      // Per step only the decay a, the input gradient g and the coefficients that map
      // dh_t to each output gradient are kept; the ring slot is refilled right after.
      //   linear:  da = dh h_{t-1},  db = dh
      //   MinGRU:  dz = dh (c - h_{t-1}) [z (1 - z)],  dc = dh z
      //   MinLSTM: df = dh (h_{t-1} (i + eps) - c i) / s^2 [f (1 - f)],
      //            di = dh (c (f + eps) - h_{t-1} f) / s^2 [i (1 - i)],  dc = dh i / s
      float a[L], gy[L], k1[L], k2[L], kc[L];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const int t = t0 + j;
        const bool ok = !PAD || (valid && t < seq);
        const float x1 = bits_f32(r1[sl][j]);
        const float x2 = OP == OP_MINLSTM ? bits_f32(r2[sl][j]) : 0.0f;
        const float cv = OP == OP_LINEAR ? 0.0f : bits_f32(rc[sl][j]);
        const float hp = t > 0 ? bits_f32(rh[sl][j]) : h0v;
        gy[j] = bits_f32(ry[sl][j]);  // 0 outside the sequence
        if (OP == OP_LINEAR) {
          a[j] = ok ? x1 : 1.0f;
          k1[j] = hp;
          k2[j] = 0.0f;
          kc[j] = 1.0f;
        } else if (OP == OP_MINGRU) {
          const float z = LOGITS ? sigmoid_rcp(x1) : x1;
          a[j] = ok ? 1.0f - z : 1.0f;  // padding steps are the identity map
          k1[j] = LOGITS ? (cv - hp) * (z * (1.0f - z)) : cv - hp;
          k2[j] = 0.0f;
          kc[j] = z;
        } else {
          const float f = LOGITS ? sigmoid_rcp(x1) : x1;
          const float i = LOGITS ? sigmoid_rcp(x2) : x2;
          const float r = fast_rcp(f + (i + MINLSTM_EPS));
          const float r2 = r * r;
          a[j] = ok ? f * r : 1.0f;
          float c1 = (hp * (i + MINLSTM_EPS) - cv * i) * r2;
          float c2 = (cv * (f + MINLSTM_EPS) - hp * f) * r2;
          if (LOGITS) {
            c1 *= f * (1.0f - f);
            c2 *= i * (1.0f - i);
          }
          k1[j] = c1;
          k2[j] = c2;
          kc[j] = i * r;
        }
      }
      fetch(sl, ms + P);
      float A = 1.0f, B = 0.0f;
#pragma unroll
      for (int j = L - 1; j >= 0; --j) {
        B = a[j] * (gy[j] + B);
        A *= a[j];
      }
      const int buf = ms & 1;
      sA[buf][w][lane] = A;
      sB[buf][w][lane] = B;
      __syncthreads();
      float x = u, uin = u;
#pragma unroll
      for (int v = 0; v < W; ++v) {
        if (v == w) uin = x;
        x = fmaf(sA[buf][v][lane], x, sB[buf][v][lane]);
      }
      u = x;
#pragma unroll
      for (int j = L - 1; j >= 0; --j) {
        const unsigned o = off(t0 + j);
        const float dh = gy[j] + uin;
        uin = a[j] * dh;
        bstore<T>(W1, o, dh * k1[j]);
        if (OP == OP_MINLSTM) bstore<T>(W2, o, dh * k2[j]);
        bstore<T>(WC, o, dh * kc[j]);
      }
    }
  }
  if (valid && w == 0 && dh0 != nullptr) st(dh0, (long)b * hid + c, u);
}

// ---------------------------------------------------------------------------------
// Two channels per lane (bf16, even hidden sizes): each access moves a bf16 pair (4 bytes
// per lane, 256 bytes per wave instruction instead of 128; for float32 the same layout with
// 8-byte pairs measured no faster than one channel per lane), and each
// wave is two 32-lane "virtual waves" (lanes 0-31 and 32-63) that own consecutive time
// segments of L steps, so the 64-channel tile keeps its 2W segments per macro-step.  The
// lower half's affine maps reach the upper half through v_permlane32_swap (VALU); the
// upper half forms the wave's map, the waves' maps are composed through LDS as above.
// ---------------------------------------------------------------------------------
template <typename T> struct Pair;
template <> struct Pair<bf16> {
  typedef unsigned type;
  static EDF_DEVICE type load(rsrc_t r, unsigned off) { return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0); }
  static EDF_DEVICE float lo(type v) { return __builtin_bit_cast(float, v << 16); }
  static EDF_DEVICE float hi(type v) { return __builtin_bit_cast(float, v & 0xffff0000u); }
  static EDF_DEVICE void store(rsrc_t r, unsigned off, float a, float b) {
    const unsigned v = (unsigned)__builtin_bit_cast(unsigned short, (bf16)a) |
                       ((unsigned)__builtin_bit_cast(unsigned short, (bf16)b) << 16);
    __builtin_amdgcn_raw_buffer_store_b32(v, r, (int)off, 0, 0);
  }
};

// Value of x held by lane l - 32, delivered to lanes 32..63 (lanes 0..31 get y's upper
// half, unused).  The second operand must be a different register from the first.
EDF_DEVICE float from_lower(float y, float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, y), __builtin_bit_cast(unsigned, x),
                                                  false, false);
  return __builtin_bit_cast(float, s[0]);
}

template <typename T, int OP, bool LOGITS, int L, int W, int P, bool PAD>
__global__ __launch_bounds__(64 * W) void linscan2_fwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                              const T* __restrict__ cand, const T* __restrict__ h0,
                                                              T* __restrict__ out, int seq, int hid) {
  typedef Pair<T> PR;
  typedef typename PR::type PB;
  constexpr unsigned ES = sizeof(T);
  __shared__ float sA[2][W][64];
  __shared__ float sB[2][W][64];
  const int lane = threadIdx.x & 63, pi = lane & 31, hf = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int vw = 2 * w + hf;  // virtual wave: time-segment index within a macro-step
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + 2 * pi;  // the lane's channels c, c + 1 (hid is even)
  const bool valid = c < hid;
  const long slab = (long)b * seq * hid;
  const unsigned bytes = (unsigned)((long)seq * hid * ES);
  const rsrc_t R1 = make_rsrc(g1 + slab, bytes);
  const rsrc_t R2 = make_rsrc((OP == OP_MINLSTM ? g2 : g1) + slab, bytes);
  const rsrc_t RC = make_rsrc(cand + slab, bytes);
  const rsrc_t RO = make_rsrc(out + slab, bytes);
  // a channel's base offset plus t rows: rows at and past seq lie beyond the resource (the
  // hardware returns 0 / drops the store), channels past hid start out of range
  const unsigned cb = valid ? (unsigned)c * ES : OOB_OFF, rowb = (unsigned)hid * ES;
  auto off = [&](int t) -> unsigned { return cb + (unsigned)t * rowb; };

  PB r1[P][L], r2[P][L], rc[P][L];
  auto fetch = [&](int slot, int ms) {
    const int t0 = (ms * 2 * W + vw) * L;
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const unsigned o = off(t0 + j);
      r1[slot][j] = PR::load(R1, o);
      if (OP == OP_MINLSTM) r2[slot][j] = PR::load(R2, o);
      rc[slot][j] = PR::load(RC, o);
    }
  };

  float h[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) h[k] = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c + k) : 0.0f;
  const int steps = (seq + 2 * W * L - 1) / (2 * W * L);
  const int npad = (steps + P - 1) / P * P;
#pragma unroll
  for (int j = 0; j < P; ++j) fetch(j, j);
  for (int ms0 = 0; ms0 < npad; ms0 += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const int ms = ms0 + u;
      const int t0 = (ms * 2 * W + vw) * L;
      float a[L][2], bb[L][2];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const bool ok = !PAD || (valid && t0 + j < seq);  // padding steps are the identity map
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          Step<OP, LOGITS> st;
          const float x1 = k ? PR::hi(r1[u][j]) : PR::lo(r1[u][j]);
          const float x2 = OP == OP_MINLSTM ? (k ? PR::hi(r2[u][j]) : PR::lo(r2[u][j])) : 0.0f;
          const float xc = k ? PR::hi(rc[u][j]) : PR::lo(rc[u][j]);
          st.make(x1, x2, xc);
          a[j][k] = ok ? st.a : 1.0f;
          bb[j][k] = ok ? st.b : 0.0f;
        }
      }
      fetch(u, ms + P);
      float A[2], B[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        A[k] = 1.0f;
        B[k] = 0.0f;
#pragma unroll
        for (int j = 0; j < L; ++j) {
          B[k] = fmaf(a[j][k], B[k], bb[j][k]);
          A[k] *= a[j][k];
        }
      }
      // the lower half's maps (the earlier segment) in the upper half's lanes
      float Al[2], Bl[2];
      Al[0] = from_lower(A[1], A[0]);
      Al[1] = from_lower(A[0], A[1]);
      Bl[0] = from_lower(B[1], B[0]);
      Bl[1] = from_lower(B[0], B[1]);
      const int buf = ms & 1;
      if (hf) {  // the wave's map: upper segment after lower segment
        *reinterpret_cast<float2*>(&sA[buf][w][2 * pi]) = make_float2(A[0] * Al[0], A[1] * Al[1]);
        *reinterpret_cast<float2*>(&sB[buf][w][2 * pi]) = make_float2(fmaf(A[0], Bl[0], B[0]), fmaf(A[1], Bl[1], B[1]));
      }
      __syncthreads();
      float x[2] = {h[0], h[1]}, hin[2] = {h[0], h[1]};
#pragma unroll
      for (int v = 0; v < W; ++v) {
        if (v == w) {
          hin[0] = x[0];
          hin[1] = x[1];
        }
        const float2 av = *reinterpret_cast<const float2*>(&sA[buf][v][2 * pi]);
        const float2 bv = *reinterpret_cast<const float2*>(&sB[buf][v][2 * pi]);
        x[0] = fmaf(av.x, x[0], bv.x);
        x[1] = fmaf(av.y, x[1], bv.y);
      }
      h[0] = x[0];
      h[1] = x[1];
      float hh[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) hh[k] = hf ? fmaf(Al[k], hin[k], Bl[k]) : hin[k];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        hh[0] = fmaf(a[j][0], hh[0], bb[j][0]);
        hh[1] = fmaf(a[j][1], hh[1], bb[j][1]);
        PR::store(RO, off(t0 + j), hh[0], hh[1]);
      }
    }
  }
}

// Backward with the same layout, walking macro-steps from the end of the padded sequence;
// virtual wave 0 (the lower half of wave 0) owns the latest segment of each macro-step.
template <typename T, int OP, bool LOGITS, int L, int W, int P, bool PAD>
__global__ __launch_bounds__(64 * W) void linscan2_bwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                              const T* __restrict__ cand, const T* __restrict__ h0,
                                                              const T* __restrict__ fwd, const T* __restrict__ dy,
                                                              T* __restrict__ d1, T* __restrict__ d2,
                                                              T* __restrict__ dcand, T* __restrict__ dh0, int seq,
                                                              int hid) {
  typedef Pair<T> PR;
  typedef typename PR::type PB;
  constexpr unsigned ES = sizeof(T);
  __shared__ float sA[2][W][64];
  __shared__ float sB[2][W][64];
  const int lane = threadIdx.x & 63, pi = lane & 31, hf = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int vw = 2 * w + hf;
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + 2 * pi;
  const bool valid = c < hid;
  const long slab = (long)b * seq * hid;
  const unsigned bytes = (unsigned)((long)seq * hid * ES);
  const rsrc_t R1 = make_rsrc(g1 + slab, bytes);
  const rsrc_t R2 = make_rsrc((OP == OP_MINLSTM ? g2 : g1) + slab, bytes);
  const rsrc_t RC = make_rsrc((OP == OP_LINEAR ? g1 : cand) + slab, bytes);  // b is not needed
  const rsrc_t RH = make_rsrc(fwd + slab, bytes);
  const rsrc_t RY = make_rsrc(dy + slab, bytes);
  const rsrc_t W1 = make_rsrc(d1 + slab, bytes);
  const rsrc_t W2 = make_rsrc((OP == OP_MINLSTM ? d2 : d1) + slab, bytes);
  const rsrc_t WC = make_rsrc(dcand + slab, bytes);
  // a channel's base offset plus t rows: rows at and past seq lie beyond the resource (the
  // hardware returns 0 / drops the store), channels past hid start out of range
  const unsigned cb = valid ? (unsigned)c * ES : OOB_OFF, rowb = (unsigned)hid * ES;
  auto off = [&](int t) -> unsigned { return cb + (unsigned)t * rowb; };
  // h_{t-1}: t = 0 wraps below zero, out of range (0), and takes h0
  auto offp = [&](int t) -> unsigned { return cb + (unsigned)(t - 1) * rowb; };
  float h0v[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) h0v[k] = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c + k) : 0.0f;

  const int steps = (seq + 2 * W * L - 1) / (2 * W * L);
  const int npad = (steps + P - 1) / P * P;
  const int tpad = npad * 2 * W * L;
  auto first_t = [&](int ms) { return tpad - (ms + 1) * 2 * W * L + (2 * W - 1 - vw) * L; };
  PB r1[P][L], r2[P][L], rc[P][L], rh[P][L], ry[P][L];
  auto fetch = [&](int slot, int ms) {
    const int t0 = first_t(ms);
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const unsigned o = off(t0 + j);
      r1[slot][j] = PR::load(R1, o);
      if (OP == OP_MINLSTM) r2[slot][j] = PR::load(R2, o);
      if (OP != OP_LINEAR) rc[slot][j] = PR::load(RC, o);
      rh[slot][j] = PR::load(RH, offp(t0 + j));
      ry[slot][j] = PR::load(RY, o);
    }
  };

  float u[2] = {0.0f, 0.0f};  // u_{t+1} entering the macro-step from the right
#pragma unroll
  for (int j = 0; j < P; ++j) fetch(j, j);
  for (int ms0 = 0; ms0 < npad; ms0 += P) {
#pragma unroll
    for (int sl = 0; sl < P; ++sl) {
      const int ms = ms0 + sl;
      const int t0 = first_t(ms);
      // per step and channel: decay a, input gradient g and the dh -> output coefficients
      float a[L][2], gy[L][2], k1[L][2], k2[L][2], kc[L][2];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const int t = t0 + j;
        const bool ok = !PAD || (valid && t < seq);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const float x1 = k ? PR::hi(r1[sl][j]) : PR::lo(r1[sl][j]);
          const float x2 = OP == OP_MINLSTM ? (k ? PR::hi(r2[sl][j]) : PR::lo(r2[sl][j])) : 0.0f;
          const float cv = OP == OP_LINEAR ? 0.0f : (k ? PR::hi(rc[sl][j]) : PR::lo(rc[sl][j]));
          const float hp = t > 0 ? (k ? PR::hi(rh[sl][j]) : PR::lo(rh[sl][j])) : h0v[k];
          gy[j][k] = k ? PR::hi(ry[sl][j]) : PR::lo(ry[sl][j]);  // 0 outside the sequence
          if (OP == OP_LINEAR) {
            a[j][k] = ok ? x1 : 1.0f;
            k1[j][k] = hp;
            k2[j][k] = 0.0f;
            kc[j][k] = 1.0f;
          } else if (OP == OP_MINGRU) {
            const float z = LOGITS ? sigmoid_rcp(x1) : x1;
            a[j][k] = ok ? 1.0f - z : 1.0f;
            k1[j][k] = LOGITS ? (cv - hp) * (z * (1.0f - z)) : cv - hp;
            k2[j][k] = 0.0f;
            kc[j][k] = z;
          } else {
            const float f = LOGITS ? sigmoid_rcp(x1) : x1;
            const float i = LOGITS ? sigmoid_rcp(x2) : x2;
            const float r = fast_rcp(f + (i + MINLSTM_EPS));
            const float r2v = r * r;
            a[j][k] = ok ? f * r : 1.0f;
            float c1 = (hp * (i + MINLSTM_EPS) - cv * i) * r2v;
            float c2 = (cv * (f + MINLSTM_EPS) - hp * f) * r2v;
            if (LOGITS) {
              c1 *= f * (1.0f - f);
              c2 *= i * (1.0f - i);
            }
            k1[j][k] = c1;
            k2[j][k] = c2;
            kc[j][k] = i * r;
          }
        }
      }
      fetch(sl, ms + P);
      float A[2], B[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        A[k] = 1.0f;
        B[k] = 0.0f;
#pragma unroll
        for (int j = L - 1; j >= 0; --j) {
          B[k] = a[j][k] * (gy[j][k] + B[k]);
          A[k] *= a[j][k];
        }
      }
      float Al[2], Bl[2];
      Al[0] = from_lower(A[1], A[0]);
      Al[1] = from_lower(A[0], A[1]);
      Bl[0] = from_lower(B[1], B[0]);
      Bl[1] = from_lower(B[0], B[1]);
      const int buf = ms & 1;
      if (hf) {
        *reinterpret_cast<float2*>(&sA[buf][w][2 * pi]) = make_float2(A[0] * Al[0], A[1] * Al[1]);
        *reinterpret_cast<float2*>(&sB[buf][w][2 * pi]) = make_float2(fmaf(A[0], Bl[0], B[0]), fmaf(A[1], Bl[1], B[1]));
      }
      __syncthreads();
      float x[2] = {u[0], u[1]}, uin[2] = {u[0], u[1]};
#pragma unroll
      for (int v = 0; v < W; ++v) {
        if (v == w) {
          uin[0] = x[0];
          uin[1] = x[1];
        }
        const float2 av = *reinterpret_cast<const float2*>(&sA[buf][v][2 * pi]);
        const float2 bv = *reinterpret_cast<const float2*>(&sB[buf][v][2 * pi]);
        x[0] = fmaf(av.x, x[0], bv.x);
        x[1] = fmaf(av.y, x[1], bv.y);
      }
      u[0] = x[0];
      u[1] = x[1];
      float uu[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) uu[k] = hf ? fmaf(Al[k], uin[k], Bl[k]) : uin[k];
#pragma unroll
      for (int j = L - 1; j >= 0; --j) {
        const unsigned o = off(t0 + j);
        float dh[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          dh[k] = gy[j][k] + uu[k];
          uu[k] = a[j][k] * dh[k];
        }
        PR::store(W1, o, dh[0] * k1[j][0], dh[1] * k1[j][1]);
        if (OP == OP_MINLSTM) PR::store(W2, o, dh[0] * k2[j][0], dh[1] * k2[j][1]);
        PR::store(WC, o, dh[0] * kc[j][0], dh[1] * kc[j][1]);
      }
    }
  }
  if (valid && w == 0 && hf == 0 && dh0 != nullptr) {
    st(dh0, (long)b * hid + c, u[0]);
    st(dh0, (long)b * hid + c + 1, u[1]);
  }
}

// ---------------------------------------------------------------------------------
// Look-back scan (long sequences): the sequence is split into parts of SR = 16 R steps, one
// workgroup per (batch row, 64-lane channel tile, part), so that a bf16 tile of 128 channels
// (two per lane) or an f32 tile of 64 is read as whole 256-byte row pieces by 16 waves x
// (parts) workgroups.  A copy kernel of the bandwidth row's shape reads and writes at
// 36 us with the one-workgroup-per-tile layout above and at 29.6 us with 256-byte pieces
// over eight parts; the parts need the carry of the steps before them.
//
// Each workgroup loads its rows (R per wave) into registers, folds them into per-wave affine
// maps, and its first wave composes them into the part's map (A, B) and publishes it.  The
// part's carry is h0 taken through the maps of all earlier parts of its tile: its waves fetch
// those maps together (wave v parts v, v + 16, ...), so the wait is for the earlier parts to
// fold their own rows, not a chain of carries passed from part to part.
//
// Published values are 64-bit words {call epoch, f32 bits} written and read as device-scope
// atomics (coherent across the XCDs' separate L2 caches); a word counts only when its epoch
// is this call's, so words of earlier calls or of a call running at the same time on another
// stream are never taken for this one's.  A wave that polls LB_SPIN times without finding a
// part's words (overwritten by such a concurrent call, or a part not yet running) folds that
// part's map from its rows itself: every workgroup finishes, whatever the dispatch order.
// EDF_LIN_LOOKBACK_SPIN sets the poll limit (0 folds every map not published at the first
// look, which the tests use to run that path).  Calls being captured into a graph use the
// kernels above (a replay would repeat the captured epoch).
// ---------------------------------------------------------------------------------
constexpr int LB_W = 16;                // waves per workgroup
constexpr int LB_R = 8;                 // steps per wave: parts of 128 steps (768 workgroups at
                                        // the bandwidth row in bf16; two per CU fit)
constexpr int LB_SPIN = 1 << 12;        // default polls of a part's words before folding them here
constexpr int LB_MAXP = 32;             // parts per sequence
constexpr size_t LB_WORDS = 1u << 20;   // published words per device (8 MiB)
static __device__ __align__(256) unsigned long long lb_flags[LB_WORDS];

EDF_DEVICE void lb_put(unsigned long long* p, unsigned epoch, float v) {
  const unsigned long long x = ((unsigned long long)epoch << 32) | __builtin_bit_cast(unsigned, v);
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
EDF_DEVICE bool lb_get(unsigned long long* p, unsigned epoch, float& v) {
  const unsigned long long x = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v = __builtin_bit_cast(float, (unsigned)x);
  return (unsigned)(x >> 32) == epoch;
}

// 4 bytes per lane per row: a bf16 pair (two channels) or one f32 channel
template <typename T> struct Lane4;
template <> struct Lane4<bf16> {
  static constexpr int C = 2;
  static EDF_DEVICE unsigned load(rsrc_t r, unsigned off) { return Pair<bf16>::load(r, off); }
  static EDF_DEVICE float get(unsigned v, int k) { return k ? Pair<bf16>::hi(v) : Pair<bf16>::lo(v); }
  static EDF_DEVICE void store(rsrc_t r, unsigned off, const float* x) { Pair<bf16>::store(r, off, x[0], x[1]); }
};
template <> struct Lane4<float> {
  static constexpr int C = 1;
  static EDF_DEVICE unsigned load(rsrc_t r, unsigned off) { return bload<float>(r, off); }
  static EDF_DEVICE float get(unsigned v, int) { return bits_f32(v); }
  static EDF_DEVICE unsigned pack(float x0, float) { return __builtin_bit_cast(unsigned, x0); }
  static EDF_DEVICE void store(rsrc_t r, unsigned off, const float* x) { bstore<float>(r, off, x[0]); }
};

// flags: [part][batch row x tile][A | B][channel of the lane][lane]
template <typename T, int OP, bool LOGITS, int R>
__global__ __launch_bounds__(64 * LB_W) void linscan_lb_fwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                                   const T* __restrict__ cand, const T* __restrict__ h0,
                                                                   T* __restrict__ out, int seq, int hid, int ntile,
                                                                   unsigned long long* __restrict__ flags,
                                                                   unsigned epoch, int spin_limit) {
  typedef Lane4<T> LN;
  constexpr int W = LB_W, C = LN::C, SR = W * R;
  constexpr unsigned ES = sizeof(T);
  __shared__ float sA[W][C][64];
  __shared__ float sB[W][C][64];
  __shared__ float sH[C][64];
  __shared__ float sPA[LB_MAXP][C][64];  // the earlier parts' maps
  __shared__ float sPB[LB_MAXP][C][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bt = blockIdx.x, nbt = gridDim.x, part = blockIdx.y, nparts = gridDim.y;
  const int b = bt / ntile, tile = bt % ntile;
  const int c = (tile * 64 + lane) * C;  // the lane's first channel (hid is a multiple of C)
  const bool valid = c < hid;
  const long slab = (long)b * seq * hid;
  const unsigned bytes = (unsigned)((long)seq * hid * ES);
  const rsrc_t R1 = make_rsrc(g1 + slab, bytes);
  const rsrc_t R2 = make_rsrc((OP == OP_MINLSTM ? g2 : g1) + slab, bytes);
  const rsrc_t RC = make_rsrc(cand + slab, bytes);
  const rsrc_t RO = make_rsrc(out + slab, bytes);
  const unsigned cb = valid ? (unsigned)c * ES : OOB_OFF, rowb = (unsigned)hid * ES;
  auto off = [&](int t) -> unsigned { return cb + (unsigned)t * rowb; };
  // gate logits -> gates, in place (f32: exactly; the gated bf16 forwards do not run here), so
  // that both passes over the rows and a fold of another part's rows use one sigmoid per gate
  static_assert(!LOGITS || std::is_same<T, float>::value, "gated forwards of bf16 pairs use the per-tile kernel");
  auto gate = [&](unsigned x) -> unsigned {
    if constexpr (LOGITS) return LN::pack(sigmoid_rcp(LN::get(x, 0)), 0.0f);
    else return x;
  };
  // coefficients of channel k of a row from its gates; steps past the sequence and channels
  // past hid are identity maps
  auto coef = [&](unsigned x1, unsigned x2, unsigned xc, int k, bool ok, float& a, float& bb) {
    Step<OP, false> st;
    st.make(LN::get(x1, k), OP == OP_MINLSTM ? LN::get(x2, k) : 0.0f, LN::get(xc, k));
    a = ok ? st.a : 1.0f;
    bb = ok ? st.b : 0.0f;
  };

  const int t0 = part * SR + w * R;
  unsigned r1[R], r2[R], rc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const unsigned o = off(t0 + j);
    r1[j] = LN::load(R1, o);
    if (OP == OP_MINLSTM) r2[j] = LN::load(R2, o);
    rc[j] = LN::load(RC, o);
  }
  {
    float A[C], B[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
      A[k] = 1.0f;
      B[k] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {  // row by row: each row's gates formed as it is folded
      r1[j] = gate(r1[j]);
      if (OP == OP_MINLSTM) r2[j] = gate(r2[j]);
#pragma unroll
      for (int k = 0; k < C; ++k) {
        float a, bb;
        coef(r1[j], OP == OP_MINLSTM ? r2[j] : 0u, rc[j], k, valid && t0 + j < seq, a, bb);
        B[k] = fmaf(a, B[k], bb);
        A[k] *= a;
      }
    }
#pragma unroll
    for (int k = 0; k < C; ++k) {
      sA[w][k][lane] = A[k];
      sB[w][k][lane] = B[k];
    }
  }
  __syncthreads();

  // the part's map: wave 0 composes the 16 wave maps (in groups of four: issued all at once,
  // their 4 C W LDS reads held the kernel's peak registers) and publishes it
  auto words = [&](int pt) { return flags + (long)(pt * nbt + bt) * 2 * C * 64 + lane; };
  if (w == 0 && part + 1 < nparts) {
    float Ag[C], Bg[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
      Ag[k] = 1.0f;
      Bg[k] = 0.0f;
    }
#pragma unroll
    for (int v0 = 0; v0 < W; v0 += 4) {
#pragma unroll
      for (int v = v0; v < v0 + 4; ++v)
#pragma unroll
        for (int k = 0; k < C; ++k) {
          Bg[k] = fmaf(sA[v][k][lane], Bg[k], sB[v][k][lane]);
          Ag[k] *= sA[v][k][lane];
        }
      asm volatile("" ::: "memory");
    }
    unsigned long long* mine = words(part);
#pragma unroll
    for (int k = 0; k < C; ++k) {
      lb_put(mine + k * 64, epoch, Ag[k]);
      lb_put(mine + (C + k) * 64, epoch, Bg[k]);
    }
  }
  // the maps of the earlier parts, wave v fetching parts v, v + 16, ...: every part's map is
  // published as soon as its own rows are folded, so the fetches of all predecessors wait
  // together, not one after another
  for (int j = w; j < part; j += W) {
    unsigned long long* pj = words(j);
    float av[C], bv[C];
    for (int spins = 0;; ++spins) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < C; ++k) {
        ok = lb_get(pj + k * 64, epoch, av[k]) && ok;
        ok = lb_get(pj + (C + k) * 64, epoch, bv[k]) && ok;
      }
      if (__all(ok)) break;
      if (spins >= spin_limit) {
        // no words from part j: its map folded here from its rows
#pragma unroll
        for (int k = 0; k < C; ++k) {
          av[k] = 1.0f;
          bv[k] = 0.0f;
        }
#pragma unroll 1
        for (int t = j * SR; t < (j + 1) * SR; ++t) {
          const unsigned o = off(t);
          const unsigned y1 = gate(LN::load(R1, o)), y2 = OP == OP_MINLSTM ? gate(LN::load(R2, o)) : 0u;
          const unsigned yc = LN::load(RC, o);
#pragma unroll
          for (int k = 0; k < C; ++k) {
            float a, bb;
            coef(y1, y2, yc, k, valid && t < seq, a, bb);
            bv[k] = fmaf(a, bv[k], bb);
            av[k] *= a;
          }
        }
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int k = 0; k < C; ++k) {
      sPA[j][k][lane] = av[k];
      sPB[j][k][lane] = bv[k];
    }
  }
  __syncthreads();
  if (w == 0) {  // the part's carry: h0 through the earlier parts' maps, in order
    float x[C];
#pragma unroll
    for (int k = 0; k < C; ++k) x[k] = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c + k) : 0.0f;
    for (int j = 0; j < part; ++j)
#pragma unroll
      for (int k = 0; k < C; ++k) x[k] = fmaf(sPA[j][k][lane], x[k], sPB[j][k][lane]);
#pragma unroll
    for (int k = 0; k < C; ++k) sH[k][lane] = x[k];
  }
  __syncthreads();

  // the coefficients are formed again from the raw values (opaque to the compiler here, so
  // that it does not keep the first pass's 2 C R coefficients live across the look-back)
#pragma unroll
  for (int j = 0; j < R; ++j) {
    asm volatile("" : "+v"(r1[j]), "+v"(rc[j]));
    if (OP == OP_MINLSTM) asm volatile("" : "+v"(r2[j]));
  }
  // this wave's carry: the maps of the waves before it applied to the part's carry
  float h[C];
#pragma unroll
  for (int k = 0; k < C; ++k) h[k] = sH[k][lane];
#pragma unroll
  for (int v0 = 0; v0 < W; v0 += 4) {
#pragma unroll
    for (int v = v0; v < v0 + 4; ++v)
#pragma unroll
      for (int k = 0; k < C; ++k)
        if (v < w) h[k] = fmaf(sA[v][k][lane], h[k], sB[v][k][lane]);
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int j = 0; j < R; ++j) {
#pragma unroll
    for (int k = 0; k < C; ++k) {
      float a, bb;
      coef(r1[j], OP == OP_MINLSTM ? r2[j] : 0u, rc[j], k, valid && t0 + j < seq, a, bb);
      h[k] = fmaf(a, h[k], bb);
    }
    LN::store(RO, off(t0 + j), h);
  }
}

// Backward look-back: the reverse scan u_t = a_t (g_t + u_{t+1}) with the same parts, each
// part's carry (u entering it from the right) from the maps of all later parts.
template <typename T, int OP, bool LOGITS, int R>
__global__ __launch_bounds__(64 * LB_W) void linscan_lb_bwd_kernel(
    const T* __restrict__ g1, const T* __restrict__ g2, const T* __restrict__ cand, const T* __restrict__ h0,
    const T* __restrict__ fwd, const T* __restrict__ dy, T* __restrict__ d1, T* __restrict__ d2,
    T* __restrict__ dcand, T* __restrict__ dh0, int seq, int hid, int ntile, unsigned long long* __restrict__ flags,
    unsigned epoch, int spin_limit) {
  typedef Lane4<T> LN;
  constexpr int W = LB_W, C = LN::C, SR = W * R;
  constexpr unsigned ES = sizeof(T);
  __shared__ float sA[W][C][64];
  __shared__ float sB[W][C][64];
  __shared__ float sU[C][64];
  __shared__ float sPA[LB_MAXP][C][64];  // the later parts' maps
  __shared__ float sPB[LB_MAXP][C][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // the last parts first: workgroups are dispatched in id order, and a part waits for the
  // parts after it
  const int bt = blockIdx.x, nbt = gridDim.x, nparts = gridDim.y, part = nparts - 1 - (int)blockIdx.y;
  const int b = bt / ntile, tile = bt % ntile;
  const int c = (tile * 64 + lane) * C;
  const bool valid = c < hid;
  const long slab = (long)b * seq * hid;
  const unsigned bytes = (unsigned)((long)seq * hid * ES);
  const rsrc_t R1 = make_rsrc(g1 + slab, bytes);
  const rsrc_t R2 = make_rsrc((OP == OP_MINLSTM ? g2 : g1) + slab, bytes);
  const rsrc_t RC = make_rsrc((OP == OP_LINEAR ? g1 : cand) + slab, bytes);
  const rsrc_t RH = make_rsrc(fwd + slab, bytes);
  const rsrc_t RY = make_rsrc(dy + slab, bytes);
  const rsrc_t W1 = make_rsrc(d1 + slab, bytes);
  const rsrc_t W2 = make_rsrc((OP == OP_MINLSTM ? d2 : d1) + slab, bytes);
  const rsrc_t WC = make_rsrc(dcand + slab, bytes);
  const unsigned cb = valid ? (unsigned)c * ES : OOB_OFF, rowb = (unsigned)hid * ES;
  auto off = [&](int t) -> unsigned { return cb + (unsigned)t * rowb; };
  // h_{t-1}: the forward output one row up; t = 0 wraps below zero, out of range (0), and
  // takes h0
  auto offp = [&](int t) -> unsigned { return cb + (unsigned)(t - 1) * rowb; };
  float hz[C];
#pragma unroll
  for (int k = 0; k < C; ++k) hz[k] = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c + k) : 0.0f;
  // per step and channel: the decay a, dy, and the factors that turn dh_t into each output
  // gradient (as in linscan_bwd_kernel)
  auto coef = [&](unsigned x1, unsigned x2, unsigned xc, unsigned xh, unsigned xy, int k, int t, float& a, float& gy,
                  float& k1, float& k2, float& kc) {
    const bool ok = valid && t < seq;
    const float v1 = LN::get(x1, k);
    const float v2 = OP == OP_MINLSTM ? LN::get(x2, k) : 0.0f;
    const float cv = OP == OP_LINEAR ? 0.0f : LN::get(xc, k);
    const float hp = t > 0 ? LN::get(xh, k) : hz[k];
    gy = LN::get(xy, k);  // 0 outside the sequence
    if (OP == OP_LINEAR) {
      a = ok ? v1 : 1.0f;
      k1 = hp;
      k2 = 0.0f;
      kc = 1.0f;
    } else if (OP == OP_MINGRU) {
      const float z = LOGITS ? sigmoid_rcp(v1) : v1;
      a = ok ? 1.0f - z : 1.0f;
      k1 = LOGITS ? (cv - hp) * (z * (1.0f - z)) : cv - hp;
      k2 = 0.0f;
      kc = z;
    } else {
      const float f = LOGITS ? sigmoid_rcp(v1) : v1;
      const float i = LOGITS ? sigmoid_rcp(v2) : v2;
      const float r = fast_rcp(f + (i + MINLSTM_EPS));
      const float r2 = r * r;
      a = ok ? f * r : 1.0f;
      float c1 = (hp * (i + MINLSTM_EPS) - cv * i) * r2;
      float c2 = (cv * (f + MINLSTM_EPS) - hp * f) * r2;
      if (LOGITS) {
        c1 *= f * (1.0f - f);
        c2 *= i * (1.0f - i);
      }
      k1 = c1;
      k2 = c2;
      kc = i * r;
    }
  };

  const int t0 = part * SR + w * R;
  unsigned r1[R], r2[R], rc[R], rh[R], ry[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const unsigned o = off(t0 + j);
    r1[j] = LN::load(R1, o);
    if (OP == OP_MINLSTM) r2[j] = LN::load(R2, o);
    if (OP != OP_LINEAR) rc[j] = LN::load(RC, o);
    rh[j] = LN::load(RH, offp(t0 + j));
    ry[j] = LN::load(RY, o);
  }
  // this wave's reverse map: u entering its last step from the right -> u leaving its first
#pragma unroll
  for (int k = 0; k < C; ++k) {
    float A = 1.0f, B = 0.0f;
#pragma unroll
    for (int j = R - 1; j >= 0; --j) {
      float a, gy, k1, k2, kc;
      coef(r1[j], OP == OP_MINLSTM ? r2[j] : 0u, OP != OP_LINEAR ? rc[j] : 0u, rh[j], ry[j], k, t0 + j, a, gy, k1, k2,
           kc);
      B = a * (gy + B);
      A *= a;
    }
    sA[w][k][lane] = A;
    sB[w][k][lane] = B;
  }
  __syncthreads();

  auto words = [&](int pt) { return flags + (long)(pt * nbt + bt) * 2 * C * 64 + lane; };
  if (w == 0 && part > 0) {  // the part's map, waves in reverse order, published for the parts before it
    float Ag[C], Bg[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
      Ag[k] = 1.0f;
      Bg[k] = 0.0f;
    }
#pragma unroll
    for (int v0 = W - 1; v0 >= 0; v0 -= 4) {
#pragma unroll
      for (int v = v0; v > v0 - 4; --v)
#pragma unroll
        for (int k = 0; k < C; ++k) {
          Bg[k] = fmaf(sA[v][k][lane], Bg[k], sB[v][k][lane]);
          Ag[k] *= sA[v][k][lane];
        }
      asm volatile("" ::: "memory");
    }
    unsigned long long* mine = words(part);
#pragma unroll
    for (int k = 0; k < C; ++k) {
      lb_put(mine + k * 64, epoch, Ag[k]);
      lb_put(mine + (C + k) * 64, epoch, Bg[k]);
    }
  }
  // the maps of the later parts, wave v fetching parts part + 1 + v, part + 17 + v, ...
  for (int j = part + 1 + w; j < nparts; j += W) {
    unsigned long long* pj = words(j);
    float av[C], bv[C];
    for (int spins = 0;; ++spins) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < C; ++k) {
        ok = lb_get(pj + k * 64, epoch, av[k]) && ok;
        ok = lb_get(pj + (C + k) * 64, epoch, bv[k]) && ok;
      }
      if (__all(ok)) break;
      if (spins >= spin_limit) {
        // no words from part j: its reverse map folded here from its rows
#pragma unroll
        for (int k = 0; k < C; ++k) {
          av[k] = 1.0f;
          bv[k] = 0.0f;
        }
#pragma unroll 1
        for (int t = (j + 1) * SR - 1; t >= j * SR; --t) {
          const unsigned o = off(t);
          const unsigned y1 = LN::load(R1, o), y2 = OP == OP_MINLSTM ? LN::load(R2, o) : 0u;
          const unsigned yc = OP != OP_LINEAR ? LN::load(RC, o) : 0u, yh = LN::load(RH, offp(t)), yy = LN::load(RY, o);
#pragma unroll
          for (int k = 0; k < C; ++k) {
            float a, gy, k1, k2, kc;
            coef(y1, y2, yc, yh, yy, k, t, a, gy, k1, k2, kc);
            bv[k] = a * (gy + bv[k]);
            av[k] *= a;
          }
        }
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int k = 0; k < C; ++k) {
      sPA[j - part - 1][k][lane] = av[k];
      sPB[j - part - 1][k][lane] = bv[k];
    }
  }
  __syncthreads();
  if (w == 0) {  // the part's carry: 0 at the sequence end through the later parts' maps
    float x[C];
#pragma unroll
    for (int k = 0; k < C; ++k) x[k] = 0.0f;
    for (int j = nparts - 1; j > part; --j)
#pragma unroll
      for (int k = 0; k < C; ++k) x[k] = fmaf(sPA[j - part - 1][k][lane], x[k], sPB[j - part - 1][k][lane]);
#pragma unroll
    for (int k = 0; k < C; ++k) sU[k][lane] = x[k];
  }
  __syncthreads();

  // coefficients formed again from the raw values (opaque here, as in the forward)
#pragma unroll
  for (int j = 0; j < R; ++j) {
    asm volatile("" : "+v"(r1[j]), "+v"(rh[j]), "+v"(ry[j]));
    if (OP == OP_MINLSTM) asm volatile("" : "+v"(r2[j]));
    if (OP != OP_LINEAR) asm volatile("" : "+v"(rc[j]));
  }
  // this wave's carry: the maps of the waves after it applied to the part's carry
  float u[C];
#pragma unroll
  for (int k = 0; k < C; ++k) u[k] = sU[k][lane];
#pragma unroll
  for (int v0 = W - 1; v0 >= 0; v0 -= 4) {
#pragma unroll
    for (int v = v0; v > v0 - 4; --v)
#pragma unroll
      for (int k = 0; k < C; ++k)
        if (v > w) u[k] = fmaf(sA[v][k][lane], u[k], sB[v][k][lane]);
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int j = R - 1; j >= 0; --j) {
    float o1[C], o2[C], oc[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
      float a, gy, k1, k2, kc;
      coef(r1[j], OP == OP_MINLSTM ? r2[j] : 0u, OP != OP_LINEAR ? rc[j] : 0u, rh[j], ry[j], k, t0 + j, a, gy, k1, k2,
           kc);
      const float dh = gy + u[k];
      u[k] = a * dh;
      o1[k] = dh * k1;
      o2[k] = dh * k2;
      oc[k] = dh * kc;
    }
    const unsigned o = off(t0 + j);
    LN::store(W1, o, o1);
    if (OP == OP_MINLSTM) LN::store(W2, o, o2);
    LN::store(WC, o, oc);
  }
  if (valid && part == 0 && w == 0 && dh0 != nullptr) {
#pragma unroll
    for (int k = 0; k < C; ++k) st(dh0, (long)b * hid + c + k, u[k]);
  }
}

constexpr int LB_MAX_DEVICES = 64;
std::mutex g_lb_mu;
unsigned long long* g_lb_ptr[LB_MAX_DEVICES] = {};
std::atomic<unsigned> g_lb_epoch{0x6c620000u};

// The device copy of lb_flags for the stream's device (nullptr if it cannot be found).
unsigned long long* lb_flags_address(hipStream_t s) {
  int cur = 0, dev = 0;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  dev = cur;
  if (s != nullptr && hipStreamGetDevice(s, &dev) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= LB_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(g_lb_mu);
  if (g_lb_ptr[dev] == nullptr) {
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(lb_flags));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_lb_ptr[dev] = (unsigned long long*)p;
  }
  return g_lb_ptr[dev];
}

int lb_spin_limit() {
  const char* env = getenv("EDF_LIN_LOOKBACK_SPIN");
  return env != nullptr ? std::max(0, atoi(env)) : LB_SPIN;
}

unsigned lb_next_epoch() {
  unsigned e;
  do e = ++g_lb_epoch; while (e == 0);
  return e;
}

// The look-back scan serves sequences of at least 512 steps whose words fit lb_flags, on a
// stream that is not capturing; EDF_LIN_LOOKBACK=0 selects the one-workgroup-per-tile kernels.
template <typename T, int R>
unsigned long long* lb_plan(hipStream_t s, int bsz, int seq, int hid, int& ntile, int& nparts) {
  constexpr int C = Lane4<T>::C, SR = LB_W * R;
  const char* env = getenv("EDF_LIN_LOOKBACK");
  if (env != nullptr && !strcmp(env, "0")) return nullptr;
  if (hid % C != 0 || seq < 512) return nullptr;
  ntile = (hid + 64 * C - 1) / (64 * C);
  nparts = (seq + SR - 1) / SR;
  const long words = (long)nparts * bsz * ntile * 2 * C * 64;
  if (words > (long)LB_WORDS || nparts > LB_MAXP) return nullptr;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (st != hipStreamCaptureStatusNone) return nullptr;
  return lb_flags_address(s);
}

inline const char* op_name(int op, bool backward = false) {
  static const char* const names[3][2] = {{"mingru scan", "mingru scan backward"},
                                          {"minlstm scan", "minlstm scan backward"},
                                          {"linear scan", "linear scan backward"}};
  return names[op][backward ? 1 : 0];
}

// PAD: the launch has steps past the sequence inside a macro-step, or channels past hid;
// those are masked into identity steps.  Without them the masks are compiled out (whole
// padding macro-steps past the sequence only feed values that are never stored: zeros
// entering the reverse scan, states past the end in the forward).
template <int L, int W, bool PAIRS>
inline bool needs_pad(int seq, int hid) {
  return seq % ((PAIRS ? 2 : 1) * W * L) != 0 || hid % 64 != 0;
}

template <typename T, int OP, bool LOGITS>
int launch_fwd(hipStream_t s, const void* g1, const void* g2, const void* cand, const void* h0, void* out, int bsz,
               int seq, int hid) {
  const dim3 grid((hid + 63) / 64, bsz);
  const T* a = (const T*)g1;
  const T* b = (const T*)g2;
  const T* c = (const T*)cand;
  const T* i = (const T*)h0;
  T* o = (T*)out;
  int ntile = 0, nparts = 0;
  // the forward look-back for f32 and the bf16 linear scan.  The bf16 MinGRU / MinLSTM forward
  // keeps the per-tile kernel: it would form its gates' sigmoids a second time after the wait
  // (measured no faster), and gates kept in place as bf16 pairs lose too much (3.6e-2
  // element-wise against the oracle)
  if constexpr (!std::is_same<T, bf16>::value || OP == OP_LINEAR) {
    if (unsigned long long* flags = lb_plan<T, LB_R>(s, bsz, seq, hid, ntile, nparts)) {
      linscan_lb_fwd_kernel<T, OP, LOGITS, LB_R><<<dim3(bsz * ntile, nparts), 64 * LB_W, 0, s>>>(
          a, b, c, i, o, seq, hid, ntile, flags, lb_next_epoch(), lb_spin_limit());
      return check_launch(op_name(OP));
    }
  }
#define EDF_LIN_LAUNCH(KERNEL, L, W, P, PAIRS)                                                      \
  do {                                                                                            \
    if (needs_pad<L, W, PAIRS>(seq, hid))                                                         \
      KERNEL<T, OP, LOGITS, L, W, P, true><<<grid, 64 * W, 0, s>>>(a, b, c, i, o, seq, hid);      \
    else                                                                                          \
      KERNEL<T, OP, LOGITS, L, W, P, false><<<grid, 64 * W, 0, s>>>(a, b, c, i, o, seq, hid);     \
  } while (0)
  if constexpr (std::is_same<T, bf16>::value) {
    if (hid % 2 == 0) {  // two channels per lane
      if (seq >= 512) EDF_LIN_LAUNCH(linscan2_fwd_kernel, LIN2_LF, LIN2_W, LIN_PF, true);
      else EDF_LIN_LAUNCH(linscan2_fwd_kernel, LIN2_LF, 4, 2, true);
      return check_launch(op_name(OP));
    }
  }
  if (seq >= 512) EDF_LIN_LAUNCH(linscan_fwd_kernel, LIN_LF, 16, LIN_PF, false);
  else EDF_LIN_LAUNCH(linscan_fwd_kernel, LIN_LF, 4, 2, false);
#undef EDF_LIN_LAUNCH
  return check_launch(op_name(OP));
}

template <typename T, int OP, bool LOGITS>
int launch_bwd(hipStream_t s, const void* g1, const void* g2, const void* cand, const void* h0, const void* fwd,
               const void* dy, void* d1, void* d2, void* dcand, void* dh0, int bsz, int seq, int hid) {
  const dim3 grid((hid + 63) / 64, bsz);
  const T* a = (const T*)g1;
  const T* b = (const T*)g2;
  const T* c = (const T*)cand;
  const T* i = (const T*)h0;
  const T* f = (const T*)fwd;
  const T* y = (const T*)dy;
  T* o1 = (T*)d1;
  T* o2 = (T*)d2;
  T* oc = (T*)dcand;
  T* oh = (T*)dh0;
  int ntile = 0, nparts = 0;
  if (unsigned long long* flags = lb_plan<T, LB_R>(s, bsz, seq, hid, ntile, nparts)) {
    linscan_lb_bwd_kernel<T, OP, LOGITS, LB_R><<<dim3(bsz * ntile, nparts), 64 * LB_W, 0, s>>>(
        a, b, c, i, f, y, o1, o2, oc, oh, seq, hid, ntile, flags, lb_next_epoch(), lb_spin_limit());
    return check_launch(op_name(OP, true));
  }
#define EDF_LIN_LAUNCH(KERNEL, L, W, P, PAIRS)                                                                 \
  do {                                                                                                       \
    if (needs_pad<L, W, PAIRS>(seq, hid))                                                                    \
      KERNEL<T, OP, LOGITS, L, W, P, true><<<grid, 64 * W, 0, s>>>(a, b, c, i, f, y, o1, o2, oc, oh, seq, hid);  \
    else                                                                                                     \
      KERNEL<T, OP, LOGITS, L, W, P, false><<<grid, 64 * W, 0, s>>>(a, b, c, i, f, y, o1, o2, oc, oh, seq, hid); \
  } while (0)
  if constexpr (std::is_same<T, bf16>::value) {
    if (hid % 2 == 0) {  // two channels per lane
      if (seq >= 512) EDF_LIN_LAUNCH(linscan2_bwd_kernel, LIN2_LB, LIN2_W, LIN_PB, true);
      else EDF_LIN_LAUNCH(linscan2_bwd_kernel, LIN2_LB, 4, 2, true);
      return check_launch(op_name(OP, true));
    }
  }
  if (seq >= 512) EDF_LIN_LAUNCH(linscan_bwd_kernel, LIN_LB, 16, LIN_PB, false);
  else EDF_LIN_LAUNCH(linscan_bwd_kernel, LIN_LB, 4, 2, false);
#undef EDF_LIN_LAUNCH
  return check_launch(op_name(OP, true));
}

template <int OP, bool LOGITS>
int fwd_dispatch(void* stream, const void* g1, const void* g2, const void* cand, const void* h0, void* out, int bsz,
                 int seq, int hid, int dtype) {
  EDF_REQUIRE(bsz > 0 && seq > 0 && hid > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE((long)(seq + 512) * hid * (dtype == EDF_BF16 ? 2 : 4) < (1L << 31), EDF_ERR_UNSUPPORTED,
              "seq_len * hidden too large (one batch row plus padding must stay below 2 GiB)");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(g1 && cand && out && (OP != OP_MINLSTM || g2), EDF_ERR_INVALID_ARG, "null tensor pointer");
  if (dtype == EDF_BF16) return launch_fwd<bf16, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, out, bsz, seq, hid);
  return launch_fwd<float, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, out, bsz, seq, hid);
}

template <int OP, bool LOGITS>
int bwd_dispatch(void* stream, const void* g1, const void* g2, const void* cand, const void* h0, const void* fwd,
                 const void* dy, void* d1, void* d2, void* dcand, void* dh0, int bsz, int seq, int hid, int dtype) {
  EDF_REQUIRE(bsz > 0 && seq > 0 && hid > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE((long)(seq + 512) * hid * (dtype == EDF_BF16 ? 2 : 4) < (1L << 31), EDF_ERR_UNSUPPORTED,
              "seq_len * hidden too large (one batch row plus padding must stay below 2 GiB)");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(g1 && (OP == OP_LINEAR || cand) && fwd && dy && d1 && dcand && (OP != OP_MINLSTM || (g2 && d2)),
              EDF_ERR_INVALID_ARG, "null tensor pointer");
  if (dtype == EDF_BF16)
    return launch_bwd<bf16, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, fwd, dy, d1, d2, dcand, dh0, bsz, seq,
                                        hid);
  return launch_bwd<float, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, fwd, dy, d1, d2, dcand, dh0, bsz, seq,
                                       hid);
}

// ---------------------------------------------------------------------------------
// Multi-layer blocks, inference.  Per layer l, with x_0 the input and n = LayerNorm(x_l)
// (biased variance, eps 1e-5, gamma, beta), P projections p_k = n W_k + b_k feed one scan
// from h0[:, l] and x_{l+1} = x_l + h:
//   MinGRU  (P = 2: z, c)     h = (1 - sigmoid(z)) h + sigmoid(z) c
//           native/cuda/fused_mingru_block_scan.cu:45-140, fused_scan.ex:4521-4571
//   MinLSTM (P = 3: f, i, c)  h = f' h + i' c, f' = s(f) / (s(f) + s(i) + 1e-6), ...
//           fused_minlstm_block_scan.cu:59-140, fused_scan.ex:4647-4705
//   linear  (P = 2: a, b)     h = a h + b
//           fused_linear_block_scan.cu:100-126, fused_scan.ex:4785-4835
// The reference walks timesteps and layers one by one in one workgroup per batch row
// (every step a matrix-vector product).  The projections depend on x only, so here each
// layer is one parallel pass over all (b, t) rows: a projection kernel (the previous
// layer's residual, the LayerNorm and the P products on f32 MFMA, 32 rows per workgroup)
// and the scan above (sigmoids fused); activations stay in f32 between layers, as in the
// reference's registers.  Packed weights per layer: W_1 [H][H] (input-major), b_1, ..,
// W_P, b_P, gamma, beta, in the I/O dtype.
// ---------------------------------------------------------------------------------
constexpr int MGB_ROWS = 32;                // rows (b, t) per projection workgroup
constexpr int MGB_HMAX = 256;
constexpr int MGB_LD = MGB_HMAX + 2;        // LDS row stride: the A-operand reads are conflict-free
constexpr float MGB_LN_EPS = 1.0e-5f;

typedef __attribute__((ext_vector_type(16))) float mgb_f32x16;

struct MgbOut {
  float* p[3];  // the P projection outputs, [rows][H] each
};

// Layer input x_l (the input for l = 0, else x_{l-1} + h_{l-1}) written back to X, its
// LayerNorm, and the P projections n W_k + b_k.
template <typename T, int P>
__global__ __launch_bounds__(256) void mgb_proj_kernel(const T* __restrict__ input, float* __restrict__ X,
                                                       const float* __restrict__ Hprev, const T* __restrict__ Wl,
                                                       const MgbOut po, long rows, int H, int first) {
  __shared__ float sn[MGB_ROWS * MGB_LD];  // normalized rows, zero-padded to an even H
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long row0 = (long)blockIdx.x * MGB_ROWS;
  const long pstride = (long)H * H + H;  // W_k [H][H] then b_k [H]
  const T* gamma = Wl + P * pstride;
  const T* beta = gamma + H;
  // ---- residual + LayerNorm: wave w normalizes rows 8 w .. 8 w + 7 ----
  for (int rr = 0; rr < MGB_ROWS / 4; ++rr) {
    const int r = w * (MGB_ROWS / 4) + rr;
    const long row = row0 + r;
    const bool rok = row < rows;
    float x[MGB_HMAX / 64];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < MGB_HMAX / 64; ++j) {
      const int c = lane + 64 * j;
      const bool ok = rok && c < H;
      const long idx = ok ? row * H + c : 0;
      const float v = first ? to_f32(input[idx]) : X[idx] + Hprev[idx];
      x[j] = ok ? v : 0.0f;
      if (ok) X[idx] = x[j];
      sum += x[j];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float mean = sum / (float)H;
    float var = 0.0f;
#pragma unroll
    for (int j = 0; j < MGB_HMAX / 64; ++j) {
      const float d = (lane + 64 * j < H) ? x[j] - mean : 0.0f;
      var = fmaf(d, d, var);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) var += __shfl_xor(var, off);
    const float inv = 1.0f / sqrtf(var / (float)H + MGB_LN_EPS);
#pragma unroll
    for (int j = 0; j < MGB_HMAX / 64; ++j) {
      const int c = lane + 64 * j;
      if (c < H) sn[r * MGB_LD + c] = fmaf((x[j] - mean) * inv, to_f32(gamma[c]), to_f32(beta[c]));
      else if (c < MGB_LD) sn[r * MGB_LD + c] = 0.0f;
    }
  }
  __syncthreads();
  // ---- [32 rows] x [P H columns] on v_mfma_f32_32x32x2_f32: wave w takes column tiles w, w+4, ..;
  // lane (li, g) supplies A[row li][k = 2 kk + g] and B[k][column li] for k step kk.  The W
  // column values of 16 k steps are loaded a chunk ahead into one of two register sets.
  const int li = lane & 31, g = lane >> 5;
  const int ntile = (P * H + 31) / 32, nch = ((H + 1) / 2 + 15) / 16;
  for (int nt = w; nt < ntile; nt += 4) {
    const int n = nt * 32 + li;  // this lane's output column: projection n / H, column n % H
    const bool nok = n < P * H;
    const int nc = min(n, P * H - 1), pj = nc / H, cj = nc % H;
    const T* Wc = Wl + pj * pstride + cj;
    float b0[16], b1[16];
    auto ldb = [&](float* bb, int ch) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int k = 2 * (16 * ch + i) + g;
        const float v = to_f32(Wc[(long)min(k, H - 1) * H]);
        bb[i] = (nok && k < H) ? v : 0.0f;  // zero past H: the zero-padded A rows meet zero B
      }
    };
    mgb_f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    auto mm = [&](const float* bb, int ch) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(sn[li * MGB_LD + 2 * (16 * ch + i) + g], bb[i], acc, 0, 0, 0);
    };
    ldb(b0, 0);
    ldb(b1, min(1, nch - 1));
    int ch = 0;
    for (; ch + 1 < nch; ch += 2) {
      mm(b0, ch);
      ldb(b0, min(ch + 2, nch - 1));
      mm(b1, ch + 1);
      ldb(b1, min(ch + 3, nch - 1));
    }
    if (ch < nch) mm(b0, ch);
    if (nok) {
      const float bias = to_f32(Wl[pj * pstride + (long)H * H + cj]);
      float* dst = (pj == 0 ? po.p[0] : pj == 1 ? po.p[1] : po.p[2]) + cj;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const long row = row0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (row < rows) dst[row * H] = acc[r] + bias;
      }
    }
  }
}

// h0[:, l, :] (or zeros) as a contiguous f32 [B, H] initial state
template <typename T>
__global__ __launch_bounds__(256) void mgb_h0_kernel(const T* __restrict__ h0, float* __restrict__ dst, int B, int L,
                                                     int l, int H) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= B * H) return;
  const int b = e / H, c = e % H;
  dst[e] = h0 != nullptr ? to_f32(h0[((long)b * L + l) * H + c]) : 0.0f;
}

// output = x_{L-1} + h_{L-1}
template <typename T>
__global__ __launch_bounds__(256) void mgb_out_kernel(const float* __restrict__ X, const float* __restrict__ Hs,
                                                      T* __restrict__ out, long n) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e < n) out[e] = (T)(X[e] + Hs[e]);
}

struct MgbWs {
  float *X, *Hs, *h0s;
  float* p[3];
  size_t total;
};
inline MgbWs mgb_layout(void* base, long bth, int B, int H, int P) {
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  MgbWs L{};
  size_t off = 0;
  char* c = (char*)base;
  L.X = (float*)(c + off); off += up(bth * 4);
  L.Hs = (float*)(c + off); off += up(bth * 4);
  for (int k = 0; k < P; ++k) {
    L.p[k] = (float*)(c + off);
    off += up(bth * 4);
  }
  L.h0s = (float*)(c + off); off += up((size_t)B * H * 4);
  L.total = off;
  return L;
}

enum { BLK_MINGRU = 0, BLK_MINLSTM = 1, BLK_LINEAR = 2 };
constexpr int blk_projections(int kind) { return kind == BLK_MINLSTM ? 3 : 2; }

template <typename T, int KIND>
int mgb_run(hipStream_t s, const void* input, const void* weights, const void* h0, void* out, const MgbWs& ws,
            int B, int Tn, int H, int L) {
  constexpr int P = blk_projections(KIND);
  const long bth = (long)B * Tn * H, rows = (long)B * Tn;
  const long lstride = P * ((long)H * H + H) + 2L * H;
  const MgbOut po{{ws.p[0], ws.p[1], ws.p[P - 1]}};
  for (int l = 0; l < L; ++l) {
    mgb_proj_kernel<T, P><<<(unsigned)((rows + MGB_ROWS - 1) / MGB_ROWS), 256, 0, s>>>(
        (const T*)input, ws.X, ws.Hs, (const T*)weights + l * lstride, po, rows, H, l == 0 ? 1 : 0);
    if (int rc = check_launch("block projection")) return rc;
    mgb_h0_kernel<T><<<(B * H + 255) / 256, 256, 0, s>>>((const T*)h0, ws.h0s, B, L, l, H);
    if (int rc = check_launch("block h0")) return rc;
    int rc;
    if constexpr (KIND == BLK_MINGRU)
      rc = launch_fwd<float, OP_MINGRU, true>(s, ws.p[0], nullptr, ws.p[1], ws.h0s, ws.Hs, B, Tn, H);
    else if constexpr (KIND == BLK_MINLSTM)
      rc = launch_fwd<float, OP_MINLSTM, true>(s, ws.p[0], ws.p[1], ws.p[2], ws.h0s, ws.Hs, B, Tn, H);
    else
      rc = launch_fwd<float, OP_LINEAR, false>(s, ws.p[0], nullptr, ws.p[1], ws.h0s, ws.Hs, B, Tn, H);
    if (rc) return rc;
  }
  mgb_out_kernel<T><<<(unsigned)((bth + 255) / 256), 256, 0, s>>>(ws.X, ws.Hs, (T*)out, bth);
  return check_launch("block output");
}

template <int KIND>
int block_dispatch(void* stream, const void* input, const void* weights, const void* h0, void* out, void* workspace,
                   size_t workspace_bytes, int batch, int seq_len, int hidden, int num_layers, int dtype) {
  EDF_REQUIRE(batch > 0 && seq_len > 0 && hidden > 0 && num_layers > 0, EDF_ERR_INVALID_ARG,
              "dimensions and num_layers must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(hidden <= MGB_HMAX, EDF_ERR_UNSUPPORTED, "hidden %d unsupported (the block scans take H <= %d)",
              hidden, MGB_HMAX);
  EDF_REQUIRE((long)(seq_len + 512) * hidden * 4 < (1L << 31), EDF_ERR_UNSUPPORTED,
              "seq_len * hidden too large (one batch row of f32 activations plus padding must stay below 2 GiB)");
  EDF_REQUIRE(input && weights && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const MgbWs L = mgb_layout(workspace, (long)batch * seq_len * hidden, batch, hidden, blk_projections(KIND));
  EDF_REQUIRE(workspace && workspace_bytes >= L.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              L.total);
  if (dtype == EDF_BF16)
    return mgb_run<bf16, KIND>(as_stream(stream), input, weights, h0, out, L, batch, seq_len, hidden, num_layers);
  return mgb_run<float, KIND>(as_stream(stream), input, weights, h0, out, L, batch, seq_len, hidden, num_layers);
}

inline size_t block_ws_bytes(int batch, int seq_len, int hidden, int kind) {
  if (batch <= 0 || seq_len <= 0 || hidden <= 0) return 0;
  return mgb_layout(nullptr, (long)batch * seq_len * hidden, batch, hidden, blk_projections(kind)).total;
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_mingru_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype) {
  (void)num_layers;
  (void)dtype;
  return edf::block_ws_bytes(batch, seq_len, hidden, edf::BLK_MINGRU);
}

int edf_fused_mingru_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                                void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                                int num_layers, int dtype) {
  return edf::block_dispatch<edf::BLK_MINGRU>(stream, input, weights, h0, out, workspace, workspace_bytes, batch,
                                              seq_len, hidden, num_layers, dtype);
}

size_t edf_minlstm_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype) {
  (void)num_layers;
  (void)dtype;
  return edf::block_ws_bytes(batch, seq_len, hidden, edf::BLK_MINLSTM);
}

int edf_fused_minlstm_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                                 void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                                 int num_layers, int dtype) {
  return edf::block_dispatch<edf::BLK_MINLSTM>(stream, input, weights, h0, out, workspace, workspace_bytes, batch,
                                               seq_len, hidden, num_layers, dtype);
}

size_t edf_linear_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype) {
  (void)num_layers;
  (void)dtype;
  return edf::block_ws_bytes(batch, seq_len, hidden, edf::BLK_LINEAR);
}

int edf_fused_linear_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                                void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                                int num_layers, int dtype) {
  return edf::block_dispatch<edf::BLK_LINEAR>(stream, input, weights, h0, out, workspace, workspace_bytes, batch,
                                              seq_len, hidden, num_layers, dtype);
}

int edf_fused_mingru_scan(void* stream, const void* z, const void* cand, const void* h0, void* out, int batch,
                          int seq_len, int hidden, int dtype) {
  return edf::fwd_dispatch<edf::OP_MINGRU, false>(stream, z, nullptr, cand, h0, out, batch, seq_len, hidden, dtype);
}

int edf_fused_mingru_scan_backward(void* stream, const void* z, const void* cand, const void* h0,
                                   const void* forward_out, const void* grad_out, void* grad_z, void* grad_cand,
                                   void* grad_h0, int batch, int seq_len, int hidden, int dtype) {
  return edf::bwd_dispatch<edf::OP_MINGRU, false>(stream, z, nullptr, cand, h0, forward_out, grad_out, grad_z,
                                                  nullptr, grad_cand, grad_h0, batch, seq_len, hidden, dtype);
}

int edf_mingru(void* stream, const void* gates, const void* cand, void* out, int batch, int seq_len, int hidden,
               int dtype) {
  return edf::fwd_dispatch<edf::OP_MINGRU, true>(stream, gates, nullptr, cand, nullptr, out, batch, seq_len, hidden,
                                                 dtype);
}

int edf_mingru_backward(void* stream, const void* gates, const void* cand, const void* forward_out,
                        const void* grad_out, void* grad_gates, void* grad_cand, int batch, int seq_len, int hidden,
                        int dtype) {
  return edf::bwd_dispatch<edf::OP_MINGRU, true>(stream, gates, nullptr, cand, nullptr, forward_out, grad_out,
                                                 grad_gates, nullptr, grad_cand, nullptr, batch, seq_len, hidden,
                                                 dtype);
}

int edf_fused_minlstm_scan(void* stream, const void* f, const void* i, const void* cand, const void* h0, void* out,
                           int batch, int seq_len, int hidden, int dtype) {
  return edf::fwd_dispatch<edf::OP_MINLSTM, false>(stream, f, i, cand, h0, out, batch, seq_len, hidden, dtype);
}

int edf_fused_minlstm_scan_backward(void* stream, const void* f, const void* i, const void* cand, const void* h0,
                                    const void* forward_out, const void* grad_out, void* grad_f, void* grad_i,
                                    void* grad_cand, void* grad_h0, int batch, int seq_len, int hidden, int dtype) {
  return edf::bwd_dispatch<edf::OP_MINLSTM, false>(stream, f, i, cand, h0, forward_out, grad_out, grad_f, grad_i,
                                                   grad_cand, grad_h0, batch, seq_len, hidden, dtype);
}

int edf_minlstm(void* stream, const void* forget_gates, const void* input_gates, const void* cand, void* out,
                int batch, int seq_len, int hidden, int dtype) {
  return edf::fwd_dispatch<edf::OP_MINLSTM, true>(stream, forget_gates, input_gates, cand, nullptr, out, batch,
                                                  seq_len, hidden, dtype);
}

int edf_minlstm_backward(void* stream, const void* forget_gates, const void* input_gates, const void* cand,
                         const void* forward_out, const void* grad_out, void* grad_forget, void* grad_input,
                         void* grad_cand, int batch, int seq_len, int hidden, int dtype) {
  return edf::bwd_dispatch<edf::OP_MINLSTM, true>(stream, forget_gates, input_gates, cand, nullptr, forward_out,
                                                  grad_out, grad_forget, grad_input, grad_cand, nullptr, batch,
                                                  seq_len, hidden, dtype);
}

int edf_fused_linear_scan(void* stream, const void* a, const void* b, const void* h0, void* out, int batch,
                          int seq_len, int hidden, int dtype) {
  return edf::fwd_dispatch<edf::OP_LINEAR, false>(stream, a, nullptr, b, h0, out, batch, seq_len, hidden, dtype);
}

int edf_fused_linear_scan_backward(void* stream, const void* a, const void* h0, const void* forward_out,
                                   const void* grad_out, void* grad_a, void* grad_b, void* grad_h0, int batch,
                                   int seq_len, int hidden, int dtype) {
  return edf::bwd_dispatch<edf::OP_LINEAR, false>(stream, a, nullptr, nullptr, h0, forward_out, grad_out, grad_a,
                                                  nullptr, grad_b, grad_h0, batch, seq_len, hidden, dtype);
}

}  // extern "C"
