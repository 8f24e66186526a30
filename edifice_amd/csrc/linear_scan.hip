// MinGRU / MinLSTM linear scans, forward and backward, for gfx950.
//
// Semantics (reference):
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
//   * backward runs the same scan in reverse time on u_t = a_t (g_t + u_{t+1}).
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr float MINLSTM_EPS = 1.0e-6f;

enum { OP_MINGRU = 0, OP_MINLSTM = 1 };

// Coefficients of step t: h_t = a h_{t-1} + b.
template <int OP, bool LOGITS>
struct Step {
  float a, b;
  EDF_DEVICE void make(float g1, float g2, float c) {
    if (OP == OP_MINGRU) {
      const float z = LOGITS ? sigmoidf(g1) : g1;
      a = 1.0f - z;
      b = z * c;
    } else {
      const float f = LOGITS ? sigmoidf(g1) : g1;
      const float i = LOGITS ? sigmoidf(g2) : g2;
      const float r = 1.0f / (f + (i + MINLSTM_EPS));
      a = f * r;
      b = (i * r) * c;
    }
  }
};

template <typename T, int OP, bool LOGITS, int L, int W>
__global__ __launch_bounds__(64 * W) void linscan_fwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                             const T* __restrict__ cand, const T* __restrict__ h0,
                                                             T* __restrict__ out, int seq, int hid) {
  __shared__ float sA[2][W][64];
  __shared__ float sB[2][W][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool valid = c < hid;
  const long base = (long)b * seq * hid + min(c, hid - 1);  // loads stay in bounds; stores are guarded

  float h = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c) : 0.0f;
  const int steps = (seq + W * L - 1) / (W * L);
  for (int ms = 0; ms < steps; ++ms) {
    const int t0 = ms * W * L + w * L;
    float a[L], bb[L];
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int t = t0 + j;
      const long idx = base + (long)min(t, seq - 1) * hid;
      Step<OP, LOGITS> s;
      s.make(ld(g1, idx), OP == OP_MINLSTM ? ld(g2, idx) : 0.0f, ld(cand, idx));
      const bool ok = valid && t < seq;  // padding steps are the identity map
      a[j] = ok ? s.a : 1.0f;
      bb[j] = ok ? s.b : 0.0f;
    }
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
    float hin = h;
    for (int v = 0; v < w; ++v) hin = fmaf(sA[buf][v][lane], hin, sB[buf][v][lane]);
    float hend = fmaf(A, hin, B);
    for (int v = w + 1; v < W; ++v) hend = fmaf(sA[buf][v][lane], hend, sB[buf][v][lane]);
    float hh = hin;
#pragma unroll
    for (int j = 0; j < L; ++j) {
      hh = fmaf(a[j], hh, bb[j]);
      const int t = t0 + j;
      if (valid && t < seq) st(out, base + (long)t * hid, hh);
    }
    h = hend;
  }
}

// Backward: reverse scan u_t = a_t (g_t + u_{t+1}), dh_t = g_t + u_{t+1}, dh0 = u_0.
template <typename T, int OP, bool LOGITS, int L, int W>
__global__ __launch_bounds__(64 * W) void linscan_bwd_kernel(const T* __restrict__ g1, const T* __restrict__ g2,
                                                             const T* __restrict__ cand, const T* __restrict__ h0,
                                                             const T* __restrict__ fwd, const T* __restrict__ dy,
                                                             T* __restrict__ d1, T* __restrict__ d2,
                                                             T* __restrict__ dcand, T* __restrict__ dh0, int seq,
                                                             int hid) {
  __shared__ float sA[2][W][64];
  __shared__ float sB[2][W][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int b = blockIdx.y;
  const int c = blockIdx.x * 64 + lane;
  const bool valid = c < hid;
  const long base = (long)b * seq * hid + min(c, hid - 1);  // loads stay in bounds; stores are guarded
  const float h0v = (valid && h0 != nullptr) ? ld(h0, (long)b * hid + c) : 0.0f;

  float u = 0.0f;  // u_{t+1} entering the macro-step from the right
  const int steps = (seq + W * L - 1) / (W * L);
  const int tpad = steps * W * L;
  for (int ms = 0; ms < steps; ++ms) {
    // wave 0 owns the latest L timesteps of this macro-step
    const int t0 = tpad - (ms + 1) * W * L + (W - 1 - w) * L;
    float x1[L], x2[L], cc[L], hp[L], gy[L];
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int t = t0 + j;
      const bool ok = valid && t < seq;
      const long idx = base + (long)min(t, seq - 1) * hid;
      const long pidx = base + (long)max(min(t, seq - 1) - 1, 0) * hid;
      const float v1 = ld(g1, idx);
      const float v2 = OP == OP_MINLSTM ? ld(g2, idx) : 0.0f;
      const float vc = ld(cand, idx);
      const float vh = ld(fwd, pidx);
      const float vy = ld(dy, idx);
      x1[j] = ok ? v1 : 0.0f;
      x2[j] = ok ? v2 : 0.0f;
      cc[j] = ok ? vc : 0.0f;
      hp[j] = ok ? (t > 0 ? vh : h0v) : 0.0f;
      gy[j] = ok ? vy : 0.0f;
    }
    // per-step decay a_t (1 for padding)
    float a[L];
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int t = t0 + j;
      Step<OP, LOGITS> s;
      s.make(x1[j], x2[j], cc[j]);
      a[j] = (valid && t < seq) ? s.a : 1.0f;
    }
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
    float uin = u;
    for (int v = 0; v < w; ++v) uin = fmaf(sA[buf][v][lane], uin, sB[buf][v][lane]);
    float uend = fmaf(A, uin, B);
    for (int v = w + 1; v < W; ++v) uend = fmaf(sA[buf][v][lane], uend, sB[buf][v][lane]);
#pragma unroll
    for (int j = L - 1; j >= 0; --j) {
      const int t = t0 + j;
      const float dh = gy[j] + uin;
      uin = a[j] * dh;
      if (!(valid && t < seq)) continue;
      const long idx = base + (long)t * hid;
      if (OP == OP_MINGRU) {
        const float z = LOGITS ? sigmoidf(x1[j]) : x1[j];
        float dz = dh * (cc[j] - hp[j]);
        if (LOGITS) dz *= z * (1.0f - z);
        st(d1, idx, dz);
        st(dcand, idx, dh * z);
      } else {
        const float f = LOGITS ? sigmoidf(x1[j]) : x1[j];
        const float i = LOGITS ? sigmoidf(x2[j]) : x2[j];
        const float s = f + (i + MINLSTM_EPS);
        const float r = 1.0f / s;
        const float dfn = dh * hp[j];
        const float din = dh * cc[j];
        const float r2 = r * r;
        float df = (dfn * (i + MINLSTM_EPS) - din * i) * r2;
        float di = (din * (f + MINLSTM_EPS) - dfn * f) * r2;
        if (LOGITS) {
          df *= f * (1.0f - f);
          di *= i * (1.0f - i);
        }
        st(d1, idx, df);
        st(d2, idx, di);
        st(dcand, idx, dh * (i * r));
      }
    }
    u = uend;
  }
  if (valid && w == 0 && dh0 != nullptr) st(dh0, (long)b * hid + c, u);
}

template <typename T, int OP, bool LOGITS>
int launch_fwd(hipStream_t s, const void* g1, const void* g2, const void* cand, const void* h0, void* out, int bsz,
               int seq, int hid) {
  constexpr int L = 8;
  const dim3 grid((hid + 63) / 64, bsz);
  if (seq >= 512) {
    constexpr int W = 16;
    linscan_fwd_kernel<T, OP, LOGITS, L, W><<<grid, 64 * W, 0, s>>>((const T*)g1, (const T*)g2, (const T*)cand,
                                                                    (const T*)h0, (T*)out, seq, hid);
  } else {
    constexpr int W = 4;
    linscan_fwd_kernel<T, OP, LOGITS, L, W><<<grid, 64 * W, 0, s>>>((const T*)g1, (const T*)g2, (const T*)cand,
                                                                    (const T*)h0, (T*)out, seq, hid);
  }
  return check_launch(OP == OP_MINGRU ? "mingru scan" : "minlstm scan");
}

template <typename T, int OP, bool LOGITS>
int launch_bwd(hipStream_t s, const void* g1, const void* g2, const void* cand, const void* h0, const void* fwd,
               const void* dy, void* d1, void* d2, void* dcand, void* dh0, int bsz, int seq, int hid) {
  constexpr int L = 8;
  const dim3 grid((hid + 63) / 64, bsz);
  if (seq >= 512) {
    constexpr int W = 16;
    linscan_bwd_kernel<T, OP, LOGITS, L, W><<<grid, 64 * W, 0, s>>>(
        (const T*)g1, (const T*)g2, (const T*)cand, (const T*)h0, (const T*)fwd, (const T*)dy, (T*)d1, (T*)d2,
        (T*)dcand, (T*)dh0, seq, hid);
  } else {
    constexpr int W = 4;
    linscan_bwd_kernel<T, OP, LOGITS, L, W><<<grid, 64 * W, 0, s>>>(
        (const T*)g1, (const T*)g2, (const T*)cand, (const T*)h0, (const T*)fwd, (const T*)dy, (T*)d1, (T*)d2,
        (T*)dcand, (T*)dh0, seq, hid);
  }
  return check_launch(OP == OP_MINGRU ? "mingru scan backward" : "minlstm scan backward");
}

template <int OP, bool LOGITS>
int fwd_dispatch(void* stream, const void* g1, const void* g2, const void* cand, const void* h0, void* out, int bsz,
                 int seq, int hid, int dtype) {
  EDF_REQUIRE(bsz > 0 && seq > 0 && hid > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(g1 && cand && out && (OP == OP_MINGRU || g2), EDF_ERR_INVALID_ARG, "null tensor pointer");
  if (dtype == EDF_BF16) return launch_fwd<bf16, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, out, bsz, seq, hid);
  return launch_fwd<float, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, out, bsz, seq, hid);
}

template <int OP, bool LOGITS>
int bwd_dispatch(void* stream, const void* g1, const void* g2, const void* cand, const void* h0, const void* fwd,
                 const void* dy, void* d1, void* d2, void* dcand, void* dh0, int bsz, int seq, int hid, int dtype) {
  EDF_REQUIRE(bsz > 0 && seq > 0 && hid > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(g1 && cand && fwd && dy && d1 && dcand && (OP == OP_MINGRU || (g2 && d2)), EDF_ERR_INVALID_ARG,
              "null tensor pointer");
  if (dtype == EDF_BF16)
    return launch_bwd<bf16, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, fwd, dy, d1, d2, dcand, dh0, bsz, seq,
                                        hid);
  return launch_bwd<float, OP, LOGITS>(as_stream(stream), g1, g2, cand, h0, fwd, dy, d1, d2, dcand, dh0, bsz, seq,
                                       hid);
}

}  // namespace
}  // namespace edf

extern "C" {

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

}  // extern "C"
