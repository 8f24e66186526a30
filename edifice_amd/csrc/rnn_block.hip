// Multi-layer LSTM and GRU block scans (inference): per layer LayerNorm -> input projection
// -> recurrence with R h_{t-1} -> residual, for a stack of layers
// (native/cuda/fused_lstm_block_scan.cu, fused_gru_block_scan.cu; fallbacks
// lib/edifice/cuda/fused_scan.ex:4911-4990, 5055-5120).
//
// Per-layer weight packing (as the reference): W_x [H, G H], b_x [G H], R [H, G H], gamma [H],
// beta [H]; G = 4 (LSTM gates i, f, g, o) or 3 (GRU r, z, n).  LSTM: c = f c + i g,
// h = o tanh(c).  GRU: n = tanh(x_n + r (R h)_n), h = (1 - z) h + z n.  LayerNorm eps 1e-5.
//
// Layout: the reference walks every layer inside one sequential loop over time, one block
// per batch element streaming both weight matrices from memory at every step.  Here each
// layer runs as (1) one MFMA kernel for LayerNorm + the input projection of ALL B T rows (the
// residual add of the previous layer fused into its prologue), then (2) one small launch per
// time step for the recurrence: the step's B x G H recurrent dot products spread over H / 4
// workgroups, each holding 4 units of every gate for 8 batch rows: a workgroup stages its
// R columns (H x 4 G floats, laid out contiguously once per layer) into LDS and splits each
// dot product over a lane pair, so R is read once per step from
// L2 by the whole grid, and the cell update needs no cross-workgroup exchange; the launch
// boundary orders the steps (no grid-wide barrier inside a kernel).
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr int RNB_ROWS = 32;   // rows per projection workgroup (one 32x32 MFMA tile height)
constexpr int RNB_HMAX = 256;  // reference limit (one thread per hidden unit)
constexpr int RNB_LD = RNB_HMAX + 2;
constexpr float RNB_LN_EPS = 1.0e-5f;  // fused_lstm_block_scan.cu:113
constexpr int RNB_U = 4;   // hidden units per step workgroup
constexpr int RNB_BS = 8;  // batch rows per step workgroup

enum { RNB_LSTM = 4, RNB_GRU = 3 };  // value = number of gates

typedef float rnb_f32x16 __attribute__((ext_vector_type(16)));

// Residual + LayerNorm of 32 rows into LDS, then [32 rows] x [G H columns] on
// v_mfma_f32_32x32x2_f32 with W_x input-major: column n of row k at Wl[k G H + n].
template <typename T, int G>
__global__ __launch_bounds__(256) void rnb_proj_kernel(const T* __restrict__ input, float* __restrict__ X,
                                                       const float* __restrict__ Hprev, const T* __restrict__ Wl,
                                                       float* __restrict__ xp, long rows, int H, int first) {
  __shared__ float sn[RNB_ROWS * RNB_LD];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int GH = G * H;
  const long row0 = (long)blockIdx.x * RNB_ROWS;
  const T* gamma = Wl + 2L * H * GH + GH;
  const T* beta = gamma + H;
  for (int rr = 0; rr < RNB_ROWS / 4; ++rr) {
    const int r = w * (RNB_ROWS / 4) + rr;
    const long row = row0 + r;
    const bool rok = row < rows;
    float x[RNB_HMAX / 64];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < RNB_HMAX / 64; ++j) {
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
    for (int j = 0; j < RNB_HMAX / 64; ++j) {
      const float d = (lane + 64 * j < H) ? x[j] - mean : 0.0f;
      var = fmaf(d, d, var);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) var += __shfl_xor(var, off);
    const float inv = 1.0f / sqrtf(var / (float)H + RNB_LN_EPS);
#pragma unroll
    for (int j = 0; j < RNB_HMAX / 64; ++j) {
      const int c = lane + 64 * j;
      if (c < H) sn[r * RNB_LD + c] = fmaf((x[j] - mean) * inv, to_f32(gamma[c]), to_f32(beta[c]));
      else if (c < RNB_LD) sn[r * RNB_LD + c] = 0.0f;
    }
  }
  __syncthreads();
  // wave w takes column tiles w, w + 4, ..; lane (li, g) supplies A[row li][k = 2 kk + g] and
  // B[k][column li]; W values of 16 k steps are loaded a chunk ahead.
  const int li = lane & 31, g = lane >> 5;
  const int ntile = (GH + 31) / 32, nch = ((H + 1) / 2 + 15) / 16;
  for (int nt = w; nt < ntile; nt += 4) {
    const int n = nt * 32 + li;
    const bool nok = n < GH;
    const T* Wc = Wl + min(n, GH - 1);
    float b0[16], b1[16];
    auto ldb = [&](float* bb, int ch) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int k = 2 * (16 * ch + i) + g;
        const float v = to_f32(Wc[(long)min(k, H - 1) * GH]);
        bb[i] = (nok && k < H) ? v : 0.0f;
      }
    };
    rnb_f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    auto mm = [&](const float* bb, int ch) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(sn[li * RNB_LD + 2 * (16 * ch + i) + g], bb[i], acc, 0, 0, 0);
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
      const float bias = to_f32(Wl[(long)H * GH + n]);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const long row = row0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (row < rows) xp[row * GH + n] = acc[r] + bias;
      }
    }
  }
}

// h0[:, l, :] and c0[:, l, :] (or zeros) into the f32 step states.
template <typename T>
__global__ __launch_bounds__(256) void rnb_init_kernel(const T* __restrict__ h0, const T* __restrict__ c0,
                                                       float* __restrict__ hs0, float* __restrict__ cs, int B, int L,
                                                       int l, int H) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= B * H) return;
  const int b = e / H, u = e % H;
  const long src = ((long)b * L + l) * H + u;
  hs0[e] = h0 != nullptr ? to_f32(h0[src]) : 0.0f;
  cs[e] = c0 != nullptr ? to_f32(c0[src]) : 0.0f;
}

// One time step of one layer: gates = xp_t + R h_{t-1}, then the cell update.
// R [H, G H] -> Rt [H / U groups][G U][H] f32: each step workgroup's columns become one
// contiguous block (read with 16-byte loads every step instead of 16-byte pieces of
// H rows).  Once per layer and call.
template <typename T, int G>
__global__ __launch_bounds__(256) void rnb_rt_kernel(const T* __restrict__ R, float* __restrict__ Rt, int H) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  const int ngrp = (H + RNB_U - 1) / RNB_U;
  if (e >= (long)ngrp * G * RNB_U * H) return;
  const int k = (int)(e % H);
  const long r = e / H;
  const int gu = (int)(r % (G * RNB_U)), grp = (int)(r / (G * RNB_U));
  const int g = gu / RNB_U, u = grp * RNB_U + gu % RNB_U;
  Rt[e] = u < H ? to_f32(R[(long)k * G * H + g * H + u]) : 0.0f;
}

template <int G>
__global__ __launch_bounds__(256) void rnb_step_kernel(const float* __restrict__ Rt, const float* __restrict__ xp,
                                                       const float* __restrict__ hs0, float* __restrict__ Hs,
                                                       float* __restrict__ cs, int B, int Tn, int H, int t) {
  __shared__ float sh[RNB_BS][RNB_HMAX];
  constexpr int LDR = RNB_HMAX + 2;  // sR row stride: the lane pairs' reads hit distinct banks
  __shared__ float sR[G * RNB_U * LDR];  // this workgroup's R columns [gate, unit][k]
  __shared__ float sd[RNB_BS][G][RNB_U];
  const int tid = threadIdx.x, GH = G * H;
  const int u0 = blockIdx.x * RNB_U, b0 = blockIdx.y * RNB_BS;
  {
    const float* src = Rt + (long)blockIdx.x * G * RNB_U * H;
    for (int e = tid; e < G * RNB_U * H; e += 256) sR[(e / H) * LDR + e % H] = src[e];
  }
  for (int e = tid; e < RNB_BS * H; e += 256) {
    const int bb = e / H, k = e % H, b = b0 + bb;
    float v = 0.0f;
    if (b < B) v = t == 0 ? hs0[(long)b * H + k] : Hs[((long)b * Tn + t - 1) * H + k];
    sh[bb][k] = v;
  }
  __syncthreads();
  // each dot product is split over a lane pair (even / odd k), combined with one swizzle
  {
    const int dot = tid >> 1, half = tid & 1;
    const int bb = dot / (G * RNB_U), gu = dot % (G * RNB_U);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (dot < RNB_BS * G * RNB_U) {
      int k = half;
      for (; k + 6 < H; k += 8) {
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[m] = fmaf(sh[bb][k + 2 * m], sR[gu * LDR + k + 2 * m], acc[m]);
      }
      for (; k < H; k += 2) acc[0] = fmaf(sh[bb][k], sR[gu * LDR + k], acc[0]);
    }
    float v = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    v += __shfl_xor(v, 1);
    if (half == 0 && dot < RNB_BS * G * RNB_U) sd[bb][gu / RNB_U][gu % RNB_U] = v;
  }
  __syncthreads();
  if (tid < RNB_BS * RNB_U) {
    const int bb = tid / RNB_U, uu = tid % RNB_U, b = b0 + bb, u = u0 + uu;
    if (b >= B || u >= H) return;
    const float* x = xp + ((long)b * Tn + t) * GH + u;
    const float hp = sh[bb][u];
    float h;
    if constexpr (G == RNB_LSTM) {
      const float ig = 1.0f / (1.0f + __expf(-(x[0] + sd[bb][0][uu])));
      const float fg = 1.0f / (1.0f + __expf(-(x[H] + sd[bb][1][uu])));
      const float gg = tanhf(x[2 * H] + sd[bb][2][uu]);
      const float og = 1.0f / (1.0f + __expf(-(x[3 * H] + sd[bb][3][uu])));
      const float c = fmaf(fg, cs[(long)b * H + u], ig * gg);
      cs[(long)b * H + u] = c;
      h = og * tanhf(c);
    } else {
      const float rg = 1.0f / (1.0f + __expf(-(x[0] + sd[bb][0][uu])));
      const float zg = 1.0f / (1.0f + __expf(-(x[H] + sd[bb][1][uu])));
      const float ng = tanhf(fmaf(rg, sd[bb][2][uu], x[2 * H]));
      h = fmaf(zg, ng - hp, hp);
    }
    Hs[((long)b * Tn + t) * H + u] = h;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rnb_out_kernel(const float* __restrict__ X, const float* __restrict__ Hs,
                                                      T* __restrict__ out, long n) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e < n) st(out, e, X[e] + Hs[e]);
}

struct RnbWs {
  float *X, *Hs, *xp, *hs0, *cs, *Rt;
  size_t total;
};

inline size_t rnb_align(size_t v) { return (v + 255) & ~(size_t)255; }

inline RnbWs rnb_layout(void* base, long bth, int B, int H, int G) {
  RnbWs w{};
  size_t off = 0;
  char* p = (char*)base;
  w.X = (float*)(p + off);
  off += rnb_align((size_t)bth * 4);
  w.Hs = (float*)(p + off);
  off += rnb_align((size_t)bth * 4);
  w.xp = (float*)(p + off);
  off += rnb_align((size_t)bth * G * 4);
  w.hs0 = (float*)(p + off);
  off += rnb_align((size_t)B * H * 4);
  w.cs = (float*)(p + off);
  off += rnb_align((size_t)B * H * 4);
  w.Rt = (float*)(p + off);
  off += rnb_align((size_t)((H + RNB_U - 1) / RNB_U) * RNB_U * G * H * 4);
  w.total = off;
  return w;
}

template <typename T, int G>
int rnb_run(hipStream_t s, const void* input, const void* weights, const void* h0, const void* c0, void* out,
            const RnbWs& ws, int B, int Tn, int H, int L) {
  const long bth = (long)B * Tn * H, rows = (long)B * Tn;
  const long lstride = 2L * H * G * H + (long)G * H + 2L * H;
  const dim3 gstep((H + RNB_U - 1) / RNB_U, (B + RNB_BS - 1) / RNB_BS);
  for (int l = 0; l < L; ++l) {
    const T* Wl = (const T*)weights + l * lstride;
    rnb_proj_kernel<T, G><<<(unsigned)((rows + RNB_ROWS - 1) / RNB_ROWS), 256, 0, s>>>(
        (const T*)input, ws.X, ws.Hs, Wl, ws.xp, rows, H, l == 0 ? 1 : 0);
    if (int rc = check_launch("rnn block projection")) return rc;
    rnb_init_kernel<T><<<(B * H + 255) / 256, 256, 0, s>>>((const T*)h0, G == RNB_LSTM ? (const T*)c0 : nullptr,
                                                           ws.hs0, ws.cs, B, L, l, H);
    if (int rc = check_launch("rnn block initial state")) return rc;
    const T* Rl = Wl + (long)H * G * H + (long)G * H;
    const long nrt = (long)gstep.x * G * RNB_U * H;
    rnb_rt_kernel<T, G><<<(unsigned)((nrt + 255) / 256), 256, 0, s>>>(Rl, ws.Rt, H);
    if (int rc = check_launch("rnn block R layout")) return rc;
    for (int t = 0; t < Tn; ++t) rnb_step_kernel<G><<<gstep, 256, 0, s>>>(ws.Rt, ws.xp, ws.hs0, ws.Hs, ws.cs, B, Tn, H, t);
    if (int rc = check_launch("rnn block step")) return rc;
  }
  rnb_out_kernel<T><<<(unsigned)((bth + 255) / 256), 256, 0, s>>>(ws.X, ws.Hs, (T*)out, bth);
  return check_launch("rnn block output");
}

template <int G>
int rnb_dispatch(void* stream, const void* input, const void* weights, const void* h0, const void* c0, void* out,
                 void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden, int num_layers,
                 int dtype) {
  EDF_REQUIRE(batch > 0 && seq_len > 0 && hidden > 0 && num_layers > 0, EDF_ERR_INVALID_ARG,
              "dimensions and num_layers must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(hidden <= RNB_HMAX, EDF_ERR_UNSUPPORTED, "hidden %d unsupported (the block scans take H <= %d)", hidden,
              RNB_HMAX);
  EDF_REQUIRE((long)seq_len * hidden * G * 4 < (1L << 31), EDF_ERR_UNSUPPORTED,
              "seq_len * hidden too large (one batch row of f32 gate projections must stay below 2 GiB)");
  EDF_REQUIRE(input && weights && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const RnbWs L = rnb_layout(workspace, (long)batch * seq_len * hidden, batch, hidden, G);
  EDF_REQUIRE(workspace && workspace_bytes >= L.total, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes",
              L.total);
  if (dtype == EDF_BF16)
    return rnb_run<bf16, G>(as_stream(stream), input, weights, h0, c0, out, L, batch, seq_len, hidden, num_layers);
  return rnb_run<float, G>(as_stream(stream), input, weights, h0, c0, out, L, batch, seq_len, hidden, num_layers);
}

inline size_t rnb_ws_bytes(int batch, int seq_len, int hidden, int G) {
  if (batch <= 0 || seq_len <= 0 || hidden <= 0) return 0;
  return rnb_layout(nullptr, (long)batch * seq_len * hidden, batch, hidden, G).total;
}

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_lstm_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype) {
  (void)num_layers;
  (void)dtype;
  return edf::rnb_ws_bytes(batch, seq_len, hidden, edf::RNB_LSTM);
}

size_t edf_gru_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype) {
  (void)num_layers;
  (void)dtype;
  return edf::rnb_ws_bytes(batch, seq_len, hidden, edf::RNB_GRU);
}

int edf_fused_lstm_block_scan(void* stream, const void* input, const void* weights, const void* h0, const void* c0,
                              void* out, void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                              int num_layers, int dtype) {
  return edf::rnb_dispatch<edf::RNB_LSTM>(stream, input, weights, h0, c0, out, workspace, workspace_bytes, batch,
                                          seq_len, hidden, num_layers, dtype);
}

int edf_fused_gru_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                             void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                             int num_layers, int dtype) {
  return edf::rnb_dispatch<edf::RNB_GRU>(stream, input, weights, h0, nullptr, out, workspace, workspace_bytes, batch,
                                         seq_len, hidden, num_layers, dtype);
}

}  // extern "C"
