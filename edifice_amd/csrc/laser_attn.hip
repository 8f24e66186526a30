// LASER attention (reference native/cuda/fused_laser_attention.cu:1-25, fallback
// lib/edifice/cuda/fused_scan.ex:3667-3704, backward :3720-3771):
//   O = log(max(softmax(Q K^T / sqrt(d) [+ causal]) exp(V - vmax), 1e-7)) + vmax,
// vmax [B, H, 1, d] the per-column maximum of V over the sequence.
//
// Design: the attention itself is the flash kernels (flash_attn*.hip) applied to E =
// exp(V - vmax); small elementwise passes do the transforms around them.
//   forward:  E = exp(V - vmax);  O_lin = flash(Q, K, E);  O = log(max(O_lin, 1e-7)) + vmax
//   backward: with O_lin = exp(O - vmax) (the clamped value the forward took the log of) and
//             dR = dO exp(vmax - O) (reference :3751-3752), the flash backward of (Q, K, E)
//             with output O_lin and output gradient dR gives dQ, dK and dE; dV = dE E
//             (:3757-3758).  The flash backward's D = rowsum(dR O_lin) uses the clamped
//             O_lin; the reference's uses the unclamped product, which differs only where
//             every attended exp(V - vmax) is below 1e-7.
#include "edf_abi.hpp"
#include "edf_common.hpp"

namespace edf {
namespace {

constexpr float LASER_CLAMP = 1.0e-7f;

// element e of [BH][T][d] and its column's vmax [BH][d]
EDF_DEVICE long vmax_index(long e, int T, int d) { return (e / ((long)T * d)) * d + e % d; }

template <typename TT>
__global__ __launch_bounds__(256) void laser_exp_kernel(const TT* __restrict__ V, const TT* __restrict__ vmax,
                                                        TT* __restrict__ E, long n, int T, int d) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e < n) E[e] = (TT)__expf(ld(V, e) - ld(vmax, vmax_index(e, T, d)));
}

template <typename TT>
__global__ __launch_bounds__(256) void laser_log_kernel(TT* __restrict__ O, const TT* __restrict__ vmax, long n,
                                                        int T, int d) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e < n) O[e] = (TT)(__logf(fmaxf(ld(O, e), LASER_CLAMP)) + ld(vmax, vmax_index(e, T, d)));
}

// E = exp(V - vmax), O_lin = exp(O - vmax), dR = dO exp(vmax - O)
template <typename TT>
__global__ __launch_bounds__(256) void laser_bwd_pre_kernel(const TT* __restrict__ V, const TT* __restrict__ vmax,
                                                            const TT* __restrict__ O, const TT* __restrict__ dO,
                                                            TT* __restrict__ E, TT* __restrict__ Olin,
                                                            TT* __restrict__ dR, long n, int T, int d) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const float vm = ld(vmax, vmax_index(e, T, d));
  const float o = ld(O, e) - vm;
  E[e] = (TT)__expf(ld(V, e) - vm);
  Olin[e] = (TT)__expf(o);
  dR[e] = (TT)(ld(dO, e) * __expf(-o));
}

template <typename TT>
__global__ __launch_bounds__(256) void laser_dv_kernel(TT* __restrict__ dV, const TT* __restrict__ E, long n) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e < n) dV[e] = (TT)(ld(dV, e) * ld(E, e));
}

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace
}  // namespace edf

extern "C" {

size_t edf_laser_attention_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim, int dtype) {
  if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  return edf::align256((size_t)batch * num_heads * seq_len * head_dim * (dtype == EDF_BF16 ? 2 : 4));
}

int edf_fused_laser_attention(void* stream, const void* q, const void* k, const void* v, const void* v_max,
                              void* out, float* lse, void* workspace, size_t workspace_bytes, int batch,
                              int num_heads, int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(q && k && v && v_max && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf_laser_attention_workspace_bytes(batch, num_heads, seq_len, head_dim, dtype);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  const long n = (long)batch * num_heads * seq_len * head_dim;
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (dtype == EDF_BF16)
    laser_exp_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)v, (const bf16*)v_max, (bf16*)workspace, n, seq_len,
                                                head_dim);
  else
    laser_exp_kernel<float><<<grid, 256, 0, s>>>((const float*)v, (const float*)v_max, (float*)workspace, n, seq_len,
                                                 head_dim);
  if (int rc = check_launch("laser exp")) return rc;
  if (int rc = edf_fused_flash_attention(stream, q, k, workspace, out, lse, batch, num_heads, seq_len, head_dim,
                                         causal, dtype))
    return rc;
  if (dtype == EDF_BF16)
    laser_log_kernel<bf16><<<grid, 256, 0, s>>>((bf16*)out, (const bf16*)v_max, n, seq_len, head_dim);
  else
    laser_log_kernel<float><<<grid, 256, 0, s>>>((float*)out, (const float*)v_max, n, seq_len, head_dim);
  return check_launch("laser log");
}

size_t edf_laser_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim, int dtype) {
  if (batch <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  const size_t t = edf::align256((size_t)batch * num_heads * seq_len * head_dim * (dtype == EDF_BF16 ? 2 : 4));
  return 3 * t + edf::align256(edf_flash_attention_backward_workspace_bytes(batch, num_heads, seq_len, head_dim));
}

int edf_fused_laser_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* v_max,
                                       const void* out, const void* grad_out, const float* lse, void* grad_q,
                                       void* grad_k, void* grad_v, void* workspace, size_t workspace_bytes,
                                       int batch, int num_heads, int seq_len, int head_dim, int causal, int dtype) {
  using namespace edf;
  EDF_REQUIRE(batch > 0 && num_heads > 0 && seq_len > 0 && head_dim > 0, EDF_ERR_INVALID_ARG,
              "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(q && k && v && v_max && out && grad_out && lse && grad_q && grad_k && grad_v, EDF_ERR_INVALID_ARG,
              "null tensor pointer (the forward's lse is required)");
  const size_t need = edf_laser_attention_backward_workspace_bytes(batch, num_heads, seq_len, head_dim, dtype);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  hipStream_t s = as_stream(stream);
  const long n = (long)batch * num_heads * seq_len * head_dim;
  const size_t t = align256((size_t)n * (dtype == EDF_BF16 ? 2 : 4));
  char* ws = (char*)workspace;
  void *E = ws, *Olin = ws + t, *dR = ws + 2 * t, *fws = ws + 3 * t;
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (dtype == EDF_BF16)
    laser_bwd_pre_kernel<bf16><<<grid, 256, 0, s>>>((const bf16*)v, (const bf16*)v_max, (const bf16*)out,
                                                    (const bf16*)grad_out, (bf16*)E, (bf16*)Olin, (bf16*)dR, n,
                                                    seq_len, head_dim);
  else
    laser_bwd_pre_kernel<float><<<grid, 256, 0, s>>>((const float*)v, (const float*)v_max, (const float*)out,
                                                     (const float*)grad_out, (float*)E, (float*)Olin, (float*)dR, n,
                                                     seq_len, head_dim);
  if (int rc = check_launch("laser backward transforms")) return rc;
  if (int rc = edf_fused_flash_attention_backward(stream, q, k, E, Olin, dR, lse, grad_q, grad_k, grad_v, fws,
                                                  workspace_bytes - 3 * t, batch, num_heads, seq_len, head_dim,
                                                  causal, dtype))
    return rc;
  if (dtype == EDF_BF16)
    laser_dv_kernel<bf16><<<grid, 256, 0, s>>>((bf16*)grad_v, (const bf16*)E, n);
  else
    laser_dv_kernel<float><<<grid, 256, 0, s>>>((float*)grad_v, (const float*)E, n);
  return check_launch("laser dV");
}

}  // extern "C"
