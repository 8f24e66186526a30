// C-ABI entry points of the delta rule (DeltaNet / GatedDeltaNet), forward and backward.
// Dispatch: the chunked MFMA kernels (delta_rule_chunk.hip) take bf16, per-head beta,
// head_dim 64 .. 128 (a multiple of 8; zero-padded to 128 inside), seq >= 64 (forward and
// backward); the exact per-step kernels
// (delta_rule_seq.hip) serve every other case.
#include "edf_abi.hpp"

namespace edf {
size_t dr_seq_backward_workspace_bytes(int batch, int heads, int seq, int d);
size_t dr_seq_context_bytes(int batch, int heads, int seq, int d);
int dr_seq_run(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
               void* out, int batch, int seq, int heads, int d, int dtype, int beta_per_head, int alpha_per_row,
               float* context);
int dr_seq_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                        const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                        void* dalpha, void* workspace, int batch, int seq, int heads, int d, int dtype,
                        int beta_per_head, int alpha_per_row, const float* context);
bool dr_chunk_eligible(int seq, int d, int dtype, int beta_per_head);
size_t dr_chunk_workspace_bytes(int batch, int seq, int heads, int d);
int dr_chunk_run(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
                 void* out, void* workspace, int batch, int seq, int heads, int d);
size_t dr_chunk_backward_workspace_bytes(int batch, int seq, int heads, int d);
size_t dr_chunk_saved_backward_workspace_bytes(int batch, int seq, int heads, int d);
int dr_chunk_saved_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                                void* dalpha, const void* fwd_workspace, void* workspace, int batch, int seq,
                                int heads, int d);
int dr_chunk_backward_run(void* stream, const void* q, const void* k, const void* v, const void* beta,
                          const void* alpha, const void* grad_out, void* dq, void* dk, void* dv, void* dbeta,
                          void* dalpha, void* workspace, int batch, int seq, int heads, int d);

namespace {
int check_dr(int batch, int seq, int heads, int d, int dtype, int beta_mode) {
  EDF_REQUIRE(batch > 0 && seq > 0 && heads > 0 && d > 0, EDF_ERR_INVALID_ARG, "dimensions must be positive");
  EDF_REQUIRE(valid_dtype(dtype), EDF_ERR_INVALID_ARG, "dtype must be 0 (f32) or 1 (bf16)");
  EDF_REQUIRE(d <= 128, EDF_ERR_UNSUPPORTED, "head_dim %d > 128 unsupported", d);
  EDF_REQUIRE(beta_mode == EDF_BETA_PER_ELEMENT || beta_mode == EDF_BETA_PER_HEAD, EDF_ERR_INVALID_ARG,
              "unknown beta mode %d", beta_mode);
  return EDF_OK;
}

int fwd(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha, void* out,
        void* workspace, size_t ws_bytes, int batch, int seq, int heads, int d, int dtype, int beta_mode) {
  int rc = check_dr(batch, seq, heads, d, dtype, beta_mode);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && beta && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const int per_head = beta_mode == EDF_BETA_PER_HEAD;
  if (dr_chunk_eligible(seq, d, dtype, per_head)) {
    // As the backward: a missing or short workspace is the caller's error, not a reason to
    // run the (exact-state, ~10x slower) per-step kernels with different numerics.
    const size_t need = dr_chunk_workspace_bytes(batch, seq, heads, d);
    EDF_REQUIRE(workspace && ws_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
    return dr_chunk_run(stream, q, k, v, beta, alpha, out, workspace, batch, seq, heads, d);
  }
  // per-step path: a workspace of edf_delta_rule_forward_context_bytes() (optional) also
  // receives the states every 16 steps, which the saved backward then reads
  const bool keep = workspace && ws_bytes >= dr_seq_context_bytes(batch, heads, seq, d);
  return dr_seq_run(stream, q, k, v, beta, alpha, out, batch, seq, heads, d, dtype, per_head, 0,
                    keep ? (float*)workspace : nullptr);
}

int bwd(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
        const void* grad_out, void* dq, void* dk, void* dv, void* dbeta, void* dalpha, void* workspace,
        size_t ws_bytes, int batch, int seq, int heads, int d, int dtype, int beta_mode) {
  int rc = check_dr(batch, seq, heads, d, dtype, beta_mode);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && beta && grad_out && dq && dk && dv && dbeta, EDF_ERR_INVALID_ARG,
              "null tensor pointer");
  const int per_head = beta_mode == EDF_BETA_PER_HEAD;
  if (dr_chunk_eligible(seq, d, dtype, per_head)) {
    const size_t need = dr_chunk_backward_workspace_bytes(batch, seq, heads, d);
    EDF_REQUIRE(workspace && ws_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
    return dr_chunk_backward_run(stream, q, k, v, beta, alpha, grad_out, dq, dk, dv, dbeta, dalpha, workspace, batch,
                                 seq, heads, d);
  }
  const size_t need = dr_seq_backward_workspace_bytes(batch, heads, seq, d);
  EDF_REQUIRE(workspace && ws_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  return dr_seq_backward_run(stream, q, k, v, beta, alpha, grad_out, dq, dk, dv, dbeta, dalpha, workspace, batch,
                             seq, heads, d, dtype, beta_mode == EDF_BETA_PER_HEAD, 0, nullptr);
}
int bwd_saved(void* stream, const void* q, const void* k, const void* v, const void* beta, const void* alpha,
              const void* grad_out, void* dq, void* dk, void* dv, void* dbeta, void* dalpha, const void* fwd_ws,
              size_t fwd_ws_bytes, void* workspace, size_t ws_bytes, int batch, int seq, int heads, int d, int dtype,
              int beta_mode) {
  int rc = check_dr(batch, seq, heads, d, dtype, beta_mode);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && beta && grad_out && dq && dk && dv && dbeta, EDF_ERR_INVALID_ARG,
              "null tensor pointer");
  EDF_REQUIRE((alpha == nullptr) == (dalpha == nullptr), EDF_ERR_INVALID_ARG,
              "alpha and grad_alpha must both be given (gated) or both be null");
  const int per_head = beta_mode == EDF_BETA_PER_HEAD;
  if (dr_chunk_eligible(seq, d, dtype, per_head)) {
    const size_t need_f = dr_chunk_workspace_bytes(batch, seq, heads, d);
    EDF_REQUIRE(fwd_ws && fwd_ws_bytes >= need_f, EDF_ERR_WORKSPACE,
                "forward workspace too small: need the %zu bytes the forward filled", need_f);
    const size_t need = dr_chunk_saved_backward_workspace_bytes(batch, seq, heads, d);
    EDF_REQUIRE(workspace && ws_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
    return dr_chunk_saved_backward_run(stream, q, k, v, beta, alpha, grad_out, dq, dk, dv, dbeta, dalpha, fwd_ws,
                                       workspace, batch, seq, heads, d);
  }
  // per-step path: the forward's stored states when its workspace held them, else the
  // backward recomputes them
  const size_t need = dr_seq_backward_workspace_bytes(batch, heads, seq, d);
  EDF_REQUIRE(workspace && ws_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  const bool saved = fwd_ws && fwd_ws_bytes >= dr_seq_context_bytes(batch, heads, seq, d);
  return dr_seq_backward_run(stream, q, k, v, beta, alpha, grad_out, dq, dk, dv, dbeta, dalpha, workspace, batch,
                             seq, heads, d, dtype, per_head, 0, saved ? (const float*)fwd_ws : nullptr);
}
}  // namespace
}  // namespace edf

extern "C" {

size_t edf_delta_rule_saved_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                                     int beta_mode) {
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  if (edf::dr_chunk_eligible(seq_len, head_dim, dtype, beta_mode == EDF_BETA_PER_HEAD))
    return edf::dr_chunk_saved_backward_workspace_bytes(batch, seq_len, num_heads, head_dim);
  return edf::dr_seq_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
}

int edf_fused_delta_rule_scan_backward_saved(void* stream, const void* q, const void* k, const void* v,
                                             const void* beta, const void* alpha, const void* grad_out,
                                             void* grad_q, void* grad_k, void* grad_v, void* grad_beta,
                                             void* grad_alpha, const void* forward_workspace,
                                             size_t forward_workspace_bytes, void* workspace, size_t workspace_bytes,
                                             int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                             int beta_mode) {
  return edf::bwd_saved(stream, q, k, v, beta, alpha, grad_out, grad_q, grad_k, grad_v, grad_beta, grad_alpha,
                        forward_workspace, forward_workspace_bytes, workspace, workspace_bytes, batch, seq_len,
                        num_heads, head_dim, dtype, beta_mode);
}

size_t edf_delta_rule_forward_context_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                            int beta_mode) {
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0 || head_dim > 128) return 0;
  if (edf::dr_chunk_eligible(seq_len, head_dim, dtype, beta_mode == EDF_BETA_PER_HEAD))
    return edf::dr_chunk_workspace_bytes(batch, seq_len, num_heads, head_dim);
  return edf::dr_seq_context_bytes(batch, num_heads, seq_len, head_dim);
}

size_t edf_delta_rule_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                      int beta_mode) {
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  if (edf::dr_chunk_eligible(seq_len, head_dim, dtype, beta_mode == EDF_BETA_PER_HEAD))
    return edf::dr_chunk_workspace_bytes(batch, seq_len, num_heads, head_dim);
  return 0;
}

size_t edf_delta_rule_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                               int beta_mode) {
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  if (edf::dr_chunk_eligible(seq_len, head_dim, dtype, beta_mode == EDF_BETA_PER_HEAD))
    return edf::dr_chunk_backward_workspace_bytes(batch, seq_len, num_heads, head_dim);
  return edf::dr_seq_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
}

int edf_fused_delta_net_scan(void* stream, const void* q, const void* k, const void* v, const void* beta, void* out,
                             void* workspace, size_t workspace_bytes, int batch, int seq_len, int num_heads,
                             int head_dim, int dtype, int beta_mode) {
  return edf::fwd(stream, q, k, v, beta, nullptr, out, workspace, workspace_bytes, batch, seq_len, num_heads,
                  head_dim, dtype, beta_mode);
}

int edf_fused_gated_delta_net_scan(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                   const void* alpha, void* out, void* workspace, size_t workspace_bytes, int batch,
                                   int seq_len, int num_heads, int head_dim, int dtype, int beta_mode) {
  EDF_REQUIRE(alpha != nullptr, EDF_ERR_INVALID_ARG, "null alpha pointer");
  return edf::fwd(stream, q, k, v, beta, alpha, out, workspace, workspace_bytes, batch, seq_len, num_heads,
                  head_dim, dtype, beta_mode);
}

int edf_fused_delta_rule_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                       const void* forward_out, const void* grad_out, void* grad_q, void* grad_k,
                                       void* grad_v, void* grad_beta, void* workspace, size_t workspace_bytes,
                                       int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                       int beta_mode) {
  (void)forward_out;  // accepted for signature parity; the reference never reads it either
  return edf::bwd(stream, q, k, v, beta, nullptr, grad_out, grad_q, grad_k, grad_v, grad_beta, nullptr, workspace,
                  workspace_bytes, batch, seq_len, num_heads, head_dim, dtype, beta_mode);
}

int edf_fused_gated_delta_net_scan_backward(void* stream, const void* q, const void* k, const void* v,
                                            const void* beta, const void* alpha, const void* forward_out,
                                            const void* grad_out, void* grad_q, void* grad_k, void* grad_v,
                                            void* grad_beta, void* grad_alpha, void* workspace,
                                            size_t workspace_bytes, int batch, int seq_len, int num_heads,
                                            int head_dim, int dtype, int beta_mode) {
  (void)forward_out;
  EDF_REQUIRE(alpha != nullptr && grad_alpha != nullptr, EDF_ERR_INVALID_ARG, "null alpha / grad_alpha pointer");
  return edf::bwd(stream, q, k, v, beta, alpha, grad_out, grad_q, grad_k, grad_v, grad_beta, grad_alpha, workspace,
                  workspace_bytes, batch, seq_len, num_heads, head_dim, dtype, beta_mode);
}

// KDA: per-row log-space decay, per-head beta; always the exact per-step kernels (the
// chunked form takes one decay per head).
size_t edf_kda_scan_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return edf::dr_seq_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
}

int edf_fused_kda_scan(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                       const void* beta, void* out, int batch, int seq_len, int num_heads, int head_dim, int dtype) {
  int rc = edf::check_dr(batch, seq_len, num_heads, head_dim, dtype, EDF_BETA_PER_HEAD);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  return edf::dr_seq_run(stream, q, k, v, beta, alpha, out, batch, seq_len, num_heads, head_dim, dtype, 1, 1,
                         nullptr);
}

int edf_fused_kda_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                const void* beta, const void* forward_out, const void* grad_out, void* grad_q,
                                void* grad_k, void* grad_v, void* grad_alpha, void* grad_beta, void* workspace,
                                size_t workspace_bytes, int batch, int seq_len, int num_heads, int head_dim,
                                int dtype) {
  (void)forward_out;
  int rc = edf::check_dr(batch, seq_len, num_heads, head_dim, dtype, EDF_BETA_PER_HEAD);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && grad_out && grad_q && grad_k && grad_v && grad_alpha && grad_beta,
              EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf::dr_seq_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  return edf::dr_seq_backward_run(stream, q, k, v, beta, alpha, grad_out, grad_q, grad_k, grad_v, grad_beta,
                                  grad_alpha, workspace, batch, seq_len, num_heads, head_dim, dtype, 1, 1, nullptr);
}

size_t edf_kda_scan_context_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype) {
  (void)dtype;
  if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_dim <= 0 || head_dim > 128) return 0;
  return edf::dr_seq_context_bytes(batch, num_heads, seq_len, head_dim);
}

int edf_fused_kda_scan_with_context(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                    const void* beta, void* out, void* context, size_t context_bytes, int batch,
                                    int seq_len, int num_heads, int head_dim, int dtype) {
  int rc = edf::check_dr(batch, seq_len, num_heads, head_dim, dtype, EDF_BETA_PER_HEAD);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && out, EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t need = edf::dr_seq_context_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(context && context_bytes >= need, EDF_ERR_WORKSPACE, "context too small: need %zu bytes", need);
  return edf::dr_seq_run(stream, q, k, v, beta, alpha, out, batch, seq_len, num_heads, head_dim, dtype, 1, 1,
                         (float*)context);
}

int edf_fused_kda_scan_backward_saved(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                      const void* beta, const void* grad_out, void* grad_q, void* grad_k,
                                      void* grad_v, void* grad_alpha, void* grad_beta, const void* context,
                                      size_t context_bytes, void* workspace, size_t workspace_bytes, int batch,
                                      int seq_len, int num_heads, int head_dim, int dtype) {
  int rc = edf::check_dr(batch, seq_len, num_heads, head_dim, dtype, EDF_BETA_PER_HEAD);
  if (rc) return rc;
  EDF_REQUIRE(q && k && v && alpha && beta && grad_out && grad_q && grad_k && grad_v && grad_alpha && grad_beta,
              EDF_ERR_INVALID_ARG, "null tensor pointer");
  const size_t needc = edf::dr_seq_context_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(context && context_bytes >= needc, EDF_ERR_WORKSPACE,
              "context too small: need the %zu bytes the forward filled", needc);
  const size_t need = edf::dr_seq_backward_workspace_bytes(batch, num_heads, seq_len, head_dim);
  EDF_REQUIRE(workspace && workspace_bytes >= need, EDF_ERR_WORKSPACE, "workspace too small: need %zu bytes", need);
  return edf::dr_seq_backward_run(stream, q, k, v, beta, alpha, grad_out, grad_q, grad_k, grad_v, grad_beta,
                                  grad_alpha, workspace, batch, seq_len, num_heads, head_dim, dtype, 1, 1,
                                  (const float*)context);
}

}  // extern "C"
