/*
 * edifice_hip.h — C ABI of the MI355X (gfx950) fused sequence-mixing kernels.
 *
 * This is the drop-in boundary that replaces Edifice's CUDA NIF bridge
 * (c_src/edifice_cuda_nif.c) and the kernel-library launch wrappers it dlsym's
 * (`fused_<op>_launch`, typedefs at c_src/edifice_cuda_nif.c:31-438).  Every
 * entry point below names the reference NIF it replaces (name/arity from the
 * NIF table at c_src/edifice_cuda_nif.c:4458-4507, Elixir stubs in
 * lib/edifice/cuda/nif.ex) and keeps that NIF's argument order and meaning.
 *
 * Conventions (differences from the reference are deliberate, see the notes):
 *   - All tensor arguments are device pointers (what the reference receives as
 *     u64 addresses from Nx.to_pointer(mode: :local)); sizes are plain ints.
 *   - Outputs are CALLER-OWNED: the reference NIF allocated the output with
 *     cudaMalloc per call; here the caller (the NIF shim, or any host) passes the
 *     output buffer(s).  Backward ops take one pointer per gradient; passing
 *     consecutive slices of one buffer reproduces the reference's concatenated
 *     [d1 | d2 | ...] output layout.
 *   - No allocation happens inside any entry point.  Ops that need scratch
 *     memory take (workspace, workspace_bytes) and export a *_workspace_bytes
 *     query.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Kernels are
 *     enqueued asynchronously; nothing synchronises the device (the reference
 *     called cudaDeviceSynchronize after every launch).
 *   - dtype: 0 = float32, 1 = bfloat16, the reference's dtype flag
 *     (lib/edifice/cuda/fused_scan.ex:39-44).  Arithmetic is always float32.
 *   - Return value: EDF_OK (0) or an EDF_ERR_* code; edf_last_error() returns
 *     a thread-local message for the last failing call on this thread
 *     (the reference returned {:error, "..."} strings).
 */
#ifndef EDIFICE_HIP_H
#define EDIFICE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EDF_ABI_VERSION 1

enum {
  EDF_OK = 0,
  EDF_ERR_INVALID_ARG = 1, /* "dimensions must be positive", bad dtype, null pointer */
  EDF_ERR_UNSUPPORTED = 2, /* shape / dtype combination this build does not implement */
  EDF_ERR_LAUNCH = 3,      /* "... kernel launch failed" */
  EDF_ERR_WORKSPACE = 4    /* workspace missing or smaller than the *_workspace_bytes query */
};

enum { EDF_F32 = 0, EDF_BF16 = 1 };

/* selective-scan discretisation of B: per-channel dt (kernel semantics,
 * native/cuda/fused_selective_scan.cu:68-90) or mean over channels
 * (Mamba block CPU semantics, lib/edifice/ssm/common.ex:402-445). */
enum { EDF_SS_DT_PER_CHANNEL = 0, EDF_SS_DT_MEAN = 1 };
/* Flag OR-ed into EDF_SS_DT_MEAN (dt-mean mode only; with the per-channel mode the entry
 * points return EDF_ERR_UNSUPPORTED) for the selective-scan entry points: dt holds the pre-activation,
 * the kernels take softplus(dt) wherever they read dt (clip, dt mean, in-range masks), and
 * grad_dt is the gradient with respect to that pre-activation.  No counterpart in the
 * reference, whose callers pass softplus(dt_proj(.)) (common.ex:366): it is for the block
 * callers, so the activation is not a pass (and a tensor) of its own. */
enum { EDF_SS_DT_SOFTPLUS = 2 };

int edf_version(void);
const char* edf_last_error(void);

/* ------------------------------------------------------------------------
 * MinGRU   h_t = (1 - z_t) h_{t-1} + z_t cand_t        tensors [B, T, H], h0 [B, H]
 * ------------------------------------------------------------------------ */

/* Replaces fused_mingru_scan/7 (gates_ptr, cand_ptr, h0_ptr, batch, seq_len,
 * hidden, dtype) — c_src/edifice_cuda_nif.c:630-704, nif.ex:29-30 — and
 * fused_mingru_scan_launch (native/cuda/fused_mingru_scan.cu:82-101).
 * z is post-sigmoid.  h0 may be NULL (zeros). */
int edf_fused_mingru_scan(void* stream, const void* z, const void* cand, const void* h0, void* out, int batch,
                          int seq_len, int hidden, int dtype);

/* Replaces fused_mingru_scan_backward/9 (z, cand, h0, fwd, dy, batch, seq_len,
 * hidden, dtype), c_src/edifice_cuda_nif.c:2508-2514; outputs dz (post-sigmoid),
 * dcand, dh0 (grad_h0 may be NULL). */
int edf_fused_mingru_scan_backward(void* stream, const void* z, const void* cand, const void* h0,
                                   const void* forward_out, const void* grad_out, void* grad_z, void* grad_cand,
                                   void* grad_h0, int batch, int seq_len, int hidden, int dtype);

/* Whole FusedScan.mingru/2 (lib/edifice/cuda/fused_scan.ex:60-74): gate logits
 * in, sigmoid fused, h0 = 0.  The backward returns d(gate logits), i.e. the chain
 * rule dz z (1 - z) of fused_scan.ex:474-480 fused into the kernel. */
int edf_mingru(void* stream, const void* gates, const void* cand, void* out, int batch, int seq_len, int hidden,
               int dtype);
int edf_mingru_backward(void* stream, const void* gates, const void* cand, const void* forward_out,
                        const void* grad_out, void* grad_gates, void* grad_cand, int batch, int seq_len, int hidden,
                        int dtype);

/* ------------------------------------------------------------------------
 * MinLSTM  c_t = f'_t c_{t-1} + i'_t cand_t,  f' = f/(f+i+1e-6), i' = i/(f+i+1e-6)
 * ------------------------------------------------------------------------ */

/* Replaces fused_minlstm_scan/8 (forget, input, cand, h0, batch, seq_len, hidden,
 * dtype), nif.ex:33-34; gates post-sigmoid, h0 may be NULL. */
int edf_fused_minlstm_scan(void* stream, const void* f, const void* i, const void* cand, const void* h0, void* out,
                           int batch, int seq_len, int hidden, int dtype);

/* Replaces fused_minlstm_scan_backward/10; outputs df, di (post-sigmoid),
 * dcand, dh0 (grad_h0 may be NULL). */
int edf_fused_minlstm_scan_backward(void* stream, const void* f, const void* i, const void* cand, const void* h0,
                                    const void* forward_out, const void* grad_out, void* grad_f, void* grad_i,
                                    void* grad_cand, void* grad_h0, int batch, int seq_len, int hidden, int dtype);

/* Whole FusedScan.minlstm/3 (fused_scan.ex:77-91) with fused sigmoids; backward
 * returns gradients w.r.t. the gate logits (fused_scan.ex:502-511). */
int edf_minlstm(void* stream, const void* forget_gates, const void* input_gates, const void* cand, void* out,
                int batch, int seq_len, int hidden, int dtype);
int edf_minlstm_backward(void* stream, const void* forget_gates, const void* input_gates, const void* cand,
                         const void* forward_out, const void* grad_out, void* grad_forget, void* grad_input,
                         void* grad_cand, int batch, int seq_len, int hidden, int dtype);

/* ------------------------------------------------------------------------
 * Generic linear scan  h_t = a_t h_{t-1} + b_t   (a, b precomputed by the caller)
 * ------------------------------------------------------------------------ */

/* Replaces fused_linear_scan/7 (a_ptr, b_ptr, h0_ptr, batch, seq_len, hidden, dtype),
 * c_src/edifice_cuda_nif.c:891-899 -> fused_linear_scan_launch
 * (native/cuda/fused_linear_scan.cu:77-95); h0 may be NULL (zeros, as
 * fused_scan.ex:2950-2957 passes). */
int edf_fused_linear_scan(void* stream, const void* a, const void* b, const void* h0, void* out, int batch,
                          int seq_len, int hidden, int dtype);

/* Replaces fused_linear_scan_backward/8 (a_ptr, h0_ptr, fwd_ptr, grad_ptr, batch,
 * seq_len, hidden, dtype), c_src/edifice_cuda_nif.c:2414-2474, whose single output
 * buffer [grad_a | grad_b | grad_h0] becomes three pointers here (grad_h0 may be NULL);
 * da = dh h_{t-1}, db = dh, dh0 = a_0 dh_0 (fused_linear_scan_backward.cu:42-80). */
int edf_fused_linear_scan_backward(void* stream, const void* a, const void* h0, const void* forward_out,
                                   const void* grad_out, void* grad_a, void* grad_b, void* grad_h0, int batch,
                                   int seq_len, int hidden, int dtype);

/* ------------------------------------------------------------------------
 * Multi-layer MinGRU block, inference: per layer LayerNorm -> gate / candidate
 * projections -> sigmoid -> MinGRU scan -> residual
 * ------------------------------------------------------------------------ */

/* Replaces fused_mingru_block_scan/8 (input_ptr, weights_ptr, h0_ptr, batch, seq_len,
 * hidden, num_layers, dtype), lib/edifice/cuda/nif.ex:127 -> fused_mingru_block_scan_launch
 * (native/cuda/fused_mingru_block_scan.cu:45-140, 160-180).  input, out [B, T, H];
 * weights packed per layer as W_z [H][H] (input-major), b_z [H], W_h [H][H], b_h [H],
 * gamma [H], beta [H] in the I/O dtype (lib/edifice/recurrent/min_gru.ex:217-241);
 * h0 [B, num_layers, H] or NULL (zeros); H <= 256.  Unlike the reference launch it takes
 * a caller-provided workspace of edf_mingru_block_workspace_bytes() bytes (f32
 * activations between the layers). */
size_t edf_mingru_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype);
int edf_fused_mingru_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                                void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                                int num_layers, int dtype);

/* Replaces fused_minlstm_block_scan/8, lib/edifice/cuda/nif.ex:131 ->
 * fused_minlstm_block_scan_launch (native/cuda/fused_minlstm_block_scan.cu:59-140): as the
 * MinGRU block with three projections f, i, c per layer (packing W_f, b_f, W_i, b_i, W_h,
 * b_h, gamma, beta) and h = f' h + i' c, f' = s(f) / (s(f) + s(i) + 1e-6). */
size_t edf_minlstm_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype);
int edf_fused_minlstm_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                                 void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                                 int num_layers, int dtype);

/* Replaces fused_linear_block_scan/8, lib/edifice/cuda/nif.ex:135 ->
 * fused_linear_block_scan_launch (native/cuda/fused_linear_block_scan.cu:100-126): two
 * projections a, b per layer (packing W_a, b_a, W_b, b_b, gamma, beta), no activation,
 * h = a h + b. */
size_t edf_linear_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype);
int edf_fused_linear_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                                void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                                int num_layers, int dtype);

/* Multi-layer LSTM block scan (inference).  Replaces fused_lstm_block_scan/9 (input,
 * weights, h0, c0, batch, seq, hidden, layers, dtype), lib/edifice/cuda/nif.ex:139 ->
 * native/cuda/fused_lstm_block_scan.cu (fallback fused_scan.ex:4911-4990).  Per-layer
 * packing W_x [H, 4H] (gates i, f, g, o), b_x [4H], R [H, 4H], gamma [H], beta [H]; h0, c0
 * [B, L, H] or NULL (zeros); H <= 256; workspace edf_lstm_block_workspace_bytes() bytes.
 * The recurrence (LSTM and GRU) runs as one persistent launch when the device can hold the
 * whole grid at once (a grid barrier in the workspace between step diagonals), else as one
 * launch per diagonal; EDF_RNN_BLOCK_PER_STEP=1 in the environment forces the latter. */
int edf_fused_lstm_block_scan(void* stream, const void* input, const void* weights, const void* h0, const void* c0,
                              void* out, void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                              int num_layers, int dtype);
size_t edf_lstm_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype);

/* Multi-layer GRU block scan (inference).  Replaces fused_gru_block_scan/8 (input, weights,
 * h0, batch, seq, hidden, layers, dtype), nif.ex:143 -> native/cuda/fused_gru_block_scan.cu
 * (fallback fused_scan.ex:5055-5120); packing W_x [H, 3H] (gates r, z, n), b_x [3H],
 * R [H, 3H], gamma, beta; workspace edf_gru_block_workspace_bytes() bytes. */
int edf_fused_gru_block_scan(void* stream, const void* input, const void* weights, const void* h0, void* out,
                             void* workspace, size_t workspace_bytes, int batch, int seq_len, int hidden,
                             int num_layers, int dtype);
size_t edf_gru_block_workspace_bytes(int batch, int seq_len, int hidden, int num_layers, int dtype);

/* Status of the last LSTM / GRU block call on `workspace` (no reference counterpart: the
 * reference kernels have no grid barrier).  Waits for `stream`, then returns EDF_OK, or
 * EDF_ERR_LAUNCH when the persistent kernel's bounded grid-barrier wait gave up (it cannot
 * under a cooperative launch; were it to, the kernel still finishes and writes NaN as the
 * output).  Same shape arguments as the call it checks.  EDF_RNN_BLOCK_PRESET_ABORT=1 in the
 * environment makes every call start in that state (a test hook for this path). */
int edf_lstm_block_status(void* stream, const void* workspace, size_t workspace_bytes, int batch, int seq_len,
                          int hidden, int num_layers);
int edf_gru_block_status(void* stream, const void* workspace, size_t workspace_bytes, int batch, int seq_len,
                         int hidden, int num_layers);

/* ------------------------------------------------------------------------
 * Mamba selective scan
 *   x, dt, z, out, grad_x, grad_dt, grad_z: [B, T, D] in io_dtype
 *   A [D, N], B, C [B, T, N], D [D]: param_dtype; grad_A/B/C/D: float32
 *   dt is clipped to [1e-3, 0.1]; ddt is zero where dt was clipped.
 * ------------------------------------------------------------------------ */

/* Replaces fused_selective_scan/10 (x, dt, A, B, C, batch, seq_len, hidden,
 * state, dtype), c_src/edifice_cuda_nif.c:1470-1503, and
 * fused_selective_scan_launch (native/cuda/fused_selective_scan.cu:105-123).
 * Extensions: per-tensor dtypes (io vs param), optional D skip (NULL = none)
 * and silu(z) gate (NULL = none), and `states`, an optional float32 buffer of
 * edf_selective_scan_states_bytes() that receives checkpoints for the backward.
 * state: 1..32, as the reference (fused_selective_scan.cu:57-76 keeps h_state[32]). */
int edf_fused_selective_scan(void* stream, const void* x, const void* dt, const void* A, const void* B, const void* C,
                             const void* D, const void* z, void* out, void* states, void* workspace,
                             size_t workspace_bytes, int batch, int seq_len, int hidden, int state, int io_dtype,
                             int param_dtype, int mode);
size_t edf_selective_scan_states_bytes(int batch, int seq_len, int hidden, int state);
size_t edf_selective_scan_workspace_bytes(int batch, int seq_len, int hidden, int state, int mode);

/* Replaces fused_selective_scan_backward/11 (x, dt, A, B, C, dy, batch, seq_len,
 * hidden, state, dtype), whose concatenated output was [dx | ddt | dB | dC]
 * (native/cuda/fused_selective_scan_backward.cu:198-238).  Adds grad_A, grad_D,
 * grad_z (each may be NULL).  `states` may be NULL: the checkpoints are then
 * recomputed into the workspace.  state: 1..32, as the reference (MAX_STATE 32,
 * fused_selective_scan_backward.cu:59). */
int edf_fused_selective_scan_backward(void* stream, const void* x, const void* dt, const void* A, const void* B,
                                      const void* C, const void* D, const void* z, const void* grad_out,
                                      const void* states, void* grad_x, void* grad_dt, void* grad_A, void* grad_B,
                                      void* grad_C, void* grad_D, void* grad_z, void* workspace,
                                      size_t workspace_bytes, int batch, int seq_len, int hidden, int state,
                                      int io_dtype, int param_dtype, int mode);
size_t edf_selective_scan_backward_workspace_bytes(int batch, int seq_len, int hidden, int state, int mode,
                                                   int have_states);

/* KDA (Kimi delta attention): the delta rule with a log-space decay per value row,
 * S_g = diag(exp(alpha_t)) S, and a per-head beta.  Replaces fused_kda_scan/10 (q, k, v,
 * alpha [B,T,H,d], beta [B,T,H], batch, seq, heads, head_dim, dtype), lib/edifice/cuda/
 * nif.ex:90 -> native/cuda/fused_kda_scan.cu (semantics fused_scan.ex:2632-2665); head_dim
 * <= 128; no workspace for the forward. */
int edf_fused_kda_scan(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                       const void* beta, void* out, int batch, int seq_len, int num_heads, int head_dim, int dtype);

/* Replaces fused_kda_scan_backward/12 (q, k, v, alpha, beta, fwd, grad, ...), nif.ex:206:
 * dq, dk, dv, d alpha [B,T,H,d] (log space), d beta [B,T,H]; workspace
 * edf_kda_scan_backward_workspace_bytes() bytes. */
int edf_fused_kda_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                const void* beta, const void* forward_out, const void* grad_out, void* grad_q,
                                void* grad_k, void* grad_v, void* grad_alpha, void* grad_beta, void* workspace,
                                size_t workspace_bytes, int batch, int seq_len, int num_heads, int head_dim,
                                int dtype);

/* No reference counterpart (its backward re-runs a checkpointing forward): a training KDA
 * forward that also keeps the states every 16 steps in a caller-kept context of
 * edf_kda_scan_context_bytes() bytes (one pass writes out and the states), and the backward
 * from that context (unchanged since), which then skips its forward re-run; gradients
 * bit-identical to edf_fused_kda_scan_backward, workspace edf_kda_scan_backward_workspace_bytes(). */
size_t edf_kda_scan_context_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype);
int edf_fused_kda_scan_with_context(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                    const void* beta, void* out, void* context, size_t context_bytes, int batch,
                                    int seq_len, int num_heads, int head_dim, int dtype);
int edf_fused_kda_scan_backward_saved(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                      const void* beta, const void* grad_out, void* grad_q, void* grad_k,
                                      void* grad_v, void* grad_alpha, void* grad_beta, const void* context,
                                      size_t context_bytes, void* workspace, size_t workspace_bytes, int batch,
                                      int seq_len, int num_heads, int head_dim, int dtype);
size_t edf_kda_scan_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype);

/* DeltaProduct: n_h delta-rule sub-steps per token on L2-normalised keys, then the RMS-
 * normalised contraction of the state with q over its value rows.  Replaces
 * fused_delta_product_scan/10 (q [B,T,H,d], k, v [B,T,n_h,H,d], beta [B,T,n_h,H], batch,
 * seq, n_h, heads, head_dim, dtype), lib/edifice/cuda/nif.ex:66 ->
 * native/cuda/fused_delta_product_scan.cu (fallback delta_product.ex:287-347); head_dim
 * <= 128; workspace edf_delta_product_workspace_bytes() bytes (row-block partial outputs). */
int edf_fused_delta_product_scan(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                 void* out, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                 int num_householder, int num_heads, int head_dim, int dtype);
size_t edf_delta_product_workspace_bytes(int batch, int seq_len, int num_householder, int num_heads, int head_dim,
                                         int dtype);

/* Replaces fused_delta_product_scan_backward/12 (q, k, v, beta, fwd, grad, ...), nif.ex:193
 * -> native/cuda/fused_delta_product_scan_backward.cu: dq [B,T,H,d], dk, dv [B,T,n_h,H,d],
 * d beta [B,T,n_h,H]; workspace edf_delta_product_backward_workspace_bytes() bytes.  The
 * reference kernel stops at seq 512 (MAX_SEQ_LEN); this one takes any length. */
int edf_fused_delta_product_scan_backward(void* stream, const void* q, const void* k, const void* v,
                                          const void* beta, const void* forward_out, const void* grad_out,
                                          void* grad_q, void* grad_k, void* grad_v, void* grad_beta, void* workspace,
                                          size_t workspace_bytes, int batch, int seq_len, int num_householder,
                                          int num_heads, int head_dim, int dtype);
size_t edf_delta_product_backward_workspace_bytes(int batch, int seq_len, int num_householder, int num_heads,
                                                  int head_dim, int dtype);

/* No reference counterpart (its backward re-runs the forward): a training forward that also
 * keeps, in a caller-kept context of edf_delta_product_context_bytes() bytes, the row-block
 * output partials and the state every 16 sub-steps (one pass writes out and both), and the
 * backward from that context (unchanged since), which then skips its forward re-run;
 * gradients bit-identical to edf_fused_delta_product_scan_backward, workspace
 * edf_delta_product_backward_workspace_bytes(). */
size_t edf_delta_product_context_bytes(int batch, int seq_len, int num_householder, int num_heads, int head_dim,
                                       int dtype);
int edf_fused_delta_product_scan_with_context(void* stream, const void* q, const void* k, const void* v,
                                              const void* beta, void* out, void* context, size_t context_bytes,
                                              int batch, int seq_len, int num_householder, int num_heads,
                                              int head_dim, int dtype);
int edf_fused_delta_product_scan_backward_saved(void* stream, const void* q, const void* k, const void* v,
                                                const void* beta, const void* grad_out, void* grad_q, void* grad_k,
                                                void* grad_v, void* grad_beta, const void* context,
                                                size_t context_bytes, void* workspace, size_t workspace_bytes,
                                                int batch, int seq_len, int num_householder, int num_heads,
                                                int head_dim, int dtype);

/* RLA / RDN (residual linear attention): base state S and residual state R, per-head
 * alpha, beta, gamma [B,T,H]; variant 0 = RLA, 1 = RDN; clip_threshold >= 0 bounds the
 * residual error.  Replaces fused_rla_scan/13 (q, k, v, alpha, beta, gamma, batch, seq,
 * heads, head_dim, variant, clip, dtype), lib/edifice/cuda/nif.ex:94 ->
 * native/cuda/fused_rla_scan.cu (fallback fused_scan.ex:2692-2768); head_dim <= 128; no
 * workspace for the forward. */
int edf_fused_rla_scan(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                       const void* beta, const void* gamma, void* out, int batch, int seq_len, int num_heads,
                       int head_dim, int variant, float clip_threshold, int dtype);

/* Replaces fused_rla_scan_backward/15 (q, k, v, alpha, beta, gamma, fwd, grad, ...),
 * nif.ex:210 -> native/cuda/fused_rla_scan_backward.cu: dq, dk, dv [B,T,H,d], d alpha,
 * d beta, d gamma [B,T,H]; workspace edf_rla_scan_backward_workspace_bytes() bytes.  The
 * reference kernel keeps per-step history in fixed arrays (MAX_SEQ_LEN); this one takes
 * any length. */
int edf_fused_rla_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                const void* beta, const void* gamma, const void* forward_out, const void* grad_out,
                                void* grad_q, void* grad_k, void* grad_v, void* grad_alpha, void* grad_beta,
                                void* grad_gamma, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                int num_heads, int head_dim, int variant, float clip_threshold, int dtype);
size_t edf_rla_scan_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype);

/* No reference counterpart (its backward re-runs a checkpointing forward): a training
 * forward that also keeps both states every 8 steps in a caller-kept context of
 * edf_rla_scan_context_bytes() bytes (one pass writes out and the states), and the backward
 * from that context (unchanged since), which then skips its forward re-run; gradients
 * bit-identical to edf_fused_rla_scan_backward, workspace edf_rla_scan_backward_workspace_bytes(). */
size_t edf_rla_scan_context_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype);
int edf_fused_rla_scan_with_context(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                    const void* beta, const void* gamma, void* out, void* context,
                                    size_t context_bytes, int batch, int seq_len, int num_heads, int head_dim,
                                    int variant, float clip_threshold, int dtype);
int edf_fused_rla_scan_backward_saved(void* stream, const void* q, const void* k, const void* v, const void* alpha,
                                      const void* beta, const void* gamma, const void* grad_out, void* grad_q,
                                      void* grad_k, void* grad_v, void* grad_alpha, void* grad_beta,
                                      void* grad_gamma, const void* context, size_t context_bytes, void* workspace,
                                      size_t workspace_bytes, int batch, int seq_len, int num_heads, int head_dim,
                                      int variant, float clip_threshold, int dtype);

/* TTT-Linear: an inner linear model W [B, D, D] (initial w0) updated every step by one
 * LayerNorm-ed reconstruction step; q, k, v, eta [B,T,D], ln_g, ln_b [D].  Replaces
 * fused_ttt_scan/11 (q, k, v, eta, w0, ln_g, ln_b, batch, seq, inner, dtype),
 * lib/edifice/cuda/nif.ex:82 -> native/cuda/fused_ttt_scan.cu (fallback ttt.ex:369-404);
 * inner_size <= 128; no workspace for the forward. */
int edf_fused_ttt_scan(void* stream, const void* q, const void* k, const void* v, const void* eta, const void* w0,
                       const void* ln_g, const void* ln_b, void* out, int batch, int seq_len, int inner_size,
                       int dtype);

/* Replaces fused_ttt_scan_backward/12 (q, k, v, eta, w0, ln_g, ln_b, grad, ...), nif.ex:214
 * -> native/cuda/fused_ttt_scan_backward.cu: dq, dk, dv, d eta [B,T,D], d w0 [B,D,D],
 * d ln_g, d ln_b [D]; workspace edf_ttt_scan_backward_workspace_bytes() bytes. */
int edf_fused_ttt_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* eta,
                                const void* w0, const void* ln_g, const void* ln_b, const void* grad_out,
                                void* grad_q, void* grad_k, void* grad_v, void* grad_eta, void* grad_w0,
                                void* grad_ln_g, void* grad_ln_b, void* workspace, size_t workspace_bytes,
                                int batch, int seq_len, int inner_size, int dtype);
size_t edf_ttt_scan_backward_workspace_bytes(int batch, int seq_len, int inner_size, int dtype);

/* No reference counterpart (its backward re-runs the forward): a training forward that also
 * records, into a caller-kept context of edf_ttt_scan_context_bytes() bytes, what the
 * backward needs (W every 8 steps, x_hat, err and 1/sigma per step; one pass writes out and
 * the records), and the backward from that context (unchanged since), which then skips its
 * own recording forward; gradients bit-identical to edf_fused_ttt_scan_backward, workspace
 * edf_ttt_scan_backward_workspace_bytes(). */
size_t edf_ttt_scan_context_bytes(int batch, int seq_len, int inner_size, int dtype);
int edf_fused_ttt_scan_with_context(void* stream, const void* q, const void* k, const void* v, const void* eta,
                                    const void* w0, const void* ln_g, const void* ln_b, void* out, void* context,
                                    size_t context_bytes, int batch, int seq_len, int inner_size, int dtype);
int edf_fused_ttt_scan_backward_saved(void* stream, const void* q, const void* k, const void* v, const void* eta,
                                      const void* w0, const void* ln_g, const void* ln_b, const void* grad_out,
                                      void* grad_q, void* grad_k, void* grad_v, void* grad_eta, void* grad_w0,
                                      void* grad_ln_g, void* grad_ln_b, const void* context, size_t context_bytes,
                                      void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                      int inner_size, int dtype);

/* ------------------------------------------------------------------------
 * Flash attention   O = softmax(Q K^T / sqrt(d) [+ causal -inf]) V
 *   q, k, v, out, grads: [B, H, T, d] in dtype; lse: float32 [B, H, T] (natural log)
 * ------------------------------------------------------------------------ */

/* Replaces fused_flash_attention/9 (q, k, v, batch, heads, seq_len, head_dim,
 * causal, dtype), nif.ex fused_flash_attention, and fused_flash_attention_launch
 * (native/cuda/fused_flash_attention.cu:168-191).  Extension: `lse` (may be NULL)
 * receives the row log-sum-exp for the backward.  bf16 with head_dim 32, 64 or 128
 * runs on MFMA; other head_dim (<= 256) and float32 run a wave-per-row kernel. */
int edf_fused_flash_attention(void* stream, const void* q, const void* k, const void* v, void* out, float* lse,
                              int batch, int num_heads, int seq_len, int head_dim, int causal, int dtype);

/* Replaces fused_flash_attention_backward/11 (q, k, v, out, dO, batch, heads,
 * seq_len, head_dim, causal, dtype), whose concatenated output was [dQ | dK | dV]
 * (native/cuda/fused_flash_attention_backward.cu:355-408; that code cudaMalloc'ed D
 * and lse per call).  Takes the forward's lse; the workspace holds
 * D = rowsum(dO * O), edf_flash_attention_backward_workspace_bytes() bytes. */
int edf_fused_flash_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* out,
                                       const void* grad_out, const float* lse, void* grad_q, void* grad_k,
                                       void* grad_v, void* workspace, size_t workspace_bytes, int batch,
                                       int num_heads, int seq_len, int head_dim, int causal, int dtype);
size_t edf_flash_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * flash-attention backward above with no workspace argument.  D lives in a library-owned
 * device array of EDF_FA_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds
 * until the process ends, so batch * num_heads * seq_len must not exceed
 * EDF_FA_NOALLOC_SCRATCH_BYTES / 4 (EDF_ERR_UNSUPPORTED otherwise).  Nothing is allocated
 * per call.  All calls on one GPU share that array: calls that overlap in time on one GPU
 * (e.g. on two streams) race and must be serialised by the caller.  Results are identical to
 * edf_fused_flash_attention_backward's. */
#define EDF_FA_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int edf_fused_flash_attention_backward_noalloc(void* stream, const void* q, const void* k, const void* v,
                                               const void* out, const void* grad_out, const float* lse,
                                               void* grad_q, void* grad_k, void* grad_v, int batch, int num_heads,
                                               int seq_len, int head_dim, int causal, int dtype);

/* FoX (forgetting) attention, always causal: scores QK^T/sqrt(d) + (cs_i - cs_j) with
 * cs [B, H, T] the cumulative log forget gate.  Replaces fused_fox_attention/9 (q, k, v,
 * cs, batch, heads, seq, head_dim, dtype), lib/edifice/cuda/nif.ex:106 ->
 * native/cuda/fused_fox_attention.cu (semantics fused_scan.ex:3860-3905); lse (may be NULL)
 * is the forward's per-row log-sum-exp, required by the backward. */
int edf_fused_fox_attention(void* stream, const void* q, const void* k, const void* v, const void* cs, void* out,
                            float* lse, int batch, int num_heads, int seq_len, int head_dim, int dtype);

/* Replaces fused_fox_attention_backward/11 (q, k, v, cs, o, grad_o, ...), nif.ex:227 ->
 * native/cuda/fused_fox_attention_backward.cu: dq, dk, dv and d cs = sum_j dS_ij -
 * sum_j dS_ji; workspace edf_fox_attention_backward_workspace_bytes() bytes. */
int edf_fused_fox_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* cs,
                                     const void* out, const void* grad_out, const float* lse, void* grad_q,
                                     void* grad_k, void* grad_v, void* grad_cs, void* workspace,
                                     size_t workspace_bytes, int batch, int num_heads, int seq_len, int head_dim,
                                     int dtype);
size_t edf_fox_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim);

/* LASER attention: O = log(max(softmax(Q K^T / sqrt(d)) exp(V - vmax), 1e-7)) + vmax, vmax
 * [B, H, 1, d] the per-column max of V.  Replaces fused_laser_attention/10 (q, k, v, v_max,
 * batch, heads, seq, head_dim, causal, dtype), lib/edifice/cuda/nif.ex:102 ->
 * native/cuda/fused_laser_attention.cu (semantics fused_scan.ex:3667-3704); lse (may be
 * NULL) is needed by the backward; workspace edf_laser_attention_workspace_bytes(). */
size_t edf_laser_attention_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim, int dtype);
int edf_fused_laser_attention(void* stream, const void* q, const void* k, const void* v, const void* v_max,
                              void* out, float* lse, void* workspace, size_t workspace_bytes, int batch,
                              int num_heads, int seq_len, int head_dim, int causal, int dtype);

/* Replaces fused_laser_attention_backward/12 (q, k, v, vmax, o, grad_o, ...), nif.ex:223:
 * dq, dk, dv (vmax held constant, as fused_scan.ex:3720-3771). */
size_t edf_laser_attention_backward_workspace_bytes(int batch, int num_heads, int seq_len, int head_dim, int dtype);
int edf_fused_laser_attention_backward(void* stream, const void* q, const void* k, const void* v, const void* v_max,
                                       const void* out, const void* grad_out, const float* lse, void* grad_q,
                                       void* grad_k, void* grad_v, void* workspace, size_t workspace_bytes,
                                       int batch, int num_heads, int seq_len, int head_dim, int causal, int dtype);

/* ------------------------------------------------------------------------
 * Delta rule (DeltaNet / GatedDeltaNet)
 *   q, k, v, out, grads: [B, T, H, d] in dtype (k L2-normalised by the caller, no
 *   q scaling); S is [d x d] per (b, h):
 *     S_g = alpha_t S;  S = S_g + diag(beta_t)(v_t - S_g k_t) k_t^T;  o_t = S q_t
 *   beta: [B, T, H, d] (EDF_BETA_PER_ELEMENT, the reference's layout) or [B, T, H]
 *   (EDF_BETA_PER_HEAD); alpha: [B, T, H] (gated only).  head_dim <= 128.
 *   bf16 + per-head beta + head_dim 64..128 (a multiple of 8; zero-padded to 128 inside the
 *   kernels) + seq_len >= 64 runs the chunked MFMA kernels,
 *   forward and backward, and then requires the workspace the *_workspace_bytes queries
 *   return (EDF_ERR_WORKSPACE when it is missing or short; the forward query returns 0
 *   for every other case); everything else runs the exact per-step kernels.
 * ------------------------------------------------------------------------ */
enum { EDF_BETA_PER_ELEMENT = 0, EDF_BETA_PER_HEAD = 1 };

size_t edf_delta_rule_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                      int beta_mode);
size_t edf_delta_rule_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                               int beta_mode);

/* Replaces fused_delta_net_scan/9 (q, k, v, beta, batch, seq_len, heads, head_dim,
 * dtype), c_src/edifice_cuda_nif.c, and fused_delta_net_scan_launch
 * (native/cuda/fused_delta_rule_scan.cu:234-245). */
int edf_fused_delta_net_scan(void* stream, const void* q, const void* k, const void* v, const void* beta, void* out,
                             void* workspace, size_t workspace_bytes, int batch, int seq_len, int num_heads,
                             int head_dim, int dtype, int beta_mode);

/* Replaces fused_gated_delta_net_scan/10 (+ alpha) and
 * fused_gated_delta_net_scan_launch (native/cuda/fused_delta_rule_scan.cu:247-258). */
int edf_fused_gated_delta_net_scan(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                   const void* alpha, void* out, void* workspace, size_t workspace_bytes, int batch,
                                   int seq_len, int num_heads, int head_dim, int dtype, int beta_mode);

/* Replaces fused_delta_rule_scan_backward/11 (q, k, v, beta, fwd, dy, ...), whose
 * concatenated output was [dq | dk | dv | dbeta]
 * (native/cuda/fused_delta_rule_scan_backward.cu:277-320).  grad_beta has beta's
 * layout.  forward_out is accepted and unused, as in the reference. */
int edf_fused_delta_rule_scan_backward(void* stream, const void* q, const void* k, const void* v, const void* beta,
                                       const void* forward_out, const void* grad_out, void* grad_q, void* grad_k,
                                       void* grad_v, void* grad_beta, void* workspace, size_t workspace_bytes,
                                       int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                       int beta_mode);

/* Replaces fused_gated_delta_net_scan_backward/12, output [dq | dk | dv | dbeta | dalpha]
 * (native/cuda/fused_gated_delta_net_scan_backward.cu:348-390). */
int edf_fused_gated_delta_net_scan_backward(void* stream, const void* q, const void* k, const void* v,
                                            const void* beta, const void* alpha, const void* forward_out,
                                            const void* grad_out, void* grad_q, void* grad_k, void* grad_v,
                                            void* grad_beta, void* grad_alpha, void* workspace,
                                            size_t workspace_bytes, int batch, int seq_len, int num_heads,
                                            int head_dim, int dtype, int beta_mode);

/* No reference counterpart (the reference backward recomputes everything from its inputs):
 * the backward of DeltaNet (alpha and grad_alpha NULL) or GatedDeltaNet from the per-chunk
 * context its forward call left in `forward_workspace` (the workspace of the forward with the
 * same q, k, v, beta, alpha, unchanged since).  On the chunked path (see above) this skips
 * the forward's recomputation; `workspace` needs
 * edf_delta_rule_saved_backward_workspace_bytes() bytes.  On the per-step path the forward's
 * workspace is optional (edf_delta_rule_workspace_bytes() is 0 there); a forward workspace of
 * edf_delta_rule_forward_context_bytes() also receives the states every 16 steps, which this
 * backward then reads instead of recomputing them (bit-identical gradients); with a smaller
 * or NULL forward_workspace it recomputes, as edf_fused_gated_delta_net_scan_backward does.
 * edf_delta_rule_forward_context_bytes() is the chunked path's forward workspace on that
 * path and the per-step states otherwise: the forward workspace a training caller
 * allocates for the saved backward. */
size_t edf_delta_rule_forward_context_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                            int beta_mode);
size_t edf_delta_rule_saved_backward_workspace_bytes(int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                                     int beta_mode);
int edf_fused_delta_rule_scan_backward_saved(void* stream, const void* q, const void* k, const void* v,
                                             const void* beta, const void* alpha, const void* grad_out,
                                             void* grad_q, void* grad_k, void* grad_v, void* grad_beta,
                                             void* grad_alpha, const void* forward_workspace,
                                             size_t forward_workspace_bytes, void* workspace, size_t workspace_bytes,
                                             int batch, int seq_len, int num_heads, int head_dim, int dtype,
                                             int beta_mode);

/* ------------------------------------------------------------------------
 * Causal depthwise conv1d + bias + SiLU (block callers)
 *   y[b, t, c] = silu(bias[c] + sum_{j < K} w[c, j] x[b, t - (K - 1) + j, c]), x = 0 before
 *   t = 0; x [B, T, C] with row stride x_row_stride (>= C) elements, so a column slice of a
 *   wider projection output needs no copy; out / grad_out / grad_x [B, T, C] contiguous;
 *   weight [C, K] (nn.Conv1d's [C, 1, K]), bias [C] or NULL; all in dtype; 1 <= K <= 8.
 *   Replaces the Mamba block's x-branch convolution and its activation,
 *   Axon.conv(..., padding: [{K - 1, 0}], feature_group_size: C) + Axon.activation(:silu)
 *   (lib/edifice/ssm/common.ex:251-252, 298-309), and the GatedDeltaNet short convolution
 *   (lib/edifice/recurrent/gated_delta_net.ex:239-245).
 * ------------------------------------------------------------------------ */
int edf_causal_conv1d_silu(void* stream, const void* x, int x_row_stride, const void* weight, const void* bias,
                           void* out, int batch, int seq_len, int channels, int kernel_size, int dtype);

/* Gradients of edf_causal_conv1d_silu (the reference takes them by autodiff of the Axon
 * layers): grad_x [B, T, C], grad_weight [C, K] and grad_bias [C] (either may be NULL),
 * summed in a fixed order; workspace edf_causal_conv1d_silu_backward_workspace_bytes(). */
size_t edf_causal_conv1d_silu_backward_workspace_bytes(int batch, int seq_len, int channels, int kernel_size);
int edf_causal_conv1d_silu_backward(void* stream, const void* x, int x_row_stride, const void* weight,
                                    const void* bias, const void* grad_out, void* grad_x, void* grad_weight,
                                    void* grad_bias, void* workspace, size_t workspace_bytes, int batch, int seq_len,
                                    int channels, int kernel_size, int dtype);

/* ------------------------------------------------------------------------
 * Softmax cross entropy over logits (block callers: the LM-head loss of the decoder
 * models; the reference takes it from Axon's loss inside the compiled training step)
 *   logits [rows, vocab] in dtype, targets [rows] int64; loss_rows[n] = lse[n] -
 *   logits[n, targets[n]] and lse [rows] in f32 (rows whose target lies outside [0, vocab)
 *   give loss 0 and gradient 0).  The backward writes grad_logits [rows, vocab] in dtype:
 *   (softmax - onehot) * (*grad_loss) * inv_rows, with grad_loss a device scalar (f32).
 * ------------------------------------------------------------------------ */
int edf_cross_entropy(void* stream, const void* logits, const int64_t* targets, float* loss_rows, float* lse,
                      int rows, int vocab, int dtype);
int edf_cross_entropy_backward(void* stream, const void* logits, const int64_t* targets, const float* lse,
                               const float* grad_loss, float inv_rows, void* grad_logits, int rows, int vocab,
                               int dtype);

/* ------------------------------------------------------------------------
 * Layer normalisation over the last dimension (block callers: every block model's pre-norm
 * and final norm; the reference's Axon.layer_norm, lib/edifice/ssm/common.ex:224,
 * lib/edifice/recurrent/delta_net.ex:159,199, lib/edifice/blocks/model_builder.ex:111,165)
 *   y[r, c] = (x[r, c] - mean_r) rstd_r gamma[c] + beta[c],  rstd_r = 1 / sqrt(var_r + eps)
 *   (biased variance); x, y [rows, cols] in dtype; gamma, beta [cols] in param_dtype, either
 *   NULL for 1 / 0; mean, rstd [rows] f32, written for the backward; 1 <= cols <= 8192.
 * The backward writes grad_x [rows, cols] and, where not NULL, grad_gamma / grad_beta [cols]
 * (summed over rows in a fixed order); workspace edf_layer_norm_backward_workspace_bytes().
 * ------------------------------------------------------------------------ */
int edf_layer_norm(void* stream, const void* x, const void* gamma, const void* beta, void* y, float* mean,
                   float* rstd, int rows, int cols, float eps, int dtype, int param_dtype);
size_t edf_layer_norm_backward_workspace_bytes(int rows, int cols);
int edf_layer_norm_backward(void* stream, const void* x, const void* gamma, const float* mean, const float* rstd,
                            const void* grad_y, void* grad_x, void* grad_gamma, void* grad_beta, void* workspace,
                            size_t workspace_bytes, int rows, int cols, int dtype, int param_dtype);
/* Residual form: the residual add in front of a pre-norm (transformer_block.ex:118,144,
 * common.ex:119: h' = h + block(norm h), and the next block's norm of h').
 * edf_add_layer_norm writes sum = x + res (rounded to dtype, as a separate add stores it; it may
 * not alias x or res) and y = layer_norm(sum); mean / rstd as above, of sum.
 * edf_layer_norm_backward_add is edf_layer_norm_backward (x = the sum) with grad_add [rows,
 * cols] (the gradient reaching the sum through the residual path, may be NULL) added to
 * grad_x before it is rounded and stored. */
int edf_add_layer_norm(void* stream, const void* x, const void* res, void* sum, const void* gamma, const void* beta,
                       void* y, float* mean, float* rstd, int rows, int cols, float eps, int dtype, int param_dtype);
int edf_layer_norm_backward_add(void* stream, const void* x, const void* gamma, const float* mean, const float* rstd,
                                const void* grad_y, const void* grad_add, void* grad_x, void* grad_gamma,
                                void* grad_beta, void* workspace, size_t workspace_bytes, int rows, int cols,
                                int dtype, int param_dtype);

/* ------------------------------------------------------------------------
 * Head layout around the attention kernels (block callers: the attention blocks' head split
 * and merge, Nx reshapes / transposes in the reference, e.g. transformer_block.ex:118):
 *   edf_heads_split: x [batch, seq, P H d] -> parts[p] [batch, H, seq, d], p < P
 *   edf_heads_merge: parts[p] [batch, H, seq, d] -> y [batch, seq, P H d]
 * parts: a host array of num_parts (1..4) device pointers; H = num_heads, d = head_dim.
 * ------------------------------------------------------------------------ */
int edf_heads_split(void* stream, const void* x, void* const* parts, long batch, long seq, int num_parts,
                    int num_heads, int head_dim, int dtype);
int edf_heads_merge(void* stream, const void* const* parts, void* y, long batch, long seq, int num_parts,
                    int num_heads, int head_dim, int dtype);

/* ------------------------------------------------------------------------
 * Token-embedding weight gradient (block callers: the language models' input embedding,
 * Axon.embedding, e.g. lib/edifice/generative/show_o.ex:123):
 *   grad_weight[v, :] = sum over positions p with ids[p] == v (ascending p) of grad[p, :]
 * ids [n] int64, grad [n, dim] and grad_weight [vocab, dim] in dtype; every row of
 * grad_weight is written (0 where no position names it, and for padding_idx; -1: none); ids
 * outside [0, vocab) contribute nothing.  Deterministic (stable sort of the ids, fixed
 * summation order); workspace edf_embedding_backward_workspace_bytes(n, vocab).
 * ------------------------------------------------------------------------ */
size_t edf_embedding_backward_workspace_bytes(long n, long vocab);
int edf_embedding_backward(void* stream, const int64_t* ids, const void* grad, void* grad_weight, void* workspace,
                           size_t workspace_bytes, long n, long vocab, int dim, long padding_idx, int dtype);

/* ------------------------------------------------------------------------
 * Softplus (block callers: the Mamba block's dt activation, Axon.activation(:softplus),
 * lib/edifice/ssm/common.ex:366): y = log(1 + e^x) over n values of x in dtype (evaluated as
 * max(x, 0) + log1p(e^-|x|), f32 inside); the backward writes grad_x = grad_y sigmoid(x).
 * ------------------------------------------------------------------------ */
int edf_softplus(void* stream, const void* x, void* y, long n, int dtype);
int edf_softplus_backward(void* stream, const void* x, const void* grad_y, void* grad_x, long n, int dtype);

/* ------------------------------------------------------------------------
 * Column sums (block callers: the bias gradients of the dense layers, sum over rows of the
 * output gradient; in the reference XLA derives them for Axon.dense): out[c] = sum_r x[r, c],
 * x [rows, cols] in dtype, out [cols] in out_dtype, f32 inside, summed in a fixed order;
 * workspace edf_column_sum_workspace_bytes().
 * ------------------------------------------------------------------------ */
size_t edf_column_sum_workspace_bytes(long rows, int cols);
int edf_column_sum(void* stream, const void* x, void* out, void* workspace, size_t workspace_bytes, long rows,
                   int cols, int dtype, int out_dtype);

/* ------------------------------------------------------------------------
 * L2 normalisation of rows (block callers: the DeltaNet / GatedDeltaNet key norm,
 * lib/edifice/recurrent/delta_net.ex:291, gated_delta_net.ex:387):
 *   y = x / sqrt(sum_j x_j^2 + eps) over rows of d <= 1024 elements of x [rows, d] in dtype
 *   (f32 inside); the backward writes grad_x = (grad_y - y <y, grad_y>) / sqrt(sum x^2 + eps).
 * ------------------------------------------------------------------------ */
int edf_l2_normalize(void* stream, const void* x, void* y, long rows, int d, float eps, int dtype);
int edf_l2_normalize_backward(void* stream, const void* x, const void* grad_y, void* grad_x, long rows, int d,
                              float eps, int dtype);
/* DeltaNet input split (delta_net.ex:274-300): proj [rows, 4 H d] = q | k | v | beta_pre per
 * row (the layer's qkvb projection); writes q, k / sqrt(sum_d k^2 + eps) per head, v and
 * sigmoid(beta_pre), each [rows, H, d] (H = num_heads, d = head_dim <= 1024).  The backward
 * writes grad_proj [rows, 4 H d] from the four [rows, H, d] gradients (k's norm and the sigmoid
 * recomputed from proj). */
int edf_delta_net_split(void* stream, const void* proj, void* q, void* k, void* v, void* beta, long rows,
                        int num_heads, int head_dim, float eps, int dtype);
int edf_delta_net_split_backward(void* stream, const void* proj, const void* grad_q, const void* grad_k,
                                 const void* grad_v, const void* grad_beta, void* grad_proj, long rows,
                                 int num_heads, int head_dim, float eps, int dtype);

#ifdef __cplusplus
}
#endif

#endif /* EDIFICE_HIP_H */
