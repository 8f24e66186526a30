/* Layout probes of the gfx950 HIP library: TEST INFRASTRUCTURE, not part of the C ABI in
 * include/edifice_hip.h.  libedifice_hip.so exports these three entry points only so that
 * tests/test_gpu_mfma_layout.py can pin the lane layouts the kernels assume; no caller of
 * the library binds them.  Each returns EDF_OK or an EDF_ERR_* code like the product entry
 * points. */
#ifndef EDIFICE_HIP_PROBES_H
#define EDIFICE_HIP_PROBES_H

#ifdef __cplusplus
extern "C" {
#endif

/* Diagnostic: C[32][32] = A[32][16] * B[16][32] (bf16 in, f32 out, row-major) with one
 * v_mfma_f32_32x32x16_bf16, using the lane layout the attention and delta-rule kernels
 * assume.  No reference counterpart; used by the GPU tests to pin that layout. */
int edf_debug_mfma_32x32x16_bf16(void* stream, const void* A, const void* B, float* C);

/* Diagnostic: reuse of an MFMA accumulator as the next product's operand (one
 * v_permlane32_swap per register pair).  x is a 64x32 f32 matrix (row-major) held as two
 * 32x32 accumulator tiles; out[lane][kk][e] (bf16, 64 x 4 x 8) receives the operand
 * fragment for k-step kk, which must equal x[16 kk + 8 (lane / 32) + e][lane % 32].
 * No reference counterpart; used by the GPU tests to pin the chunked delta rule's layout. */
int edf_debug_acc_kfrag_bf16(void* stream, const float* x, void* out);

/* Diagnostic: the transposed LDS read (ds_read_b64_tr_b16) the attention kernels use for
 * the V^T operand.  x is a 64x64 bf16 row-major tile; out[lane][rb][e] (bf16, 64 x 2 x 4)
 * receives, for rb = 0 and 1, what lane `lane` reads when lane i of each 16-lane group
 * addresses row 8 rb + 4 (group / 2) + i / 4, column 16 (group % 2) + 4 (i % 4); that must
 * be x[8 rb + 4 (lane / 32) + e][lane % 32].  No reference counterpart; used by the GPU
 * tests to pin that layout. */
int edf_debug_lds_read_tr16(void* stream, const void* x, void* out);

/* Streaming probe: out = in0 + in1 (nin = 2, 32-bit integer lanes) or out = in0 (nin = 1)
 * over n_bytes (a multiple of 16) with 16-byte accesses, `blocks` workgroups of 256 threads
 * striding over the buffers: the HBM rate a plain streaming kernel reaches, against which
 * bench.py reads the bandwidth-bound scans. */
int edf_probe_stream(void* stream, const void* in0, const void* in1, void* out, long n_bytes, int nin, int blocks);

#ifdef __cplusplus
}
#endif

#endif /* EDIFICE_HIP_PROBES_H */
