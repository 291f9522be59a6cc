/*
 * forge_q.h -- C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * This is the seam Forge's operator layer calls into on the GPU device.  It
 * replaces the CUDA function-pointer tables and launchers the reference
 * binds today; every entry point cites the reference interface it replaces.
 * Plain pointers, sizes and an opaque stream handle only: no C++ or torch
 * types cross this boundary, and nothing throws across it.
 *
 * Conventions (shared by all entry points)
 *  - dtype: a forge::DataType value (include/forge/types.h:7-26 of the
 *    reference): Q4_0=2, Q4_1=3, Q4_K=4, Q8_0=7, Q5_0=8, Q5_1=9, Q3_K=11,
 *    Q5_K=12, Q6_K=13, IQ4_NL=17.  The packed (aligned) layout exists for
 *    Q4_0, Q4_1, Q8_0, Q4_K and Q6_K only.
 *  - w: device pointer to a row-major [N][K/block_elems] array of on-disk
 *    GGUF blocks, rows contiguous with no padding (the layout
 *    forge::compute_quantized_bytes sizes, quant_traits.h:138-146).  No
 *    alignment beyond 2 bytes is required.
 *  - x: device fp32 [M][K] row-major; y: device fp32 [M][N] row-major.
 *  - stream: a hipStream_t passed as void*; NULL is the null stream.  All
 *    entry points are asynchronous with respect to the host, like the
 *    reference's launchers (cuda_gemv_tmpl.cuh:332-351).
 *  - K must be a multiple of the format's block size for the matmul entry
 *    points (GGUF guarantees this for every weight tensor).
 *  - Return value: FQ_OK or one of the FQ_ERR_* codes below; the reference
 *    throws std::runtime_error for the same conditions (matmul.cpp:1135-1146,
 *    1163-1165, 1315) or launches unchecked.
 *  - Calls on the M > 1 matrix-core path, the batch-1 kernel at 2..4 tokens
 *    with K split into slabs (long rows, e.g. K = 18944; under graph capture
 *    without a reserved workspace such a call takes another kernel instead)
 *    and the GGUF fused ops use a
 *    library-owned per-device, per-stream workspace (token operands, split-K
 *    partial slabs, intermediate rows; for Q6_K prefill, M > 32, the rows
 *    rewritten into 36-byte blocks of int8 codes: N * K * 9 / 8 bytes).  It grows on demand inside a call
 *    (hipMalloc, no host synchronisation; a superseded buffer is kept until
 *    fq_release_workspace) and lives until the process ends.  Under HIP-graph
 *    capture a call that would have to grow it returns FQ_ERR_WORKSPACE:
 *    size it first with fq_reserve_workspace.  The matmul.cpp:31-54
 *    thread-local grow-only buffer of the reference plays the same role.
 */
#ifndef FORGE_Q_H
#define FORGE_Q_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FQ_OK 0
#define FQ_ERR_DTYPE 1    /* dtype is not one of the ten block formats           */
#define FQ_ERR_SHAPE 2    /* M/N/K out of range or K not a multiple of the block  */
#define FQ_ERR_NULL 3     /* a required pointer is NULL                           */
#define FQ_ERR_HIP 4      /* the HIP runtime reported an error (fq_last_hip_error) */
#define FQ_ERR_NO_DEVICE 5
#define FQ_ERR_ALIGN 6     /* a packed-layout pointer is not 16-byte aligned       */
#define FQ_ERR_WORKSPACE 7 /* the workspace would have to grow during graph capture,
                              or a call exceeds fq_matmul_transB_noalloc's fixed one */

/* DataType values accepted by the entry points. */
#define FQ_DTYPE_Q4_0 2u
#define FQ_DTYPE_Q4_1 3u
#define FQ_DTYPE_Q4_K 4u
#define FQ_DTYPE_Q8_0 7u
#define FQ_DTYPE_Q5_0 8u
#define FQ_DTYPE_Q5_1 9u
#define FQ_DTYPE_Q3_K 11u
#define FQ_DTYPE_Q5_K 12u
#define FQ_DTYPE_Q6_K 13u
#define FQ_DTYPE_IQ4_NL 17u

/* Block geometry of a dtype: elements and bytes per block.
 * Replaces data_type_traits[] lookups (src/operators/cpu/quant_traits.cpp:33-52,
 * dtype_block_elements / dtype_block_size, quant_traits.h:118-124). */
int fq_block_info(uint32_t dtype, int* block_elems, int* block_bytes);

/* Human-readable text for a status code (static storage). */
const char* fq_status_str(int status);

/* The hipError_t value behind the most recent FQ_ERR_HIP on this thread. */
int fq_last_hip_error(void);

/* Batch-1 fused dequant+GEMV: y[n] = sum_k x[k] * dequant(w)[n][k].
 * Replaces cuda::gemv_dispatch[dtype](x, w, y, K, N, stream)
 * (src/operators/cuda/cuda_gemv.h:29-33, table cuda_gemv_instances.cu:36-76,
 * called from matmul.cpp:1246-1249) and the Q4_0 special launcher
 * launch_gemv_q4_0_transB (cuda_gemv.cu:183-208). */
int fq_gemv(uint32_t dtype, const float* x, const void* w, float* y, int K, int N, void* stream);

/* Small-batch fused dequant+matmul, 1 <= M <= 32: y[m][n] = x[m] . W[n].
 * Replaces cuda::gemv_batch_dispatch[dtype](x, w, y, M, K, N, stream)
 * (cuda_gemv.h:29-33, called from matmul.cpp:1156-1161).  Activations stay
 * fp32 and are not quantized, as in the reference. */
int fq_gemv_batch(uint32_t dtype, const float* x, const void* w, float* y, int M, int K, int N,
                  void* stream);

/* Prefill matmul for M > 32 (dense contraction on MFMA).
 * Replaces the reference's dequantize-to-fp32 + cublasGemmEx pair
 * (launch_dequant_*_matrix + launch_cublas_sgemm, matmul.cpp:1190-1243,
 * cuda_quant.cu:582-598) and its Q8_0 host round-trip (matmul.cpp:1216-1238). */
int fq_matmul_prefill(uint32_t dtype, const float* x, const void* w, float* y, int M, int K,
                      int N, void* stream);

/* Device branch of ops::matmul_transB (matmul.cpp:1134-1286) for block
 * weights: dispatches on M exactly as the reference does (M == 1 -> GEMV,
 * 1 < M <= 32 -> small batch, M > 32 -> prefill) and applies the optional
 * bias like apply_bias (matmul.cpp:1005-1049):
 *   bias_ndim == 1: y[m][n] += bias[n] for n < min(bias_len, N)
 *   bias_ndim == 2: y[i]    += bias[i] for i < M*N (bias_len must be >= M*N)
 *   bias == NULL or bias_ndim == 0: no bias.
 * bias must be a device pointer. */
int fq_matmul_transB(uint32_t dtype, const float* x, const void* w, const float* bias,
                     int bias_ndim, int64_t bias_len, float* y, int M, int K, int N,
                     void* stream);

/* Dequantize rows [0, N) of w into out[N][K] fp32, bit-identical to the
 * reference's dequantize_*_row (matmul.cpp:73-377), including its scalar
 * fp16 conversion (fp16 Inf/NaN scale codes map to finite values, -0 to +0).
 * K need not be a multiple of the block.  Replaces launch_dequant_*_matrix
 * (cuda_quant.cu:131-335) and backs ops::dequantize_weight
 * (matmul.cpp:980-1003). */
int fq_dequant_rows(uint32_t dtype, const void* w, float* out, int N, int K, void* stream);

/* ------------------------------------------------------------------------
 * Aligned device layout ("packed").  GGUF blocks are 18/20/34/210 bytes, so
 * most of them are only 2-byte aligned in memory.  The packed layout holds
 * the same bytes of each row, moved into 16-byte-aligned "planes" (the piece
 * a GEMV lane reads for lane unit v sits at plane + 16 v) followed by dense
 * scale arrays; the per-format layout is documented in forge_amd/csrc/fq_pack.h.
 * Rows are contiguous at a pitch of fq_packed_row_bytes, except for Q8_0
 * matrices of 65536 rows and more, whose rows are grouped in tiles of 16
 * with their 16-byte pieces interleaved row by row (the batch-1 kernel there
 * gives each lane one row).  The buffer size is the same either
 * way (N * fq_packed_row_bytes), and the arrangement depends only on dtype
 * and N: a packed matrix is always used with the N it was packed with (a
 * row range of a tiled matrix is not a packed matrix of its own).
 * Dequantized values are identical: fq_unpack_weights restores the GGUF
 * bytes exactly.  Requires K % 256 == 0 and 16-byte-aligned packed buffers.
 * No counterpart in the reference (it reads GGUF blocks in place); it backs
 * the load-time repack a loader may do when it copies a tensor to the device
 * (Tensor::to_device, src/core/tensor.cpp; GGUF mapping gguf_model.cpp:57-90).
 * ---------------------------------------------------------------------- */

/* Bytes per row in the packed layout; 0 if the dtype or K is unsupported. */
int64_t fq_packed_row_bytes(uint32_t dtype, int K);

/* GGUF rows -> packed rows (device to device, N rows of length K). */
int fq_pack_weights(uint32_t dtype, const void* w_gguf, void* w_packed, int N, int K,
                    void* stream);

/* Packed rows -> GGUF rows, bit-exact inverse of fq_pack_weights. */
int fq_unpack_weights(uint32_t dtype, const void* w_packed, void* w_gguf, int N, int K,
                      void* stream);

/* Batch-1 GEMV over packed weights: y[n] = sum_k x[k] dequant(w)[n][k] (+ bias[n]
 * for n < bias_len when bias != NULL).  Same results as fq_gemv on the GGUF
 * bytes, within the path's tolerance; deterministic. */
int fq_gemv_packed(uint32_t dtype, const float* x, const void* w_packed, const float* bias,
                   int64_t bias_len, float* y, int K, int N, void* stream);

/* ------------------------------------------------------------------------
 * Fused FFN up-projection: y[m][n] = silu(x[m] . Wgate[n]) * (x[m] . Wup[n]),
 * silu(g) = g / (1 + exp(-g)); Wgate and Wup have the same dtype and shape.
 * ---------------------------------------------------------------------- */

/* GGUF-layout weights, any M >= 1: two matmuls (as fq_matmul_transB) into a
 * library-owned per-stream buffer, then the SiLU-multiply.  Replaces the
 * device branch of ops::ffn_up_fused (matmul.cpp:1472-1533): the launchers
 * cuda::launch_ffn_up_fused_q4_0 / _q4_k and their batch forms
 * (cuda_fused.cu:15-106, 622-748) and the matmul_transB + silu_multiply
 * fallback (elementwise.cpp:89-150). */
int fq_ffn_up_fused(uint32_t dtype, const float* x, const void* w_gate, const void* w_up, float* y,
                    int M, int K, int N, void* stream);

/* M = 1 over packed weights, one launch: the two matrices are walked as one
 * GEMV of 2N interleaved rows, so the activation staging and the launch are
 * shared, and the SiLU-multiply is applied when the row sums are written.
 * Same results as fq_ffn_up_fused within the path's tolerance. */
int fq_ffn_up_fused_packed(uint32_t dtype, const float* x, const void* w_gate_packed,
                           const void* w_up_packed, float* y, int K, int N, void* stream);

/* ------------------------------------------------------------------------
 * Fused QKV projection: y[m] = [x[m] . Wq^T | x[m] . Wk^T | x[m] . Wv^T],
 * rows of y are Nq + Nk + Nv floats.  The three weights share dtype and K.
 * ---------------------------------------------------------------------- */

/* GGUF-layout weights, any M >= 1.  Replaces matmul_transB_fused_qkv_q4_0 /
 * _q4_k (matmul.cpp:1535-1600, 1639-1692) and the CUDA fused QKV launcher
 * (cuda_fused.cu:924-1024); at M > 1 the three results pass through a
 * library-owned per-stream buffer. */
int fq_fused_qkv(uint32_t dtype, const float* x, const void* wq, const void* wk, const void* wv,
                 float* y, int M, int K, int Nq, int Nk, int Nv, void* stream);

/* M = 1 over packed weights in one launch (the activation staging is shared). */
int fq_fused_qkv_packed(uint32_t dtype, const float* x, const void* wq_packed,
                        const void* wk_packed, const void* wv_packed, float* y, int K, int Nq,
                        int Nk, int Nv, void* stream);

/* ------------------------------------------------------------------------
 * Fused FFN down-projection + residual: y = x . W^T + residual, residual
 * [M][N] on the device.  Replaces matmul_transB_fused_ffn_down_residual_q4_0
 * / _q6_k (matmul.cpp:1601-1637, 1729-1764) and the CUDA launcher
 * (cuda_fused.cu:750-837): the residual is added when the row sums are
 * written, so there is no separate add pass.
 * ---------------------------------------------------------------------- */
int fq_ffn_down_residual(uint32_t dtype, const float* x, const void* w, const float* residual,
                         float* y, int M, int K, int N, void* stream);

/* M = 1 over packed weights. */
int fq_ffn_down_residual_packed(uint32_t dtype, const float* x, const void* w_packed,
                                const float* residual, float* y, int K, int N, void* stream);

/* fq_matmul_transB without any allocation: the same results (the same
 * kernels and launch plan), with the M > 1 workspace (matrix-core path,
 * split-K slabs of the batch-1 kernel at 2..4 tokens) taken
 * from a fixed 64 MiB device array that the library holds on every GPU it
 * runs on, instead of the per-stream workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP-graph
 * capture, serving loops and harnesses that forbid hipMalloc).  Returns
 * FQ_ERR_WORKSPACE when a call needs more than 64 MiB (for example M = 512 at
 * K = N = 4096 needs 40-42 MiB with 4 K-splits, 58 MiB for Q6_K, whose
 * rewritten rows take N * K * 9 / 8 bytes more).  All calls on one GPU
 * share the array: calls that overlap on one GPU (several streams or host
 * threads) race on it and must be serialised by the caller. */
int fq_matmul_transB_noalloc(uint32_t dtype, const float* x, const void* w, const float* bias,
                             int bias_ndim, int64_t bias_len, float* y, int M, int K, int N,
                             void* stream);

/* Sizes the calling stream's workspace (current device) for every call with
 * at most M_max tokens, K_max columns and N_max rows, so that later calls
 * allocate nothing and can be captured into a HIP graph.  The size covers
 * every format, Q6_K prefill's rewritten rows included.  Replaces the
 * reference's grow-on-first-use scratch (src/operators/cpu/matmul.cpp:31-54,
 * the thread-local buffer behind the CUDA Q8_0 M > 32 path), which has no
 * reserve call of its own. */
int fq_reserve_workspace(int M_max, int K_max, int N_max, void* stream);

/* Synchronises the stream and frees its workspace (current device), including
 * buffers superseded by growth.  No counterpart in the reference (its scratch
 * lives until the thread ends). */
int fq_release_workspace(void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_Q_H */
