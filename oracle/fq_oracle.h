/*
 * fq_oracle.h -- CPU restatement of Forge's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  No product code path calls it, and the product fails loudly when
 * its HIP library is missing instead of falling back to this code.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the Forge source tree).  Pinning of each function is listed beside it:
 *   - "golden":  checked bit-exactly against vectors produced by the
 *                reference's own compiled CPU code (tests/golden/*.npz);
 *   - "closed form": checked against an independent derivation
 *                (numpy float16 conversion, an independent encoder, brute
 *                force on tiny inputs).
 */
#ifndef FQ_ORACLE_H
#define FQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* forge::DataType values (include/forge/types.h:7-26). */
enum {
    FQO_FP32 = 0,
    FQO_Q4_0 = 2,
    FQO_Q4_1 = 3,
    FQO_Q4_K = 4,
    FQO_Q8_0 = 7,
    FQO_Q5_0 = 8,
    FQO_Q5_1 = 9,
    FQO_Q3_K = 11,
    FQO_Q5_K = 12,
    FQO_Q6_K = 13,
    FQO_IQ4_NL = 17,
};

/* Block geometry, include/forge/quant_traits.h:19-95.  Returns 0 on success,
 * -1 for a dtype outside the ten formats of the hot path. */
int fqo_block_info(uint32_t dtype, int* block_elems, int* block_bytes);

/* IEEE binary16 -> binary32, exact incl. subnormals.
 * Restates fp16_to_fp32, src/operators/cpu/matmul.cpp:58-71.
 * Pinned: closed form (all 65536 inputs vs numpy float16). */
float fqo_fp16_to_fp32(uint16_t bits);

/* Dequantize rows [0, N) of a row-major [N][ceil(K/blk)] block matrix into
 * out[N][K] (fp32, row stride K).  Bit-exact restatement of
 *   dequantize_q4_0_row  matmul.cpp:73-87
 *   dequantize_q4_1_row  matmul.cpp:89-104
 *   dequantize_q8_0_row  matmul.cpp:106-118
 *   get_scale_min_k4     matmul.cpp:232-240
 *   dequantize_q6_k_row  matmul.cpp:242-279
 *   dequantize_q4_k_row  matmul.cpp:340-377
 *   dequantize_q5_0_row  matmul.cpp:125-152
 *   dequantize_q5_1_row  matmul.cpp:156-186
 *   dequantize_q3_k_row  matmul.cpp:284-338
 *   dequantize_q5_k_row  matmul.cpp:382-415
 *   dequantize_iq4_nl_row matmul.cpp:849-868
 * Only the first K values of each row are written (the reference's Q6_K, Q3_K,
 * Q5_K and IQ4_NL row routines write whole blocks even past K).
 * Pinned: golden + closed form (independent encoder round trip).
 * Returns 0, or -1 for an unsupported dtype / bad shape. */
int fqo_dequant_rows(uint32_t dtype, const uint8_t* w, float* out, int N, int K);

/* y[m][n] = sum_k x[m][k] * W[n][k] in double precision over the bit-exact
 * dequantized W (the value the reference's fp32 GEMVs approximate:
 * ops::matmul_transB, matmul.cpp:1134-1403; cpu_gemv.h:84-311, 545-714,
 * 784-984, 993-1015, 1670-1930).  x is fp32 [M][K], y is double [M][N].
 * Pinned: golden (reference matmul_transB outputs agree to fp32 rounding)
 * and brute force on tiny inputs. */
int fqo_matmul_transB_f64(uint32_t dtype, const float* x, const uint8_t* w, double* y,
                          int M, int K, int N);

/* The same product accumulated in fp32 (16-element fma chunks summed in
 * order) over the dequantized row: a second legitimate fp32 order, used to
 * size how far fp32 orders drift apart at a shape.  Pinned: agrees with the
 * f64 version to fp32 rounding. */
int fqo_matmul_transB_f32(uint32_t dtype, const float* x, const uint8_t* w, float* y,
                          int M, int K, int N);

#ifdef __cplusplus
}
#endif

#endif
