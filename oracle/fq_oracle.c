/*
 * fq_oracle.c -- CPU restatement of Forge's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see
 * fq_oracle.h for who may load it and how each function is pinned.
 *
 * Built with -ffp-contract=off so that every fp32 expression rounds exactly
 * as written; the dequant expressions below are the reference's, in the
 * reference's association order.
 */
#include "fq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int fqo_block_info(uint32_t dtype, int* block_elems, int* block_bytes) {
    /* include/forge/quant_traits.h:19-95 */
    int e, b;
    switch (dtype) {
        case FQO_Q4_0: e = 32;  b = 18;  break;
        case FQO_Q4_1: e = 32;  b = 20;  break;
        case FQO_Q8_0: e = 32;  b = 34;  break;
        case FQO_Q4_K: e = 256; b = 144; break;
        case FQO_Q6_K: e = 256; b = 210; break;
        default: return -1;
    }
    if (block_elems) *block_elems = e;
    if (block_bytes) *block_bytes = b;
    return 0;
}

/* matmul.cpp:58-71: sign/exponent/mantissa split, subnormals via ldexp. */
float fqo_fp16_to_fp32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    float v;
    if (exponent == 0) {
        if (mantissa == 0) return 0.0f; /* the reference returns +0 for -0 too */
        v = ldexpf((float)mantissa / 1024.0f, -14);
        return sign ? -v : v;
    }
    /* exponent 31 (inf/nan) goes through the same formula in the reference */
    v = ldexpf(1.0f + (float)mantissa / 1024.0f, (int)exponent - 15);
    return sign ? -v : v;
}

static uint16_t rd16(const uint8_t* p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* matmul.cpp:73-87 */
static void deq_q4_0_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 31) / 32;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 18;
        float scale = fqo_fp16_to_fp32(rd16(blk));
        const uint8_t* qs = blk + 2;
        int base = bi * 32;
        for (int j = 0; j < 16 && base + j < K; ++j)
            out[base + j] = (float)((qs[j] & 0x0F) - 8) * scale;
        for (int j = 0; j < 16 && base + 16 + j < K; ++j)
            out[base + 16 + j] = (float)(((qs[j] >> 4) & 0x0F) - 8) * scale;
    }
}

/* matmul.cpp:89-104 */
static void deq_q4_1_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 31) / 32;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 20;
        float d = fqo_fp16_to_fp32(rd16(blk));
        float m = fqo_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* qs = blk + 4;
        int base = bi * 32;
        for (int j = 0; j < 16 && base + j < K; ++j)
            out[base + j] = (float)(qs[j] & 0x0F) * d + m;
        for (int j = 0; j < 16 && base + 16 + j < K; ++j)
            out[base + 16 + j] = (float)((qs[j] >> 4) & 0x0F) * d + m;
    }
}

/* matmul.cpp:106-118 */
static void deq_q8_0_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 31) / 32;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 34;
        float scale = fqo_fp16_to_fp32(rd16(blk));
        const int8_t* qs = (const int8_t*)(blk + 2);
        int base = bi * 32;
        for (int j = 0; j < 32 && base + j < K; ++j)
            out[base + j] = (float)qs[j] * scale;
    }
}

/* matmul.cpp:232-240: 6-bit scale/min pairs packed into 12 bytes. */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* matmul.cpp:340-377 */
static void deq_q4_k_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 255) / 256;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 144;
        float d = fqo_fp16_to_fp32(rd16(blk));
        float dmin = fqo_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        int is = 0;
        for (int j = 0; j < 256; j += 64) {
            uint8_t sc1, m1, sc2, m2;
            scale_min_k4(is, scales, &sc1, &m1);
            scale_min_k4(is + 1, scales, &sc2, &m2);
            float d1 = d * (float)sc1;
            float m1v = dmin * (float)m1;
            float d2 = d * (float)sc2;
            float m2v = dmin * (float)m2;
            int base = bi * 256 + j;
            for (int l = 0; l < 32; ++l)
                if (base + l < K) out[base + l] = d1 * (float)(qs[l] & 0xF) - m1v;
            for (int l = 0; l < 32; ++l)
                if (base + 32 + l < K) out[base + 32 + l] = d2 * (float)(qs[l] >> 4) - m2v;
            qs += 32;
            is += 2;
        }
    }
}

/* matmul.cpp:242-279.  The product is evaluated (d * sc) * q, left to right,
 * as the reference writes it; the second multiply rounds. */
static void deq_q6_k_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 255) / 256;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        float d = fqo_fp16_to_fp32(rd16(blk + 208));
        int y0 = bi * 256;
        for (int n = 0; n < 256; n += 128) {
            for (int l = 0; l < 32; ++l) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                int i1 = y0 + n + l, i2 = i1 + 32, i3 = i1 + 64, i4 = i1 + 96;
                if (i1 < K) out[i1] = d * (float)sc[is + 0] * (float)q1;
                if (i2 < K) out[i2] = d * (float)sc[is + 2] * (float)q2;
                if (i3 < K) out[i3] = d * (float)sc[is + 4] * (float)q3;
                if (i4 < K) out[i4] = d * (float)sc[is + 6] * (float)q4;
            }
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

typedef void (*deq_fn)(const uint8_t*, float*, int);

static deq_fn pick(uint32_t dtype) {
    switch (dtype) {
        case FQO_Q4_0: return deq_q4_0_row;
        case FQO_Q4_1: return deq_q4_1_row;
        case FQO_Q8_0: return deq_q8_0_row;
        case FQO_Q4_K: return deq_q4_k_row;
        case FQO_Q6_K: return deq_q6_k_row;
        default: return NULL;
    }
}

static size_t row_bytes(uint32_t dtype, int K) {
    int e = 0, b = 0;
    fqo_block_info(dtype, &e, &b);
    return (size_t)((K + e - 1) / e) * (size_t)b;
}

int fqo_dequant_rows(uint32_t dtype, const uint8_t* w, float* out, int N, int K) {
    deq_fn f = pick(dtype);
    if (!f || N < 0 || K < 0) return -1;
    size_t rb = row_bytes(dtype, K);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) f(w + (size_t)n * rb, out + (size_t)n * K, K);
    return 0;
}

int fqo_matmul_transB_f64(uint32_t dtype, const float* x, const uint8_t* w, double* y,
                          int M, int K, int N) {
    deq_fn f = pick(dtype);
    if (!f || M < 0 || N < 0 || K < 0) return -1;
    size_t rb = row_bytes(dtype, K);
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            f(w + (size_t)n * rb, row, K);
            for (int m = 0; m < M; ++m) {
                const float* xr = x + (size_t)m * K;
                double s = 0.0;
                for (int k = 0; k < K; ++k) s += (double)xr[k] * (double)row[k];
                y[(size_t)m * N + n] = s;
            }
        }
        free(row);
    }
    return 0;
}

/* fp32 accumulation over the dequantized row in 16-element chunks (each
 * chunk an fma chain, chunks summed in order).  A second legitimate fp32
 * order, used to size the drift between fp32 orders at a given shape. */
int fqo_matmul_transB_f32(uint32_t dtype, const float* x, const uint8_t* w, float* y,
                          int M, int K, int N) {
    deq_fn f = pick(dtype);
    if (!f || M < 0 || N < 0 || K < 0) return -1;
    size_t rb = row_bytes(dtype, K);
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            f(w + (size_t)n * rb, row, K);
            for (int m = 0; m < M; ++m) {
                const float* xr = x + (size_t)m * K;
                float acc = 0.0f;
                for (int k0 = 0; k0 < K; k0 += 16) {
                    float p = 0.0f;
                    for (int k = k0; k < k0 + 16 && k < K; ++k) p = fmaf(xr[k], row[k], p);
                    acc += p;
                }
                y[(size_t)m * N + n] = acc;
            }
        }
        free(row);
    }
    return 0;
}
