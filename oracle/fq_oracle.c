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
        case FQO_Q5_0: e = 32;  b = 22;  break;
        case FQO_Q5_1: e = 32;  b = 24;  break;
        case FQO_Q3_K: e = 256; b = 110; break;
        case FQO_Q5_K: e = 256; b = 176; break;
        case FQO_IQ4_NL: e = 32; b = 18; break;
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

static uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* matmul.cpp:125-152.  Element j (j < 32) of a block: 4 low bits from the
 * nibble j % 16 of qs (low nibble for j < 16), bit 4 from bit j of qh. */
static void deq_q5_0_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 31) / 32;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 22;
        float d = fqo_fp16_to_fp32(rd16(blk));
        uint32_t qh = rd32(blk + 2);
        const uint8_t* qs = blk + 6;
        for (int j = 0; j < 32 && bi * 32 + j < K; ++j) {
            int lo4 = j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4);
            int q = lo4 | (int)(((qh >> j) & 1u) << 4);
            out[bi * 32 + j] = (float)(q - 16) * d;
        }
    }
}

/* matmul.cpp:156-186: the same 5-bit codes, w = q * d + m. */
static void deq_q5_1_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 31) / 32;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 24;
        float d = fqo_fp16_to_fp32(rd16(blk));
        float m = fqo_fp16_to_fp32(rd16(blk + 2));
        uint32_t qh = rd32(blk + 4);
        const uint8_t* qs = blk + 8;
        for (int j = 0; j < 32 && bi * 32 + j < K; ++j) {
            int lo4 = j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4);
            int q = lo4 | (int)(((qh >> j) & 1u) << 4);
            out[bi * 32 + j] = (float)q * d + m;
        }
    }
}

/* matmul.cpp:284-338.  The 16 six-bit scales of a super-block: scale i has
 * its low 4 bits in nibble (i >> 3) of byte (i & 7) and its high 2 bits in
 * bits 2 (i >> 2) .. +1 of byte 8 + (i & 3); the value used is scale - 32. */
static int q3_k_scale(const uint8_t* raw, int i) {
    int lo4 = (raw[i & 7] >> (4 * (i >> 3))) & 0xF;
    int hi2 = (raw[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return (lo4 | (hi2 << 4)) - 32;
}

/* matmul.cpp:284-338.  Element e = 128 n + 32 j + l of a super-block
 * (n < 2, j < 4, l < 32): 2 low bits at bit 2 j of qs[32 n + l], minus 4
 * unless bit 4 n + j of hmask[l] is set; scale 8 n + 2 j + l / 16. */
static void deq_q3_k_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 255) / 256;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 110;
        const uint8_t* hm = blk;
        const uint8_t* qs = blk + 32;
        const uint8_t* sc = blk + 96;
        float d = fqo_fp16_to_fp32(rd16(blk + 108));
        for (int e = 0; e < 256 && bi * 256 + e < K; ++e) {
            int n = e / 128, j = (e % 128) / 32, l = e % 32;
            int q = (qs[32 * n + l] >> (2 * j)) & 3;
            if (!((hm[l] >> (4 * n + j)) & 1)) q -= 4;
            float dl = d * (float)q3_k_scale(sc, 8 * n + 2 * j + l / 16);
            out[bi * 256 + e] = dl * (float)q;
        }
    }
}

/* matmul.cpp:382-415.  Element 64 g + 32 h + l (g < 4, h < 2, l < 32):
 * nibble h of qs[32 g + l] plus 16 times bit 2 g + h of qh[l], scale/min
 * pair 2 g + h (get_scale_min_k4, as Q4_K). */
static void deq_q5_k_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 255) / 256;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 176;
        float d = fqo_fp16_to_fp32(rd16(blk));
        float dmin = fqo_fp16_to_fp32(rd16(blk + 2));
        const uint8_t* scales = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* qs = blk + 48;
        for (int e = 0; e < 256 && bi * 256 + e < K; ++e) {
            int g = e / 64, h = (e % 64) / 32, l = e % 32;
            uint8_t sc, m;
            scale_min_k4(2 * g + h, scales, &sc, &m);
            int q = ((qs[32 * g + l] >> (4 * h)) & 0xF) + (((qh[l] >> (2 * g + h)) & 1) ? 16 : 0);
            float d1 = d * (float)sc;
            float m1 = dmin * (float)m;
            out[bi * 256 + e] = d1 * (float)q - m1;
        }
    }
}

/* matmul.cpp:849-868: 4-bit indices into a fixed non-linear table. */
static const int8_t iq4nl_values[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                        1,    13,   25,  38,  53,  69,  89,  113};

static void deq_iq4_nl_row(const uint8_t* row, float* out, int K) {
    int nb = (K + 31) / 32;
    for (int bi = 0; bi < nb; ++bi) {
        const uint8_t* blk = row + (size_t)bi * 18;
        float d = fqo_fp16_to_fp32(rd16(blk));
        const uint8_t* qs = blk + 2;
        for (int j = 0; j < 32 && bi * 32 + j < K; ++j) {
            int idx = j < 16 ? (qs[j] & 0x0F) : (qs[j - 16] >> 4);
            out[bi * 32 + j] = d * (float)iq4nl_values[idx];
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
        case FQO_Q5_0: return deq_q5_0_row;
        case FQO_Q5_1: return deq_q5_1_row;
        case FQO_Q3_K: return deq_q3_k_row;
        case FQO_Q5_K: return deq_q5_k_row;
        case FQO_IQ4_NL: return deq_iq4_nl_row;
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
