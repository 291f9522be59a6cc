// fq_formats.h -- device-side decoding of the ten GGUF block formats.
//
// Every format is processed in "units" of 32 weights.  A unit is what one
// lane decodes per step: a whole block for Q4_0/Q4_1/Q8_0, one eighth of a
// 256-weight super-block for Q4_K/Q6_K.  A unit's 32 weights are produced in
// a format-specific "slot" order s = 0..31 that follows the byte layout, and
// the activation vector is staged in LDS in the same slot order, so the dot
// product of a unit is a straight 32-term FMA chain for every format.
//
// The slots of a unit fall into NG equal groups that share one affine
// coefficient pair (A_g, B_g): the unit's contribution to y is
//      sum_g  A_g * P_g + B_g * S_g,   P_g = sum_{s in g} x_s * q_s,
//                                      S_g = sum_{s in g} x_s,
// with q_s the raw unsigned code of slot s.  (A, B) per format:
//   Q4_0  (d, -8 d)            matmul.cpp:73-87     w = (q - 8) d
//   Q4_1  (d, m)               matmul.cpp:89-104    w = q d + m
//   Q8_0  (d, -128 d)          matmul.cpp:106-118   w = (q' - 128) d, q' = q ^ 0x80
//   Q4_K  (d sc_g, -dmin m_g)  matmul.cpp:340-377   w = d sc q - dmin m
//   Q6_K  (d sc_g, -32 d sc_g) matmul.cpp:242-279   w = (d sc)(q - 32)
//   Q5_0  (d, -16 d)           matmul.cpp:125-152   w = (q - 16) d
//   Q5_1  (d, m)               matmul.cpp:156-186   w = q d + m
//   Q3_K  (d sc_g, -4 d sc_g)  matmul.cpp:284-338   w = (d sc)(q - 4)
//   Q5_K  (d sc_g, -dmin m_g)  matmul.cpp:382-415   w = d sc q - dmin m
//   IQ4_NL (d, 0)              matmul.cpp:849-868   w = d T[q]; the "code" of
//         a slot is the table value T[q] itself (signed), not the index
// S_g is computed once per staged activation vector, so the offsets cost one
// FMA per group instead of one operation per weight.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fq {

enum : int {
    Q4_0 = 2, Q4_1 = 3, Q4_K = 4, Q8_0 = 7, Q5_0 = 8, Q5_1 = 9, Q3_K = 11, Q5_K = 12,
    Q6_K = 13, IQ4_NL = 17
};

// Calls fn(FmtTag<F>{}) for the format F named by dtype (the forge::DataType
// value); returns dflt for any other dtype.
template <int F>
struct FmtTag {
    static constexpr int value = F;
};
template <class R, class Fn>
__host__ __device__ inline R with_format(int dtype, R dflt, Fn&& fn) {
    switch (dtype) {
        case Q4_0: return fn(FmtTag<Q4_0>{});
        case Q4_1: return fn(FmtTag<Q4_1>{});
        case Q4_K: return fn(FmtTag<Q4_K>{});
        case Q8_0: return fn(FmtTag<Q8_0>{});
        case Q5_0: return fn(FmtTag<Q5_0>{});
        case Q5_1: return fn(FmtTag<Q5_1>{});
        case Q3_K: return fn(FmtTag<Q3_K>{});
        case Q5_K: return fn(FmtTag<Q5_K>{});
        case Q6_K: return fn(FmtTag<Q6_K>{});
        case IQ4_NL: return fn(FmtTag<IQ4_NL>{});
        default: return dflt;
    }
}

// ---- loads: GGUF blocks are only 2-byte aligned; gfx950 global loads accept
// unaligned addresses, and hipcc lowers these to single dwordx{1,2,4} loads.
// The NT variants set the non-temporal hint: weights are streamed exactly
// once per call, so they should not displace the activations in the caches.
typedef uint32_t fq_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t fq_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint2 ld_u64(const uint8_t* p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
__device__ __forceinline__ uint4 ld_u128(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
template <bool NT>
__device__ __forceinline__ uint32_t ldg16(const uint8_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p));
    else return ld_u16(p);
}
template <bool NT>
__device__ __forceinline__ uint32_t ldg32(const uint8_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    else return ld_u32(p);
}
template <bool NT>
__device__ __forceinline__ uint2 ldg64(const uint8_t* p) {
    if constexpr (NT) {
        fq_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const fq_u32x2*>(p));
        return make_uint2(v.x, v.y);
    } else {
        return ld_u64(p);
    }
}
template <bool NT>
__device__ __forceinline__ uint4 ldg128(const uint8_t* p) {
    if constexpr (NT) {
        fq_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const fq_u32x4*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return ld_u128(p);
    }
}

// ---- fp16 -> fp32
// Hardware conversion (v_cvt_f32_f16): what the reference's GEMVs use
// (F16C _mm256_cvtph_ps, cpu_gemv.h:25-28; __half2float in CUDA).
__device__ __forceinline__ float f16_hw(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// The reference's scalar conversion (matmul.cpp:58-71), used by the dequant
// path so dequantized values are bit-identical: -0 -> +0 and exponent 31
// (Inf/NaN codes) -> (1 + m/1024) * 2^16 instead of Inf/NaN.
__device__ __forceinline__ float f16_ref(uint32_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 0x1p-24f;  // exact: m < 2^10
        return (s && m) ? -v : v;
    }
    return __builtin_bit_cast(float, (s << 31) | ((e + 112u) << 23) | (m << 13));
}
template <bool EXACT>
__device__ __forceinline__ float f16(uint32_t h) {
    if constexpr (EXACT) return f16_ref(h);
    else return f16_hw(h);
}

__device__ __forceinline__ float ubyte(uint32_t w, int b) {
    return (float)((w >> (8 * b)) & 0xFFu);
}

// Nibble unpack of 4 bytes: low nibbles to slots [lo, lo+4), high to [hi, hi+4).
// The masks go through an opaque v_and so the compiler keeps the byte
// extracts as v_cvt_f32_ubyte{0..3} instead of folding them into bfe + cvt.
__device__ __forceinline__ uint32_t opaque_and(uint32_t a, uint32_t m) {
    uint32_t r;
    asm volatile("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(m));
    return r;
}
__device__ __forceinline__ void nibbles(uint32_t w, float* q, int lo, int hi) {
    uint32_t l = opaque_and(w, 0x0F0F0F0Fu), h = opaque_and(w >> 4, 0x0F0F0F0Fu);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        q[lo + b] = ubyte(l, b);
        q[hi + b] = ubyte(h, b);
    }
}

template <int F>
struct Fmt;

// ---------------------------------------------------------------- Q4_0 (18 B)
template <>
struct Fmt<Q4_0> {
    static constexpr int BE = 32, BB = 18, NG = 1;
    struct Raw {
        uint32_t d;
        uint4 qs;
    };
    __device__ static int k_of(int u, int s) { return 32 * u + s; }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 18 * u;
        return Raw{ldg16<NT>(p), ldg128<NT>(p + 2)};
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int, float* q, float* A, float* B) {
        float d = f16<EXACT>(r.d);
        nibbles(r.qs.x, q, 0, 16);
        nibbles(r.qs.y, q, 4, 20);
        nibbles(r.qs.z, q, 8, 24);
        nibbles(r.qs.w, q, 12, 28);
        A[0] = d;
        B[0] = -8.0f * d;
    }
    // Bit-exact dequantized value of a slot (reference expression order).
    __device__ static float value(float q, float A, float) { return (q - 8.0f) * A; }
};

// ---------------------------------------------------------------- Q4_1 (20 B)
template <>
struct Fmt<Q4_1> {
    static constexpr int BE = 32, BB = 20, NG = 1;
    struct Raw {
        uint32_t dm;
        uint4 qs;
    };
    __device__ static int k_of(int u, int s) { return 32 * u + s; }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 20 * u;
        return Raw{ldg32<NT>(p), ldg128<NT>(p + 4)};
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int, float* q, float* A, float* B) {
        nibbles(r.qs.x, q, 0, 16);
        nibbles(r.qs.y, q, 4, 20);
        nibbles(r.qs.z, q, 8, 24);
        nibbles(r.qs.w, q, 12, 28);
        A[0] = f16<EXACT>(r.dm & 0xFFFFu);
        B[0] = f16<EXACT>(r.dm >> 16);
    }
    // q*d is exact, so the fused form rounds exactly like q*d + m.
    __device__ static float value(float q, float A, float B) { return __builtin_fmaf(q, A, B); }
};

// ---------------------------------------------------------------- Q8_0 (34 B)
template <>
struct Fmt<Q8_0> {
    static constexpr int BE = 32, BB = 34, NG = 1;
    struct Raw {
        uint32_t d;
        uint4 q0, q1;
    };
    __device__ static int k_of(int u, int s) { return 32 * u + s; }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 34 * u;
        return Raw{ldg16<NT>(p), ldg128<NT>(p + 2), ldg128<NT>(p + 18)};
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int, float* q, float* A, float* B) {
        const uint32_t v[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t b = v[i] ^ 0x80808080u;  // int8 q -> unsigned q + 128
#pragma unroll
            for (int j = 0; j < 4; ++j) q[4 * i + j] = ubyte(b, j);
        }
        float d = f16<EXACT>(r.d);
        A[0] = d;
        B[0] = -128.0f * d;
    }
    __device__ static float value(float q, float A, float) { return (q - 128.0f) * A; }
};

// --------------------------------------------------------------- Q4_K (144 B)
// Super-block: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16.  Unit j of
// a super-block reads qs[16j, 16j+16): its low nibbles are elements
// 64g + 16h + [0,16) (sub-block 2g), its high nibbles 64g + 32 + 16h + [0,16)
// (sub-block 2g+1), g = j/2, h = j%2 (matmul.cpp:361-373).
template <>
struct Fmt<Q4_K> {
    static constexpr int BE = 256, BB = 144, NG = 2;
    struct Raw {
        uint4 hdr;
        uint4 qs;
    };
    __device__ static int k_of(int u, int s) {
        int sb = u >> 3, j = u & 7, g = j >> 1, h = j & 1;
        return 256 * sb + 64 * g + 16 * h + (s < 16 ? s : 16 + s);
    }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 144 * (u >> 3);
        return Raw{ldg128<NT>(p), ldg128<NT>(p + 16 + 16 * (u & 7))};
    }
    // get_scale_min_k4 (matmul.cpp:232-240) for the pair (2g, 2g+1).
    __device__ static void scale_min(const uint4& hdr, int g, uint32_t& sa, uint32_t& ma,
                                     uint32_t& sb, uint32_t& mb) {
        const uint32_t q0 = hdr.y, q4 = hdr.z, q8 = hdr.w;  // scales bytes 0-3, 4-7, 8-11
        if (g < 2) {
            int sh = 16 * g;  // byte 2g
            sa = (q0 >> sh) & 63u;
            ma = (q4 >> sh) & 63u;
            sb = (q0 >> (sh + 8)) & 63u;
            mb = (q4 >> (sh + 8)) & 63u;
        } else {
            int sh = 16 * (g - 2);  // byte index is-4 = 2g-4
            uint32_t a8 = q8 >> sh, a0 = q0 >> sh, a4 = q4 >> sh;
            sa = (a8 & 0xFu) | (((a0 >> 6) & 3u) << 4);
            ma = ((a8 >> 4) & 0xFu) | (((a4 >> 6) & 3u) << 4);
            sb = ((a8 >> 8) & 0xFu) | (((a0 >> 14) & 3u) << 4);
            mb = ((a8 >> 12) & 0xFu) | (((a4 >> 14) & 3u) << 4);
        }
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int u, float* q, float* A, float* B) {
        nibbles(r.qs.x, q, 0, 16);
        nibbles(r.qs.y, q, 4, 20);
        nibbles(r.qs.z, q, 8, 24);
        nibbles(r.qs.w, q, 12, 28);
        float d = f16<EXACT>(r.hdr.x & 0xFFFFu), dmin = f16<EXACT>(r.hdr.x >> 16);
        uint32_t sa, ma, sb, mb;
        scale_min(r.hdr, (u & 7) >> 1, sa, ma, sb, mb);
        A[0] = d * (float)sa;
        B[0] = -(dmin * (float)ma);
        A[1] = d * (float)sb;
        B[1] = -(dmin * (float)mb);
    }
    // (d*sc)*q is exact, so fma(A, q, -dmin*m) rounds like d1*q - m1.
    __device__ static float value(float q, float A, float B) { return __builtin_fmaf(A, q, B); }
};

// --------------------------------------------------------------- Q6_K (210 B)
// Super-block: ql[128] @0, qh[64] @128, sc int8[16] @192, d f16 @208.  Unit
// j = 4n + c covers l in [8c, 8c+8) of half n: slot 8g + e holds element
// 128n + 32g + 8c + e, g = 0..3 (matmul.cpp:259-276).
template <>
struct Fmt<Q6_K> {
    static constexpr int BE = 256, BB = 210, NG = 4;
    struct Raw {
        uint2 ql_lo, ql_hi, qh, sc;
        uint32_t d;
    };
    __device__ static int k_of(int u, int s) {
        int sb = u >> 3, j = u & 7, n = j >> 2, c = j & 3;
        return 256 * sb + 128 * n + 32 * (s >> 3) + 8 * c + (s & 7);
    }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 210 * (u >> 3);
        int j = u & 7, n = j >> 2, l0 = 8 * (j & 3);
        return Raw{ldg64<NT>(p + 64 * n + l0), ldg64<NT>(p + 64 * n + 32 + l0),
                   ldg64<NT>(p + 128 + 32 * n + l0), ldg64<NT>(p + 192 + 8 * n),
                   ldg16<NT>(p + 208)};
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int u, float* q, float* A, float* B) {
        const uint32_t a[2] = {r.ql_lo.x, r.ql_lo.y}, b[2] = {r.ql_hi.x, r.ql_hi.y},
                       h[2] = {r.qh.x, r.qh.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            uint32_t q1 = (a[i] & 0x0F0F0F0Fu) | ((h[i] & 0x03030303u) << 4);
            uint32_t q2 = (b[i] & 0x0F0F0F0Fu) | ((h[i] & 0x0C0C0C0Cu) << 2);
            uint32_t q3 = ((a[i] >> 4) & 0x0F0F0F0Fu) | (h[i] & 0x30303030u);
            uint32_t q4 = ((b[i] >> 4) & 0x0F0F0F0Fu) | ((h[i] >> 2) & 0x30303030u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                q[0 + 4 * i + e] = ubyte(q1, e);
                q[8 + 4 * i + e] = ubyte(q2, e);
                q[16 + 4 * i + e] = ubyte(q3, e);
                q[24 + 4 * i + e] = ubyte(q4, e);
            }
        }
        float d = f16<EXACT>(r.d);
        int is = (u & 3) >> 1;  // l/16 for l in [8c, 8c+8)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            int t = is + 2 * g;  // sc[8n + is + 2g]
            uint32_t word = t < 4 ? r.sc.x : r.sc.y;
            int sc = (int)(int8_t)((word >> (8 * (t & 3))) & 0xFFu);
            A[g] = d * (float)sc;
            B[g] = -32.0f * A[g];
        }
    }
    // (d*sc) exact; one rounding of (d*sc)*(q-32), as the reference.
    __device__ static float value(float q, float A, float) { return A * (q - 32.0f); }
};


// ------------------------------------------------- bit helpers (5-bit, IQ4_NL)
// Bits 0..3 of v spread to bit 0 of bytes 0..3.  The multiplier places bit b
// at 8 b (and at b + 7 j for j != b, which the mask drops); the partial
// products never overlap, so there are no carries.
__device__ __forceinline__ uint32_t spread4(uint32_t v) {
    return __umul24(v & 15u, 0x00204081u) & 0x01010101u;
}
// 5-bit codes of four slots: the nibbles n (in bits 0..3 of each byte) with
// bits 0..3 of hb as bit 4.
__device__ __forceinline__ uint32_t five_bit(uint32_t n, uint32_t hb) {
    return n | (spread4(hb) << 4);
}

// IQ4_NL table (matmul.cpp:849-851) as int8 bytes, four per dword.
constexpr uint32_t IQ4T0 = 0xBFAD9881u, IQ4T1 = 0xF6EADDCFu, IQ4T2 = 0x26190D01u,
                   IQ4T3 = 0x71594535u;
// Four 4-bit indices (bits 0..3 of each byte of idx) -> four int8 table values.
// v_perm_b32 picks bytes 0..7 of a dword pair: entries 0..7 and 8..15 come
// from two lookups on idx & 7, and bit 3 of each index selects between them.
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t idx) {
    const uint32_t lo7 = idx & 0x07070707u;
    const uint32_t a = __builtin_amdgcn_perm(IQ4T1, IQ4T0, lo7);
    const uint32_t b = __builtin_amdgcn_perm(IQ4T3, IQ4T2, lo7);
    const uint32_t sel = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (b & sel) | (a & ~sel);
}

// ---------------------------------------------------------------- Q5_0 (22 B)
// Block: d f16 @0, qh u32 @2, qs[16] @6.  Element j: nibble j % 16 of qs
// (low for j < 16) plus 16 times bit j of qh.  Slots are elements.
template <>
struct Fmt<Q5_0> {
    static constexpr int BE = 32, BB = 22, NG = 1;
    struct Raw {
        uint32_t d, qh;
        uint4 qs;
    };
    __device__ static int k_of(int u, int s) { return 32 * u + s; }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 22 * u;
        return Raw{ldg16<NT>(p), ldg32<NT>(p + 2), ldg128<NT>(p + 6)};
    }
    // 5-bit codes of slots 4i..4i+3 (lo) and 16+4i.. (hi)
    __device__ static void codes(uint32_t w, uint32_t qh, int i, uint32_t& lo, uint32_t& hi) {
        lo = five_bit(w & 0x0F0F0F0Fu, qh >> (4 * i));
        hi = five_bit((w >> 4) & 0x0F0F0F0Fu, qh >> (16 + 4 * i));
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int, float* q, float* A, float* B) {
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo, hi;
            codes(w[i], r.qh, i, lo, hi);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                q[4 * i + b] = ubyte(lo, b);
                q[16 + 4 * i + b] = ubyte(hi, b);
            }
        }
        const float d = f16<EXACT>(r.d);
        A[0] = d;
        B[0] = -16.0f * d;
    }
    __device__ static float value(float q, float A, float) { return (q - 16.0f) * A; }
};

// ---------------------------------------------------------------- Q5_1 (24 B)
// Block: d f16 @0, m f16 @2, qh u32 @4, qs[16] @8; codes as Q5_0.
template <>
struct Fmt<Q5_1> {
    static constexpr int BE = 32, BB = 24, NG = 1;
    struct Raw {
        uint32_t dm, qh;
        uint4 qs;
    };
    __device__ static int k_of(int u, int s) { return 32 * u + s; }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 24 * u;
        return Raw{ldg32<NT>(p), ldg32<NT>(p + 4), ldg128<NT>(p + 8)};
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int, float* q, float* A, float* B) {
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo, hi;
            Fmt<Q5_0>::codes(w[i], r.qh, i, lo, hi);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                q[4 * i + b] = ubyte(lo, b);
                q[16 + 4 * i + b] = ubyte(hi, b);
            }
        }
        A[0] = f16<EXACT>(r.dm & 0xFFFFu);
        B[0] = f16<EXACT>(r.dm >> 16);
    }
    // q*d is exact (5 x 11 bits), so the fused form rounds like q*d + m.
    __device__ static float value(float q, float A, float B) { return __builtin_fmaf(q, A, B); }
};

// -------------------------------------------------------------- IQ4_NL (18 B)
// Block: d f16 @0, qs[16] @2; element j is T[nibble j % 16] (low for j < 16).
template <>
struct Fmt<IQ4_NL> {
    static constexpr int BE = 32, BB = 18, NG = 1;
    struct Raw {
        uint32_t d;
        uint4 qs;
    };
    __device__ static int k_of(int u, int s) { return 32 * u + s; }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 18 * u;
        return Raw{ldg16<NT>(p), ldg128<NT>(p + 2)};
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int, float* q, float* A, float* B) {
        const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = iq4_lookup(w[i]), hi = iq4_lookup(w[i] >> 4);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                q[4 * i + b] = (float)(int8_t)(lo >> (8 * b));
                q[16 + 4 * i + b] = (float)(int8_t)(hi >> (8 * b));
            }
        }
        A[0] = f16<EXACT>(r.d);
        B[0] = 0.0f;
    }
    __device__ static float value(float q, float A, float) { return A * q; }
};

// --------------------------------------------------------------- Q3_K (110 B)
// Super-block: hmask[32] @0, qs[64] @32, scales[12] @96, d f16 @108.  Element
// 128 n + 32 j + l (l < 32): 2-bit code at bit 2 j of qs[32 n + l], plus 4
// when bit 4 n + j of hmask[l] is set (the reference subtracts 4 when it is
// clear), sub-scale 8 n + 2 j + l / 16 (matmul.cpp:284-338).  Unit
// u = 4 n + c covers l in [8c, 8c+8) of half n: slot 8 j + e holds element
// 128 n + 32 j + 8 c + e, group j, the same walk as Q6_K.
template <>
struct Fmt<Q3_K> {
    static constexpr int BE = 256, BB = 110, NG = 4;
    struct Raw {
        uint2 qs, hm;
        uint32_t s0, s1, s2, d;  // scale bytes 0-3, 4-7, 8-11; d
    };
    __device__ static int k_of(int u, int s) { return Fmt<Q6_K>::k_of(u, s); }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 110 * (u >> 3);
        const int j = u & 7, n = j >> 2, l0 = 8 * (j & 3);
        return Raw{ldg64<NT>(p + 32 + 32 * n + l0), ldg64<NT>(p + l0), ldg32<NT>(p + 96),
                   ldg32<NT>(p + 100), ldg32<NT>(p + 104), ldg16<NT>(p + 108)};
    }
    // Signed sub-scales of groups j = 0..3 of unit u: scale i = 8 n + 2 j + h
    // (h = l >= 16) has its low nibble in nibble n of scale byte 2 j + h and
    // its top 2 bits at bit 2 (2 n + j / 2) of byte 8 + (2 j + h) % 4.
    __device__ static void scales(const Raw& r, int u, int (&sc)[4]) {
        const int j = u & 7, n = j >> 2, h = (j & 3) >> 1;
        const uint32_t a0 = r.s0 >> (8 * h), a1 = r.s1 >> (8 * h), b = r.s2 >> (8 * h);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t lo = ((g < 2 ? a0 : a1) >> (16 * (g & 1) + 4 * n)) & 15u;
            const uint32_t hi = (b >> (16 * (g & 1) + 4 * n + 2 * (g >> 1))) & 3u;
            sc[g] = (int)(lo | (hi << 4)) - 32;
        }
    }
    // unsigned 3-bit codes (value + 4) of slots 8g + 4i .. +3
    __device__ static uint32_t codes(const Raw& r, int u, int g, int i) {
        const int n = (u & 7) >> 2;
        const uint32_t q = i ? r.qs.y : r.qs.x, h = i ? r.hm.y : r.hm.x;
        return ((q >> (2 * g)) & 0x03030303u) | (((h >> (4 * n + g)) & 0x01010101u) << 2);
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int u, float* q, float* A, float* B) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t c = codes(r, u, g, i);
#pragma unroll
                for (int e = 0; e < 4; ++e) q[8 * g + 4 * i + e] = ubyte(c, e);
            }
        int sc[4];
        scales(r, u, sc);
        const float d = f16<EXACT>(r.d);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            A[g] = d * (float)sc[g];
            B[g] = -4.0f * A[g];
        }
    }
    __device__ static float value(float q, float A, float) { return A * (q - 4.0f); }
};

// --------------------------------------------------------------- Q5_K (176 B)
// Super-block: d f16 @0, dmin f16 @2, scales[12] @4, qh[32] @16, qs[128] @48.
// Element 64 g + 32 h + l: nibble h of qs[32 g + l] plus 16 times bit 2 g + h
// of qh[l], scale/min pair 2 g + h (matmul.cpp:382-415).  Units as Q4_K:
// unit j = 2 g + t reads qs[32 g + 16 t, +16) and qh[16 t, +16).
template <>
struct Fmt<Q5_K> {
    static constexpr int BE = 256, BB = 176, NG = 2;
    struct Raw {
        uint4 hdr, qs, qh;
    };
    __device__ static int k_of(int u, int s) { return Fmt<Q4_K>::k_of(u, s); }
    template <bool NT = false>
    __device__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + 176 * (u >> 3);
        const int j = u & 7;
        return Raw{ldg128<NT>(p), ldg128<NT>(p + 48 + 16 * j), ldg128<NT>(p + 16 + 16 * (j & 1))};
    }
    // 5-bit codes: slots 4i.. (low nibbles, bit 2g of qh) and 16+4i.. (bit 2g+1)
    __device__ static void codes(const Raw& r, int u, int i, uint32_t& lo, uint32_t& hi) {
        const int g = (u & 7) >> 1;
        const uint32_t w = i == 0 ? r.qs.x : i == 1 ? r.qs.y : i == 2 ? r.qs.z : r.qs.w;
        const uint32_t h = i == 0 ? r.qh.x : i == 1 ? r.qh.y : i == 2 ? r.qh.z : r.qh.w;
        lo = (w & 0x0F0F0F0Fu) | (((h >> (2 * g)) & 0x01010101u) << 4);
        hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * g + 1)) & 0x01010101u) << 4);
    }
    template <bool EXACT>
    __device__ static void decode(const Raw& r, int u, float* q, float* A, float* B) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t lo, hi;
            codes(r, u, i, lo, hi);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                q[4 * i + b] = ubyte(lo, b);
                q[16 + 4 * i + b] = ubyte(hi, b);
            }
        }
        const float d = f16<EXACT>(r.hdr.x & 0xFFFFu), dmin = f16<EXACT>(r.hdr.x >> 16);
        uint32_t sa, ma, sb, mb;
        Fmt<Q4_K>::scale_min(r.hdr, (u & 7) >> 1, sa, ma, sb, mb);
        A[0] = d * (float)sa;
        B[0] = -(dmin * (float)ma);
        A[1] = d * (float)sb;
        B[1] = -(dmin * (float)mb);
    }
    // (d*sc)*q is exact (11 + 6 + 5 bits), so fma rounds like d1*q - m1.
    __device__ static float value(float q, float A, float B) { return __builtin_fmaf(A, q, B); }
};

// ---------------------------------------------------------------- int8 limbs
// Batch-1 path: the activations of one 32-slot unit are staged as three int8
// limbs a1, a2, a3 (slot order, 4 slots per dword) and a power-of-two scale
// s1:  x_s ~= s1 * (a1_s + a2_s / 2^7 + a3_s / 2^14), |a| <= 127, with a
// residual below s1 * 2^-15 <= 2^-14 * max|x| / 127 of the unit.  A unit's
// contribution  sum_g A_g P_g + B_g S_g  then needs P_g = sum x_s q_s only,
// which is  s1 * (D1 + D2 / 2^7 + D3 / 2^14)  with D_l = sum a_l,s q_s exact
// int32 dot products (v_dot4c_i32_i8: 4 multiply-adds per instruction).
struct Limbs {
    int l1[8], l2[8], l3[8];  // dword i = slots 4i..4i+3
    float s1;
    float S[4];
};

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}
__device__ __forceinline__ float limb_sum(int d1, int d2, int d3) {
    return __builtin_fmaf((float)d3, 0x1p-14f, __builtin_fmaf((float)d2, 0x1p-7f, (float)d1));
}

// The same sum times 2^14 for 4-bit quants, combined in integers first: with
// q <= 15 each |d| <= 32 * 127 * 15, so d1 2^14 + d2 2^7 + d3 < 2^30 fits an
// int32, and one conversion replaces three (rounding: 2^-24 relative).
__device__ __forceinline__ float limb_sum4(int d1, int d2, int d3) {
    return (float)((d1 << 14) + (d2 << 7) + d3);
}
// q dword holding slots 4i..4i+3 (bytes 0..127 as signed int8), group g
template <int G>
__device__ __forceinline__ void acc_dword(int q, int i, const Limbs& L, int (&D)[3][G], int g) {
    D[0][g] = sdot4(q, L.l1[i], D[0][g]);
    D[1][g] = sdot4(q, L.l2[i], D[1][g]);
    D[2][g] = sdot4(q, L.l3[i], D[2][g]);
}

// Nibble formats (Q4_0, Q4_1, Q4_K): qs dword i -> low nibbles are slots
// 4i..4i+3 (group 0 for Q4_K), high nibbles slots 16+4i.. (group 1 for Q4_K).
template <int G>
__device__ __forceinline__ void nibble_dots(const uint4& qs, const Limbs& L, int (&D)[3][G]) {
    const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int lo = (int)(w[i] & 0x0F0F0F0Fu), hi = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
        acc_dword<G>(lo, i, L, D, 0);
        acc_dword<G>(hi, 4 + i, L, D, G - 1);
    }
}

template <int F>
__device__ __forceinline__ float limb_dot(const typename Fmt<F>::Raw& r, int u, const Limbs& L);

template <>
__device__ __forceinline__ float limb_dot<Q4_0>(const Fmt<Q4_0>::Raw& r, int, const Limbs& L) {
    int D[3][1] = {{0}, {0}, {0}};
    nibble_dots<1>(r.qs, L, D);
    const float d = f16_hw(r.d);
    // d * (sum x q) - 8 d * (sum x)
    return __builtin_fmaf(d * L.s1 * 0x1p-14f, limb_sum4(D[0][0], D[1][0], D[2][0]),
                          -8.0f * d * L.S[0]);
}

template <>
__device__ __forceinline__ float limb_dot<Q4_1>(const Fmt<Q4_1>::Raw& r, int, const Limbs& L) {
    int D[3][1] = {{0}, {0}, {0}};
    nibble_dots<1>(r.qs, L, D);
    const float d = f16_hw(r.dm & 0xFFFFu), m = f16_hw(r.dm >> 16);
    return __builtin_fmaf(d * L.s1 * 0x1p-14f, limb_sum4(D[0][0], D[1][0], D[2][0]), m * L.S[0]);
}

template <>
__device__ __forceinline__ float limb_dot<Q8_0>(const Fmt<Q8_0>::Raw& r, int, const Limbs& L) {
    int D[3][1] = {{0}, {0}, {0}};
    const uint32_t v[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) acc_dword<1>((int)v[i], i, L, D, 0);
    return f16_hw(r.d) * L.s1 * limb_sum(D[0][0], D[1][0], D[2][0]);
}

template <>
__device__ __forceinline__ float limb_dot<Q4_K>(const Fmt<Q4_K>::Raw& r, int u, const Limbs& L) {
    int D[3][2] = {{0, 0}, {0, 0}, {0, 0}};
    nibble_dots<2>(r.qs, L, D);
    const float d = f16_hw(r.hdr.x & 0xFFFFu), dmin = f16_hw(r.hdr.x >> 16);
    uint32_t sa, ma, sb, mb;
    Fmt<Q4_K>::scale_min(r.hdr, (u & 7) >> 1, sa, ma, sb, mb);
    const float ds = d * L.s1 * 0x1p-14f;
    float acc = -(dmin * (float)ma) * L.S[0];
    acc = __builtin_fmaf(-(dmin * (float)mb), L.S[1], acc);
    acc = __builtin_fmaf(ds * (float)sa, limb_sum4(D[0][0], D[1][0], D[2][0]), acc);
    return __builtin_fmaf(ds * (float)sb, limb_sum4(D[0][1], D[1][1], D[2][1]), acc);
}

template <>
__device__ __forceinline__ float limb_dot<Q6_K>(const Fmt<Q6_K>::Raw& r, int u, const Limbs& L) {
    const uint32_t a[2] = {r.ql_lo.x, r.ql_lo.y}, b[2] = {r.ql_hi.x, r.ql_hi.y},
                   h[2] = {r.qh.x, r.qh.y};
    int q[4][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        q[0][i] = (int)((a[i] & 0x0F0F0F0Fu) | ((h[i] & 0x03030303u) << 4));
        q[1][i] = (int)((b[i] & 0x0F0F0F0Fu) | ((h[i] & 0x0C0C0C0Cu) << 2));
        q[2][i] = (int)(((a[i] >> 4) & 0x0F0F0F0Fu) | (h[i] & 0x30303030u));
        q[3][i] = (int)(((b[i] >> 4) & 0x0F0F0F0Fu) | ((h[i] >> 2) & 0x30303030u));
    }
    // Group g (slots 8g .. 8g+7) sums E_g = D1 2^14 + D2 2^7 + D3 in one int32
    // chain: limb-1 dots, shift by 7, limb-2 dots, shift, limb-3 dots.  With
    // q <= 63, |a1| <= 127, |a2|, |a3| <= 64: |E_g| <= 8 * 63 * (127 * 2^14 +
    // 64 * 2^7 + 64) < 2^30.
    float E[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        int e = sdot4(q[g][1], L.l1[2 * g + 1], sdot4(q[g][0], L.l1[2 * g], 0));
        e = sdot4(q[g][1], L.l2[2 * g + 1], sdot4(q[g][0], L.l2[2 * g], e << 7));
        e = sdot4(q[g][1], L.l3[2 * g + 1], sdot4(q[g][0], L.l3[2 * g], e << 7));
        E[g] = (float)e;  // rounding: 2^-24 relative
    }
    const int is = (u & 3) >> 1;
    float sc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int t = is + 2 * g;
        const uint32_t word = t < 4 ? r.sc.x : r.sc.y;
        sc[g] = (float)(int)(int8_t)((word >> (8 * (t & 3))) & 0xFFu);
    }
    float P = sc[0] * E[0], sS = sc[0] * L.S[0];
#pragma unroll
    for (int g = 1; g < 4; ++g) {
        P = __builtin_fmaf(sc[g], E[g], P);
        sS = __builtin_fmaf(sc[g], L.S[g], sS);
    }
    const float d = f16_hw(r.d);
    // d * sum_g sc_g (P_g - 32 S_g)
    return d * __builtin_fmaf(L.s1 * 0x1p-14f, P, -32.0f * sS);
}

// 5-bit nibble formats (Q5_0, Q5_1): one group; |sum| <= 32 * 127 * 31.
template <class Fm>
__device__ __forceinline__ void five_bit_dots(const uint4& qs, uint32_t qh, const Limbs& L,
                                              int (&D)[3][1]) {
    const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo, hi;
        Fmt<Q5_0>::codes(w[i], qh, i, lo, hi);
        acc_dword<1>((int)lo, i, L, D, 0);
        acc_dword<1>((int)hi, 4 + i, L, D, 0);
    }
}

template <>
__device__ __forceinline__ float limb_dot<Q5_0>(const Fmt<Q5_0>::Raw& r, int, const Limbs& L) {
    int D[3][1] = {{0}, {0}, {0}};
    five_bit_dots<Fmt<Q5_0>>(r.qs, r.qh, L, D);
    const float d = f16_hw(r.d);
    return __builtin_fmaf(d * L.s1, limb_sum(D[0][0], D[1][0], D[2][0]), -16.0f * d * L.S[0]);
}

template <>
__device__ __forceinline__ float limb_dot<Q5_1>(const Fmt<Q5_1>::Raw& r, int, const Limbs& L) {
    int D[3][1] = {{0}, {0}, {0}};
    five_bit_dots<Fmt<Q5_1>>(r.qs, r.qh, L, D);
    const float d = f16_hw(r.dm & 0xFFFFu), m = f16_hw(r.dm >> 16);
    return __builtin_fmaf(d * L.s1, limb_sum(D[0][0], D[1][0], D[2][0]), m * L.S[0]);
}

template <>
__device__ __forceinline__ float limb_dot<IQ4_NL>(const Fmt<IQ4_NL>::Raw& r, int, const Limbs& L) {
    int D[3][1] = {{0}, {0}, {0}};
    const uint32_t w[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc_dword<1>((int)iq4_lookup(w[i]), i, L, D, 0);
        acc_dword<1>((int)iq4_lookup(w[i] >> 4), 4 + i, L, D, 0);
    }
    return f16_hw(r.d) * L.s1 * limb_sum(D[0][0], D[1][0], D[2][0]);
}

template <>
__device__ __forceinline__ float limb_dot<Q3_K>(const Fmt<Q3_K>::Raw& r, int u, const Limbs& L) {
    int D[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc_dword<4>((int)Fmt<Q3_K>::codes(r, u, g, i), 2 * g + i, L, D, g);
    int sc[4];
    Fmt<Q3_K>::scales(r, u, sc);
    // sub-scales folded in integers: |sum_g sc_g D_g| <= 4 * 32 * 8 * 127 * 7
    int E[3];
    float sS = 0.0f;
#pragma unroll
    for (int l = 0; l < 3; ++l) {
        int e = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) e = __mul24(sc[g], D[l][g]) + e;
        E[l] = e;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) sS = __builtin_fmaf((float)sc[g], L.S[g], sS);
    // d * sum_g sc_g (P_g - 4 S_g), P_g over the unsigned codes
    return f16_hw(r.d) * __builtin_fmaf(L.s1, limb_sum(E[0], E[1], E[2]), -4.0f * sS);
}

template <>
__device__ __forceinline__ float limb_dot<Q5_K>(const Fmt<Q5_K>::Raw& r, int u, const Limbs& L) {
    int D[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo, hi;
        Fmt<Q5_K>::codes(r, u, i, lo, hi);
        acc_dword<2>((int)lo, i, L, D, 0);
        acc_dword<2>((int)hi, 4 + i, L, D, 1);
    }
    const float d = f16_hw(r.hdr.x & 0xFFFFu), dmin = f16_hw(r.hdr.x >> 16);
    uint32_t sa, ma, sb, mb;
    Fmt<Q4_K>::scale_min(r.hdr, (u & 7) >> 1, sa, ma, sb, mb);
    const float ds = d * L.s1;
    float acc = -(dmin * (float)ma) * L.S[0];
    acc = __builtin_fmaf(-(dmin * (float)mb), L.S[1], acc);
    acc = __builtin_fmaf(ds * (float)sa, limb_sum(D[0][0], D[1][0], D[2][0]), acc);
    return __builtin_fmaf(ds * (float)sb, limb_sum(D[0][1], D[1][1], D[2][1]), acc);
}

}  // namespace fq
