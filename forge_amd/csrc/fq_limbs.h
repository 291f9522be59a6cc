// fq_limbs.h -- activation staging shared by the batch-1 kernels: the int8
// limb records (see Limbs in fq_formats.h), the 64-lane DPP sum and the
// scalar-path bias pointer type.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fq_formats.h"

namespace fq {

// Work-group barrier that orders LDS accesses only.  __syncthreads() also
// waits for every global load in flight (its release fence covers global
// memory), which would stall a kernel that issues weight loads before the
// barrier until they have all arrived.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Full 64-lane sum; the result is valid in lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
    return v;
}

// Stage x as int8 limbs (see Limbs in fq_formats.h).  Record of unit u at
// byte 144*u: a1[32] @0, a2[32] @32, a3[32] @64, s1 @96, S[4] @100.  Eight
// lanes build one record: lane i owns slots 4i .. 4i+3, which are four
// consecutive activations for every format (one float4 load), and writes one
// aligned dword of each limb.  The unit max and the group sums are all-reduce
// trees over the eight lanes in DPP (quad_perm, row_half_mirror): no LDS
// traffic and a fixed order, so the staging is deterministic.
//
// Staging is split in two so the caller can put the first weight loads
// between them: stage_load() issues every activation load first (they are
// then older than the weight loads in the in-order memory counter, so
// stage_build() never waits for weight bytes), stage_build() computes and
// writes the records.
constexpr int RECB = 144;
constexpr int XPMAX = 10;  // activation loads a thread keeps in flight

// Task t = 8 w + i: slots 4i .. 4i+3 of record w.  With U > 0 the records
// of several tokens follow each other (U records, K activations per token);
// U = 0: one token.  w0 offsets the record index within a token.
template <class Fm>
__device__ __forceinline__ float4 stage_x4(const float* __restrict__ x, int w0, int t, int U,
                                           int K) {
    const int w = t >> 3, i = t & 7;
    int m = 0;
    if (U > 0) m = w / U;  // uniform branch: no division for one token
    return *reinterpret_cast<const float4*>(x + (size_t)m * K + Fm::k_of(w0 + w - m * U, 4 * i));
}

template <class Fm, int WG>
struct XStage {
    float4 v[XPMAX];
};

// nrec records in all; U records per token (0: one token).
template <class Fm, int WG>
__device__ __forceinline__ void stage_load(XStage<Fm, WG>& st, const float* __restrict__ x,
                                           int nrec, int w0, int U = 0, int K = 0) {
    const int tasks = 8 * nrec;
#pragma unroll
    for (int p = 0; p < XPMAX; ++p)
        if (p * WG < tasks)  // uniform
            st.v[p] = stage_x4<Fm>(x, w0, min(p * WG + (int)threadIdx.x, tasks - 1), U, K);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                          0xf, 0xf, false));
}

// all-reduce over aligned groups of 2, 4 or 8 lanes
template <int LANES>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);                      // quad_perm [1,0,3,2]
    if (LANES >= 4) v += dpp_f<0x4E>(v);      // quad_perm [2,3,0,1]
    if (LANES >= 8) v += dpp_f<0x141>(v);     // row_half_mirror
    return v;
}
__device__ __forceinline__ float group_max8(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    return fmaxf(v, dpp_f<0x141>(v));
}

__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
    return ((uint32_t)(int)a & 0xFFu) | (((uint32_t)(int)b & 0xFFu) << 8) |
           (((uint32_t)(int)c & 0xFFu) << 16) | ((uint32_t)(int)d << 24);
}

// The limbs of four consecutive activations (one float4) of a 32-slot unit
// whose eight aligned lanes work together: a1, a2, a3 packed four to a dword,
// the unit's power-of-two scale s1, and the sum of the activations over
// aligned groups of GS slots (GS / 4 lanes).
struct LimbQuad {
    uint32_t a1, a2, a3;
    float s1, gs;
};

template <int GS>
__device__ __forceinline__ LimbQuad limb_quad(float4 xv) {
    float m = fmaxf(fmaxf(__builtin_fabsf(xv.x), __builtin_fabsf(xv.y)),
                    fmaxf(__builtin_fabsf(xv.z), __builtin_fabsf(xv.w)));
    m = group_max8(m);
    int e = (int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xFFu);
    e = max(e, 21);  // keeps s1 * 2^-14 a normal number
    float s1 = __builtin_bit_cast(float, (uint32_t)(e - 6) << 23);
    if (m >= 127.5f * s1) {
        ++e;
        s1 *= 2.0f;
    }
    const float inv = __builtin_bit_cast(float, (uint32_t)(254 - (e - 6)) << 23);
    const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
    float a1[4], a2[4], a3[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a1[j] = __builtin_rintf(xs[j] * inv);
        const float r1 = __builtin_fmaf(-a1[j], s1, xs[j]);
        a2[j] = __builtin_rintf(r1 * (inv * 128.0f));
        const float r2 = __builtin_fmaf(-a2[j], s1 * 0x1p-7f, r1);
        a3[j] = __builtin_rintf(r2 * (inv * 16384.0f));
    }
    if (!(m <= 3.0e38f)) s1 = __builtin_nanf("");  // Inf/NaN in x propagates
    float gs = (xv.x + xv.y) + (xv.z + xv.w);
    if (GS >= 8) gs = group_sum<GS / 4>(gs);
    return LimbQuad{pack4(a1[0], a1[1], a1[2], a1[3]), pack4(a2[0], a2[1], a2[2], a2[3]),
                    pack4(a3[0], a3[1], a3[2], a3[3]), s1, gs};
}

// Nibble records (record traits with NIB = true: the 4-bit formats, dotted
// with v_dot8_i32_i4).  The unit's activations become n = rint(x / s1),
// s1 = 2^(ilogb(max |x|) - 21), so |n| < 2^22, held as six signed hex digits
// n = sum_i a_i 16^i, a_i in [-8, 7] (from u = n + 0x888888, whose nibble i
// is a_i + 8).  Limb i takes bytes 16 i .. 16 i + 15 of the record, dword k
// holding the digits of elements 4 k, 4 k + 16, 4 k + 1, 4 k + 17, ... in
// nibble order: the order of a 16-byte block of low / high code nibbles.
// s1 @96 and the unit sum S @100 as in the byte records.
template <class Fm, class = void>
struct NibRec : std::false_type {};
template <class Fm>
struct NibRec<Fm, std::void_t<decltype(Fm::NIB)>> : std::bool_constant<Fm::NIB> {};

// Every lane of the wave runs it (the ds_swizzle exchange and the DPP group
// reductions read the other lanes); `live` only gates the record writes.
__device__ __forceinline__ void build_nib(uint8_t* rec, float4 xv, int i, bool live) {
    float m = fmaxf(fmaxf(__builtin_fabsf(xv.x), __builtin_fabsf(xv.y)),
                    fmaxf(__builtin_fabsf(xv.z), __builtin_fabsf(xv.w)));
    m = group_max8(m);
    const int e = max((int)((__builtin_bit_cast(uint32_t, m) >> 23) & 0xFFu), 22);
    float s1 = __builtin_bit_cast(float, (uint32_t)(e - 21) << 23);
    const float inv = __builtin_bit_cast(float, (uint32_t)(275 - e) << 23);
    const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
    // v = u ^ 0x888888: nibble i of v is digit a_i as a signed nibble
    uint32_t v[4], pv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        v[j] = ((uint32_t)(int)__builtin_rintf(xs[j] * inv) + 0x888888u) ^ 0x888888u;
#pragma unroll
    for (int j = 0; j < 4; ++j)  // lane i ^ 4 of the unit (ds_swizzle, xor mask 4)
        pv[j] = (uint32_t)__builtin_amdgcn_ds_swizzle((int)v[j], 0x101F);
    if (!(m <= 3.0e38f)) s1 = __builtin_nanf("");  // Inf/NaN in x propagates
    float gs = (xv.x + xv.y) + (xv.z + xv.w);
    gs = group_sum<8>(gs);
    if (!live) return;
    // lanes 0..3 hold elements 4 i .. 4 i + 3 and write dword i of limbs 0..3
    // (bytes 0, 1 of v); lanes 4..7 hold elements 16 + 4 (i - 4) .. and write
    // dword i - 4 of limbs 4, 5 (byte 2)
    const bool low = i < 4;
    const uint32_t* lo = low ? v : pv;
    const uint32_t* hi = low ? pv : v;
    auto gather = [](const uint32_t* q, int b) {  // byte b of q[0..3] as one dword
        const uint32_t sel = (uint32_t)b | ((uint32_t)(4 + b) << 8) | 0x0C0C0000u;
        const uint32_t t01 = __builtin_amdgcn_perm(q[1], q[0], sel);
        const uint32_t t23 = __builtin_amdgcn_perm(q[3], q[2], sel);
        return __builtin_amdgcn_perm(t23, t01, 0x05040100u);
    };
    uint32_t* r = reinterpret_cast<uint32_t*>(rec) + (i & 3);
    auto put = [&](int b) {  // limbs 2 b (low nibbles) and 2 b + 1 (high nibbles)
        const uint32_t xl = gather(lo, b), xh = gather(hi, b);
        r[4 * (2 * b)] = (xl & 0x0F0F0F0Fu) | ((xh << 4) & 0xF0F0F0F0u);
        r[4 * (2 * b + 1)] = ((xl >> 4) & 0x0F0F0F0Fu) | (xh & 0xF0F0F0F0u);
    };
    if (low) {
        put(0);
        put(1);
    } else {
        put(2);
    }
    if (i == 0) {
        *reinterpret_cast<float*>(rec + 96) = s1;
        *reinterpret_cast<float*>(rec + 100) = gs;
    }
}

template <class Fm>
__device__ __forceinline__ void build_task(uint8_t* lds, float4 xv, int t, int tasks) {
    if constexpr (NibRec<Fm>::value) {
        build_nib(lds + RECB * (t >> 3), xv, t & 7, t < tasks);
        return;
    }
    constexpr int NG = Fm::NG, GS = 32 / NG;
    const int i = t & 7;
    const LimbQuad lq = limb_quad<GS>(xv);
    if (t < tasks) {
        uint8_t* rec = lds + RECB * (t >> 3);
        reinterpret_cast<uint32_t*>(rec)[i] = lq.a1;
        reinterpret_cast<uint32_t*>(rec + 32)[i] = lq.a2;
        reinterpret_cast<uint32_t*>(rec + 64)[i] = lq.a3;
        if (i == 0) *reinterpret_cast<float*>(rec + 96) = lq.s1;
        if ((4 * i) % GS == 0) reinterpret_cast<float*>(rec + 100)[(4 * i) / GS] = lq.gs;
    }
}

template <class Fm, int WG, bool SYNC = true>
__device__ __forceinline__ void stage_build(uint8_t* lds, const XStage<Fm, WG>& st,
                                            const float* __restrict__ x, int nrec, int w0,
                                            int U = 0, int K = 0) {
    const int tasks = 8 * nrec;
#pragma unroll
    for (int p = 0; p < XPMAX; ++p) {
        if (p * WG < tasks) build_task<Fm>(lds, st.v[p], p * WG + (int)threadIdx.x, tasks);
    }
    // rows longer than XPMAX * WG / 8 records: the rest, loaded and built in turn
    for (int base = XPMAX * WG; base < tasks; base += WG) {
        const int t = base + (int)threadIdx.x;
        build_task<Fm>(lds, stage_x4<Fm>(x, w0, min(t, tasks - 1), U, K), t, tasks);
    }
    if (SYNC) __syncthreads();
}

// One-call form for kernels with nothing to overlap.
template <class Fm, int WG>
__device__ __forceinline__ void stage_limbs(uint8_t* lds, const float* __restrict__ x, int nrec,
                                            int w0 = 0) {
    XStage<Fm, WG> st;
    stage_load<Fm, WG>(st, x, nrec, w0);
    stage_build<Fm, WG>(lds, st, x, nrec, w0);
}

// The bias is read through the constant address space with a wave-uniform
// index, i.e. with a scalar load: it does not join the vector-memory queue,
// so adding it never waits on weight fetches in flight.
typedef const __attribute__((address_space(4))) float* const_fp;

__device__ __forceinline__ void read_limbs(Limbs& L, const uint8_t* lds, int u) {
    const int4* rp = reinterpret_cast<const int4*>(lds + RECB * u);
    const int4 v0 = rp[0], v1 = rp[1], v2 = rp[2], v3 = rp[3], v4 = rp[4], v5 = rp[5];
    L.l1[0] = v0.x; L.l1[1] = v0.y; L.l1[2] = v0.z; L.l1[3] = v0.w;
    L.l1[4] = v1.x; L.l1[5] = v1.y; L.l1[6] = v1.z; L.l1[7] = v1.w;
    L.l2[0] = v2.x; L.l2[1] = v2.y; L.l2[2] = v2.z; L.l2[3] = v2.w;
    L.l2[4] = v3.x; L.l2[5] = v3.y; L.l2[6] = v3.z; L.l2[7] = v3.w;
    L.l3[0] = v4.x; L.l3[1] = v4.y; L.l3[2] = v4.z; L.l3[3] = v4.w;
    L.l3[4] = v5.x; L.l3[5] = v5.y; L.l3[6] = v5.z; L.l3[7] = v5.w;
    const float4 t = reinterpret_cast<const float4*>(lds + RECB * u)[6];
    L.s1 = t.x;
    L.S[0] = t.y;
    L.S[1] = t.z;
    L.S[2] = t.w;
    L.S[3] = reinterpret_cast<const float*>(lds + RECB * u)[28];
}

// 16 / 8 bytes at a 2-byte-aligned LDS address.  A misaligned ds_read_b128
// runs at a fraction of the aligned rate (about 9 cycles of LDS issue per
// instruction against under 2 aligned), so the bytes are read as aligned
// dwords and shifted into place with v_alignbyte_b32 (shift 0 or 2 bytes).
__device__ __forceinline__ uint32_t lds_dword(const uint8_t* p) {
    return *reinterpret_cast<const __attribute__((address_space(3))) uint32_t*>(
        reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ uint4 lds16_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* q = reinterpret_cast<const uint8_t*>(a & ~(uintptr_t)3);
    const uint32_t s = (uint32_t)(a & 3);
    const uint32_t w0 = lds_dword(q), w1 = lds_dword(q + 4), w2 = lds_dword(q + 8),
                   w3 = lds_dword(q + 12), w4 = lds_dword(q + 16);
    return {__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s),
            __builtin_amdgcn_alignbyte(w3, w2, s), __builtin_amdgcn_alignbyte(w4, w3, s)};
}
__device__ __forceinline__ uint32_t lds4_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* q = reinterpret_cast<const uint8_t*>(a & ~(uintptr_t)3);
    return __builtin_amdgcn_alignbyte(lds_dword(q + 4), lds_dword(q), (uint32_t)(a & 3));
}
__device__ __forceinline__ uint2 lds8_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t* q = reinterpret_cast<const uint8_t*>(a & ~(uintptr_t)3);
    const uint32_t s = (uint32_t)(a & 3);
    const uint32_t w0 = lds_dword(q), w1 = lds_dword(q + 4), w2 = lds_dword(q + 8);
    return {__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s)};
}

}  // namespace fq
