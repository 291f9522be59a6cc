// fq_gemvp.hip -- batch-1 GEMV over the aligned device layout (fq_pack.h).
//
// Every quant payload a lane needs is a 16-byte-aligned run, so weights go
// straight from HBM to registers with coalesced 16-byte buffer loads (plus
// small dense loads of the scale arrays): no LDS staging of weights.  As in
// the row-step kernel of fq_gemv1.hip, lane l owns the same "lane units" of
// every row (l and l + 64), its activation limbs stay in registers, and a
// wave walks its rows with D rows of weight bytes in flight, reducing each row
// once with DPP and storing 64 row results at a time.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_buf.h"
#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"
#include "fq_pack.h"

namespace fq {
namespace {

// Packed traits: a "lane unit" is what one lane decodes per row step; it spans
// NREC 32-slot activation records.  Map::k_of(w, s) places slot s of record
// w for staging; NG is the number of offset groups per record.
template <int F>
struct Pk;

// The 4-bit formats take nibble records (fq_limbs.h): code dword k holds
// elements 4 k, 4 k + 16, 4 k + 1, ... in nibble order, as do the records'
// hex digits, so v_dot8_i32_i4 multiplies them in place.  q ^ 8 is the code
// q - 8 as a signed nibble; E = sum (q - 8) n over the unit, in three
// independent chains over digit pairs (2 j + 1, 2 j): P_j = 16 D_{2j+1} +
// D_{2j}, then E = 2^16 P_2 + 2^8 P_1 + P_0 (|E| < 32 * 8 * 2^22).
__device__ __forceinline__ int nib_dot(const uint4& qs, const Limbs& L) {
    const int w[4] = {(int)(qs.x ^ 0x88888888u), (int)(qs.y ^ 0x88888888u),
                      (int)(qs.z ^ 0x88888888u), (int)(qs.w ^ 0x88888888u)};
    const int* lim[3] = {L.l1, L.l2, L.l3};  // pair j: digits 2 j (dwords 0..3), 2 j + 1 (4..7)
    int P[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        int e = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) e = __builtin_amdgcn_sdot8(w[k], lim[j][4 + k], e, false);
        e *= 16;
#pragma unroll
        for (int k = 0; k < 4; ++k) e = __builtin_amdgcn_sdot8(w[k], lim[j][k], e, false);
        P[j] = e;
    }
    return P[2] * 65536 + P[1] * 256 + P[0];
}

template <>
struct Pk<Q4_0> {
    static constexpr int NREC = 1, NG = 1;
    static constexpr bool NIB = true;
    using Raw = Fmt<Q4_0>::Raw;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg16<true>(row + 16 * U + 2 * v), ldg128<true>(row + 16 * v)};
    }
    // unit v0 + l of the row whose descriptor is b (v0: the slice's first unit)
    __device__ static Raw bload(Buf b, int v0, int l, int U) {
        return Raw{bld16(b, 16 * U + 2 * v0, 2 * l), bld128(b, 16 * v0, 16 * l)};
    }
    // d (q - 8) . x = d s1 E
    __device__ static float dot(const Raw& r, int, const Limbs* L) {
        return f16_hw(r.d) * L[0].s1 * (float)nib_dot(r.qs, L[0]);
    }
};

template <>
struct Pk<Q4_1> {
    static constexpr int NREC = 1, NG = 1;
    static constexpr bool NIB = true;
    using Raw = Fmt<Q4_1>::Raw;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg32<true>(row + 16 * U + 4 * v), ldg128<true>(row + 16 * v)};
    }
    __device__ static Raw bload(Buf b, int v0, int l, int U) {
        return Raw{bld32(b, 16 * U + 4 * v0, 4 * l), bld128(b, 16 * v0, 16 * l)};
    }
    // (d q + m) . x = d s1 E + (8 d + m) S
    __device__ static float dot(const Raw& r, int, const Limbs* L) {
        const float d = f16_hw(r.dm & 0xFFFFu), m = f16_hw(r.dm >> 16);
        return __builtin_fmaf(d * L[0].s1, (float)nib_dot(r.qs, L[0]),
                              __builtin_fmaf(8.0f, d, m) * L[0].S[0]);
    }
};

template <>
struct Pk<Q8_0> {
    static constexpr int NREC = 1, NG = 1;
    using Raw = Fmt<Q8_0>::Raw;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg16<true>(row + 32 * U + 2 * v), ldg128<true>(row + 16 * v),
                   ldg128<true>(row + 16 * U + 16 * v)};
    }

    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        return limb_dot<Q8_0>(r, v, L[0]);
    }
};

// Q4_K lane unit v = 4 s + g: the 32 qs bytes of sub-block pair g of super-
// block s (64 weights).  Record 2v holds the low nibbles (sub-block 2g), record
// 2v + 1 the high nibbles (sub-block 2g + 1), 32 slots each in element order.
struct Q4KP {
    uint4 hdr, q0, q1;  // d dmin scales[12]; qs[32g .. 32g+16); qs[32g+16 .. 32g+32)
};

template <>
struct Pk<Q4_K> {  // planes q0, q1 (U x 16 each), then the headers (S x 16)
    static constexpr int NREC = 2, NG = 1;
    using Raw = Q4KP;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg128<true>(row + 32 * U + 16 * (v >> 2)), ldg128<true>(row + 16 * v),
                   ldg128<true>(row + 16 * U + 16 * v)};
    }
    // v0 is a multiple of 64, so (v0 + l) >> 2 = v0 / 4 + l / 4
    __device__ static Raw bload(Buf b, int v0, int l, int U) {
        return Raw{bld128(b, 32 * U + 4 * v0, 16 * (l >> 2)), bld128(b, 16 * v0, 16 * l),
                   bld128(b, 16 * U + 16 * v0, 16 * l)};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        int D[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int lo = (int)(w[i] & 0x0F0F0F0Fu), hi = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
            D[0][0] = sdot4(lo, L[0].l1[i], D[0][0]);
            D[1][0] = sdot4(lo, L[0].l2[i], D[1][0]);
            D[2][0] = sdot4(lo, L[0].l3[i], D[2][0]);
            D[0][1] = sdot4(hi, L[1].l1[i], D[0][1]);
            D[1][1] = sdot4(hi, L[1].l2[i], D[1][1]);
            D[2][1] = sdot4(hi, L[1].l3[i], D[2][1]);
        }
        const float d = f16_hw(r.hdr.x & 0xFFFFu), dmin = f16_hw(r.hdr.x >> 16);
        uint32_t sa, ma, sb, mb;
        Fmt<Q4_K>::scale_min(r.hdr, v & 3, sa, ma, sb, mb);
        const float d14 = d * 0x1p-14f;
        float acc = -(dmin * (float)ma) * L[0].S[0];
        acc = __builtin_fmaf(-(dmin * (float)mb), L[1].S[0], acc);
        acc = __builtin_fmaf(d14 * (float)sa * L[0].s1, limb_sum4(D[0][0], D[1][0], D[2][0]), acc);
        return __builtin_fmaf(d14 * (float)sb * L[1].s1, limb_sum4(D[0][1], D[1][1], D[2][1]),
                              acc);
    }
};

// Q6_K lane unit v = 4 s + p: 64 weights, quarter p = 2n + h of super-block
// s: columns l = 16h .. 16h+15 of 128-half n, all four 32-row groups g.  Its
// two activation records are groups {0,1} and {2,3}: slot 16 g' + e of record
// 2v + r holds element 256 s + 128 n + 32 (2r + g') + 16 h + e.
struct Q6P {
    uint4 lo, hi, qh;  // ql[64n+16h..], ql[64n+32+16h..], qh[32n+16h..]
    uint2 sc;          // sc[8n .. 8n+8)
    uint32_t d;
};

template <>
struct Pk<Q6_K> {
    static constexpr int NREC = 2, NG = 2;
    using Raw = Q6P;
    __device__ static int k_of(int w, int s) {
        const int v = w >> 1, r = w & 1, sb = v >> 2, p = v & 3, n = p >> 1, h = p & 1;
        const int g = 2 * r + (s >> 4), e = s & 15;
        return 256 * sb + 128 * n + 32 * g + 16 * h + e;
    }
    // U here = lane units per row = K / 64; super-blocks S = U / 4.
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        const int S = U >> 2, sb = v >> 2, n = (v & 3) >> 1;
        return Raw{ldg128<true>(row + 16 * v), ldg128<true>(row + 16 * U + 16 * v),
                   ldg128<true>(row + 32 * U + 16 * v),
                   ldg64<true>(row + 192 * S + 16 * sb + 8 * n),
                   ldg16<true>(row + 208 * S + 2 * sb)};
    }
    // v0 is a multiple of 64: super-block v0 / 4 + l / 4, half (l & 3) / 2
    __device__ static Raw bload(Buf b, int v0, int l, int U) {
        const int S = U >> 2;
        return Raw{bld128(b, 16 * v0, 16 * l), bld128(b, 16 * U + 16 * v0, 16 * l),
                   bld128(b, 32 * U + 16 * v0, 16 * l),
                   bld64(b, 192 * S + 4 * v0, 16 * (l >> 2) + 8 * ((l & 3) >> 1)),
                   bld16(b, 208 * S + v0 / 2, 2 * (l >> 2))};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        const uint32_t A[4] = {r.lo.x, r.lo.y, r.lo.z, r.lo.w};
        const uint32_t B[4] = {r.hi.x, r.hi.y, r.hi.z, r.hi.w};
        const uint32_t H[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        // Group g (quants q1 .. q4 of the dword) sums E_g = D1 2^14 + D2 2^7 + D3
        // over its 16 elements in one int32 chain: the limb-1 dots, a shift by
        // 7, the limb-2 dots on top, a shift, the limb-3 dots.  With q <= 63,
        // |a1| <= 127 and |a2|, |a3| <= 64: |E_g| <= 16 * 63 * (127 * 2^14 +
        // 64 * 2^7 + 64) < 2^31.
        int q[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[0][i] = (int)((A[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4));
            q[1][i] = (int)((B[i] & 0x0F0F0F0Fu) | ((H[i] & 0x0C0C0C0Cu) << 2));
            q[2][i] = (int)(((A[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u));
            q[3][i] = (int)(((B[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u));
        }
        float E[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const Limbs& Lg = L[g >> 1];
            const int o = 4 * (g & 1);
            int e = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) e = sdot4(q[g][i], Lg.l1[o + i], e);
            e <<= 7;
#pragma unroll
            for (int i = 0; i < 4; ++i) e = sdot4(q[g][i], Lg.l2[o + i], e);
            e <<= 7;
#pragma unroll
            for (int i = 0; i < 4; ++i) e = sdot4(q[g][i], Lg.l3[o + i], e);
            E[g] = (float)e;  // rounding: 2^-24 relative
        }
        const int h = v & 1;  // sub-scale index l/16 = h: sc[8n + h + 2g]
        float sc[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t = h + 2 * g;
            const uint32_t word = t < 4 ? r.sc.x : r.sc.y;
            sc[g] = (float)(int)(int8_t)((word >> (8 * (t & 3))) & 0xFFu);
        }
        float sS = sc[0] * L[0].S[0];
        sS = __builtin_fmaf(sc[1], L[0].S[1], sS);
        sS = __builtin_fmaf(sc[2], L[1].S[0], sS);
        sS = __builtin_fmaf(sc[3], L[1].S[1], sS);
        const float Ea = __builtin_fmaf(sc[1], E[1], sc[0] * E[0]);
        const float Eb = __builtin_fmaf(sc[3], E[3], sc[2] * E[2]);
        const float P = __builtin_fmaf(L[1].s1, Eb, L[0].s1 * Ea);
        return f16_hw(r.d) * __builtin_fmaf(0x1p-14f, P, -32.0f * sS);
    }
};

// ---- GGUF rows.  The same lane units, read from the reference's unmodified
// block bytes.  A wave fetches the 16-byte-aligned superset of one K-slice
// (64 lane units) of one row with coalesced dwordx4 loads (lane p loads piece
// p, so each load instruction covers 1 KiB of contiguous HBM), writes the
// pieces to its own LDS buffer and every lane then reads its unit at the
// block layout's offsets, which are only 2-byte aligned (LDS reads on gfx950
// need no alignment).  Fetching the aligned superset never crosses a page.
// BB: block bytes; UPB: lane units per block.
template <int F>
struct Gk;

template <>
struct Gk<Q4_0> {  // d @0, qs[16] @2
    static constexpr int BB = 18, UPB = 1;
    __device__ static Pk<Q4_0>::Raw read(const uint8_t* s, int u) {
        const uint8_t* b = s + 18 * u;
        return {ld_u16(b), lds16_a2(b + 2)};
    }
};

template <>
struct Gk<Q4_1> {  // d @0, m @2, qs[16] @4
    static constexpr int BB = 20, UPB = 1;
    __device__ static Pk<Q4_1>::Raw read(const uint8_t* s, int u) {
        const uint8_t* b = s + 20 * u;
        return {lds4_a2(b), lds16_a2(b + 4)};
    }
};

template <>
struct Gk<Q8_0> {  // d @0, qs[32] @2
    static constexpr int BB = 34, UPB = 1;
    __device__ static Pk<Q8_0>::Raw read(const uint8_t* s, int u) {
        const uint8_t* b = s + 34 * u;
        return {ld_u16(b), lds16_a2(b + 2), lds16_a2(b + 18)};
    }
};

template <>
struct Gk<Q4_K> {  // d dmin scales[12] @0, qs[128] @16; unit u = 4 s + g
    static constexpr int BB = 144, UPB = 4;
    __device__ static Q4KP read(const uint8_t* s, int u) {
        const uint8_t* b = s + 144 * (u >> 2);
        const int g = u & 3;
        return {ld_u128(b), ld_u128(b + 16 + 32 * g), ld_u128(b + 32 + 32 * g)};
    }
};

template <>
struct Gk<Q6_K> {  // ql[128] @0, qh[64] @128, sc[16] @192, d @208; unit u = 4 s + 2 n + h
    static constexpr int BB = 210, UPB = 4;
    __device__ static Q6P read(const uint8_t* s, int u) {
        const uint8_t* b = s + 210 * (u >> 2);
        const int n = (u >> 1) & 1, h = u & 1;
        return {lds16_a2(b + 64 * n + 16 * h), lds16_a2(b + 64 * n + 32 + 16 * h),
                lds16_a2(b + 128 + 32 * n + 16 * h), lds8_a2(b + 192 + 8 * n), ld_u16(b + 208)};
    }
};

// Bytes of one K-slice (64 NL lane units) of a GGUF row, and the dwordx4
// pieces per lane that cover the aligned superset of `units` lane units (at
// most 14 bytes of misalignment).
template <int F, int NL>
constexpr int slice_bytes() {
    return 64 * NL / Gk<F>::UPB * Gk<F>::BB;
}
template <int F>
constexpr int slice_pieces(int units) {
    return ((units / Gk<F>::UPB * Gk<F>::BB + 14 + 15) / 16 + 63) / 64;
}

// Lane units per lane and step: two for the 4-bit 32-weight formats on rows
// of 65 to 192 units (halves the per-step reduction and bookkeeping per
// weight; K = 3584 rows become one K-slice), one otherwise: longer rows keep
// one unit per lane and 1024-thread work-groups, twice the waves to hide the
// loads (Q4_0 3584 x 18944 13.6 -> 12.8 us aligned, 14.2 -> 13.4 GGUF;
// 4096 x 8192 GGUF 8.6 -> 7.5 us; against 60.7 instead of 47.4 us for the
// K = 3584 lm_head with one unit).
template <int F>
constexpr int lane_units(int units) {
    return (F == Q4_0 || F == Q4_1) && units > 64 && units <= 192 ? 2 : 1;
}

template <int GP>
struct Pieces {
    uint4 v[GP];
};

// Work distribution.  Work-group g owns the contiguous rows [lo, hi) =
// [N g / G, N (g+1) / G).  Its work is the sequence of (K-slice, row) steps
// in slice-major order, f = s * rows + r (a K-slice is 64 lane units).  Waves
// claim steps one at a time from an LDS counter, each claim made one step
// before the wave needs it, so a wave that the SIMD arbiter serves less often
// simply takes fewer steps and the work-group's waves finish within one step
// of each other.  A wave reloads its activation limbs only when its slice
// changes.  The row sum of step f goes to the LDS buffer part[f]; at the end
// the work-group adds the slices of each row in slice order (so the result
// does not depend on which wave took which step) and writes y coalesced.  The
// pipelined loop issues no global stores and no global atomics.
constexpr int YBUF = 4096;     // row x slice partial sums a work-group buffers in LDS

struct Claims {
    int* ctr;
    int total, rows;
    float inv_rows;
};

// Uniform claim of the next step (-1: none left).
__device__ __forceinline__ int claim(const Claims& cl, int lane) {
    int i = 0;
    if (lane == 0) i = atomicAdd(cl.ctr, 1);
    i = __builtin_amdgcn_readfirstlane(i);
    return i < cl.total ? i : -1;
}

// Row sources.  ONE: row v of a.w.  PAIR: two matrices of the same shape
// interleaved row by row (virtual row 2n is row n of a.w, 2n + 1 row n of
// a.w2).  CAT: a.w, a.w2, a.w3 stacked (a.n1 and a.n2 rows in the first two).
enum { ONE = 0, PAIR = 1, CAT = 2 };

template <int MODE>
__device__ __forceinline__ const uint8_t* row_ptr(const GemvArgs& a, int v) {
    if constexpr (MODE == PAIR) return ((v & 1) ? a.w2 : a.w) + (size_t)(v >> 1) * a.row_bytes;
    if constexpr (MODE == CAT) {
        const int n12 = a.n1 + a.n2;
        const uint8_t* base = v < a.n1 ? a.w : v < n12 ? a.w2 : a.w3;
        return base + (size_t)(v - (v < a.n1 ? 0 : v < n12 ? a.n1 : n12)) * a.row_bytes;
    }
    return a.w + (size_t)v * a.row_bytes;
}

// Per-step weight registers: the lane's packed unit (GP = 0), or GP pieces of
// the aligned superset of a GGUF K-slice.
template <int F, int GP>
struct RegSel {
    using T = Pieces<GP>;
};
template <int F>
struct RegSel<F, 0> {
    using T = typename Pk<F>::Raw;
};

// First byte of step t's K-slice in a GGUF row.
template <int F, int NL, int MODE>
__device__ __forceinline__ const uint8_t* gslice(const GemvArgs& a, int sl, int r, int lo) {
    return row_ptr<MODE>(a, min(lo + r, a.N - 1)) + (size_t)sl * slice_bytes<F, NL>();
}

template <int F, int NL, int MODE, int GP>
__device__ __forceinline__ void pload(typename RegSel<F, GP>::T (&f)[NL], const GemvArgs& a,
                                      int sl, int row, int lo, int lane) {
    if constexpr (GP == 0 && F != Q8_0) {
        // the row's base and size in a scalar descriptor, the slice in the
        // scalar offset: the lane's offsets do not change from step to step.
        // Lane units past the row's end read bytes of the row's other planes
        // (or zeros past its last byte) and are masked out of the sum.
        // (Q8_0 measured 4 % slower this way at 18944 x 3584 and keeps
        // per-lane pointers; Q4_K gate, Q6_K down, Q4_0 down and lm_head
        // gained 1.5-3.5 %.)
        const Buf rb = make_buf(row_ptr<MODE>(a, min(lo + row, a.N - 1)), a.row_bytes);
        const int v0 = sl * 64 * NL;
#pragma unroll
        for (int c = 0; c < NL; ++c) f[c] = Pk<F>::bload(rb, v0, lane + 64 * c, a.U);
    } else if constexpr (GP == 0) {
        const uint8_t* r = row_ptr<MODE>(a, min(lo + row, a.N - 1));
        const int v0 = sl * 64 * NL;
#pragma unroll
        for (int c = 0; c < NL; ++c)
            f[c] = Pk<F>::load(r, min(v0 + lane + 64 * c, a.U - 1), a.U);
    } else {
        // pointer arithmetic (not integer casts) keeps the global address
        // space, so these stay global_load (vmcnt only)
        const uint8_t* g0 = gslice<F, NL, MODE>(a, sl, row, lo);
        const int shift = (int)(reinterpret_cast<uintptr_t>(g0) & 15);
        const uint8_t* a0 = g0 - shift;
        const int units = min(64 * NL, a.U - 64 * NL * sl);
        const int n16 = (shift + units / Gk<F>::UPB * Gk<F>::BB + 15) >> 4;
        // the slice's n16 pieces in a scalar descriptor: pieces past them
        // read as zeros (no lane reads their bytes back from LDS)
        const Buf rb = make_buf(a0, 16 * n16);
#pragma unroll
        for (int i = 0; i < GP; ++i) f[0].v[i] = bld128(rb, 0, 16 * (lane + 64 * i));
    }
}

template <int F, int NL>
__device__ __forceinline__ void load_slice_limbs(Limbs (&L)[NL][Pk<F>::NREC], const uint8_t* lds,
                                                 int s, int U, int lane) {
#pragma unroll
    for (int c = 0; c < NL; ++c)
#pragma unroll
        for (int r = 0; r < Pk<F>::NREC; ++r)
            read_limbs(L[c][r], lds, min(s * 64 * NL + lane + 64 * c, U - 1) * Pk<F>::NREC + r);
}

// The slot's step (-1: none) as (slice, row).  f < rows * slices <= YBUF:
// (f + 0.5) / rows in fp32 lies at least 0.5 / rows from an integer and is
// off by at most 2^-22 (f / rows) <= 2^-10 / rows, so its floor is exact.
struct Step {
    int f, s, r;
};
__device__ __forceinline__ Step step_of(int f, int rows, float inv_rows) {
    const int s = f >= 0 ? (int)(((float)f + 0.5f) * inv_rows) : 0;
    return Step{f, s, f >= 0 ? f - s * rows : 0};
}

// One slot of the pipeline: the compute side of the step whose loads the
// slot holds, then the loads of the wave's next claimed step into the same
// registers (past the last step they load row lo again, so the number of
// loads in flight never varies).
// GGUF (GP > 0): the step's pieces go to the wave's LDS buffer wbuf first,
// the next loads are issued into the freed registers, then each lane reads
// its unit from the buffer.  A wave's LDS accesses execute in order, so no
// barrier separates the writes from the reads.
// A work-group's K range: its first K-slice sl0 (steps count slices from
// there), its lane units Ul and each token's records Rl in LDS (the whole row
// unless the host splits K over blockIdx.y).
struct KRange {
    int sl0, Ul, Rl;
};

// Limb reloads: RL 0 never (rows of one K-slice: loaded before the loop),
// 1 when the step's slice differs from the wave's last, 2 every step.
template <int F, int NL, int MODE, int GP, int NT, int RL>
__device__ __forceinline__ void pstep(typename RegSel<F, GP>::T (&f)[NL], Step& st, int& nxt,
                                      const Claims& cl, const GemvArgs& a, const KRange& kr,
                                      Limbs (&L)[NT][NL][Pk<F>::NREC], const uint8_t* lds,
                                      uint8_t* wbuf, float* part, int lo, int lane, int& cur_s) {
    __builtin_amdgcn_sched_barrier(0);
    const Step cp = st;
    st = step_of(nxt, cl.rows, cl.inv_rows);
    if (nxt >= 0) nxt = claim(cl, lane);  // wave-uniform
    if (RL == 2 || (RL == 1 && cp.f >= 0 && cp.s != cur_s)) {  // wave-uniform
#pragma unroll
        for (int t = 0; t < NT; ++t)
            load_slice_limbs<F, NL>(L[t], lds + (size_t)t * kr.Rl * RECB, cp.s, kr.Ul, lane);
        cur_s = cp.s;
    }
    const int v0 = (kr.sl0 + cp.s) * 64 * NL;  // the step's first lane unit in the row
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    if constexpr (GP == 0) {
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const int v = v0 + lane + 64 * c;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float d = Pk<F>::dot(f[c], min(v, a.U - 1), L[t][c]);
                acc[t] += v < a.U ? d : 0.0f;
            }
        }
        pload<F, NL, MODE, GP>(f, a, kr.sl0 + st.s, st.r, lo, lane);
    } else {
#pragma unroll
        for (int i = 0; i < GP; ++i) reinterpret_cast<uint4*>(wbuf)[lane + 64 * i] = f[0].v[i];
        const int shift = (int)(reinterpret_cast<uintptr_t>(
                                    gslice<F, NL, MODE>(a, kr.sl0 + cp.s, cp.r, lo)) & 15);
        typename Pk<F>::Raw raw[NL];
#pragma unroll
        for (int c = 0; c < NL; ++c)
            raw[c] = Gk<F>::read(wbuf + shift, min(v0 + lane + 64 * c, a.U - 1) - v0);
        pload<F, NL, MODE, GP>(f, a, kr.sl0 + st.s, st.r, lo, lane);
#pragma unroll
        for (int c = 0; c < NL; ++c) {
            const int v = v0 + lane + 64 * c;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float d = Pk<F>::dot(raw[c], min(v, a.U - 1), L[t][c]);
                acc[t] += v < a.U ? d : 0.0f;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float sum = wave_sum(acc[t]);
        if (cp.f >= 0 && lane == 63) part[t * cl.total + cp.f] = sum;
    }
    __builtin_amdgcn_sched_barrier(0);
}

// MODE PAIR: y[n] = silu(x . w[n]) * (x . w2[n]) over a.N = 2 N virtual
// rows (the fused FFN gate and up projections); work-group row ranges are
// even.  MODE CAT: y is the concatenation of the three GEMVs (fused QKV).
// GP > 0: GGUF rows, GP pieces per lane per K-slice; the dynamic LDS holds
// the limb records, then one GP KiB buffer per wave, then the partial sums
// (sized by the host).  NT tokens (MODE ONE, GGUF rows): every weight unit
// read and decoded once is dotted with each token's limbs; token t's records
// follow token t - 1's, and y, the partial sums and a full bias
// (a.bias_mode 2) are token-major.  Where the tokens' records of a whole row
// do not fit LDS the host splits K: work-group (g, y) stages the records of
// K-slices y a.spl .. (y + 1) a.spl - 1 only and writes its row sums, without
// the bias, to slab y of a.part for the slab sum.
template <int F, int NL, int D, bool BIAS, int WG, int MODE = ONE, int GP = 0, int NT = 1,
          bool OS = false>
__global__ __launch_bounds__(WG) void gemvp_kernel(GemvArgs a) {
    static_assert(NT == 1 || (MODE == ONE && GP > 0), "several tokens: GGUF rows, MODE ONE");
    constexpr bool DUAL = MODE == PAIR;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int ctr;
    constexpr int W = WG / 64;
    float* part;
    uint8_t* wbuf = nullptr;
    if constexpr (GP == 0) {
        __shared__ float part_s[YBUF];
        part = part_s;
    }
    using P = Pk<F>;
    // K split over blockIdx.y (several tokens only; a.spl slices per split,
    // 0: unsplit): this work-group's slices, lane units and records per token
    const bool split = NT > 1 && a.spl > 0;
    const int ns_all = (a.U + 64 * NL - 1) / (64 * NL);
    KRange kr{0, a.U, a.Uc};
    if (split) {
        kr.sl0 = (int)blockIdx.y * a.spl;
        kr.Ul = min(a.U - kr.sl0 * 64 * NL, a.spl * 64 * NL);
        kr.Rl = kr.Ul * P::NREC;
    }
    if constexpr (GP > 0) {
        wbuf = lds + (size_t)NT * kr.Rl * RECB + (threadIdx.x >> 6) * (GP * 1024);
        part = reinterpret_cast<float*>(lds + (size_t)NT * kr.Rl * RECB + W * GP * 1024);
    }
    const int lane = threadIdx.x & 63;
    const int ns = split ? min(ns_all - kr.sl0, a.spl) : ns_all;
    const int G = gridDim.x, g = blockIdx.x;
    // the host sizes the grid so (hi - lo) * ns <= YBUF
    const int lo = DUAL ? 2 * (int)((int64_t)(a.N / 2) * g / G) : (int)((int64_t)a.N * g / G);
    const int hi = DUAL ? 2 * (int)((int64_t)(a.N / 2) * (g + 1) / G)
                        : (int)((int64_t)a.N * (g + 1) / G);
    const int rows = hi - lo;
    const Claims cl{&ctr, rows * ns, rows, 1.0f / (float)max(rows, 1)};

    // Wave w's first D steps are w, W + w, ..., and its first claim is
    // D W + w; the counter hands out the rest from (D + 1) W.  The activation
    // loads go first, so they never queue behind the weight stream; the first
    // step's weight loads go out between them and the limb build, so HBM is
    // busy during the staging without delaying the activations (the remaining
    // first loads follow the barrier: issued all at once they would queue
    // ahead of other work-groups' activation loads).
    if (threadIdx.x == 0) ctr = (D + 1) * W;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    Step st[D];
#pragma unroll
    for (int j = 0; j < D; ++j) st[j] = step_of(j * W + w < cl.total ? j * W + w : -1, rows, cl.inv_rows);
    int nxt = D * W + w < cl.total ? D * W + w : -1;
    typename RegSel<F, GP>::T f[D][NL];
    {
        XStage<P, WG> xs;
        const int r0 = kr.sl0 * 64 * NL * P::NREC;  // the range's first record
        stage_load<P, WG>(xs, a.x, NT * kr.Rl, r0, NT > 1 ? kr.Rl : 0, a.K);
        pload<F, NL, MODE, GP>(f[0], a, kr.sl0 + st[0].s, st[0].r, lo, lane);
        stage_build<P, WG, false>(lds, xs, a.x, NT * kr.Rl, r0, NT > 1 ? kr.Rl : 0, a.K);
    }
    lds_barrier();  // the weight loads stay in flight
#pragma unroll
    for (int j = 1; j < D; ++j)
        pload<F, NL, MODE, GP>(f[j], a, kr.sl0 + st[j].s, st[j].r, lo, lane);
    Limbs L[NT][NL][P::NREC];
    int cur_s = -1;
    // every iteration runs all D slots, each issuing its loads, so the number
    // of loads in flight at the loop head is always the same and the compiler
    // waits for exactly one slot's loads (a skipped load would make it drain
    // the whole queue); steps are claimed in order, so once slot 0 holds no
    // step neither does any later slot.  The wave reloads its limbs when the
    // slice changes.  For the nibble records (4-bit formats) that conditional
    // reload leaves the compiler copying all the limb registers at the loop's
    // back edge (about 50 VALU instructions per iteration), so their kernels
    // come in two forms: rows of one K-slice (OS) load the limbs once, longer
    // rows reload them at every step (the LDS reads cost less).
    constexpr int RL = !NibRec<P>::value ? 1 : OS ? 0 : 2;
    if constexpr (RL == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
            load_slice_limbs<F, NL>(L[t], lds + (size_t)t * kr.Rl * RECB, 0, kr.Ul, lane);
    }
    while (st[0].f >= 0) {
#pragma unroll
        for (int j = 0; j < D; ++j)
            pstep<F, NL, MODE, GP, NT, RL>(f[j], st[j], nxt, cl, a, kr, L, lds, wbuf, part, lo,
                                           lane, cur_s);
    }
    __syncthreads();
    if constexpr (DUAL) {
        for (int r = threadIdx.x; 2 * r < rows; r += WG) {
            float gt = part[2 * r], up = part[2 * r + 1];
            for (int s = 1; s < ns; ++s) {
                gt += part[s * rows + 2 * r];
                up += part[s * rows + 2 * r + 1];
            }
            a.y[(lo >> 1) + r] = gt / (1.0f + expf(-gt)) * up;  // silu(gate) * up
        }
    } else {
        // the bias is added to the finished row sum, as apply_bias adds it to
        // the finished product (matmul.cpp:1005-1049); a K split writes its
        // slab of partial sums (split-major, then token-major) and the slab
        // sum adds the bias
        float* out = split ? a.part + (size_t)blockIdx.y * NT * a.N : a.y;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float* bias = a.bias + (a.bias_mode == 2 ? (size_t)t * a.N : 0);
            for (int r = threadIdx.x; r < rows; r += WG) {
                float v = part[t * cl.total + r];
                for (int s = 1; s < ns; ++s) v += part[t * cl.total + s * rows + r];
                if constexpr (BIAS) v += lo + r < a.bias_len ? bias[lo + r] : 0.0f;
                out[(size_t)t * a.N + lo + r] = v;
            }
        }
    }
}

constexpr int WGP = 1024;
// Steps of weight loads a wave keeps in flight.  One, with 16 waves per CU,
// measured fastest at every packed shape (cfg2 gate 10.3 us against 10.7 with
// two and 12.3 with three).  GGUF rows of matrices of 64k rows and more
// (lm_head) keep more: 81.4 us against 86.3 with one for Q6_K.  At
// 152064 x 3584 (us, two / three / four steps): Q6_K 75.3 / 76.2 / 82.3,
// Q8_0 91.3 / 92.8 / 94.3, Q4_0 67.1 / 65.4 / 65.3.
constexpr int DP = 1;
template <int F>
constexpr int deep_depth() {
    return F == Q4_0 || F == Q4_1 ? 3 : 2;
}
constexpr int DPG_DEEP = 3;  // the deepest of deep_depth<F>() (launch geometry)
constexpr int DEEP_ROWS = 65536;

// Two lane units per lane hold both units' activation limbs in registers:
// more than the 128 VGPRs of a 1024-thread work-group, so they run 512.  With
// half the waves per CU they keep two steps of loads in flight (132-135
// VGPRs): Q4_0 3584 x 18944 14.7 -> 14.1 us aligned, 16.3 -> 15.3 GGUF;
// three steps measured slower (15.5 / 16.8).
template <int NL>
constexpr int depth() {
    return NL == 2 ? 2 : DP;
}
template <int NL, int WG>
constexpr int nl_wg() {
    return NL == 2 ? 512 : WG;
}

// The kernel's address; os: rows of one K-slice (its own form for the 4-bit
// formats, whose limbs are then loaded once).
template <int F, int NL, int D, bool BIAS, int WG, int MODE = ONE, int GP = 0, int NT = 1>
const void* kfn(bool os) {
    if constexpr (F == Q4_0 || F == Q4_1)
        if (os)
            return reinterpret_cast<const void*>(&gemvp_kernel<F, NL, D, BIAS, WG, MODE, GP, NT, true>);
    return reinterpret_cast<const void*>(&gemvp_kernel<F, NL, D, BIAS, WG, MODE, GP, NT>);
}

template <int F, int NL>
const void* pfn2(bool bias, bool os) {
    constexpr int WG = nl_wg<NL, WGP>();
    return bias ? kfn<F, NL, depth<NL>(), true, WG>(os) : kfn<F, NL, depth<NL>(), false, WG>(os);
}

template <int F>
const void* pfn(int units, bool bias, int* nl) {
    *nl = lane_units<F>(units);
    const bool os = units <= 64 * *nl;
    if constexpr (F == Q4_0 || F == Q4_1)
        if (*nl == 2) return pfn2<F, 2>(bias, os);
    return pfn2<F, 1>(bias, os);
}

template <int F>
const void* pfn_mode(int mode, int units) {
    const bool os = units <= 64;
    return mode == PAIR ? kfn<F, 1, DP, false, WGP, PAIR>(os) : kfn<F, 1, DP, false, WGP, CAT>(os);
}

// GGUF rows: GP pieces per lane cover a K-slice; only the counts a format's
// slices can need are instantiated.
template <int F>
constexpr int max_pieces() {
    return slice_pieces<F>(64);
}

// Four pieces per lane with three steps in flight need more than the 128
// VGPRs of a 1024-thread work-group: 512 threads.  With one step in flight
// they fit (92 VGPRs): cfg2 down on GGUF bytes 16.6-19.3 us against
// 18.9-21.1 at 512 threads.
template <int GP, int D>
constexpr int gwg() {
    return GP >= 4 && D > 1 ? 512 : WGP;
}

template <int F, int NL, int GP, int D>
const void* gfn3(bool bias, bool os) {
    constexpr int WG = nl_wg<NL, gwg<GP, D>()>();
    return bias ? kfn<F, NL, D, true, WG, ONE, GP>(os) : kfn<F, NL, D, false, WG, ONE, GP>(os);
}

template <int F, int NL, int GP>
const void* gfn2(bool bias, bool deep, bool os) {
    if constexpr (GP > max_pieces<F>() * NL) {
        return nullptr;
    } else {
        return deep ? gfn3<F, NL, GP, deep_depth<F>()>(bias, os)
                    : gfn3<F, NL, GP, depth<NL>()>(bias, os);
    }
}

template <int F>
const void* gfn(int units, bool bias, bool deep, int* gp, int* nl) {
    *nl = lane_units<F>(units);
    const bool os = units <= 64 * *nl;
    *gp = slice_pieces<F>(units < 64 * *nl ? units : 64 * *nl);
    if constexpr (F == Q4_0 || F == Q4_1) {
        if (*nl == 2) switch (*gp) {
            case 2: return gfn2<F, 2, 2>(bias, deep, os);
            case 3: return gfn2<F, 2, 3>(bias, deep, os);
            default: return nullptr;
        }
    }
    switch (*gp) {
        case 1: return gfn2<F, 1, 1>(bias, deep, os);
        case 2: return gfn2<F, 1, 2>(bias, deep, os);
        case 3: return gfn2<F, 1, 3>(bias, deep, os);
        case 4: return gfn2<F, 1, 4>(bias, deep, os);
        default: return nullptr;
    }
}

// Two to four tokens: every token's limbs stay in registers, more than the
// 128 VGPRs of a 1024-thread work-group.  Two tokens with one lane unit per
// lane fit 168 (768 threads: cfg3 M = 2 12.5-13.5 us against 13.3 at 512,
// GGUF lm_head 101 against 107); two lane units, or three and four tokens,
// need up to 256, so 512 threads (three and four tokens: one lane unit).
// Three tokens against the other kernels: cfg3 Q4_K 16.3 against 20.7 us,
// Q6_K lm_head 128 against 227, Q8_0 14336 x 4096 19.3 against 22.7; four
// tokens (Q4_0, Q4_1, Q8_0): Q8_0 22.7 against 26.4.  Q4_0 and Q4_1 with one
// lane unit per lane (nibble records: fewer live registers) and Q8_0 with
// three tokens fit 1024 threads: 3584 x 18944 Q4_0 M = 2 / 3 / 4 20.2 /
// 29.4 / 37.4 -> 19.1 / 26.2 / 30.8 us, 14336 x 4096 Q8_0 M = 3 19.0 ->
// 16.8 (Q8_0 M = 4 22.3 -> 34.2, Q4_K and Q6_K three to six times slower:
// they spill).
constexpr int wg_tok(int f, int nl, int nt) {
    return nl == 2                           ? 512
           : f == Q4_0 || f == Q4_1          ? 1024
           : f == Q8_0 && nt == 3            ? 1024
           : nt > 2                          ? 512
                                             : 768;
}
template <int F, int NL, int NT>
constexpr int wg_t() {
    return wg_tok(F, NL, NT);
}

template <int F, int NL, int GP, int NT>
const void* gfn_t(bool bias, bool os) {
    if constexpr (GP > max_pieces<F>() * NL) {
        return nullptr;
    } else {
        constexpr int WG = wg_t<F, NL, NT>();
        return bias ? kfn<F, NL, DP, true, WG, ONE, GP, NT>(os)
                    : kfn<F, NL, DP, false, WG, ONE, GP, NT>(os);
    }
}

// one lane unit per lane
template <int F, int NT>
const void* gfnt_one(int units, bool bias, int* gp) {
    const bool os = units <= 64;
    *gp = slice_pieces<F>(units < 64 ? units : 64);
    switch (*gp) {
        case 1: return gfn_t<F, 1, 1, NT>(bias, os);
        case 2: return gfn_t<F, 1, 2, NT>(bias, os);
        case 3: return gfn_t<F, 1, 3, NT>(bias, os);
        case 4: return gfn_t<F, 1, 4, NT>(bias, os);
        default: return nullptr;
    }
}

template <int F, int NT>
const void* gfnt(int units, bool bias, int* gp, int* nl) {
    *nl = lane_units<F>(units);
    const bool os = units <= 64 * *nl;
    *gp = slice_pieces<F>(units < 64 * *nl ? units : 64 * *nl);
    if constexpr (F == Q4_0 || F == Q4_1) {
        if (*nl == 2) {
            if constexpr (NT == 2) {
                switch (*gp) {
                    case 2: return gfn_t<F, 2, 2, NT>(bias, os);
                    case 3: return gfn_t<F, 2, 3, NT>(bias, os);
                }
                return nullptr;
            } else if constexpr (NT == 3) {
                // three tokens: one lane unit per lane (four: the other
                // kernels, 4096 x 4096 9.7 against 10.7 us this way)
                *nl = 1;
                return gfnt_one<F, NT>(units, bias, gp);
            } else {
                return nullptr;
            }
        }
    }
    return gfnt_one<F, NT>(units, bias, gp);
}

template <int F>
const void* gfn_tokens(int tokens, int units, bool bias, int* gp, int* nl) {
    switch (tokens) {
        case 2: return gfnt<F, 2>(units, bias, gp, nl);
        case 3: return gfnt<F, 3>(units, bias, gp, nl);
        case 4:
            // Q4_K and Q6_K units hold two records per token: four tokens'
            // limbs spill (Q6_K lm_head at M = 4 271 us against 257 on the
            // other kernels, cfg3 Q4_K 21.1 against 20.7)
            if constexpr (F == Q4_K || F == Q6_K) return nullptr;
            else return gfnt<F, 4>(units, bias, gp, nl);
    }
    return nullptr;
}

// The fused forms (MODE PAIR: gate/up; CAT: QKV) over GGUF rows: one lane
// unit per lane, one step of loads in flight.
template <int F, int MODE, int GP>
const void* gfn_mode3(bool os) {
    if constexpr (GP > max_pieces<F>()) {
        return nullptr;
    } else {
        return kfn<F, 1, DP, false, gwg<GP, DP>(), MODE, GP>(os);
    }
}

template <int F>
const void* gfn_mode(int mode, int units, int* gp) {
    *gp = slice_pieces<F>(units < 64 ? units : 64);
    const bool os = units <= 64;
    const bool pair = mode == PAIR;
    switch (*gp) {
        case 1: return pair ? gfn_mode3<F, PAIR, 1>(os) : gfn_mode3<F, CAT, 1>(os);
        case 2: return pair ? gfn_mode3<F, PAIR, 2>(os) : gfn_mode3<F, CAT, 2>(os);
        case 3: return pair ? gfn_mode3<F, PAIR, 3>(os) : gfn_mode3<F, CAT, 3>(os);
        case 4: return pair ? gfn_mode3<F, PAIR, 4>(os) : gfn_mode3<F, CAT, 4>(os);
    }
    return nullptr;
}

}  // namespace

// Lane units per row and activation records for a packed GEMV of length K.
int gemvp_record_bytes() { return RECB; }

void gemvp_geometry(int dtype, int K, int* units, int* records) {
    if (dtype == Q6_K || dtype == Q4_K) {
        *units = K / 64;
        *records = K / 32;
    } else {
        *units = K / 32;
        *records = K / 32;
    }
}

// Kernel for a row of `units` lane units: K-slices of 64 nl units (nl per
// lane).  mode 1: the fused gate/up form, 2: the fused QKV form (bias unused
// in both).
const void* gemvp_kernel_fn(int dtype, int units, int records, bool bias, size_t* lds, int* wg,
                            int* nl, int mode) {
    const void* fn = nullptr;
    *nl = 1;
    switch (dtype) {
        case Q4_0: fn = mode ? pfn_mode<Q4_0>(mode, units) : pfn<Q4_0>(units, bias, nl); break;
        case Q4_1: fn = mode ? pfn_mode<Q4_1>(mode, units) : pfn<Q4_1>(units, bias, nl); break;
        case Q8_0: fn = mode ? pfn_mode<Q8_0>(mode, units) : pfn<Q8_0>(units, bias, nl); break;
        case Q4_K: fn = mode ? pfn_mode<Q4_K>(mode, units) : pfn<Q4_K>(units, bias, nl); break;
        case Q6_K: fn = mode ? pfn_mode<Q6_K>(mode, units) : pfn<Q6_K>(units, bias, nl); break;
    }
    if (mode) *nl = 1;
    *lds = (size_t)records * RECB;
    *wg = *nl == 2 ? nl_wg<2, WGP>() : WGP;
    return fn;
}

// The same kernel over GGUF rows (K-slices staged through a per-wave LDS
// buffer).  *lds_fixed: the records and the wave buffers; the host adds the
// partial-sum buffer after them.
const void* gemvg_kernel_fn(int dtype, int units, int records, bool bias, size_t* lds_fixed,
                            int* wg, int* nl, int rows, int tokens, int mode) {
    int gp = 0;
    const bool deep = rows >= DEEP_ROWS;
    const void* fn = nullptr;
    *nl = 1;
    if (mode) {
        if (tokens != 1 || bias) return nullptr;
        switch (dtype) {
            case Q4_0: fn = gfn_mode<Q4_0>(mode, units, &gp); break;
            case Q4_1: fn = gfn_mode<Q4_1>(mode, units, &gp); break;
            case Q8_0: fn = gfn_mode<Q8_0>(mode, units, &gp); break;
            case Q4_K: fn = gfn_mode<Q4_K>(mode, units, &gp); break;
            case Q6_K: fn = gfn_mode<Q6_K>(mode, units, &gp); break;
        }
        *wg = gp >= 4 ? gwg<4, DP>() : WGP;
        *lds_fixed = (size_t)records * RECB + (size_t)(*wg / 64) * gp * 1024;
        return fn;
    }
    if (tokens >= 2) {
        switch (dtype) {
            case Q4_0: fn = gfn_tokens<Q4_0>(tokens, units, bias, &gp, nl); break;
            case Q4_1: fn = gfn_tokens<Q4_1>(tokens, units, bias, &gp, nl); break;
            case Q8_0: fn = gfn_tokens<Q8_0>(tokens, units, bias, &gp, nl); break;
            case Q4_K: fn = gfn_tokens<Q4_K>(tokens, units, bias, &gp, nl); break;
            case Q6_K: fn = gfn_tokens<Q6_K>(tokens, units, bias, &gp, nl); break;
        }
        *wg = wg_tok(dtype, *nl, tokens);
        *lds_fixed = (size_t)tokens * records * RECB + (size_t)(*wg / 64) * gp * 1024;
        return fn;
    }
    if (tokens != 1) return nullptr;
    switch (dtype) {
        case Q4_0: fn = gfn<Q4_0>(units, bias, deep, &gp, nl); break;
        case Q4_1: fn = gfn<Q4_1>(units, bias, deep, &gp, nl); break;
        case Q8_0: fn = gfn<Q8_0>(units, bias, deep, &gp, nl); break;
        case Q4_K: fn = gfn<Q4_K>(units, bias, deep, &gp, nl); break;
        case Q6_K: fn = gfn<Q6_K>(units, bias, deep, &gp, nl); break;
    }
    *wg = *nl == 2 ? nl_wg<2, WGP>() : gp >= 4 && deep ? gwg<4, DPG_DEEP>() : WGP;
    *lds_fixed = (size_t)records * RECB + (size_t)(*wg / 64) * gp * 1024;
    return fn;
}

}  // namespace fq
