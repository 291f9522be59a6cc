// fq_mmq.hip -- quantized matmul for M > 1 on the matrix cores (MFMA).
//
// y[m][n] = sum_k x[m][k] w[n][k], w[n][k] = A_{n,s} q_{n,k} + B_{n,s} for the
// sub-block s holding k (32 elements; 16 for Q6_K, whose scales cover 16).
// The quants q are small integers, exact in fp16.  Each activation row is
// scaled by a power of two 2^-e_m into [2^14, 2^15) and split into two fp16
// halves, x' = x_hi + x_lo (x_lo = fp16(x' - x_hi)), which carry 22 of fp32's
// 24 significand bits.  Per sub-block and 16x16 tile, two MFMAs
//     R = q . x_hi + q . x_lo          (exact products, fp32 accumulation)
// give sum_k q x' for 16 rows x 16 tokens, and the fp32 epilogue adds
//     acc += A_{n,s} R  (+ B_{n,s} S_{m,s},  S = sum of x' over the sub-block)
// so the block scales never touch fp16.  y = 2^e_m acc at the end.
//
// Two kernels:
//  xprep_kernel  one work-group per (16 tokens, chunk of KC = 64 elements):
//                per-(token, chunk) exponents, x_hi/x_lo in MFMA operand
//                order, the sub-block sums S.
//  mmq_kernel    one work-group per (BN rows x BM tokens x K-split) tile:
//                per chunk it stages the token operands (a straight copy) and
//                the weight tile (decoded to fp16 quants plus A, B per
//                sub-block) in LDS, then every wave runs its WN x WM 16x16
//                tiles.  With several K-splits each split writes a partial
//                [M][N] slab and reduce_kernel sums them in split order, so
//                results do not depend on timing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_mfma16.h"

namespace fq {
namespace {

constexpr int KC = 64;        // K elements per chunk
constexpr int XOP = 2048;     // halves per (token tile, chunk): hi and lo operands
constexpr int XSUM = 64;      // group-sum floats per (token tile, chunk)

// Operand geometry of a sub-block of SB elements (SB = 32: MFMA 16x16x32,
// SB = 16: MFMA 16x16x16).  Lane l = 16 g + c supplies EPL = SB / 4
// consecutive elements [EPL g, EPL g + EPL) of row/token c.  Per chunk there
// are NS = KC / SB sub-blocks; operand block of one sub-block = 16 * SB halves.
template <int SB>
struct Geo {
    static constexpr int NS = KC / SB, EPL = SB / 4, BLK = 16 * SB;
};

template <int F>
struct SubBlock {
    static constexpr int SB = F == Q6_K || F == Q3_K ? 16 : 32;
    static constexpr bool HAS_B = F == Q4_1 || F == Q4_K || F == Q5_1 || F == Q5_K;
};

// ------------------------------------------------------------------ xprep
// Token m of tile t = m / 16 is column c = m % 16.  Chunk ch has its own
// exponent e = ex[(t NC + ch) 16 + c], chosen so the chunk's max |x| 2^-e
// lies in [2^14, 2^15).  Element kl of the chunk, sub-block s = kl / SB,
// group g = (kl % SB) / EPL, is slot e' (slot_elem(e') = kl % EPL) of
//   xop[(t NC + ch) XOP + s 2 BLK + hl BLK + (16 g + c) EPL + e']
// and xsum[(t NC + ch) XSUM + s 16 + c] is the sum of x 2^-e over sub-block s.
// Work-group (t, ch): 16 tokens x 64 elements; thread (c, p) handles the
// aligned quad [4 p, 4 p + 4) of token c (slot_elem permutes within quads).
template <int SB>
__global__ __launch_bounds__(256) void xprep_kernel(const float* __restrict__ x, int M, int K,
                                                    int NC, _Float16* __restrict__ xop,
                                                    float* __restrict__ xsum, int* __restrict__ ex) {
    using G = Geo<SB>;
    constexpr int EPL = G::EPL;
    const int c = threadIdx.x >> 4, p = threadIdx.x & 15;
    const int t = blockIdx.x, ch = blockIdx.y, m = 16 * t + c;
    const int k0 = ch * KC + 4 * p;
    const bool live = m < M && k0 < K;  // K is a multiple of 32: quads are all in or all out
    const float* xr = x + (size_t)min(m, M - 1) * K + (live ? k0 : 0);
    float v[4];
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = live ? xr[i] : 0.0f;
        mx = fmaxf(mx, fabsf(v[i]));
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) e = ilogbf(mx) - 14;
    const size_t blk = (size_t)t * NC + ch;
    if (p == 0) ex[blk * 16 + c] = e;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = ldexpf(v[i], -e);
    const int kl = 4 * p, s = kl / SB, g = (kl % SB) / EPL;
    _Float16* dst = xop + blk * XOP + s * 2 * G::BLK + (16 * g + c) * EPL + (kl % EPL);
    h4 hi, lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float w = v[slot_elem(i)];
        hi[i] = (_Float16)w;
        lo[i] = (_Float16)(w - (float)hi[i]);
    }
    *reinterpret_cast<h4*>(dst) = hi;
    *reinterpret_cast<h4*>(dst + G::BLK) = lo;
    // sub-block sums: a fixed tree over the SB / 4 threads of the sub-block
    float sum = (v[0] + v[1]) + (v[2] + v[3]);
#pragma unroll
    for (int o = 1; o < SB / 4; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if ((p % (SB / 4)) == 0) xsum[blk * XSUM + s * 16 + c] = sum;
}

// ------------------------------------------------------------ weight decode
// A task is one sub-block of one row.  Task<F>::load issues its global loads
// (into registers, so the next chunk's loads are in flight while the current
// chunk runs on the matrix cores); Task<F>::put decodes them into the operand
// layout (dst + (16 g + c) * EPL) and the sub-block's A, B.
//
// Quants become fp16 with the byte-pair helpers of fq_mfma16.h, in slot
// order; the token operands use the same order (xprep_kernel).

__device__ __forceinline__ fq_u32x4 ldv(const uint8_t* p) {
    const uint4 v = ld_u128(p);
    return fq_u32x4{v.x, v.y, v.z, v.w};
}

template <int F>
struct Task;

template <>
struct Task<Q4_0> {  // block 2ch + s: d | qs[16]; elements j (low), j + 16 (high)
    uint32_t d;
    fq_u32x4 q;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* b = row + 18 * (2 * ch + s);
        d = ld_u16(b);
        q = ldv(b + 2);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(d);
        B = 0.0f;
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int g = 0; g < 4; ++g)  // elements 8g .. 8g+7
            *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) =
                nib8(w[2 * (g & 1)], w[2 * (g & 1) + 1], g < 2 ? 0 : 4, (_Float16)1032.0f);
    }
};

template <>
struct Task<Q4_1> {  // block 2ch + s: d m | qs[16]
    uint32_t dm;
    fq_u32x4 q;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* b = row + 20 * (2 * ch + s);
        dm = ld_u32(b);
        q = ldv(b + 4);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(dm & 0xFFFFu);
        B = f16_hw(dm >> 16);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) =
                nib8(w[2 * (g & 1)], w[2 * (g & 1) + 1], g < 2 ? 0 : 4, (_Float16)1024.0f);
    }
};

template <>
struct Task<Q8_0> {  // block 2ch + s: d | qs int8[32]
    uint32_t d;
    fq_u32x4 q0, q1;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* b = row + 34 * (2 * ch + s);
        d = ld_u16(b);
        q0 = ldv(b + 2);
        q1 = ldv(b + 18);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(d);
        B = 0.0f;
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int g = 0; g < 4; ++g)  // signed bytes: +128 by flipping the sign bit
            *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) =
                byte8(w[2 * g] ^ 0x80808080u, w[2 * g + 1] ^ 0x80808080u, (_Float16)1152.0f);
    }
};

template <>
struct Task<Q4_K> {  // chunk ch = pair j of super-block ch / 4; s = 0 low, 1 high nibbles
    fq_u32x4 hdr, q0, q1;
    int j, s;
    __device__ void load(const uint8_t* row, int ch, int s_) {
        const uint8_t* sb = row + 144 * (ch >> 2);
        j = ch & 3;
        s = s_;
        hdr = ldv(sb);
        q0 = ldv(sb + 16 + 32 * j);
        q1 = ldv(sb + 32 + 32 * j);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        uint32_t sa, ma, sb2, mb;
        Fmt<Q4_K>::scale_min(uint4{hdr.x, hdr.y, hdr.z, hdr.w}, j, sa, ma, sb2, mb);
        const float d = f16_hw(hdr.x & 0xFFFFu), dmin = f16_hw(hdr.x >> 16);
        A = d * (float)(s ? sb2 : sa);
        B = -(dmin * (float)(s ? mb : ma));
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) =
                nib8(w[2 * g], w[2 * g + 1], 4 * s, (_Float16)1024.0f);
    }
};

template <>
struct Task<Q6_K> {
    // chunk ch: super-block ch / 4, quarter qq = ch % 4 -> half n = qq / 2,
    // groups g' = 2 (qq % 2) + {0, 1} (elements 128 n + 32 g' + l).  Sub-block
    // s (16 elements): g' = 2 (qq % 2) + s / 2, l in [16 (s % 2), +16), scale
    // sc[8 n + s % 2 + 2 g'] (matmul.cpp:259-276).
    fq_u32x4 ql, qh;
    uint32_t d, sc;
    int gp;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* sb = row + 210 * (ch >> 2);
        const int qq = ch & 3, n = qq >> 1, l0 = 16 * (s & 1);
        gp = 2 * (qq & 1) + (s >> 1);
        d = ld_u16(sb + 208);
        sc = sb[192 + 8 * n + (s & 1) + 2 * gp];
        ql = ldv(sb + 64 * n + 32 * (gp & 1) + l0);
        qh = ldv(sb + 128 + 32 * n + l0);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(d) * (float)(int)(int8_t)sc;
        B = 0.0f;
        const uint32_t L[4] = {ql.x, ql.y, ql.z, ql.w};
        const uint32_t H[4] = {qh.x, qh.y, qh.z, qh.w};
        const int lsh = gp < 2 ? 0 : 4, hsh = 2 * gp;
#pragma unroll
        for (int g = 0; g < 4; ++g) {  // elements l0 + 4g .. +4: 6-bit codes, then -32
            const uint32_t q6 = ((L[g] >> lsh) & 0x0F0F0F0Fu) | (((H[g] >> hsh) & 0x03030303u) << 4);
            h2 p0, p1;
            byte_pairs(q6, (_Float16)1056.0f, p0, p1);
            *reinterpret_cast<h4*>(dst + (16 * g + c) * 4) = h4{p0[0], p0[1], p1[0], p1[1]};
        }
    }
};

// Q5_0 / Q5_1: element e of a block is nibble e % 16 of qs (low for e < 16)
// with bit e of qh as bit 4.  Lane group g holds elements 8g .. 8g+7.
template <int OFF>
__device__ __forceinline__ void put_five_bit(const fq_u32x4& q, uint32_t qh, int c, _Float16* dst) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int sh = g < 2 ? 0 : 4, i0 = 2 * (g & 1);
        const uint32_t c0 = five_bit((w[i0] >> sh) & 0x0F0F0F0Fu, qh >> (8 * g));
        const uint32_t c1 = five_bit((w[i0 + 1] >> sh) & 0x0F0F0F0Fu, qh >> (8 * g + 4));
        *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) = byte8(c0, c1, (_Float16)(float)OFF);
    }
}

template <>
struct Task<Q5_0> {  // block 2ch + s: d | qh | qs[16]
    uint32_t d, qh;
    fq_u32x4 q;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* b = row + 22 * (2 * ch + s);
        d = ld_u16(b);
        qh = ld_u32(b + 2);
        q = ldv(b + 6);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(d);
        B = 0.0f;
        put_five_bit<1040>(q, qh, c, dst);  // 1024 + 16
    }
};

template <>
struct Task<Q5_1> {  // block 2ch + s: d m | qh | qs[16]
    uint32_t dm, qh;
    fq_u32x4 q;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* b = row + 24 * (2 * ch + s);
        dm = ld_u32(b);
        qh = ld_u32(b + 4);
        q = ldv(b + 8);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(dm & 0xFFFFu);
        B = f16_hw(dm >> 16);
        put_five_bit<1024>(q, qh, c, dst);
    }
};

template <>
struct Task<IQ4_NL> {  // block 2ch + s: d | qs[16]; table values as int8
    uint32_t d;
    fq_u32x4 q;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* b = row + 18 * (2 * ch + s);
        d = ld_u16(b);
        q = ldv(b + 2);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(d);
        B = 0.0f;
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int sh = g < 2 ? 0 : 4, i0 = 2 * (g & 1);
            const uint32_t v0 = iq4_lookup(w[i0] >> sh), v1 = iq4_lookup(w[i0 + 1] >> sh);
            *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) =
                byte8(v0 ^ 0x80808080u, v1 ^ 0x80808080u, (_Float16)1152.0f);
        }
    }
};

template <>
struct Task<Q5_K> {  // chunk ch = pair j of super-block ch / 4; s = 0 low, 1 high nibbles
    fq_u32x4 hdr, q0, q1, h0, h1;
    int j, s;
    __device__ void load(const uint8_t* row, int ch, int s_) {
        const uint8_t* sb = row + 176 * (ch >> 2);
        j = ch & 3;
        s = s_;
        hdr = ldv(sb);
        h0 = ldv(sb + 16);
        h1 = ldv(sb + 32);
        q0 = ldv(sb + 48 + 32 * j);
        q1 = ldv(sb + 64 + 32 * j);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        uint32_t sa, ma, sb2, mb;
        Fmt<Q4_K>::scale_min(uint4{hdr.x, hdr.y, hdr.z, hdr.w}, j, sa, ma, sb2, mb);
        const float d = f16_hw(hdr.x & 0xFFFFu), dmin = f16_hw(hdr.x >> 16);
        A = d * (float)(s ? sb2 : sa);
        B = -(dmin * (float)(s ? mb : ma));
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        const int hb = 2 * j + s;  // qh bit of this sub-block
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t c0 = ((w[2 * g] >> (4 * s)) & 0x0F0F0F0Fu) |
                                (((h[2 * g] >> hb) & 0x01010101u) << 4);
            const uint32_t c1 = ((w[2 * g + 1] >> (4 * s)) & 0x0F0F0F0Fu) |
                                (((h[2 * g + 1] >> hb) & 0x01010101u) << 4);
            *reinterpret_cast<h8*>(dst + (16 * g + c) * 8) = byte8(c0, c1, (_Float16)1024.0f);
        }
    }
};

template <>
struct Task<Q3_K> {
    // chunk ch: super-block ch / 4, quarter qq = ch % 4 -> half n = qq / 2,
    // rows j' = 2 (qq % 2) + {0, 1} of 32 elements 128 n + 32 j' + l.
    // Sub-block s (16 elements): j' = 2 (qq % 2) + s / 2, l in [16 (s % 2), +16),
    // sub-scale 8 n + 2 j' + s % 2 (matmul.cpp:284-338).
    fq_u32x4 qs, hm;
    uint32_t d, lo, hi;
    int n, jp;
    __device__ void load(const uint8_t* row, int ch, int s) {
        const uint8_t* sb = row + 110 * (ch >> 2);
        const int qq = ch & 3, l0 = 16 * (s & 1);
        n = qq >> 1;
        jp = 2 * (qq & 1) + (s >> 1);
        const int i = 8 * n + 2 * jp + (s & 1);  // sub-scale index
        d = ld_u16(sb + 108);
        lo = sb[96 + (i & 7)] >> (4 * (i >> 3));
        hi = sb[104 + (i & 3)] >> (2 * (i >> 2));
        qs = ldv(sb + 32 + 32 * n + l0);
        hm = ldv(sb + l0);
    }
    __device__ void put(int c, _Float16* dst, float& A, float& B) const {
        A = f16_hw(d) * (float)((int)((lo & 15u) | ((hi & 3u) << 4)) - 32);
        B = 0.0f;
        const uint32_t Q[4] = {qs.x, qs.y, qs.z, qs.w};
        const uint32_t H[4] = {hm.x, hm.y, hm.z, hm.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {  // elements l0 + 4g .. +4: codes + 4, then -4
            const uint32_t q3 = ((Q[g] >> (2 * jp)) & 0x03030303u) |
                                (((H[g] >> (4 * n + jp)) & 0x01010101u) << 2);
            h2 p0, p1;
            byte_pairs(q3, (_Float16)1028.0f, p0, p1);
            *reinterpret_cast<h4*>(dst + (16 * g + c) * 4) = h4{p0[0], p0[1], p1[0], p1[1]};
        }
    }
};

template <int SB>
struct Mfma;

template <>
struct Mfma<32> {
    using V = h8;
    __device__ static f4 run(V a, V b, f4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<16> {
    using V = h4;
    __device__ static f4 run(V a, V b, f4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
};

// Registers holding one chunk's global loads: this thread's weight tasks,
// its share of the token operands, group sums and exponents.
template <int F, int TPT, int XPT, int SPT>
struct Pre {
    Task<F> tk[TPT];
    fq_u32x4 xv[XPT];
    float sv[SPT];
    int ev;
};

template <int F, int TPT, int XPT, int SPT, int NT, int BMT, bool HB>
__device__ __forceinline__ void prefetch(const MmqArgs& a, Pre<F, TPT, XPT, SPT>& P, int ch,
                                         int n0, int t0, int Tp) {
    constexpr int SB = SubBlock<F>::SB, NS = KC / SB;
    const _Float16* xop = static_cast<const _Float16*>(a.xop);
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
        const int i = threadIdx.x + u * NT;
        const int r = i / NS, s = i % NS;
        const int n = min(n0 + r, a.N - 1);
        // a K tail's missing sub-block re-reads sub-block 0 (its A, B are zeroed)
        const bool in = ch * KC + s * SB < a.K;
        P.tk[u].load(a.w + (size_t)n * a.row_bytes, ch, in ? s : 0);
    }
#pragma unroll
    for (int u = 0; u < XPT; ++u) {
        const int i = threadIdx.x + u * NT;
        const int tt = i / (XOP / 8), o = i % (XOP / 8);
        const int t = min(t0 + tt, Tp - 1);
        P.xv[u] = reinterpret_cast<const fq_u32x4*>(xop + (size_t)(t * a.NC + ch) * XOP)[o];
    }
    if constexpr (HB) {
#pragma unroll
        for (int u = 0; u < SPT; ++u) {
            const int i = min((int)threadIdx.x + u * NT, BMT * XSUM - 1);
            const int tt = i / XSUM, o = i % XSUM;
            const int t = min(t0 + tt, Tp - 1);
            P.sv[u] = a.xsum[(size_t)(t * a.NC + ch) * XSUM + o];
        }
    }
    {
        const int i = min((int)threadIdx.x, BMT * 16 - 1);
        const int t = min(t0 + i / 16, Tp - 1);
        P.ev = a.ex[((size_t)t * a.NC + ch) * 16 + (i & 15)];
    }
}

// ------------------------------------------------------------------ mmq
// Work-group: NWN x NWM waves; wave (wn, wm) owns WN row tiles and WM token
// tiles of 16.  BN = 16 WN NWN rows, BM = 16 WM NWM tokens.  Per chunk:
// decode the prefetched weights and copy the prefetched token operands into
// LDS, barrier, issue the global loads of the chunk PD ahead, run the MFMAs,
// barrier.  PD register sets keep PD chunks of loads in flight.
template <int F, int WN, int WM, int NWN, int NWM>
struct MmqT {
    static constexpr int SB = SubBlock<F>::SB;
    static constexpr bool HB = SubBlock<F>::HAS_B;
    using G = Geo<SB>;
    using MF = Mfma<SB>;
    using V = typename MF::V;
    static constexpr int NT = 64 * NWN * NWM;
    static constexpr int BNT = WN * NWN, BMT = WM * NWM;  // row / token tiles
    static constexpr int TASKS = 16 * BNT * G::NS, TPT = TASKS / NT;
    static constexpr int XV = BMT * (XOP / 8), XPT = XV / NT;
    static constexpr int SPT = (BMT * XSUM + NT - 1) / NT;
    static_assert(TASKS % NT == 0 && XV % NT == 0 && BMT * 16 <= NT, "tile shape");
    using P = Pre<F, TPT, XPT, SPT>;
    struct Smem {
        _Float16 xs[BMT * XOP];
        float xsum[BMT * XSUM];
        int ex[BMT * 16];
        _Float16 ws[BNT * G::NS * G::BLK];
        float As[BNT * G::NS * 16];
        float Bs[HB ? BNT * G::NS * 16 : 4];
    };

    __device__ static void step(const MmqArgs& a, Smem& sm, P& R, int ch, int ch_next, int c_end,
                                int n0, int t0, int Tp, int wn, int wm, int lane,
                                f4 (&acc)[WN][WM]) {
        // ---- registers -> LDS
#pragma unroll
        for (int u = 0; u < XPT; ++u) reinterpret_cast<fq_u32x4*>(sm.xs)[threadIdx.x + u * NT] = R.xv[u];
        if constexpr (HB) {
#pragma unroll
            for (int u = 0; u < SPT; ++u)
                if (threadIdx.x + u * NT < BMT * XSUM) sm.xsum[threadIdx.x + u * NT] = R.sv[u];
        }
        if (threadIdx.x < BMT * 16) sm.ex[threadIdx.x] = R.ev;
#pragma unroll
        for (int u = 0; u < TPT; ++u) {
            const int i = threadIdx.x + u * NT;
            const int r = i / G::NS, s = i % G::NS;
            const int nt = r >> 4, c = r & 15;
            float A, B;
            R.tk[u].put(c, sm.ws + (nt * G::NS + s) * G::BLK, A, B);
            if (ch * KC + s * SB >= a.K) A = B = 0.0f;  // K tail: an empty sub-block
            sm.As[(nt * G::NS + s) * 16 + c] = A;
            if constexpr (HB) sm.Bs[(nt * G::NS + s) * 16 + c] = B;
        }
        __syncthreads();
        if (ch_next < c_end) prefetch<F, TPT, XPT, SPT, NT, BMT, HB>(a, R, ch_next, n0, t0, Tp);
        // ---- MFMA over the chunk's sub-blocks; R is in units of 2^-e per token
        int ej[WM];
#pragma unroll
        for (int j = 0; j < WM; ++j) ej[j] = sm.ex[(wm * WM + j) * 16 + (lane & 15)];
#pragma unroll
        for (int s = 0; s < G::NS; ++s) {
            V xh[WM], xl[WM];
            float sx[WM];
#pragma unroll
            for (int j = 0; j < WM; ++j) {
                const _Float16* xb = sm.xs + (wm * WM + j) * XOP + s * 2 * G::BLK + lane * G::EPL;
                xh[j] = *reinterpret_cast<const V*>(xb);
                xl[j] = *reinterpret_cast<const V*>(xb + G::BLK);
                if constexpr (HB)
                    sx[j] = ldexpf(sm.xsum[(wm * WM + j) * XSUM + s * 16 + (lane & 15)], ej[j]);
            }
#pragma unroll
            for (int i = 0; i < WN; ++i) {
                const int nt = wn * WN + i;
                const V wv = *reinterpret_cast<const V*>(sm.ws + (nt * G::NS + s) * G::BLK +
                                                         lane * G::EPL);
                const f4 Av = *reinterpret_cast<const f4*>(sm.As + (nt * G::NS + s) * 16 +
                                                           4 * (lane >> 4));
                f4 Bv = f4{0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (HB)
                    Bv = *reinterpret_cast<const f4*>(sm.Bs + (nt * G::NS + s) * 16 +
                                                      4 * (lane >> 4));
#pragma unroll
                for (int j = 0; j < WM; ++j) {
                    f4 Rr = MF::run(wv, xh[j], f4{0.0f, 0.0f, 0.0f, 0.0f});
                    Rr = MF::run(wv, xl[j], Rr);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float v = __builtin_fmaf(ldexpf(Rr[r], ej[j]), Av[r], acc[i][j][r]);
                        if constexpr (HB) v = __builtin_fmaf(Bv[r], sx[j], v);
                        acc[i][j][r] = v;
                    }
                }
            }
        }
        __syncthreads();
    }
};

template <int F, int WN, int WM, int NWN, int NWM, int PD>
__global__ __launch_bounds__(64 * NWN * NWM) void mmq_kernel(MmqArgs a) {
    using T = MmqT<F, WN, WM, NWN, NWM>;
    __shared__ __attribute__((aligned(16))) typename T::Smem sm;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wn = wave % NWN, wm = wave / NWN;
    const int n0 = blockIdx.x * 16 * T::BNT, t0 = blockIdx.y * T::BMT;
    const int cps = (a.NC + gridDim.z - 1) / gridDim.z;
    const int c_begin = blockIdx.z * cps, c_end = min(a.NC, c_begin + cps);
    const int Tp = (a.M + 15) >> 4;

    f4 acc[WN][WM];
#pragma unroll
    for (int i = 0; i < WN; ++i)
#pragma unroll
        for (int j = 0; j < WM; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    typename T::P R0, R1;
    if (c_begin < c_end)
        prefetch<F, T::TPT, T::XPT, T::SPT, T::NT, T::BMT, T::HB>(a, R0, c_begin, n0, t0, Tp);
    if (PD == 2 && c_begin + 1 < c_end)
        prefetch<F, T::TPT, T::XPT, T::SPT, T::NT, T::BMT, T::HB>(a, R1, c_begin + 1, n0, t0, Tp);
    for (int ch = c_begin; ch < c_end; ch += PD) {
        T::step(a, sm, R0, ch, ch + PD, c_end, n0, t0, Tp, wn, wm, lane, acc);
        if (PD == 2 && ch + 1 < c_end)
            T::step(a, sm, R1, ch + 1, ch + 1 + PD, c_end, n0, t0, Tp, wn, wm, lane, acc);
    }

    // ---- epilogue: lane holds rows n = tile + 4 (lane / 16) + r, token lane % 16
    float* out = gridDim.z > 1 ? a.part + (size_t)blockIdx.z * a.M * a.N : a.y;
    const bool fin = gridDim.z == 1;
#pragma unroll
    for (int j = 0; j < WM; ++j) {
        const int m = (t0 + wm * WM + j) * 16 + (lane & 15);
        if (m >= a.M) continue;
#pragma unroll
        for (int i = 0; i < WN; ++i) {
            const int nb = n0 + (wn * WN + i) * 16 + 4 * (lane >> 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = nb + r;
                if (n >= a.N) continue;
                float v = acc[i][j][r];
                if (fin && a.bias_mode == 1) v += n < a.bias_len ? a.bias[n] : 0.0f;
                if (fin && a.bias_mode == 2) v += a.bias[(size_t)m * a.N + n];
                out[(size_t)m * a.N + n] = v;
            }
        }
    }
}

// y = sum over splits of the partial slabs, in split order, plus the bias.
// Four consecutive outputs per thread (16-byte loads and stores), the same
// split order: bit-identical to reduce_kernel.  Needs M N and N multiples of
// 4 and a 16-byte aligned y.  S > 0: the split count at compile time, so all
// S slab loads of a thread are in flight at once (a runtime count loop waits
// for each load before issuing the next); S = 0: any count.
template <int S>
__global__ __launch_bounds__(256) void reduce4_kernel(MmqArgs a, int splits) {
    const size_t total = (size_t)a.M * a.N, t4 = total / 4;
    const float4* part = reinterpret_cast<const float4*>(a.part);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < t4; i += (size_t)gridDim.x * 256) {
        float4 v = part[i];
        if constexpr (S > 0) {
            float4 u[S];
#pragma unroll
            for (int z = 1; z < S; ++z) u[z] = part[(size_t)z * t4 + i];
#pragma unroll
            for (int z = 1; z < S; ++z) {
                v.x += u[z].x;
                v.y += u[z].y;
                v.z += u[z].z;
                v.w += u[z].w;
            }
        } else {
            for (int z = 1; z < splits; ++z) {
                const float4 u = part[(size_t)z * t4 + i];
                v.x += u.x;
                v.y += u.y;
                v.z += u.z;
                v.w += u.w;
            }
        }
        const int n = (int)((4 * i) % a.N);
        if (a.bias_mode == 1) {
            v.x += n < a.bias_len ? a.bias[n] : 0.0f;
            v.y += n + 1 < a.bias_len ? a.bias[n + 1] : 0.0f;
            v.z += n + 2 < a.bias_len ? a.bias[n + 2] : 0.0f;
            v.w += n + 3 < a.bias_len ? a.bias[n + 3] : 0.0f;
        } else if (a.bias_mode == 2) {
            v.x += a.bias[4 * i];
            v.y += a.bias[4 * i + 1];
            v.z += a.bias[4 * i + 2];
            v.w += a.bias[4 * i + 3];
        }
        reinterpret_cast<float4*>(a.y)[i] = v;
    }
}

__global__ __launch_bounds__(256) void reduce_kernel(MmqArgs a, int splits) {
    const size_t total = (size_t)a.M * a.N;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (size_t)gridDim.x * 256) {
        float v = a.part[i];
        for (int z = 1; z < splits; ++z) v += a.part[(size_t)z * total + i];
        const int n = (int)(i % a.N);
        if (a.bias_mode == 1) v += n < a.bias_len ? a.bias[n] : 0.0f;
        if (a.bias_mode == 2) v += a.bias[i];
        a.y[i] = v;
    }
}

template <int F, int WN, int WM, int NWN, int NWM, int PD>
hipError_t launch_t(const MmqArgs& a, int gx, int gy, int splits, hipStream_t st) {
    hipLaunchKernelGGL((mmq_kernel<F, WN, WM, NWN, NWM, PD>), dim3(gx, gy, splits),
                       dim3(64 * NWN * NWM), 0, st, a);
    return hipGetLastError();
}

template <int F>
hipError_t launch_f(const MmqArgs& a, int shape, int gx, int gy, int splits, hipStream_t st) {
    switch (shape) {
        case MMQ_SMALL1: return launch_t<F, 2, 1, 4, 1, 2>(a, gx, gy, splits, st);
        case MMQ_SMALL2: return launch_t<F, 2, 2, 4, 1, 2>(a, gx, gy, splits, st);
        case MMQ_MID: return launch_t<F, 2, 4, 4, 1, 1>(a, gx, gy, splits, st);
        default: return launch_t<F, 4, 4, 2, 2, 1>(a, gx, gy, splits, st);
    }
}

}  // namespace

void mmq_shape(int shape, int* bn, int* bm) {
    switch (shape) {
        case MMQ_SMALL1: *bn = 128; *bm = 16; return;
        case MMQ_SMALL2: *bn = 128; *bm = 32; return;
        case MMQ_MID: *bn = 128; *bm = 64; return;
        default: *bn = 128; *bm = 128; return;
    }
}

hipError_t launch_xprep(int dtype, const float* x, int M, int K, int NC, _Float16* xop,
                        float* xsum, int* ex, hipStream_t st) {
    const dim3 grid((M + 15) / 16, NC);
    if (dtype == Q6_K || dtype == Q3_K)
        hipLaunchKernelGGL(xprep_kernel<16>, grid, dim3(256), 0, st, x, M, K, NC, xop, xsum, ex);
    else
        hipLaunchKernelGGL(xprep_kernel<32>, grid, dim3(256), 0, st, x, M, K, NC, xop, xsum, ex);
    return hipGetLastError();
}

hipError_t launch_reduce(const MmqArgs& a, int splits, hipStream_t st) {
    const size_t total = (size_t)a.M * a.N;
    if (a.N % 4 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(a.part) & 15) == 0) {
        const size_t t4 = total / 4;
        const int grid = (int)((t4 + 255) / 256 < 4096 ? (t4 + 255) / 256 : 4096);
        switch (splits) {
            case 2: hipLaunchKernelGGL(reduce4_kernel<2>, dim3(grid), dim3(256), 0, st, a, splits); break;
            case 3: hipLaunchKernelGGL(reduce4_kernel<3>, dim3(grid), dim3(256), 0, st, a, splits); break;
            case 4: hipLaunchKernelGGL(reduce4_kernel<4>, dim3(grid), dim3(256), 0, st, a, splits); break;
            case 5: hipLaunchKernelGGL(reduce4_kernel<5>, dim3(grid), dim3(256), 0, st, a, splits); break;
            case 6: hipLaunchKernelGGL(reduce4_kernel<6>, dim3(grid), dim3(256), 0, st, a, splits); break;
            case 8: hipLaunchKernelGGL(reduce4_kernel<8>, dim3(grid), dim3(256), 0, st, a, splits); break;
            default: hipLaunchKernelGGL(reduce4_kernel<0>, dim3(grid), dim3(256), 0, st, a, splits);
        }
        return hipGetLastError();
    }
    const int grid = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    hipLaunchKernelGGL(reduce_kernel, dim3(grid), dim3(256), 0, st, a, splits);
    return hipGetLastError();
}

hipError_t launch_mmq(int dtype, const MmqArgs& a, int shape, int gx, int gy, int splits,
                      hipStream_t st) {
    const hipError_t e = with_format(dtype, hipErrorInvalidValue, [&](auto f) {
        return launch_f<decltype(f)::value>(a, shape, gx, gy, splits, st);
    });
    if (e != hipSuccess || splits <= 1) return e;
    return launch_reduce(a, splits, st);
}

}  // namespace fq
