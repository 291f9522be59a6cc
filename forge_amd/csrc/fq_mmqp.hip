// fq_mmqp.hip -- prefill (M > 32 tokens) for Q8_0, Q4_0, Q4_1, Q5_0, Q5_1,
// Q4_K and Q6_K on v_mfma_f32_32x32x16_f16.
//
//   D[token][n] = X[token][k] . W[n][k]^T on the fp16 matrix cores, with the
// tokens as x 2^-e(token) in fp16 hi + lo and the weights' integer codes
// exact in fp16; one FMA per output and 32-element block folds in the block
// scale, and the formats with a per-block minimum (Q4_1, Q4_K) add it as an
// fp32 outer product (mmqp_kernel below).
//
// Token prep is one launch (xprep4_kernel): the per-token exponent, then the
// hi/lo operands in the A-operand layout (and the per-token block sums for
// the minimum term).  Q6_K, whose scales cover 16 elements, first goes
// through q6c_kernel into 36-byte blocks of int8 codes (below) and uses the
// operand order in which each MFMA covers one 16-element sub-block.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fq_dma.h"
#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"
#include "fq_mfma16.h"

namespace fq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BMT = 128, BNT = 256;  // tokens, rows per work-group
constexpr int KS = 64;               // K elements per step (two blocks)
constexpr int XT = 1024;             // halves per (32-token tile, 16-k quarter): hi then lo
constexpr int NBUF = 3;              // LDS buffers per operand: steps s, s + 1, s + 2
constexpr int NW = 8;                // waves per work-group

// ------------------------------------------------------------- token prep
// Per token an exponent e = ilogb(max |x|) - 14 (0 for an all-zero token),
// so that x 2^-e lies below 2^15 in magnitude, and x 2^-e split into fp16
// hi + lo, written as the A operand of v_mfma_f32_32x32x16_f16: for token
// tile T = m / 32 and quarter kq (the MFMA half kq % 2 of block kq / 2), lane
// (m % 32) + 32 g holds elements 32 (kq / 2) + 16 g + 8 (kq % 2) +
// slot_elem(j), j = 0..7, the hi block then the lo block 512 halves on
// (SUB16: elements 16 kq + 8 g + slot_elem(j), so that each quarter is one
// 16-element sub-block).
//
// One launch: work-group j owns tokens 4 j .. 4 j + 3 (all of K).  Piece p = ((2 kq + g) 4 + t): token t's eight elements of quarter kq,
// lane group g -- four consecutive threads write one 64-byte run (hi, and
// lo 1 KiB on).  Pass 1 finds each token's largest |x| (x read once from
// HBM), pass 2 writes the operands from the values kept in registers (those
// of K beyond 8192 are read again, from L2).  The work-groups cover every
// token slot of the last tile (slots past M are zero).
template <bool SUB16>
__global__ __launch_bounds__(1024) void xprep4_kernel(const float* __restrict__ x, int M, int K,
                                                      int* __restrict__ ex,
                                                      _Float16* __restrict__ xop,
                                                      float* __restrict__ xsum) {
    __shared__ float wmax[16][4];
    __shared__ int es[4];
    const int tid = threadIdx.x, t = tid & 3;
    const int m = 4 * blockIdx.x + t;
    const bool live = m < M;
    const float* xr = x + (size_t)min(m, M - 1) * K;
    const int KQ = K / 16, P = 8 * KQ;  // pieces per work-group
    auto src = [&](int p) {
        const int gq = p >> 2, g = gq & 1, kq = gq >> 1;
        return SUB16 ? xr + 16 * kq + 8 * g : xr + 32 * (kq >> 1) + 16 * g + 8 * (kq & 1);
    };
    // the first CP pieces of a thread stay in registers for the second pass
    // (all of them up to K = 8192); the rest are read again, from L2
    constexpr int CP = 4;
    float4 ca[CP], cb[CP];
    float mx = 0.0f;
    auto amax = [](float4 a, float4 b) {
        return fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                     fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    };
#pragma unroll
    for (int it = 0; it < CP; ++it) {
        const int p = tid + 1024 * it;
        ca[it] = cb[it] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (p < P) {
            const float* s = src(p);
            ca[it] = *reinterpret_cast<const float4*>(s);
            cb[it] = *reinterpret_cast<const float4*>(s + 4);
            mx = fmaxf(mx, amax(ca[it], cb[it]));
        }
    }
    for (int p = tid + 1024 * CP; p < P; p += 1024) {
        const float* s = src(p);
        mx = fmaxf(mx, amax(*reinterpret_cast<const float4*>(s),
                            *reinterpret_cast<const float4*>(s + 4)));
    }
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) < 4) wmax[tid >> 6][t] = mx;
    __syncthreads();
    if (tid < 4) {
        float v = 0.0f;
        for (int w = 0; w < 16; ++w) v = fmaxf(v, wmax[w][tid]);
        const int e = (v > 0.0f && v <= 3.0e38f) ? ilogbf(v) - 14 : 0;
        es[tid] = e;
        if (4 * blockIdx.x + tid < M) ex[4 * blockIdx.x + tid] = e;
    }
    __syncthreads();
    const int e = es[t];
    const int T = m >> 5, lm = m & 31;
    auto piece = [&](int p, float4 a, float4 b) {
        const int gq = p >> 2, g = gq & 1, kq = gq >> 1;
        h8 hi = {}, lo = {};
        float w[8] = {};
        if (live) {
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) w[j] = __builtin_amdgcn_ldexpf(v[j], -e);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float u = w[slot_elem(j)];
                hi[j] = (_Float16)u;
                lo[j] = (_Float16)(u - (float)hi[j]);
            }
        }
        _Float16* dst = xop + ((size_t)T * KQ + kq) * XT + (lm + 32 * g) * 8;
        *reinterpret_cast<h8*>(dst) = hi;
        *reinterpret_cast<h8*>(dst + 512) = lo;
        if (xsum) {
            // the token's sum of x 2^-e over its 32-element sub-block kq / 2:
            // pieces p, p ^ 4, p ^ 8, p ^ 12 of one wave, added in a fixed tree
            float t8 = ((w[0] + w[1]) + (w[2] + w[3])) + ((w[4] + w[5]) + (w[6] + w[7]));
            t8 += __shfl_xor(t8, 4, 64);
            t8 += __shfl_xor(t8, 8, 64);
            if ((p & 12) == 0) xsum[((size_t)T * (K / 32) + (kq >> 1)) * 32 + lm] = t8;
        }
    };
    // P is a multiple of 64: whole waves take part in each piece's shuffles
#pragma unroll
    for (int it = 0; it < CP; ++it) {
        const int p = tid + 1024 * it;
        if (p < P) piece(p, ca[it], cb[it]);
    }
    for (int p = tid + 1024 * CP; p < P; p += 1024) {
        const float* s = src(p);
        piece(p, *reinterpret_cast<const float4*>(s), *reinterpret_cast<const float4*>(s + 4));
    }
}

// -------------------------------------------------------- weight operands
template <int F>
struct PB;

// The K order inside a 32-element block: MFMA half h takes from lane group g
// the elements 16 g + 8 h + j, so a lane's 16 elements of a block are
// contiguous (one 16-byte read of Q8_0 codes; the 16 Q4_0 bytes, low nibbles
// for g = 0, high for g = 1).  xprep4_kernel lays the tokens out the same
// way.
//
// Q8_0 block (34 B): d @0, qs int8[32] @2.  Lane group g: bytes
// qs[16 g, 16 g + 16) as fp16 (+128 via the sign bit, so the bytes are
// unsigned, then -1152 = -(1024 + 128)); half h = bytes 8 h .. 8 h + 7.
template <>
struct PB<Q8_0> {
    static constexpr int BB = 34, SB = 2 * BB;  // bytes per block, per step
    static constexpr int GS = 16;               // byte offset of lane group g
    static constexpr int QOFF = 2;              // codes after the scale
    static constexpr bool MIN = false;          // no per-block minimum term
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int, h8& b0, h8& b1) {
        b0 = byte8(q[0] ^ 0x80808080u, q[1] ^ 0x80808080u, (_Float16)1152.0f);
        b1 = byte8(q[2] ^ 0x80808080u, q[3] ^ 0x80808080u, (_Float16)1152.0f);
    }
};

// Q4_0 block (18 B): d @0, qs[16] @2; element j < 16 is the low nibble of
// byte j, element j + 16 the high nibble (value - 8).  Lane group g: nibble
// g of bytes 8 h .. 8 h + 7 for half h.
template <>
struct PB<Q4_0> {
    static constexpr int BB = 18, SB = 2 * BB;
    static constexpr int GS = 0;
    static constexpr int QOFF = 2;
    static constexpr bool MIN = false;
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int g, h8& b0, h8& b1) {
        b0 = nib8(q[0], q[1], 4 * g, (_Float16)1032.0f);
        b1 = nib8(q[2], q[3], 4 * g, (_Float16)1032.0f);
    }
};

// Q4_1 block (20 B): d @0, m @2, qs[16] @4 as Q4_0 but unsigned, w = d q +
// m: the m term goes through the per-token block sums of xprep4_kernel.
template <>
struct PB<Q4_1> {
    static constexpr int BB = 20, SB = 2 * BB;
    static constexpr int GS = 0;
    static constexpr int QOFF = 4;
    static constexpr bool MIN = true;
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int g, h8& b0, h8& b1) {
        b0 = nib8(q[0], q[1], 4 * g, (_Float16)1024.0f);
        b1 = nib8(q[2], q[3], 4 * g, (_Float16)1024.0f);
    }
};

// Q5_0 block (22 B): d @0, qh @2 (bit j: the fifth bit of element j),
// qs[16] @6 (element j < 16: low nibble of byte j, j + 16: high nibble),
// value - 16.  Q5_1 block (24 B): d @0, m @2, qh @4, qs[16] @8, unsigned,
// w = d q + m.  codes() hands ops() the lane group's 16 five-bit codes.
template <>
struct PB<Q5_0> {
    static constexpr int BB = 22, SB = 2 * BB;
    static constexpr int GS = 0, QOFF = 6, HOFF = 2;
    static constexpr bool MIN = false;
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int, h8& b0, h8& b1) {
        b0 = byte8(q[0], q[1], (_Float16)1040.0f);
        b1 = byte8(q[2], q[3], (_Float16)1040.0f);
    }
};
template <>
struct PB<Q5_1> {
    static constexpr int BB = 24, SB = 2 * BB;
    static constexpr int GS = 0, QOFF = 8, HOFF = 4;
    static constexpr bool MIN = true;
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int, h8& b0, h8& b1) {
        b0 = byte8(q[0], q[1], (_Float16)1024.0f);
        b1 = byte8(q[2], q[3], (_Float16)1024.0f);
    }
};

// Q4_K super-block (144 B, matmul.cpp:340-377): d @0, dmin @2, scales[12]
// @4 (6-bit scale and min per 32-element sub-block), qs[128] @16.  A step
// (64 elements) is sub-block pair p = s mod 4 of super-block s / 4: the
// low nibbles of qs[32 p, 32 p + 32) are sub-block 2 p (block b = 0), the
// high nibbles sub-block 2 p + 1 (b = 1).  Per row and step three 16-byte
// chunks are copied, all aligned: the header and the pair's 32 code bytes.
// Lane group g: bytes 16 g .. 16 g + 15 of the pair, nibble b; half h =
// bytes 8 h .. 8 h + 7.  w = d sc q - dmin m: the min term goes through
// the per-token sub-block sums of xprep4_kernel.
template <>
struct PB<Q4_K> {
    static constexpr int CH = 3;
    static constexpr bool MIN = true;
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int, h8& b0, h8& b1) {
        b0 = nib8(q[0], q[1], 4 * B, (_Float16)1024.0f);
        b1 = nib8(q[2], q[3], 4 * B, (_Float16)1024.0f);
    }
};

// Q6_K as converted by q6c_kernel (36-byte blocks of 32 elements): d @0,
// the two sub-block scales int8 @2, @3, then the 32 six-bit codes q (0..63)
// @4, stored so that lane group g's 16 bytes are elements 8 g .. 8 g + 7 of
// sub-block 0 then of sub-block 1: half h of the MFMA is sub-block h, in the
// SUB16 operand order of xprep4_kernel.  A code becomes fp16 1024 + q, then
// q - 32 after subtracting 1056.
template <>
struct PB<Q6_K> {
    static constexpr int BB = 36, SB = 2 * BB;
    static constexpr int GS = 16;
    static constexpr int QOFF = 4;
    static constexpr bool MIN = false;
    template <int B>
    __device__ static void ops(const uint32_t (&q)[4], int, h8& b0, h8& b1) {
        b0 = byte8(q[0], q[1], (_Float16)1056.0f);
        b1 = byte8(q[2], q[3], (_Float16)1056.0f);
    }
};

// Chunks per row and step, and the byte offset (within the row) of chunk p
// of step s, less 16 p.  Q8_0 / Q4_0: a step of a row (68 / 36 bytes)
// starts (s SB) mod 16 = 0, 4, 8 or 12 bytes into a 16-byte chunk (rows are
// 16-byte aligned), so CH chunks cover it for every step.
template <int F>
struct Chunks {
    static constexpr int CH = (PB<F>::SB + 12 + 15) / 16;
    // step s0 + u starts (u SB) mod 16 bytes into its first chunk (s0 a
    // multiple of 4 and rows 16-byte aligned)
    static constexpr int o4(int u) { return u * PB<F>::SB & 15; }
    __device__ static size_t off(int s, int) { return (size_t)s * PB<F>::SB & ~(size_t)15; }
};
template <>
struct Chunks<Q6_K> {  // a step (72 bytes) starts 0 or 8 bytes into a chunk
    static constexpr int CH = 5;
    static constexpr int o4(int u) { return u * 72 & 15; }
    __device__ static size_t off(int s, int) { return (size_t)s * 72 & ~(size_t)15; }
};
template <>
struct Chunks<Q5_1> {  // a step (48 bytes) starts on a chunk
    static constexpr int CH = 3;
    static constexpr int o4(int) { return 0; }
    __device__ static size_t off(int s, int) { return (size_t)s * 48; }
};
template <>
struct Chunks<Q4_1> {  // a step (40 bytes) starts 0 or 8 bytes into a chunk
    static constexpr int CH = 3;
    static constexpr int o4(int u) { return u * 40 & 15; }
    __device__ static size_t off(int s, int) { return (size_t)s * 40 & ~(size_t)15; }
};
template <>
struct Chunks<Q4_K> {
    static constexpr int CH = 3;
    static constexpr int o4(int u) { return 4 * u; }  // the pair index, as 4 p
    __device__ static size_t off(int s, int p) {
        return (size_t)144 * (s >> 2) + (p ? 32 * (s & 3) : 0);
    }
};

// The 16 code bytes of lane group g of block b, for a row whose step starts
// O4 bytes into its LDS slot (the slot holds the step's 16-byte chunks, so
// O4 = (s SB) mod 16, a multiple of 4).  One or two aligned 16-byte reads
// (16-byte reads at the slots' 80 / 48-byte stride fall on distinct banks),
// then dword selection and byte alignment by constants.
template <int F, int O4, int B>
__device__ __forceinline__ void codes16(const uint8_t* row, int g, uint32_t (&q)[4]) {
    using P = PB<F>;
    constexpr int X = O4 + P::BB * B + P::QOFF;  // first code byte, lane group 0
    constexpr int SH = X & 15, SD = SH >> 2, R = SH & 3;
    const uint8_t* c0 = row + (X & ~15) + P::GS * g;
    typedef const __attribute__((address_space(3))) fq_u32x4* lds_v4;
    const fq_u32x4 v0 = *reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(c0));
    fq_u32x4 v1 = v0;
    if constexpr (SH != 0) v1 = *reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(c0 + 16));
    const uint32_t w[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if constexpr (R == 0) q[k] = w[SD + k];
        else q[k] = __builtin_amdgcn_alignbyte(w[SD + k + 1], w[SD + k], R);
    }
}

// The 16 code bytes of lane group g of block B and the block's scale and
// minimum coefficient (d sc, dmin m; the minimum is 0 without a min term),
// for a row slot whose step starts O4 bytes into its first chunk.
template <int F, int O4, int B>
__device__ __forceinline__ void codes(const uint8_t* row, int g, uint32_t (&q)[4]) {
    if constexpr (F == Q4_K) {  // planes of BNT x 16 bytes: header, codes 0..15, codes 16..31
        typedef const __attribute__((address_space(3))) fq_u32x4* lds_v4;
        const fq_u32x4 v =
            *reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(row + BNT * 16 * (1 + g)));
        q[0] = v[0];
        q[1] = v[1];
        q[2] = v[2];
        q[3] = v[3];
    } else if constexpr (F == Q5_0 || F == Q5_1) {
        uint32_t n[4];
        codes16<F, O4, B>(row, g, n);  // the 16 qs bytes
        const uint32_t qh = lds4_a2(row + O4 + PB<F>::BB * B + PB<F>::HOFF) >> (16 * g);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // fifth bits of elements 16 g + 4 k .. + 3 to bit 4 of each byte
            const uint32_t hb = ((((qh >> (4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
            q[k] = ((n[k] >> (4 * g)) & 0x0F0F0F0Fu) | hb;
        }
    } else {
        codes16<F, O4, B>(row, g, q);
    }
}
template <int F, int O4, int B>
__device__ __forceinline__ void scales(const uint8_t* row, float& db, float& mn) {
    if constexpr (F == Q4_K) {
        typedef const __attribute__((address_space(3))) fq_u32x4* lds_v4;
        const fq_u32x4 h = *reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(row));
        uint32_t sa, ma, sb, mb;
        Fmt<Q4_K>::scale_min(uint4{h[0], h[1], h[2], h[3]}, O4 / 4, sa, ma, sb, mb);
        db = f16_hw(h[0] & 0xFFFFu) * (float)(B ? sb : sa);
        mn = f16_hw(h[0] >> 16) * (float)(B ? mb : ma);
    } else if constexpr (F == Q6_K) {  // db = d sc1 and mn = sc0 / sc1 (sc1 = 0: d sc0, 1)
        const uint32_t h = lds4_a2(row + O4 + PB<F>::BB * B);
        const float d = f16_hw(h & 0xFFFFu);
        const float s0 = (float)(int8_t)(h >> 16), s1 = (float)(int8_t)(h >> 24);
        db = d * (s1 != 0.0f ? s1 : s0);
        mn = s1 != 0.0f ? s0 / s1 : 1.0f;
    } else if constexpr (F == Q4_1 || F == Q5_1) {
        const uint32_t dm = lds4_a2(row + O4 + PB<F>::BB * B);
        db = f16_hw(dm & 0xFFFFu);
        mn = -f16_hw(dm >> 16);  // w = d q + m: the term is -(-m) S
    } else {
        db = f16_hw(*reinterpret_cast<const uint16_t*>(row + O4 + PB<F>::BB * B));
        mn = 0.0f;
    }
}

template <int F>
struct Tile {
    static constexpr int CH = Chunks<F>::CH;            // chunks per row and step
    // Q8_0 / Q4_0: rows of CH chunks; Q4_K: CH planes of one chunk per row
    static constexpr bool PLANES = F == Q4_K;
    static constexpr int WROW = PLANES ? 16 : 16 * CH;  // LDS bytes between rows
    static constexpr int WCH = BNT * CH;                // chunks of a step's weight tile
    static constexpr int WIN = WCH / 64;                // copy instructions per step (whole)
    static_assert(WCH % 64 == 0, "whole copy instructions");
    static constexpr int WI_LO = WIN / NW, WI_HI = (WIN + NW - 1) / NW;
    static constexpr int W_HI = WIN - NW * WI_LO;       // waves that issue WI_HI copies
    static constexpr int WBUF = BNT * 16 * CH;          // bytes per weight buffer
    static constexpr bool MIN = PB<F>::MIN;
    // token copies per wave: 1 KiB each, plus one of 128 bytes (8 lanes) of
    // sub-block sums with a min term
    static constexpr int XI = 4 + (MIN ? 1 : 0);
    static constexpr int XOPB = 16 * XT * 2;            // token operand bytes per buffer
    static constexpr int XBUF = XOPB + (MIN ? 1024 : 0);
    static constexpr int LDS = NBUF * (XBUF + WBUF);
};

// A work-group owns 128 tokens x 256 rows and a K range (split-K when that
// shortens the busiest CU's work; the reduce adds the slabs in split order).
// Eight waves, each 64 tokens x 64 rows (2 x 2 tiles of 32 x 32).
//
// Per 32-element block b:
//   A (32 tokens x 16 k): x 2^-e(token) as fp16 hi + lo (xprep4_kernel),
//   B (16 k x 32 rows):   the block's integer codes, exact in fp16,
//   D_b = A_hi B + A_lo B  (two MFMAs per 16 k, one fp32 result per block),
//   acc += d_b(n) D_b      (one FMA per output and block),
//   acc -= S_b(token) m_b(n) (Q4_1, Q4_K: v_mfma_f32_32x32x2_f32 over a
//                          step's two blocks, S_b the token's scaled sum),
// y = 2^e(token) acc at the end.  Weights are the B operand so that a lane's
// 16 results all belong to one row n: the block scale d_b(n) is one value
// per lane.  x_hi + x_lo carry 22 significant bits.
//
// Both operands reach LDS by direct copies into three buffers: while step s
// is computed, the copies of steps s + 1 and s + 2 are in flight, and one
// barrier per step publishes the next step's buffers.
template <int F>
__global__ __launch_bounds__(512) void mmqp_kernel(MmqArgs a, int steps_per_split) {
    using P = PB<F>;
    using TL = Tile<F>;
    constexpr int WROW = TL::WROW;
    __shared__ __attribute__((aligned(16))) uint8_t lds[TL::LDS];
    uint8_t* const xs0 = lds;                       // NBUF token buffers
    uint8_t* const ws0 = lds + NBUF * TL::XBUF;     // NBUF weight buffers
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;  // 64-token / 64-row quadrant
    const int n0 = blockIdx.x * BNT, m0 = blockIdx.y * BMT;
    const int nsteps = a.K / KS;
    const int s0 = blockIdx.z * steps_per_split, s1 = min(nsteps, s0 + steps_per_split);
    const int Tn = (a.M + 31) / 32;         // token tiles in the operand buffer
    const int KQ = a.K / 16;

    // copy sources of this lane: token run (tile T0 + wave / 2, half wave & 1
    // of its 8 KiB per step), and the 16-byte weight chunks L = 64 (NW q +
    // wave) + lane of the row-major [row][CH] step tile (rows clamped to a
    // real row)
    const int T = min(m0 / 32 + (wave >> 1), Tn - 1);
    // wave-uniform bases (scalar registers) and per-lane 32-bit offsets (the
    // host keeps the weights under 4 GiB)
    const uint8_t* const xbase =
        reinterpret_cast<const uint8_t*>(a.xop) + ((size_t)T * KQ * XT) * 2 + (wave & 1) * 4096;
    const int nwi = wave < TL::W_HI ? TL::WI_HI : TL::WI_LO;  // wave-uniform
    uint32_t woff[TL::WI_HI];
#pragma unroll
    for (int q = 0; q < TL::WI_HI; ++q) {
        const int L = min(64 * (NW * q + wave) + lane, TL::WCH - 1);
        // row-major [row][CH] slots, or (PLANES) chunk-major [CH][row]: copy
        // instruction k = NW q + wave is plane k / 4, wave-uniform
        const int r = TL::PLANES ? L % BNT : L / TL::CH;
        const int p = TL::PLANES ? L / BNT : L - r * TL::CH;
        woff[q] = (uint32_t)min(n0 + r, a.N - 1) * (uint32_t)a.row_bytes + 16 * p;
    }
    // sub-block sums (min term): tile T, block wave & 1, lanes 0..7
    const float* const sbase =
        TL::MIN ? a.xsum + ((size_t)T * (a.K / 32) + (wave & 1)) * 32 : nullptr;
    // Q5_0: a 44-byte step that starts 4 bytes into its first chunk ends 16
    // bytes before the last of its four: on the matrix's last row that chunk
    // lies past the end (its bytes are never read)
    const uint32_t wend = (uint32_t)a.N * (uint32_t)a.row_bytes - 16;
    const uint32_t lds_base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds);
    auto issue = [&](int s) {
        const int buf = s % NBUF;
        const uint32_t xl = lds_base + buf * TL::XBUF + wave * 4096;
        const uint8_t* xg = xbase + (size_t)s * 4 * XT * 2;
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16s(16 * lane + 1024 * i, xg, xl + 1024 * i);
        if constexpr (TL::MIN) {
            const uint32_t sl = lds_base + buf * TL::XBUF + TL::XOPB + wave * 128;
            if (lane < 8)
                dma16s(16 * lane, reinterpret_cast<const uint8_t*>(sbase + (size_t)64 * s), sl);
        }
        const uint32_t wl = lds_base + NBUF * TL::XBUF + buf * TL::WBUF + wave * 1024;
#pragma unroll
        for (int q = 0; q < TL::WI_HI; ++q)
            if (q < nwi) {
                const uint32_t so =
                    (uint32_t)Chunks<F>::off(s, TL::PLANES ? (NW * q + wave) >> 2 : 0);
                const uint32_t vo = F == Q5_0 ? min(woff[q], wend - so) : woff[q];
                dma16s(vo, a.w + so, wl + NW * 1024 * q);
            }
    };
    // this wave's copies of step s are complete (those of step s + 1 may
    // still be in flight)
    auto wait_step = [&](bool next_in_flight) {
        if (!next_in_flight) wait_vm<0>();
        else if (nwi == TL::WI_HI) wait_vm<TL::XI + TL::WI_HI>();
        else wait_vm<TL::XI + TL::WI_LO>();
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int g = lane >> 5, c = lane & 31;
    // The operands of the next (block, token tile) are read from LDS while
    // the current one's MFMAs run, and a stage's block-scale fold (FMAs on
    // its chain results) waits until the next stage's MFMAs are issued, so
    // the matrix cores and the LDS reads of a wave overlap.
    auto read_a = [&](const _Float16* xs, int b, int i, h8 (&r)[4]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const _Float16* xp = xs + ((2 * wm + i) * 4 + 2 * b + h) * XT + lane * 8;
            r[2 * h] = *reinterpret_cast<const h8*>(xp);
            r[2 * h + 1] = *reinterpret_cast<const h8*>(xp + 512);
        }
    };
    f32x16 dp[2];   // chain results of the previous stage (token tile 1 at a step's end)
    float dbp[2];
    bool pend = false;
    auto step = [&](auto o4, const _Float16* xs, const uint8_t* ws) {
        constexpr int O4 = decltype(o4)::value;
        float mn[2][2];  // dmin m of row tile j, block b (0 without a min term)
        h8 A[2][4];
        read_a(xs, 0, 0, A[0]);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            // the block's weight operands (both row tiles, both halves) and scales
            h8 B[2][2];
            float db[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint8_t* row = ws + (64 * wn + 32 * j + c) * WROW;
                uint32_t q[4];
                if (b == 0) {
                    codes<F, O4, 0>(row, g, q);
                    P::template ops<0>(q, g, B[j][0], B[j][1]);
                    scales<F, O4, 0>(row, db[j], mn[j][0]);
                } else {
                    codes<F, O4, 1>(row, g, q);
                    P::template ops<1>(q, g, B[j][0], B[j][1]);
                    scales<F, O4, 1>(row, db[j], mn[j][1]);
                }
                if constexpr (F == Q6_K) {
                    // sc1 = 0: the second sub-block's weights are zero
                    const h8 zero = {};
                    if (mn[j][b] == 1.0f && *(row + O4 + PB<F>::BB * b + 3) == 0) B[j][1] = zero;
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int st = 2 * b + i;  // stage within the step
                h8(&cur)[4] = A[st & 1];
                if (st < 3) read_a(xs, (st + 1) >> 1, (st + 1) & 1, A[(st + 1) & 1]);
                if constexpr (F == Q6_K) {
                    // one chain over both 16-element sub-blocks: the first
                    // sub-block's partial sums are scaled by r = sc0 / sc1
                    // before the second's MFMAs add to them, and the block
                    // folds with d sc1 (scales(): db = d sc1, mn = r); a zero
                    // sc1 zeroes the second sub-block's codes instead (r = 1,
                    // db = d sc0)
                    f32x16 d[2];
                    const f32x16 z = {};
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[0], B[j][0], z, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[1], B[j][0], d[j], 0, 0, 0);
                    // the previous stage's fold covers these MFMAs' latency
                    if (pend) {
#pragma unroll
                        for (int j = 0; j < 2; ++j)
#pragma unroll
                            for (int e = 0; e < 16; ++e)
                                acc[1 - i][j][e] = __builtin_fmaf(dbp[j], dp[j][e], acc[1 - i][j][e]);
                    }
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int e = 0; e < 16; ++e) d[j][e] *= mn[j][b];
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[2], B[j][1], d[j], 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[3], B[j][1], d[j], 0, 0, 0);
                    dp[0] = d[0];
                    dp[1] = d[1];
                    dbp[0] = db[0];
                    dbp[1] = db[1];
                    pend = true;
                } else {
                    f32x16 d[2];
                    const f32x16 z = {};
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[0], B[j][0], z, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[1], B[j][0], d[j], 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[2], B[j][1], d[j], 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        d[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[3], B[j][1], d[j], 0, 0, 0);
                    // fold the previous stage (token tile 1 - i)
                    if (pend) {
#pragma unroll
                        for (int j = 0; j < 2; ++j)
#pragma unroll
                            for (int e = 0; e < 16; ++e)
                                acc[1 - i][j][e] = __builtin_fmaf(dbp[j], dp[j][e], acc[1 - i][j][e]);
                    }
                    dp[0] = d[0];
                    dp[1] = d[1];
                    dbp[0] = db[0];
                    dbp[1] = db[1];
                    pend = true;
                }
            }
        }
        if constexpr (TL::MIN) {
            // acc -= S (token) x dmin m (row) over the step's two sub-blocks:
            // one v_mfma_f32_32x32x2_f32 per tile (K = the two sub-blocks),
            // A = lane (c, g): the scaled sum of token c over block g, B =
            // -dmin m of row c of the row tile for block g
            const float* sv = reinterpret_cast<const float*>(
                reinterpret_cast<const uint8_t*>(xs) + TL::XOPB);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float sa = sv[((2 * wm + i) * 2 + g) * 32 + c];
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        sa, -(g ? mn[j][1] : mn[j][0]), acc[i][j], 0, 0, 0);
            }
        }
    };
    if (s0 < s1) issue(s0);
    if (s0 + 1 < s1) issue(s0 + 1);
    // one step: this wave's copies of step s are done; the barrier makes
    // every wave's visible and ends every wave's reads of step s - 1, whose
    // buffers step s + 2 then refills
    auto run = [&](auto o4, int s) {
        wait_step(s + 1 < s1);
        __syncthreads();
        if (s + 2 < s1) issue(s + 2);
        const int buf = s % NBUF;
        step(o4, reinterpret_cast<const _Float16*>(xs0 + buf * TL::XBUF), ws0 + buf * TL::WBUF);
    };
    // a row's step s starts 4 (s mod 4) bytes into its LDS slot (68 and 36
    // are 4 mod 16; s0 is a multiple of 4), so four steps per iteration
    // give every read a constant offset
    for (int s = s0; s < s1; s += 4) {
        run(std::integral_constant<int, Chunks<F>::o4(0)>{}, s);
        if (s + 1 < s1) run(std::integral_constant<int, Chunks<F>::o4(1)>{}, s + 1);
        if (s + 2 < s1) run(std::integral_constant<int, Chunks<F>::o4(2)>{}, s + 2);
        if (s + 3 < s1) run(std::integral_constant<int, Chunks<F>::o4(3)>{}, s + 3);
    }
    if (pend) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[1][j][e] = __builtin_fmaf(dbp[j], dp[j][e], acc[1][j][e]);
    }
    // lane (c, g): column n = 32 j + c of its quadrant, rows 8 (e / 4) + 4 g + e % 4
    const bool split = gridDim.z > 1;
    float* out = split ? a.part + (size_t)blockIdx.z * a.M * a.N : a.y;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int ei[16];
#pragma unroll
        for (int e = 0; e < 16; ++e)
            ei[e] = a.ex[min(m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3), a.M - 1)];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + 64 * wn + 32 * j + c;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
                if (m < a.M && n < a.N) {
                    float v = __builtin_amdgcn_ldexpf(acc[i][j][e], ei[e]);
                    if (!split) {
                        if (a.bias_mode == 1) v += n < a.bias_len ? a.bias[n] : 0.0f;
                        else if (a.bias_mode == 2) v += a.bias[(size_t)m * a.N + n];
                    }
                    out[(size_t)m * a.N + n] = v;
                }
            }
        }
    }
}

// ------------------------------------------------------ Q6_K conversion
// GGUF Q6_K rows (210-byte super-blocks, matmul.cpp:242-279: element
// 128 h + 32 k + l of a super-block is nibble k / 2 of ql[64 h + 32 (k % 2)
// + l] with bits 2 k, 2 k + 1 of qh[32 h + l] on top, minus 32, scale
// sc[8 h + 2 k + l / 16]) -> 36-byte blocks of 32 elements (PB<Q6_K>): d,
// the block's two sub-block scales, the 32 codes 0..63, bytes 8 g .. 8 g + 7
// of each 16 holding elements 8 g .. of sub-block 0 then of sub-block 1 --
// in dwords of four codes, the element dwords 0, 1, 4, 5, 2, 3, 6, 7.
// One thread per half super-block (the four blocks k = 0..3 of half h share
// its 32 qh bytes and two 32-byte ql runs): six 16-byte loads from the
// 2-byte-aligned GGUF bytes (gfx950 serves unaligned loads) and the 144
// output bytes as nine 16-byte stores (a half super-block's output starts
// on a multiple of 144 bytes, rows being 288 bytes per super-block).
__global__ __launch_bounds__(256) void q6c_kernel(const uint8_t* __restrict__ w, int N, int K,
                                                  int64_t row_bytes, uint8_t* __restrict__ out) {
    const int nh = K / 128;  // half super-blocks per row
    const size_t total = (size_t)N * nh;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (size_t)gridDim.x * 256) {
        const int n = (int)(i / nh), u = (int)(i - (size_t)n * nh);
        const int h = u & 1;
        const uint8_t* sb = w + (size_t)n * row_bytes + (size_t)210 * (u >> 1);
        const uint8_t* qlp = sb + 64 * h;
        const uint8_t* qhp = sb + 128 + 32 * h;
        const uint4 l0 = ld_u128(qlp), l1 = ld_u128(qlp + 16), l2 = ld_u128(qlp + 32),
                    l3 = ld_u128(qlp + 48), h0 = ld_u128(qhp), h1 = ld_u128(qhp + 16);
        const uint32_t L[2][8] = {{l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w},
                                  {l2.x, l2.y, l2.z, l2.w, l3.x, l3.y, l3.z, l3.w}};
        const uint32_t H[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        const uint32_t s01 = ld_u32(sb + 192 + 8 * h), s23 = ld_u32(sb + 196 + 8 * h);
        const uint32_t d = ld_u16(sb + 208);
        uint32_t o[36];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t sc = k < 2 ? (s01 >> (16 * k)) & 0xFFFFu : (s23 >> (16 * (k - 2))) & 0xFFFFu;
            o[9 * k] = d | (sc << 16);
            constexpr int ED[8] = {0, 1, 4, 5, 2, 3, 6, 7};  // element dword of output dword p
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const int j = ED[p];
                const uint32_t nib = (L[k & 1][j] >> (4 * (k >> 1))) & 0x0F0F0F0Fu;
                const uint32_t hb = (H[j] >> (2 * k)) & 0x03030303u;
                o[9 * k + 1 + p] = nib | (hb << 4);
            }
        }
        uint4* dst = reinterpret_cast<uint4*>(out + i * 144);
#pragma unroll
        for (int p = 0; p < 9; ++p) dst[p] = make_uint4(o[4 * p], o[4 * p + 1], o[4 * p + 2], o[4 * p + 3]);
    }
}

}  // namespace

bool mmqp_supported(int dtype) {
    return dtype == Q8_0 || dtype == Q4_0 || dtype == Q4_1 || dtype == Q5_0 || dtype == Q5_1 ||
           dtype == Q4_K || dtype == Q6_K;
}

int64_t mmqp_q6c_bytes(int N, int K) { return (int64_t)N * (K / 32) * 36; }

hipError_t launch_q6c(const uint8_t* w, int N, int K, int64_t row_bytes, uint8_t* out,
                      hipStream_t st) {
    const size_t total = (size_t)N * (K / 128);
    const int grid = (int)std::min<size_t>((total + 255) / 256, 16384);
    hipLaunchKernelGGL(q6c_kernel, dim3(grid), dim3(256), 0, st, w, N, K, row_bytes, out);
    return hipGetLastError();
}
int mmqp_tile_rows() { return BNT; }
int mmqp_tile_tokens() { return BMT; }

hipError_t launch_xprep32(const float* x, int M, int K, _Float16* xop, int* ex, float* xsum,
                          bool sub16, hipStream_t st) {
    if (K % 256 != 0) return hipErrorInvalidValue;
    if (sub16)
        hipLaunchKernelGGL(xprep4_kernel<true>, dim3(8 * ((M + 31) / 32)), dim3(1024), 0, st, x, M,
                           K, ex, xop, xsum);
    else
        hipLaunchKernelGGL(xprep4_kernel<false>, dim3(8 * ((M + 31) / 32)), dim3(1024), 0, st, x,
                           M, K, ex, xop, xsum);
    return hipGetLastError();
}

hipError_t launch_mmqp(int dtype, const MmqArgs& a, int splits, hipStream_t st) {
    const int nsteps = a.K / KS;
    const int sps = ((nsteps + splits - 1) / splits + 3) & ~3;  // a multiple of 4 steps
    if ((long)sps * (splits - 1) >= nsteps) return hipErrorInvalidValue;
    const dim3 grid((a.N + BNT - 1) / BNT, (a.M + BMT - 1) / BMT, splits);
    if (dtype == Q8_0)
        hipLaunchKernelGGL(mmqp_kernel<Q8_0>, grid, dim3(64 * NW), 0, st, a, sps);
    else if (dtype == Q4_0)
        hipLaunchKernelGGL(mmqp_kernel<Q4_0>, grid, dim3(64 * NW), 0, st, a, sps);
    else if (dtype == Q4_1)
        hipLaunchKernelGGL(mmqp_kernel<Q4_1>, grid, dim3(64 * NW), 0, st, a, sps);
    else if (dtype == Q5_0)
        hipLaunchKernelGGL(mmqp_kernel<Q5_0>, grid, dim3(64 * NW), 0, st, a, sps);
    else if (dtype == Q5_1)
        hipLaunchKernelGGL(mmqp_kernel<Q5_1>, grid, dim3(64 * NW), 0, st, a, sps);
    else if (dtype == Q4_K)
        hipLaunchKernelGGL(mmqp_kernel<Q4_K>, grid, dim3(64 * NW), 0, st, a, sps);
    else if (dtype == Q6_K)
        hipLaunchKernelGGL(mmqp_kernel<Q6_K>, grid, dim3(64 * NW), 0, st, a, sps);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace fq
