// fq_mmqs.hip -- small-batch (M <= 16 tokens) matmul on the fp16 matrix
// cores, streaming the GGUF rows once: Q4_K (below), and Q4_0, Q4_1, Q5_0,
// Q5_1, Q5_K, IQ4_NL, Q8_0, Q6_K and Q3_K through their Band<> decoders
// further down.
//
// A work-group owns a band of rows, cut into TW tiles of 16; its waves split
// the K dimension by super-blocks (super-block s goes to wave s % W), so each
// wave walks its super-blocks over ALL the band's tiles and every weight byte
// is read once by one wave.  A super-block of a tile (16 rows x 144 bytes for
// Q4_K) is fetched with 16-byte loads along the rows into the wave's LDS
// panel (an MFMA operand gathers 16 rows per load instruction, which costs
// the texture addresser several times a row-contiguous load), and per
// 64-element chunk of it (tile, chunk) the wave issues
//
//   D_s = A_s (16 rows x 32) . B_s (32 x 16 tokens), s = the chunk's two
//         32-element sub-blocks, as v_mfma_f32_16x16x32_f16 twice per
//         sub-block: x_hi and x_lo accumulate into the same fp32 D_s;
//   A_s: exact fp16 quants (lane 16 q + r: row r, elements 8 q .. 8 q + 7 in
//        the slot order of fq_mfma16.h);
//   B_s: the token operands of xprep_kernel (fq_mmq.hip): x of the chunk
//        scaled by 2^-e (one exponent per token and chunk), split into fp16
//        hi + lo (22 significant bits), in the same slot order;
//
// and adds  2^e (A_0 D_0 + A_1 D_1 + B_0 S_0 + B_1 S_1)  to its accumulators,
// with (A_s, B_s) the sub-block's affine pair of the format (Q4_K: d sc and
// -dmin m, matmul.cpp:340-377) and S_s the scaled sub-block sums of x.  The
// token operands of a chunk are loaded once per wave (one chunk ahead) and
// reused by every tile of the band.
//
// The scale coefficients of a row come from its super-block header; D's lanes
// hold rows 4 q' .. 4 q' + 3 of token c, so the coefficients go through a
// small per-wave LDS table: once per super-block lane (r, q) decodes the four
// coefficients of pair q of row r, and per chunk lane (c, q') reads those of
// rows 4 q' .. +3.
//
// At the end every wave's accumulators go to LDS and the work-group adds the
// W partial sums of each output in wave order: deterministic, no atomics.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_mfma16.h"

namespace fq {
namespace {

constexpr int KC = 64;      // K elements per chunk (as xprep_kernel)
constexpr int XOP = 2048;   // halves per (token tile, chunk)
constexpr int XSUM = 64;    // sub-block sums per (token tile, chunk)

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int F>
struct Band;

// SB16: 16-element sub-blocks (four 16x16x16 MFMA sub-blocks per chunk);
// SHIFT: rows not 16-byte aligned (each row's super-block is loaded from its
// aligned-down start, and read back at its byte shift)
struct BandFlags {
    static constexpr bool SB16 = false, SHIFT = false;
};

// Q4_K: one super-block of 16 rows is a 16 x 144-byte panel.  It is loaded
// with 16-byte pieces (piece p of the panel: row p / 9, bytes 16 (p % 9) of
// the row's super-block: each row a contiguous 144-byte run) and written to
// the wave's LDS panel in the same order; the MFMA operands are then read
// from the panel.  Chunk g of the super-block = sub-block pair g: lane
// (r, q) takes qs bytes [32 g + 8 q, +8) of row r (low nibbles: sub-block
// 2 g, high nibbles: 2 g + 1); the row's header is the panel's first 16
// bytes.
template <>
struct Band<Q4_K> : BandFlags {
    // SBB bytes of a row per 256 elements; NPL 16-byte pieces per lane
    static constexpr int SBK = 256, SBB = 144, PANEL = 16 * SBB, PIECES = PANEL / 16, NPL = 3;
    static constexpr bool MIN = true;  // the -dmin m terms
    __device__ static void operands(const uint8_t* panel, int g, int r, int q, h8& a0, h8& a1) {
        const fq_u32x2 qs =
            *reinterpret_cast<const fq_u32x2*>(panel + 144 * r + 16 + 32 * g + 8 * q);
        a0 = nib8(qs.x, qs.y, 0, (_Float16)1024.0f);
        a1 = nib8(qs.x, qs.y, 4, (_Float16)1024.0f);
    }
    // the four coefficients of row r for pair g: d sc_2g, d sc_2g+1,
    // -dmin m_2g, -dmin m_2g+1
    __device__ static float4 coef4(const uint8_t* panel, int g, int r) {
        const fq_u32x4 h = *reinterpret_cast<const fq_u32x4*>(panel + 144 * r);
        uint32_t sa, ma, sb, mb;
        Fmt<Q4_K>::scale_min(uint4{h.x, h.y, h.z, h.w}, g, sa, ma, sb, mb);
        const float d = f16_hw(h.x & 0xFFFFu), dmin = f16_hw(h.x >> 16);
        return float4{d * (float)sa, d * (float)sb, -dmin * (float)ma, -dmin * (float)mb};
    }
};

// Q5_K: the Q4_K super-block with a 32-byte plane of fifth bits (d dmin
// scales[12] @0, qh[32] @16, qs[128] @48; 176 bytes, 16-byte aligned rows on
// the conditions of Q4_0).  Lane (r, q) of pair g takes qs bytes 32 g + 8 q
// .. + 7 (low nibbles: sub-block 2 g, high: 2 g + 1) and bits 2 g, 2 g + 1
// of qh bytes 8 q .. + 7 as the codes' fifth bits (0 .. 31, exact in fp16);
// the coefficients are those of Q4_K.
template <>
struct Band<Q5_K> : BandFlags {
    static constexpr int SBK = 256, SBB = 176, PANEL = 16 * SBB, PIECES = PANEL / 16, NPL = 3;
    static constexpr bool MIN = true;
    __device__ static void operands(const uint8_t* panel, int g, int r, int q, h8& a0, h8& a1) {
        const fq_u32x2 qs =
            *reinterpret_cast<const fq_u32x2*>(panel + SBB * r + 48 + 32 * g + 8 * q);
        const fq_u32x2 qh = *reinterpret_cast<const fq_u32x2*>(panel + SBB * r + 16 + 8 * q);
        auto code = [&](uint32_t w, uint32_t h, int sh, int bit) {
            return ((w >> sh) & 0x0F0F0F0Fu) | (((h >> bit) & 0x01010101u) << 4);
        };
        a0 = byte8(code(qs.x, qh.x, 0, 2 * g), code(qs.y, qh.y, 0, 2 * g), (_Float16)1024.0f);
        a1 = byte8(code(qs.x, qh.x, 4, 2 * g + 1), code(qs.y, qh.y, 4, 2 * g + 1),
                   (_Float16)1024.0f);
    }
    __device__ static float4 coef4(const uint8_t* panel, int g, int r) {
        const fq_u32x4 h = *reinterpret_cast<const fq_u32x4*>(panel + SBB * r);
        uint32_t sa, ma, sb, mb;
        Fmt<Q4_K>::scale_min(uint4{h.x, h.y, h.z, h.w}, g, sa, ma, sb, mb);
        const float d = f16_hw(h.x & 0xFFFFu), dmin = f16_hw(h.x >> 16);
        return float4{d * (float)sa, d * (float)sb, -dmin * (float)ma, -dmin * (float)mb};
    }
};

// Eight bytes of a panel at byte offset o, o = 2 (mod 4) when ODD2 (else a
// multiple of 4).
template <bool ODD2>
__device__ __forceinline__ fq_u32x2 pan_ld8(const uint8_t* panel, int o) {
    if constexpr (ODD2) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(panel + o - 2);
        return fq_u32x2{__builtin_amdgcn_alignbyte(w[1], w[0], 2),
                        __builtin_amdgcn_alignbyte(w[2], w[1], 2)};
    } else {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(panel + o);
        return fq_u32x2{w[0], w[1]};
    }
}

// Q4_0: eight 18-byte blocks (d | qs[16], element j the low nibble of qs[j],
// j + 16 the high one) make the same 144 bytes per 256 elements and row, so
// the panels and their loads are those of Q4_K (the host takes this kernel
// only for rows that start 16-byte aligned: K a multiple of 256 and an
// aligned base).  Chunk g = blocks 2 g and 2 g + 1: lane (r, q) takes
// elements 8 q .. 8 q + 7 of each, the low (q < 2) or high nibbles of qs
// bytes 8 (q & 1) .. + 7, as quant - 8; the coefficients are the blocks'
// scales d, and there is no minimum term.
template <>
struct Band<Q4_0> : BandFlags {
    static constexpr int SBK = 256, SBB = 144, PANEL = 16 * SBB, PIECES = PANEL / 16, NPL = 3;
    static constexpr bool MIN = false;
    __device__ static void operands(const uint8_t* panel, int g, int r, int q, h8& a0, h8& a1) {
        // block 2 g + s of row r starts at 144 r + 36 g + 18 s; its qs at + 2
        const int o = 144 * r + 36 * g + 2 + 8 * (q & 1), sh = q < 2 ? 0 : 4;
        const fq_u32x2 b0 = pan_ld8<true>(panel, o), b1 = pan_ld8<false>(panel, o + 18);
        a0 = nib8(b0.x, b0.y, sh, (_Float16)1032.0f);
        a1 = nib8(b1.x, b1.y, sh, (_Float16)1032.0f);
    }
    __device__ static float4 coef4(const uint8_t* panel, int g, int r) {
        const uint16_t* d = reinterpret_cast<const uint16_t*>(panel + 144 * r + 36 * g);
        return float4{f16_hw(d[0]), f16_hw(d[9]), 0.0f, 0.0f};
    }
};

// Q4_1: eight 20-byte blocks (d | m | qs[16], nibbles as Q4_0's, w = d q +
// m) are 160 bytes per 256 elements and row, ten pieces per panel row.  The
// operands are the nibbles as they stand (0 .. 15), the coefficients the
// blocks' d and, for the sub-block sums of x, m.
template <>
struct Band<Q4_1> : BandFlags {
    static constexpr int SBK = 256, SBB = 160, PANEL = 16 * SBB, PIECES = PANEL / 16, NPL = 3;
    static constexpr bool MIN = true;
    __device__ static void operands(const uint8_t* panel, int g, int r, int q, h8& a0, h8& a1) {
        // block 2 g + s of row r starts at 160 r + 40 g + 20 s; its qs at + 4
        const int o = SBB * r + 40 * g + 4 + 8 * (q & 1), sh = q < 2 ? 0 : 4;
        const fq_u32x2 b0 = pan_ld8<false>(panel, o), b1 = pan_ld8<false>(panel, o + 20);
        a0 = nib8(b0.x, b0.y, sh, (_Float16)1024.0f);
        a1 = nib8(b1.x, b1.y, sh, (_Float16)1024.0f);
    }
    __device__ static float4 coef4(const uint8_t* panel, int g, int r) {
        const uint32_t* h = reinterpret_cast<const uint32_t*>(panel + SBB * r + 40 * g);
        const uint32_t h0 = h[0], h1 = h[5];  // d | m of the two blocks
        return float4{f16_hw(h0 & 0xFFFFu), f16_hw(h1 & 0xFFFFu), f16_hw(h0 >> 16),
                      f16_hw(h1 >> 16)};
    }
};

// Q8_0: eight 34-byte blocks (d | qs[32] int8) are 272 bytes per 256
// elements and row (16-byte aligned on the same conditions as Q4_0), a
// 16 x 272-byte panel of 17 pieces per row.  Chunk g = blocks 2 g and 2 g + 1:
// lane (r, q) takes their qs bytes 8 q .. 8 q + 7 as fp16 (the sign bit
// flipped and 1152 subtracted: exact); the coefficients are the scales d.
template <>
struct Band<Q8_0> : BandFlags {
    static constexpr int SBK = 256, SBB = 272, PANEL = 16 * SBB, PIECES = PANEL / 16, NPL = 5;
    static constexpr bool MIN = false;
    __device__ static void operands(const uint8_t* panel, int g, int r, int q, h8& a0, h8& a1) {
        // block 2 g + s of row r starts at 272 r + 68 g + 34 s; its qs at + 2
        const int o = SBB * r + 68 * g + 2 + 8 * q;
        const fq_u32x2 b0 = pan_ld8<true>(panel, o), b1 = pan_ld8<false>(panel, o + 34);
        a0 = byte8(b0.x ^ 0x80808080u, b0.y ^ 0x80808080u, (_Float16)1152.0f);
        a1 = byte8(b1.x ^ 0x80808080u, b1.y ^ 0x80808080u, (_Float16)1152.0f);
    }
    __device__ static float4 coef4(const uint8_t* panel, int g, int r) {
        const uint16_t* d = reinterpret_cast<const uint16_t*>(panel + SBB * r + 68 * g);
        return float4{f16_hw(d[0]), f16_hw(d[17]), 0.0f, 0.0f};
    }
};

// A dword of the panel at byte offset o, o even.
__device__ __forceinline__ uint32_t pan_ld4(const uint8_t* panel, int o) {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(panel + (o & ~3));
    return __builtin_amdgcn_alignbyte(w[1], w[0], o & 3);
}

// Q6_K: 210-byte super-blocks (ql[128] | qh[64] | scales[16] int8 | d),
// rows only 2-byte aligned.  A row's super-block is loaded as the 14 aligned
// 16-byte pieces from its aligned-down start (224 bytes: the start's shift
// is even and at most 14), so a panel row holds it at that shift; the last
// piece ends inside the aligned block of the row's last byte.  Element e of
// the super-block, n = e / 128, l = e % 32, quarter u = (e % 128) / 32: the
// low (u < 2) or high nibble of ql[64 n + 32 (u & 1) + l] and bits 2 u .. 2 u
// + 1 of qh[32 n + l], weight d sc[e / 16] (q - 32).  Chunk g (64 elements)
// = n = g / 2, quarters 2 (g & 1) and 2 (g & 1) + 1: sub-block s (16
// elements) takes quarter 2 (g & 1) + s / 2, l = 16 (s & 1) + 4 q + 0 .. 3
// for lane (r, q), as q - 32 in fp16 (1024 + q - 1056: exact).
template <>
struct Band<Q6_K> {
    static constexpr bool SB16 = true, SHIFT = true, MIN = false;
    static constexpr int SBK = 256, SBB = 210, PANEL = 16 * 224, PIECES = PANEL / 16, NPL = 4;
    // ro: the row's byte offset in the panel (224 r + its shift)
    __device__ static void operands(const uint8_t* panel, int ro, int g, int q, h4 (&a)[4]) {
        const int n = g >> 1, hn = g & 1;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const uint32_t qh = pan_ld4(panel, ro + 128 + 32 * n + 16 * hf + 4 * q);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t ql = pan_ld4(panel, ro + 64 * n + 32 * j + 16 * hf + 4 * q);
                const uint32_t v = ((ql >> (4 * hn)) & 0x0F0F0F0Fu) |
                                   (((qh >> (2 * (2 * hn + j))) & 0x03030303u) << 4);
                h2 p0, p1;
                byte_pairs(v, (_Float16)1056.0f, p0, p1);
                a[2 * j + hf] = h4{p0[0], p0[1], p1[0], p1[1]};
            }
        }
    }
    // d sc of the chunk's four sub-blocks
    __device__ static float4 coef4(const uint8_t* panel, int ro, int g) {
        const uint32_t sc = pan_ld4(panel, ro + 192 + 4 * g);
        const float d = f16_hw(pan_ld4(panel, ro + 208) & 0xFFFFu);
        return float4{d * (float)(int8_t)(sc & 0xFF), d * (float)(int8_t)((sc >> 8) & 0xFF),
                      d * (float)(int8_t)((sc >> 16) & 0xFF), d * (float)(int8_t)(sc >> 24)};
    }
};

// Q5_0 (22-byte blocks: d | qh u32 | qs[16]), Q5_1 (24: d m | qh | qs) and
// IQ4_NL (18: d | qs, a 16-entry int8 table): eight blocks are 176 / 192 /
// 144 bytes per 256 elements and row (16-byte aligned on the conditions of
// Q4_0).  Lane (r, q) takes elements 8 q .. 8 q + 7 of blocks 2 g and 2 g + 1:
// the low (q < 2) or high nibbles of qs bytes 8 (q & 1) .. + 7 with, for the
// 5-bit formats, bits 8 q .. 8 q + 7 of qh as the fifth bits; Q5_0 enters as
// q - 16, Q5_1 as q with m on the sub-block sums, IQ4_NL as its table value.
template <int F>
struct BandSmall : BandFlags {
    static constexpr int BB = F == Q5_0 ? 22 : F == Q5_1 ? 24 : 18;
    static constexpr int SBK = 256, SBB = 8 * BB, PANEL = 16 * SBB, PIECES = PANEL / 16, NPL = 3;
    static constexpr bool MIN = F == Q5_1;
    static constexpr int QS = F == Q5_0 ? 6 : F == Q5_1 ? 8 : 2, QH = F == Q5_1 ? 4 : 2;
    // the block's eight codes as an h8 (o: the block's offset in the panel)
    template <int OFF>
    __device__ static h8 block(const uint8_t* panel, int o, int q) {
        const int oq = o + QS + 8 * (q & 1), sh = q < 2 ? 0 : 4;
        const fq_u32x2 b = (OFF + QS) % 4 == 2 ? pan_ld8<true>(panel, oq) : pan_ld8<false>(panel, oq);
        uint32_t w0 = (b.x >> sh) & 0x0F0F0F0Fu, w1 = (b.y >> sh) & 0x0F0F0F0Fu;
        if constexpr (F == IQ4_NL) {
            return byte8(iq4_lookup(w0) ^ 0x80808080u, iq4_lookup(w1) ^ 0x80808080u,
                         (_Float16)1152.0f);
        } else {
            const uint32_t qh = pan_ld4(panel, o + QH) >> (8 * q);
            return byte8(five_bit(w0, qh), five_bit(w1, qh >> 4),
                         (_Float16)(F == Q5_0 ? 1040.0f : 1024.0f));
        }
    }
    __device__ static void operands(const uint8_t* panel, int g, int r, int q, h8& a0, h8& a1) {
        const int o = SBB * r + 2 * BB * g;  // block 2 g (SBB r and 2 BB g are multiples of 4)
        a0 = block<0>(panel, o, q);
        a1 = block<BB>(panel, o + BB, q);
    }
    __device__ static float4 coef4(const uint8_t* panel, int g, int r) {
        const int o = SBB * r + 2 * BB * g;
        const uint32_t h0 = pan_ld4(panel, o), h1 = pan_ld4(panel, o + BB);
        return float4{f16_hw(h0 & 0xFFFFu), f16_hw(h1 & 0xFFFFu),
                      MIN ? f16_hw(h0 >> 16) : 0.0f, MIN ? f16_hw(h1 >> 16) : 0.0f};
    }
};
template <>
struct Band<Q5_0> : BandSmall<Q5_0> {};
template <>
struct Band<Q5_1> : BandSmall<Q5_1> {};
template <>
struct Band<IQ4_NL> : BandSmall<IQ4_NL> {};

// Q3_K: 110-byte super-blocks (hmask[32] | qs[64] | scales[12] | d), rows
// 2-byte aligned: loaded from the aligned-down start like Q6_K, at most
// eight pieces (a panel row of 128 bytes; only pieces that start before the
// row's end are loaded).  Element e, n = e / 128, plane j = (e % 128) / 32,
// l = e % 32: bits 2 j .. 2 j + 1 of qs[32 n + l] and bit 4 n + j of
// hmask[l] make the code c = q2 + 4 h, weight d (sc[e / 16] - 32) (c - 4).
// Chunk g: n = g / 2, sub-block s takes plane 2 (g & 1) + s / 2 and l = 16
// (s & 1) + 4 q + 0 .. 3 for lane (r, q), as c - 4 (1024 + c - 1028).
// Sub-block scale i (6 bits): the low four in nibble i / 8 of scales[i % 8],
// the top two at bit 2 (i / 4) of scales[8 + i % 4].
template <>
struct Band<Q3_K> {
    static constexpr bool SB16 = true, SHIFT = true, MIN = false;
    static constexpr int SBK = 256, SBB = 110, PANEL = 16 * 128, PIECES = PANEL / 16, NPL = 2;
    __device__ static void operands(const uint8_t* panel, int ro, int g, int q, h4 (&a)[4]) {
        const int n = g >> 1, jb = 2 * (g & 1);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const uint32_t hm = pan_ld4(panel, ro + 16 * hf + 4 * q);
            const uint32_t qs = pan_ld4(panel, ro + 32 + 32 * n + 16 * hf + 4 * q);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = jb + jj;
                const uint32_t v = ((qs >> (2 * j)) & 0x03030303u) |
                                   (((hm >> (4 * n + j)) & 0x01010101u) << 2);
                h2 p0, p1;
                byte_pairs(v, (_Float16)1028.0f, p0, p1);
                a[2 * jj + hf] = h4{p0[0], p0[1], p1[0], p1[1]};
            }
        }
    }
    // d (sc - 32) of the chunk's four sub-blocks i = 4 g .. 4 g + 3
    __device__ static float4 coef4(const uint8_t* panel, int ro, int g) {
        const uint32_t lo = pan_ld4(panel, ro + 96 + 4 * (g & 1));  // scales[i % 8], 4 of them
        const uint32_t hi = pan_ld4(panel, ro + 104);               // scales[8 .. 11]
        const float d = f16_hw(pan_ld4(panel, ro + 108) & 0xFFFFu);
        float c[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int i = 4 * g + s;
            const uint32_t l4 = (lo >> (8 * s + 4 * (i >> 3))) & 15u;
            const uint32_t h2b = (hi >> (8 * (i & 3) + 2 * (i >> 2))) & 3u;
            c[s] = d * (float)((int)(l4 | (h2b << 4)) - 32);
        }
        return float4{c[0], c[1], c[2], c[3]};
    }
};

template <int F, int TW, int WG, bool BIAS>
__global__ __launch_bounds__(WG) void mmqs_kernel(MmqArgs a, int rows_per_wg, int sb_per_split) {
    using B = Band<F>;
    constexpr int W = WG / 64;
    // per wave: TW panels (one super-block of 16 rows each) and TW tiles x 4
    // coefficients x 16 rows; then the partial sums
    __shared__ __attribute__((aligned(16))) uint8_t panels[W][TW][B::PANEL];
    // per wave and tile: coefficient v of pair g, row r at coef[..][g][v][r]
    __shared__ __attribute__((aligned(16))) float coef[W][TW][4][4][16];
    __shared__ float part[W][TW][16][16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;  // A operand: row r, element group q
    const int c = lane & 15;                 // D and B operands: token column c
    const int lo = blockIdx.x * rows_per_wg;
    const int hi = min(a.N, lo + rows_per_wg);
    const int ntl = (hi - lo + 15) >> 4;
    // this work-group's super-blocks: all of K, or split blockIdx.y of a K
    // split whose partial sums go to slab blockIdx.y of a.part
    const int sb0 = blockIdx.y * sb_per_split;
    const int nsb = min(a.K / B::SBK, sb0 + sb_per_split);

    // piece p of a tile's panel (rows clamped into the matrix)
    const uint8_t* prow[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) prow[t] = a.w + (size_t)min(lo + 16 * t, a.N - 1) * a.row_bytes;
    // pieces per lane, per panel row
    constexpr int NPL = B::NPL, PPR = B::PANEL / 256;
    int pp[NPL], rmax[TW];
#pragma unroll
    for (int i = 0; i < NPL; ++i) pp[i] = min(lane + 64 * i, B::PIECES - 1);
#pragma unroll
    for (int t = 0; t < TW; ++t) rmax[t] = a.N - 1 - min(lo + 16 * t, a.N - 1);

    f32x4 acc[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const fq_u32x4* xop = reinterpret_cast<const fq_u32x4*>(a.xop);
    auto load_panels = [&](int sb, fq_u32x4 (&pv)[TW][NPL]) {
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int i = 0; i < NPL; ++i) {
                const int rr = min(pp[i] / PPR, rmax[t]);  // rows past N repeat the last
                const uint8_t* rs = prow[t] + (size_t)rr * a.row_bytes + B::SBB * sb;
                const int pj = pp[i] - PPR * (pp[i] / PPR);  // piece of the panel row
                if constexpr (B::SHIFT) {
                    // from the aligned-down start; pieces wholly past the
                    // row's end are not loaded (they could leave its page)
                    const int sh = (int)(reinterpret_cast<uintptr_t>(rs) & 15);
                    rs -= sh;
                    pv[t][i] = fq_u32x4{0u, 0u, 0u, 0u};
                    if (16 * pj < sh + B::SBB)
                        pv[t][i] = __builtin_nontemporal_load(
                            reinterpret_cast<const fq_u32x4*>(rs + 16 * pj));
                } else {
                    pv[t][i] = __builtin_nontemporal_load(
                        reinterpret_cast<const fq_u32x4*>(rs + 16 * pj));
                }
            }
    };

    // SB = 32: x_hi, x_lo of sub-block 0, then of 1, eight halves per lane;
    // SB = 16: four sub-blocks' x_hi, x_lo, four halves per lane (as the
    // halves of one 16-byte load: lane 16 g + c of each 256-half block)
    auto load_x = [&](int ch, fq_u32x4 (&xv)[4]) {
        if constexpr (B::SB16) {
            const fq_u32x2* x2 = reinterpret_cast<const fq_u32x2*>(a.xop);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const fq_u32x2 h = x2[(size_t)ch * (XOP / 4) + 128 * i + lane];
                const fq_u32x2 l = x2[(size_t)ch * (XOP / 4) + 128 * i + 64 + lane];
                xv[i] = fq_u32x4{h.x, h.y, l.x, l.y};
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[i] = xop[(size_t)ch * (XOP / 8) + 64 * i + lane];
        }
    };

    // exponent and the two sub-block sums of token c in chunk ch
    struct Xs {
        int e;
        float S0, S1;
    };
    auto load_s = [&](int ch) {
        return Xs{a.ex[(size_t)ch * 16 + c], a.xsum[(size_t)ch * XSUM + c],
                  a.xsum[(size_t)ch * XSUM + 16 + c]};
    };

    // Token operands are prefetched one chunk ahead, the next super-block's
    // panels two chunks ahead (below).  (Loading all four chunks of the next
    // super-block ahead of its panel loads needs about 250 VGPRs and
    // measured slower.)
    int sb = sb0 + wave;
    fq_u32x4 pv[TW][NPL];
    fq_u32x4 xv[4];  // the token operands of the chunk computed next
    Xs xs{0, 0.0f, 0.0f};
    if (sb < nsb) {
        load_x(4 * sb, xv);
        xs = load_s(4 * sb);
        load_panels(sb, pv);
    }
    while (sb < nsb) {  // wave-uniform
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
            for (int i = 0; i < NPL; ++i)
                if (lane + 64 * i < B::PIECES)
                    *reinterpret_cast<fq_u32x4*>(&panels[wave][t][16 * (lane + 64 * i)]) = pv[t][i];
        const int nx = sb + W;
        // the super-block's coefficients: lane (r, q) decodes pair q of row r
        // (the wave's own LDS writes precede its reads: in order)
        // (every tile of the band, also those past its last row: their
        // panels repeat the matrix's last row and their sums are never
        // written, and a branch per tile would keep the tiles' LDS reads,
        // MFMAs and FMAs from overlapping)
        // SHIFT: the byte offset of lane row r's super-block in its panel
        int ro[TW];
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            ro[t] = 0;
            if constexpr (B::SHIFT)
                ro[t] = (int)(reinterpret_cast<uintptr_t>(prow[t] + (size_t)min(r, rmax[t]) *
                                                                        a.row_bytes +
                                                          B::SBB * sb) &
                              15) +
                        (B::PANEL / 16) * r;
        }
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            float4 cv;
            if constexpr (B::SB16) cv = B::coef4(panels[wave][t], ro[t], q);
            else cv = B::coef4(panels[wave][t], q, r);
            coef[wave][t][q][0][r] = cv.x;
            coef[wave][t][q][1][r] = cv.y;
            coef[wave][t][q][2][r] = cv.z;
            coef[wave][t][q][3][r] = cv.w;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int ch = 4 * sb + g;
            // the following chunk's token operands (the next super-block's
            // first after the last), in flight while this chunk computes
            fq_u32x4 xn[4];
            const int cn = g < 3 ? ch + 1 : 4 * min(nx, nsb - 1);
            load_x(cn, xn);
            const Xs xsn = load_s(cn);
            // the next super-block's weight panels (clamped), two chunks
            // ahead of their use and behind the last token loads this
            // super-block waits for, so that no chunk's token operands queue
            // behind them in the in-order vector memory counter
            if (g == 2) load_panels(min(nx, nsb - 1), pv);
            const float S0 = xs.S0, S1 = xs.S1;
            const float p2 = __builtin_amdgcn_ldexpf(1.0f, xs.e);
            if constexpr (B::SB16) {
                // sub-block u: x_hi in the first two dwords of xv[u], x_lo in
                // the last two
                h4 xh[4], xl[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    xh[u] = __builtin_bit_cast(h4, fq_u32x2{xv[u].x, xv[u].y});
                    xl[u] = __builtin_bit_cast(h4, fq_u32x2{xv[u].z, xv[u].w});
                }
#pragma unroll
                for (int t = 0; t < TW; ++t) {
                    h4 av[4];
                    B::operands(panels[wave][t], ro[t], g, q, av);
                    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                    f32x4 d[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        d[u] = __builtin_amdgcn_mfma_f32_16x16x16f16(av[u], xh[u], z, 0, 0, 0);
                        d[u] = __builtin_amdgcn_mfma_f32_16x16x16f16(av[u], xl[u], d[u], 0, 0, 0);
                    }
                    float cf[4][4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float4 C =
                            *reinterpret_cast<const float4*>(&coef[wave][t][g][u][4 * q]);
                        cf[u][0] = C.x;
                        cf[u][1] = C.y;
                        cf[u][2] = C.z;
                        cf[u][3] = C.w;
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float sm = cf[0][i] * d[0][i];
                        sm = __builtin_fmaf(cf[1][i], d[1][i], sm);
                        sm = __builtin_fmaf(cf[2][i], d[2][i], sm);
                        sm = __builtin_fmaf(cf[3][i], d[3][i], sm);
                        acc[t][i] = __builtin_fmaf(sm, p2, acc[t][i]);
                    }
                }
            } else {
            const h8 xh0 = __builtin_bit_cast(h8, xv[0]), xl0 = __builtin_bit_cast(h8, xv[1]);
            const h8 xh1 = __builtin_bit_cast(h8, xv[2]), xl1 = __builtin_bit_cast(h8, xv[3]);
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                h8 a0, a1;
                B::operands(panels[wave][t], g, r, q, a0, a1);
                const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                f32x4 d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, xh0, z, 0, 0, 0);
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, xl0, d0, 0, 0, 0);
                f32x4 d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, xh1, z, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, xl1, d1, 0, 0, 0);
                const float4 A0 = *reinterpret_cast<const float4*>(&coef[wave][t][g][0][4 * q]);
                const float4 A1 = *reinterpret_cast<const float4*>(&coef[wave][t][g][1][4 * q]);
                const float4 B0 = *reinterpret_cast<const float4*>(&coef[wave][t][g][2][4 * q]);
                const float4 B1 = *reinterpret_cast<const float4*>(&coef[wave][t][g][3][4 * q]);
                const float a0v[4] = {A0.x, A0.y, A0.z, A0.w};
                const float a1v[4] = {A1.x, A1.y, A1.z, A1.w};
                const float b0v[4] = {B0.x, B0.y, B0.z, B0.w};
                const float b1v[4] = {B1.x, B1.y, B1.z, B1.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float s = a0v[i] * d0[i];
                    s = __builtin_fmaf(a1v[i], d1[i], s);
                    if constexpr (B::MIN) {
                        s = __builtin_fmaf(b0v[i], S0, s);
                        s = __builtin_fmaf(b1v[i], S1, s);
                    }
                    acc[t][i] = __builtin_fmaf(s, p2, acc[t][i]);
                }
            }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[i] = xn[i];
            xs = xsn;
        }
        sb = nx;
    }
    // partial sums: D lane (c, q) holds rows 4 q + i of token c
#pragma unroll
    for (int t = 0; t < TW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][t][4 * q + i][c] = acc[t][i];
    __syncthreads();
    const bool split = gridDim.y > 1;
    float* const out = split ? a.part + (size_t)blockIdx.y * a.M * a.N : a.y;
    for (int o = threadIdx.x; o < ntl * 256; o += WG) {
        const int t = o >> 8, rr = (o >> 4) & 15, m = o & 15;
        const int row = lo + 16 * t + rr;
        if (m >= a.M || row >= hi) continue;
        float v = part[0][t][rr][m];
        for (int w = 1; w < W; ++w) v += part[w][t][rr][m];
        if constexpr (BIAS) {
            if (!split) {
                if (a.bias_mode == 2) v += a.bias[(size_t)m * a.N + row];
                else v += row < a.bias_len ? a.bias[row] : 0.0f;
            }
        }
        out[(size_t)m * a.N + row] = v;
    }
}

template <int F, int TW, int WG>
const void* sfn(bool bias) {
    return bias ? reinterpret_cast<const void*>(&mmqs_kernel<F, TW, WG, true>)
                : reinterpret_cast<const void*>(&mmqs_kernel<F, TW, WG, false>);
}

template <int F, int WG>
const void* sfn_tw(int tw, bool bias) {
    switch (tw) {
        case 1: return sfn<F, 1, WG>(bias);
        case 2: return sfn<F, 2, WG>(bias);
    }
    // Q8_0, Q6_K: two tiles (LDS); Q3_K: two (four spill)
    if constexpr (WG <= 512 && F == Q8_0) {
        if (tw == 3) return sfn<F, 3, WG>(bias);
    }
    if constexpr (WG <= 512 && F != Q8_0 && F != Q6_K && F != Q3_K) {
        switch (tw) {
            case 3: return sfn<F, 3, WG>(bias);
            case 4: return sfn<F, 4, WG>(bias);
        }
    }
    return nullptr;
}

}  // namespace

bool mmqs_supported(int dtype) {
    return dtype == Q4_K || dtype == Q4_0 || dtype == Q4_1 || dtype == Q8_0 || dtype == Q6_K ||
           dtype == Q5_K || dtype == Q5_0 || dtype == Q5_1 || dtype == IQ4_NL || dtype == Q3_K;
}

// Tiles per work-group the kernel is instantiated for (bands of up to 16 TW
// rows): Q8_0's 272-byte panels fit three per wave in LDS at 512 threads
// (the host takes two or three);
// Q6_K and Q3_K take two (their 16-element sub-blocks need twice the
// operand registers per tile).
int mmqs_max_tiles(int dtype) { return dtype == Q8_0 ? 3 : dtype == Q6_K || dtype == Q3_K ? 2 : 4; }

hipError_t launch_mmqs(int dtype, const MmqArgs& a, int rows_per_wg, int wg, int splits,
                       hipStream_t st) {
    const int tw = (rows_per_wg + 15) / 16;
    const void* fn = nullptr;
    if (dtype == Q4_K) {
        fn = wg == 256   ? sfn_tw<Q4_K, 256>(tw, a.bias_mode != 0)
             : wg == 1024 ? sfn_tw<Q4_K, 1024>(tw, a.bias_mode != 0)
                          : sfn_tw<Q4_K, 512>(tw, a.bias_mode != 0);
    } else if (dtype == Q4_0 || dtype == Q4_1 || dtype == Q8_0 || dtype == Q5_K ||
               dtype == Q5_0 || dtype == Q5_1 || dtype == IQ4_NL) {
        // rows must start 16-byte aligned (the panel loads are 16 bytes)
        if (a.K % 256 != 0 || a.row_bytes % 16 != 0 ||
            (reinterpret_cast<uintptr_t>(a.w) & 15) != 0 || wg != 512)
            return hipErrorInvalidValue;
        fn = dtype == Q4_0   ? sfn_tw<Q4_0, 512>(tw, a.bias_mode != 0)
             : dtype == Q4_1 ? sfn_tw<Q4_1, 512>(tw, a.bias_mode != 0)
             : dtype == Q5_K ? sfn_tw<Q5_K, 512>(tw, a.bias_mode != 0)
             : dtype == Q5_0 ? sfn_tw<Q5_0, 512>(tw, a.bias_mode != 0)
             : dtype == Q5_1 ? sfn_tw<Q5_1, 512>(tw, a.bias_mode != 0)
             : dtype == IQ4_NL ? sfn_tw<IQ4_NL, 512>(tw, a.bias_mode != 0)
                             : sfn_tw<Q8_0, 512>(tw, a.bias_mode != 0);
    } else if (dtype == Q6_K || dtype == Q3_K) {  // rows at even addresses (shifts <= 14)
        if (a.K % 256 != 0 || (reinterpret_cast<uintptr_t>(a.w) & 1) != 0 || wg != 512)
            return hipErrorInvalidValue;
        fn = dtype == Q6_K ? sfn_tw<Q6_K, 512>(tw, a.bias_mode != 0)
                           : sfn_tw<Q3_K, 512>(tw, a.bias_mode != 0);
    }
    if (!fn) return hipErrorInvalidValue;
    const int nsb = a.K / 256;
    if (splits < 1 || splits > nsb || (splits > 1 && !a.part)) return hipErrorInvalidValue;
    int sps = (nsb + splits - 1) / splits;
    splits = (nsb + sps - 1) / sps;  // no empty split
    const int grid = (a.N + rows_per_wg - 1) / rows_per_wg;
    MmqArgs args = a;
    int rpw = rows_per_wg;
    void* params[] = {&args, &rpw, &sps};
    const hipError_t e = hipLaunchKernel(fn, dim3(grid, splits), dim3(wg), params, 0, st);
    if (e != hipSuccess || splits == 1) return e;
    return launch_reduce(a, splits, st);
}

}  // namespace fq
