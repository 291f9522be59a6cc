// fq_pack.h -- the aligned device layout ("packed") of the five block formats.
//
// GGUF rows are arrays of 18/20/34/144/210-byte blocks, so most blocks sit at
// 2-byte alignment.  The packed layout holds exactly the same bytes per row,
// rearranged into "planes" (the table below, in 16-byte pieces; the per-block
// scales form small dense arrays after the quant planes).  A row takes
// packed_row_bytes(K) bytes, a multiple of 16, and K must be a multiple of
// 256.  N rows take N packed_row_bytes(K) bytes, arranged one of two ways
// (packed_tiled() decides from the format and N; fq_pack_weights and the
// GEMVs apply the same rule):
//  - row-major: row n at n packed_row_bytes(K), its pieces in plane order;
//    a batch-1 lane reads piece v of a row, so a wave's load moves 1 KiB of
//    one row (fq_gemvp.hip);
//  - 16-row tiles (Q8_0 with at least TILED_MIN_ROWS rows):
//    tile t starts at byte 16 t packed_row_bytes(K), and within a tile of R
//    rows (the last tile holds the N mod 16 remaining rows) piece J of row r
//    sits at (J R + r) 16.  Pieces J .. J+3 of the tile's rows are one
//    contiguous 1 KiB run, read by a wave whose 64 lanes work on 16 rows
//    times four pieces (fq_gemvt.hip).
// Dequantizing packed bytes gives exactly the values of the original blocks
// (the bytes are only moved).
//
// The per-row plane table (byte offsets within a row's pieces):
//
//   Q4_0  [qs: U x 16][d: U x 2, padded to 16]                  U = K/32
//   Q4_1  [qs: U x 16][d,m: U x 4]
//   Q8_0  [qs[0,16): U x 16][qs[16,32): U x 16][d: U x 2, padded to 16]
//   Q4_K  [q0: V x 16][q1: V x 16][hdr: S x 16]        V = K/64, S = K/256
//         unit v = 4s + g: q0 = qs[32g, +16), q1 = qs[32g + 16, +16) of
//         super-block s; hdr = d | dmin | scales[12]
//   Q6_K  [lo: V x 16][hi: V x 16][qh: V x 16][sc: S x 16][d: S x 2, pad 16]
//         unit v = 4s + p, p = 2n + h (n = 128-half, h = which 16 of its 32
//         columns): lo = ql[64n + 16h, +16), hi = ql[64n + 32 + 16h, +16),
//         qh = qh[32n + 16h, +16) of super-block s
#pragma once

#include <stdint.h>

namespace fq {

__host__ __device__ inline int64_t pad16(int64_t b) { return (b + 15) & ~(int64_t)15; }

// The tiled arrangement: the one-row-per-lane kernel (fq_gemvt.hip) against
// the one-row-per-step kernel (fq_gemvp.hip), 152064 x 3584, M = 1: Q8_0 87.5
// against 97.5 us.  The 4-bit formats, dotted nibble-in-place on the latter,
// do better row-major (Q4_0 49.6 against 53.3 us, Q4_1 54.8 / 55.4, 65536 x
// 4096 Q4_0 25.5 / 28.8); the superblock formats do not gain (Q4_K 55.2 /
// 55.0, Q6_K 77.4 / 69.1), nor do matrices of fewer rows.
constexpr int64_t TILED_MIN_ROWS = 65536;
__host__ __device__ inline bool packed_tiled(int dtype, int64_t N) {
    return dtype == 7 && N >= TILED_MIN_ROWS;
}

// Packed row stride in bytes (0 when the format has no packed form).
__host__ __device__ inline int64_t packed_row_bytes(int dtype, int64_t K) {
    const int64_t U = K / 32, S = K / 256;
    switch (dtype) {
        case 2: return U * 16 + pad16(U * 2);              // Q4_0
        case 3: return U * 16 + pad16(U * 4);              // Q4_1
        case 7: return U * 32 + pad16(U * 2);              // Q8_0
        case 4: return S * 144;                            // Q4_K
        case 13: return S * 192 + S * 16 + pad16(S * 2);   // Q6_K
        default: return 0;
    }
}

}  // namespace fq
