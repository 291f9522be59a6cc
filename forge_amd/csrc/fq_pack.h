// fq_pack.h -- the aligned device layout ("packed") of the five block formats.
//
// GGUF rows are arrays of 18/20/34/144/210-byte blocks, so most blocks sit at
// 2-byte alignment.  The packed layout holds exactly the same bytes per row,
// rearranged into "planes": the 16-byte pieces a GEMV lane reads for lane
// unit v sit at plane + 16 v, so one load instruction of a wave reads 1 KiB
// of contiguous bytes, and the per-block scales form small dense arrays after
// the planes.  Rows stay contiguous; the row stride is packed_row_bytes(K), a
// multiple of 16, and K must be a multiple of 256.  Dequantizing packed bytes
// gives exactly the values of the original blocks (the bytes are only moved).
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
