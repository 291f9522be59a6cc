// fq_mfma16.h -- fp16 MFMA operand helpers shared by the M > 1 kernels.
//
// Quants become fp16 two at a time: a byte pair (b0, b2) of a dword masked
// into the low bits of 0x6400'6400 reads as the halves 1024 + b0, 1024 + b2,
// and one packed fp16 subtract removes 1024 (plus the format's offset), all
// exact.  Slot e of a lane's group of eight quants therefore holds element
// slot_elem(e) = {0, 2, 1, 3} within each quad; the token operands are
// written in the same order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Slot e of a lane's elements holds element slot_elem(e) of its group: the
// order in which the weight decode below produces fp16 quants.
__device__ __forceinline__ int slot_elem(int e) {
    return (e & ~3) | ((e & 1) << 1) | ((e >> 1) & 1);
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Two fp16 pairs from the bytes of w selected by mask, offset: value - off.
__device__ __forceinline__ void byte_pairs(uint32_t w, uint32_t mask, _Float16 off, h2& p0, h2& p1) {
    const uint32_t a = (w & mask) | 0x64006400u, b = ((w >> 8) & mask) | 0x64006400u;
    const h2 o = {off, off};
    p0 = __builtin_bit_cast(h2, a) - o;
    p1 = __builtin_bit_cast(h2, b) - o;
}

// Eight quants (two dwords of nibbles at shift sh, or of bytes) as one h8.
__device__ __forceinline__ h8 nib8(uint32_t w0, uint32_t w1, int sh, _Float16 off) {
    h2 a, b, c, d;
    byte_pairs(w0 >> sh, 0x000F000Fu, off, a, b);
    byte_pairs(w1 >> sh, 0x000F000Fu, off, c, d);
    return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
__device__ __forceinline__ h8 byte8(uint32_t w0, uint32_t w1, _Float16 off) {
    h2 a, b, c, d;
    byte_pairs(w0, 0x00FF00FFu, off, a, b);
    byte_pairs(w1, 0x00FF00FFu, off, c, d);
    return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}


}  // namespace fq
