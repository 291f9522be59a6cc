// fq_mfma16.h -- fp16 MFMA operand helpers shared by the M > 1 kernels.
//
// Quants become fp16 two at a time: a byte pair (b0, b2) of a dword placed
// in the low bytes of 0x6400'6400 reads as the halves 1024 + b0, 1024 + b2,
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

// The four bytes of w as two fp16 pairs, value - off: v_perm pairs each byte
// with 0x64, so a half reads 1024 + byte (exact), and one packed fp16
// subtract removes the offset.  p0 = bytes 0 and 2, p1 = bytes 1 and 3.
__device__ __forceinline__ void byte_pairs(uint32_t w, _Float16 off, h2& p0, h2& p1) {
    const h2 o = {off, off};
    p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u)) - o;
    p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u)) - o;
}

// Eight quants (two dwords of nibbles at shift sh, or of bytes) as one h8.
__device__ __forceinline__ h8 nib8(uint32_t w0, uint32_t w1, int sh, _Float16 off) {
    h2 a, b, c, d;
    byte_pairs((w0 >> sh) & 0x0F0F0F0Fu, off, a, b);
    byte_pairs((w1 >> sh) & 0x0F0F0F0Fu, off, c, d);
    return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
__device__ __forceinline__ h8 byte8(uint32_t w0, uint32_t w1, _Float16 off) {
    h2 a, b, c, d;
    byte_pairs(w0, off, a, b);
    byte_pairs(w1, off, c, d);
    return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}


}  // namespace fq
