// fq_buf.h -- raw buffer loads for the batch-1 kernels: the uniform part of
// an address (a row's or tile's base, a slice's offset) lives in the buffer
// descriptor and the scalar soffset, the lane adds a 32-bit voffset, so no
// 64-bit vector address arithmetic is spent per load.  A load past the
// descriptor's size returns zeros (no fault).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fq {

typedef __amdgpu_buffer_rsrc_t Buf;
typedef uint32_t fq_v4u __attribute__((ext_vector_type(4)));
typedef uint32_t fq_v2u __attribute__((ext_vector_type(2)));
constexpr int BUF_NT = 2;  // non-temporal: the weights are read once per call

__device__ __forceinline__ Buf make_buf(const uint8_t* p, uint32_t bytes) {
    // word 3 = 0x00020000: raw (untyped) access on gfx9
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ uint4 bld128(Buf b, uint32_t so, uint32_t vo) {
    const fq_v4u v = __builtin_amdgcn_raw_buffer_load_b128(b, vo, so, BUF_NT);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bld64(Buf b, uint32_t so, uint32_t vo) {
    const fq_v2u v = __builtin_amdgcn_raw_buffer_load_b64(b, vo, so, BUF_NT);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t bld32(Buf b, uint32_t so, uint32_t vo) {
    return __builtin_amdgcn_raw_buffer_load_b32(b, vo, so, BUF_NT);
}
__device__ __forceinline__ uint32_t bld16(Buf b, uint32_t so, uint32_t vo) {
    return __builtin_amdgcn_raw_buffer_load_b16(b, vo, so, BUF_NT);
}

}  // namespace fq
