// fq_dequant.hip -- the bit-exact dequant kernel (fq_dequant_rows) and small
// elementwise kernels: a fill kernel used instead of memset nodes (so callers
// may capture it) and the SiLU-multiply of the fused FFN.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"

namespace fq {

// Dequantize: one thread per (row, unit), bit-identical to the reference's
// row routines (scalar fp16 conversion, reference expression order).
template <int F>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      float* __restrict__ out, int N, int K,
                                                      int U, int row_bytes) {
    using Fm = Fmt<F>;
    constexpr int NG = Fm::NG, GS = 32 / NG;
    const size_t total = (size_t)N * U;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (size_t)gridDim.x * 256) {
        const int row = (int)(i / U), u = (int)(i - (size_t)row * U);
        const uint8_t* wr = w + (size_t)row * row_bytes;
        float q[32], A[NG], B[NG];
        Fm::template decode<true>(Fm::load(wr, u), u, q, A, B);
        float* o = out + (size_t)row * K;
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            const int k = Fm::k_of(u, s);
            if (k < K) o[k] = Fm::value(q[s], A[s / GS], B[s / GS]);
        }
    }
}

// Clears n words.
__global__ __launch_bounds__(256) void zero_kernel(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        p[i] = 0u;
}

// y = silu(gate) * up = gate / (1 + exp(-gate)) * up, as the reference's
// silu_multiply (src/operators/cpu/elementwise.cpp:89-150).
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gate,
                                                       const float* __restrict__ up,
                                                       float* __restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float g = gate[i];
        y[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

hipError_t launch_silu_mul(const float* gate, const float* up, float* y, size_t n, int cus,
                           hipStream_t st) {
    const size_t want = (n + 255) / 256, cap = (size_t)cus * 8;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, st,
                       gate, up, y, n);
    return hipGetLastError();
}

// y[m][off + n] = src[m][n]: places one matrix's outputs into the
// concatenated rows of a fused QKV result.
__global__ __launch_bounds__(256) void copy_cols_kernel(const float* __restrict__ src,
                                                        float* __restrict__ y, int M, int n_src,
                                                        int ld, int off) {
    const size_t total = (size_t)M * n_src;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (size_t)gridDim.x * 256) {
        const int m = (int)(i / n_src), n = (int)(i % n_src);
        y[(size_t)m * ld + off + n] = src[i];
    }
}

hipError_t launch_copy_cols(const float* src, float* y, int M, int n_src, int ld, int off, int cus,
                            hipStream_t st) {
    const size_t want = ((size_t)M * n_src + 255) / 256, cap = (size_t)cus * 8;
    hipLaunchKernelGGL(copy_cols_kernel, dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0,
                       st, src, y, M, n_src, ld, off);
    return hipGetLastError();
}

hipError_t launch_zero(uint32_t* p, size_t n, int grid, hipStream_t st) {
    hipLaunchKernelGGL(zero_kernel, dim3(grid), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

hipError_t launch_dequant(int dtype, const uint8_t* w, float* out, int N, int K, int U,
                          int row_bytes, int grid, hipStream_t st) {
return with_format(dtype, hipErrorInvalidValue, [&](auto f) {
        hipLaunchKernelGGL(dequant_kernel<decltype(f)::value>, dim3(grid), dim3(256), 0, st, w,
                           out, N, K, U, row_bytes);
        return hipGetLastError();
    });
}

}  // namespace fq
