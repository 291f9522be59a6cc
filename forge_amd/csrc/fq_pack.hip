// fq_pack.hip -- GGUF block layout <-> aligned device layout (see fq_pack.h).
// One thread per block (Q4_0/Q4_1/Q8_0) or super-block (Q4_K/Q6_K); bytes are
// moved in 2-byte units (every field offset is even).  Packing zero-fills the
// row padding, so a packed matrix is a deterministic function of the input.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_kernels.h"
#include "fq_pack.h"

namespace fq {
namespace {

__device__ __forceinline__ void copy2(uint8_t* dst, const uint8_t* src, int n) {
    for (int i = 0; i < n; i += 2)
        *reinterpret_cast<uint16_t*>(dst + i) = *reinterpret_cast<const uint16_t*>(src + i);
}

// PACK = true: raw -> packed; false: packed -> raw.
template <bool PACK>
__device__ __forceinline__ void move(uint8_t* raw, uint8_t* pk, int n) {
    if (PACK) copy2(pk, raw, n);
    else copy2(raw, pk, n);
}

// Byte o of packed row n in the tiled arrangement: rows are grouped in tiles
// of 16 (the last tile holds the remaining rows), and within a tile of R rows
// the 16-byte piece J of row r sits at (J R + r) 16.  Fields never straddle a piece (every plane
// starts on a 16-byte boundary and fields are 2, 4, 8 or 16 bytes at offsets
// that are multiples of their size), so a field moves as one run.
__device__ __forceinline__ uint8_t* tpos(uint8_t* pk, int64_t PB, int N, int n, int64_t o) {
    const int t = n >> 4, r = n & 15, R = min(16, N - 16 * t);
    return pk + (int64_t)t * 16 * PB + (((o >> 4) * R + r) << 4) + (o & 15);
}

template <bool PACK>
__global__ __launch_bounds__(256) void pack_kernel(int dtype, uint8_t* raw, uint8_t* pk, int N,
                                                   int K) {
    const int U = K / 32, S = K / 256;
    const int64_t RB = dtype == 2 ? 18LL * U : dtype == 3 ? 20LL * U : dtype == 7 ? 34LL * U
                       : dtype == 4 ? 144LL * S : 210LL * S;
    const int64_t PB = packed_row_bytes(dtype, K);
    const int per_row = (dtype == 4 || dtype == 13) ? S : U;
    const bool tiled = packed_tiled(dtype, N);
    const int64_t total = (int64_t)N * per_row;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int r = (int)(i / per_row), b = (int)(i - (int64_t)r * per_row);
        uint8_t* rr = raw + r * RB;
        auto P = [&](int64_t o) { return tiled ? tpos(pk, PB, N, r, o) : pk + r * PB + o; };
        switch (dtype) {
            case 2:  // Q4_0: d | qs[16]
                move<PACK>(rr + 18 * b + 2, P(16 * b), 16);
                move<PACK>(rr + 18 * b, P(16 * U + 2 * b), 2);
                break;
            case 3:  // Q4_1: d m | qs[16]
                move<PACK>(rr + 20 * b + 4, P(16 * b), 16);
                move<PACK>(rr + 20 * b, P(16 * U + 4 * b), 4);
                break;
            case 7:  // Q8_0: d | qs[32]
                move<PACK>(rr + 34 * b + 2, P(16 * b), 16);
                move<PACK>(rr + 34 * b + 18, P(16 * U + 16 * b), 16);
                move<PACK>(rr + 34 * b, P(32 * U + 2 * b), 2);
                break;
            case 4: {  // Q4_K: d dmin scales[12] | qs[128]
                const int V = K / 64;
                uint8_t* sb = rr + 144 * b;
                for (int g = 0; g < 4; ++g) {
                    move<PACK>(sb + 16 + 32 * g, P(16 * (4 * b + g)), 16);
                    move<PACK>(sb + 32 + 32 * g, P(16 * V + 16 * (4 * b + g)), 16);
                }
                move<PACK>(sb, P(32 * V + 16 * b), 16);
                break;
            }
            case 13: {  // Q6_K: ql[128] qh[64] sc[16] d
                const int V = K / 64;
                uint8_t* sb = rr + 210 * b;
                for (int p = 0; p < 4; ++p) {
                    const int n = p >> 1, h = p & 1, v = 4 * b + p;
                    move<PACK>(sb + 64 * n + 16 * h, P(16 * v), 16);
                    move<PACK>(sb + 64 * n + 32 + 16 * h, P(16 * V + 16 * v), 16);
                    move<PACK>(sb + 128 + 32 * n + 16 * h, P(32 * V + 16 * v), 16);
                }
                move<PACK>(sb + 192, P(192 * S + 16 * b), 16);
                move<PACK>(sb + 208, P(208 * S + 2 * b), 2);
                break;
            }
        }
        if (PACK && b == 0) {  // zero the row's tail padding
            const int64_t used = dtype == 2 ? 18LL * U : dtype == 3 ? 20LL * U
                                 : dtype == 7 ? 34LL * U : dtype == 4 ? 144LL * S : 210LL * S;
            for (int64_t t = used; t < PB; ++t) *P(t) = 0;
        }
    }
}

}  // namespace

hipError_t launch_pack(int dtype, const uint8_t* src, uint8_t* dst, int N, int K, bool pack,
                       int grid, hipStream_t st) {
    if (pack)
        hipLaunchKernelGGL(pack_kernel<true>, dim3(grid), dim3(256), 0, st, dtype,
                           const_cast<uint8_t*>(src), dst, N, K);
    else
        hipLaunchKernelGGL(pack_kernel<false>, dim3(grid), dim3(256), 0, st, dtype, dst,
                           const_cast<uint8_t*>(src), N, K);
    return hipGetLastError();
}

}  // namespace fq
