// fq_kernels.h -- launch interface between the C ABI (fq_capi.cpp) and the
// HIP kernels (fq_gemv.hip, fq_mmq.hip).  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fq {

struct GemvArgs {
    const float* x;       // [M][K]
    const uint8_t* w;     // [N] rows of row_bytes
    float* y;             // [M][N]
    float* part;          // [splits][M][N] when splits > 1, else nullptr
    const float* bias;    // optional, see bias_mode
    int64_t bias_len;
    int bias_mode;        // 0 none, 1 row vector over n, 2 full [M][N]
    int M, K, N;
    int U;                // 32-weight units per row (K / 32)
    int Uc;               // units per K-split
    int row_bytes;
};

struct LaunchCfg {
    int T;                // lanes per row: 16 or 64
    int MT;               // tokens per work-group: 1, 2 or 4
    int grid_x;           // persistent work-groups per (split, token group)
    int splits;           // grid.y
    int token_groups;     // grid.z
    size_t lds_bytes;
};

hipError_t launch_gemv(int dtype, const GemvArgs& a, const LaunchCfg& c, hipStream_t st);
const void* gemv_kernel_fn(int dtype, int T, int MT);
hipError_t launch_finalize(const float* part, float* y, int S, int M, int N, const float* bias,
                           int bias_mode, int64_t bias_len, int grid, hipStream_t st);
hipError_t launch_dequant(int dtype, const uint8_t* w, float* out, int N, int K, int U,
                          int row_bytes, int grid, hipStream_t st);

}  // namespace fq
