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
    unsigned* counters;   // [token_groups][rg_total] split arrival counters (zero between calls)
    int rg_total;         // row groups of 16 rows: ceil(N / 16)
    const float* bias;    // optional, see bias_mode
    int64_t bias_len;
    int bias_mode;        // 0 none, 1 row vector over n, 2 full [M][N]
    int M, K, N;
    int U;                // 32-weight units per row (K / 32)
    int Uc;               // units per K-split
    int row_bytes;
    int split_units;      // packed split-K: lane units per K-slice
    int waves_total;      // packed split-K: counter stride (waves in the grid)
};

struct LaunchCfg {
    int T;                // lanes per row (16)
    int MT;               // tokens per work-group: 1, 2 or 4
    int NU;               // max units per lane per row: 2, 4 or 8
    int grid_x;           // persistent work-groups per (split, token group)
    int splits;           // grid.y
    int token_groups;     // grid.z
    size_t lds_bytes;
};

hipError_t launch_gemv(int dtype, const GemvArgs& a, const LaunchCfg& c, hipStream_t st);
const void* gemv_kernel_fn(int dtype, int T, int MT, int NU);
// batch-1 persistent kernel (fq_gemv1.hip)
const void* gemv1_kernel_fn(int dtype, bool bias, int wg);
size_t gemv1_lds_bytes(int dtype, int U, int wg);
hipError_t launch_gemv1(int dtype, const GemvArgs& a, int grid, int wg, hipStream_t st);
const void* gemv1r_kernel_fn(int dtype, int U, int row_bytes, bool bias, int* npr_out,
                             size_t* lds_out, int* wg_out);
hipError_t launch_raw(const void* fn, const GemvArgs& a, int grid, int wg, size_t lds,
                      hipStream_t st);
// packed-layout batch-1 kernels (fq_gemvp.hip)
void gemvp_geometry(int dtype, int K, int* units, int* records);
const void* gemvp_kernel_fn(int dtype, int units, int records, bool bias, size_t* lds, int* wg);
hipError_t launch_pack(int dtype, const uint8_t* src, uint8_t* dst, int N, int K, bool pack,
                       int grid, hipStream_t st);
hipError_t launch_zero(uint32_t* p, size_t n, int grid, hipStream_t st);
hipError_t launch_dequant(int dtype, const uint8_t* w, float* out, int N, int K, int U,
                          int row_bytes, int grid, hipStream_t st);

}  // namespace fq
