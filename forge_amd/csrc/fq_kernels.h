// fq_kernels.h -- launch interface between the C ABI (fq_capi.cpp) and the
// HIP kernels.  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fq {

struct GemvArgs {
    const float* x;       // [M][K]
    const uint8_t* w;     // [N] rows of row_bytes
    const uint8_t* w2;    // fused gate/up: the up matrix (w is the gate matrix); QKV: K
    const uint8_t* w3;    // fused QKV: V (w is Q, w2 is K)
    int n1, n2;           // fused QKV: rows of Q and K
    float* y;             // [M][N]
    const float* bias;    // optional, see bias_mode
    int64_t bias_len;
    int bias_mode;        // 0 none, 1 row vector over n, 2 full [M][N]
    int M, K, N;
    int U;                // 32-weight units per row (K / 32)
    int Uc;               // kernel-specific count: batch-1 activation records per
                          // token (gemvp), units or steps per chunk (the others)
    int row_bytes;
    float* part;          // gemvp K split: [splits][M][N] partial sums
    int spl;              // gemvp K split: K-slices per split (0: unsplit)
};

// batch-1 persistent kernel (fq_gemv1.hip)
const void* gemv1_kernel_fn(int dtype, bool bias, int wg);
size_t gemv1_lds_bytes(int dtype, int U, int wg);
// batch-1 chunk kernel over 2..4 tokens sharing each weight fetch (a.M tokens)
const void* gemv1_multi_fn(int dtype, bool bias, int nt, size_t* lds, int U);
hipError_t launch_gemv1(int dtype, const GemvArgs& a, int grid, int wg, hipStream_t st);
// row-step kernel for rows of at most 128 units, over nt = 1 or 2 tokens (a.M)
const void* gemv1r_kernel_fn(int dtype, int U, int row_bytes, bool bias, int* npr_out,
                             size_t* lds_out, int* wg_out, int nt = 1);
hipError_t launch_raw(const void* fn, const GemvArgs& a, int grid, int wg, size_t lds,
                      hipStream_t st, int grid_y = 1);
// packed-layout batch-1 kernels (fq_gemvp.hip)
void gemvp_geometry(int dtype, int K, int* units, int* records);
int gemvp_record_bytes();  // LDS bytes of one activation record
// nl: lane units per lane and step (K-slices are 64 nl units)
const void* gemvp_kernel_fn(int dtype, int units, int records, bool bias, size_t* lds, int* wg,
                            int* nl, int mode = 0);
// the same kernel over GGUF rows; *lds_fixed excludes the partial-sum buffer
// (4 bytes per token, row and K-slice of a work-group, placed after it);
// rows: the matrix's rows (the load depth depends on it); tokens: 1 … 4
// (y, a full bias and x token-major); mode 1 / 2: the fused gate/up and QKV
// forms, one token, no bias
const void* gemvg_kernel_fn(int dtype, int units, int records, bool bias, size_t* lds_fixed,
                            int* wg, int* nl, int rows, int tokens = 1, int mode = 0);
// batch-1 GEMV over the tiled aligned layout (fq_gemvt.hip; Q8_0 matrices
// for which packed_tiled() holds), one row per lane
struct TArgs {
    const float* x;             // [K]
    const uint8_t *w, *w2, *w3; // packed matrices (w2: up for the fused gate/up; w2, w3: K, V)
    int n1, n2;                 // fused QKV: rows of Q and K
    float* y;                   // [N]
    const float* bias;          // optional row vector, bias[n] for n < bias_len
    int64_t bias_len;
    int mode;                   // 0 plain, 1 fused gate/up (N rows each), 2 fused QKV
    int N, K;                   // output rows; K
    int U;                      // blocks per row (gemvt_units)
    int GR;                     // steps of four blocks per row (U / 4)
    int T;                      // tiles
    int recs;                   // activation records in each wave's LDS area
    int64_t row_bytes;          // packed row bytes
};
int gemvt_units(int dtype, int K);
int gemvt_max_records();    // per wave
int gemvt_max_tiles();      // per work-group
int gemvt_max_waves();      // per work-group
int gemvt_tile_rows();
int gemvt_record_bytes();
const void* gemvt_kernel_fn(int dtype, int mode);
hipError_t launch_gemvt(const void* fn, const TArgs& a, int grid, int waves, size_t lds,
                        hipStream_t st);
hipError_t launch_pack(int dtype, const uint8_t* src, uint8_t* dst, int N, int K, bool pack,
                       int grid, hipStream_t st);
hipError_t launch_zero(uint32_t* p, size_t n, int grid, hipStream_t st);
hipError_t launch_silu_mul(const float* gate, const float* up, float* y, size_t n, int cus,
                           hipStream_t st);
// y[m][off + n] = src[m][n] for n < n_src (rows of y are ld floats long)
hipError_t launch_copy_cols(const float* src, float* y, int M, int n_src, int ld, int off, int cus,
                            hipStream_t st);
// 2..8 tokens per pass, Q4_K on the int8 matrix cores (fq_mmqi.hip): a.M tokens,
// a.U tiles of 16 rows, a.Uc steps per chunk
bool mmqi_supported(int dtype);
const void* mmqi_kernel_fn(int mt_needed, bool bias, int K, int tiles_per_wg, int chunk,
                           size_t lds_cap, size_t* lds, int* wg);
// M > 1 on MFMA (fq_mmq.hip)
struct MmqArgs {
    const uint8_t* w;     // GGUF rows
    const void* xop;      // fp16 token operands, [Tp][NC][2048]
    const float* xsum;    // [Tp][NC][64] sub-block sums of the scaled activations
    const int* ex;        // [Tp][NC][16] power-of-two exponent per (token, chunk)
    float* y;             // [M][N]
    float* part;          // [splits][M][N] when splits > 1
    const float* bias;
    int64_t bias_len;
    int bias_mode;
    int M, N, K, NC, row_bytes;
};
enum { MMQ_SMALL1 = 0, MMQ_SMALL2 = 1, MMQ_MID = 2, MMQ_BIG = 3 };
void mmq_shape(int shape, int* bn, int* bm);
hipError_t launch_xprep(int dtype, const float* x, int M, int K, int NC, _Float16* xop,
                        float* xsum, int* ex, hipStream_t st);
hipError_t launch_mmq(int dtype, const MmqArgs& a, int shape, int gx, int gy, int splits,
                      hipStream_t st);
// 2..16 tokens on the fp16 matrix cores, weights streamed once (fq_mmqs.hip):
// the token operands of launch_xprep (one token tile), bands of rows_per_wg
// rows (at most 16 mmqs_max_tiles()) per work-group
bool mmqs_supported(int dtype);
int mmqs_max_tiles(int dtype);  // 16-row tiles per band
// splits > 1: K split over blockIdx.y into a.part slabs (super-blocks
// ceil(K/256 / splits) each), then launch_reduce adds them and the bias
hipError_t launch_mmqs(int dtype, const MmqArgs& a, int rows_per_wg, int wg, int splits,
                       hipStream_t st);
// prefill on v_mfma_f32_32x32x16_f16 (fq_mmqp.hip): token
// operands of launch_xprep32 (a.xop, a.ex = one exponent per token), a.part
// holds the split-K slabs when splits > 1 (then reduce with launch_reduce)
bool mmqp_supported(int dtype);
int mmqp_tile_rows();    // rows per work-group tile
int mmqp_tile_tokens();  // tokens per work-group tile
// sub16: the operand order of the Q6_K kernel (each 16-element quarter one
// sub-block)
hipError_t launch_xprep32(const float* x, int M, int K, _Float16* xop, int* ex, float* xsum,
                          bool sub16, hipStream_t st);
// Q6_K: the kernel reads 36-byte blocks that launch_q6c writes from the GGUF
// rows (mmqp_q6c_bytes(N, K) bytes, 16-byte aligned)
int64_t mmqp_q6c_bytes(int N, int K);
hipError_t launch_q6c(const uint8_t* w, int N, int K, int64_t row_bytes, uint8_t* out,
                      hipStream_t st);
hipError_t launch_mmqp(int dtype, const MmqArgs& a, int splits, hipStream_t st);
hipError_t launch_reduce(const MmqArgs& a, int splits, hipStream_t st);
hipError_t launch_dequant(int dtype, const uint8_t* w, float* out, int N, int K, int U,
                          int row_bytes, int grid, hipStream_t st);

}  // namespace fq
