// fq_mmqp.hip -- prefill (M > 32 tokens) for the 32-weight block formats
// Q8_0 and Q4_0 on v_mfma_f32_32x32x16_f16.
//
//   D[token][n] = X[token][k] . W[n][k]^T, per 32-element block b:
//     A (32 tokens x 16 k): x 2^-e(token) as fp16 hi + lo (xprep32_kernel),
//     B (16 k x 32 rows):   the block's integer codes, exact in fp16,
//     D_b = A_hi B + A_lo B  (two MFMAs per 16 k, one fp32 result per block),
//     acc += d_b(n) D_b      (one FMA per output and block),
//   y = 2^e(token) acc at the end.
// Weights are the B operand so that a lane's 16 results all belong to one
// row n: the block scale d_b(n) is one value per lane.  One exponent per
// token over all of K (the token's largest |x| scaled into [2^14, 2^15))
// keeps the per-block epilogue to that single FMA; x_hi + x_lo carry 22
// significant bits.
//
// A work-group owns 128 tokens x 128 rows (4 waves, 64 x 64 each: 2 x 2
// MFMA tiles) and a K range (split-K when the tiles alone leave CUs idle;
// reduce_kernel adds the slabs in split order).  Per 64-element K-step every
// global load of the next step is issued at once -- the token operands (four
// contiguous 8 KiB runs, copied straight into the other of two LDS buffers)
// and the 128 weight rows' 68 / 36 bytes (into registers, written to LDS
// after the step's compute).  So each step waits once, at its barrier, for
// loads issued a whole step earlier, and no short load queues behind a long
// one in the in-order vector memory counter.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"
#include "fq_mfma16.h"

namespace fq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BMT = 128, BNT = 128;  // tokens, rows per work-group
constexpr int KS = 64;               // K elements per step (two blocks)
constexpr int XT = 1024;             // halves per (32-token tile, 16-k quarter): hi then lo

// ------------------------------------------------------------- token prep
// One work-group per token: e = ilogb(max |x|) - 14, then x 2^-e split into
// fp16 hi + lo, written as the A operand of v_mfma_f32_32x32x16_f16: for
// token tile T = m / 32 and quarter kq = k / 16, lane (m % 32) + 32 g holds
// elements 16 kq + 8 g + slot_elem(j), j = 0..7 (hi block, then lo block).
__global__ __launch_bounds__(256) void xprep32_kernel(const float* __restrict__ x, int K,
                                                      _Float16* __restrict__ xop,
                                                      int* __restrict__ ex) {
    __shared__ float wmax[4];
    const int m = blockIdx.x;
    const float* xr = x + (size_t)m * K;
    float mx = 0.0f;
    for (int k = threadIdx.x * 4; k < K; k += 1024) {
        const float4 v = *reinterpret_cast<const float4*>(xr + k);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e = 0;
    if (mx > 0.0f && mx <= 3.0e38f) e = ilogbf(mx) - 14;
    if (threadIdx.x == 0) ex[m] = e;
    const int T = m >> 5, lm = m & 31;
    for (int grp = threadIdx.x; grp < K / 8; grp += 256) {
        const float4 a = *reinterpret_cast<const float4*>(xr + 8 * grp);
        const float4 b = *reinterpret_cast<const float4*>(xr + 8 * grp + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        h8 hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float w = __builtin_amdgcn_ldexpf(v[slot_elem(j)], -e);
            hi[j] = (_Float16)w;
            lo[j] = (_Float16)(w - (float)hi[j]);
        }
        const int kq = grp >> 1, g = grp & 1;
        _Float16* dst = xop + ((size_t)T * (K / 16) + kq) * XT + (lm + 32 * g) * 8;
        *reinterpret_cast<h8*>(dst) = hi;
        *reinterpret_cast<h8*>(dst + 512) = lo;
    }
}

// -------------------------------------------------------- weight operands
template <int F>
struct PB;

// Q8_0 block (34 B): d @0, qs int8[32] @2.  The B operand of half h (16 k)
// for lane k-group g: qs bytes [16 h + 8 g, +8) as fp16 (+128 via the sign
// bit, so the bytes are unsigned, then -1152 = -(1024 + 128)).
template <>
struct PB<Q8_0> {
    static constexpr int BB = 34, SB = 2 * BB;  // bytes per block, per step
    __device__ static h8 op(const uint8_t* blk, int h, int g) {
        const uint2 q = lds8_a2(blk + 2 + 16 * h + 8 * g);
        return byte8(q.x ^ 0x80808080u, q.y ^ 0x80808080u, (_Float16)1152.0f);
    }
};

// Q4_0 block (18 B): d @0, qs[16] @2; element j < 16 is the low nibble of
// byte j, element j + 16 the high nibble (value - 8).
template <>
struct PB<Q4_0> {
    static constexpr int BB = 18, SB = 2 * BB;
    __device__ static h8 op(const uint8_t* blk, int h, int g) {
        const uint2 q = lds8_a2(blk + 2 + 8 * g);
        return nib8(q.x, q.y, 4 * h, (_Float16)1032.0f);
    }
};

template <int F>
__global__ __launch_bounds__(256) void mmqp_kernel(MmqArgs a, int steps_per_split) {
    using P = PB<F>;
    constexpr int WROW = (P::SB + 3) / 4 * 4;     // LDS bytes per weight row and step
    constexpr int WDW = BNT * WROW / 4;            // dwords of the weight tile
    constexpr int WPT = (WDW + 255) / 256;         // weight dwords per thread
    // token operands: two buffers (the next step's arrive by DMA while this
    // step reads the other), 4 token tiles x 4 quarters each
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][4 * 4 * XT];
    __shared__ __attribute__((aligned(16))) uint8_t ws[BNT * WROW];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6, wm = wave >> 1, wn = wave & 1;  // 64-token / 64-row quadrant
    const int n0 = blockIdx.x * BNT, m0 = blockIdx.y * BMT;
    const int nsteps = a.K / KS;
    const int s0 = blockIdx.z * steps_per_split, s1 = min(nsteps, s0 + steps_per_split);
    const int T0 = m0 / 32;                 // first token tile
    const int Tn = (a.M + 31) / 32;         // token tiles in the operand buffer
    const int KQ = a.K / 16;

    // loads of step s: the token operands straight into LDS buffer s & 1
    // (wave w copies token tile w's contiguous 8 KiB run, 1 KiB per
    // instruction), the weight rows into registers
    uint32_t wr[WPT];
    auto gload = [&](int s) {
        {
            const int T = min(T0 + wave, Tn - 1);
            const uint8_t* src = reinterpret_cast<const uint8_t*>(
                reinterpret_cast<const _Float16*>(a.xop) + ((size_t)T * KQ + 4 * s) * XT);
            uint8_t* dst = reinterpret_cast<uint8_t*>(xs[s & 1]) + wave * 8192;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void*)(src + 1024 * i + 16 * lane),
                    (__attribute__((address_space(3))) void*)(dst + 1024 * i), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const int idx = min(tid + 256 * i, WDW - 1);
            const int r = idx / (WROW / 4), c = idx - r * (WROW / 4);
            const int row = min(n0 + r, a.N - 1);
            const uint8_t* src = a.w + (size_t)row * a.row_bytes + (size_t)s * P::SB + 4 * c;
            wr[i] = ld_u32(src);  // a step of a row is 68 / 36 bytes: whole dwords
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int i = 0; i < WPT; ++i) {
            const int idx = tid + 256 * i;
            if (idx < WDW) reinterpret_cast<uint32_t*>(ws)[idx] = wr[i];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int g = lane >> 5, c = lane & 31;
    if (s0 < s1) gload(s0);
    for (int s = s0; s < s1; ++s) {
        __syncthreads();  // the previous step's LDS reads are done
        lstore();
        __syncthreads();
        if (s + 1 < s1) gload(s + 1);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            // token operands of both 16-k halves of the block, then per
            // weight tile the four MFMAs of both token tiles and the fold
            h8 ah[2][2], al[2][2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const _Float16* xp =
                        xs[s & 1] + ((2 * wm + i) * 4 + 2 * b + h) * XT + lane * 8;
                    ah[h][i] = *reinterpret_cast<const h8*>(xp);
                    al[h][i] = *reinterpret_cast<const h8*>(xp + 512);
                }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint8_t* wrow = ws + (64 * wn + 32 * j + c) * WROW + P::BB * b;
                const h8 b0 = P::op(wrow, 0, g), b1 = P::op(wrow, 1, g);
                const f32x16 z = {};
                f32x16 d[2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    d[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0][i], b0, z, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    d[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0][i], b0, d[i], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    d[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1][i], b1, d[i], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    d[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1][i], b1, d[i], 0, 0, 0);
                const float db = f16_hw(*reinterpret_cast<const uint16_t*>(wrow));
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[i][j][e] = __builtin_fmaf(db, d[i][e], acc[i][j][e]);
            }
        }
    }
    // lane (c, g): column n = 32 j + c of its quadrant, rows 8 (e / 4) + 4 g + e % 4
    const bool split = gridDim.z > 1;
    float* out = split ? a.part + (size_t)blockIdx.z * a.M * a.N : a.y;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int ei[16];
#pragma unroll
        for (int e = 0; e < 16; ++e)
            ei[e] = a.ex[min(m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3), a.M - 1)];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + 64 * wn + 32 * j + c;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
                if (m < a.M && n < a.N) {
                    float v = __builtin_amdgcn_ldexpf(acc[i][j][e], ei[e]);
                    if (!split) {
                        if (a.bias_mode == 1) v += n < a.bias_len ? a.bias[n] : 0.0f;
                        else if (a.bias_mode == 2) v += a.bias[(size_t)m * a.N + n];
                    }
                    out[(size_t)m * a.N + n] = v;
                }
            }
        }
    }
}

}  // namespace

bool mmqp_supported(int dtype) { return dtype == Q8_0 || dtype == Q4_0; }

hipError_t launch_xprep32(const float* x, int M, int K, _Float16* xop, int* ex, hipStream_t st) {
    hipLaunchKernelGGL(xprep32_kernel, dim3(M), dim3(256), 0, st, x, K, xop, ex);
    return hipGetLastError();
}

hipError_t launch_mmqp(int dtype, const MmqArgs& a, int splits, hipStream_t st) {
    const int nsteps = a.K / KS;
    const int sps = (nsteps + splits - 1) / splits;
    const dim3 grid((a.N + BNT - 1) / BNT, (a.M + BMT - 1) / BMT, splits);
    if (dtype == Q8_0)
        hipLaunchKernelGGL(mmqp_kernel<Q8_0>, grid, dim3(256), 0, st, a, sps);
    else if (dtype == Q4_0)
        hipLaunchKernelGGL(mmqp_kernel<Q4_0>, grid, dim3(256), 0, st, a, sps);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace fq
