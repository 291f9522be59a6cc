// fq_gemv.hip -- fused dequant + GEMV (M = 1) and small-batch (M <= 32)
// kernels for gfx950, plus the split-K finalize and the dequant kernel.
//
// Work decomposition (one launch):
//   grid.x  persistent work-groups striding over row groups,
//   grid.y  K-splits (contiguous ranges of 32-weight units),
//   grid.z  token groups of MT activations (small batch only).
// A work-group of 256 threads (4 wave64) first stages its activation slice
// in LDS, in the unit/slot order of the format (see fq_formats.h), together
// with the per-group activation sums.  Then each wave takes 64/T rows at a
// time; the T lanes of a row walk the row's units with stride T, loading each
// unit's bytes straight from HBM (one or two wide loads per unit, consecutive
// lanes on consecutive units, so a row segment is read contiguously), decode
// nibbles/bytes in registers and FMA against conflict-free ds_read_b128 of
// the staged activations.  The T partial sums of a row are combined with
// cross-lane shuffles inside the wave; no LDS round-trip, no atomics, so the
// result is deterministic.  With more than one K-split the per-split
// partials go to a workspace and fq_finalize sums them in split order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"

namespace fq {

constexpr int WG = 256;

template <int T>
__device__ __forceinline__ float row_reduce(float v) {
#pragma unroll
    for (int off = T / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Stage x[m0 .. m0+mt) restricted to units [u0, u0+uc) in slot order, with
// the per-group sums in each unit record's padding.  LDS layout (floats):
//   rec[t][u][0..31] = x[t][k_of(u0+u, s)]     (slot order)
//   rec[t][u][32+g]  = sum of group g's slots  (g < NG <= 4)
// A record is 36 floats = 144 B: consecutive lanes reading consecutive
// records with ds_read_b128 hit distinct banks, and every access of a unit
// is an immediate offset from one per-lane base address.
constexpr int REC = 36;

template <int F, int MT>
__device__ __forceinline__ void stage_x(float* lds, const float* __restrict__ x, int K, int m0,
                                        int mt, int u0, int uc) {
    using Fm = Fmt<F>;
    constexpr int NG = Fm::NG, GS = 32 / NG;
    const int per_tok = 32 * uc;
    for (int idx = threadIdx.x; idx < MT * per_tok; idx += WG) {
        int t = idx / per_tok, r = idx - t * per_tok;
        int u = r >> 5, s = r & 31;
        float v = 0.0f;
        if (t < mt) v = x[(size_t)(m0 + t) * K + Fm::k_of(u0 + u, s)];
        lds[t * REC * uc + REC * u + s] = v;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < MT * NG * uc; idx += WG) {
        int t = idx / (NG * uc), r = idx - t * NG * uc;
        int u = r / NG, g = r - u * NG;
        float* rec = lds + t * REC * uc + REC * u;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < GS; ++i) s += rec[g * GS + i];
        rec[32 + g] = s;
    }
    __syncthreads();
}

// One unit's contribution for MT tokens.
template <int F, int MT>
__device__ __forceinline__ void unit_dot(const typename Fmt<F>::Raw& raw, int u_abs, int u_loc,
                                         int uc, const float* lds, float* acc) {
    using Fm = Fmt<F>;
    constexpr int NG = Fm::NG, GS = 32 / NG;
    float q[32], A[NG], B[NG];
    Fm::template decode<false>(raw, u_abs, q, A, B);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const float4* xv = reinterpret_cast<const float4*>(lds + t * REC * uc + REC * u_loc);
        float P[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) P[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float4 xx = xv[c];
            int g = (4 * c) / GS;
            P[g] = __builtin_fmaf(xx.x, q[4 * c + 0], P[g]);
            P[g] = __builtin_fmaf(xx.y, q[4 * c + 1], P[g]);
            P[g] = __builtin_fmaf(xx.z, q[4 * c + 2], P[g]);
            P[g] = __builtin_fmaf(xx.w, q[4 * c + 3], P[g]);
        }
        const float4 sv = xv[8];
        const float S[4] = {sv.x, sv.y, sv.z, sv.w};
        float a = acc[t];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            a = __builtin_fmaf(A[g], P[g], a);
            a = __builtin_fmaf(B[g], S[g], a);
        }
        acc[t] = a;
    }
}

template <int F, int T, int MT>
__global__ __launch_bounds__(WG) void gemv_kernel(GemvArgs a) {
    extern __shared__ float lds[];
    using Fm = Fmt<F>;
    constexpr int RPW = 64 / T;            // rows per wave per step
    constexpr int RPB = (WG / 64) * RPW;   // rows per work-group per step
    const int m0 = blockIdx.z * MT;
    const int mt = min(MT, a.M - m0);
    const int u0 = blockIdx.y * a.Uc;
    const int uc = min(a.Uc, a.U - u0);
    stage_x<F, MT>(lds, a.x, a.K, m0, mt, u0, uc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane % T, rsub = lane / T;
    for (int rg = blockIdx.x; rg * RPB < a.N; rg += gridDim.x) {
        const int row = rg * RPB + wave * RPW + rsub;
        float acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
        if (row < a.N) {
            const uint8_t* wr = a.w + (size_t)row * a.row_bytes;
            int uu = li;
            // two units in flight per lane: issue both loads, then compute
            for (; uu + T < uc; uu += 2 * T) {
                auto r0 = Fm::load(wr, u0 + uu);
                auto r1 = Fm::load(wr, u0 + uu + T);
                unit_dot<F, MT>(r0, u0 + uu, uu, uc, lds, acc);
                unit_dot<F, MT>(r1, u0 + uu + T, uu + T, uc, lds, acc);
            }
            if (uu < uc) {
                auto r0 = Fm::load(wr, u0 + uu);
                unit_dot<F, MT>(r0, u0 + uu, uu, uc, lds, acc);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = row_reduce<T>(acc[t]);
        if (li == 0 && row < a.N) {
            for (int t = 0; t < mt; ++t) {
                const int m = m0 + t;
                if (a.part) {
                    a.part[((size_t)blockIdx.y * a.M + m) * a.N + row] = acc[t];
                } else {
                    float v = acc[t];
                    if (a.bias_mode == 1) {
                        if (row < a.bias_len) v += a.bias[row];
                    } else if (a.bias_mode == 2) {
                        size_t i = (size_t)m * a.N + row;
                        if ((int64_t)i < a.bias_len) v += a.bias[i];
                    }
                    a.y[(size_t)m * a.N + row] = v;
                }
            }
        }
    }
}

// y[m][n] = sum_s part[s][m][n] (+ bias), split order fixed.
__global__ __launch_bounds__(256) void finalize_kernel(const float* __restrict__ part, float* y,
                                                       int S, int M, int N, const float* bias,
                                                       int bias_mode, int64_t bias_len) {
    const size_t MN = (size_t)M * N;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < MN; i += (size_t)gridDim.x * 256) {
        float v = 0.0f;
        for (int s = 0; s < S; ++s) v += part[s * MN + i];
        const int n = (int)(i % N);
        if (bias_mode == 1) {
            if (n < bias_len) v += bias[n];
        } else if (bias_mode == 2) {
            if ((int64_t)i < bias_len) v += bias[i];
        }
        y[i] = v;
    }
}

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

// ---------------------------------------------------------------- launchers
template <int F, int T, int MT>
static hipError_t launch_t(const GemvArgs& a, const LaunchCfg& c, hipStream_t st) {
    hipLaunchKernelGGL((gemv_kernel<F, T, MT>), dim3(c.grid_x, c.splits, c.token_groups), dim3(WG),
                       c.lds_bytes, st, a);
    return hipGetLastError();
}

template <int F, int MT>
static hipError_t launch_mt(const GemvArgs& a, const LaunchCfg& c, hipStream_t st) {
    switch (c.T) {
        case 16: return launch_t<F, 16, MT>(a, c, st);
        case 64: return launch_t<F, 64, MT>(a, c, st);
        default: return hipErrorInvalidValue;
    }
}

template <int F>
static hipError_t launch_f(const GemvArgs& a, const LaunchCfg& c, hipStream_t st) {
    switch (c.MT) {
        case 1: return launch_mt<F, 1>(a, c, st);
        case 2: return launch_mt<F, 2>(a, c, st);
        case 4: return launch_mt<F, 4>(a, c, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(int dtype, const GemvArgs& a, const LaunchCfg& c, hipStream_t st) {
    switch (dtype) {
        case Q4_0: return launch_f<Q4_0>(a, c, st);
        case Q4_1: return launch_f<Q4_1>(a, c, st);
        case Q8_0: return launch_f<Q8_0>(a, c, st);
        case Q4_K: return launch_f<Q4_K>(a, c, st);
        case Q6_K: return launch_f<Q6_K>(a, c, st);
        default: return hipErrorInvalidValue;
    }
}

template <int F, int T, int MT>
static const void* fn_t() {
    return reinterpret_cast<const void*>(&gemv_kernel<F, T, MT>);
}

template <int F>
static const void* fn_f(int T, int MT) {
    if (T == 16) {
        if (MT == 1) return fn_t<F, 16, 1>();
        if (MT == 2) return fn_t<F, 16, 2>();
        if (MT == 4) return fn_t<F, 16, 4>();
    } else if (T == 64) {
        if (MT == 1) return fn_t<F, 64, 1>();
        if (MT == 2) return fn_t<F, 64, 2>();
        if (MT == 4) return fn_t<F, 64, 4>();
    }
    return nullptr;
}

const void* gemv_kernel_fn(int dtype, int T, int MT) {
    switch (dtype) {
        case Q4_0: return fn_f<Q4_0>(T, MT);
        case Q4_1: return fn_f<Q4_1>(T, MT);
        case Q8_0: return fn_f<Q8_0>(T, MT);
        case Q4_K: return fn_f<Q4_K>(T, MT);
        case Q6_K: return fn_f<Q6_K>(T, MT);
        default: return nullptr;
    }
}

hipError_t launch_finalize(const float* part, float* y, int S, int M, int N, const float* bias,
                           int bias_mode, int64_t bias_len, int grid, hipStream_t st) {
    hipLaunchKernelGGL(finalize_kernel, dim3(grid), dim3(256), 0, st, part, y, S, M, N, bias,
                       bias_mode, bias_len);
    return hipGetLastError();
}

hipError_t launch_dequant(int dtype, const uint8_t* w, float* out, int N, int K, int U,
                          int row_bytes, int grid, hipStream_t st) {
#define FQ_DQ(F)                                                                              \
    hipLaunchKernelGGL(dequant_kernel<F>, dim3(grid), dim3(256), 0, st, w, out, N, K, U,      \
                       row_bytes);                                                            \
    return hipGetLastError();
    switch (dtype) {
        case Q4_0: FQ_DQ(Q4_0)
        case Q4_1: FQ_DQ(Q4_1)
        case Q8_0: FQ_DQ(Q8_0)
        case Q4_K: FQ_DQ(Q4_K)
        case Q6_K: FQ_DQ(Q6_K)
        default: return hipErrorInvalidValue;
    }
#undef FQ_DQ
}

}  // namespace fq
