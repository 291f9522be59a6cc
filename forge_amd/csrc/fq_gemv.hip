// fq_gemv.hip -- fused dequant + GEMV (M = 1) and small-batch (M <= 32)
// kernels for gfx950, and the bit-exact dequant kernel.
//
// Work decomposition (one launch):
//   grid.x  persistent work-groups striding over row groups,
//   grid.y  K-splits (contiguous ranges of 32-weight units),
//   grid.z  token groups of MT activations.
// A work-group of 256 threads (4 wave64) owns 16 rows per step: each wave
// takes 64/T rows and the T lanes of a row own units li, li+T, ... of the
// row (at most NU per lane).  Per step a lane first issues the wide loads of
// ALL its units (consecutive lanes on consecutive units, so each row segment
// streams contiguously) and only then waits, decodes and FMAs against the
// activations staged in LDS; the very first step's loads are issued before
// the activations are staged, so staging overlaps the first HBM round trip,
// and each later step's loads are issued before the previous step's
// reduction and stores.  The T partial sums of a row are combined with
// cross-lane shuffles inside the wave: no LDS round trip and no atomics on
// y, so results are deterministic.  With several K-splits each split writes
// its partial row sums to a workspace and the last split to arrive for a
// row group (device counter) adds them in split order and writes y.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"

namespace fq {

constexpr int WG = 256;
constexpr int RPB = 16;  // rows per work-group step (4 waves x 64/T rows; T = 16)

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

template <int F, int T, int NU>
__device__ __forceinline__ void load_units(typename Fmt<F>::Raw* raw, const uint8_t* __restrict__ w,
                                           int row, int N, int row_bytes, int u0, int uc,
                                           int li) {
    if (row < N) {
        const uint8_t* wr = w + (size_t)row * row_bytes;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int uu = li + i * T;
            if (uu < uc) raw[i] = Fmt<F>::load(wr, u0 + uu);
        }
    }
}

template <int F, int T, int MT, int NU>
__global__ __launch_bounds__(WG) void gemv_kernel(GemvArgs a) {
    extern __shared__ float lds[];
    using Raw = typename Fmt<F>::Raw;
    constexpr int RPW = 64 / T;
    static_assert(RPW * (WG / 64) == RPB, "16 rows per work-group step");
    __shared__ int last_flag;

    const int m0 = blockIdx.z * MT;
    const int mt = min(MT, a.M - m0);
    const int u0 = blockIdx.y * a.Uc;
    const int uc = min(a.Uc, a.U - u0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane % T, rsub = lane / T;
    const int S = gridDim.y;

    Raw raw[NU];
    int rg = blockIdx.x;
    // the first step's weight loads go out before the activations are staged
    load_units<F, T, NU>(raw, a.w, rg * RPB + wave * RPW + rsub, a.N, a.row_bytes, u0, uc, li);
    stage_x<F, MT>(lds, a.x, a.K, m0, mt, u0, uc);

    for (; rg * RPB < a.N; rg += gridDim.x) {
        const int row = rg * RPB + wave * RPW + rsub;
        float acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
        if (row < a.N) {
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                const int uu = li + i * T;
                if (uu < uc) unit_dot<F, MT>(raw[i], u0 + uu, uu, uc, lds, acc);
            }
        }
        // the next step's loads fly during the reduction and the stores
        const int rg_next = rg + gridDim.x;
        if (rg_next * RPB < a.N)
            load_units<F, T, NU>(raw, a.w, rg_next * RPB + wave * RPW + rsub, a.N, a.row_bytes,
                                 u0, uc, li);
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = row_reduce<T>(acc[t]);

        if (S == 1) {
            if (li == 0 && row < a.N) {
                for (int t = 0; t < mt; ++t) {
                    const int m = m0 + t;
                    float v = acc[t];
                    if (a.bias_mode == 1) {
                        if (row < a.bias_len) v += a.bias[row];
                    } else if (a.bias_mode == 2) {
                        const size_t i = (size_t)m * a.N + row;
                        if ((int64_t)i < a.bias_len) v += a.bias[i];
                    }
                    a.y[(size_t)m * a.N + row] = v;
                }
            }
            continue;
        }
        // ---- split-K: publish partials; the last split of this row group reduces
        if (li == 0 && row < a.N) {
            for (int t = 0; t < mt; ++t)
                a.part[((size_t)blockIdx.y * a.M + m0 + t) * a.N + row] = acc[t];
        }
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned* cnt = a.counters + (size_t)blockIdx.z * a.rg_total + rg;
            const unsigned old = atomicAdd(cnt, 1u);
            const int is_last = old == (unsigned)(S - 1);
            if (is_last) atomicExch(cnt, 0u);  // leave the counter zeroed for the next call
            last_flag = is_last;
        }
        __syncthreads();
        if (last_flag) {
            __threadfence();
            for (int i = threadIdx.x; i < RPB * mt; i += WG) {
                const int r = rg * RPB + (i % RPB), t = i / RPB;
                if (r >= a.N) continue;
                const int m = m0 + t;
                float v = 0.0f;
                for (int s = 0; s < S; ++s)
                    v += __builtin_nontemporal_load(&a.part[((size_t)s * a.M + m) * a.N + r]);
                if (a.bias_mode == 1) {
                    if (r < a.bias_len) v += a.bias[r];
                } else if (a.bias_mode == 2) {
                    const size_t j = (size_t)m * a.N + r;
                    if ((int64_t)j < a.bias_len) v += a.bias[j];
                }
                a.y[(size_t)m * a.N + r] = v;
            }
        }
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

// Clears n words (used instead of a memset node, so callers may capture it).
__global__ __launch_bounds__(256) void zero_kernel(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        p[i] = 0u;
}

// ---------------------------------------------------------------- launchers
template <int F, int MT>
static const void* kfn_mt(int NU) {
    switch (NU) {
        case 2: return reinterpret_cast<const void*>(&gemv_kernel<F, 16, MT, 2>);
        case 4: return reinterpret_cast<const void*>(&gemv_kernel<F, 16, MT, 4>);
        case 8: return reinterpret_cast<const void*>(&gemv_kernel<F, 16, MT, 8>);
        default: return nullptr;
    }
}

template <int F>
static const void* kfn_f(int MT, int NU) {
    switch (MT) {
        case 1: return kfn_mt<F, 1>(NU);
        case 2: return kfn_mt<F, 2>(NU);
        case 4: return kfn_mt<F, 4>(NU);
        default: return nullptr;
    }
}

const void* gemv_kernel_fn(int dtype, int T, int MT, int NU) {
    if (T != 16) return nullptr;
    switch (dtype) {
        case Q4_0: return kfn_f<Q4_0>(MT, NU);
        case Q4_1: return kfn_f<Q4_1>(MT, NU);
        case Q8_0: return kfn_f<Q8_0>(MT, NU);
        case Q4_K: return kfn_f<Q4_K>(MT, NU);
        case Q6_K: return kfn_f<Q6_K>(MT, NU);
        default: return nullptr;
    }
}

hipError_t launch_gemv(int dtype, const GemvArgs& a, const LaunchCfg& c, hipStream_t st) {
    const void* fn = gemv_kernel_fn(dtype, c.T, c.MT, c.NU);
    if (!fn) return hipErrorInvalidValue;
    GemvArgs args = a;
    void* params[] = {&args};
    return hipLaunchKernel(fn, dim3(c.grid_x, c.splits, c.token_groups), dim3(WG), params,
                           c.lds_bytes, st);
}

hipError_t launch_zero(uint32_t* p, size_t n, int grid, hipStream_t st) {
    hipLaunchKernelGGL(zero_kernel, dim3(grid), dim3(256), 0, st, p, n);
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
