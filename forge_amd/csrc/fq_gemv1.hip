// fq_gemv1.hip -- batch-1 fused dequant + GEMV for gfx950.
//
// One persistent work-group of 1024 threads (16 wave64) per CU slot.  The
// work-group stages the whole activation vector once, in the unit/slot
// record layout of fq_formats.h, then its waves stream rows: wave g of G
// takes rows g, g + G, ...; all 64 lanes of a wave work on the same row, lane
// l owning the row's units l, l + 64, ...  Each lane walks a flat sequence of
// (row, unit-slot) items in batches of NB items and software-pipelines the
// batches -- the next batch's non-temporal wide loads are in flight while the
// current batch is decoded and FMA'd -- so every lane keeps NB units of
// weight bytes in flight at all times, across row boundaries.  A finished
// row is summed across the wave with DPP (row_shr, row_bcast) and stored by
// one lane: no atomics, deterministic.
//
// Why this shape: rows are the natural work item (16 waves x 256 CUs = 4096
// agents against 3.5k-152k rows), the x vector is staged once per CU instead
// of once per 16 rows, and consecutive lanes read consecutive units so each
// wave-wide load instruction covers one contiguous stretch of the row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"

namespace fq {
namespace {


template <int F>
__device__ __forceinline__ float unit_dot1(const typename Fmt<F>::Raw& raw, int u,
                                           const uint8_t* lds, float acc) {
    const int4* rp = reinterpret_cast<const int4*>(lds + RECB * u);
    Limbs L;
    const int4 v0 = rp[0], v1 = rp[1], v2 = rp[2], v3 = rp[3], v4 = rp[4], v5 = rp[5];
    L.l1[0] = v0.x; L.l1[1] = v0.y; L.l1[2] = v0.z; L.l1[3] = v0.w;
    L.l1[4] = v1.x; L.l1[5] = v1.y; L.l1[6] = v1.z; L.l1[7] = v1.w;
    L.l2[0] = v2.x; L.l2[1] = v2.y; L.l2[2] = v2.z; L.l2[3] = v2.w;
    L.l2[4] = v3.x; L.l2[5] = v3.y; L.l2[6] = v3.z; L.l2[7] = v3.w;
    L.l3[0] = v4.x; L.l3[1] = v4.y; L.l3[2] = v4.z; L.l3[3] = v4.w;
    L.l3[4] = v5.x; L.l3[5] = v5.y; L.l3[6] = v5.z; L.l3[7] = v5.w;
    const float4 t = reinterpret_cast<const float4*>(lds + RECB * u)[6];
    L.s1 = t.x;
    L.S[0] = t.y;
    L.S[1] = t.z;
    L.S[2] = t.w;
    L.S[3] = Fmt<F>::NG == 4 ? reinterpret_cast<const float*>(lds + RECB * u)[28] : 0.0f;
    return acc + limb_dot<F>(raw, u, L);
}

// ---------------------------------------------------------------- streaming
// A wave processes one row at a time, 64 units (one per lane) per chunk.  A
// chunk's bytes are fetched as the 16-byte-aligned superset of its byte
// range -- lane p loads piece p, so one wave-wide dwordx4 covers 1 KB of
// contiguous HBM -- and written to the wave's LDS buffer; each lane then
// reads its own unit at whatever alignment the block layout gives it
// (gfx950 LDS reads need no alignment).  Reading the superset is safe: an
// aligned 16-byte piece that holds a valid byte never crosses a page.
template <int F>
struct Chunk {
    static constexpr int UPB = Fmt<F>::BE / 32;                 // units per block
    static constexpr int BYTES = 64 / UPB * Fmt<F>::BB;         // bytes of 64 units
    static constexpr int PIECES = (BYTES + 15) / 16 + 1;        // + misalignment
    static constexpr int NP = (PIECES + 63) / 64;               // loads per lane
    static constexpr int WBUF = PIECES * 16;                    // LDS bytes per wave
};

// Wave-uniform position (row, chunk) of a wave's stream; rows r0, r0 + stride, ...
struct Pos {
    int row, c;
    __device__ __forceinline__ void next(int nc, int stride) {
        if (++c == nc) {
            c = 0;
            row += stride;
        }
    }
};

template <int F>
struct Fetch {
    uint4 v[Chunk<F>::NP];
};

// Byte range of chunk (row, c): start address and unit count.
template <int F>
__device__ __forceinline__ const uint8_t* chunk_addr(const GemvArgs& a, const Pos& p) {
    const int row = min(p.row, a.N - 1);
    return a.w + (size_t)row * a.row_bytes + (size_t)p.c * Chunk<F>::BYTES;
}

template <int F>
__device__ __forceinline__ void fetch(Fetch<F>& f, const GemvArgs& a, const Pos& p, int lane) {
    // pointer arithmetic (not integer casts) keeps the global address space,
    // so these stay global_load (vmcnt only) instead of flat_load
    const uint8_t* g0 = chunk_addr<F>(a, p);
    const int shift = (int)(reinterpret_cast<uintptr_t>(g0) & 15);
    const uint8_t* a0 = g0 - shift;
    const int nunits = min(64, a.U - 64 * p.c);
    const int nbytes = nunits / Chunk<F>::UPB * Fmt<F>::BB;
    const int n16 = (shift + nbytes + 15) >> 4;
#pragma unroll
    for (int i = 0; i < Chunk<F>::NP; ++i) {
        const int piece = min(lane + 64 * i, n16 - 1);
        f.v[i] = ldg128<true>(a0 + 16 * piece);
    }
}

template <int F>
__device__ __forceinline__ void spill(const Fetch<F>& f, uint8_t* wbuf, int lane) {
    // unconditional stores (clamped slot): a branch here would make the
    // compiler drain every load in flight before it
#pragma unroll
    for (int i = 0; i < Chunk<F>::NP; ++i) {
        const int piece = min(lane + 64 * i, Chunk<F>::PIECES - 1);
        reinterpret_cast<uint4*>(wbuf)[piece] = f.v[i];
    }
}

// Finished rows are not stored one by one: the k-th row of a block of up to
// 64 rows goes to lane k of a result register and the block is written with
// one store.  The steady-state loop body has no branches (row ends are
// selects) and no stores: a store or a branch between the fetches would sit
// in the same in-order counter as the weight loads and make the compiler
// drain every load in flight, collapsing the two-deep pipeline.
// NT tokens: the unit's weights are read and unpacked once and dotted with
// each token's limb records (token m's records start at lds + m U RECB).
template <int F, bool BIAS, int NT>
__device__ __forceinline__ void consume(const GemvArgs& a, const Pos& p, const uint8_t* wbuf,
                                        const uint8_t* lds, int lane, int nc, float (&acc)[NT],
                                        float (&res)[NT], int& k) {
    const int shift = (int)(reinterpret_cast<uintptr_t>(chunk_addr<F>(a, p)) & 15);
    const int nunits = min(64, a.U - 64 * p.c);
    const int ul = min(lane, nunits - 1);
    const auto raw = Fmt<F>::template load<false>(wbuf + shift, ul);
    const bool row_end = p.c == nc - 1;  // wave-uniform
#pragma unroll
    for (int m = 0; m < NT; ++m) {
        const float t = unit_dot1<F>(raw, 64 * p.c + ul, lds + (size_t)m * a.U * RECB, acc[m]);
        acc[m] = lane < nunits ? t : acc[m];
        float s = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum(acc[m])), 63));
        if constexpr (BIAS) {
            const int r = min(p.row, a.N - 1);
            if (a.bias_mode == 2)
                s += ((const_fp)(uintptr_t)a.bias)[(size_t)m * a.N + r];
            else
                s += r < a.bias_len ? ((const_fp)(uintptr_t)a.bias)[r] : 0.0f;
        }
        res[m] = (row_end && lane == k) ? s : res[m];
        acc[m] = row_end ? 0.0f : acc[m];
    }
    k += row_end ? 1 : 0;
}

template <int F, bool BIAS, int NT>
__device__ __forceinline__ void step(Fetch<F>& f, Pos& ld, Pos& cp, const GemvArgs& a,
                                     uint8_t* wbuf, const uint8_t* lds, int lane, int nc,
                                     int stride, float (&acc)[NT], float (&res)[NT], int& k) {
    // sched_barrier keeps the scheduler from hoisting the next step's spill
    // (and the wait for its loads) above this step's fetch
    __builtin_amdgcn_sched_barrier(0);
    spill<F>(f, wbuf, lane);
    fetch<F>(f, a, ld, lane);
    ld.next(nc, stride);
    consume<F, BIAS, NT>(a, cp, wbuf, lds, lane, nc, acc, res, k);
    cp.next(nc, stride);
    __builtin_amdgcn_sched_barrier(0);
}

// NT tokens (a.M == NT) share each weight fetch; records of all NT tokens
// are staged.
template <int F, bool BIAS, int WG1, int NT = 1>
__global__ __launch_bounds__(WG1) void gemv1_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int stride = gridDim.x * (WG1 / 64);
    const int first = __builtin_amdgcn_readfirstlane(blockIdx.x * (WG1 / 64) + wave);
    const int nc = (a.U + 63) >> 6;
    uint8_t* wbuf = lds + (size_t)NT * a.U * RECB + wave * Chunk<F>::WBUF;

    // two chunks in flight per wave; the first two are fetched before the
    // activations are staged
    XStage<Fmt<F>, WG1> xs;
    stage_load<Fmt<F>, WG1>(xs, a.x, NT * a.U, 0, a.U, a.K);  // activation loads first
    Pos ld{first, 0}, cp{first, 0};
    Fetch<F> f0, f1;
    fetch<F>(f0, a, ld, lane);
    ld.next(nc, stride);
    fetch<F>(f1, a, ld, lane);
    ld.next(nc, stride);
    stage_build<Fmt<F>, WG1>(lds, xs, a.x, NT * a.U, 0, a.U, a.K);

    float acc[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) acc[m] = 0.0f;
    while (cp.row < a.N) {
        // a block of up to 64 rows with an even number of chunks
        const int rows_left = (a.N - 1 - cp.row) / stride + 1;
        int nrows = min(64, rows_left);
        if ((nrows * nc) & 1) nrows -= nrows > 1 ? 1 : 0;
        const int nchunks = nrows * nc;
        const int row0 = cp.row;
        float res[NT];
#pragma unroll
        for (int m = 0; m < NT; ++m) res[m] = 0.0f;
        int k = 0;
        for (int i = 0; i + 1 < nchunks; i += 2) {
            step<F, BIAS, NT>(f0, ld, cp, a, wbuf, lds, lane, nc, stride, acc, res, k);
            step<F, BIAS, NT>(f1, ld, cp, a, wbuf, lds, lane, nc, stride, acc, res, k);
        }
        if (nchunks & 1) {  // only the wave's very last row can end here
            step<F, BIAS, NT>(f0, ld, cp, a, wbuf, lds, lane, nc, stride, acc, res, k);
            Fetch<F> t = f0;
            f0 = f1;
            f1 = t;
        }
        if (lane < k) {
#pragma unroll
            for (int m = 0; m < NT; ++m) a.y[(size_t)m * a.N + row0 + lane * stride] = res[m];
        }
    }
}

// ---------------------------------------------------------------- row-step
// Rows of at most 64*NC units (K <= 2048*NC, the decode projections of 1-8B
// models).  Lane l owns units l and l + 64 of EVERY row, so its activation
// limbs are read from LDS into registers once and stay there; the LDS then
// only carries the streamed weight bytes.  A step handles one whole row: its
// 16-byte pieces (NPR per lane) are spilled to the wave's LDS buffer, the row
// two steps ahead is fetched, each lane decodes its NC units and the row is
// reduced across the wave once.
template <int NPR>
struct RowFetch {
    uint4 v[NPR];
};

template <int NPR>
__device__ __forceinline__ void rfetch(RowFetch<NPR>& f, const GemvArgs& a, int row, int lane) {
    const uint8_t* g0 = a.w + (size_t)min(row, a.N - 1) * a.row_bytes;
    const int shift = (int)(reinterpret_cast<uintptr_t>(g0) & 15);
    const uint8_t* a0 = g0 - shift;
    const int n16 = (shift + a.row_bytes + 15) >> 4;
#pragma unroll
    for (int i = 0; i < NPR; ++i) f.v[i] = ldg128<true>(a0 + 16 * min(lane + 64 * i, n16 - 1));
}

template <int NPR>
__device__ __forceinline__ void rspill(const RowFetch<NPR>& f, uint8_t* wbuf, int lane) {
#pragma unroll
    for (int i = 0; i < NPR; ++i) reinterpret_cast<uint4*>(wbuf)[lane + 64 * i] = f.v[i];
}

// NT tokens: each unit is loaded and unpacked once and dotted with every
// token's limbs (L[m * NC + c]); bias_mode 2 adds bias[m N + row].
template <int F, int NC, int NPR, bool BIAS, int NT>
__device__ __forceinline__ void row_step(RowFetch<NPR>& f, int row, int prefetch_row,
                                         const GemvArgs& a, uint8_t* wbuf, const Limbs* L,
                                         int lane, float (&res)[NT], int& k) {
    __builtin_amdgcn_sched_barrier(0);
    rspill<NPR>(f, wbuf, lane);
    rfetch<NPR>(f, a, prefetch_row, lane);
    const uint8_t* g0 = a.w + (size_t)min(row, a.N - 1) * a.row_bytes;
    const uint8_t* rowp = wbuf + (reinterpret_cast<uintptr_t>(g0) & 15);
    float acc[NT];
#pragma unroll
    for (int m = 0; m < NT; ++m) acc[m] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int u = lane + 64 * c;
        const int ul = min(u, a.U - 1);
        const auto raw = Fmt<F>::template load<false>(rowp, ul);
#pragma unroll
        for (int m = 0; m < NT; ++m) {
            const float t = limb_dot<F>(raw, ul, L[m * NC + c]);
            acc[m] += u < a.U ? t : 0.0f;
        }
    }
#pragma unroll
    for (int m = 0; m < NT; ++m) {
        float s = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum(acc[m])), 63));
        if constexpr (BIAS) {
            const int r = min(row, a.N - 1);
            if (a.bias_mode == 2)
                s += ((const_fp)(uintptr_t)a.bias)[(size_t)m * a.N + r];
            else
                s += r < a.bias_len ? ((const_fp)(uintptr_t)a.bias)[r] : 0.0f;
        }
        res[m] = lane == k ? s : res[m];
    }
    ++k;
    __builtin_amdgcn_sched_barrier(0);
}

// NT tokens (a.M == NT): the records of all NT tokens are staged, and every
// lane holds each token's limbs of its units in registers.
template <int F, int NC, int NPR, bool BIAS, int WG, int D, int NT = 1>
__global__ __launch_bounds__(WG) void gemv1r_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int stride = gridDim.x * (WG / 64);
    const int first = __builtin_amdgcn_readfirstlane(blockIdx.x * (WG / 64) + wave);
    uint8_t* wbuf = lds + (size_t)NT * a.U * RECB + wave * (NPR * 1024);

    // D rows in flight per wave: buffer i always holds row (next + i * stride)
    XStage<Fmt<F>, WG> xs;
    // activation loads before weight loads
    stage_load<Fmt<F>, WG>(xs, a.x, NT * a.U, 0, NT > 1 ? a.U : 0, a.K);
    RowFetch<NPR> f[D];
#pragma unroll
    for (int i = 0; i < D; ++i) rfetch<NPR>(f[i], a, first + i * stride, lane);
    stage_build<Fmt<F>, WG>(lds, xs, a.x, NT * a.U, 0, NT > 1 ? a.U : 0, a.K);
    Limbs L[NT * NC];
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
        for (int c = 0; c < NC; ++c)
            read_limbs(L[m * NC + c], lds, m * a.U + min(lane + 64 * c, a.U - 1));

    int row = first;
    while (row < a.N) {
        const int rows_left = (a.N - 1 - row) / stride + 1;
        const int nrows = rows_left < D ? rows_left : min(64, rows_left) / D * D;
        const int row0 = row;
        float res[NT];
#pragma unroll
        for (int m = 0; m < NT; ++m) res[m] = 0.0f;
        int k = 0;
        if (nrows >= D) {
            for (int i = 0; i < nrows; i += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    row_step<F, NC, NPR, BIAS, NT>(f[j], row, row + D * stride, a, wbuf, L, lane, res,
                                               k);
                    row += stride;
                }
            }
        } else {  // the wave's last rows: buffers 0 .. nrows-1 hold them
#pragma unroll
            for (int j = 0; j < D - 1; ++j) {
                if (j < nrows) {
                    row_step<F, NC, NPR, BIAS, NT>(f[j], row, row + D * stride, a, wbuf, L, lane, res,
                                               k);
                    row += stride;
                }
            }
        }
        if (lane < k) {
#pragma unroll
            for (int m = 0; m < NT; ++m) a.y[(size_t)m * a.N + row0 + lane * stride] = res[m];
        }
    }
}

}  // namespace

template <int F, int W>
static const void* gemv1_fn_w(bool bias) {
    return bias ? reinterpret_cast<const void*>(&gemv1_kernel<F, true, W>)
                : reinterpret_cast<const void*>(&gemv1_kernel<F, false, W>);
}

template <int F>
static const void* gemv1_fn(bool bias, int wg) {
    switch (wg) {
        case 256: return gemv1_fn_w<F, 256>(bias);
        case 512: return gemv1_fn_w<F, 512>(bias);
        case 1024: return gemv1_fn_w<F, 1024>(bias);
        default: return nullptr;
    }
}

const void* gemv1_kernel_fn(int dtype, bool bias, int wg) {
    return with_format(dtype, (const void*)nullptr,
                       [&](auto f) { return gemv1_fn<decltype(f)::value>(bias, wg); });
}

template <int F>
static size_t lds_of(int U, int wg, int nt = 1) {
    return (size_t)nt * U * RECB + (size_t)(wg / 64) * Chunk<F>::WBUF;
}

// Several tokens (2 <= nt <= 4) at 1024 threads.
const void* gemv1_multi_fn(int dtype, bool bias, int nt, size_t* lds, int U) {
    return with_format(dtype, (const void*)nullptr, [&](auto f) -> const void* {
        constexpr int F = decltype(f)::value;
        *lds = lds_of<F>(U, 1024, nt);
        switch (nt) {
            case 2: return bias ? (const void*)&gemv1_kernel<F, true, 1024, 2>
                                : (const void*)&gemv1_kernel<F, false, 1024, 2>;
            case 3: return bias ? (const void*)&gemv1_kernel<F, true, 1024, 3>
                                : (const void*)&gemv1_kernel<F, false, 1024, 3>;
            case 4: return bias ? (const void*)&gemv1_kernel<F, true, 1024, 4>
                                : (const void*)&gemv1_kernel<F, false, 1024, 4>;
            default: return nullptr;
        }
    });
}

size_t gemv1_lds_bytes(int dtype, int U, int wg) {
    return with_format(dtype, (size_t)0, [&](auto f) { return lds_of<decltype(f)::value>(U, wg); });
}

constexpr int WGR = 512;

#ifndef FQ_ROW_DEPTH
#define FQ_ROW_DEPTH 3
#endif

template <int F, int NC, int NPR, int NT>
static const void* rfn3(bool bias) {
    constexpr int D = FQ_ROW_DEPTH;
    return bias ? reinterpret_cast<const void*>(&gemv1r_kernel<F, NC, NPR, true, WGR, D, NT>)
                : reinterpret_cast<const void*>(&gemv1r_kernel<F, NC, NPR, false, WGR, D, NT>);
}

template <int F, int NT>
static const void* rfn(int nc, int npr, bool bias) {
    if (nc == 1) {
        switch (npr) {
            case 1: return rfn3<F, 1, 1, NT>(bias);
            case 2: return rfn3<F, 1, 2, NT>(bias);
            case 3: return rfn3<F, 1, 3, NT>(bias);
        }
    } else if (nc == 2) {
        switch (npr) {
            case 2: return rfn3<F, 2, 2, NT>(bias);
            case 3: return rfn3<F, 2, 3, NT>(bias);
            case 4: return rfn3<F, 2, 4, NT>(bias);
            case 5: return rfn3<F, 2, 5, NT>(bias);
        }
    }
    return nullptr;
}

// Row-step variant for U <= 128 and nt = 1 or 2 tokens: returns nullptr when
// the shape does not fit.
const void* gemv1r_kernel_fn(int dtype, int U, int row_bytes, bool bias, int* npr_out,
                             size_t* lds_out, int* wg_out, int nt) {
    if (U > 128 || nt < 1 || nt > 2) return nullptr;
    const int nc = U > 64 ? 2 : 1;
    const int npr = (row_bytes + 16 + 1023) / 1024;
    const void* fn = with_format(dtype, (const void*)nullptr, [&](auto f) {
        constexpr int F = decltype(f)::value;
        return nt == 1 ? rfn<F, 1>(nc, npr, bias) : rfn<F, 2>(nc, npr, bias);
    });
    if (!fn) return nullptr;
    *npr_out = npr;
    *lds_out = (size_t)nt * U * RECB + (size_t)(WGR / 64) * npr * 1024;
    *wg_out = WGR;
    return fn;
}

hipError_t launch_raw(const void* fn, const GemvArgs& a, int grid, int wg, size_t lds,
                      hipStream_t st, int grid_y) {
    GemvArgs args = a;
    void* params[] = {&args};
    return hipLaunchKernel(fn, dim3(grid, grid_y), dim3(wg), params, lds, st);
}

hipError_t launch_gemv1(int dtype, const GemvArgs& a, int grid, int wg, hipStream_t st) {
    const void* fn = gemv1_kernel_fn(dtype, a.bias_mode != 0, wg);
    if (!fn) return hipErrorInvalidValue;
    GemvArgs args = a;
    void* params[] = {&args};
    return hipLaunchKernel(fn, dim3(grid), dim3(wg), params, gemv1_lds_bytes(dtype, a.U, wg), st);
}

}  // namespace fq
