// fq_gemvp.hip -- batch-1 GEMV over the aligned device layout (fq_pack.h).
//
// Every quant payload a lane needs is a 16-byte-aligned run, so weights go
// straight from HBM to registers with coalesced global_load_dwordx4 (plus
// small dense loads of the scale arrays): no LDS staging of weights.  As in
// the row-step kernel of fq_gemv1.hip, lane l owns the same "lane units" of
// every row (l and l + 64), its activation limbs stay in registers, and a
// wave walks its rows with D rows of weight bytes in flight, reducing each row
// once with DPP and storing 64 row results at a time.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"
#include "fq_pack.h"

namespace fq {
namespace {

// Packed traits: a "lane unit" is what one lane decodes per row step; it spans
// NREC 32-slot activation records.  Map::k_of(w, s) places slot s of record
// w for staging; NG is the number of offset groups per record.
template <int F>
struct Pk;

template <>
struct Pk<Q4_0> {
    static constexpr int NREC = 1, NG = 1;
    using Raw = Fmt<Q4_0>::Raw;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg16<true>(row + 16 * U + 2 * v), ldg128<true>(row + 16 * v)};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        return limb_dot<Q4_0>(r, v, L[0]);
    }
};

template <>
struct Pk<Q4_1> {
    static constexpr int NREC = 1, NG = 1;
    using Raw = Fmt<Q4_1>::Raw;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg32<true>(row + 16 * U + 4 * v), ldg128<true>(row + 16 * v)};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        return limb_dot<Q4_1>(r, v, L[0]);
    }
};

template <>
struct Pk<Q8_0> {
    static constexpr int NREC = 1, NG = 1;
    using Raw = Fmt<Q8_0>::Raw;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg16<true>(row + 32 * U + 2 * v), ldg128<true>(row + 16 * v),
                   ldg128<true>(row + 16 * U + 16 * v)};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        return limb_dot<Q8_0>(r, v, L[0]);
    }
};

// Q4_K lane unit v = 4 s + g: the 32 qs bytes of sub-block pair g of super-
// block s (64 weights).  Record 2v holds the low nibbles (sub-block 2g), record
// 2v + 1 the high nibbles (sub-block 2g + 1), 32 slots each in element order.
struct Q4KP {
    uint4 hdr, q0, q1;  // d dmin scales[12]; qs[32g .. 32g+16); qs[32g+16 .. 32g+32)
};

template <>
struct Pk<Q4_K> {  // planes q0, q1 (U x 16 each), then the headers (S x 16)
    static constexpr int NREC = 2, NG = 1;
    using Raw = Q4KP;
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        return Raw{ldg128<true>(row + 32 * U + 16 * (v >> 2)), ldg128<true>(row + 16 * v),
                   ldg128<true>(row + 16 * U + 16 * v)};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        int D[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int lo = (int)(w[i] & 0x0F0F0F0Fu), hi = (int)((w[i] >> 4) & 0x0F0F0F0Fu);
            D[0][0] = sdot4(lo, L[0].l1[i], D[0][0]);
            D[1][0] = sdot4(lo, L[0].l2[i], D[1][0]);
            D[2][0] = sdot4(lo, L[0].l3[i], D[2][0]);
            D[0][1] = sdot4(hi, L[1].l1[i], D[0][1]);
            D[1][1] = sdot4(hi, L[1].l2[i], D[1][1]);
            D[2][1] = sdot4(hi, L[1].l3[i], D[2][1]);
        }
        const float d = f16_hw(r.hdr.x & 0xFFFFu), dmin = f16_hw(r.hdr.x >> 16);
        uint32_t sa, ma, sb, mb;
        Fmt<Q4_K>::scale_min(r.hdr, v & 3, sa, ma, sb, mb);
        float acc = -(dmin * (float)ma) * L[0].S[0];
        acc = __builtin_fmaf(-(dmin * (float)mb), L[1].S[0], acc);
        acc = __builtin_fmaf(d * (float)sa * L[0].s1, limb_sum(D[0][0], D[1][0], D[2][0]), acc);
        return __builtin_fmaf(d * (float)sb * L[1].s1, limb_sum(D[0][1], D[1][1], D[2][1]), acc);
    }
};

// Q6_K lane unit v = 4 s + p: 64 weights, quarter p = 2n + h of super-block
// s: columns l = 16h .. 16h+15 of 128-half n, all four 32-row groups g.  Its
// two activation records are groups {0,1} and {2,3}: slot 16 g' + e of record
// 2v + r holds element 256 s + 128 n + 32 (2r + g') + 16 h + e.
struct Q6P {
    uint4 lo, hi, qh;  // ql[64n+16h..], ql[64n+32+16h..], qh[32n+16h..]
    uint2 sc;          // sc[8n .. 8n+8)
    uint32_t d;
};

template <>
struct Pk<Q6_K> {
    static constexpr int NREC = 2, NG = 2;
    using Raw = Q6P;
    __device__ static int k_of(int w, int s) {
        const int v = w >> 1, r = w & 1, sb = v >> 2, p = v & 3, n = p >> 1, h = p & 1;
        const int g = 2 * r + (s >> 4), e = s & 15;
        return 256 * sb + 128 * n + 32 * g + 16 * h + e;
    }
    // U here = lane units per row = K / 64; super-blocks S = U / 4.
    __device__ static Raw load(const uint8_t* row, int v, int U) {
        const int S = U >> 2, sb = v >> 2, n = (v & 3) >> 1;
        return Raw{ldg128<true>(row + 16 * v), ldg128<true>(row + 16 * U + 16 * v),
                   ldg128<true>(row + 32 * U + 16 * v),
                   ldg64<true>(row + 192 * S + 16 * sb + 8 * n),
                   ldg16<true>(row + 208 * S + 2 * sb)};
    }
    __device__ static float dot(const Raw& r, int v, const Limbs* L) {
        const uint32_t A[4] = {r.lo.x, r.lo.y, r.lo.z, r.lo.w};
        const uint32_t B[4] = {r.hi.x, r.hi.y, r.hi.z, r.hi.w};
        const uint32_t H[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        int D[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q1 = (int)((A[i] & 0x0F0F0F0Fu) | ((H[i] & 0x03030303u) << 4));
            const int q2 = (int)((B[i] & 0x0F0F0F0Fu) | ((H[i] & 0x0C0C0C0Cu) << 2));
            const int q3 = (int)(((A[i] >> 4) & 0x0F0F0F0Fu) | (H[i] & 0x30303030u));
            const int q4 = (int)(((B[i] >> 4) & 0x0F0F0F0Fu) | ((H[i] >> 2) & 0x30303030u));
#pragma unroll
            for (int l = 0; l < 3; ++l) {
                const int* la = l == 0 ? L[0].l1 : l == 1 ? L[0].l2 : L[0].l3;
                const int* lb = l == 0 ? L[1].l1 : l == 1 ? L[1].l2 : L[1].l3;
                D[l][0] = sdot4(q1, la[i], D[l][0]);
                D[l][1] = sdot4(q2, la[4 + i], D[l][1]);
                D[l][2] = sdot4(q3, lb[i], D[l][2]);
                D[l][3] = sdot4(q4, lb[4 + i], D[l][3]);
            }
        }
        const int h = v & 1;  // sub-scale index l/16 = h: sc[8n + h + 2g]
        int sc[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t = h + 2 * g;
            const uint32_t word = t < 4 ? r.sc.x : r.sc.y;
            sc[g] = (int)(int8_t)((word >> (8 * (t & 3))) & 0xFFu);
        }
        int Ea[3], Eb[3];
#pragma unroll
        for (int l = 0; l < 3; ++l) {
            Ea[l] = __mul24(sc[0], D[l][0]) + __mul24(sc[1], D[l][1]);
            Eb[l] = __mul24(sc[2], D[l][2]) + __mul24(sc[3], D[l][3]);
        }
        float sS = (float)sc[0] * L[0].S[0];
        sS = __builtin_fmaf((float)sc[1], L[0].S[1], sS);
        sS = __builtin_fmaf((float)sc[2], L[1].S[0], sS);
        sS = __builtin_fmaf((float)sc[3], L[1].S[1], sS);
        const float P = __builtin_fmaf(L[1].s1, limb_sum(Eb[0], Eb[1], Eb[2]),
                                       L[0].s1 * limb_sum(Ea[0], Ea[1], Ea[2]));
        return f16_hw(r.d) * __builtin_fmaf(-32.0f, sS, P);
    }
};

// Work distribution.  Work-group g owns the contiguous rows [N g / G,
// N (g+1) / G); within it, waves claim chunks of CR rows through an LDS
// counter, so a wave that the SIMD arbiter serves less often simply takes
// fewer chunks (static striding left waves of one CU finishing up to 20%
// apart).  A chunk is processed slice-major: for each K-slice of 64*NL lane
// units, the slice's activation limbs are loaded into registers and that
// slice of every row of the chunk is accumulated into the row's lane of the
// result register; slices are added in slice order, so the result is
// deterministic.  Finished chunk results go to an LDS row buffer that the
// work-group writes to y, coalesced, when its rows are done: the pipelined
// loop issues no global stores and no global atomics.
constexpr int CR = 2;          // rows per claimed chunk (at least)
constexpr int YBUF = 4096;     // rows of results a work-group buffers in LDS

struct Chunk {
    int r0, n;  // first row, rows (0: no more work)
};

struct It {
    int r0, n, s, r;  // chunk, slice, row within chunk
};

// Uniform claim of the next chunk from the work-group's LDS counter.
__device__ __forceinline__ Chunk claim(int* ctr, int hi, int cr, int lane) {
    int r0 = 0;
    if (lane == 0) r0 = atomicAdd(ctr, cr);
    r0 = __builtin_amdgcn_readfirstlane(r0);
    return Chunk{r0, r0 < hi ? min(cr, hi - r0) : 0};
}

// The chunk the load side has claimed beyond the compute side's chunk (n = 0:
// none).  A chunk spans at least D steps (the host picks CR so) and only a
// work-group's last chunk is shorter, so the load side, D steps ahead, is at
// most one chunk ahead and one slot suffices.  Uniform scalars only: an
// indexed queue would live in scratch memory, whose loads share the in-order
// vector memory counter with the weight loads and drain them.
struct Next {
    int r0, n;
};

template <int F, int NL>
__device__ __forceinline__ void pload(typename Pk<F>::Raw (&f)[NL], const GemvArgs& a,
                                      const It& t, int lane) {
    const uint8_t* r = a.w + (size_t)min(t.r0 + t.r, a.N - 1) * a.row_bytes;
    const int v0 = t.s * 64 * NL;
#pragma unroll
    for (int c = 0; c < NL; ++c) f[c] = Pk<F>::load(r, min(v0 + lane + 64 * c, a.U - 1), a.U);
}

template <int F, int NL>
__device__ __forceinline__ void load_slice_limbs(Limbs (&L)[NL][Pk<F>::NREC], const uint8_t* lds,
                                                 int s, int U, int lane) {
#pragma unroll
    for (int c = 0; c < NL; ++c)
#pragma unroll
        for (int r = 0; r < Pk<F>::NREC; ++r)
            read_limbs(L[c][r], lds, min(s * 64 * NL + lane + 64 * c, U - 1) * Pk<F>::NREC + r);
}

__device__ __forceinline__ void advance_load(It& ld, Next& q, int ns, int cr, int* ctr, int hi,
                                             int lane) {
    if (ld.n == 0) return;
    if (++ld.r == ld.n) {
        ld.r = 0;
        if (++ld.s == ns) {
            ld.s = 0;
            const Chunk c = claim(ctr, hi, cr, lane);
            ld.r0 = c.r0;
            ld.n = c.n;
            if (c.n > 0) q = Next{c.r0, c.n};
        }
    }
}

// One step of the compute side (slice cp.s of row cp.r0 + cp.r), then the
// loads of the load side's step into the same registers.
template <int F, int NL, int D, bool BIAS>
__device__ __forceinline__ void pstep(typename Pk<F>::Raw (&f)[NL], It& cp, It& ld, Next& q,
                                      int ns, int cr, int* ctr, int hi, const GemvArgs& a,
                                      Limbs (&L)[NL][Pk<F>::NREC], const uint8_t* lds,
                                      float* ybuf, int lo, int lane, float& res) {
    __builtin_amdgcn_sched_barrier(0);
    if (cp.r == 0) load_slice_limbs<F, NL>(L, lds, cp.s, a.U, lane);  // wave-uniform
    const int v0 = cp.s * 64 * NL;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NL; ++c) {
        const int v = v0 + lane + 64 * c;
        const float t = Pk<F>::dot(f[c], min(v, a.U - 1), L[c]);
        acc += v < a.U ? t : 0.0f;
    }
    pload<F, NL>(f, a, ld, lane);
    float s = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum(acc)), 63));
    if constexpr (BIAS) {
        if (cp.s == 0) {
            const int r = cp.r0 + cp.r;
            s += r < a.bias_len ? ((const_fp)(uintptr_t)a.bias)[r] : 0.0f;
        }
    }
    res = lane == cp.r ? res + s : res;
    // advance the compute side; a finished chunk goes to the LDS row buffer
    if (++cp.r == cp.n) {
        cp.r = 0;
        if (++cp.s == ns) {
            cp.s = 0;
            if (lane < cp.n) ybuf[cp.r0 - lo + lane] = res;
            res = 0.0f;
            cp.r0 = q.r0;
            cp.n = q.n;
            q.n = 0;
        }
    }
    // after the compute side has taken the pending chunk, so the slot is free
    advance_load(ld, q, ns, cr, ctr, hi, lane);
    __builtin_amdgcn_sched_barrier(0);
}

template <int F, int NL, int D, bool BIAS, int WG>
__global__ __launch_bounds__(WG) void gemvp_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int ctr;
    __shared__ float ybuf[YBUF];
    using P = Pk<F>;
    const int lane = threadIdx.x & 63;
    const int ns = (a.U + 64 * NL - 1) / (64 * NL);
    const int G = gridDim.x, g = blockIdx.x;
    const int lo_all = (int)((int64_t)a.N * g / G), hi_all = (int)((int64_t)a.N * (g + 1) / G);

    // the host sizes the grid so a work-group owns at most YBUF rows
    const int lo = lo_all, hi = hi_all;
    if (threadIdx.x == 0) ctr = lo;
    XStage<P, WG> xs;
    stage_load<P, WG>(xs, a.x, a.Uc, 0);  // activation loads before any weight load
    __syncthreads();
    // the first D steps' weight loads; the limb records are built while they
    // are in flight
    const int cr = max(CR, (D + ns - 1) / ns);  // a chunk spans >= D steps
    Next q{0, 0};
    const Chunk c0 = claim(&ctr, hi, cr, lane);
    It ld{c0.r0, c0.n, 0, 0}, cp{c0.r0, c0.n, 0, 0};
    typename P::Raw f[D][NL];
#pragma unroll
    for (int j = 0; j < D; ++j) {
        pload<F, NL>(f[j], a, ld, lane);
        advance_load(ld, q, ns, cr, &ctr, hi, lane);
    }
    stage_build<P, WG>(lds, xs, a.x, a.Uc, 0);
    Limbs L[NL][P::NREC];
    float res = 0.0f;
    while (cp.n > 0) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            if (cp.n > 0)
                pstep<F, NL, D, BIAS>(f[j], cp, ld, q, ns, cr, &ctr, hi, a, L, lds, ybuf, lo, lane,
                                      res);
        }
    }
    __syncthreads();
    for (int r = threadIdx.x; r < hi - lo; r += WG) a.y[lo + r] = ybuf[r];
}

constexpr int WGP = 512;
constexpr int DP = 3;

template <int F, int NL>
const void* pfn2(bool bias) {
    return bias ? reinterpret_cast<const void*>(&gemvp_kernel<F, NL, DP, true, WGP>)
                : reinterpret_cast<const void*>(&gemvp_kernel<F, NL, DP, false, WGP>);
}

template <int F>
const void* pfn(int nl, bool bias) {
    return nl == 1 ? pfn2<F, 1>(bias) : pfn2<F, 2>(bias);
}

}  // namespace

// Lane units per row and activation records for a packed GEMV of length K.
void gemvp_geometry(int dtype, int K, int* units, int* records) {
    if (dtype == Q6_K || dtype == Q4_K) {
        *units = K / 64;
        *records = K / 32;
    } else {
        *units = K / 32;
        *records = K / 32;
    }
}

// Kernel for a row of `units` lane units: K-slices of 64 units (one per lane)
// or, for the 32-weight units of long rows, of 128 (two per lane).
const void* gemvp_kernel_fn(int dtype, int units, int records, bool bias, size_t* lds, int* wg) {
    // 64-weight lane units (Q4_K, Q6_K) keep one unit per lane: two would
    // need ~230 registers and halve the resident waves
    const int nl = (units <= 64 || dtype == Q4_K || dtype == Q6_K) ? 1 : 2;
    const void* fn = nullptr;
    switch (dtype) {
        case Q4_0: fn = pfn<Q4_0>(nl, bias); break;
        case Q4_1: fn = pfn<Q4_1>(nl, bias); break;
        case Q8_0: fn = pfn<Q8_0>(nl, bias); break;
        case Q4_K: fn = pfn<Q4_K>(nl, bias); break;
        case Q6_K: fn = pfn<Q6_K>(nl, bias); break;
    }
    *lds = (size_t)records * RECB;
    *wg = WGP;
    return fn;
}

}  // namespace fq
