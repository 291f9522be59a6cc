// fq_gemvt.hip -- batch-1 GEMV over the tiled aligned layout, one matrix row
// per lane: Q8_0 matrices of at least TILED_MIN_ROWS rows (fq_pack.h), the
// lm_head-type shapes where it beats the K-sliced kernel of fq_gemvp.hip
// (152064 x 3584: 87.5 against 97.5 us).  The 4-bit formats, whose K-sliced
// kernel dots the code nibbles in place (v_dot8_i32_i4), run faster there.
//
// The tiled layout groups rows in tiles of 16, storing the 16-byte pieces
// piece-major and row-minor, so pieces j .. j+3 of the tile's 16 rows are one
// contiguous 1 KiB run.  A wave steps through a tile four lane units (blocks)
// at a time: lane l works on row l & 15 and on block 4 g + (l >> 4) of step
// g, so one load instruction of the wave moves 1 KiB.
//
// Every lane accumulates its own row over its blocks: there is no cross-lane
// reduction in the inner loop.  The activation operand of a block is the
// same for the 16 lanes of a DPP row (16 matrix rows, one block): each wave
// builds the int8 limb records of its K range (x ~ s1 (a1 + a2 / 2^7 + a3 /
// 2^14), the batch-1 representation of fq_limbs.h) in a wave-private LDS
// area, reads the record of its block into two registers (lane k of the DPP
// row holds dword k, respectively 16 + k) and feeds dword k to v_dot4c_i32_i8
// through the DPP row_newbcast:k operand swizzle.
//
// A work-group of W waves splits K into W ranges and walks the tiles b,
// b + G, b + 2G, ... (G work-groups, a few per CU, the tiles dealt out in
// turn): each wave builds its records once, and its load pipeline runs on
// from one tile into the next.  At the end the four blocks' sums of a row are
// added across the DPP rows and the waves' sums in wave order, through LDS
// (deterministic).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_buf.h"
#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"
#include "fq_pack.h"

namespace fq {
namespace {

constexpr int TR = 16;      // rows per tile
constexpr int TREC = 128;   // bytes per activation record in a wave's LDS area
constexpr int MAXREC = 48;  // records a wave builds (its K range)
constexpr int NTMAX = 16;   // tiles per work-group
constexpr int WMAX = 16;    // waves per work-group

// Record layout (dwords): 0..7 a1, 8..15 a2, 16..23 a3 (dword i = slots
// 4i..4i+3), 24 s1, 25.. the group sums S[g].  A = dwords 0..15, B = 16..31.
struct Rec {
    int A, B;
};

// The record of local unit record index `rec` (lane-varying: the lane's unit).
__device__ __forceinline__ Rec read_rec(const uint8_t* area, int rec, int lane) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(area + TREC * rec) + (lane & 15);
    return Rec{(int)p[0], (int)p[16]};
}
// Dword 16 + K of the lane's record (the B register's lane K of its DPP row).
template <int K>
__device__ __forceinline__ float rec_f(const Rec& r) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, r.B, 0x150 + K, 0xF, 0xF, false));
}
__device__ __forceinline__ float rec_s1(const Rec& r) { return rec_f<8>(r); }
template <int G>
__device__ __forceinline__ float rec_S(const Rec& r) {
    return rec_f<9 + G>(r);
}

#define FQ_STR2(x) #x
#define FQ_STR(x) FQ_STR2(x)
#define FQ_DOTB(acc, src, w, k)                                                          \
    "v_dot4c_i32_i8_dpp " acc ", " src ", " w " row_newbcast:" FQ_STR(k)                 \
    " row_mask:0xf bank_mask:0xf\n"

// The three limb sums D1 = q . a1, D2 = q . a2, D3 = q . a3 of one record,
// q[i] the code dword of slots 4i..4i+3.  One asm block, because the
// compiler does not see the hazards of its instructions:
//  - a DPP instruction needs two wait states after any VALU write of ANY VGPR
//    it reads, its accumulator included: the three sums are interleaved (each
//    accumulator is written two instructions before it is read again) and
//    the block starts with s_nop 1 for the code dwords the compiler just wrote;
//  - a VALU instruction other than the same dot needs three wait states to
//    read a VGPR a dot instruction wrote: the block ends with s_nop 2, before
//    the compiler's code reads the sums.
// |D| <= 32 * 128 * 127 for int8 codes.
__device__ __forceinline__ void sums32(const Rec& r, const int (&q)[8], int& d1, int& d2, int& d3) {
    int e1, e2, e3;
    asm("s_nop 1\n"
        "v_mov_b32 %0, 0\n"
        "v_mov_b32 %1, 0\n"
        "v_mov_b32 %2, 0\n"
        FQ_DOTB("%0", "%3", "%5", 0) FQ_DOTB("%1", "%3", "%5", 8) FQ_DOTB("%2", "%4", "%5", 0)
        FQ_DOTB("%0", "%3", "%6", 1) FQ_DOTB("%1", "%3", "%6", 9) FQ_DOTB("%2", "%4", "%6", 1)
        FQ_DOTB("%0", "%3", "%7", 2) FQ_DOTB("%1", "%3", "%7", 10) FQ_DOTB("%2", "%4", "%7", 2)
        FQ_DOTB("%0", "%3", "%8", 3) FQ_DOTB("%1", "%3", "%8", 11) FQ_DOTB("%2", "%4", "%8", 3)
        FQ_DOTB("%0", "%3", "%9", 4) FQ_DOTB("%1", "%3", "%9", 12) FQ_DOTB("%2", "%4", "%9", 4)
        FQ_DOTB("%0", "%3", "%10", 5) FQ_DOTB("%1", "%3", "%10", 13) FQ_DOTB("%2", "%4", "%10", 5)
        FQ_DOTB("%0", "%3", "%11", 6) FQ_DOTB("%1", "%3", "%11", 14) FQ_DOTB("%2", "%4", "%11", 6)
        FQ_DOTB("%0", "%3", "%12", 7) FQ_DOTB("%1", "%3", "%12", 15) FQ_DOTB("%2", "%4", "%12", 7)
        "s_nop 2\n"
        : "=&v"(e1), "=&v"(e2), "=&v"(e3)
        : "v"(r.A), "v"(r.B), "v"(q[0]), "v"(q[1]), "v"(q[2]), "v"(q[3]), "v"(q[4]), "v"(q[5]),
          "v"(q[6]), "v"(q[7]));
    d1 = e1;
    d2 = e2;
    d3 = e3;
}

// Weight loads are raw buffer loads (one 32-bit address space per matrix,
// bounds-checked by the hardware): the uniform part of an address -- the
// tile's offset, the plane and the piece index times the tile's rows -- is the
// scalar soffset operand and the lane adds its 32-bit voffset, so no vector
// or 64-bit scalar address arithmetic is spent per load (fq_buf.h).

// A tile as the loads see it: its matrix, its byte offset there, its rows.
struct TileRef {
    Buf b;
    uint32_t off;
    int R;
};
// soffset of piece j of the plane at row offset o (bytes) of a tile
__device__ __forceinline__ uint32_t pso(const TileRef& t, uint32_t o, uint32_t j) {
    return t.off + (o + 16 * j) * (uint32_t)t.R;
}

// Format traits.  One step ("group") g covers lane units 4g .. 4g+3; lane l
// works on unit 4g + q, q = l >> 4, of row r = l & 15.  NREC activation
// records per unit, GS slots per group sum, k_of(record, slot) the element of
// slot s of a record, NB register buffers in the load pipeline.
template <int F>
struct T;

template <>
struct T<Q8_0> {  // planes: qs[0,16) (U x 16), qs[16,32) (U x 16), d (U x 2, padded)
    static constexpr int NREC = 1, GS = 32, NB = 6;
    struct Raw {
        uint4 q0, q1;
        uint32_t d;
    };
    __device__ static int k_of(int w, int s) { return 32 * w + s; }
    __device__ static void load(Raw& f, const TileRef& t, int r, int q, int g, int U) {
        f.q0 = bld128(t.b, pso(t, 0, 4 * g), 16 * (q * t.R + r));
        f.q1 = bld128(t.b, pso(t, 16 * U, 4 * g), 16 * (q * t.R + r));
        f.d = bld16(t.b, pso(t, 32 * U, g >> 1), 16 * r + 2 * (4 * (g & 1) + q));
    }
    __device__ static float dot(const Raw& f, const Rec (&rr)[NREC], int) {
        const Rec& rc = rr[0];
        const int q[8] = {(int)f.q0.x, (int)f.q0.y, (int)f.q0.z, (int)f.q0.w,
                          (int)f.q1.x, (int)f.q1.y, (int)f.q1.z, (int)f.q1.w};
        int d1, d2, d3;
        sums32(rc, q, d1, d2, d3);
        return f16_hw(f.d) * rec_s1(rc) * limb_sum(d1, d2, d3);
    }
};

// The limb records of lane units [u0, u0 + nu) of the wave's area: eight
// lanes per record, lane i of a record owning slots 4i .. 4i+3.  xload()
// issues the activation loads (before the weight loads, so that the build
// waits for nothing but them in the in-order memory counter); build() writes
// the records.
constexpr int XP = MAXREC / 8;  // activation float4s per lane at most

template <int F>
__device__ __forceinline__ void xload(float4 (&xv)[XP], const float* __restrict__ x, int u0,
                                      int nu, int lane) {
    using Tr = T<F>;
    const int tasks = 8 * nu * Tr::NREC, w0 = u0 * Tr::NREC;
    // all XP loads are issued (past the wave's records: its last one again),
    // so the compiler can count them and the build waits for these alone
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        const int t = min(64 * p + lane, max(tasks - 1, 0));
        xv[p] = *reinterpret_cast<const float4*>(x + Tr::k_of(w0 + (t >> 3), 4 * (t & 7)));
    }
}

template <int F>
__device__ __forceinline__ void build(uint8_t* area, const float4 (&xv)[XP], int nu, int lane) {
    using Tr = T<F>;
    const int tasks = 8 * nu * Tr::NREC;
#pragma unroll
    for (int p = 0; p < XP; ++p) {
        if (64 * p < tasks) {  // wave-uniform: all 64 lanes take part in the DPP reductions
            const int t = 64 * p + lane, i = t & 7;
            const LimbQuad lq = limb_quad<Tr::GS>(xv[p]);
            if (t < tasks) {
                uint32_t* rec = reinterpret_cast<uint32_t*>(area + TREC * (t >> 3));
                rec[i] = lq.a1;
                rec[8 + i] = lq.a2;
                rec[16 + i] = lq.a3;
                if (i == 0) rec[24] = __builtin_bit_cast(uint32_t, lq.s1);
                if ((4 * i) % Tr::GS == 0)
                    rec[25 + (4 * i) / Tr::GS] = __builtin_bit_cast(uint32_t, lq.gs);
            }
        }
    }
}

// Tile t: its matrix m, byte offset there, first output row and rows.  ONE:
// one matrix of a.N rows.  PAIR: the gate (w) and up (w2) matrices, a.N rows
// each, walked together (the same offset in both).  CAT: w, w2, w3 stacked
// (n1, n2 and the rest of a.N rows).
struct TileSel {
    int m;
    uint32_t off;
    int row0, R;
};

template <int MODE>
__device__ __forceinline__ TileSel select_tile(const TArgs& a, int t) {
    const uint32_t RB = (uint32_t)a.row_bytes;
    if constexpr (MODE == 2) {
        const int t1 = (a.n1 + TR - 1) / TR, t2 = (a.n2 + TR - 1) / TR;
        int m, rows, lt, r0;
        if (t < t1) {
            m = 0, rows = a.n1, lt = t, r0 = 0;
        } else if (t < t1 + t2) {
            m = 1, rows = a.n2, lt = t - t1, r0 = a.n1;
        } else {
            m = 2, rows = a.N - a.n1 - a.n2, lt = t - t1 - t2, r0 = a.n1 + a.n2;
        }
        return TileSel{m, (uint32_t)lt * TR * RB, r0 + TR * lt, min(TR, rows - TR * lt)};
    } else {
        return TileSel{0, (uint32_t)t * TR * RB, TR * t, min(TR, a.N - TR * t)};
    }
}

// MODE 0 (ONE), 1 (PAIR: y = silu(gate) * up), 2 (CAT: fused QKV).  The
// work-group has blockDim.x / 64 waves (at most WMAX).  Work-group b owns K
// split b % S of the tiles b / S, b / S + GT, ... (GT = gridDim.x / S).
template <int F, int MODE>
__global__ __launch_bounds__(64 * WMAX, 4) void gemvt_kernel(TArgs a) {
    using Tr = T<F>;
    constexpr int NB = Tr::NB;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int NV = MODE == 1 ? 2 : 1;  // row sums per lane
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, q = lane >> 4, r16 = lane & 15;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int GT = gridDim.x, slot = blockIdx.x;
    const int nt = (a.T - slot + GT - 1) / GT;  // tiles of this work-group
    // this split's steps, then this wave's share of them
    const int g0 = (int)((int64_t)a.GR * wv / W), g1 = (int)((int64_t)a.GR * (wv + 1) / W);
    const int ng = g1 - g0;
    uint8_t* area = lds + (size_t)wv * a.recs * TREC;
    // per tile, matrix and wave: each lane's sum over its units of the wave's K range
    float* part = reinterpret_cast<float*>(lds + (size_t)W * a.recs * TREC);

    if (ng > 0) {
        // Items (tile k, step g, matrix v), v fastest, then g, then k; item i
        // loads into buffer i % NB.  Every load is issued (past the end: the
        // last item again), so the compiler waits for exactly one buffer's
        // loads.
        const int items = nt * ng * NV;
        struct Cur {
            int k, g, v;
        };
        auto advance = [&](Cur& c) {
            if (++c.v == NV) {
                c.v = 0;
                if (++c.g == g1) {
                    c.g = g0;
                    ++c.k;
                }
            }
        };
        // one buffer per matrix (the host checks each is under 4 GiB)
        const uint32_t mb = (uint32_t)((int64_t)a.N * a.row_bytes);
        Buf bufs[3];
        if constexpr (MODE == 2) {
            bufs[0] = make_buf(a.w, (uint32_t)((int64_t)a.n1 * a.row_bytes));
            bufs[1] = make_buf(a.w2, (uint32_t)((int64_t)a.n2 * a.row_bytes));
            bufs[2] = make_buf(a.w3, (uint32_t)((int64_t)(a.N - a.n1 - a.n2) * a.row_bytes));
        } else {
            bufs[0] = make_buf(a.w, mb);
            bufs[1] = make_buf(MODE == 1 ? a.w2 : a.w, mb);
        }
        // the load cursor's tile, looked up when the cursor enters a tile
        int lk = -1;
        TileSel lt{};
        auto ld = [&](typename Tr::Raw& f, Cur c) {
            if (c.k >= nt) c = Cur{nt - 1, g1 - 1, NV - 1};
            if (c.k != lk) {  // wave-uniform
                lk = c.k;
                lt = select_tile<MODE>(a, slot + c.k * GT);
            }
            const TileRef tr{bufs[MODE == 1 ? c.v : lt.m], lt.off, lt.R};
            Tr::load(f, tr, min(r16, lt.R - 1), q, c.g, a.U);
        };
        typename Tr::Raw f[NB];
        {
            // a CU's address unit takes one 1 KiB load instruction every ~16
            // cycles, so a wave that issued all its first loads before the
            // record build would queue its build behind them: one buffer
            // goes out first, the others after the build
            float4 xv[XP];
            xload<F>(xv, a.x, 4 * g0, 4 * ng, lane);
            Cur lc{0, g0, 0};
            ld(f[0], lc);
            build<F>(area, xv, 4 * ng, lane);
#pragma unroll
            for (int b = 1; b < NB; ++b) {
                advance(lc);
                ld(f[b], lc);
            }
        }
        Cur lc{0, g0, 0}, cc{0, g0, 0};
        for (int b = 0; b < NB; ++b) advance(lc);
        // the activation records of the unit of step g (one item ahead, so the
        // LDS latency hides behind the item before)
        auto rd = [&](Rec (&rr)[Tr::NREC], int g) {
#pragma unroll
            for (int j = 0; j < Tr::NREC; ++j)
                rr[j] = read_rec(area, (4 * (g - g0) + q) * Tr::NREC + j, lane);
        };
        Rec rc[Tr::NREC];
        rd(rc, g0);
        float acc[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
        for (int i = 0; i < items; i += NB) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (i + b < items) {  // wave-uniform
                    Cur cn = cc;
                    advance(cn);
                    Rec rn[Tr::NREC];
                    rd(rn, cn.k < nt ? cn.g : cc.g);
                    const float d = Tr::dot(f[b], rc, lane);
                    if constexpr (NV == 2) acc[cc.v] += d;
                    else acc[0] += d;
                    if (cc.g == g1 - 1 && cc.v == NV - 1) {  // the tile's last item
#pragma unroll
                        for (int v = 0; v < NV; ++v) {
                            part[((cc.k * NV + v) * W + wv) * 64 + lane] = acc[v];
                            acc[v] = 0.0f;
                        }
                    }
                    cc = cn;
#pragma unroll
                    for (int j = 0; j < Tr::NREC; ++j) rc[j] = rn[j];
                }
                ld(f[b], lc);
                advance(lc);
            }
        }
    } else {
        for (int k = 0; k < nt; ++k)
#pragma unroll
            for (int v = 0; v < NV; ++v) part[((k * NV + v) * W + wv) * 64 + lane] = 0.0f;
    }
    __syncthreads();
    // tile k is finished by wave k % W: its waves' sums in wave order
    for (int k = wv; k < nt; k += W) {
        const TileSel ts = select_tile<MODE>(a, slot + k * GT);
        if (lane >= ts.R) continue;
        float s[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            // wave by wave, each wave's four units of the row in order
            const float* pv = part + (size_t)(k * NV + v) * W * 64 + lane;
            s[v] = pv[0] + pv[16] + pv[32] + pv[48];
            for (int i = 1; i < W; ++i)
                s[v] += pv[i * 64] + pv[i * 64 + 16] + pv[i * 64 + 32] + pv[i * 64 + 48];
        }
        const int n = ts.row0 + lane;
        if constexpr (MODE == 1) {
            a.y[n] = s[0] / (1.0f + expf(-s[0])) * s[1];  // silu(gate) * up
        } else {
            float v = s[0];
            if (a.bias && n < a.bias_len) v += a.bias[n];  // added to the finished row sum
            a.y[n] = v;
        }
    }
}

template <int F>
const void* tfn_mode(int mode) {
    switch (mode) {
        case 0: return reinterpret_cast<const void*>(&gemvt_kernel<F, 0>);
        case 1: return reinterpret_cast<const void*>(&gemvt_kernel<F, 1>);
        case 2: return reinterpret_cast<const void*>(&gemvt_kernel<F, 2>);
    }
    return nullptr;
}

}  // namespace

int gemvt_units(int, int K) { return K / 32; }
int gemvt_max_records() { return MAXREC; }
int gemvt_record_bytes() { return TREC; }
int gemvt_max_tiles() { return NTMAX; }
int gemvt_max_waves() { return WMAX; }
int gemvt_tile_rows() { return TR; }

const void* gemvt_kernel_fn(int dtype, int mode) {
    switch (dtype) {
        case Q8_0: return tfn_mode<Q8_0>(mode);
    }
    return nullptr;
}

hipError_t launch_gemvt(const void* fn, const TArgs& a, int grid, int W, size_t lds,
                        hipStream_t st) {
    void* args[] = {const_cast<TArgs*>(&a)};
    return hipLaunchKernel(fn, dim3(grid), dim3(64 * W), args, lds, st);
}

}  // namespace fq
