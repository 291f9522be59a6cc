// fq_mmqi.hip -- small-batch (2 <= M <= 8 tokens per pass) Q4_K matmul on the
// int8 matrix cores, over the GGUF bytes.
//
// The weight rows are cut into tiles of 16.  A wave handles one (tile,
// super-block) "step" at a time: it loads the 16 rows' 144-byte super-blocks
// (144 16-byte pieces, three per lane, coalesced along each row), writes them
// to its LDS panel in the same order, and runs per 32-element sub-block three
// MFMAs v_mfma_i32_16x16x32_i8, one per activation limb:
//
//   A (weights, 16 x 32): lane l = 16 q + r holds row r's eight quants of
//     positions 8 q .. 8 q + 7 of the sub-block: the low nibbles of
//     qs[32 j + 8 q, +8) for sub-block 2 j, the high nibbles for 2 j + 1.
//   B (activations, 32 x 16): lane l = 16 q + c holds limb t of token c at
//     the same positions (zeros for c >= M).
//   D_t[r][c] = sum over the sub-block of q * a_t(x_c): exact int32.
//
// With the limbs x ~= s1 (a1 + a2 2^-7 + a3 2^-14) of each token's 32-element
// sub-block, y[c][r] gains
//     d sc_{r,sb} s1_{c,sb} (D_1 2^14 + D_2 2^7 + D_3) 2^-14 - dmin m_{r,sb} S_{c,sb}
// (matmul.cpp:340-377: w = d sc q - dmin m).  The three limb sums combine in
// int32 (|D_1| <= 32 * 127 * 15, so D_1 2^14 fits), then one conversion and
// one FMA per output element; the min terms, a 16 x 8 by 8 x 16 product per
// super-block, take two v_mfma_f32_16x16x4f32.  Lane l of D holds rows 4 (l / 16) .. +3 of
// token l % 16, so every lane owns distinct outputs and no cross-lane
// reduction is needed.  Per step the lanes (r, q) decode the header of row r
// for sub-blocks 2 q, 2 q + 1 into a per-wave LDS table of d sc 2^-14.
//
// Work distribution is that of a persistent batch-1 kernel: work-group g owns
// the tiles [T g / G, T (g+1) / G); its (tile, super-block) steps, tile-major,
// are cut into chunks of C >= DT steps; wave w starts on chunk w and claims
// further chunks from an LDS counter.  A wave keeps DT steps of loads in
// flight.  Partial sums for the part of a chunk inside one tile go to an LDS
// slot of (tile, chunk); the work-group adds each output's slots in chunk
// order at the end, so results do not depend on which wave took which chunk.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fq_formats.h"
#include "fq_kernels.h"
#include "fq_limbs.h"

namespace fq {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int DT = 3;  // steps in flight per wave

// Partial-sum slots per tile: one per chunk that can overlap the tile.
__host__ __device__ inline int slots(int S, int C) { return (S + C - 1) / C + 1; }

// B staging: limb t of token m at positions 8 q .. 8 q + 7 of sub-block sbg.
// A sub-block's 96 mt bytes are padded by 8: a wave's staging stores cover
// eight sub-blocks at once, and an unpadded stride (768 B at mt = 8, a
// multiple of the 256-byte bank row) put all eight on the same banks.
__host__ __device__ constexpr int sbstride(int mt) { return 96 * mt + 8; }
__device__ __forceinline__ int boff(int sbg, int t, int q, int m, int mt) {
    return sbg * sbstride(mt) + ((t * 4 + q) * mt + m) * 8;
}

struct Layout {  // LDS byte offsets
    int s1, S, zero, wave, part, total;
    static constexpr int PANEL = 2304, WAVE = 2304 + 128 * 4;  // panel, wv
};
__host__ __device__ inline Layout layout(int K, int mt, int nw, int ntl, int C) {
    Layout L;
    const int NSB = K / 32;
    L.s1 = NSB * sbstride(mt);
    L.S = L.s1 + 4 * mt * NSB;
    L.zero = L.S + 4 * mt * NSB;
    L.wave = (L.zero + 16 + 15) & ~15;
    L.part = L.wave + nw * Layout::WAVE;
    L.total = L.part + ntl * slots(K / 256, C) * 16 * mt * 4;
    return L;
}

// floor(i / S) for 0 <= i < 2^22 from a precomputed 1 / S (the quotient's
// error is below 2^-23 i / S, less than the 1 / (2 S) margin of i + 1/2),
// broadcast as a uniform value.
__device__ __forceinline__ int div_small(int i, float inv) {
    return __builtin_amdgcn_readfirstlane((int)(((float)i + 0.5f) * inv));
}

struct Raw {
    fq_u32x4 v[3];  // pieces lane, lane + 64, lane + 128 (clamped to 143) of the panel
};

// Loads of local step n (clamped to the last step): the 16 rows' super-block
// sb of tile t0 + n / S.
__device__ __forceinline__ void load_step(Raw& f, const GemvArgs& a, int S, float invS, int t0,
                                          int n, int last, const int (&prow)[3],
                                          const int (&pcol)[3]) {
    const int il = min(n, last);
    const int tt = div_small(il, invS);
    const int sb = il - tt * S;
    const int row0 = 16 * (t0 + tt);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int row = min(row0 + prow[i], a.N - 1);
        const uint8_t* p = a.w + (size_t)row * a.row_bytes + 144 * sb + 16 * pcol[i];
        f.v[i] = __builtin_nontemporal_load(reinterpret_cast<const fq_u32x4*>(p));
    }
}

template <int MT, int WG, bool BIAS>
__global__ __launch_bounds__(WG) void mmqi_kernel(GemvArgs a) {
    constexpr int NWV = WG / 64;
    // sub-block pairs unrolled: all four at 512 threads (up to 256 VGPRs),
    // one at 1024 (128 VGPRs)
    constexpr int JU = WG >= 1024 ? 1 : 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, S = K / 256, NSB = K / 32, M = a.M;
    const float invS = 1.0f / (float)max(S, 1);
    const int T = a.U, C = a.Uc, JS = slots(S, C);
    const int G = gridDim.x, g = blockIdx.x;
    const int t0 = (int)((int64_t)T * g / G), t1 = (int)((int64_t)T * (g + 1) / G);
    const int ntl = t1 - t0;
    const Layout Lo = layout(K, MT, NWV, ntl, C);
    float* s1a = reinterpret_cast<float*>(lds + Lo.s1);
    float* Sa = reinterpret_cast<float*>(lds + Lo.S);
    uint8_t* panel = lds + Lo.wave + wave * Layout::WAVE;
    float* wv = reinterpret_cast<float*>(panel + Layout::PANEL);
    float* part = reinterpret_cast<float*>(lds + Lo.part);

    // ---- work: chunks of C >= DT steps (see the head comment)
    const int items = ntl * S;
    const int nchunks = (items + C - 1) / C;
    const int clampi = max(items - 1, 0);
    int prow[3], pcol[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int p = min(lane + 64 * i, 143);
        prow[i] = p / 9;
        pcol[i] = p - 9 * prow[i];
    }
    int ld_pos = wave * C, ld_end = ld_pos < items ? min(items, ld_pos + C) : -1;
    int cp_pos = ld_pos, cp_end = max(ld_end, ld_pos);
    int pend_pos = -1, pend_end = -1, pend_k = 0;
    int cp_k = wave;
    Raw f[DT];

    // ---- staging of every token's limbs, with the wave's first DT steps of
    // weight loads (inside its first chunk: no claims yet) issued between the
    // first activation loads and their limb build, so HBM streams while the
    // work-group builds.  The activation loads are unconditional (tokens past
    // M repeat the last one) so the compiler knows how many weight loads
    // follow them.
    const int tpt = K / 4;  // tasks per token: 8 lanes per 32-element sub-block
    float4 v[MT];           // every token's loads in flight together
    auto xload = [&](int base) {
        const int t = min(base + (int)threadIdx.x, tpt - 1);
#pragma unroll
        for (int m = 0; m < MT; ++m)
            v[m] = reinterpret_cast<const float4*>(a.x + (size_t)min(m, M - 1) * K)[t];
    };
    auto xbuild = [&](int base) {
        const int t = base + (int)threadIdx.x;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= M) break;
            const LimbQuad lq = limb_quad<32>(v[m]);
            if (t < tpt) {
                const int sbg = t >> 3, i = t & 7, q = i >> 1;
                const uint32_t l[3] = {lq.a1, lq.a2, lq.a3};
#pragma unroll
                for (int tl = 0; tl < 3; ++tl)
                    *reinterpret_cast<uint32_t*>(lds + boff(sbg, tl, q, m, MT) + 4 * (i & 1)) =
                        l[tl];
                if (i == 0) {  // token-minor, so the lanes of a sub-block read one run
                    s1a[sbg * MT + m] = lq.s1;
                    Sa[sbg * MT + m] = lq.gs;
                }
            }
        }
    };
    xload(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < DT; ++j) {
        load_step(f[j], a, S, invS, t0, ld_pos, clampi, prow, pcol);
        ++ld_pos;
    }
    __builtin_amdgcn_sched_barrier(0);
    xbuild(0);
    for (int base = WG; base < tpt; base += WG) {
        xload(base);
        xbuild(base);
    }
    __shared__ int ctr;
    if (threadIdx.x == 0) ctr = NWV;
    if (threadIdx.x < 4) reinterpret_cast<uint32_t*>(lds + Lo.zero)[threadIdx.x] = 0u;
    for (int i = threadIdx.x; i < ntl * JS * 16 * MT; i += WG) part[i] = 0.0f;
    lds_barrier();  // the weight loads stay in flight
    if (ld_end >= 0 && ld_pos > ld_end) ld_end = -1;

    auto load_next = [&](Raw& rb) {
        if (ld_end >= 0 && ld_pos >= ld_end) {
            int k = 0;
            if (lane == 0) k = atomicAdd(&ctr, 1);
            k = __builtin_amdgcn_readfirstlane(k);
            if (k < nchunks) {
                ld_pos = k * C;
                ld_end = min(items, ld_pos + C);
                pend_pos = ld_pos;
                pend_end = ld_end;
                pend_k = k;
            } else {
                ld_end = -1;  // nothing left: keep loading clamped addresses
            }
        }
        load_step(rb, a, S, invS, t0, ld_pos, clampi, prow, pcol);
        ++ld_pos;
    };

    const int r = lane & 15, q = lane >> 4, c = lane & 15;
    const bool live_c = c < M;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 Dm = {0.0f, 0.0f, 0.0f, 0.0f};  // min-term sums of the open tile
    int tt = div_small(min(cp_pos, clampi), invS);
    int sb = cp_pos - tt * S;
    while (cp_pos < cp_end) {
#pragma unroll
        for (int j = 0; j < DT; ++j) {
            __builtin_amdgcn_sched_barrier(0);
            if (cp_pos < cp_end) {  // wave-uniform
                // the 16 rows' super-blocks into this wave's panel
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    *reinterpret_cast<fq_u32x4*>(panel + 16 * (prow[i] * 9 + pcol[i])) = f[j].v[i];
                const uint8_t* rowp = panel + 144 * r;
                const fq_u32x4 h = *reinterpret_cast<const fq_u32x4*>(rowp);
                // header of row r: sub-blocks 2 q, 2 q + 1
                uint32_t sa, ma, sb2, mb;
                Fmt<Q4_K>::scale_min(uint4{h.x, h.y, h.z, h.w}, q, sa, ma, sb2, mb);
                const float d = f16_hw(h.x & 0xFFFFu) * 0x1p-14f, dmin = f16_hw(h.x >> 16);
                wv[(2 * q) * 16 + r] = d * (float)sa;
                wv[(2 * q + 1) * 16 + r] = d * (float)sb2;
                // min term sum_sb dmin m_{r,sb} S_{c,sb} on the matrix cores:
                // A[r][k] = dmin m of sub-block 2 k (+1), B[k][c] = S of token c
                {
                    const int sb0 = 8 * sb + 2 * q;
                    const float Sk0 = live_c ? Sa[sb0 * MT + c] : 0.0f;
                    const float Sk1 = live_c ? Sa[(sb0 + 1) * MT + c] : 0.0f;
                    Dm = __builtin_amdgcn_mfma_f32_16x16x4f32(dmin * (float)ma, Sk0, Dm, 0, 0, 0);
                    Dm = __builtin_amdgcn_mfma_f32_16x16x4f32(dmin * (float)mb, Sk1, Dm, 0, 0, 0);
                }
                // one 64-element group (two sub-blocks) per iteration, kept
                // rolled so the operands of one group at a time are live
#pragma unroll JU
                for (int jj = 0; jj < 4; ++jj) {
                    const fq_u32x2 qs =
                        *reinterpret_cast<const fq_u32x2*>(rowp + 16 + 32 * jj + 8 * q);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int sl = 2 * jj + hh, sbg = 8 * sb + sl;
                        const uint32_t x0 = ((hh ? qs.x >> 4 : qs.x)) & 0x0F0F0F0Fu;
                        const uint32_t x1 = ((hh ? qs.y >> 4 : qs.y)) & 0x0F0F0F0Fu;
                        const long A = (long)(((uint64_t)x1 << 32) | x0);
                        const uint8_t* bp =
                            live_c ? lds + boff(sbg, 0, q, c, MT) : lds + Lo.zero;
                        const int bstep = live_c ? 4 * MT * 8 : 0;
                        const long B0 = *reinterpret_cast<const long*>(bp);
                        const long B1 = *reinterpret_cast<const long*>(bp + bstep);
                        const long B2 = *reinterpret_cast<const long*>(bp + 2 * bstep);
                        const i32x4 z = {0, 0, 0, 0};
                        const i32x4 D0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B0, z, 0, 0, 0);
                        const i32x4 D1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B1, z, 0, 0, 0);
                        const i32x4 D2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B2, z, 0, 0, 0);
                        const float4 w4 = *reinterpret_cast<const float4*>(wv + sl * 16 + 4 * q);
                        const float s1c = live_c ? s1a[sbg * MT + c] : 0.0f;
                        const float ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int E = (D0[e] << 14) + (D1[e] << 7) + D2[e];
                            acc[e] = __builtin_fmaf(ww[e] * s1c, (float)E, acc[e]);
                        }
                    }
                }
                ++cp_pos;
                if (sb == S - 1 || cp_pos == cp_end) {  // flush tile tt (wave-uniform)
                    const int slot = cp_k - (tt * S) / C;
                    if (live_c) {
                        float* ps = part + ((tt * JS + slot) * 16) * MT;
#pragma unroll
                        for (int e = 0; e < 4; ++e) ps[(4 * q + e) * MT + c] = acc[e] - Dm[e];
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[e] = 0.0f;
                    Dm = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
                if (++sb == S) {
                    sb = 0;
                    ++tt;
                }
                if (cp_pos == cp_end && pend_pos >= 0) {  // into the chunk loaded next
                    cp_pos = pend_pos;
                    cp_end = pend_end;
                    cp_k = pend_k;
                    pend_pos = -1;
                    tt = div_small(cp_pos, invS);
                    sb = cp_pos - tt * S;
                }
            }
            load_next(f[j]);  // always issued (clamped), so the count in flight is fixed
        }
    }
    lds_barrier();

    // ---- each output: its slots in chunk order
    for (int e = threadIdx.x; e < ntl * 16 * M; e += WG) {
        const int tl = e / (16 * M), rest = e - tl * 16 * M, rr = rest / M, m = rest - rr * M;
        float v = 0.0f;
        for (int j = 0; j < JS; ++j) v += part[((tl * JS + j) * 16 + rr) * MT + m];
        const int row = 16 * (t0 + tl) + rr;
        if (row < a.N) {
            if constexpr (BIAS) {
                if (a.bias_mode == 2) v += a.bias[(size_t)m * a.N + row];
                else v += row < a.bias_len ? a.bias[row] : 0.0f;
            }
            a.y[(size_t)m * a.N + row] = v;
        }
    }
}

}  // namespace

bool mmqi_supported(int dtype) { return dtype == Q4_K; }

// Kernel, LDS bytes and threads for a pass of up to 8 tokens (nullptr: LDS
// too small for this K).
const void* mmqi_kernel_fn(int mt_needed, bool bias, int K, int tiles_per_wg, int chunk,
                           size_t lds_cap, size_t* lds, int* wg) {
    if (mt_needed <= 4) {
        const Layout L = layout(K, 4, 16, tiles_per_wg, chunk);
        if ((size_t)L.total <= lds_cap) {
            *lds = L.total;
            *wg = 1024;
            return bias ? (const void*)&mmqi_kernel<4, 1024, true>
                        : (const void*)&mmqi_kernel<4, 1024, false>;
        }
    }
    const Layout L = layout(K, 8, 8, tiles_per_wg, chunk);
    if ((size_t)L.total > lds_cap) return nullptr;
    *lds = L.total;
    *wg = 512;
    return bias ? (const void*)&mmqi_kernel<8, 512, true> : (const void*)&mmqi_kernel<8, 512, false>;
}

}  // namespace fq
