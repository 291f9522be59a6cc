// fq_capi.cpp -- the extern "C" entry points declared in include/forge_q.h:
// argument validation, launch planning and the per-stream scratch memory.
//
// Dispatch by token count (run_matmul): M = 1 runs the batch-1 GEMV kernels
// (fq_gemvp.hip over GGUF bytes or the aligned layout, fq_gemvt.hip for Q8_0
// matrices of 64k rows and more on the aligned layout, the row-step kernels
// of fq_gemv1.hip under about 4 MB of weights); M = 2..4
// the same batch-1 kernels with each weight unit dotted with every token;
// M = 2..16 (by format and shape) the band kernel of fq_mmqs.hip
// (Q6_K M = 4 on wide matrices: three tokens, then the fourth); M > 32 the
// prefill kernel
// of fq_mmqp.hip (rows in 16-byte chunks, K a multiple of 256); the rest --
// the reference's batched GEMV (1 < M <= 32) and dequant + GEMM prefill
// (M > 32), matmul.cpp:1150-1286 -- the int8 and fp16 MFMA kernels of
// fq_mmqi.hip and fq_mmq.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cstdio>
#include <cstdint>
#include <map>
#include <memory>
#include <vector>
#include <tuple>
#include <mutex>
#include <utility>

#include "../../include/forge_q.h"
#include "fq_kernels.h"
#include "fq_pack.h"

namespace {

thread_local int g_last_hip = 0;

int hip_fail(hipError_t e) {
    g_last_hip = (int)e;
    return FQ_ERR_HIP;
}

struct Geometry {
    int be, bb, ng;
};

bool geometry(uint32_t dtype, Geometry& g) {
    switch (dtype) {
        case FQ_DTYPE_Q4_0: g = {32, 18, 1}; return true;
        case FQ_DTYPE_Q4_1: g = {32, 20, 1}; return true;
        case FQ_DTYPE_Q8_0: g = {32, 34, 1}; return true;
        case FQ_DTYPE_Q4_K: g = {256, 144, 2}; return true;
        case FQ_DTYPE_Q6_K: g = {256, 210, 4}; return true;
        case FQ_DTYPE_Q5_0: g = {32, 22, 1}; return true;
        case FQ_DTYPE_Q5_1: g = {32, 24, 1}; return true;
        case FQ_DTYPE_Q3_K: g = {256, 110, 4}; return true;
        case FQ_DTYPE_Q5_K: g = {256, 176, 2}; return true;
        case FQ_DTYPE_IQ4_NL: g = {32, 18, 1}; return true;
        default: return false;
    }
}

// Formats with the aligned packed layout (fq_pack.h).
bool packable(uint32_t dtype) { return fq::packed_row_bytes((int)dtype, 256) > 0; }

struct DevInfo {
    int cus = 0;
    size_t lds = 0;
};

DevInfo device_info(int dev) {
    static std::mutex mu;
    static std::map<int, DevInfo> cache;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    DevInfo d;
    if (hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) d.cus = 0;
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lds = 0;
    d.lds = (size_t)lds;
    if (d.cus <= 0) d.cus = 256;
    if (d.lds == 0) d.lds = 64 * 1024;
    cache[dev] = d;
    return d;
}

// Device scratch per (device, stream, slot) for the MFMA path (slot 0: token
// operands, group sums, exponents and split-K partial slabs) and the GGUF
// fused FFN / QKV (slot 1: the gate/up or per-matrix rows).
//
// A call holds its slot's lock (StreamScratch::Lease) from taking the pointer
// until its launches are enqueued, so two host threads sharing a stream never
// see a buffer change under them.  The buffer only grows, at least doubling;
// a superseded buffer is not freed inside a compute call (queued work may
// still read it, and waiting for it would block the host mid-stream): it is
// kept until fq_release_workspace(), so the workspace of a stream holds less
// than twice its largest request.  fq_reserve_workspace() sizes it up front;
// during HIP-graph capture a call that would have to grow it fails with
// FQ_ERR_WORKSPACE instead of allocating.
struct StreamScratch {
    std::mutex mu;
    uint8_t* p = nullptr;
    size_t n = 0;
    std::vector<uint8_t*> retired;

    class Lease {
      public:
        explicit Lease(StreamScratch& s) : lk_(s.mu), s_(s) {}
        // the slot's buffer, at least `bytes` long
        int get(size_t bytes, hipStream_t st, uint8_t** out) {
            if (s_.n < bytes) {
                hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
                if (st && hipStreamIsCapturing(st, &cs) == hipSuccess &&
                    cs != hipStreamCaptureStatusNone)
                    return FQ_ERR_WORKSPACE;
                const size_t want = std::max(bytes, 2 * s_.n);
                uint8_t* np = nullptr;
                const hipError_t e = hipMalloc(reinterpret_cast<void**>(&np), want);
                if (e != hipSuccess) return hip_fail(e);
                if (s_.p) s_.retired.push_back(s_.p);
                s_.p = np;
                s_.n = want;
            }
            *out = s_.p;
            return FQ_OK;
        }

      private:
        std::unique_lock<std::mutex> lk_;
        StreamScratch& s_;
    };
};

std::mutex g_scratch_mu;
std::map<std::tuple<int, hipStream_t, int>, std::unique_ptr<StreamScratch>> g_scratch;

StreamScratch& stream_scratch(int dev, hipStream_t st, int slot) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto& p = g_scratch[{dev, st, slot}];
    if (!p) p.reset(new StreamScratch);
    return *p;
}

// Workspace bytes of the MFMA path for one call (the same plan run_mmq makes).
struct MmqPlan {
    int Tp, NC, shape, gx, gy, splits;
    size_t xop_b, xsum_b, ex_b, part_b, total;
};

MmqPlan plan_mmq(int M, int K, int N, int cus) {
    MmqPlan p{};
    p.Tp = (M + 15) / 16;
    p.NC = (K + 63) / 64;
    p.shape = p.Tp == 1 ? fq::MMQ_SMALL1 : p.Tp == 2 ? fq::MMQ_SMALL2
              : p.Tp <= 4 ? fq::MMQ_MID : fq::MMQ_BIG;
    int bn = 0, bm = 0;
    fq::mmq_shape(p.shape, &bn, &bm);
    p.gx = (N + bn - 1) / bn;
    p.gy = (p.Tp + bm / 16 - 1) / (bm / 16);
    const long tiles = (long)p.gx * p.gy;
    // K-splits only when the tiles alone leave CUs idle, to about two
    // work-groups per CU for the 128x128 prefill tiles and three for the
    // small-batch tiles (measured: cfg4 448 tiles fastest unsplit, 128 tiles
    // with 4 splits; 18944-row Q5_K at M = 8 41 -> 37 us with 6 splits)
    const long per_cu = p.shape == fq::MMQ_BIG ? 2 : 3;
    int splits = tiles >= cus ? 1
                              : (int)std::max(1L, std::min<long>((per_cu * cus + tiles - 1) / tiles, 8));
    p.splits = std::max(1, std::min(splits, p.NC / 4));
    p.xop_b = (size_t)p.Tp * p.NC * 2048 * 2;
    p.xsum_b = (size_t)p.Tp * p.NC * 64 * 4;
    p.ex_b = (size_t)p.Tp * p.NC * 16 * 4;
    p.part_b = p.splits > 1 ? (size_t)p.splits * M * N * 4 : 0;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    p.total = 256 + al(p.xop_b) + al(p.xsum_b) + al(p.ex_b) + al(p.part_b);
    return p;
}

// Rows per band and K-splits of the small-batch band kernel.  Short rows:
// bands of up to four 16-row tiles, as few rows per band as fill every CU,
// unsplit.  Long rows (32 super-blocks and more) with few rows: each band
// re-reads the token operands of all of K, 4 KiB per 64 elements, for as
// few as 16 rows, so the bands take four tiles and K is split to fill the
// CUs (each wave keeping at least one super-block per split; the slabs are
// summed in split order).  Measured at 3584 x 18944 (M = 4 / 16): 30.3 /
// 30.8 us unsplit on 16-row bands, 27.1 / 28.0 us on 64-row bands in four
// splits; at K = 4096 every split measured slower.
int mmqs_plan(int N, int K, int cus, int* rows_per_wg, int mt) {
    const int nsb = K / 256;
    const long bands4 = (N + 16 * mt - 1) / (16 * mt);
    if (nsb >= 32 && 2 * bands4 <= cus) {
        *rows_per_wg = 16 * mt;
        const int s = (int)std::max(1L, std::min<long>(cus / bands4, nsb / 8));
        const int sps = (nsb + s - 1) / s;
        return (nsb + sps - 1) / sps;
    }
    *rows_per_wg = 16 * std::min(mt, std::max(1, (N + 16 * cus - 1) / (16 * cus)));
    return 1;
}

// Workspace bytes of a band-kernel call: the token operands of plan_mmq's
// single token tile and, when K is split, the slabs.
size_t mmqs_need(int M, int K, int N, int cus, int mt) {
    const MmqPlan pl = plan_mmq(M, K, N, cus);
    int rpw = 0;
    const int splits = mmqs_plan(N, K, cus, &rpw, mt);
    const size_t part_b = splits > 1 ? (size_t)splits * M * N * 4 : 0;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    return 256 + al(pl.xop_b) + al(pl.xsum_b) + al(pl.ex_b) + al(part_b);
}

// Workspace bytes and K-splits of the prefill kernel (M > 32, K a multiple
// of 256): one work-group per CU and tile, K split when that
// shortens the busiest CU's work, each split a multiple of four 64-element
// steps.
struct MmqpPlan {
    int splits;
    size_t xop_b, ex_b, sum_b, part_b, q6c_b, total;
};

MmqpPlan plan_mmqp(int M, int K, int N, int cus, bool q6k = false) {
    MmqpPlan p{};
    const int Tn = (M + 31) / 32, nsteps = K / 64;
    const int tn = fq::mmqp_tile_rows(), tm = fq::mmqp_tile_tokens();
    const long tiles = (long)((N + tn - 1) / tn) * ((M + tm - 1) / tm);
    // the split count with the fewest steps on the busiest CU (rounds of
    // work-groups x steps per split), taken only when it saves at least a
    // quarter of the unsplit count: every split adds a partial slab and its
    // share of the reduce (14336 x 4096 x 512: 224 tiles run fastest
    // unsplit, 4096 x 4096 x 512: 64 tiles with 4 splits)
    const long cost1 = ((tiles + cus - 1) / cus) * nsteps;
    long best = cost1;
    p.splits = 1;
    for (int sp = 2; sp <= std::min(16, nsteps / 4); ++sp) {
        const int sps = ((nsteps + sp - 1) / sp + 3) & ~3;
        const int eff = (nsteps + sps - 1) / sps;  // non-empty splits
        const long cost = ((tiles * eff + cus - 1) / cus) * sps;
        if (4 * cost <= 3 * cost1 && cost < best) {
            best = cost;
            p.splits = eff;
        }
    }
    p.xop_b = (size_t)Tn * K * 64 * 2;
    p.ex_b = (size_t)M * 4;
    p.sum_b = (size_t)Tn * 32 * K / 32 * 4;  // sub-block sums (formats with a min term)
    p.part_b = p.splits > 1 ? (size_t)p.splits * M * N * 4 : 0;
    p.q6c_b = q6k ? (size_t)fq::mmqp_q6c_bytes(N, K) : 0;  // Q6_K rows as 36-byte blocks
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    p.total = 256 + al(p.xop_b) + al(p.ex_b) + al(p.sum_b) + al(p.part_b) + al(p.q6c_b);
    return p;
}

// M > 1 on the matrix cores: token operand preparation, then one tile per
// work-group (K-split when the tiles alone do not fill the chip).  The
// workspace is `fixed` (fixed_cap bytes) when given, else the stream's.
int run_mmq(uint32_t dtype, const Geometry& g, const float* x, const void* w, const float* bias,
            int bias_mode, int64_t bias_len, float* y, int M, int K, int N, int dev,
            const DevInfo& di, hipStream_t st, uint8_t* fixed, size_t fixed_cap) {
    const MmqPlan pl = plan_mmq(M, K, N, di.cus);
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    std::unique_ptr<StreamScratch::Lease> lease;
    uint8_t* buf = fixed;
    if (fixed) {
        if (pl.total > fixed_cap) return FQ_ERR_WORKSPACE;
    } else {
        lease.reset(new StreamScratch::Lease(stream_scratch(dev, st, 0)));
        const int rc = lease->get(pl.total, st, &buf);
        if (rc != FQ_OK) return rc;
    }
    fq::MmqArgs a{};
    a.w = static_cast<const uint8_t*>(w);
    a.xop = buf;
    a.xsum = reinterpret_cast<const float*>(buf + al(pl.xop_b));
    a.ex = reinterpret_cast<const int*>(buf + al(pl.xop_b) + al(pl.xsum_b));
    a.part = pl.splits > 1
                 ? reinterpret_cast<float*>(buf + al(pl.xop_b) + al(pl.xsum_b) + al(pl.ex_b))
                 : nullptr;
    a.y = y;
    a.bias = bias;
    a.bias_len = bias_mode ? bias_len : 0;
    a.bias_mode = bias_mode;
    a.M = M;
    a.N = N;
    a.K = K;
    a.NC = pl.NC;
    a.row_bytes = (K / g.be) * g.bb;
    hipError_t e = hipSuccess;
    if (pl.NC > 0) {  // K == 0 only writes the bias (or zeros)
        e = fq::launch_xprep((int)dtype, x, M, K, pl.NC, reinterpret_cast<_Float16*>(buf),
                             const_cast<float*>(a.xsum), const_cast<int*>(a.ex), st);
        if (e != hipSuccess) return hip_fail(e);
    }
    e = fq::launch_mmq((int)dtype, a, pl.shape, pl.gx, pl.gy, pl.splits, st);
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

// band_x (optional): in, true when the stream's slot-0 workspace already
// holds the band kernel's token operands of this x, M, K and format (a call
// just before with the same x, M, K, N and format took the band kernel:
// same plan, same workspace size, so the buffer was not replaced); out,
// whether this call took the band kernel.
int run_matmul(uint32_t dtype, const float* x, const void* w, const float* bias, int bias_mode,
               int64_t bias_len, float* y, int M, int K, int N, hipStream_t st,
               uint8_t* fixed = nullptr, size_t fixed_cap = 0, bool* band_x = nullptr);

// Fixed workspace of fq_matmul_transB_noalloc, for callers that cannot
// allocate (HIP-graph capture, serving loops that forbid hipMalloc).  Every
// GPU the library runs on holds its own copy until the process ends.  It is
// shared by every call of that entry point on the device: calls that overlap
// on one GPU race on it.  Nothing in it has to start at zero (the token
// preparation writes every operand, each K-split writes its whole slab).
constexpr size_t kNoAllocBytes = (size_t)64 << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocBytes];

// The device address of `scratch` on the current device, looked up once per
// device (the host-side name is only a stand-in for the symbol).
int noalloc_workspace(int dev, uint8_t** out) {
    static std::mutex mu;
    static std::map<int, uint8_t*> ptrs;
    std::lock_guard<std::mutex> lk(mu);
    auto it = ptrs.find(dev);
    if (it == ptrs.end()) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e);
        it = ptrs.emplace(dev, static_cast<uint8_t*>(p)).first;
    }
    *out = it->second;
    return FQ_OK;
}

int packed_gemv(uint32_t dtype, const float* x, const void* w_packed, const void* w2_packed,
                const void* w3_packed, int n1, int n2, int mode, const float* bias,
                int64_t bias_len, float* y, int K, int N, hipStream_t st, bool gguf, int M = 1,
                bool bias_full = false, uint8_t* fixed = nullptr, size_t fixed_cap = 0);

int run_matmul(uint32_t dtype, const float* x, const void* w, const float* bias, int bias_mode,
               int64_t bias_len, float* y, int M, int K, int N, hipStream_t st, uint8_t* fixed,
               size_t fixed_cap, bool* band_x) {
    const bool x_ready = band_x && *band_x;
    if (band_x) *band_x = false;
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
    if (M < 0 || N < 0 || K < 0) return FQ_ERR_SHAPE;
    if (K % g.be != 0) return FQ_ERR_SHAPE;
    if (M == 0 || N == 0) return FQ_OK;
    if (!x || !w || !y) return FQ_ERR_NULL;
    if (bias_mode != 0 && !bias) return FQ_ERR_NULL;
    if (bias_mode == 2 && bias_len < (int64_t)M * N) return FQ_ERR_SHAPE;
    if ((int64_t)(K / g.be) * g.bb > INT32_MAX) return FQ_ERR_SHAPE;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    if (K == 0 && bias_mode == 0) {
        // a zero-length contraction: y = 0 (with a bias the kernel writes y = bias)
        e = fq::launch_zero(reinterpret_cast<uint32_t*>(y), (size_t)M * N, di.cus, st);
        return e == hipSuccess ? FQ_OK : hip_fail(e);
    }

    if (M == 1 && K > 0 && packable(dtype) &&
        (dtype == FQ_DTYPE_Q6_K || (int64_t)N * (K / g.be) * g.bb >= (4 << 20))) {
        // batch 1 on the five benchmark formats: the aligned-layout kernel,
        // reading the GGUF rows through per-wave LDS buffers (with one token a
        // full [1][N] bias is a row vector of N).  Below ~4 MB of weights the
        // row-step kernels start faster (2048 x 2048 Q4_0, 2.4 MB: 3.6 us
        // against 4.2); from 4.5 MB this one is (2048 x 2048 Q8_0 4.4 against
        // 4.7 us, TinyLlama Q4_0 5632 x 2048 4.8 against 5.15); Q6_K always
        // runs here.
        const int rc = packed_gemv(dtype, x, w, nullptr, nullptr, 0, 0, 0,
                                   bias_mode ? bias : nullptr, bias_mode == 2 ? N : bias_len, y,
                                   K, N, st, true);
        if (rc != FQ_ERR_SHAPE) return rc;
    }

    if (dtype == FQ_DTYPE_Q6_K && M == 4 && K > 0 && N > 16384 &&
        (int64_t)N * (K / g.be) * g.bb >= (24 << 20)) {
        // four Q6_K tokens on 24 MB and more of more than 16384 rows: three on
        // the batch-1 kernel, then the fourth (its four-token form spills;
        // 152064 x 3584 196-203 us against 209 on the band kernel, 18944 x
        // 3584 34.7 against 37.3); fewer rows, and five tokens, take the band
        // kernel below (3584 x 18944 35.0 against 45.9 this way, 14336 x 4096
        // 27.8 against 30.8, lm_head at M = 5 about 211 against 222)
        for (int t0 = 0; t0 < M; t0 += 3) {
            const int m = std::min(3, M - t0);
            const int rc = run_matmul(dtype, x + (size_t)t0 * K, w,
                                      bias_mode == 2 ? bias + (size_t)t0 * N : bias, bias_mode,
                                      bias_mode == 2 ? (int64_t)m * N : bias_len,
                                      y + (size_t)t0 * N, m, K, N, st, fixed, fixed_cap);
            if (rc != FQ_OK) return rc;
        }
        return FQ_OK;
    }

    // Q4_0 and Q8_0 on the band kernel below: rows that start 16-byte aligned
    // (K a multiple of 256), 5..16 tokens, or 4 from 16 MB (below, the
    // kernels further down take M = 4 0.4-0.7 us faster for Q4_0; Q8_0 only
    // while the bands number at most one per CU: lm_head 157 us on the
    // batch-1 kernel against 173), or, Q4_0 only, 3 from 16 MB with K of
    // 14336 and more (3584 x 18944: 26.4 us on the batch-1 kernel).  At 3
    // and 4 tokens Q4_0 needs at most one band per CU or at least eight
    // (152064 rows at M = 4 129 against 151 us); from 5 tokens any count
    // (18944 rows in three-tile bands, below: 24.5 against 27.5 us at M =
    // 8).  Q8_0 takes any count (the fp16 MFMA path is slower at every one
    // measured: 14336 x 4096 at M = 8 24.1 against 37.6 us)
    const int bmt = fq::mmqs_max_tiles((int)dtype);
    const long bands = ((long)N + 16 * bmt - 1) / (16 * bmt);
    // (Q4_1 as Q4_0)
    const bool q4x = dtype == FQ_DTYPE_Q4_0 || dtype == FQ_DTYPE_Q4_1;
    const bool blk_band = (q4x || dtype == FQ_DTYPE_Q8_0) && K % 256 == 0 &&
                          (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                          (M >= 5 ||
                           ((M == 4 ? q4x || bands <= di.cus : M == 3 && q4x && K >= 14336) &&
                            (int64_t)N * (K / g.be) * g.bb >= (16 << 20))) &&
                          (dtype == FQ_DTYPE_Q8_0 || M >= 5 || bands <= di.cus ||
                           bands >= 8L * di.cus);
    if (M >= 2 && M <= 4 && !blk_band && K > 0 && packable(dtype) &&
        (dtype == FQ_DTYPE_Q6_K || (int64_t)N * (K / g.be) * g.bb >= (8 << 20))) {
        // two to four tokens: the same kernel dots each weight unit it reads
        // with every token's limbs, K split into slabs where the tokens'
        // records of a whole row do not fit LDS (FQ_ERR_SHAPE: no split fits,
        // or the slabs need workspace the call cannot have)
        const int rc = packed_gemv(dtype, x, w, nullptr, nullptr, 0, 0, 0,
                                   bias_mode ? bias : nullptr, bias_mode == 2 ? N : bias_len, y,
                                   K, N, st, true, M, bias_mode == 2, fixed, fixed_cap);
        if (rc != FQ_ERR_SHAPE) return rc;
    }

    // Q5_K (rows 16-byte aligned): 5..16 tokens; 4 while the bands number at
    // most one per CU or at least eight per CU (18944 x 3584: 33.4 against
    // 31.7 us on the fp16 MFMA path); 3 at K >= 14336 or eight bands per CU
    // and more (3584 x 18944 54.1 -> 27.0 us at M = 4, lm_head at M = 3 166
    // against about 150; 18944 x 3584 at M = 3 26.0 against 33); 2 at K >=
    // 14336 (3584 x 18944: 53.9 on the fp16 MFMA path; lm_head at M = 2
    // 111.5 against about 150 stays there)
    const bool al16 = K % 256 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    // Q5_0 and IQ4_NL: K >= 14336 from 2 tokens (3584 x 18944 at M = 2..8:
    // 55.3 -> 27.9 and 47.4 -> 28.3 us), or 4..16 tokens in one round of
    // bands (14336 x 4096 at M = 8: 33.2 -> 21.3, 29.2 -> 21.6); 18944 rows
    // at M = 8 measured slower (35.5 against 32.7, 36.1 against 28.4).
    // Q5_1 (160 KB of LDS per work-group): K >= 14336 only (43.8 -> 37.5;
    // lm_head at M = 8 216 against 159)
    const bool q5x_band =
        al16 && M >= 2 &&
        (((dtype == FQ_DTYPE_Q5_0 || dtype == FQ_DTYPE_IQ4_NL) &&
          (K >= 14336 || (M >= 4 && bands <= di.cus))) ||
         (dtype == FQ_DTYPE_Q5_1 && K >= 14336));
    // Q3_K (rows at even addresses): K >= 14336 from two tokens (3584 x 18944
    // 61 -> 28.7 us), 4..16 tokens for any row count (152064 x 3584 at M = 8
    // 262 -> 184, 14336 x 4096 41.9 -> 32.0; equal at M = 4)
    const bool q3k_band = dtype == FQ_DTYPE_Q3_K && K % 256 == 0 &&
                          (reinterpret_cast<uintptr_t>(w) & 1) == 0 && M >= 2 &&
                          (K >= 14336 || M >= 4);
    const bool q5k_band =
        q3k_band || (dtype == FQ_DTYPE_Q5_K && al16 &&
         (M >= 5 || (M == 4 && (bands <= di.cus || bands >= 8L * di.cus)) ||
          (M == 3 && (K >= 14336 || bands >= 8L * di.cus)) || (M == 2 && K >= 14336))) ||
        q5x_band;
    if (fq::mmqs_supported((int)dtype) && M >= (q5k_band ? 2 : blk_band ? 3 : 4) && M <= 16 &&
        K > 0 &&
        (dtype == FQ_DTYPE_Q4_K   ? N <= 16 * bmt * di.cus || M > 8
         : dtype == FQ_DTYPE_Q6_K ? (reinterpret_cast<uintptr_t>(w) & 1) == 0
         : (dtype == FQ_DTYPE_Q4_0 || dtype == FQ_DTYPE_Q4_1 || dtype == FQ_DTYPE_Q8_0)
             ? blk_band
             : q5k_band)) {
        // (Q4_0, Q8_0: see blk_band.  Q4_K beyond one band per CU only above
        // 8 tokens, which the int8 kernel does not take: 18944 x 3584 at M =
        // 16 31.2 against 34.4 us on the fp16 MFMA path, 152064 x 3584 143.5
        // against 170.4; at M = 4..8 the int8 kernel is faster, 21.1-27.5
        // against 30.2-30.4 and 108-130 against 137-139)
        // 2..16 tokens (by format and shape, above): token operands, then one
        // pass over the weights on the fp16 matrix cores, one band of rows per
        // work-group (Q4_K at 14336 x 4096: 19.2-19.7 us for every M in 4..16,
        // against 21-30 us on the int8 matrix-core and fp16 MFMA paths; Q4_K
        // at M = 2, 3 is faster on the batch-1 and int8 kernels, and at M =
        // 4..8 on rows beyond one band per CU on the int8 kernel)
        const int NC = K / 64;
        const MmqPlan pl = plan_mmq(M, K, N, di.cus);
        auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
        // Q8_0: two- or three-tile bands, whichever the estimate (rounds of
        // work-groups x tiles x super-blocks per split) puts lower, three
        // within 5 % (14336 x 4096 at M = 8: 24.2 us on two, 30.1 on three;
        // 152064 x 3584: 175.4 / 170.0; 18944 x 3584: 31.3 / 29.6)
        int tiles = bmt;
        if (bmt == 4 && K / 256 < 32) {
            // four-tile bands whose last round of work-groups is mostly idle
            // (18944 rows: 296 bands on 256 CUs) take three tiles when those
            // fill their rounds better (395 bands: Q4_0 at M = 8 27.5 ->
            // 24.5 us, Q4_K at M = 16 31.3 -> 26.4, Q5_K 33.2 -> 27.7; at
            // 14336 and 152064 rows four tiles measured faster)
            auto fill = [&](int t) {
                const long b = ((long)N + 16 * t - 1) / (16 * t);
                return (double)b / (double)(((b + di.cus - 1) / di.cus) * di.cus);
            };
            if (N > 64L * di.cus && fill(4) < 0.6 && fill(3) > fill(4)) tiles = 3;
        } else if (dtype == FQ_DTYPE_Q8_0) {
            auto est = [&](int mt) {
                int r = 0;
                const long sp = mmqs_plan(N, K, di.cus, &r, mt);
                const long wgs = ((long)N + r - 1) / r * sp;
                return (double)((wgs + di.cus - 1) / di.cus) * (r / 16) *
                       (double)((K / 256 + sp - 1) / sp);
            };
            tiles = est(3) <= 1.05 * est(2) ? 3 : 2;
        }
        int rpw = 0;
        const int splits = mmqs_plan(N, K, di.cus, &rpw, tiles);
        const size_t need = mmqs_need(M, K, N, di.cus, tiles);
        std::unique_ptr<StreamScratch::Lease> lease;
        uint8_t* buf = fixed;
        if (fixed) {
            if (need > fixed_cap) return FQ_ERR_WORKSPACE;
        } else {
            lease.reset(new StreamScratch::Lease(stream_scratch(dev, st, 0)));
            const int rc = lease->get(need, st, &buf);
            if (rc != FQ_OK) return rc;
        }
        fq::MmqArgs a{};
        a.w = static_cast<const uint8_t*>(w);
        a.xop = buf;
        a.xsum = reinterpret_cast<const float*>(buf + al(pl.xop_b));
        a.ex = reinterpret_cast<const int*>(buf + al(pl.xop_b) + al(pl.xsum_b));
        a.part = splits > 1 ? reinterpret_cast<float*>(buf + al(pl.xop_b) + al(pl.xsum_b) +
                                                       al(pl.ex_b))
                            : nullptr;
        a.y = y;
        a.bias = bias;
        a.bias_len = bias_mode ? bias_len : 0;
        a.bias_mode = bias_mode;
        a.M = M;
        a.N = N;
        a.K = K;
        a.NC = NC;
        a.row_bytes = (K / g.be) * g.bb;
        if (!x_ready) {
            e = fq::launch_xprep((int)dtype, x, M, K, NC, reinterpret_cast<_Float16*>(buf),
                                 const_cast<float*>(a.xsum), const_cast<int*>(a.ex), st);
            if (e != hipSuccess) return hip_fail(e);
        }
        e = fq::launch_mmqs((int)dtype, a, rpw, 512, splits, st);
        if (e != hipSuccess) return hip_fail(e);
        if (band_x) *band_x = true;
        return FQ_OK;
    }

    if ((M == 1 || M == 2) && K > 0) {
        // batch 1 (and two tokens on rows of at most 128 units, where the
        // row-step kernel keeps both tokens' limbs in registers): persistent
        // work-groups, as many as fit on every CU
        const int U1 = K / 32;
        int wg = 1024;
        size_t lds = M == 1 ? fq::gemv1_lds_bytes((int)dtype, U1, wg) : 0;
        const void* fn = M == 1 ? fq::gemv1_kernel_fn((int)dtype, bias_mode != 0, wg) : nullptr;
        int npr = 0;
        size_t lds_r = 0;
        int wg_r = 0;
        const void* fr = fq::gemv1r_kernel_fn((int)dtype, U1, (K / g.be) * g.bb, bias_mode != 0,
                                              &npr, &lds_r, &wg_r, M);
        if (fr && lds_r <= std::min<size_t>(di.lds, 160 * 1024)) {
            fn = fr;
            lds = lds_r;
            wg = wg_r;
        }
        if (fn && lds <= std::min<size_t>(di.lds, 160 * 1024)) {
            int per_cu = 0;
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, wg, lds);
            if (e != hipSuccess) return hip_fail(e);
            if (per_cu >= 1) {
                fq::GemvArgs a{};
                a.x = x;
                a.w = static_cast<const uint8_t*>(w);
                a.y = y;
                a.bias = bias;
                a.bias_len = bias_mode == 0 ? 0 : bias_len;
                a.bias_mode = bias_mode;
                a.M = M;
                a.K = K;
                a.N = N;
                a.U = U1;
                a.Uc = U1;
                a.row_bytes = (K / g.be) * g.bb;
                const int wpb = wg / 64;
                const long waves = (long)di.cus * per_cu * wpb;
                const long need = std::min<long>(waves, N);
                const int grid = (int)std::max(1L, (need + wpb - 1) / wpb);
                e = fq::launch_raw(fn, a, grid, wg, lds, st);
                return e == hipSuccess ? FQ_OK : hip_fail(e);
            }
        }
    }

    if (fq::mmqi_supported((int)dtype) && M >= 3 && M <= 8 && K > 0) {
        // Q4_K, 3..8 tokens that the kernels above do not take: three tokens
        // on weights under 8 MB (from 8 MB the batch-1 kernel takes them, with
        // K split where the records overflow its LDS), and 4..8 tokens on more
        // rows than one mmqs band per CU covers.  The int8 matrix-core kernel
        // runs them in one pass (M = 9..16 takes the band kernel above)
        const long T = (N + 15) / 16;
        const long G = std::max(1L, std::min<long>(di.cus, T));
        const int tpw = (int)((T + G - 1) / G);
        bool ok = true;
        for (int m0 = 0; m0 < M && ok; m0 += 8) {
            const int mt = std::min(8, M - m0);
            size_t lds = 0;
            int wg = 0;
            // chunk: >= 3 steps, about 4 per wave
            int chunk = 3;
            const void* fn = nullptr;
            for (int pass = 0; pass < 2; ++pass) {
                const int waves = (pass == 0 && mt <= 4) ? 16 : 8;
                chunk = (int)std::max(3L, std::min(16L, (long)tpw * (K / 256) / (4L * waves)));
                fn = fq::mmqi_kernel_fn(mt, bias_mode != 0, K, tpw, chunk,
                                        std::min<size_t>(di.lds, 160 * 1024), &lds, &wg);
                if (fn && wg / 64 == waves) break;
            }
            if (!fn) {
                ok = false;
                break;
            }
            fq::GemvArgs a{};
            a.x = x + (size_t)m0 * K;
            a.w = static_cast<const uint8_t*>(w);
            a.y = y + (size_t)m0 * N;
            a.bias = bias_mode == 2 ? bias + (size_t)m0 * N : bias;
            a.bias_len = bias_mode == 0 ? 0 : bias_len;
            a.bias_mode = bias_mode;
            a.M = mt;
            a.K = K;
            a.N = N;
            a.U = (int)T;
            a.Uc = chunk;
            a.row_bytes = (K / g.be) * g.bb;
            e = fq::launch_raw(fn, a, (int)G, wg, lds, st);
            if (e != hipSuccess) return hip_fail(e);
        }
        if (ok) return FQ_OK;
    }

    if (M >= 2 && M <= 4 && K > 0) {
        // a few tokens: the batch-1 chunk kernel reads and unpacks each weight
        // unit once and dots it with every token's activation limbs
        const int U1 = K / 32;
        size_t lds = 0;
        const void* fn = fq::gemv1_multi_fn((int)dtype, bias_mode != 0, M, &lds, U1);
        if (fn && lds <= std::min<size_t>(di.lds, 160 * 1024)) {
            int per_cu = 0;
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 1024, lds);
            if (e != hipSuccess) return hip_fail(e);
            if (per_cu >= 1) {
                fq::GemvArgs a{};
                a.x = x;
                a.w = static_cast<const uint8_t*>(w);
                a.y = y;
                a.bias = bias;
                a.bias_len = bias_mode == 0 ? 0 : bias_len;
                a.bias_mode = bias_mode;
                a.M = M;
                a.K = K;
                a.N = N;
                a.U = U1;
                a.Uc = U1;
                a.row_bytes = (K / g.be) * g.bb;
                const long waves = (long)di.cus * per_cu * 16;
                const long need = std::min<long>(waves, N);
                const int grid = (int)std::max(1L, (need + 15) / 16);
                e = fq::launch_raw(fn, a, grid, 1024, lds, st);
                return e == hipSuccess ? FQ_OK : hip_fail(e);
            }
        }
    }

    const bool q6k = dtype == FQ_DTYPE_Q6_K;
    if (fq::mmqp_supported((int)dtype) && M > 32 && K > 0 && K % 256 == 0 &&
        (q6k || (reinterpret_cast<uintptr_t>(w) & 15) == 0) &&
        (int64_t)N * (q6k ? fq::mmqp_q6c_bytes(1, K) : (K / g.be) * g.bb) < ((int64_t)1 << 32)) {
        // prefill, rows that are whole 16-byte chunks (K a multiple of 256,
        // 16-byte aligned weights, under 4 GiB of them: the copies take
        // 32-bit offsets): per-token operands, then one work-group per CU and
        // tile on v_mfma_f32_32x32x16_f16 (K-split while the tiles leave CUs
        // idle).  Q6_K rows are first rewritten into 36-byte blocks in the
        // workspace
        const MmqpPlan pl = plan_mmqp(M, K, N, di.cus, q6k);
        const int splits = pl.splits;
        auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
        const size_t xop_b = pl.xop_b, ex_b = pl.ex_b, sum_b = pl.sum_b, need = pl.total;
        std::unique_ptr<StreamScratch::Lease> lease;
        uint8_t* buf = fixed;
        if (fixed) {
            if (need > fixed_cap) return FQ_ERR_WORKSPACE;
        } else {
            lease.reset(new StreamScratch::Lease(stream_scratch(dev, st, 0)));
            const int rc = lease->get(need, st, &buf);
            if (rc != FQ_OK) return rc;
        }
        fq::MmqArgs a{};
        a.w = static_cast<const uint8_t*>(w);
        a.row_bytes = (K / g.be) * g.bb;
        if (q6k) {
            uint8_t* conv = buf + al(xop_b) + al(ex_b) + al(sum_b) + al(pl.part_b);
            e = fq::launch_q6c(static_cast<const uint8_t*>(w), N, K, a.row_bytes, conv, st);
            if (e != hipSuccess) return hip_fail(e);
            a.w = conv;
            a.row_bytes = (int)fq::mmqp_q6c_bytes(1, K);
        }
        a.xop = buf;
        a.ex = reinterpret_cast<const int*>(buf + al(xop_b));
        a.xsum = dtype == FQ_DTYPE_Q4_K || dtype == FQ_DTYPE_Q4_1 || dtype == FQ_DTYPE_Q5_1
                     ? reinterpret_cast<const float*>(buf + al(xop_b) + al(ex_b))
                               : nullptr;
        a.part = splits > 1 ? reinterpret_cast<float*>(buf + al(xop_b) + al(ex_b) + al(sum_b))
                            : nullptr;
        a.y = y;
        a.bias = bias;
        a.bias_len = bias_mode ? bias_len : 0;
        a.bias_mode = bias_mode;
        a.M = M;
        a.N = N;
        a.K = K;
        e = fq::launch_xprep32(x, M, K, reinterpret_cast<_Float16*>(buf),
                               const_cast<int*>(a.ex), const_cast<float*>(a.xsum), q6k, st);
        if (e != hipSuccess) return hip_fail(e);
        e = fq::launch_mmqp((int)dtype, a, splits, st);
        if (e == hipSuccess && splits > 1) e = fq::launch_reduce(a, splits, st);
        return e == hipSuccess ? FQ_OK : hip_fail(e);
    }

    // M > 4, and rows too long for the batch-1 kernels' LDS
    return run_mmq(dtype, g, x, w, bias, bias_mode, bias_len, y, M, K, N, dev, di, st, fixed,
                   fixed_cap);
}

// Batch-1 GEMV over the tiled aligned layout, one row per lane
// (fq_gemvt.hip; every matrix involved satisfies packed_tiled()).  N output
// rows (mode 1: rows of each of the two matrices).  W waves per work-group
// (one K range each), 16 / W work-groups per CU, the tiles dealt out in turn
// so every work-group gets the same number within one; W shrinks until a
// work-group's tiles fit its LDS (gemvt_max_tiles()).
int run_gemvt(uint32_t dtype, const float* x, const void* w, const void* w2, const void* w3,
              int n1, int n2, int mode, const float* bias, int64_t bias_len, float* y, int K,
              int N, hipStream_t st, const DevInfo& di) {
    const int U = fq::gemvt_units((int)dtype, K);
    if (U % 4 != 0) return FQ_ERR_SHAPE;
    const int GR = U / 4;
    const int TRW = fq::gemvt_tile_rows();
    const long tiles = mode == 2 ? (long)(n1 + TRW - 1) / TRW + (n2 + TRW - 1) / TRW +
                                       (N - n1 - n2 + TRW - 1) / TRW
                                 : (long)(N + TRW - 1) / TRW;
    if (tiles > INT32_MAX / TRW) return FQ_ERR_SHAPE;
    // the kernel addresses each matrix through a 32-bit buffer offset
    const int64_t RB = fq::packed_row_bytes((int)dtype, K);
    if ((int64_t)(mode == 2 ? std::max(n1, std::max(n2, N - n1 - n2)) : N) * RB >= ((int64_t)1 << 32))
        return FQ_ERR_SHAPE;
    const int WM = fq::gemvt_max_waves(), ntmax = fq::gemvt_max_tiles();
    const int maxrec = fq::gemvt_max_records(), RBY = fq::gemvt_record_bytes();
    const int NV = mode == 1 ? 2 : 1;
    const size_t cu_lds = std::min<size_t>(di.lds, 160 * 1024);
    auto recs_of = [&](int w) { return ((GR + w - 1) / w) * 4; };
    auto lds_of = [&](int w, long nt) {
        return (size_t)w * recs_of(w) * RBY + (size_t)nt * NV * w * 64 * 4;
    };
    // the fewest waves per work-group (more work-groups per CU, the same 16
    // waves) whose records fit and whose tiles stay within gemvt_max_tiles()
    // and the CU's LDS
    int W = 0;
    long GT = 0;
    for (int w = std::min(WM, GR); w >= 1; w = w > 1 ? std::max(1, w / 2) : 0) {
        if (recs_of(w) > maxrec) break;
        const int wpc = std::max(1, WM / w);
        const long gt = std::min<long>(tiles, (long)di.cus * wpc);
        const long nt = (tiles + gt - 1) / gt;
        if (nt <= ntmax && lds_of(w, nt) * wpc <= cu_lds) {
            W = w;
            GT = gt;
            if (nt * 2 > ntmax) break;  // fewer waves would not fit the next halving
        } else if (W) {
            break;
        }
    }
    if (!W) {  // very long rows or very many tiles: the smallest fitting W, more work-groups
        W = std::min(WM, GR);
        while (W < WM && recs_of(W) > maxrec) W = std::min(WM, 2 * W);
        if (recs_of(W) > maxrec) return FQ_ERR_SHAPE;
        const size_t fixed = lds_of(W, 0);
        if (fixed >= cu_lds) return FQ_ERR_SHAPE;
        const long ntcap = std::max<long>(1, std::min<long>(ntmax, (long)((cu_lds - fixed) / ((size_t)NV * W * 64 * 4))));
        GT = (tiles + ntcap - 1) / ntcap;
    }
    const int recs = recs_of(W);
    const int nt_max = (int)((tiles + GT - 1) / GT);
    const size_t lds = lds_of(W, nt_max);
    if (lds > cu_lds) return FQ_ERR_SHAPE;
    const void* fn = fq::gemvt_kernel_fn((int)dtype, mode);
    if (!fn) return FQ_ERR_DTYPE;
    fq::TArgs a{};
    a.x = x;
    a.w = static_cast<const uint8_t*>(w);
    a.w2 = static_cast<const uint8_t*>(w2);
    a.w3 = static_cast<const uint8_t*>(w3);
    a.n1 = n1;
    a.n2 = n2;
    a.y = y;
    a.bias = bias;
    a.bias_len = bias ? bias_len : 0;
    a.mode = mode;
    a.N = N;
    a.K = K;
    a.U = U;
    a.GR = GR;
    a.recs = recs;
    a.T = (int)tiles;
    a.row_bytes = RB;
    const hipError_t e = fq::launch_gemvt(fn, a, (int)GT, W, lds, st);
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

// Batch-1 GEMV over packed rows.  mode 0: y = x . w (+ bias).  mode 1 (fused
// gate/up): y[n] = silu(x . w[n]) * (x . w2[n]), run as one GEMV over 2 N
// interleaved rows.  mode 2 (fused QKV): y = [x . w | x . w2 | x . w3] with
// n1 and n2 rows in w and w2 and N rows in all.
// gguf: the same kernel over the unmodified GGUF rows (the caller has
// validated the arguments as run_matmul does).
int packed_gemv(uint32_t dtype, const float* x, const void* w_packed, const void* w2_packed,
                const void* w3_packed, int n1, int n2, int mode, const float* bias,
                int64_t bias_len, float* y, int K, int N, hipStream_t st, bool gguf, int M,
                bool bias_full, uint8_t* fixed, size_t fixed_cap) {
    Geometry g;
    if (!geometry(dtype, g) || !packable(dtype)) return FQ_ERR_DTYPE;
    if (N < 0 || K < 0 || K % (gguf ? g.be : 256) != 0) return FQ_ERR_SHAPE;
    if (N == 0) return FQ_OK;
    if (!x || !w_packed || !y) return FQ_ERR_NULL;
    if (M != 1 && !(gguf && mode == 0 && M >= 2 && M <= 4)) return FQ_ERR_SHAPE;
    const uintptr_t amask = gguf ? 1 : 15;
    if ((reinterpret_cast<uintptr_t>(w_packed) & amask) != 0) return FQ_ERR_ALIGN;
    for (const void* p : {w2_packed, w3_packed})
        if (p && (reinterpret_cast<uintptr_t>(p) & amask) != 0) return FQ_ERR_ALIGN;
    const bool dual = mode == 1;
    const int NV = dual ? 2 * N : N;  // rows the kernel walks
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    if (K == 0) {  // y = 0 (silu(0) * 0 = 0 for the fused form)
        if (bias) return FQ_ERR_SHAPE;
        e = fq::launch_zero(reinterpret_cast<uint32_t*>(y), (size_t)N, di.cus, st);
        return e == hipSuccess ? FQ_OK : hip_fail(e);
    }
    if (!gguf) {
        // the arrangement of each packed matrix follows from its rows
        const int nr[3] = {mode == 2 ? n1 : N, mode == 2 ? n2 : N, mode == 2 ? N - n1 - n2 : N};
        const int nm = mode == 0 ? 1 : mode == 1 ? 2 : 3;
        int tiled = 0;
        for (int i = 0; i < nm; ++i) tiled += fq::packed_tiled((int)dtype, nr[i]) ? 1 : 0;
        if (tiled == nm)
            return run_gemvt(dtype, x, w_packed, w2_packed, w3_packed, n1, n2, mode, bias,
                             bias_len, y, K, N, st, di);
        if (tiled > 0) {  // fused QKV over both arrangements: one GEMV per matrix
            const void* ws[3] = {w_packed, w2_packed, w3_packed};
            int off = 0;
            for (int i = 0; i < 3; ++i) {
                if (nr[i] > 0) {
                    const int rc = packed_gemv(dtype, x, ws[i], nullptr, nullptr, 0, 0, 0, nullptr,
                                               0, y + off, K, nr[i], st, false);
                    if (rc != FQ_OK) return rc;
                }
                off += nr[i];
            }
            return FQ_OK;
        }
    }
    int units = 0, records = 0;
    fq::gemvp_geometry((int)dtype, K, &units, &records);
    size_t lds = 0;
    int wg = 0;
    const size_t lds_cap = std::min<size_t>(di.lds, 160 * 1024);
    // partial sums a work-group can buffer: a static 4096-entry array for the
    // packed kernel, the LDS left after the records and wave buffers for GGUF
    long pcap = 4096;
    int nl = 1;
    const void* fn =
        gguf ? fq::gemvg_kernel_fn((int)dtype, units, records, bias != nullptr, &lds, &wg, &nl, NV,
                                   M, mode)
             : fq::gemvp_kernel_fn((int)dtype, units, records, bias != nullptr, &lds, &wg, &nl,
                                   mode);
    // K split over blockIdx.y for several tokens whose records of a whole row
    // do not fit LDS (K = 18944: 2 x 85 KB): each work-group stages only the
    // records of its own K-slices and writes partial sums, [splits][M][N],
    // which the slab sum adds with the bias (the fewest splits that fit)
    int splits = 1, spl = 0;
    if (gguf && fn && M >= 2 && lds + 64 * 4 * M + 256 > lds_cap) {
        fn = fq::gemvg_kernel_fn((int)dtype, units, records, false, &lds, &wg, &nl, NV, M, mode);
        if (!fn) return FQ_ERR_SHAPE;
        const size_t rb = (size_t)fq::gemvp_record_bytes();
        const size_t wbufs = lds - (size_t)M * records * rb;
        const int nrec = records / units, ns_all = (units + 64 * nl - 1) / (64 * nl);
        for (int s = 2; s <= 8 && !spl; ++s) {
            const int sp = (ns_all + s - 1) / s;
            const size_t l = (size_t)M * std::min(units, sp * 64 * nl) * nrec * rb + wbufs;
            if (l + 64 * 4 * M * (size_t)sp + 256 <= lds_cap) {
                spl = sp;
                splits = (ns_all + sp - 1) / sp;
                lds = l;
            }
        }
        if (!spl) return FQ_ERR_SHAPE;
    }
    std::unique_ptr<StreamScratch::Lease> lease;
    uint8_t* slab = fixed;
    if (splits > 1) {
        const size_t need = (size_t)splits * M * NV * sizeof(float);
        if (fixed) {
            if (need > fixed_cap) return FQ_ERR_SHAPE;
        } else {
            lease.reset(new StreamScratch::Lease(stream_scratch(dev, st, 0)));
            const int rc = lease->get(need, st, &slab);
            // under graph capture without a reserved workspace: another kernel
            if (rc == FQ_ERR_WORKSPACE) return FQ_ERR_SHAPE;
            if (rc != FQ_OK) return rc;
        }
    }
    if (gguf) {
        // M tokens' partial sums per row and K-slice
        // (256 bytes left for the kernel's static LDS: its step counter)
        if (lds + 64 * 4 * M + 256 > lds_cap) return FQ_ERR_SHAPE;
        pcap = std::min<long>(4096, (long)(lds_cap - lds - 256) / (4 * M));
    }
    if (!fn || lds > lds_cap) return FQ_ERR_SHAPE;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, wg,
                                                     gguf ? lds + 4 * (size_t)M * pcap : lds);
    if (e != hipSuccess) return hip_fail(e);
    if (per_cu < 1) return FQ_ERR_SHAPE;
    const int wpb = wg / 64;
    // one work-group per resident slot, each owning a contiguous row range
    // with at least one row per wave, and whose row x K-slice partial sums fit
    // its LDS buffer (slices of 64 lane units)
    const long ns = spl ? spl : (units + 64 * nl - 1) / (64 * nl);
    long G = ((long)di.cus * per_cu + splits - 1) / splits;
    G = std::max(1L, std::min<long>(G, ((long)NV + wpb - 1) / wpb));
    auto max_rows = [&](long g) { return dual ? 2 * ((N + g - 1) / g) : (NV + g - 1) / g; };
    G = std::max<long>(G, ((long)NV * ns + pcap - 1) / pcap);
    while (max_rows(G) * ns > pcap) ++G;
    if (gguf) lds += 4 * (size_t)M * (max_rows(G) * ns);
    fq::GemvArgs a{};
    a.x = x;
    a.w = static_cast<const uint8_t*>(w_packed);
    a.w2 = static_cast<const uint8_t*>(w2_packed);
    a.w3 = static_cast<const uint8_t*>(w3_packed);
    a.n1 = n1;
    a.n2 = n2;
    a.y = y;
    a.bias = bias;
    a.bias_len = bias ? bias_len : 0;
    a.bias_mode = bias ? (bias_full ? 2 : 1) : 0;
    a.M = M;
    a.K = K;
    a.N = NV;
    a.U = units;
    a.Uc = records;
    a.row_bytes = gguf ? (K / g.be) * g.bb : (int)fq::packed_row_bytes((int)dtype, K);
    if (splits > 1) {
        a.part = reinterpret_cast<float*>(slab);
        a.spl = spl;
        a.bias = nullptr;
        a.bias_len = 0;
        a.bias_mode = 0;
    }
    e = fq::launch_raw(fn, a, (int)G, wg, lds, st, splits);
    if (e != hipSuccess || splits == 1) return e == hipSuccess ? FQ_OK : hip_fail(e);
    fq::MmqArgs r{};
    r.part = a.part;
    r.y = y;
    r.bias = bias;
    r.bias_len = bias ? bias_len : 0;
    r.bias_mode = bias ? (bias_full ? 2 : 1) : 0;
    r.M = M;
    r.N = NV;
    e = fq::launch_reduce(r, splits, st);
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

}  // namespace

extern "C" {

int fq_block_info(uint32_t dtype, int* block_elems, int* block_bytes) {
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
    if (block_elems) *block_elems = g.be;
    if (block_bytes) *block_bytes = g.bb;
    return FQ_OK;
}

const char* fq_status_str(int status) {
    switch (status) {
        case FQ_OK: return "ok";
        case FQ_ERR_DTYPE: return "unsupported quantized type";
        case FQ_ERR_SHAPE: return "invalid shape";
        case FQ_ERR_NULL: return "null pointer";
        case FQ_ERR_HIP: return "HIP runtime error";
        case FQ_ERR_NO_DEVICE: return "no HIP device";
        case FQ_ERR_ALIGN: return "packed buffer not 16-byte aligned";
        case FQ_ERR_WORKSPACE:
            return "workspace too small (reserve it with fq_reserve_workspace before graph "
                   "capture; fq_matmul_transB_noalloc: the call needs more than its fixed "
                   "64 MiB)";
        default: return "unknown status";
    }
}

int fq_last_hip_error(void) { return g_last_hip; }

int fq_gemv(uint32_t dtype, const float* x, const void* w, float* y, int K, int N, void* stream) {
    return run_matmul(dtype, x, w, nullptr, 0, 0, y, 1, K, N,
                      static_cast<hipStream_t>(stream));
}

int fq_gemv_batch(uint32_t dtype, const float* x, const void* w, float* y, int M, int K, int N,
                  void* stream) {
    if (M < 1 || M > 32) return FQ_ERR_SHAPE;
    return run_matmul(dtype, x, w, nullptr, 0, 0, y, M, K, N,
                      static_cast<hipStream_t>(stream));
}

int fq_matmul_prefill(uint32_t dtype, const float* x, const void* w, float* y, int M, int K,
                      int N, void* stream) {
    if (M < 1) return FQ_ERR_SHAPE;
    return run_matmul(dtype, x, w, nullptr, 0, 0, y, M, K, N,
                      static_cast<hipStream_t>(stream));
}

int fq_matmul_transB(uint32_t dtype, const float* x, const void* w, const float* bias,
                     int bias_ndim, int64_t bias_len, float* y, int M, int K, int N,
                     void* stream) {
    int mode = 0;
    if (bias && bias_ndim == 1) mode = 1;
    else if (bias && bias_ndim == 2) mode = 2;
    else if (bias && bias_ndim != 0) return FQ_ERR_SHAPE;
    return run_matmul(dtype, x, w, bias, mode, bias_len, y, M, K, N,
                      static_cast<hipStream_t>(stream));
}

int fq_matmul_transB_noalloc(uint32_t dtype, const float* x, const void* w, const float* bias,
                             int bias_ndim, int64_t bias_len, float* y, int M, int K, int N,
                             void* stream) {
    int mode = 0;
    if (bias && bias_ndim == 1) mode = 1;
    else if (bias && bias_ndim == 2) mode = 2;
    else if (bias && bias_ndim != 0) return FQ_ERR_SHAPE;
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    uint8_t* ws = nullptr;
    const int rc = noalloc_workspace(dev, &ws);
    if (rc != FQ_OK) return rc;
    return run_matmul(dtype, x, w, bias, mode, bias_len, y, M, K, N,
                      static_cast<hipStream_t>(stream), ws, kNoAllocBytes);
}

int fq_dequant_rows(uint32_t dtype, const void* w, float* out, int N, int K, void* stream) {
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
    if (N < 0 || K < 0) return FQ_ERR_SHAPE;
    if (N == 0 || K == 0) return FQ_OK;
    if (!w || !out) return FQ_ERR_NULL;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    const int nblk = (K + g.be - 1) / g.be;
    const int U = nblk * (g.be / 32);
    const size_t total = (size_t)N * U;
    int grid = (int)std::min<size_t>((total + 255) / 256, (size_t)di.cus * 16);
    e = fq::launch_dequant((int)dtype, static_cast<const uint8_t*>(w), out, N, K, U,
                           nblk * g.bb, grid, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

int64_t fq_packed_row_bytes(uint32_t dtype, int K) {
    Geometry g;
    if (!geometry(dtype, g) || !packable(dtype) || K <= 0 || K % 256 != 0) return 0;
    return fq::packed_row_bytes((int)dtype, K);
}

static int pack_common(uint32_t dtype, const void* src, void* dst, int N, int K, bool pack,
                       void* stream) {
    Geometry g;
    if (!geometry(dtype, g) || !packable(dtype)) return FQ_ERR_DTYPE;
    if (N < 0 || K < 0 || K % 256 != 0) return FQ_ERR_SHAPE;
    if (N == 0 || K == 0) return FQ_OK;
    if (!src || !dst) return FQ_ERR_NULL;
    const void* packed = pack ? dst : src;
    const void* gguf = pack ? src : dst;
    if ((reinterpret_cast<uintptr_t>(packed) & 15) != 0) return FQ_ERR_ALIGN;
    if ((reinterpret_cast<uintptr_t>(gguf) & 1) != 0) return FQ_ERR_ALIGN;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    e = fq::launch_pack((int)dtype, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst),
                        N, K, pack, di.cus * 8, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

int fq_pack_weights(uint32_t dtype, const void* w_gguf, void* w_packed, int N, int K,
                    void* stream) {
    return pack_common(dtype, w_gguf, w_packed, N, K, true, stream);
}

int fq_unpack_weights(uint32_t dtype, const void* w_packed, void* w_gguf, int N, int K,
                      void* stream) {
    return pack_common(dtype, w_packed, w_gguf, N, K, false, stream);
}


int fq_gemv_packed(uint32_t dtype, const float* x, const void* w_packed, const float* bias,
                   int64_t bias_len, float* y, int K, int N, void* stream) {
    return packed_gemv(dtype, x, w_packed, nullptr, nullptr, 0, 0, 0, bias, bias_len, y, K, N,
                       static_cast<hipStream_t>(stream), false);
}

int fq_ffn_up_fused_packed(uint32_t dtype, const float* x, const void* w_gate_packed,
                           const void* w_up_packed, float* y, int K, int N, void* stream) {
    if (!w_up_packed) return FQ_ERR_NULL;
    return packed_gemv(dtype, x, w_gate_packed, w_up_packed, nullptr, 0, 0, 1, nullptr, 0, y, K,
                       N, static_cast<hipStream_t>(stream), false);
}

int fq_fused_qkv_packed(uint32_t dtype, const float* x, const void* wq, const void* wk,
                        const void* wv, float* y, int K, int Nq, int Nk, int Nv, void* stream) {
    if (Nq < 0 || Nk < 0 || Nv < 0 || (int64_t)Nq + Nk + Nv > INT32_MAX) return FQ_ERR_SHAPE;
    if ((Nk && !wk) || (Nv && !wv)) return FQ_ERR_NULL;
    return packed_gemv(dtype, x, wq, wk, wv, Nq, Nk, 2, nullptr, 0, y, K, Nq + Nk + Nv,
                       static_cast<hipStream_t>(stream), false);
}

int fq_fused_qkv(uint32_t dtype, const float* x, const void* wq, const void* wk, const void* wv,
                 float* y, int M, int K, int Nq, int Nk, int Nv, void* stream) {
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
    if (M < 0 || K < 0 || Nq < 0 || Nk < 0 || Nv < 0 || K % g.be != 0) return FQ_ERR_SHAPE;
    if ((int64_t)Nq + Nk + Nv > INT32_MAX) return FQ_ERR_SHAPE;
    const int Nt = Nq + Nk + Nv;
    if (M == 0 || Nt == 0) return FQ_OK;
    if (!x || !y || (Nq && !wq) || (Nk && !wk) || (Nv && !wv)) return FQ_ERR_NULL;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const void* ws[3] = {wq, wk, wv};
    const int ns[3] = {Nq, Nk, Nv};
    if (M == 1) {  // the three outputs are contiguous slices of y
        // one launch over the three matrices' GGUF rows (the five formats
        // the batch-1 kernel reads; at every size: against three launches,
        // TinyLlama QKV 9.4 -> 4.5 us for Q4_0, 12.3 -> 4.5 us for Q8_0)
        if (packable(dtype)) {
            // a matrix of no rows is never read: any valid pointer stands in
            const void* any = Nq ? wq : Nk ? wk : wv;
            const int rc = packed_gemv(dtype, x, Nq ? wq : any, Nk ? wk : any, Nv ? wv : any, Nq,
                                       Nk, 2, nullptr, 0, y, K, Nt, st, true);
            if (rc != FQ_ERR_SHAPE) return rc;
        }
        int off = 0;
        for (int i = 0; i < 3; ++i) {
            if (ns[i] > 0) {
                const int rc = run_matmul(dtype, x, ws[i], nullptr, 0, 0, y + off, 1, K, ns[i], st);
                if (rc != FQ_OK) return rc;
            }
            off += ns[i];
        }
        return FQ_OK;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    uint8_t* buf = nullptr;
    const int nmax = std::max(Nq, std::max(Nk, Nv));
    StreamScratch::Lease lease(stream_scratch(dev, st, 1));
    const int rs = lease.get((size_t)M * nmax * sizeof(float), st, &buf);
    if (rs != FQ_OK) return rs;
    float* tmp = reinterpret_cast<float*>(buf);
    // The band kernel's token operands serve every matmul here that takes
    // it, one after another: the stream's slot-0 workspace is first grown to
    // the largest of their band-kernel needs, so none of these calls replaces
    // it (a call on another path clears the flag, and the next band call
    // prepares again).  Where that growth is refused (graph capture with a
    // smaller reserve) each call prepares its own.
    bool share = false;
    if (M <= 16 && K % 256 == 0) {
        size_t need = 0;
        for (int i = 0; i < 3; ++i)
            if (ns[i] > 0)
                for (int mt : {4, 3, 2}) need = std::max(need, mmqs_need(M, K, ns[i], di.cus, mt));
        StreamScratch::Lease l0(stream_scratch(dev, st, 0));
        uint8_t* p0 = nullptr;
        share = l0.get(need, st, &p0) == FQ_OK;
    }
    bool band_x = false;
    int off = 0;
    for (int i = 0; i < 3; ++i) {
        if (ns[i] > 0) {
            const int rc = run_matmul(dtype, x, ws[i], nullptr, 0, 0, tmp, M, K, ns[i], st,
                                      nullptr, 0, share ? &band_x : nullptr);
            if (rc != FQ_OK) return rc;
            e = fq::launch_copy_cols(tmp, y, M, ns[i], Nt, off, di.cus, st);
            if (e != hipSuccess) return hip_fail(e);
        }
        off += ns[i];
    }
    return FQ_OK;
}

int fq_ffn_down_residual(uint32_t dtype, const float* x, const void* w, const float* residual,
                         float* y, int M, int K, int N, void* stream) {
    if (!residual) return FQ_ERR_NULL;
    return run_matmul(dtype, x, w, residual, 2, (int64_t)M * N, y, M, K, N,
                      static_cast<hipStream_t>(stream));
}

int fq_ffn_down_residual_packed(uint32_t dtype, const float* x, const void* w_packed,
                                const float* residual, float* y, int K, int N, void* stream) {
    if (!residual) return FQ_ERR_NULL;
    return packed_gemv(dtype, x, w_packed, nullptr, nullptr, 0, 0, 0, residual, N, y, K, N,
                       static_cast<hipStream_t>(stream), false);
}

int fq_ffn_up_fused(uint32_t dtype, const float* x, const void* w_gate, const void* w_up, float* y,
                    int M, int K, int N, void* stream) {
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
    if (M < 0 || N < 0 || K < 0 || K % g.be != 0) return FQ_ERR_SHAPE;
    if (M == 0 || N == 0) return FQ_OK;
    if (!x || !w_gate || !w_up || !y) return FQ_ERR_NULL;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (M == 1 && packable(dtype)) {
        // one launch at every size: gate and up rows interleaved,
        // silu(gate) * up in the epilogue, straight from the GGUF bytes
        // (against two matmuls and the SiLU-multiply launch)
        const int rc = packed_gemv(dtype, x, w_gate, w_up, nullptr, 0, 0, 1, nullptr, 0, y, K, N,
                                   st, true);
        if (rc != FQ_ERR_SHAPE) return rc;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    uint8_t* buf = nullptr;
    StreamScratch::Lease lease(stream_scratch(dev, st, 1));
    const int rs = lease.get(2 * (size_t)M * N * sizeof(float), st, &buf);
    if (rs != FQ_OK) return rs;
    float* gate = reinterpret_cast<float*>(buf);
    float* up = gate + (size_t)M * N;
    // gate and up share x, M, K, N and the format: when the gate call takes
    // the band kernel, the up call does too and reuses its token operands
    // (one token-prep launch fewer: about 5 us)
    bool band_x = false;
    int rc = run_matmul(dtype, x, w_gate, nullptr, 0, 0, gate, M, K, N, st, nullptr, 0, &band_x);
    if (rc != FQ_OK) return rc;
    rc = run_matmul(dtype, x, w_up, nullptr, 0, 0, up, M, K, N, st, nullptr, 0, &band_x);
    if (rc != FQ_OK) return rc;
    e = fq::launch_silu_mul(gate, up, y, (size_t)M * N, di.cus, st);
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

int fq_reserve_workspace(int M_max, int K_max, int N_max, void* stream) {
    if (M_max < 0 || K_max < 0 || N_max < 0) return FQ_ERR_SHAPE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    // slot 0: the largest MFMA-path plan for up to M_max tokens (the split-K
    // slabs grow with splits x N, and fewer rows can mean more splits: every
    // row count that changes the tile count is tried, with K_max and, for the
    // prefill and band kernels, the largest multiple of 256 up to K_max)
    size_t need0 = 0;
    const int Kp = K_max - K_max % 256;
    for (int n = N_max; n > 0; n = n > 128 ? ((n - 1) / 128) * 128 : 0) {
        for (int m = 2; m <= M_max; ++m) {
            need0 = std::max(need0, plan_mmq(m, K_max, n, di.cus).total);
            if (m <= 16 && Kp > 0)  // band kernel (from M = 2), four- and two-tile bands
                for (int mt : {4, 3, 2}) need0 = std::max(need0, mmqs_need(m, Kp, n, di.cus, mt));
            if (m > 32 && Kp > 0) need0 = std::max(need0, plan_mmqp(m, Kp, n, di.cus, true).total);
            // the batch-1 kernel's K-split slabs for 2..4 tokens (at most 8)
            if (m <= 4) need0 = std::max(need0, (size_t)8 * m * n * sizeof(float));
        }
    }
    const size_t need1 = 2 * (size_t)M_max * N_max * sizeof(float);
    uint8_t* p = nullptr;
    if (need0) {
        StreamScratch::Lease l(stream_scratch(dev, st, 0));
        const int rc = l.get(need0, st, &p);
        if (rc != FQ_OK) return rc;
    }
    if (need1) {
        StreamScratch::Lease l(stream_scratch(dev, st, 1));
        const int rc = l.get(need1, st, &p);
        if (rc != FQ_OK) return rc;
    }
    return FQ_OK;
}

int fq_release_workspace(void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    e = hipStreamSynchronize(st);  // queued work may still read the buffers
    if (e != hipSuccess) return hip_fail(e);
    for (int slot = 0; slot < 2; ++slot) {
        StreamScratch& s = stream_scratch(dev, st, slot);
        std::lock_guard<std::mutex> lk(s.mu);
        for (uint8_t* r : s.retired) hipFree(r);
        s.retired.clear();
        if (s.p) hipFree(s.p);
        s.p = nullptr;
        s.n = 0;
    }
    return FQ_OK;
}

}  // extern "C"
