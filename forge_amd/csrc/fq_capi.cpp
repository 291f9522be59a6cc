// fq_capi.cpp -- the extern "C" entry points declared in include/forge_q.h:
// argument validation, launch planning and the split-K workspace.
//
// The planner mirrors the reference's dispatch on M (matmul.cpp:1150-1286:
// M == 1 -> GEMV, 1 < M <= 32 -> batched GEMV, M > 32 -> prefill) and picks,
// per call, how many K-splits and persistent work-groups fill the chip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cstdio>
#include <cstdint>
#include <map>
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
        default: return false;
    }
}

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
    hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev);
    int lds = 0;
    hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    d.lds = (size_t)lds;
    if (d.cus <= 0) d.cus = 256;
    if (d.lds == 0) d.lds = 64 * 1024;
    cache[dev] = d;
    return d;
}

// Split-K workspace: one grow-only pair of buffers per (device, stream) --
// partial sums and arrival counters -- kept until process exit, so calls on
// different streams never share one.  Counters are zeroed when allocated and
// every call leaves them zero again.
struct Workspace {
    float* part = nullptr;
    size_t part_bytes = 0;
    unsigned* cnt = nullptr;
    size_t cnt_words = 0;
};

hipError_t workspace(int dev, hipStream_t st, size_t part_bytes, size_t cnt_words, int grid,
                     float** part, unsigned** cnt) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, Workspace> bufs;
    std::lock_guard<std::mutex> lk(mu);
    Workspace& w = bufs[{dev, st}];
    hipError_t err = hipSuccess;
    if (w.part_bytes < part_bytes || w.cnt_words < cnt_words) {
        // the old buffers may still be in use by queued work on this stream
        if (w.part || w.cnt) {
            err = hipStreamSynchronize(st);
            if (err != hipSuccess) return err;
        }
        if (w.part_bytes < part_bytes) {
            if (w.part) hipFree(w.part);
            w.part = nullptr;
            w.part_bytes = 0;
            err = hipMalloc(reinterpret_cast<void**>(&w.part), part_bytes);
            if (err != hipSuccess) return err;
            w.part_bytes = part_bytes;
        }
        if (w.cnt_words < cnt_words) {
            if (w.cnt) hipFree(w.cnt);
            w.cnt = nullptr;
            w.cnt_words = 0;
            err = hipMalloc(reinterpret_cast<void**>(&w.cnt), cnt_words * sizeof(unsigned));
            if (err != hipSuccess) return err;
            w.cnt_words = cnt_words;
            err = fq::launch_zero(w.cnt, cnt_words, grid, st);
            if (err != hipSuccess) return err;
        }
    }
    *part = w.part;
    *cnt = w.cnt;
    return hipSuccess;
}

constexpr int kWG = 256;
constexpr int kT = 16;
constexpr int kRowsPerWG = 16;
constexpr int kMaxNU = 8;

// Plan a launch of gemv_kernel for M tokens processed MT at a time: as few
// K-splits as keep every lane at <= 8 units per row (more only when there are
// fewer row groups than CUs), then enough persistent work-groups to fill the
// chip once.
int plan(uint32_t dtype, const Geometry& g, int M, int K, int N, int MT, const DevInfo& di,
         fq::LaunchCfg& c, int& U, int& Uc) {
    (void)g;
    U = K / 32;
    const long RG = (N + kRowsPerWG - 1) / kRowsPerWG;
    const int TG = (M + MT - 1) / MT;
    int S = std::max(1, (U + kMaxNU * kT - 1) / (kMaxNU * kT));
    while (RG * S * TG < di.cus && (U + S) / (S + 1) >= 2 * kT) ++S;
    auto lds_of = [&](int uc) { return (size_t)MT * uc * 36 * sizeof(float); };
    const size_t lds_cap = std::min<size_t>(di.lds, 160 * 1024);
    while (lds_of((U + S - 1) / S) > lds_cap) ++S;
    Uc = U > 0 ? (U + S - 1) / S : 0;
    S = U > 0 ? (U + Uc - 1) / Uc : 1;
    const int nu = (Uc + kT - 1) / kT;
    c.T = kT;
    c.MT = MT;
    c.NU = nu <= 2 ? 2 : nu <= 4 ? 4 : 8;
    c.splits = S;
    c.token_groups = TG;
    c.lds_bytes = lds_of(Uc);
    const void* fn = fq::gemv_kernel_fn((int)dtype, kT, MT, c.NU);
    if (!fn) return FQ_ERR_DTYPE;
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWG, c.lds_bytes);
    if (e != hipSuccess) return hip_fail(e);
    if (per_cu < 1) per_cu = 1;
    const long gx = (long)di.cus * per_cu / ((long)S * TG);
    c.grid_x = (int)std::max(1L, std::min(RG, gx));
    return FQ_OK;
}

int run_matmul(uint32_t dtype, const float* x, const void* w, const float* bias, int bias_mode,
               int64_t bias_len, float* y, int M, int K, int N, int MT, hipStream_t st) {
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

    if (M == 1 && K > 0) {
        // batch 1: persistent work-groups, as many as fit on every CU
        const int U1 = K / 32;
        static const int wg_env = [] {
            const char* v = getenv("FQ_GEMV1_WG");
            return v ? atoi(v) : 1024;
        }();
        int wg = wg_env;
        size_t lds = fq::gemv1_lds_bytes((int)dtype, U1, wg);
        const void* fn = fq::gemv1_kernel_fn((int)dtype, bias_mode != 0, wg);
        static const bool no_rowstep = getenv("FQ_NO_ROWSTEP") != nullptr;
        int npr = 0;
        size_t lds_r = 0;
        int wg_r = 0;
        const void* fr = no_rowstep ? nullptr
                                    : fq::gemv1r_kernel_fn((int)dtype, U1, (K / g.be) * g.bb,
                                                           bias_mode != 0, &npr, &lds_r, &wg_r);
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
                a.M = 1;
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

    fq::LaunchCfg c{};
    int U = 0, Uc = 0;
    int rc = plan(dtype, g, M, K, N, MT, di, c, U, Uc);
    if (rc != FQ_OK) return rc;

    fq::GemvArgs a{};
    a.x = x;
    a.w = static_cast<const uint8_t*>(w);
    a.y = y;
    a.bias = bias;
    a.bias_len = bias_len;
    a.bias_mode = bias_mode;
    a.M = M;
    a.K = K;
    a.N = N;
    a.U = U;
    a.Uc = std::max(Uc, 1);
    a.row_bytes = (K / g.be) * g.bb;
    a.rg_total = (N + kRowsPerWG - 1) / kRowsPerWG;
    a.part = nullptr;
    a.counters = nullptr;
    if (c.splits > 1) {
        e = workspace(dev, st, sizeof(float) * (size_t)c.splits * M * N,
                      (size_t)c.token_groups * a.rg_total, di.cus, &a.part, &a.counters);
        if (e != hipSuccess) return hip_fail(e);
    }
    e = fq::launch_gemv((int)dtype, a, c, st);
    if (e != hipSuccess) return hip_fail(e);
    return FQ_OK;
}

int pick_mt(int M) {
    if (M <= 1) return 1;
    if (M == 2) return 2;
    return 4;
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
        default: return "unknown status";
    }
}

int fq_last_hip_error(void) { return g_last_hip; }

int fq_gemv(uint32_t dtype, const float* x, const void* w, float* y, int K, int N, void* stream) {
    return run_matmul(dtype, x, w, nullptr, 0, 0, y, 1, K, N, 1,
                      static_cast<hipStream_t>(stream));
}

int fq_gemv_batch(uint32_t dtype, const float* x, const void* w, float* y, int M, int K, int N,
                  void* stream) {
    if (M < 1 || M > 32) return FQ_ERR_SHAPE;
    return run_matmul(dtype, x, w, nullptr, 0, 0, y, M, K, N, pick_mt(M),
                      static_cast<hipStream_t>(stream));
}

int fq_matmul_prefill(uint32_t dtype, const float* x, const void* w, float* y, int M, int K,
                      int N, void* stream) {
    if (M < 1) return FQ_ERR_SHAPE;
    return run_matmul(dtype, x, w, nullptr, 0, 0, y, M, K, N, pick_mt(M),
                      static_cast<hipStream_t>(stream));
}

int fq_matmul_transB(uint32_t dtype, const float* x, const void* w, const float* bias,
                     int bias_ndim, int64_t bias_len, float* y, int M, int K, int N,
                     void* stream) {
    int mode = 0;
    if (bias && bias_ndim == 1) mode = 1;
    else if (bias && bias_ndim == 2) mode = 2;
    else if (bias && bias_ndim != 0) return FQ_ERR_SHAPE;
    return run_matmul(dtype, x, w, bias, mode, bias_len, y, M, K, N, pick_mt(M),
                      static_cast<hipStream_t>(stream));
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
    if (!geometry(dtype, g) || K <= 0 || K % 256 != 0) return 0;
    return fq::packed_row_bytes((int)dtype, K);
}

static int pack_common(uint32_t dtype, const void* src, void* dst, int N, int K, bool pack,
                       void* stream) {
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
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
    Geometry g;
    if (!geometry(dtype, g)) return FQ_ERR_DTYPE;
    if (N < 0 || K < 0 || K % 256 != 0) return FQ_ERR_SHAPE;
    if (N == 0) return FQ_OK;
    if (!x || !w_packed || !y) return FQ_ERR_NULL;
    if ((reinterpret_cast<uintptr_t>(w_packed) & 15) != 0) return FQ_ERR_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);
    if (K == 0) {
        if (bias) return FQ_ERR_SHAPE;
        e = fq::launch_zero(reinterpret_cast<uint32_t*>(y), (size_t)N, di.cus, st);
        return e == hipSuccess ? FQ_OK : hip_fail(e);
    }
    int units = 0, records = 0;
    fq::gemvp_geometry((int)dtype, K, &units, &records);
    size_t lds = 0;
    int wg = 0;
    const void* fn = fq::gemvp_kernel_fn((int)dtype, units, records, bias != nullptr, &lds, &wg);
    if (!fn || lds > std::min<size_t>(di.lds, 160 * 1024)) return FQ_ERR_SHAPE;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, wg, lds);
    if (e != hipSuccess) return hip_fail(e);
    if (per_cu < 1) return FQ_ERR_SHAPE;
    const int wpb = wg / 64;
    // one work-group per resident slot, each owning a contiguous row range of
    // at most 4096 rows (its LDS result buffer) and at least one row per wave
    long G = (long)di.cus * per_cu;
    G = std::max(1L, std::min<long>(G, ((long)N + wpb - 1) / wpb));
    G = std::max<long>(G, ((long)N + 4095) / 4096);
    fq::GemvArgs a{};
    a.x = x;
    a.w = static_cast<const uint8_t*>(w_packed);
    a.y = y;
    a.bias = bias;
    a.bias_len = bias ? bias_len : 0;
    a.bias_mode = bias ? 1 : 0;
    a.M = 1;
    a.K = K;
    a.N = N;
    a.U = units;
    a.Uc = records;
    a.row_bytes = (int)fq::packed_row_bytes((int)dtype, K);
    e = fq::launch_raw(fn, a, (int)G, wg, lds, st);
    return e == hipSuccess ? FQ_OK : hip_fail(e);
}

}  // extern "C"
