// fq_capi.cpp -- the extern "C" entry points declared in include/forge_q.h:
// argument validation, launch planning and the split-K workspace.
//
// The planner mirrors the reference's dispatch on M (matmul.cpp:1150-1286:
// M == 1 -> GEMV, 1 < M <= 32 -> batched GEMV, M > 32 -> prefill) and picks,
// per call, how many K-splits and persistent work-groups fill the chip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/forge_q.h"
#include "fq_kernels.h"

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

// Split-K partial buffers: one grow-only buffer per (device, stream), kept
// until process exit, so calls on different streams never share one.
float* workspace(int dev, hipStream_t st, size_t bytes, hipError_t& err) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> bufs;
    std::lock_guard<std::mutex> lk(mu);
    auto& b = bufs[{dev, st}];
    err = hipSuccess;
    if (b.second < bytes) {
        if (b.first) {
            // the old buffer may still be read by queued work on this stream
            err = hipStreamSynchronize(st);
            if (err != hipSuccess) return nullptr;
            hipFree(b.first);
            b = {nullptr, 0};
        }
        err = hipMalloc(&b.first, bytes);
        if (err != hipSuccess) {
            b = {nullptr, 0};
            return nullptr;
        }
        b.second = bytes;
    }
    return static_cast<float*>(b.first);
}

constexpr int kWG = 256;
constexpr int kT = 16;

// Plan a launch of gemv_kernel for M tokens processed MT at a time.
int plan(uint32_t dtype, const Geometry& g, int M, int K, int N, int MT, const DevInfo& di,
         fq::LaunchCfg& c, int& U, int& Uc) {
    U = K / 32;
    const int rows_per_wg = (kWG / 64) * (64 / kT);
    const long RG = (N + rows_per_wg - 1) / rows_per_wg;
    const int TG = (M + MT - 1) / MT;
    const long target = 2L * di.cus;
    int S = 1;
    while (RG * S * TG < target && U / (2 * S) >= 2 * kT) S *= 2;
    auto lds_of = [&](int uc) { return (size_t)MT * uc * 36 * sizeof(float); };
    const size_t lds_cap = std::min<size_t>(di.lds, 160 * 1024);
    while (lds_of((U + S - 1) / S) > lds_cap) ++S;
    Uc = (U + S - 1) / S;
    S = (U + Uc - 1) / Uc;
    c.T = kT;
    c.MT = MT;
    c.splits = S;
    c.token_groups = TG;
    c.lds_bytes = lds_of(Uc);
    int per_cu = 0;
    const void* fn = fq::gemv_kernel_fn((int)dtype, kT, MT);
    if (!fn) return FQ_ERR_DTYPE;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kWG, c.lds_bytes);
    if (e != hipSuccess) return hip_fail(e);
    if (per_cu < 1) per_cu = 1;
    long gx = (long)di.cus * per_cu / ((long)S * TG);
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
    if (K == 0) {
        hipError_t e = hipMemsetAsync(y, 0, sizeof(float) * (size_t)M * N, st);
        return e == hipSuccess ? FQ_OK : hip_fail(e);
    }
    if (!x || !w || !y) return FQ_ERR_NULL;
    if (bias_mode != 0 && !bias) return FQ_ERR_NULL;
    if (bias_mode == 2 && bias_len < (int64_t)M * N) return FQ_ERR_SHAPE;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    const DevInfo di = device_info(dev);

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
    a.Uc = Uc;
    a.row_bytes = (K / g.be) * g.bb;
    a.part = nullptr;
    if (c.splits > 1) {
        a.part = workspace(dev, st, sizeof(float) * (size_t)c.splits * M * N, e);
        if (!a.part) return hip_fail(e);
    }
    e = fq::launch_gemv((int)dtype, a, c, st);
    if (e != hipSuccess) return hip_fail(e);
    if (c.splits > 1) {
        size_t MN = (size_t)M * N;
        int grid = (int)std::min<size_t>((MN + 255) / 256, (size_t)di.cus * 8);
        e = fq::launch_finalize(a.part, y, c.splits, M, N, bias, bias_mode, bias_len, grid, st);
        if (e != hipSuccess) return hip_fail(e);
    }
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

}  // extern "C"
