// ref_harness.cpp -- C entry points over the reference's OWN compiled CPU
// operator path, for use as a checker and as the timed CPU baseline.
//
// TEST INFRASTRUCTURE ONLY.  The Makefile beside this file compiles the
// reference's sources in place (/root/reference/src/...) together with this
// harness into oracle/_ref/libforge_ref.so.  Nothing here restates the
// reference: every call goes into the reference's own functions.
//
//   fqr_dequant_rows     -> forge::get_dequant_row_fn(dtype)  (quant_traits.cpp:33-52,
//                           rows from matmul.cpp:73-377)
//   fqr_matmul_transB    -> forge::ops::matmul_transB on CPU   (matmul.cpp:1134-1403,
//                           AVX2 kernels cpu_gemv.h)
//   fqr_ffn_up_fused     -> forge::ops::ffn_up_fused on CPU    (matmul.cpp:1472-1533)
//   fqr_fused_qkv        -> matmul_transB_fused_qkv_q4_0 / _q4_k (matmul.cpp:1535-1600,
//                           1639-1692)
//   fqr_fused_ffn_up     -> matmul_transB_fused_ffn_up_q4_0 / _q4_k (matmul.cpp:1766-1799,
//                           1694-1727)
//   fqr_fused_down_residual -> matmul_transB_fused_ffn_down_residual_q4_0 / _q6_k
//                           (matmul.cpp:1601-1637, 1729-1764)
#include <cstdint>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

#include <omp.h>

#include "forge/operator_matmul.h"
#include "forge/tensor.h"
#include "forge/types.h"

using forge::DataType;
using forge::DeviceType;
using forge::Tensor;
using forge::TensorPtr;

static TensorPtr wrap(const void* p, DataType dt, int64_t rows, int64_t cols) {
    return std::make_shared<Tensor>(Tensor::from_buffer(const_cast<void*>(p), dt, {rows, cols},
                                                        DeviceType::CPU, false));
}

extern "C" {

int fqr_dequant_rows(uint32_t dtype, const uint8_t* w, float* out, int N, int K) {
    auto fn = forge::get_dequant_row_fn(static_cast<DataType>(dtype));
    if (!fn) return -1;
    // The reference's Q6_K/K-quant row routines may write whole super-blocks
    // past K, so give them a buffer rounded up to 256.
    std::vector<float> row(((size_t)K + 255) / 256 * 256 + 256);
    for (int n = 0; n < N; ++n) {
        fn(w, row.data(), K, n);
        std::memcpy(out + (size_t)n * K, row.data(), sizeof(float) * (size_t)K);
    }
    return 0;
}

int fqr_matmul_transB(uint32_t dtype, const float* a, const uint8_t* w, float* out, int M, int K,
                      int N, int nthreads) {
    try {
        if (nthreads > 0) omp_set_num_threads(nthreads);
        auto ta = wrap(a, DataType::FP32, M, K);
        auto tb = wrap(w, static_cast<DataType>(dtype), N, K);
        auto y = forge::ops::matmul_transB(ta, tb, nullptr);
        std::memcpy(out, y->data(), sizeof(float) * (size_t)M * (size_t)N);
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

int fqr_ffn_up_fused(uint32_t dtype, const float* a, const uint8_t* w1, const uint8_t* w3,
                     float* out, int M, int K, int N, int nthreads) {
    try {
        if (nthreads > 0) omp_set_num_threads(nthreads);
        auto ta = wrap(a, DataType::FP32, M, K);
        auto t1 = wrap(w1, static_cast<DataType>(dtype), N, K);
        auto t3 = wrap(w3, static_cast<DataType>(dtype), N, K);
        auto y = forge::ops::ffn_up_fused(ta, t1, t3, N);
        std::memcpy(out, y->data(), sizeof(float) * (size_t)M * (size_t)N);
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

int fqr_fused_qkv(uint32_t dtype, const float* a, const uint8_t* wq, const uint8_t* wk,
                  const uint8_t* wv, float* out, int M, int K, int Nq, int Nk, int Nv,
                  int nthreads) {
    try {
        if (nthreads > 0) omp_set_num_threads(nthreads);
        const DataType dt = static_cast<DataType>(dtype);
        auto ta = wrap(a, DataType::FP32, M, K);
        auto tq = wrap(wq, dt, Nq, K), tk = wrap(wk, dt, Nk, K), tv = wrap(wv, dt, Nv, K);
        TensorPtr y;
        if (dt == DataType::Q4_0) y = forge::ops::matmul_transB_fused_qkv_q4_0(ta, tq, tk, tv);
        else if (dt == DataType::Q4_K) y = forge::ops::matmul_transB_fused_qkv_q4_k(ta, tq, tk, tv);
        else return -1;
        std::memcpy(out, y->data(), sizeof(float) * (size_t)M * (size_t)(Nq + Nk + Nv));
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

int fqr_fused_ffn_up(uint32_t dtype, const float* a, const uint8_t* wg, const uint8_t* wu,
                     float* out, int M, int K, int N, int nthreads) {
    try {
        if (nthreads > 0) omp_set_num_threads(nthreads);
        const DataType dt = static_cast<DataType>(dtype);
        auto ta = wrap(a, DataType::FP32, M, K);
        auto tg = wrap(wg, dt, N, K), tu = wrap(wu, dt, N, K);
        TensorPtr y;
        if (dt == DataType::Q4_0) y = forge::ops::matmul_transB_fused_ffn_up_q4_0(ta, tg, tu);
        else if (dt == DataType::Q4_K) y = forge::ops::matmul_transB_fused_ffn_up_q4_k(ta, tg, tu);
        else return -1;
        std::memcpy(out, y->data(), sizeof(float) * (size_t)M * (size_t)N);
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

int fqr_fused_down_residual(uint32_t dtype, const float* a, const uint8_t* w, const float* r,
                            float* out, int M, int K, int N, int nthreads) {
    try {
        if (nthreads > 0) omp_set_num_threads(nthreads);
        const DataType dt = static_cast<DataType>(dtype);
        auto ta = wrap(a, DataType::FP32, M, K);
        auto tw = wrap(w, dt, N, K);
        auto tr = wrap(r, DataType::FP32, M, N);
        TensorPtr y;
        if (dt == DataType::Q4_0)
            y = forge::ops::matmul_transB_fused_ffn_down_residual_q4_0(ta, tw, tr);
        else if (dt == DataType::Q6_K)
            y = forge::ops::matmul_transB_fused_ffn_down_residual_q6_k(ta, tw, tr);
        else return -1;
        std::memcpy(out, y->data(), sizeof(float) * (size_t)M * (size_t)N);
        return 0;
    } catch (const std::exception&) {
        return -2;
    }
}

int fqr_max_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
