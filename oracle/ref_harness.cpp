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

int fqr_max_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
