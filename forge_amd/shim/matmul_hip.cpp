// matmul_hip.cpp -- the reference-side half of the drop-in: compiled into
// Forge's operator library (not into libforge_q.so) in place of the USE_CUDA
// device branches of src/operators/cpu/matmul.cpp.  It turns Forge tensors
// into the plain pointers of include/forge_q.h and the library's int status
// back into the std::runtime_error Forge's callers expect.
//
//   matmul_transB_device     the device branch of ops::matmul_transB
//                            (matmul.cpp:1149-1286), including apply_bias
//                            (matmul.cpp:1005-1049);
//   dequantize_weight_device ops::dequantize_weight for a weight that lives on
//                            the device (matmul.cpp:980-1003);
//   ffn_up_fused_device      the device branch of ops::ffn_up_fused
//                            (matmul.cpp:1472-1533).
//
// Every call is asynchronous on the null stream, as the reference's launchers
// are (cuda_gemv.h:29-33 pass stream 0).  tests/test_shim.py compiles this file
// against the reference's own headers.
#include <stdexcept>
#include <string>

#include "forge/operator_matmul.h"
#include "forge_q.h"

namespace forge {
namespace ops {

namespace {

void fq_check(int st, const char* what) {
    if (st == FQ_OK) return;
    if (st == FQ_ERR_DTYPE)  // the reference's text (matmul.cpp:1163-1165)
        throw std::runtime_error("Unsupported quantized type in matmul_transB CUDA");
    std::string msg = std::string(what) + ": " + fq_status_str(st);
    if (st == FQ_ERR_HIP) msg += " (hipError " + std::to_string(fq_last_hip_error()) + ")";
    throw std::runtime_error(msg);
}

// bias on the output's device, as apply_bias copies a host bias (matmul.cpp:1011-1019)
TensorPtr bias_on(const TensorPtr& bias, DeviceType dev) {
    if (!bias || bias->device() == dev) return bias;
    auto b = std::make_shared<Tensor>(bias->dtype(), bias->shape(), dev);
    b->copy_from(*bias);
    return b;
}

}  // namespace

// After matmul_transB's own ndim / K checks (matmul.cpp:1135-1146) and the
// allocation of `out` on a's device (matmul.cpp:1148).
void matmul_transB_device(const TensorPtr& a, const TensorPtr& b, const TensorPtr& bias,
                          const TensorPtr& out, int M, int K, int N) {
    const TensorPtr bd = bias_on(bias, out->device());
    fq_check(fq_matmul_transB(static_cast<uint32_t>(b->dtype()),
                              static_cast<const float*>(a->data()), b->data(),
                              bd ? static_cast<const float*>(bd->data()) : nullptr,
                              bd ? static_cast<int>(bd->ndim()) : 0, bd ? bd->numel() : 0,
                              static_cast<float*>(out->data()), M, K, N, nullptr),
             "matmul_transB");
}

// A quantized [N, K] weight on the device -> a new FP32 [N, K] tensor there,
// bit-identical to dequantize_weight's CPU rows.
TensorPtr dequantize_weight_device(const TensorPtr& weight) {
    const int N = static_cast<int>(weight->shape()[0]);
    const int K = static_cast<int>(weight->shape()[1]);
    auto out = std::make_shared<Tensor>(DataType::FP32, weight->shape(), weight->device());
    fq_check(fq_dequant_rows(static_cast<uint32_t>(weight->dtype()), weight->data(),
                             static_cast<float*>(out->data()), N, K, nullptr),
             "dequantize_weight");
    return out;
}

// SiLU(input . w1^T) * (input . w3^T) for input [M, K] and w1, w3 [N, K] of
// one dtype: a new FP32 [M, N] tensor on input's device.
TensorPtr ffn_up_fused_device(const TensorPtr& input, const TensorPtr& w1, const TensorPtr& w3,
                              int intermediate_dim) {
    const int M = static_cast<int>(input->shape()[0]);
    const int K = static_cast<int>(input->shape()[1]);
    const int N = intermediate_dim;
    if (w1->dtype() != w3->dtype() || w1->shape()[0] != N || w3->shape()[0] != N ||
        w1->shape()[1] != K || w3->shape()[1] != K)
        throw std::runtime_error("ffn_up_fused: gate and up weights differ in shape or dtype");
    auto out = std::make_shared<Tensor>(DataType::FP32, std::vector<int64_t>{M, N},
                                        input->device());
    fq_check(fq_ffn_up_fused(static_cast<uint32_t>(w1->dtype()),
                             static_cast<const float*>(input->data()), w1->data(), w3->data(),
                             static_cast<float*>(out->data()), M, K, N, nullptr),
             "ffn_up_fused");
    return out;
}

}  // namespace ops
}  // namespace forge
