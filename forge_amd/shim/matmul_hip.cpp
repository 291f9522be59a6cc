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
//                            (matmul.cpp:1472-1533);
//   matmul_transB_dual_device            ops::matmul_transB_dual
//                                        (matmul.cpp:1405-1470);
//   matmul_transB_fused_qkv_device       the fused QKV operators
//                                        (_q4_0 matmul.cpp:1535-1600, _q4_k :1639-1692);
//   matmul_transB_fused_ffn_up_device    the fused gate+up+SiLU operators
//                                        (_q4_0 :1766-1799, _q4_k :1694-1727);
//   matmul_transB_fused_ffn_down_residual_device
//                                        the fused down + residual operators
//                                        (_q4_0 :1601-1637, _q6_k :1729-1764).
// The reference's fused operators are CPU-only: on a device tensor they throw
// "... is CPU-only".  The device branches below take the place of that throw,
// after the same 2-D and dtype checks, so the engines' calls
// (generic_engine.cpp:345, 378, 770-806) run on the GPU unchanged.
//
// Every call is asynchronous on the null stream, as the reference's launchers
// are (cuda_gemv.h:29-33 pass stream 0).  tests/test_shim.py compiles this file
// against the reference's own headers.
#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>
#include <vector>

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

void need_2d(const char* op, std::initializer_list<const TensorPtr*> ts) {
    for (const TensorPtr* t : ts)
        if ((*t)->ndim() != 2) throw std::runtime_error(std::string(op) + " expects 2D tensors");
}

void need_dtype(const char* op, const char* name, DataType dt,
                std::initializer_list<const TensorPtr*> ws) {
    for (const TensorPtr* w : ws)
        if ((*w)->dtype() != dt)
            throw std::runtime_error(std::string(op) + " requires " + name + " weights");
}

TensorPtr fp32_on(DeviceType dev, int64_t rows, int64_t cols) {
    return std::make_shared<Tensor>(DataType::FP32, std::vector<int64_t>{rows, cols}, dev);
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

// [M, N1 + N2] = [a . b1^T | a . b2^T].  One dtype: one fq_fused_qkv call
// (a single activation staging at M = 1).  Two dtypes (a Q4_K_M model's Q4_K
// key and Q6_K value projections): two matmuls.  At M = 1 each writes its
// slice of the output row directly; for more rows each writes a stream-ordered
// temporary (hipMallocAsync) whose rows a strided device copy interleaves
// into the output, as the reference's CUDA branch does with per-row
// cudaMemcpyAsync, and the temporary is released in stream order
// (hipFreeAsync): nothing waits on the host.
TensorPtr matmul_transB_dual_device(const TensorPtr& a, const TensorPtr& b1,
                                    const TensorPtr& b2) {
    need_2d("matmul_transB_dual", {&a, &b1, &b2});
    const int M = static_cast<int>(a->shape()[0]);
    const int K = static_cast<int>(a->shape()[1]);
    const int N1 = static_cast<int>(b1->shape()[0]);
    const int N2 = static_cast<int>(b2->shape()[0]);
    if (b1->shape()[1] != K || b2->shape()[1] != K)
        throw std::runtime_error("matmul_transB_dual: dimension mismatch");
    auto out = fp32_on(a->device(), M, N1 + N2);
    const float* x = static_cast<const float*>(a->data());
    float* y = static_cast<float*>(out->data());
    if (b1->dtype() == b2->dtype()) {
        fq_check(fq_fused_qkv(static_cast<uint32_t>(b1->dtype()), x, b1->data(), b2->data(),
                              nullptr, y, M, K, N1, N2, 0, nullptr),
                 "matmul_transB_dual");
        return out;
    }
    const TensorPtr* ws[2] = {&b1, &b2};
    const int ns[2] = {N1, N2};
    auto hip_check = [](hipError_t e, const char* what) {
        if (e != hipSuccess)
            throw std::runtime_error(std::string("matmul_transB_dual: ") + what + " failed (" +
                                     std::to_string(static_cast<int>(e)) + ")");
    };
    int off = 0;
    for (int i = 0; i < 2; ++i) {
        const uint32_t dt = static_cast<uint32_t>((*ws[i])->dtype());
        if (M == 1 || ns[i] == 0) {
            fq_check(fq_matmul_transB(dt, x, (*ws[i])->data(), nullptr, 0, 0, y + off, M, K, ns[i],
                                      nullptr),
                     "matmul_transB_dual");
        } else if (M > 0) {
            void* part = nullptr;
            hip_check(hipMallocAsync(&part, sizeof(float) * (size_t)M * ns[i], nullptr),
                      "hipMallocAsync");
            fq_check(fq_matmul_transB(dt, x, (*ws[i])->data(), nullptr, 0, 0,
                                      static_cast<float*>(part), M, K, ns[i], nullptr),
                     "matmul_transB_dual");
            hip_check(hipMemcpy2DAsync(y + off, sizeof(float) * (N1 + N2), part,
                                       sizeof(float) * ns[i], sizeof(float) * ns[i], M,
                                       hipMemcpyDeviceToDevice, nullptr),
                      "hipMemcpy2DAsync");
            hip_check(hipFreeAsync(part, nullptr), "hipFreeAsync");
        }
        off += ns[i];
    }
    return out;
}

// Fused QKV for a device input: [M, Nq + Nk + Nv].  `op` / `dt` name the
// reference operator and the dtype it requires (Q4_0 or Q4_K).
TensorPtr matmul_transB_fused_qkv_device(const char* op, DataType dt, const char* dt_name,
                                         const TensorPtr& input, const TensorPtr& wq,
                                         const TensorPtr& wk, const TensorPtr& wv) {
    need_2d(op, {&input, &wq, &wk, &wv});
    need_dtype(op, dt_name, dt, {&wq, &wk, &wv});
    const int M = static_cast<int>(input->shape()[0]);
    const int K = static_cast<int>(input->shape()[1]);
    const int Nq = static_cast<int>(wq->shape()[0]);
    const int Nk = static_cast<int>(wk->shape()[0]);
    const int Nv = static_cast<int>(wv->shape()[0]);
    auto out = fp32_on(input->device(), M, static_cast<int64_t>(Nq) + Nk + Nv);
    fq_check(fq_fused_qkv(static_cast<uint32_t>(dt), static_cast<const float*>(input->data()),
                          wq->data(), wk->data(), wv->data(), static_cast<float*>(out->data()), M,
                          K, Nq, Nk, Nv, nullptr),
             op);
    return out;
}

// Fused gate + up + SiLU for a device input: [M, N] = silu(x . g^T) * (x . u^T).
TensorPtr matmul_transB_fused_ffn_up_device(const char* op, DataType dt, const char* dt_name,
                                            const TensorPtr& input, const TensorPtr& w_gate,
                                            const TensorPtr& w_up) {
    need_2d(op, {&input, &w_gate, &w_up});
    need_dtype(op, dt_name, dt, {&w_gate, &w_up});
    const int M = static_cast<int>(input->shape()[0]);
    const int K = static_cast<int>(input->shape()[1]);
    const int N = static_cast<int>(w_gate->shape()[0]);
    if (w_up->shape()[0] != N)
        throw std::runtime_error(std::string(op) + ": gate and up weights differ in shape");
    auto out = fp32_on(input->device(), M, N);
    fq_check(fq_ffn_up_fused(static_cast<uint32_t>(dt), static_cast<const float*>(input->data()),
                             w_gate->data(), w_up->data(), static_cast<float*>(out->data()), M, K,
                             N, nullptr),
             op);
    return out;
}

// Fused down projection + residual for a device input: [M, N] = x . w^T + r.
TensorPtr matmul_transB_fused_ffn_down_residual_device(const char* op, DataType dt,
                                                       const char* dt_name,
                                                       const TensorPtr& input,
                                                       const TensorPtr& weight,
                                                       const TensorPtr& residual) {
    need_2d(op, {&input, &weight, &residual});
    need_dtype(op, dt_name, dt, {&weight});
    const int M = static_cast<int>(input->shape()[0]);
    const int K = static_cast<int>(input->shape()[1]);
    const int N = static_cast<int>(weight->shape()[0]);
    if (residual->shape()[0] != M || residual->shape()[1] != N)
        throw std::runtime_error(std::string(op) + ": residual shape mismatch");
    const TensorPtr r = bias_on(residual, input->device());
    auto out = fp32_on(input->device(), M, N);
    fq_check(fq_ffn_down_residual(static_cast<uint32_t>(dt),
                                  static_cast<const float*>(input->data()), weight->data(),
                                  static_cast<const float*>(r->data()),
                                  static_cast<float*>(out->data()), M, K, N, nullptr),
             op);
    return out;
}

// The six named operators, each its reference name and required dtype.
TensorPtr matmul_transB_fused_qkv_q4_0_device(const TensorPtr& input, const TensorPtr& wq,
                                              const TensorPtr& wk, const TensorPtr& wv) {
    return matmul_transB_fused_qkv_device("matmul_transB_fused_qkv_q4_0", DataType::Q4_0, "Q4_0",
                                          input, wq, wk, wv);
}
TensorPtr matmul_transB_fused_qkv_q4_k_device(const TensorPtr& input, const TensorPtr& wq,
                                              const TensorPtr& wk, const TensorPtr& wv) {
    return matmul_transB_fused_qkv_device("matmul_transB_fused_qkv_q4_k", DataType::Q4_K, "Q4_K",
                                          input, wq, wk, wv);
}
TensorPtr matmul_transB_fused_ffn_up_q4_0_device(const TensorPtr& input, const TensorPtr& w_gate,
                                                 const TensorPtr& w_up) {
    return matmul_transB_fused_ffn_up_device("matmul_transB_fused_ffn_up_q4_0", DataType::Q4_0,
                                             "Q4_0", input, w_gate, w_up);
}
TensorPtr matmul_transB_fused_ffn_up_q4_k_device(const TensorPtr& input, const TensorPtr& w_gate,
                                                 const TensorPtr& w_up) {
    return matmul_transB_fused_ffn_up_device("matmul_transB_fused_ffn_up_q4_k", DataType::Q4_K,
                                             "Q4_K", input, w_gate, w_up);
}
TensorPtr matmul_transB_fused_ffn_down_residual_q4_0_device(const TensorPtr& input,
                                                            const TensorPtr& weight,
                                                            const TensorPtr& residual) {
    return matmul_transB_fused_ffn_down_residual_device(
        "matmul_transB_fused_ffn_down_residual_q4_0", DataType::Q4_0, "Q4_0", input, weight,
        residual);
}
TensorPtr matmul_transB_fused_ffn_down_residual_q6_k_device(const TensorPtr& input,
                                                            const TensorPtr& weight,
                                                            const TensorPtr& residual) {
    return matmul_transB_fused_ffn_down_residual_device(
        "matmul_transB_fused_ffn_down_residual_q6_k", DataType::Q6_K, "Q6_K", input, weight,
        residual);
}

}  // namespace ops
}  // namespace forge
