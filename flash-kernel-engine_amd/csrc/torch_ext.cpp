// torch_ext.cpp — torch C++ extension `flash_engine_cuda` (the reference's
// module name, setup.py:51, imported by python/flash_engine/ops.py:9-13): the
// quantized GEMM path (and the SwiGLU it feeds) in the binding idiom of
// reference python/bindings.cpp:101-140 (TORCH_CHECKs on device / dtype /
// shape, a fresh output tensor, the current stream, one `*_forward` function
// per op).  The reference module exposes no quantized GEMM; these are the
// entries its ops.quantized_gemm_int8 (python/flash_engine/ops.py:180-186)
// would bind, beside its fused_swiglu_forward (ops.py:222-223).
// Every call goes through the C ABI of libfke_qgemm.so (include/fke_qgemm.h);
// this file holds no kernels and no CPU compute.
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <string>

#include "fke_qgemm.h"

namespace {

hipStream_t current_stream(const torch::Tensor& t) {
    return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

void check_dev(const torch::Tensor& t, const char* name, at::ScalarType dtype, const torch::Device& dev) {
    TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
    TORCH_CHECK(t.device() == dev, name, " is on ", t.device(), ", expected ", dev);
    TORCH_CHECK(t.scalar_type() == dtype, name, " must be ", dtype, ", got ", t.scalar_type());
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

const float* vec_ptr(const c10::optional<torch::Tensor>& t, const char* name, int64_t n, const torch::Device& dev) {
    if (!t.has_value()) return nullptr;
    check_dev(*t, name, at::kFloat, dev);
    TORCH_CHECK(t->numel() == n, name, " must have ", n, " elements, got ", t->numel());
    return t->data_ptr<float>();
}

int layout_code(const std::string& b_layout) {
    TORCH_CHECK(b_layout == "nk" || b_layout == "kn", "b_layout must be \"nk\" ([N,K]) or \"kn\" ([K,N])");
    return b_layout == "nk" ? FKE_B_NK : FKE_B_KN;
}

void check_status(int st, const char* what) {
    TORCH_CHECK(st == 0, what, " failed: ", fke_status_string(st));
}

// acc = A . B (exact int32), y = fp32(acc) * fp32(scale_a[m] * scale_b[n]) (+ bias[n] by one fma),
// out = y (fp32 / bf16) or acc (int32).  scale_a / scale_b absent -> the scalars sa / sb.
torch::Tensor quantized_gemm_int8_forward(torch::Tensor A, torch::Tensor B, c10::optional<torch::Tensor> scale_a,
                                          c10::optional<torch::Tensor> scale_b, c10::optional<torch::Tensor> bias,
                                          at::ScalarType out_dtype, std::string b_layout, double sa, double sb) {
    const auto dev = A.device();
    check_dev(A, "A", at::kChar, dev);
    check_dev(B, "B", at::kChar, dev);
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2, "A and B must be 2-D");
    const int layout = layout_code(b_layout);
    const int64_t M = A.size(0), K = A.size(1);
    const int64_t N = layout == FKE_B_NK ? B.size(0) : B.size(1);
    TORCH_CHECK((layout == FKE_B_NK ? B.size(1) : B.size(0)) == K, "K mismatch between A and B");
    int code;
    if (out_dtype == at::kFloat) code = FKE_OUT_F32;
    else if (out_dtype == at::kBFloat16) code = FKE_OUT_BF16;
    else if (out_dtype == at::kInt) code = FKE_OUT_I32;
    else TORCH_CHECK(false, "out_dtype must be float32, bfloat16 or int32");
    const float* pa = vec_ptr(scale_a, "scale_a", M, dev);
    const float* pb = vec_ptr(scale_b, "scale_b", N, dev);
    const float* pbias = vec_ptr(bias, "bias", N, dev);
    auto out = torch::empty({M, N}, A.options().dtype(out_dtype));
    check_status(fke_qgemm_i8(A.data_ptr<int8_t>(), B.data_ptr<int8_t>(), out.data_ptr(), static_cast<int>(M),
                              static_cast<int>(N), static_cast<int>(K), pa, pb, static_cast<float>(sa),
                              static_cast<float>(sb), pbias, code, layout, current_stream(A)),
                 "fke_qgemm_i8");
    return out;
}

// Scaled FP8 E4M3 GEMM (reference src/quantized_gemm.cu:99-139); A, B as uint8 codes.
torch::Tensor fp8_gemm_scaled_forward(torch::Tensor A, torch::Tensor B, double scale_a, double scale_b,
                                      c10::optional<torch::Tensor> bias, at::ScalarType out_dtype,
                                      std::string b_layout) {
    const auto dev = A.device();
    check_dev(A, "A", at::kByte, dev);
    check_dev(B, "B", at::kByte, dev);
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2, "A and B must be 2-D");
    const int layout = layout_code(b_layout);
    const int64_t M = A.size(0), K = A.size(1);
    const int64_t N = layout == FKE_B_NK ? B.size(0) : B.size(1);
    TORCH_CHECK((layout == FKE_B_NK ? B.size(1) : B.size(0)) == K, "K mismatch between A and B");
    TORCH_CHECK(out_dtype == at::kFloat || out_dtype == at::kBFloat16, "FP8 GEMM writes float32 or bfloat16");
    const float* pbias = vec_ptr(bias, "bias", N, dev);
    auto out = torch::empty({M, N}, A.options().dtype(out_dtype));
    check_status(fke_qgemm_f8(A.data_ptr<uint8_t>(), B.data_ptr<uint8_t>(), out.data_ptr(), static_cast<int>(M),
                              static_cast<int>(N), static_cast<int>(K), static_cast<float>(scale_a),
                              static_cast<float>(scale_b), pbias,
                              out_dtype == at::kFloat ? FKE_OUT_F32 : FKE_OUT_BF16, layout, current_stream(A)),
                 "fke_qgemm_f8");
    return out;
}

// Per-token INT8 quantiser: x [M,K] fp32 / bf16 -> (q int8 [M,K], scale fp32 [M]).
std::vector<torch::Tensor> quantize_per_token_forward(torch::Tensor x) {
    TORCH_CHECK(x.is_cuda(), "x must be a GPU tensor");
    TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16, "x must be float32 or bfloat16");
    TORCH_CHECK(x.is_contiguous() && x.dim() == 2, "x must be a contiguous 2-D tensor");
    const int64_t M = x.size(0), K = x.size(1);
    auto q = torch::empty({M, K}, x.options().dtype(at::kChar));
    auto s = torch::empty({M}, x.options().dtype(at::kFloat));
    check_status(fke_quantize_rows_i8(x.data_ptr(), x.scalar_type() == at::kFloat ? FKE_IN_F32 : FKE_IN_BF16,
                                      static_cast<int>(M), static_cast<int>(K), q.data_ptr<int8_t>(),
                                      s.data_ptr<float>(), current_stream(x)),
                 "fke_quantize_rows_i8");
    return {q, s};
}

// Gate/up GEMM with SwiGLU in the epilogue: W [2I, K] = [gate; up], out [M, I].
torch::Tensor quantized_gemm_int8_swiglu_forward(torch::Tensor A, torch::Tensor W,
                                                 c10::optional<torch::Tensor> scale_a,
                                                 c10::optional<torch::Tensor> scale_b,
                                                 c10::optional<torch::Tensor> bias, at::ScalarType out_dtype,
                                                 double sa, double sb) {
    const auto dev = A.device();
    check_dev(A, "A", at::kChar, dev);
    check_dev(W, "W", at::kChar, dev);
    TORCH_CHECK(A.dim() == 2 && W.dim() == 2, "A and W must be 2-D");
    const int64_t M = A.size(0), K = A.size(1);
    TORCH_CHECK(W.size(1) == K && W.size(0) % 2 == 0, "W must be [2I, K]");
    const int64_t I = W.size(0) / 2;
    TORCH_CHECK(out_dtype == at::kFloat || out_dtype == at::kBFloat16, "SwiGLU GEMM writes float32 or bfloat16");
    const float* pa = vec_ptr(scale_a, "scale_a", M, dev);
    const float* pb = vec_ptr(scale_b, "scale_b", 2 * I, dev);
    const float* pbias = vec_ptr(bias, "bias", 2 * I, dev);
    auto out = torch::empty({M, I}, A.options().dtype(out_dtype));
    check_status(fke_qgemm_i8_swiglu(A.data_ptr<int8_t>(), W.data_ptr<int8_t>(), out.data_ptr(),
                                     static_cast<int>(M), static_cast<int>(I), static_cast<int>(K), pa, pb,
                                     static_cast<float>(sa), static_cast<float>(sb), pbias,
                                     out_dtype == at::kFloat ? FKE_OUT_F32 : FKE_OUT_BF16, current_stream(A)),
                 "fke_qgemm_i8_swiglu");
    return out;
}

// Reference python/bindings.cpp:101-133 (fused_swiglu_forward): float32 and
// float16 as there, bfloat16 added.
torch::Tensor fused_swiglu_forward(torch::Tensor gate, torch::Tensor up) {
    TORCH_CHECK(gate.is_cuda() && up.is_cuda(), "Inputs must be GPU tensors");
    TORCH_CHECK(gate.sizes() == up.sizes(), "Gate and Up tensors must match shapes");
    TORCH_CHECK(gate.scalar_type() == up.scalar_type(), "Gate and Up tensors must have one dtype");
    TORCH_CHECK(gate.device() == up.device(), "Gate and Up tensors must be on one device");
    TORCH_CHECK(gate.is_contiguous() && up.is_contiguous(), "Gate and Up tensors must be contiguous");
    int code;
    switch (gate.scalar_type()) {
        case at::kFloat: code = FKE_IN_F32; break;
        case at::kHalf: code = FKE_IN_F16; break;
        case at::kBFloat16: code = FKE_IN_BF16; break;
        default: TORCH_CHECK(false, "Unsupported tensor type for SwiGLU");
    }
    auto out = torch::empty_like(gate);
    check_status(fke_swiglu(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(), code,
                            current_stream(gate)),
                 "fke_swiglu");
    return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "flash-kernel-engine quantized GEMM path on MI355X (gfx950) HIP kernels";
    m.def("quantized_gemm_int8_forward", &quantized_gemm_int8_forward, "W8A8 INT8 GEMM with fused epilogue",
          py::arg("A"), py::arg("B"), py::arg("scale_a") = py::none(), py::arg("scale_b") = py::none(),
          py::arg("bias") = py::none(), py::arg("out_dtype") = at::kBFloat16, py::arg("b_layout") = "nk",
          py::arg("sa") = 1.0, py::arg("sb") = 1.0);
    m.def("fp8_gemm_scaled_forward", &fp8_gemm_scaled_forward, "Scaled FP8 E4M3 GEMM", py::arg("A"), py::arg("B"),
          py::arg("scale_a"), py::arg("scale_b"), py::arg("bias") = py::none(), py::arg("out_dtype") = at::kFloat,
          py::arg("b_layout") = "kn");
    m.def("quantize_per_token_forward", &quantize_per_token_forward, "Per-token INT8 quantiser", py::arg("x"));
    m.def("quantized_gemm_int8_swiglu_forward", &quantized_gemm_int8_swiglu_forward,
          "W8A8 gate/up GEMM with SwiGLU fused into the epilogue", py::arg("A"), py::arg("W"),
          py::arg("scale_a") = py::none(), py::arg("scale_b") = py::none(), py::arg("bias") = py::none(),
          py::arg("out_dtype") = at::kBFloat16, py::arg("sa") = 1.0, py::arg("sb") = 1.0);
    m.def("fused_swiglu_forward", &fused_swiglu_forward, "Fused SwiGLU", py::arg("gate"), py::arg("up"));
}
