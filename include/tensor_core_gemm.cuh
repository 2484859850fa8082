/*
 * tensor_core_gemm.cuh — drop-in C++ host API of the half-precision GEMM.
 *
 * Same file name, namespace, function name, parameter order and defaults as
 * reference include/tensor_core_gemm.cuh:7-36 for launch_wmma_gemm_fp16;
 * cudaError_t / cudaStream_t / half become hipError_t / hipStream_t / HIP's
 * half.  The computation runs on the MI355X MFMA GEMM (matrix cores), not on
 * a WMMA port.  The reference's WMMA attention entry (launch_wmma_attention_qk_pv)
 * and its tile constants are not part of this library.  Host-only inline layer
 * over the C ABI in fke_qgemm.h: compiles with g++ or hipcc, link -lfke_qgemm.
 */
#pragma once

#include <hip/hip_fp16.h>

#include "fke_qgemm.h"
#include "hip_utils.h"

namespace flash_engine {
namespace tensor_core {

// C = alpha * (A * B): d_A [M,K] row-major fp16, d_B [K,N] column-major
// (= [N,K] row-major, the layout the reference kernel reads), d_C [M,N] fp32,
// accumulated in fp32.  beta is accepted and unused, as in the reference
// (src/tensor_core_attention.cu:57-65): C is overwritten.  Any M, N, K >= 1.
inline hipError_t launch_wmma_gemm_fp16(const half* d_A, const half* d_B, float* d_C, int M, int N, int K,
                                        float alpha = 1.0f, float beta = 0.0f, hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(
        fke_launch_wmma_gemm_fp16(d_A, d_B, d_C, M, N, K, alpha, beta, static_cast<void*>(stream)));
}

// ---- extension (no reference counterpart): fp16 or bf16 operands, per-row /
// ---- per-column scales, bias, fp32 or bf16 output (fke_gemm_half).
enum class HalfType : int { F16 = FKE_IN_F16, BF16 = FKE_IN_BF16 };

inline hipError_t launch_half_gemm(const void* d_A, const void* d_B, void* d_C, int M, int N, int K,
                                   HalfType type, const float* d_scale_a, const float* d_scale_b,
                                   const float* d_bias, float scale_a = 1.0f, float scale_b = 1.0f,
                                   int out_dtype = FKE_OUT_F32, int b_layout = FKE_B_NK,
                                   hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(fke_gemm_half(d_A, d_B, d_C, M, N, K, static_cast<int>(type), d_scale_a,
                                                 d_scale_b, scale_a, scale_b, d_bias, out_dtype, b_layout,
                                                 static_cast<void*>(stream)));
}

}  // namespace tensor_core
}  // namespace flash_engine
