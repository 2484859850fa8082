/*
 * quantized_gemm.cuh — drop-in C++ host API of the quantized GEMM path.
 *
 * Same file name, namespace, struct, function names, parameter order and
 * defaults as reference include/quantized_gemm.cuh:6-41; cudaError_t and
 * cudaStream_t become hipError_t and hipStream_t.  Host-only inline layer over
 * the C ABI in fke_qgemm.h (libfke_qgemm.so): include it from any C++ file
 * compiled by g++ or hipcc and link -lfke_qgemm.
 */
#pragma once

#include "hip_utils.h"
#include "fke_qgemm.h"

#include <cstdint>

namespace flash_engine {
namespace quantized {

// C = (A_int8 * B_int8) * (scale_a * scale_b)   (reference :10-16)
struct QuantGEMMConfig {
    int M;  // rows of A and C
    int N;  // columns of C (rows of the [N,K] B operand)
    int K;  // reduction length

    QuantGEMMConfig(int m, int n, int k) : M(m), N(n), K(k) {}
};

// INT8 GEMM (reference :19-27).  d_A [M,K] row-major; d_B [N,K] row-major
// (K-contiguous per output column, the layout the reference kernel reads,
// src/quantized_gemm.cu:35); d_C [M,N] fp32.  K must be a multiple of 4.
inline hipError_t launch_int8_gemm_dp4a(const int8_t* d_A, const int8_t* d_B, float* d_C,
                                        float scale_a, float scale_b,
                                        const QuantGEMMConfig& config,
                                        hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(fke_launch_int8_gemm_dp4a(
        d_A, d_B, d_C, scale_a, scale_b, config.M, config.N, config.K,
        static_cast<void*>(stream)));
}

// Scaled FP8 E4M3 GEMM (reference :30-38).  d_A [M,K] row-major; d_B [K,N]
// row-major (src/quantized_gemm.cu:113); d_C [M,N] fp32.
inline hipError_t launch_fp8_gemm_scaled(const uint8_t* d_A, const uint8_t* d_B, float* d_C,
                                         float scale_a, float scale_b,
                                         const QuantGEMMConfig& config,
                                         hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(fke_launch_fp8_gemm_scaled(
        d_A, d_B, d_C, scale_a, scale_b, config.M, config.N, config.K,
        static_cast<void*>(stream)));
}

// ---- extensions (no reference counterpart; reduce to the above when scales
// ---- are uniform, bias is absent and the output is fp32) ----

enum class OutDType : int { F32 = FKE_OUT_F32, BF16 = FKE_OUT_BF16, I32 = FKE_OUT_I32 };
enum class BLayout : int { NK = FKE_B_NK, KN = FKE_B_KN };

// W8A8: per-token scale_a[M] x per-channel scale_b[N] (either may be null to
// use the scalar), optional bias[N], fp32/bf16/i32 output.
inline hipError_t launch_w8a8_gemm(const int8_t* d_A, const int8_t* d_B, void* d_C,
                                   const float* d_scale_a, const float* d_scale_b,
                                   const float* d_bias, const QuantGEMMConfig& config,
                                   OutDType out = OutDType::F32, BLayout b = BLayout::NK,
                                   float scale_a = 1.0f, float scale_b = 1.0f,
                                   hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(fke_qgemm_i8(
        d_A, d_B, d_C, config.M, config.N, config.K, d_scale_a, d_scale_b, scale_a, scale_b,
        d_bias, static_cast<int>(out), static_cast<int>(b), static_cast<void*>(stream)));
}

// Scaled FP8 with optional bias and fp32/bf16 output.
inline hipError_t launch_fp8_gemm(const uint8_t* d_A, const uint8_t* d_B, void* d_C,
                                  float scale_a, float scale_b, const float* d_bias,
                                  const QuantGEMMConfig& config, OutDType out = OutDType::F32,
                                  BLayout b = BLayout::KN, hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(fke_qgemm_f8(
        d_A, d_B, d_C, config.M, config.N, config.K, scale_a, scale_b, d_bias,
        static_cast<int>(out), static_cast<int>(b), static_cast<void*>(stream)));
}

}  // namespace quantized
}  // namespace flash_engine
