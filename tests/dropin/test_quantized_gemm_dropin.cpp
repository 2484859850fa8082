// Drop-in check of the C++ host API (include/quantized_gemm.cuh,
// include/tensor_core_gemm.cuh, include/fused_activations.cuh,
// include/flash_engine.h): the reference's own GEMM test
// (tests/test_quantized_gemm.cu:9-86 of flash-kernel-engine) restated against
// the HIP API, plus the FP8 launcher, the fp16 WMMA-GEMM launcher, SwiGLU on
// the reference's Python test vector (python/tests/test_correctness.py:166-176)
// and the argument-validation contract.
// Built by the host compiler alone and linked against libfke_qgemm.so.
//
//   test_quantized_gemm_dropin --host-only   validation checks only (no GPU)
//   test_quantized_gemm_dropin               full test; fails if no GPU
#include "flash_engine.h"

#include <cmath>
#include <cstring>
#include <iostream>
#include <vector>

using namespace flash_engine;
using namespace flash_engine::quantized;
using flash_engine::activation::launch_fused_swiglu_fp16;
using flash_engine::activation::launch_fused_swiglu_fp32;
using flash_engine::tensor_core::launch_wmma_gemm_fp16;

static int host_checks() {
    int bad = 0;
    const int8_t* p8 = reinterpret_cast<const int8_t*>(16);
    float* pf = reinterpret_cast<float*>(16);
    const uint8_t* pu = reinterpret_cast<const uint8_t*>(16);
    auto expect_invalid = [&](hipError_t e, const char* what) {
        if (e != hipErrorInvalidValue) {
            std::cerr << "[FAIL] " << what << " returned " << static_cast<int>(e) << "\n";
            ++bad;
        }
    };
    expect_invalid(launch_int8_gemm_dp4a(p8, p8, pf, 1.f, 1.f, QuantGEMMConfig(0, 8, 8)), "M=0");
    expect_invalid(launch_int8_gemm_dp4a(p8, p8, pf, 1.f, 1.f, QuantGEMMConfig(8, 0, 8)), "N=0");
    expect_invalid(launch_int8_gemm_dp4a(p8, p8, pf, 1.f, 1.f, QuantGEMMConfig(8, 8, 0)), "K=0");
    expect_invalid(launch_int8_gemm_dp4a(p8, p8, pf, 1.f, 1.f, QuantGEMMConfig(8, 8, 6)), "K%4");
    expect_invalid(launch_int8_gemm_dp4a(nullptr, p8, pf, 1.f, 1.f, QuantGEMMConfig(8, 8, 8)), "A=null");
    expect_invalid(launch_fp8_gemm_scaled(pu, nullptr, pf, 1.f, 1.f, QuantGEMMConfig(8, 8, 8)), "B=null");
    expect_invalid(launch_fp8_gemm_scaled(pu, pu, pf, 1.f, 1.f, QuantGEMMConfig(-1, 8, 8)), "M<0");
    const half* ph = reinterpret_cast<const half*>(16);
    expect_invalid(launch_wmma_gemm_fp16(ph, nullptr, pf, 8, 8, 8), "wmma B=null");
    expect_invalid(launch_wmma_gemm_fp16(ph, ph, pf, 8, 8, 0), "wmma K=0");
    expect_invalid(launch_fused_swiglu_fp32(pf, nullptr, pf, 8), "swiglu up=null");
    expect_invalid(launch_fused_swiglu_fp32(pf, pf, pf, -1), "swiglu n<0");
    if (std::strcmp(get_version(), "1.2.0") != 0 || VERSION_MAJOR != 1 || VERSION_MINOR != 2 ||
        VERSION_PATCH != 0) {
        std::cerr << "[FAIL] version\n";
        ++bad;
    }
    if (bad == 0) std::cout << "[PASS] host-side argument validation\n";
    return bad;
}

static float e4m3_decode(uint8_t x) {  // reference src/quantized_gemm.cu:81-97
    int sign = (x >> 7) & 1, e = (x >> 3) & 0xF, m = x & 7;
    float v;
    if (e == 0) v = static_cast<float>(m) / 8.0f * (1.0f / 64.0f);
    else if (e == 15 && m == 7) return 0.0f;
    else v = std::ldexp(1.0f + static_cast<float>(m) / 8.0f, e - 7);
    return sign ? -v : v;
}

int main(int argc, char** argv) {
    const bool host_only = argc > 1 && std::strcmp(argv[1], "--host-only") == 0;
    int bad = host_checks();
    if (host_only) return bad ? 1 : 0;

    int device_count = 0;
    if (hipGetDeviceCount(&device_count) != hipSuccess || device_count == 0) {
        std::cerr << "[FAIL] no GPU visible\n";
        return 1;
    }
    print_device_info(0);

    // ---- INT8: the reference test's closed-form inputs (:19-48) ----
    constexpr int M = 64, N = 64, K = 64;
    QuantGEMMConfig config(M, N, K);
    std::vector<int8_t> h_A(M * K), h_B(N * K);
    std::vector<float> h_C(M * N, 0.0f), h_ref(M * N, 0.0f);
    for (int i = 0; i < M * K; ++i) h_A[i] = static_cast<int8_t>((i % 7) - 3);
    for (int i = 0; i < N * K; ++i) h_B[i] = static_cast<int8_t>((i % 5) - 2);
    const float scale_a = 0.05f, scale_b = 0.02f;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            int32_t acc = 0;
            for (int k = 0; k < K; ++k)
                acc += static_cast<int32_t>(h_A[m * K + k]) * static_cast<int32_t>(h_B[n * K + k]);
            h_ref[m * N + n] = static_cast<float>(acc) * (scale_a * scale_b);
        }
    int8_t *d_A, *d_B;
    float* d_C;
    HIP_CHECK(hipMalloc(&d_A, h_A.size()));
    HIP_CHECK(hipMalloc(&d_B, h_B.size()));
    HIP_CHECK(hipMalloc(&d_C, h_C.size() * sizeof(float)));
    HIP_CHECK(hipMemcpy(d_A, h_A.data(), h_A.size(), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(d_B, h_B.data(), h_B.size(), hipMemcpyHostToDevice));
    HIP_CHECK(launch_int8_gemm_dp4a(d_A, d_B, d_C, scale_a, scale_b, config));
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(h_C.data(), d_C, h_C.size() * sizeof(float), hipMemcpyDeviceToHost));
    size_t mismatches = 0;
    float max_diff = 0.0f;
    for (size_t i = 0; i < h_C.size(); ++i) {
        max_diff = std::fmax(max_diff, std::fabs(h_C[i] - h_ref[i]));
        if (std::memcmp(&h_C[i], &h_ref[i], 4) != 0) ++mismatches;
    }
    std::cout << "[INFO] INT8 max abs diff " << max_diff << ", bit mismatches " << mismatches << "\n";
    if (max_diff >= 1e-3f || mismatches != 0) {
        std::cerr << "[FAIL] INT8 drop-in GEMM\n";
        ++bad;
    } else {
        std::cout << "[PASS] INT8 drop-in GEMM bit-exact vs the reference host loop\n";
    }

    // ---- FP8: every non-negative code (incl. 0x7F -> 0.0) over 64x64x256 ----
    // Codes without the sign bit keep the sums free of cancellation, so the
    // fp32 result of any summation order is within a few ulp of the exact sum
    // (with both signs this closed form cancels to exactly 0.0).
    constexpr int FK = 256;
    std::vector<uint8_t> f_A(M * FK), f_B(FK * N);
    for (int i = 0; i < M * FK; ++i) f_A[i] = static_cast<uint8_t>(((i * 37 + 11) ^ (i >> 7)) & 0x7F);
    for (int i = 0; i < FK * N; ++i) f_B[i] = static_cast<uint8_t>(((i * 101 + 5) ^ (i >> 6)) & 0x7F);
    std::vector<float> f_C(M * N), f_ref(M * N);
    const float fa = 0.125f, fb = 0.5f;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (int k = 0; k < FK; ++k) sum += e4m3_decode(f_A[m * FK + k]) * e4m3_decode(f_B[k * N + n]);
            f_ref[m * N + n] = sum * (fa * fb);
        }
    uint8_t *d_fA, *d_fB;
    HIP_CHECK(hipMalloc(&d_fA, f_A.size()));
    HIP_CHECK(hipMalloc(&d_fB, f_B.size()));
    HIP_CHECK(hipMemcpy(d_fA, f_A.data(), f_A.size(), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(d_fB, f_B.data(), f_B.size(), hipMemcpyHostToDevice));
    HIP_CHECK(launch_fp8_gemm_scaled(d_fA, d_fB, d_C, fa, fb, QuantGEMMConfig(M, N, FK)));
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(f_C.data(), d_C, f_C.size() * sizeof(float), hipMemcpyDeviceToHost));
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < f_C.size(); ++i) {
        num = std::fmax(num, std::fabs(static_cast<double>(f_C[i]) - f_ref[i]));
        den = std::fmax(den, std::fabs(static_cast<double>(f_ref[i])));
    }
    const double rel = den > 0 ? num / den : num;
    std::cout << "[INFO] FP8 max-norm relative error " << rel << "\n";
    if (!(rel <= 2e-2)) {
        std::cerr << "[FAIL] FP8 drop-in GEMM\n";
        ++bad;
    } else {
        std::cout << "[PASS] FP8 drop-in GEMM within 2e-2 of the reference loop\n";
    }

    // ---- fp16 WMMA-GEMM launcher: small-integer operands (exact sums), alpha
    // ---- applied, beta ignored, C overwritten ----
    constexpr int HM = 48, HN = 80, HK = 192;
    std::vector<half> hA(HM * HK), hB(HN * HK);
    std::vector<float> hC(HM * HN), href(HM * HN);
    for (int i = 0; i < HM * HK; ++i) hA[i] = __float2half(static_cast<float>((i * 7 + 3) % 11 - 5));
    for (int i = 0; i < HN * HK; ++i) hB[i] = __float2half(static_cast<float>((i * 5 + 1) % 9 - 4));
    for (int m = 0; m < HM; ++m)
        for (int n = 0; n < HN; ++n) {
            long acc = 0;
            for (int k = 0; k < HK; ++k)
                acc += static_cast<long>((( (m * HK + k) * 7 + 3) % 11) - 5) *
                       static_cast<long>((((n * HK + k) * 5 + 1) % 9) - 4);
            href[m * HN + n] = static_cast<float>(acc) * 0.25f;
        }
    half *d_hA, *d_hB;
    float* d_hC;
    HIP_CHECK(hipMalloc(&d_hA, hA.size() * sizeof(half)));
    HIP_CHECK(hipMalloc(&d_hB, hB.size() * sizeof(half)));
    HIP_CHECK(hipMalloc(&d_hC, hC.size() * sizeof(float)));
    HIP_CHECK(hipMemcpy(d_hA, hA.data(), hA.size() * sizeof(half), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(d_hB, hB.data(), hB.size() * sizeof(half), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemset(d_hC, 0xFF, hC.size() * sizeof(float)));  // NaN: must be overwritten
    HIP_CHECK(launch_wmma_gemm_fp16(d_hA, d_hB, d_hC, HM, HN, HK, 0.25f, 2.0f));
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(hC.data(), d_hC, hC.size() * sizeof(float), hipMemcpyDeviceToHost));
    size_t hmis = 0;
    for (size_t i = 0; i < hC.size(); ++i)
        if (std::memcmp(&hC[i], &href[i], 4) != 0) ++hmis;
    if (hmis) {
        std::cerr << "[FAIL] fp16 WMMA-GEMM drop-in: " << hmis << " mismatches\n";
        ++bad;
    } else {
        std::cout << "[PASS] fp16 WMMA-GEMM drop-in exact on integer operands (alpha applied, beta ignored)\n";
    }

    // ---- SwiGLU fp32 on the reference's test vector: max abs diff < 1e-6 ----
    const float gate[5] = {-2.0f, -0.5f, 0.0f, 0.5f, 2.0f}, up[5] = {1.0f, 2.0f, 3.0f, 4.0f, 5.0f};
    float sw[5];
    float* d_sw;
    HIP_CHECK(hipMalloc(&d_sw, 3 * 5 * sizeof(float)));
    HIP_CHECK(hipMemcpy(d_sw, gate, sizeof(gate), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(d_sw + 5, up, sizeof(up), hipMemcpyHostToDevice));
    HIP_CHECK(launch_fused_swiglu_fp32(d_sw, d_sw + 5, d_sw + 10, 5));
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(sw, d_sw + 10, sizeof(sw), hipMemcpyDeviceToHost));
    float sdiff = 0.0f;
    for (int i = 0; i < 5; ++i)
        sdiff = std::fmax(sdiff, std::fabs(sw[i] - (gate[i] / (1.0f + std::exp(-gate[i]))) * up[i]));
    if (!(sdiff < 1e-6f)) {
        std::cerr << "[FAIL] SwiGLU drop-in: max abs diff " << sdiff << "\n";
        ++bad;
    } else {
        std::cout << "[PASS] SwiGLU drop-in on the reference test vector (max abs diff " << sdiff << ")\n";
    }
    HIP_CHECK(hipFree(d_A));
    HIP_CHECK(hipFree(d_B));
    HIP_CHECK(hipFree(d_C));
    HIP_CHECK(hipFree(d_fA));
    HIP_CHECK(hipFree(d_fB));
    HIP_CHECK(hipFree(d_hA));
    HIP_CHECK(hipFree(d_hB));
    HIP_CHECK(hipFree(d_hC));
    HIP_CHECK(hipFree(d_sw));
    return bad ? 1 : 0;
}
