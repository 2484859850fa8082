// quant_i8.hip — per-token (per-row) symmetric INT8 quantiser of activations,
// the step in front of the W8A8 GEMM.  The reference has no such kernel (its
// quantized path takes int8 inputs and one scalar scale,
// src/quantized_gemm.cu:56-75); this one produces the A operand and the
// per-row scale_a of fke_qgemm_i8:
//   amax_m = max_k |x[m,k]|                    (NaN elements ignored, +-inf counted)
//   s_m    = fp32(amax_m / 127),  r_m = fp32(127 / (amax_m * f_m))   (s = r = 1 when amax_m == 0)
//   q[m,k] = clamp(rne(fp32(fp32(x[m,k] * f_m) * r_m)), -127, 127)   (a NaN product gives 0)
// with f_m = 2^64 when amax_m < 2^-64, else 1 (an exact power of two that
// keeps r_m finite for rows whose maximum is below 127/FLT_MAX; it changes no
// code of any other row), so that x ~= q * s_m and the GEMM's epilogue
// s = fp32(s_m * sb_n) dequantises.  A row holding +-inf gets s_m = inf and
// r_m = 0: every code is 0.
// One multiply per element instead of a correctly rounded division (about ten
// instructions on this GPU, which made the division-based form VALU-bound).
//
// One wave per row, four rows per workgroup.  Lane l reads 16-byte chunks
// l, l+64, ... of its row (4 fp32 or 8 bf16 values each; one wave load =
// 1 KiB contiguous), keeps the first CACHE chunks in registers while it takes
// the row maximum, reduces the maximum across the wave (no LDS, no barrier),
// then quantises from registers and writes 4 or 8 int8 codes per chunk.
// Rows longer than 64*CACHE chunks re-read the rest (L2 hits: the row was
// just streamed).  Shapes the chunked path cannot take (K not a multiple of 8,
// unaligned pointers) use the same arithmetic one element at a time, one
// 256-thread workgroup per row.
#include "fke_internal.h"

#include <type_traits>

namespace fke {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int QT = 256;    // threads per workgroup (4 rows in the chunked kernel, 1 in the scalar one)
constexpr int CACHE = 8;   // 16-byte chunks kept in registers per lane

// Element e of a 16-byte chunk as fp32 (IN: FKE_IN_F32 or FKE_IN_BF16).
template <int IN>
__device__ __forceinline__ float elem(const v4i& c, int e) {
    if constexpr (IN == FKE_IN_F32) {
        return __int_as_float(c[e]);
    } else {
        const uint32_t w = static_cast<uint32_t>(c[e >> 1]);
        return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
    }
}

// Maximum of v over the workgroup, returned to every thread.
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// The code of q8_bits, one element at a time (x already multiplied by f).
__device__ __forceinline__ int8_t q8(float x, float r) {
    const float p = x * r;
    if (p != p) return 0;
    const float v = __builtin_rintf(p);
    return static_cast<int8_t>(fminf(fmaxf(v, -127.0f), 127.0f));
}

template <int IN>
__global__ __launch_bounds__(QT) void quant_rows_kernel(const void* X, int M, int K, int8_t* Q, float* S) {
    constexpr int EPC = IN == FKE_IN_F32 ? 4 : 8;  // elements per 16-byte chunk
    constexpr int EB = IN == FKE_IN_F32 ? 4 : 2;   // bytes per element
    const int lane = threadIdx.x & 63;
    const int m = __builtin_amdgcn_readfirstlane(blockIdx.x * (QT / 64) + (threadIdx.x >> 6));
    if (m >= M) return;  // uniform per wave
    const int nch = K / EPC;
    const v4i* xr = reinterpret_cast<const v4i*>(static_cast<const char*>(X) + static_cast<size_t>(m) * K * EB);
    int8_t* qr = Q + static_cast<size_t>(m) * K;

    v4i cache[CACHE];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < CACHE; ++i) {
        const int c = lane + i * 64;
        cache[i] = c < nch ? xr[c] : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < CACHE; ++i)
#pragma unroll
        for (int e = 0; e < EPC; ++e) amax = fmaxf(amax, fabsf(elem<IN>(cache[i], e)));
    for (int c = lane + CACHE * 64; c < nch; c += 64) {
        const v4i v = xr[c];
#pragma unroll
        for (int e = 0; e < EPC; ++e) amax = fmaxf(amax, fabsf(elem<IN>(v, e)));
    }
    const RowScale rs = scale_of(wave_max(amax));

    // TINY: the row's f is 2^64 (a wave-uniform branch below; the common
    // path has no extra multiply).
    auto row = [&](auto tinyc) __attribute__((always_inline)) {
        constexpr bool TINY = decltype(tinyc)::value;
        auto x = [&](const v4i& v, int e) { return TINY ? elem<IN>(v, e) * 0x1p64f : elem<IN>(v, e); };
        auto emit = [&](const v4i& v, int c) {
            uint32_t w[EPC / 4];
#pragma unroll
            for (int j = 0; j < EPC / 4; ++j) {
                const uint32_t t0 = q8_bits(x(v, 4 * j + 0), rs.r), t1 = q8_bits(x(v, 4 * j + 1), rs.r);
                const uint32_t t2 = q8_bits(x(v, 4 * j + 2), rs.r), t3 = q8_bits(x(v, 4 * j + 3), rs.r);
                w[j] = pack_q8(t0, t1, t2, t3);
            }
            if constexpr (EPC == 4) *reinterpret_cast<uint32_t*>(qr + c * 4) = w[0];
            else *reinterpret_cast<uint2*>(qr + c * 8) = make_uint2(w[0], w[1]);
        };
#pragma unroll
        for (int i = 0; i < CACHE; ++i) {
            const int c = lane + i * 64;
            if (c < nch) emit(cache[i], c);
        }
        for (int c = lane + CACHE * 64; c < nch; c += 64) emit(xr[c], c);
    };
    if (rs.f != 1.0f) row(std::true_type{});
    else row(std::false_type{});
    if (lane == 0) S[m] = rs.s;
}

// Any K, any alignment: the same arithmetic element by element.
template <int IN>
__global__ __launch_bounds__(QT) void quant_rows_scalar_kernel(const void* X, int K, int8_t* Q, float* S) {
    __shared__ float red[QT / 64];
    const int m = blockIdx.x, tid = threadIdx.x;
    auto load = [&](int k) {
        const size_t i = static_cast<size_t>(m) * K + k;
        if constexpr (IN == FKE_IN_F32) return static_cast<const float*>(X)[i];
        else return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(X)[i]) << 16);
    };
    float amax = 0.0f;
    for (int k = tid; k < K; k += QT) amax = fmaxf(amax, fabsf(load(k)));
    const RowScale rs = scale_of(block_max(amax, red));
    for (int k = tid; k < K; k += QT) Q[static_cast<size_t>(m) * K + k] = q8(load(k) * rs.f, rs.r);
    if (tid == 0) S[m] = rs.s;
}

}  // namespace

hipError_t launch_quant_rows(const void* X, int in_dtype, int M, int K, int8_t* Q, float* S, hipStream_t stream) {
    const uintptr_t ax = reinterpret_cast<uintptr_t>(X), aq = reinterpret_cast<uintptr_t>(Q);
    const bool chunked = K % 8 == 0 && (ax & 15) == 0 && (aq & 7) == 0;
    const void* f;
    if (in_dtype == FKE_IN_F32)
        f = chunked ? reinterpret_cast<const void*>(&quant_rows_kernel<FKE_IN_F32>)
                    : reinterpret_cast<const void*>(&quant_rows_scalar_kernel<FKE_IN_F32>);
    else
        f = chunked ? reinterpret_cast<const void*>(&quant_rows_kernel<FKE_IN_BF16>)
                    : reinterpret_cast<const void*>(&quant_rows_scalar_kernel<FKE_IN_BF16>);
    if (chunked) {
        void* args[] = {&X, &M, &K, &Q, &S};
        return hipLaunchKernel(f, dim3((M + QT / 64 - 1) / (QT / 64)), dim3(QT), args, 0, stream);
    }
    void* args[] = {&X, &K, &Q, &S};
    return hipLaunchKernel(f, dim3(M), dim3(QT), args, 0, stream);
}

}  // namespace fke
