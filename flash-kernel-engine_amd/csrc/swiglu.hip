// swiglu.hip — elementwise SwiGLU, h[i] = (g[i] * sigmoid(g[i])) * u[i]
// (reference src/fused_activations.cu:17-118: launch_fused_swiglu_fp32, with a
// float4 body and a scalar tail launch, and launch_fused_swiglu_fp16, which
// computes in fp32 and rounds the result to fp16).  Here fp32, fp16 and bf16
// share one kernel: values are widened to fp32 exactly, combined by
// swiglu_pair (the same function the fused GEMM epilogues use, so an
// unfused GEMM + this op reproduces them bit for bit), and rounded to the
// output type to nearest even.
//
// HBM-bound (8 / 4 bytes read and 4 / 2 written per element): each thread
// handles one 16-byte chunk of each operand with 128-bit loads and stores;
// when any pointer is not 16-byte aligned the same kernel runs one element
// per thread.  The last, partial chunk is bounds-checked element by element.
#include "fke_internal.h"

namespace fke {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int ST = 256;  // threads per workgroup

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
    if constexpr (DT == FKE_IN_F32) return static_cast<const float*>(p)[i];
    else if constexpr (DT == FKE_IN_BF16)
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
    else return static_cast<float>(static_cast<const _Float16*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float h) {
    if constexpr (DT == FKE_IN_F32) static_cast<float*>(p)[i] = h;
    else if constexpr (DT == FKE_IN_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(h);
    else static_cast<_Float16*>(p)[i] = static_cast<_Float16>(h);  // v_cvt_f16_f32, round to nearest even
}

// Element e of a 16-byte chunk widened to fp32.
template <int DT>
__device__ __forceinline__ float chunk_elem(const v4i& c, int e) {
    if constexpr (DT == FKE_IN_F32) {
        return __int_as_float(c[e]);
    } else {
        const uint32_t w = static_cast<uint32_t>(c[e >> 1]);
        const uint32_t h = (e & 1) ? (w >> 16) : (w & 0xFFFFu);
        if constexpr (DT == FKE_IN_BF16) return __uint_as_float(h << 16);
        else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
    }
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    if constexpr (DT == FKE_IN_BF16) {
        return static_cast<uint32_t>(f32_to_bf16_rne(lo)) | (static_cast<uint32_t>(f32_to_bf16_rne(hi)) << 16);
    } else {
        const uint16_t a = __builtin_bit_cast(uint16_t, static_cast<_Float16>(lo));
        const uint16_t b = __builtin_bit_cast(uint16_t, static_cast<_Float16>(hi));
        return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
    }
}

// VEC: one 16-byte chunk per thread (all pointers 16-byte aligned); else one element.
template <int DT, bool VEC>
__global__ __launch_bounds__(ST) void swiglu_kernel(const void* G, const void* U, void* H, int64_t n) {
    constexpr int EB = DT == FKE_IN_F32 ? 4 : 2;
    constexpr int EPC = VEC ? 16 / EB : 1;  // elements per thread
    const int64_t c = static_cast<int64_t>(blockIdx.x) * ST + threadIdx.x;
    const int64_t i0 = c * EPC;
    if (i0 >= n) return;
    if (VEC && i0 + EPC <= n) {
        const v4i g = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(G) + c);
        const v4i u = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(U) + c);
        v4i h;
        if constexpr (DT == FKE_IN_F32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = __float_as_int(swiglu_pair(chunk_elem<DT>(g, e), chunk_elem<DT>(u, e)));
        } else {
#pragma unroll
            for (int w = 0; w < 4; ++w)
                h[w] = static_cast<int>(pack2<DT>(swiglu_pair(chunk_elem<DT>(g, 2 * w), chunk_elem<DT>(u, 2 * w)),
                                                  swiglu_pair(chunk_elem<DT>(g, 2 * w + 1),
                                                              chunk_elem<DT>(u, 2 * w + 1))));
        }
        __builtin_nontemporal_store(h, reinterpret_cast<v4i*>(H) + c);
        return;
    }
    const int64_t i1 = i0 + EPC < n ? i0 + EPC : n;
    for (int64_t i = i0; i < i1; ++i) store_elem<DT>(H, i, swiglu_pair(load_elem<DT>(G, i), load_elem<DT>(U, i)));
}

template <int DT>
hipError_t launch_dt(const void* G, const void* U, void* H, int64_t n, hipStream_t stream) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(G) | reinterpret_cast<uintptr_t>(U) |
                         reinterpret_cast<uintptr_t>(H);
    const bool vec = (al & 15) == 0;
    constexpr int EB = DT == FKE_IN_F32 ? 4 : 2;
    const int64_t per = vec ? 16 / EB : 1;
    const int64_t threads = (n + per - 1) / per;
    const int64_t blocks = (threads + ST - 1) / ST;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    void* args[] = {&G, &U, &H, &n};
    const void* f = vec ? reinterpret_cast<const void*>(&swiglu_kernel<DT, true>)
                        : reinterpret_cast<const void*>(&swiglu_kernel<DT, false>);
    return hipLaunchKernel(f, dim3(static_cast<unsigned>(blocks)), dim3(ST), args, 0, stream);
}

}  // namespace

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, hipStream_t stream) {
    switch (dtype) {
        case FKE_IN_F32: return launch_dt<FKE_IN_F32>(gate, up, out, n, stream);
        case FKE_IN_BF16: return launch_dt<FKE_IN_BF16>(gate, up, out, n, stream);
        default: return launch_dt<FKE_IN_F16>(gate, up, out, n, stream);
    }
}

}  // namespace fke
