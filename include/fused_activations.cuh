/*
 * fused_activations.cuh — drop-in C++ host API of the SwiGLU activation.
 *
 * Same file name, namespace, function names, parameter order and defaults as
 * reference include/fused_activations.cuh:6-25 for launch_fused_swiglu_fp32
 * and launch_fused_swiglu_fp16; cudaError_t / cudaStream_t / half become
 * hipError_t / hipStream_t / HIP's half.  out = (x * sigmoid(x)) * y computed
 * in fp32 and rounded once to the element type.  The reference's GeLU entry
 * (launch_fused_gelu_fp32) is not part of this library.  Host-only inline
 * layer over the C ABI in fke_qgemm.h (fke_swiglu): link -lfke_qgemm.
 */
#pragma once

#include <hip/hip_fp16.h>

#include <cstdint>

#include "fke_qgemm.h"
#include "hip_utils.h"

namespace flash_engine {
namespace activation {

// Fused SwiGLU: output = (x * sigmoid(x)) * y; gate (x) and up (y) are
// contiguous arrays of num_elements.
inline hipError_t launch_fused_swiglu_fp32(const float* d_gate, const float* d_up, float* d_out, int num_elements,
                                           hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(
        fke_swiglu(d_gate, d_up, d_out, num_elements, FKE_IN_F32, static_cast<void*>(stream)));
}

inline hipError_t launch_fused_swiglu_fp16(const half* d_gate, const half* d_up, half* d_out, int num_elements,
                                           hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(
        fke_swiglu(d_gate, d_up, d_out, num_elements, FKE_IN_F16, static_cast<void*>(stream)));
}

// ---- extension: bf16 (raw 16-bit values), 64-bit element count ----
inline hipError_t launch_fused_swiglu_bf16(const uint16_t* d_gate, const uint16_t* d_up, uint16_t* d_out,
                                           int64_t num_elements, hipStream_t stream = nullptr) {
    return static_cast<hipError_t>(
        fke_swiglu(d_gate, d_up, d_out, num_elements, FKE_IN_BF16, static_cast<void*>(stream)));
}

}  // namespace activation
}  // namespace flash_engine
