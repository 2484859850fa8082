/*
 * flash_engine.h — umbrella header of the MI355X build of the quantized GEMM
 * path.  Mirrors reference include/flash_engine.h:17-31 (version constants,
 * get_version, print_device_info).  Of the reference's module headers it
 * carries quantized_gemm.cuh, tensor_core_gemm.cuh (the GEMM) and
 * fused_activations.cuh (SwiGLU); attention, decoding, RMSNorm and the others
 * are not part of this library.
 */
#pragma once

#include "fused_activations.cuh"
#include "hip_utils.h"
#include "quantized_gemm.cuh"
#include "tensor_core_gemm.cuh"

namespace flash_engine {

constexpr int VERSION_MAJOR = 1;
constexpr int VERSION_MINOR = 2;
constexpr int VERSION_PATCH = 0;

inline const char* get_version() { return "1.2.0"; }

// Prints the GPU's properties (CUs, wavefront size, LDS, memory).
inline void print_device_info(int device_id = 0) {
    HIP_CHECK(static_cast<hipError_t>(fke_print_device_info(device_id)));
}

}  // namespace flash_engine
