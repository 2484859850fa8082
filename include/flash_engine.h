/*
 * flash_engine.h — umbrella header of the MI355X build of the quantized GEMM
 * path.  Mirrors reference include/flash_engine.h:17-31 (version constants,
 * get_version, print_device_info).  The reference's other module headers
 * (attention, decoding, RMSNorm, ...) are not part of this library.
 */
#pragma once

#include "hip_utils.h"
#include "quantized_gemm.cuh"

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
