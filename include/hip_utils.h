/*
 * hip_utils.h — host-side error macros for callers of the quantized GEMM API.
 * Mirrors the caller-facing part of reference include/cuda_utils.cuh:13-31
 * (CUDA_CHECK / CUDA_CHECK_LAST_ERROR: print file:line and exit on error),
 * expressed over the HIP runtime API.  Device helpers of that header
 * (warp-32 shuffles) have no counterpart: gfx950 runs 64-wide wavefronts and
 * the kernels reduce with DPP/ds_swizzle inside the library.
 */
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>

#define HIP_CHECK(call)                                                       \
    do {                                                                      \
        hipError_t err_ = (call);                                             \
        if (err_ != hipSuccess) {                                             \
            fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,   \
                    hipGetErrorString(err_));                                 \
            exit(EXIT_FAILURE);                                               \
        }                                                                     \
    } while (0)

#define HIP_CHECK_LAST_ERROR()                                                \
    do {                                                                      \
        hipError_t err_ = hipGetLastError();                                  \
        if (err_ != hipSuccess) {                                             \
            fprintf(stderr, "HIP kernel launch error at %s:%d: %s\n",         \
                    __FILE__, __LINE__, hipGetErrorString(err_));             \
            exit(EXIT_FAILURE);                                               \
        }                                                                     \
    } while (0)
