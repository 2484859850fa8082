// probe_mfma.hip — measurement probe, not part of the GEMM path: the INT8
// matrix-core ceiling on a given operand distribution.  Each wave streams
// v_mfma_i32_32x32x32_i8 in the order the GEMM's 256x256 tile issues them
// (4 x 4 blocks of 32x32 per k step, two fragment sets alternating), on
// operands loaded once into registers from `src`, with no LDS or global
// traffic in the loop.  With random int8 in `src` the matrix cores toggle as
// in the GEMM, so the sustained rate under the board's power limit is the
// ceiling the GEMM's time is measured against; on constant operands it is
// the clock-limited peak.  Built into libfke_probe.so (bench.py
// --mfma-ceiling), separately from libfke_qgemm.so.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kFrags = 16;  // two sets of 4 A and 4 B fragments per wave

// One workgroup of 4 waves per CU (256 accumulator AGPRs per lane leave room
// for one wave per SIMD).  Wave w of the grid reads kFrags x 64 lanes x 16
// bytes of src from w * 16 KiB; `out` gets one xor of its accumulators per
// lane so the MFMAs are live.
__global__ __launch_bounds__(256, 1) void probe_mfma_i8_kernel(const v4i* __restrict__ src, int32_t* __restrict__ out,
                                                              int iters) {
    const int lane = threadIdx.x & 63;
    const size_t gw = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const v4i* s = src + gw * kFrags * 64 + lane;
    v4i fa[2][4], fb[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            fa[t][i] = s[(8 * t + i) * 64];
            fb[t][i] = s[(8 * t + 4 + i) * 64];
        }
    v16i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[t][i], fb[t][j], acc[i][j], 0, 0, 0);
    }
    int32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) x ^= acc[i][j][v];
    out[gw * 64 + lane] = x;
}

}  // namespace

extern "C" {

// Bytes of src and elements of out a launch of `grid` workgroups reads and writes.
size_t fke_probe_mfma_src_bytes(int grid) { return static_cast<size_t>(grid) * 4 * kFrags * 64 * 16; }
size_t fke_probe_mfma_out_elems(int grid) { return static_cast<size_t>(grid) * 4 * 64; }

// grid workgroups x 4 waves x iters x 32 MFMAs of 2*32*32*32 operations each.
int fke_probe_mfma_i8(const void* src, int32_t* out, int grid, int iters, void* stream) {
    if (!src || !out || grid < 1 || iters < 1) return hipErrorInvalidValue;
    const v4i* s = static_cast<const v4i*>(src);
    void* args[] = {&s, &out, &iters};
    return hipLaunchKernel(reinterpret_cast<const void*>(&probe_mfma_i8_kernel), dim3(grid), dim3(256), args, 0,
                           static_cast<hipStream_t>(stream));
}

}  // extern "C"
