// probe_read.hip — measurement probe, not part of the GEMM path: how fast a
// kernel that does nothing but read can stream a given number of bytes from
// HBM on this GPU.  The decode GEMV reads its weight panel once, so the
// fastest plain read of the same bytes, on the same box, is the attainable
// floor its time is measured against (beside the 8 TB/s specification).
// Each wave reads blocks of U KiB (lane l takes bytes 16l..16l+15 of each
// KiB, so one load instruction covers 1 KiB of contiguous bytes, as in the
// decode kernels' weight streams), non-temporal like them, blocks gw,
// gw + waves, ... of the whole grid; the loaded words are folded into one
// value per lane that is stored only when it equals `key`, so the loads stay
// live and the kernel writes (almost) nothing.  Built into libfke_probe.so
// (bench.py), separately from libfke_qgemm.so.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(512) void probe_read_kernel(const int8_t* __restrict__ src, int64_t nbytes,
                                                         int32_t* __restrict__ out, int32_t key) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t nblk = nbytes / (1024 * U);
    // 32-bit offsets: the host keeps nbytes below 2^31
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(src), 0, static_cast<int>(nbytes), 0x00020000);
    int32_t x = 0;
    for (int64_t b = gw; b < nblk; b += waves) {
        v4i v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            v[u] = __builtin_bit_cast(
                v4i, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(b * 1024 * U + u * 1024 + lane * 16), 0, 2));
#pragma unroll
        for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (x == key) out[gw] = x;
}

}  // namespace

extern "C" {

// Elements of out a launch of `grid` workgroups of `waves` waves may write.
size_t fke_probe_read_out_elems(int grid, int waves) { return static_cast<size_t>(grid) * waves; }

// Reads nbytes of src (a multiple of unit_kib KiB, below 2^31; unit_kib 4 or 8)
// with grid workgroups of `waves` waves (1..8).
int fke_probe_read(const void* src, int64_t nbytes, int32_t* out, int grid, int waves, int unit_kib, int32_t key,
                   void* stream) {
    if (!src || !out || grid < 1 || waves < 1 || waves > 8 || (unit_kib != 4 && unit_kib != 8) || nbytes <= 0 ||
        nbytes >= (int64_t{1} << 31) || nbytes % (1024 * unit_kib) != 0)
        return hipErrorInvalidValue;
    const int8_t* s = static_cast<const int8_t*>(src);
    void* args[] = {&s, &nbytes, &out, &key};
    const void* f = unit_kib == 4 ? reinterpret_cast<const void*>(&probe_read_kernel<4>)
                                  : reinterpret_cast<const void*>(&probe_read_kernel<8>);
    return hipLaunchKernel(f, dim3(grid), dim3(waves * 64), args, 0, static_cast<hipStream_t>(stream));
}

}  // extern "C"
