// gemm_generic.hip — any-shape fallback GEMM (INT8, FP8, fp16, bf16; both B layouts).
//
// Used when a call does not meet the fast families' shape/alignment needs
// (e.g. K % 128 != 0 for prefill, odd K, unaligned pointers).  It keeps the
// reference's arithmetic exactly:
//   INT8 — reference src/quantized_gemm.cu:33-52 (int32 sum of byte products,
//          here over the full K like tests/test_quantized_gemm.cu:43-45);
//   FP8  — reference src/quantized_gemm.cu:109-116: each output is summed in
//          fp32 over k = 0..K-1 in increasing order, so the result is
//          bit-identical to the reference's sequential loop.
//   fp16 / bf16 — the same sequential fp32 sum of exact products (reference
//          src/tensor_core_attention.cu:13-66 leaves the order to the WMMA unit).
// 64x64 output tile per 256-thread workgroup, 4x4 outputs per thread, K staged
// through LDS 64 elements at a time with bounds-checked element loads (zero
// fill past M/N/K adds exact zeros).
//
// SwiGLU (INT8, B = [gate; up] of 2I rows): a tile covers 32 outputs; its
// B column c = 4t + j holds gate row o (j = 0, 1) or up row I + o (j = 2, 3)
// of output o = n0 + 2t + (j & 1), so each thread's columns j and j + 2 are
// the two operands of one output.
#include "fke_internal.h"

namespace fke {
namespace {

constexpr int T = 64;   // tile edge
constexpr int KC = 64;  // K elements per LDS stage

// Raw bits of element idx (a byte, or 16 bits for fp16 / bf16).
template <int ELEM>
__device__ __forceinline__ uint32_t load_raw(const void* base, size_t idx) {
    if constexpr (elem_bytes(ELEM) == 2) return static_cast<const uint16_t*>(base)[idx];
    else return static_cast<const uint8_t*>(base)[idx];
}

// Value of a float-type element (FP8, fp16, bf16), exact in fp32.
template <int ELEM>
__device__ __forceinline__ float decode(uint32_t raw) {
    if constexpr (ELEM == ELEM_F8) return e4m3_decode(raw);
    else if constexpr (ELEM == ELEM_F16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(raw)));
    else return __uint_as_float(raw << 16);
}

template <int ELEM, int OUT, bool SWI = false>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmArgs p) {
    static_assert(!SWI || (ELEM == ELEM_I8 && OUT != FKE_OUT_I32), "SwiGLU: INT8, float out");
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * T, n0 = blockIdx.x * (SWI ? T / 2 : T);  // n0: first output column
    const int M = p.M, N = p.N, K = p.K;
    const int NO = SWI ? N >> 1 : N;  // output columns
    const bool kn = p.b_layout == FKE_B_KN;

    // INT8: packed 4-byte words (KC/4 per row, +1 pad); FP8 / fp16 / bf16: decoded floats.
    constexpr bool INT = ELEM == ELEM_I8;
    __shared__ int32_t Aw[INT ? T : 1][KC / 4 + 1];
    __shared__ int32_t Bw[INT ? T : 1][KC / 4 + 1];
    __shared__ float Af[INT ? 1 : T][KC + 1];
    __shared__ float Bf[INT ? 1 : T][KC + 1];

    int32_t iacc[4][4];
    float facc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            iacc[i][j] = 0;
            facc[i][j] = 0.0f;
        }

    for (int k0 = 0; k0 < K; k0 += KC) {
        // Stage: thread t loads 16 elements of A (row t/4, k 16*(t%4)..) and
        // 16 elements of B for one (n row, 16 k) slice.
        {
            const int r = tid >> 2, kq = (tid & 3) * 16;
            const int m = m0 + r;
            uint32_t a[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int k = k0 + kq + q;
                a[q] = (m < M && k < K) ? load_raw<ELEM>(p.A, static_cast<size_t>(m) * K + k) : 0;
            }
            uint32_t b[16];
            int bn, bk;
            if (kn) {  // coalesce along n: thread t -> column t%64, k block t/64
                bn = tid & 63;
                bk = (tid >> 6) * 16;
            } else {
                bn = r;
                bk = kq;
            }
            int n = n0 + bn;  // B row (NK) / column (KN) of tile column bn
            bool n_ok = n < N;
            if constexpr (SWI) {
                const int o = n0 + 2 * (bn >> 2) + (bn & 1);
                n = (bn & 2) ? NO + o : o;
                n_ok = o < NO;
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int k = k0 + bk + q;
                uint32_t v = 0;
                if (n_ok && k < K)
                    v = load_raw<ELEM>(p.B, kn ? static_cast<size_t>(k) * N + n : static_cast<size_t>(n) * K + k);
                b[q] = v;
            }
            if constexpr (INT) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    Aw[r][kq / 4 + q] = static_cast<int32_t>(a[4 * q] | (a[4 * q + 1] << 8) |
                                                             (a[4 * q + 2] << 16) |
                                                             (static_cast<uint32_t>(a[4 * q + 3]) << 24));
                    Bw[bn][bk / 4 + q] = static_cast<int32_t>(b[4 * q] | (b[4 * q + 1] << 8) |
                                                              (b[4 * q + 2] << 16) |
                                                              (static_cast<uint32_t>(b[4 * q + 3]) << 24));
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    Af[r][kq + q] = decode<ELEM>(a[q]);
                    Bf[bn][bk + q] = decode<ELEM>(b[q]);
                }
            }
        }
        __syncthreads();
        if constexpr (ELEM == ELEM_I8) {
#pragma unroll 4
            for (int kw = 0; kw < KC / 4; ++kw) {
                int32_t a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = Aw[ty * 4 + i][kw];
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = Bw[tx * 4 + j][kw];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        iacc[i][j] = __builtin_amdgcn_sdot4(a[i], b[j], iacc[i][j], false);
            }
        } else {
            const int kend = min(KC, K - k0);  // reference order: k ascending, stop at K
            for (int k = 0; k < kend; ++k) {
                float a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = Af[ty * 4 + i][k];
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = Bf[tx * 4 + j][k];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) facc[i][j] += a[i] * b[j];  // exact product
            }
        }
        __syncthreads();
    }

    if constexpr (SWI) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + ty * 4 + i;
            if (m >= M) continue;
            const float sam = p.scale_a ? p.scale_a[m] : p.sa;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + 2 * tx + j;
                if (n >= NO) continue;
                const float yg = epilogue_value(static_cast<float>(iacc[i][j]),
                                                sam * (p.scale_b ? p.scale_b[n] : p.sb), p.bias, n);
                const float yu = epilogue_value(static_cast<float>(iacc[i][j + 2]),
                                                sam * (p.scale_b ? p.scale_b[NO + n] : p.sb), p.bias, NO + n);
                store_out<OUT>(p.C, static_cast<size_t>(m) * NO + n, swiglu_pair(yg, yu), 0);
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n >= N) continue;
            const size_t idx = static_cast<size_t>(m) * N + n;
            // (FP8 calls carry no scale vectors: s = fp32(sa * sb))
            const float s = (p.scale_a ? p.scale_a[m] : p.sa) * (p.scale_b ? p.scale_b[n] : p.sb);
            if constexpr (ELEM == ELEM_I8)
                store_out<OUT>(p.C, idx, epilogue_value(static_cast<float>(iacc[i][j]), s, p.bias, n),
                               iacc[i][j]);
            else
                store_out<OUT>(p.C, idx, epilogue_value(facc[i][j], s, p.bias, n), 0);
        }
    }
}

template <int ELEM, int OUT>
hipError_t launch_t(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const dim3 grid((p.N + T - 1) / T, (p.M + T - 1) / T);
    return hipLaunchKernel(reinterpret_cast<const void*>(&gemm_generic_kernel<ELEM, OUT>), grid,
                           dim3(256), args, 0, stream);
}

}  // namespace

hipError_t launch_generic(const GemmArgs& p, int elem, hipStream_t s) {
    if (p.swiglu) {
        GemmArgs a = p;
        void* args[] = {&a};
        const dim3 grid((p.N / 2 + T / 2 - 1) / (T / 2), (p.M + T - 1) / T);
        const void* f = p.out_dtype == FKE_OUT_F32
            ? reinterpret_cast<const void*>(&gemm_generic_kernel<ELEM_I8, FKE_OUT_F32, true>)
            : reinterpret_cast<const void*>(&gemm_generic_kernel<ELEM_I8, FKE_OUT_BF16, true>);
        return hipLaunchKernel(f, grid, dim3(256), args, 0, s);
    }
    if (elem == ELEM_I8) {
        switch (p.out_dtype) {
            case FKE_OUT_F32: return launch_t<ELEM_I8, FKE_OUT_F32>(p, s);
            case FKE_OUT_BF16: return launch_t<ELEM_I8, FKE_OUT_BF16>(p, s);
            default: return launch_t<ELEM_I8, FKE_OUT_I32>(p, s);
        }
    }
    if (elem == ELEM_F16)
        return p.out_dtype == FKE_OUT_F32 ? launch_t<ELEM_F16, FKE_OUT_F32>(p, s)
                                          : launch_t<ELEM_F16, FKE_OUT_BF16>(p, s);
    if (elem == ELEM_BF16)
        return p.out_dtype == FKE_OUT_F32 ? launch_t<ELEM_BF16, FKE_OUT_F32>(p, s)
                                          : launch_t<ELEM_BF16, FKE_OUT_BF16>(p, s);
    return p.out_dtype == FKE_OUT_F32 ? launch_t<ELEM_F8, FKE_OUT_F32>(p, s)
                                      : launch_t<ELEM_F8, FKE_OUT_BF16>(p, s);
}

}  // namespace fke
