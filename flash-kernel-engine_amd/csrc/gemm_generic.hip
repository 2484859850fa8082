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

// ===========================================================================
// INT8 word kernel: B [N,K] with K % 4 == 0 and A, B 4-byte aligned (the
// reference's own INT8 domain: K / 4 packed words per row,
// src/quantized_gemm.cu:28-37), for the shapes the MFMA GEMM's 16-byte copies
// cannot take (K % 16 != 0, or pointers not 16-byte aligned).  128x128 output
// tile per 256-thread workgroup, wave w the 64x64 block (w / 2, w % 2).  K
// runs in stages of 64 bytes through a ring of WNS stages in LDS, copied with
// 4-byte LDS-DMA loads (buffer_load_dword ... lds: lane l's word lands at
// 4l of the instruction's 256 bytes), so no registers hold the stages in
// flight; words past M, N or K read zero through the buffer range (K % 4 ==
// 0: a word is all in K or all out).  A stage row (one M row of A, one N row
// of B) is 64 bytes, logical 16-byte chunk c at physical chunk c ^ w_swz(r):
// the 16 rows of a 16-lane fragment read then cover all 64 banks once.  The
// waves multiply each stage with v_mfma_i32_16x16x64_i8, lane (g, r) of a
// fragment taking bytes 16g .. 16g + 15 of row r.  Exact int32 sums, then the
// same epilogue as the generic kernel.
// ===========================================================================
constexpr int WT = 128;                   // tile edge
constexpr int WKC = 64;                   // K bytes per stage
constexpr int WNS = 4;                    // ring stages (64 KiB of LDS)
constexpr int WOP = WT * WKC;             // bytes of one operand's stage (8 KiB)
constexpr int WCP = WOP / (4 * 256);      // 4-byte copies per wave, operand and stage (8)
static_assert(WCP == 8 && WNS == 4, "copy and wait counts below");

typedef int w4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t w_lds;

// Physical chunk of a stage row r is logical chunk ^ w_swz(r).
__device__ __forceinline__ int w_swz(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ w4i w_rd128(const w_lds* a) {
    w4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

template <int OUT>
__global__ __launch_bounds__(256) void gemm_i8_words_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[WNS][2][WOP];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int M = p.M, N = p.N, K = p.K;
    const int m0 = blockIdx.y * WT, n0 = blockIdx.x * WT;
    const int nst = (K + WKC - 1) / WKC;

    // Copy i of wave w (each operand): stage bytes 256 (8w + i) + 4l = tile
    // row r = 4 (8w + i) + l / 16, physical chunk (l % 16) / 4, word l % 4,
    // which holds logical chunk ((l % 16) / 4) ^ w_swz(r), w_swz(r) = i & 3.
    // Offsets are 32-bit (M K and N K below 2^31); bit 31 set reads zero.
    const int lr = lane >> 4, pc = (lane & 15) >> 2, dw = lane & 3;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, M * K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, N * K);
    uint32_t arow[WCP], brow[WCP];
#pragma unroll
    for (int i = 0; i < WCP; ++i) {
        const int r = 4 * (WCP * wave + i) + lr;
        arow[i] = m0 + r < M ? static_cast<uint32_t>((m0 + r) * K) : 0x80000000u;
        brow[i] = n0 + r < N ? static_cast<uint32_t>((n0 + r) * K) : 0x80000000u;
    }
    int kof[4];  // byte of the stage this lane copies, for copies with i % 4 == j
#pragma unroll
    for (int j = 0; j < 4; ++j) kof[j] = 16 * (pc ^ j) + 4 * dw;
    auto issue = [&](int s) __attribute__((always_inline)) {
        const int k0 = s * WKC, slot = s % WNS;
#pragma unroll
        for (int i = 0; i < WCP; ++i) {
            const int kb = k0 + kof[i & 3];
            const bool in = kb < K;
            const int dst = (WCP * wave + i) * 256;
            dma4(ra, in ? arow[i] + static_cast<uint32_t>(kb) : 0x80000000u, 0, &ring[slot][0][dst]);
            dma4(rb, in ? brow[i] + static_cast<uint32_t>(kb) : 0x80000000u, 0, &ring[slot][1][dst]);
        }
    };

    // Fragment reads: lane (g, r) = (lane / 16, lane % 16) reads logical
    // chunk g of row 16 x + r of the wave's 64 rows.
    const int g = lane >> 4, rr = lane & 15;
    uint32_t fa[4], fb[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        const int ra_ = wm * 64 + 16 * x + rr, rb_ = wn * 64 + 16 * x + rr;
        fa[x] = static_cast<uint32_t>(ra_ * WKC + 16 * (g ^ w_swz(ra_)));
        fb[x] = static_cast<uint32_t>(WOP + rb_ * WKC + 16 * (g ^ w_swz(rb_)));
    }
    const w_lds* const lring = (const w_lds*)(&ring[0][0][0]);

    w4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = w4i{0, 0, 0, 0};

#pragma unroll
    for (int s = 0; s < WNS - 1; ++s)
        if (s < nst) issue(s);
    for (int s = 0; s < nst; ++s) {
        // Stage s has landed once at most the copies of the stages issued
        // after it (s + 1 .. s + WNS - 2, those below nst) are in flight; the
        // barrier then also says that every wave is done with stage s - 1,
        // whose slot takes stage s + WNS - 1.
        const int later = min(nst - 1 - s, WNS - 2);
        if (later == 0) wait_vm<0>();
        else if (later == 1) wait_vm<2 * WCP>();
        else wait_vm<4 * WCP>();
        barrier();
        if (s + WNS - 1 < nst) issue(s + WNS - 1);
        const w_lds* st = lring + (s % WNS) * 2 * WOP;
        w4i af[4], bf[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) af[x] = w_rd128(st + fa[x]);
#pragma unroll
        for (int x = 0; x < 4; ++x) bf[x] = w_rd128(st + fb[x]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int x = 0; x < 4; ++x) asm volatile("" : "+v"(af[x]), "+v"(bf[x]));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }

    // Lane (g, c) of block (i, j) holds rows 16i + 4g + v, column 16j + c of the wave's block.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = m0 + wm * 64 + 16 * i + 4 * g + v;
            if (m >= M) continue;
            const float sam = p.scale_a ? p.scale_a[m] : p.sa;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = n0 + wn * 64 + 16 * j + rr;
                if (n >= N) continue;
                const int32_t s32 = acc[i][j][v];
                const float s = sam * (p.scale_b ? p.scale_b[n] : p.sb);
                store_out<OUT>(p.C, static_cast<size_t>(m) * N + n, epilogue_value(static_cast<float>(s32), s, p.bias, n),
                               s32);
            }
        }
}

}  // namespace

bool words_supports(const GemmArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (p.M < 1 || p.N < 1 || p.K < 4 || p.K % 4 != 0 || p.swiglu || p.b_layout != FKE_B_NK) return false;
    if ((a | b) & 3) return false;
    if ((static_cast<int64_t>(p.M) + WT - 1) / WT > 65535) return false;  // grid y
    // 32-bit buffer offsets
    return static_cast<int64_t>(p.M) * p.K <= INT32_MAX && static_cast<int64_t>(p.N) * p.K <= INT32_MAX;
}

hipError_t launch_words(const GemmArgs& p, hipStream_t s) {
    if (!words_supports(p)) return hipErrorInvalidValue;
    GemmArgs a = p;
    void* args[] = {&a};
    const dim3 grid((p.N + WT - 1) / WT, (p.M + WT - 1) / WT);
    const void* f = p.out_dtype == FKE_OUT_F32    ? reinterpret_cast<const void*>(&gemm_i8_words_kernel<FKE_OUT_F32>)
                    : p.out_dtype == FKE_OUT_BF16 ? reinterpret_cast<const void*>(&gemm_i8_words_kernel<FKE_OUT_BF16>)
                                                  : reinterpret_cast<const void*>(&gemm_i8_words_kernel<FKE_OUT_I32>);
    return hipLaunchKernel(f, grid, dim3(256), args, 0, s);
}

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
