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

#include <type_traits>

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
// Word kernel: INT8 and FP8 with K % 4 == 0, A and B 4-byte aligned (and
// N % 4 == 0 for B [K,N]), for the shapes the MFMA GEMM's 16-byte copies
// cannot take (K or, for B [K,N], N not a multiple of 16, or pointers not
// 16-byte aligned).  The reference's INT8 kernel takes any K that is a
// multiple of 4 (K / 4 packed words per row, src/quantized_gemm.cu:28-37);
// its FP8 kernel any shape with B [K,N] (src/quantized_gemm.cu:99-118).
// 128x128 output tile per 256-thread workgroup, wave w the 64x64 block
// (w / 2, w % 2), or 128x64 with 64x32 blocks (launch_words says when).  K
// runs in stages of 64 bytes through a ring of 3 (INT8) or 4 (FP8) stages
// in LDS, copied with 4-byte LDS-DMA loads (buffer_load_dword ... lds: lane
// l's word lands at 4l of the instruction's 256 bytes), so no registers hold
// the stages in flight; words past M, N or K read zero through the buffer
// range (a word is all in or all out).  Stage rows of A and of B [N,K] are 64
// k bytes, logical 16-byte chunk c of row r at physical chunk c ^ ((r >> 2) &
// 3); B [K,N] is 64 k rows of the tile's column bytes, chunk c of k row r at
// c ^ (r & 7) (128 bytes) or c ^ ((r >> 2) & 1) (64 bytes), read with the
// transposing ds_read_b64_tr_b8.  Either way a 16-lane
// fragment read covers the 64 banks once.  Lane (g, r) of a fragment holds k
// bytes 16g .. 16g + 15 of row (column) r: INT8 multiplies them with
// v_mfma_i32_16x16x64_i8 (exact int32 sums); FP8 with
// v_mfma_scale_f32_16x16x128_f8f6f4, each lane's 32-byte operand being its
// 16 bytes and 16 zero bytes in A and B alike (half the MFMA's k slots hold
// zeros; the kernel is bound by its copies, not its MFMAs).  FP8 codes 0x7F
// / 0xFF (NaN to the MFMA, 0.0 to the reference) make a sum NaN; the
// workgroup then runs its K loop again with them cleared.  The epilogue is
// the generic kernel's.
// ===========================================================================
constexpr int WT = 128;               // tile rows (and columns of the wide tile)
constexpr int WKC = 64;               // K bytes per stage
constexpr int WOP = WT * WKC;         // bytes of A's stage (8 KiB)
constexpr int WCP = WOP / (4 * 256);  // 4-byte copies per wave and stage of A (8)
static_assert(WCP == 8, "copy and wait counts below");
// Ring stages: INT8 3 (48 / 36 KiB of LDS for the wide / narrow tile, 138
// registers: three workgroups per CU), FP8 4 (its replay's registers allow
// two workgroups per CU either way, and the deeper ring keeps more in
// flight).  Same box, bf16 out: INT8 4096 x 11008 x 4100 401.9 against 443.5
// us with 4 stages, 16 x 14336 x 4100 32.8 against 34.1; FP8 B [K,N] 64 x
// 14336 x 4100 45.8 with 4 stages against 48.2 with 3.
template <int EL>
constexpr int words_stages() {
    return EL == ELEM_F8 ? 4 : 3;
}

typedef int w2i __attribute__((ext_vector_type(2)));
typedef int w4i __attribute__((ext_vector_type(4)));
typedef int w8i __attribute__((ext_vector_type(8)));
typedef float w4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t w_lds;

__device__ __forceinline__ w4i w_rd128(const w_lds* a) {
    w4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ w2i w_rdtr(const w_lds* a) {
    w2i r;
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

// BN: tile columns, 128 or 64 (the narrow tile doubles the workgroups of
// shapes with few 128x128 tiles); wave w takes columns (w % 2) BN / 2 ...
// SWI (INT8, B [N,K] = [gate; up], N = 2I): tile column c < BN / 2 is gate
// row o0 + c and column BN / 2 + c up row I + o0 + c, o0 the tile's first
// of its BN / 2 outputs, so the waves with w % 2 = 0 hold gate sums and
// those with w % 2 = 1 the matching up sums; the up values meet the gate
// values in LDS and each output is swiglu_pair of the two epilogue values.
template <int EL, int BL, int OUT, int BN, bool SWI = false>
__global__ __launch_bounds__(256) void gemm_words_kernel(GemmArgs p) {
    constexpr bool F8 = EL == ELEM_F8, KN = BL == FKE_B_KN;
    static_assert(BN == 128 || BN == 64, "tile columns");
    static_assert(!SWI || (EL == ELEM_I8 && !KN && OUT != FKE_OUT_I32), "SwiGLU: INT8, B [N,K], float out");
    constexpr int NJ = BN / 32;                  // 16-column blocks per wave
    constexpr int WOPB = BN * WKC;               // bytes of B's stage
    constexpr int WCPB = WOPB / (4 * 256);       // 4-byte copies per wave and stage of B (8 or 4)
    constexpr int WNS = words_stages<EL>();
    static_assert(WNS >= 3 && WNS <= 4, "the waits below count at most two later stages");
    using Acc = typename std::conditional<F8, w4f, w4i>::type;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[WNS][WOP + WOPB];
    __shared__ int nan_seen;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int M = p.M, N = p.N, K = p.K;
    const int m0 = blockIdx.y * WT, n0 = blockIdx.x * BN;
    const int nst = (K + WKC - 1) / WKC;
    if constexpr (F8) {
        if (tid == 0) nan_seen = 0;
        __syncthreads();  // before any wave can set it (no copy is in flight yet)
    }

    // Copy i of wave w, 64-byte rows (A; B [N,K]): stage bytes 256 (c w + i)
    // + 4l, c = the wave's copies, = row r = 4 (c w + i) + l / 16, physical
    // chunk (l % 16) / 4, word l % 4, holding logical chunk ((l % 16) / 4) ^
    // (i & 3) (c is a multiple of 4).  B [K,N], 128-byte rows: stage bytes
    // 256 (8w + i) + 4l = k row kr = 2 (8w + i) + l / 32, physical chunk
    // (l % 32) / 4, word l % 4, holding logical chunk ((l % 32) / 4) ^ (kr &
    // 7); 64-byte rows: k row kr = 4 (4w + i) + l / 16, physical chunk (l %
    // 16) / 4, holding logical chunk ((l % 16) / 4) ^ ((kr >> 2) & 1).
    // Offsets are 32-bit (M K and N K below 2^31); bit 31 set reads zero.
    const int lr = lane >> 4, pc = (lane & 15) >> 2, dw = lane & 3;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, M * K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, N * K);
    uint32_t arow[WCP], brow[WCPB];
    int bkr[WCPB];
#pragma unroll
    for (int i = 0; i < WCP; ++i) {
        const int r = 4 * (WCP * wave + i) + lr;
        arow[i] = m0 + r < M ? static_cast<uint32_t>((m0 + r) * K) : 0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < WCPB; ++i) {
        if constexpr (KN) {
            int kr, c;
            if constexpr (BN == 128) {
                kr = 2 * (WCPB * wave + i) + (lane >> 5);
                c = ((lane & 31) >> 2) ^ (kr & 7);
            } else {
                kr = 4 * (WCPB * wave + i) + lr;
                c = pc ^ ((kr >> 2) & 1);
            }
            const int col = n0 + 16 * c + 4 * dw;
            bkr[i] = kr;
            brow[i] = col < N ? static_cast<uint32_t>(col) : 0x80000000u;
        } else if constexpr (SWI) {
            const int r = 4 * (WCPB * wave + i) + lr, half = BN / 2, I = N >> 1;
            const int o = blockIdx.x * half + (r < half ? r : r - half);  // the row's output
            bkr[i] = 0;
            brow[i] = o < I ? static_cast<uint32_t>((r < half ? o : I + o) * K) : 0x80000000u;
        } else {
            const int r = 4 * (WCPB * wave + i) + lr;
            bkr[i] = 0;
            brow[i] = n0 + r < N ? static_cast<uint32_t>((n0 + r) * K) : 0x80000000u;
        }
    }
    int kof[4];  // byte of the stage this lane copies (64-byte rows), for copies with i % 4 == j
#pragma unroll
    for (int j = 0; j < 4; ++j) kof[j] = 16 * (pc ^ j) + 4 * dw;
    auto issue = [&](int s) __attribute__((always_inline)) {
        const int k0 = s * WKC, slot = s % WNS;
#pragma unroll
        for (int i = 0; i < WCP; ++i) {
            const int kb = k0 + kof[i & 3];
            dma4(ra, kb < K ? arow[i] + static_cast<uint32_t>(kb) : 0x80000000u, 0,
                 &ring[slot][(WCP * wave + i) * 256]);
        }
#pragma unroll
        for (int i = 0; i < WCPB; ++i) {
            uint8_t* dst = &ring[slot][WOP + (WCPB * wave + i) * 256];
            if constexpr (KN) {
                const int k = k0 + bkr[i];
                dma4(rb, k < K ? brow[i] + static_cast<uint32_t>(k * N) : 0x80000000u, 0, dst);
            } else {
                const int kb = k0 + kof[i & 3];
                dma4(rb, kb < K ? brow[i] + static_cast<uint32_t>(kb) : 0x80000000u, 0, dst);
            }
        }
    };

    // Fragment reads: lane (g, rr) = (lane / 16, lane % 16); A and B [N,K]:
    // logical chunk g of row 16 x + rr of the wave's rows.  B [K,N]: two
    // transposing reads, k rows 16g + 8t + b (b = rr / 2) at the 8-byte half
    // rr % 2 of the wave's column block x.
    const int g = lane >> 4, rr = lane & 15;
    uint32_t fa[4], fb[NJ][2];
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        const int ar = wm * 64 + 16 * x + rr;
        fa[x] = static_cast<uint32_t>(ar * WKC + 16 * (g ^ ((ar >> 2) & 3)));
    }
#pragma unroll
    for (int x = 0; x < NJ; ++x) {
        if constexpr (KN) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int kr = 16 * g + 8 * t + (rr >> 1);
                const int c = NJ * wn + x, sw = BN == 128 ? (kr & 7) : ((kr >> 2) & 1);
                fb[x][t] = static_cast<uint32_t>(WOP + kr * BN + 16 * (c ^ sw) + 8 * (rr & 1));
            }
        } else {
            const int br = wn * (BN / 2) + 16 * x + rr;
            fb[x][0] = fb[x][1] = static_cast<uint32_t>(WOP + br * WKC + 16 * (g ^ ((br >> 2) & 3)));
        }
    }
    const w_lds* const lring = (const w_lds*)(&ring[0][0]);

    Acc acc[4][NJ];
    auto k_loop = [&](auto sanc) __attribute__((always_inline)) {
        constexpr bool SAN = decltype(sanc)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[i][j] = Acc{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < WNS - 1; ++s)
            if (s < nst) issue(s);
        for (int s = 0; s < nst; ++s) {
            // Stage s has landed once at most the copies of the stages issued
            // after it (s + 1 .. s + WNS - 2, those below nst) are in flight;
            // the barrier then also says that every wave is done with stage
            // s - 1, whose slot takes stage s + WNS - 1.
            const int later = min(nst - 1 - s, WNS - 2);
            if (later == 0) wait_vm<0>();
            else if (later == 1) wait_vm<WCP + WCPB>();
            else wait_vm<2 * (WCP + WCPB)>();
            barrier();
            if (s + WNS - 1 < nst) issue(s + WNS - 1);
            const w_lds* st = lring + (s % WNS) * (WOP + WOPB);
            w4i af[4], bf[NJ];
#pragma unroll
            for (int x = 0; x < 4; ++x) af[x] = w_rd128(st + fa[x]);
            if constexpr (KN) {
                w2i t0[NJ], t1[NJ];
#pragma unroll
                for (int x = 0; x < NJ; ++x) {
                    t0[x] = w_rdtr(st + fb[x][0]);
                    t1[x] = w_rdtr(st + fb[x][1]);
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int x = 0; x < 4; ++x) asm volatile("" : "+v"(af[x]));
#pragma unroll
                for (int x = 0; x < NJ; ++x) {
                    asm volatile("" : "+v"(t0[x]), "+v"(t1[x]));
                    bf[x] = w4i{t0[x][0], t0[x][1], t1[x][0], t1[x][1]};
                }
            } else {
#pragma unroll
                for (int x = 0; x < NJ; ++x) bf[x] = w_rd128(st + fb[x][0]);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int x = 0; x < 4; ++x) asm volatile("" : "+v"(af[x]));
#pragma unroll
                for (int x = 0; x < NJ; ++x) asm volatile("" : "+v"(bf[x]));
            }
            if constexpr (F8) {
                if constexpr (SAN) {
#pragma unroll
                    for (int x = 0; x < 4; ++x)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            af[x][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(af[x][e])));
#pragma unroll
                    for (int x = 0; x < NJ; ++x)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            bf[x][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(bf[x][e])));
                }
                const w4i z = {0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const w8i a8 = __builtin_shufflevector(af[i], z, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            a8, __builtin_shufflevector(bf[j], z, 0, 1, 2, 3, 4, 5, 6, 7), acc[i][j], 0, 0, 0, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };
    k_loop(std::false_type{});
    if constexpr (F8) {
        // Every product of finite codes is finite and no sum of them
        // overflows fp32, so a NaN sum proves a NaN code; the workgroup
        // decides together (the K loop has barriers), after every wave is
        // done with the ring.
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) bad |= __builtin_isnan(acc[i][j][v]);
        if (__builtin_amdgcn_ballot_w64(bad) != 0 && lane == 0) nan_seen = 1;
        __syncthreads();
        if (nan_seen) k_loop(std::true_type{});
    }

    // Lane (g, c) of block (i, j) holds rows 16i + 4g + v, column 16j + c of the wave's block.
    if constexpr (SWI) {
        // the up waves' epilogue values, [wm][64 rows][BN / 2 outputs] fp32, in the ring's first bytes
        static_assert(2 * 64 * (BN / 2) * 4 <= WNS * (WOP + WOPB), "the exchange fits the ring");
        float* const xu = reinterpret_cast<float*>(&ring[0][0]);
        const int I = N >> 1, o0 = blockIdx.x * (BN / 2);
        __syncthreads();  // every wave is done with the ring
        if (wn == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = 16 * i + 4 * g + v, m = m0 + wm * 64 + row;
                    const float sam = m < M ? (p.scale_a ? p.scale_a[m] : p.sa) : 0.0f;
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int col = 16 * j + rr, o = o0 + col;
                        float y = 0.0f;
                        if (m < M && o < I)
                            y = epilogue_value(static_cast<float>(acc[i][j][v]),
                                               sam * (p.scale_b ? p.scale_b[I + o] : p.sb), p.bias, I + o);
                        xu[(wm * 64 + row) * (BN / 2) + col] = y;
                    }
                }
        }
        __syncthreads();
        if (wn == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = 16 * i + 4 * g + v, m = m0 + wm * 64 + row;
                    if (m >= M) continue;
                    const float sam = p.scale_a ? p.scale_a[m] : p.sa;
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const int col = 16 * j + rr, o = o0 + col;
                        if (o >= I) continue;
                        const float yg = epilogue_value(static_cast<float>(acc[i][j][v]),
                                                        sam * (p.scale_b ? p.scale_b[o] : p.sb), p.bias, o);
                        store_out<OUT>(p.C, static_cast<size_t>(m) * I + o,
                                       swiglu_pair(yg, xu[(wm * 64 + row) * (BN / 2) + col]), 0);
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = m0 + wm * 64 + 16 * i + 4 * g + v;
            if (m >= M) continue;
            const float sam = p.scale_a ? p.scale_a[m] : p.sa;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int n = n0 + wn * (BN / 2) + 16 * j + rr;
                if (n >= N) continue;
                // (FP8 calls carry no scale vectors: s = fp32(sa * sb))
                const float s = sam * (p.scale_b ? p.scale_b[n] : p.sb);
                if constexpr (F8) {
                    store_out<OUT>(p.C, static_cast<size_t>(m) * N + n, epilogue_value(acc[i][j][v], s, p.bias, n), 0);
                } else {
                    const int32_t s32 = acc[i][j][v];
                    store_out<OUT>(p.C, static_cast<size_t>(m) * N + n,
                                   epilogue_value(static_cast<float>(s32), s, p.bias, n), s32);
                }
            }
        }
}

}  // namespace

bool words_supports(const GemmArgs& p, int elem) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (elem != ELEM_I8 && elem != ELEM_F8) return false;
    if (elem == ELEM_F8 && p.out_dtype == FKE_OUT_I32) return false;
    if (p.M < 1 || p.N < 1 || p.K < 4 || p.K % 4 != 0) return false;
    if (p.swiglu && (elem != ELEM_I8 || p.b_layout != FKE_B_NK || p.out_dtype == FKE_OUT_I32 || p.N % 2)) return false;
    if (p.b_layout != FKE_B_NK && (p.b_layout != FKE_B_KN || p.N % 4 != 0)) return false;
    if ((a | b) & 3) return false;
    if ((static_cast<int64_t>(p.M) + WT - 1) / WT > 65535) return false;  // grid y
    // 32-bit buffer offsets
    return static_cast<int64_t>(p.M) * p.K <= INT32_MAX && static_cast<int64_t>(p.N) * p.K <= INT32_MAX;
}

namespace {
template <int EL, int BL, int BN>
const void* words_kernel(int out) {
    if constexpr (EL == ELEM_I8)
        if (out == FKE_OUT_I32) return reinterpret_cast<const void*>(&gemm_words_kernel<EL, BL, FKE_OUT_I32, BN>);
    return out == FKE_OUT_F32 ? reinterpret_cast<const void*>(&gemm_words_kernel<EL, BL, FKE_OUT_F32, BN>)
                              : reinterpret_cast<const void*>(&gemm_words_kernel<EL, BL, FKE_OUT_BF16, BN>);
}
template <int BN>
const void* words_kernel_for(int elem, bool kn, int out) {
    return elem == ELEM_I8 ? (kn ? words_kernel<ELEM_I8, FKE_B_KN, BN>(out) : words_kernel<ELEM_I8, FKE_B_NK, BN>(out))
                           : (kn ? words_kernel<ELEM_F8, FKE_B_KN, BN>(out) : words_kernel<ELEM_F8, FKE_B_NK, BN>(out));
}
}  // namespace

// 128x128 tiles, or 128x64 while those still number at most one per CU
// (decode-sized M): twice the workgroups, each streaming half the columns,
// each re-reading its A rows.  Same box, bf16 out + bias, 14336 x 4100:
// B [N,K] M = 16 34.0 against 48.4 us, B [K,N] M = 64 42.0 against 58.9; at
// M = 256 (224 wide tiles) 63.1 against 60.0 on the wide tile.  A SwiGLU
// tile's BN columns are BN / 2 outputs.
hipError_t launch_words(const GemmArgs& p, int elem, hipStream_t s) {
    if (!words_supports(p, elem)) return hipErrorInvalidValue;
    GemmArgs a = p;
    void* args[] = {&a};
    const int cols = p.swiglu ? p.N / 2 : p.N;  // output columns
    const int per = p.swiglu ? WT / 2 : WT;     // output columns of a wide tile
    const int64_t rows = (p.M + WT - 1) / WT, wide = (cols + per - 1) / per * rows;
    const bool kn = p.b_layout == FKE_B_KN, narrow = 2 * wide <= device_cus();
    const void* f;
    if (p.swiglu) {
        const bool f32 = p.out_dtype == FKE_OUT_F32;
        f = narrow ? (f32 ? reinterpret_cast<const void*>(&gemm_words_kernel<ELEM_I8, FKE_B_NK, FKE_OUT_F32, 64, true>)
                          : reinterpret_cast<const void*>(&gemm_words_kernel<ELEM_I8, FKE_B_NK, FKE_OUT_BF16, 64, true>))
                   : (f32 ? reinterpret_cast<const void*>(&gemm_words_kernel<ELEM_I8, FKE_B_NK, FKE_OUT_F32, 128, true>)
                          : reinterpret_cast<const void*>(&gemm_words_kernel<ELEM_I8, FKE_B_NK, FKE_OUT_BF16, 128, true>));
    } else {
        f = narrow ? words_kernel_for<64>(elem, kn, p.out_dtype) : words_kernel_for<128>(elem, kn, p.out_dtype);
    }
    const int tile_cols = narrow ? per / 2 : per;
    const dim3 grid((cols + tile_cols - 1) / tile_cols, static_cast<unsigned>(rows));
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
