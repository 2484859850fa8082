// gemv_i8.hip — W8A8 decode path (M <= 16, and batches up to
// FKE_GEMV_MAX_M rows where it beats the MFMA GEMM; B stored [N,K]).
//
// Same arithmetic as reference src/quantized_gemm.cu:15-54 (exact int32 dot
// products, the fused epilogue applied after), re-shaped for an HBM-bound
// problem: the B panel is streamed once with 128-bit coalesced loads.
//
// Four kernels:
//  * gemv_lds_kernel (3 <= M <= 16 with K >= 4096; 17 <= M <= 512 with
//    K >= 2048), described at its definition: the weight panel streamed
//    through LDS by one workgroup per CU, each weight fragment multiplied
//    with up to four 16-row activation blocks.
//  * gemv_rows_kernel (M <= 4): NB B rows per wave (one at M = 1, two for
//    M = 2..4 and for SwiGLU's gate/up pairs) over the full K.  Lane l reads
//    16-byte chunks l, l+64, l+128, l+192 of each 256-chunk block (one wave
//    load = 1 KiB contiguous) with non-temporal buffer loads, keeps the M
//    activation chunks in registers for the NB rows, and reduces its partial
//    sums with DPP row rotations, one ds_swizzle and two readlanes - no LDS
//    and no barrier, so a wave retires as soon as its rows are done and the
//    load queue never drains.  Also the FP8 decode at M = 1 (E4M3 codes
//    converted to fp32 in registers, fp32 FMAs).
//  * gemv_i8_kernel (5 <= M <= 16 when neither MFMA kernel's 32-bit offsets
//    reach), described below; it amortises the activation chunks over R
//    rows per wave.
//  * gemv_mfma_kernel (5 <= M <= 16, K < 4096), described at its definition.
//
// gemv_i8_kernel: workgroup = 4 waves = R consecutive B rows (output columns n0..n0+R-1).
// The K bytes of a row are split in four quarters, one per wave (split-K);
// lane l of a wave reads 16-byte chunks l, l+64, ... of its quarter, so each
// load instruction of a wave covers 1 KiB of contiguous bytes of one row.
// The wave keeps its A chunks (MT rows x 16 bytes) in registers and issues
// the R row loads back to back before any arithmetic.
// Partial int32 sums (R x MT per lane) are reduced across the 256 threads
// through LDS: every thread writes its partials, then G = 256/(R*MT)
// consecutive lanes sum one output's 256 partials and finish with a DPP/
// swizzle butterfly inside the wave.  Integer addition is associative, so any
// split and order is bit-exact.
#include "fke_internal.h"

#include <algorithm>

namespace fke {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int32_t dot16(v4i a, v4i b, int32_t acc) {
    acc = __builtin_amdgcn_sdot4(a[0], b[0], acc, false);
    acc = __builtin_amdgcn_sdot4(a[1], b[1], acc, false);
    acc = __builtin_amdgcn_sdot4(a[2], b[2], acc, false);
    acc = __builtin_amdgcn_sdot4(a[3], b[3], acc, false);
    return acc;
}

// Sum over groups of G consecutive lanes (G a power of two <= 64); every lane
// of the group ends with the group sum.
template <int G>
__device__ __forceinline__ int32_t group_sum(int32_t v) {
    if constexpr (G >= 2) v += __shfl_xor(v, 1);
    if constexpr (G >= 4) v += __shfl_xor(v, 2);
    if constexpr (G >= 8) v += __shfl_xor(v, 4);
    if constexpr (G >= 16) v += __shfl_xor(v, 8);
    if constexpr (G >= 32) v += __shfl_xor(v, 16);
    if constexpr (G >= 64) v += __shfl_xor(v, 32);
    return v;
}

template <int MT, int R, int OUT>
__global__ __launch_bounds__(256) void gemv_i8_kernel(GemmArgs p) {
    constexpr int V = R * MT;      // outputs per workgroup
    constexpr int G = 256 / V;     // threads per output in the final sum
    constexpr int S = 256 / G;     // partials each of those threads adds (= V)
    static_assert(V >= 4 && V <= 64 && (V & (V - 1)) == 0, "R*MT must be a power of two in [4,64]");
    __shared__ __attribute__((aligned(16))) int32_t red[4 * V * 64];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int M = p.M, N = p.N, K = p.K;
    const int n0 = blockIdx.x * R;
    const int8_t* A = static_cast<const int8_t*>(p.A);
    const int8_t* B = static_cast<const int8_t*>(p.B);

    const int cpw = K >> 6;  // 16-byte chunks per wave quarter (K % 64 == 0)
    const int c_begin = wave * cpw, c_end = c_begin + cpw;

    int32_t acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0;

    for (int c = c_begin + lane; c < c_end; c += 64) {
        v4i b[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(n0 + r, N - 1);  // rows past N repeat the last row; never stored
            b[r] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(B + static_cast<size_t>(n) * K) + c);
        }
        v4i a[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m)
            a[m] = (m < M) ? *(reinterpret_cast<const v4i*>(A + static_cast<size_t>(m) * K) + c)
                           : v4i{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[r][m] = dot16(a[m], b[r], acc[r][m]);
    }

    // red[(wave*V + v)*64 + lane]: conflict-free writes, contiguous reads.
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) red[(wave * V + r * MT + m) * 64 + lane] = acc[r][m];
    __syncthreads();

    // Output v = tid / G sums partials e in [part*S, part*S+S) of the 256
    // (wave, lane) partials; S divides 64, so a run stays inside one wave row.
    const int v = tid / G, part = tid % G;
    const int e0 = part * S;
    const int w = e0 >> 6, l0 = e0 & 63;
    const int32_t* src = red + (w * V + v) * 64 + l0;
    int32_t s = 0;
#pragma unroll
    for (int q = 0; q < S; q += 4) {
        const v4i x = *reinterpret_cast<const v4i*>(src + q);
        s += x[0] + x[1] + x[2] + x[3];
    }
    s = group_sum<G>(s);

    if (part == 0) {
        const int r = v / MT, m = v % MT;
        const int n = n0 + r;
        if (m < M && n < N) {
            const float sc = (p.scale_a ? p.scale_a[m] : p.sa) * (p.scale_b ? p.scale_b[n] : p.sb);
            store_out<OUT>(p.C, static_cast<size_t>(m) * N + n,
                           epilogue_value(static_cast<float>(s), sc, p.bias, n), s);
        }
    }
}


// Sum over all 64 lanes, result uniform: DPP quad swaps and row rotations inside
// each 16-lane row, a ds_swizzle across row pairs (lane ^ 16), then the two
// 32-lane halves through readlane.
__device__ __forceinline__ int32_t wave_sum(int32_t v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xF, 0xF, false);  // row_ror:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false);  // row_ror:8
    v += __builtin_amdgcn_ds_swizzle(v, 0x401F);                     // bit mode, xor 16
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 32);
}

// The same sum in fp32, in the same fixed order (FP8 row kernel).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // bit mode, xor 16
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

constexpr int ROWS_WAVES = 2;  // waves per workgroup of gemv_rows_kernel
// Weight rows per wave of the plain kernel.  One: at N = 14336, K = 4096 the
// launch is bounded by its ramp and drain, and 2 / 4 / 8 rows per wave
// (fewer, longer waves) measured 10.3 / 10.8 / 13.0 us against 9.8 us.
constexpr int ROWS_NB = 1;

// Wave w streams NB weight rows side by side: rows NB*w .. NB*w+NB-1 (plain),
// or gate row w and up row I + w (SWI: B is [gate; up], N = 2I rows, and the
// wave stores swiglu_pair of the two epilogue values).
// FULLK: K is a multiple of 4096, so every 256-chunk block is whole: the
// activation chunks come with plain loads and no offset needs the 2^31 guard.
// EL = ELEM_F8 (E4M3 codes, M = 1; plain GEMM, fp32 / bf16 out): each lane
// turns its codes into fp32 with v_cvt_pk_f32_fp8 and sums the exact products
// with fp32 FMAs in a fixed order (its chunks in order, then the wave sum), so
// the result is the same on every call.  Codes 0x7F / 0xFF are NaN to the
// conversion but 0.0 to the reference: the stream runs on the raw codes (no
// sum of finite E4M3 products overflows fp32, so a NaN total proves such a
// code in the row or in the activations) and a wave whose total comes out NaN
// streams its row again with those codes cleared.
// DW: 4-byte loads (K % 4 == 0, 4-byte-aligned operands: the shapes the
// 16-byte loads cannot take), 1024 words (4 KiB) of the row per block, 16 per
// lane, lane l taking words l, l + 64, ...; each word is all in K or all out.
template <int MT, int OUT, bool FULLK, int NB, bool SWI = false, int EL = ELEM_I8, bool DW = false>
__global__ __launch_bounds__(ROWS_WAVES * 64) void gemv_rows_kernel(GemmArgs p) {
    constexpr bool F8 = EL == ELEM_F8;
    static_assert(!DW || !FULLK, "4-byte loads: K is not a multiple of 4096 bytes of 16-byte chunks");
    static_assert(!SWI || NB == 2, "SwiGLU streams one gate and one up row");
    static_assert(MT * NB <= 64, "one storing lane per output");
    static_assert(!F8 || (!SWI && OUT != FKE_OUT_I32 && (DW || (MT == 1 && NB == 1))),
                  "FP8: fp32 or bf16 out; M = 1 with 16-byte loads");
    using Acc = typename std::conditional<F8, float, int32_t>::type;
    const int lane = threadIdx.x & 63;
    const int NO = SWI ? p.N >> 1 : p.N;           // output columns
    const int NU = SWI ? NO : (p.N + NB - 1) / NB;  // waves with work
    // Uniform per wave; readfirstlane keeps the rows' buffer resources in
    // SGPRs.  A wave past the last row re-reads it and stores nothing, so
    // nothing stands between the kernel arguments and the first weight load.
    const int nw = __builtin_amdgcn_readfirstlane(blockIdx.x * ROWS_WAVES + (threadIdx.x >> 6));
    const int n = min(nw, NU - 1);
    auto row_of = [&](int q) __attribute__((always_inline)) { return SWI ? n + q * NO : min(n * NB + q, p.N - 1); };
    const int M = p.M, K = p.K;
    const int ck = DW ? K >> 2 : K >> 4;  // 4-byte words / 16-byte chunks per row
    // B row n and the M activation rows through buffer resources: 32-bit
    // offsets, the weight stream non-temporal (read once, never re-used),
    // and chunks past the row end pointed at offset 2^31, which lies outside
    // every range and reads as zero - so the loop needs no guard.  Rows
    // m >= M of the MT-row template read row 0 (never stored).
    __amdgpu_buffer_rsrc_t rb[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q)
        rb[q] = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(static_cast<const int8_t*>(p.B) + static_cast<size_t>(row_of(q)) * K), 0, K,
            0x00020000);
    __amdgpu_buffer_rsrc_t ra[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
        ra[m] = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int8_t*>(static_cast<const int8_t*>(p.A) + static_cast<size_t>(m < M ? m : 0) * K), 0, K,
            0x00020000);
    // blocks of 4 KiB of the row (256 chunks, 1024 words), the last one partial; >= 1
    const int nblk = DW ? (ck + 1023) >> 10 : (ck + 255) >> 8;
    // per-row epilogue operands: scalar loads (n is uniform) whose latency
    // hides behind the weight stream
    float sbn[NB], biasn[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        sbn[q] = p.scale_b ? p.scale_b[row_of(q)] : p.sb;
        biasn[q] = p.bias ? p.bias[row_of(q)] : 0.0f;
    }
    // Activation scales too, before the stream: loaded after it, their
    // latency would sit between each wave's last sum and its store.  Rows
    // m >= M of the MT-row template read row 0 (never stored).
    float sam[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) sam[m] = p.scale_a ? p.scale_a[m < M ? m : 0] : p.sa;
    Acc acc[NB][MT];
    auto stream = [&](auto clear_c) __attribute__((always_inline)) {
    constexpr bool clear = decltype(clear_c)::value;
#pragma unroll
    for (int q = 0; q < NB; ++q)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[q][m] = Acc(0);
    int blk = 0;
    if constexpr (DW) {
    do {
        int off[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int c = (blk << 10) + lane + 64 * u;
            off[u] = c < ck ? c * 4 : static_cast<int>(0x80000000u);
        }
        int a[MT][16], b[NB][16];
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
            for (int u = 0; u < 16; ++u)
                b[q][u] = __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rb[q], off[u], 0, 2));
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int u = 0; u < 16; ++u)
                a[m][u] = __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(ra[m], off[u], 0, 0));
        if constexpr (F8) {
            // each output: the lane's words in order, the 4 products of a word in k order
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                float bf[NB][4];
#pragma unroll
                for (int q = 0; q < NB; ++q) {
                    uint32_t bw = static_cast<uint32_t>(b[q][u]);
                    if constexpr (clear) bw = e4m3_sanitize(bw);
                    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(bw), false);
                    const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(bw), true);
                    bf[q][0] = lo.x;
                    bf[q][1] = lo.y;
                    bf[q][2] = hi.x;
                    bf[q][3] = hi.y;
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    uint32_t aw = static_cast<uint32_t>(a[m][u]);
                    if constexpr (clear) aw = e4m3_sanitize(aw);
                    const v2f alo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(aw), false);
                    const v2f ahi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(aw), true);
#pragma unroll
                    for (int q = 0; q < NB; ++q) {
                        acc[q][m] = __builtin_fmaf(alo.x, bf[q][0], acc[q][m]);
                        acc[q][m] = __builtin_fmaf(alo.y, bf[q][1], acc[q][m]);
                        acc[q][m] = __builtin_fmaf(ahi.x, bf[q][2], acc[q][m]);
                        acc[q][m] = __builtin_fmaf(ahi.y, bf[q][3], acc[q][m]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < NB; ++q)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int u = 0; u < 16; ++u) acc[q][m] = __builtin_amdgcn_sdot4(a[m][u], b[q][u], acc[q][m], false);
        }
    } while (++blk < nblk);
    } else {
    do {
        int off[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = (blk << 8) + lane + 64 * u;
            off[u] = FULLK || c < ck ? c * 16 : static_cast<int>(0x80000000u);
        }
        v4i a[MT][4], b[NB][4];
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                b[q][u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb[q], off[u], 0, 2));
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if constexpr (FULLK) {
                    a[m][u] = *reinterpret_cast<const v4i*>(static_cast<const int8_t*>(p.A) +
                                                            static_cast<size_t>(m < M ? m : 0) * K + off[u]);
                } else {
                    a[m][u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra[m], off[u], 0, 0));
                }
            }
        if constexpr (F8) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                v4i ac = a[0][u], bc = b[0][u];
                if constexpr (clear) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ac[e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(ac[e])));
                        bc[e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(bc[e])));
                    }
                }
                float af[16], bf[16];
                e4m3_chunk_to_f32(ac, af);
                e4m3_chunk_to_f32(bc, bf);
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[0][0] = __builtin_fmaf(af[i], bf[i], acc[0][0]);
            }
        } else {
#pragma unroll
            for (int q = 0; q < NB; ++q)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int u = 0; u < 4; ++u) acc[q][m] = dot16(a[m][u], b[q][u], acc[q][m]);
        }
    } while (++blk < nblk);
    }
    };
    Acc tot[NB][MT];
    auto totals = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                if constexpr (F8) tot[q][m] = wave_sum_f32(acc[q][m]);
                else tot[q][m] = wave_sum(acc[q][m]);
            }
    };
    stream(std::false_type{});
    totals();
    if constexpr (F8) {
        bool nan = false;  // the totals are uniform over the wave, so is the replay
#pragma unroll
        for (int q = 0; q < NB; ++q)
#pragma unroll
            for (int m = 0; m < MT; ++m) nan |= tot[q][m] != tot[q][m];
        if (nan) {  // replay with the codes cleared
            stream(std::true_type{});
            totals();
        }
    }
    // All lanes hold every total.  SWI: lane m stores output (m, n); plain:
    // lane m*NB + q stores output (m, NB*n + q).
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float y[NB];
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const float sc = sam[m] * sbn[q];
            y[q] = p.bias ? __builtin_fmaf(static_cast<float>(tot[q][m]), sc, biasn[q])
                          : static_cast<float>(tot[q][m]) * sc;
        }
        int32_t ti[NB];
#pragma unroll
        for (int q = 0; q < NB; ++q) ti[q] = F8 ? 0 : static_cast<int32_t>(tot[q][m]);
        if constexpr (SWI) {
            if (lane == m && m < M && nw < NO)
                store_out<OUT>(p.C, static_cast<size_t>(m) * NO + n, swiglu_pair(y[0], y[1]), 0);
        } else {
#pragma unroll
            for (int q = 0; q < NB; ++q)
                if (lane == m * NB + q && m < M && nw < NU && n * NB + q < p.N)
                    store_out<OUT>(p.C, static_cast<size_t>(m) * p.N + n * NB + q, y[q], ti[q]);
        }
    }
}

// gemv_mfma_kernel (5 <= M <= 16): v_mfma_i32_16x16x64_i8 with the M
// activation rows padded to 16.  The sdot kernel above re-reads every
// activation chunk for each weight chunk it multiplies, which at M = 16
// moves 4x more bytes through the caches than the weights themselves; here
// one 16x16x64 MFMA consumes 64 k bytes of 16 weight rows against all 16
// activation rows, so activations cost one 16-byte load per 16-byte weight
// load per column block (halved with two blocks per wave).
// Workgroup = KS waves over CB*16 consecutive weight rows (output columns);
// wave w takes a contiguous 1/KS of the 64-byte k steps (split-K) and loads
// T steps at a time.  Operand layouts (16x16x64 i8): lane l supplies row
// l%16 (A) / column l%16 (B) with k bytes 16*(l/16)..+15 of the step; the
// result holds column l%16, rows 4*(l/16)+v.  Activation rows >= M and
// weight rows >= N are out of their buffers' ranges and read as zero.
// Partials are summed over the KS waves through LDS (exact int32).
constexpr int SK_CB = 2, SK_KS = 4, SK_T = 16;

// SWI: B is [gate; up] (N = 2I rows); column block 0 holds gate rows
// n0..n0+15 and block 1 the up rows I+n0.., and each output is swiglu_pair of
// the two epilogue values.
template <int OUT, bool SWI = false>
__global__ __launch_bounds__(SK_KS * 64) void gemv_mfma_kernel(GemmArgs p) {
    static_assert(!SWI || SK_CB == 2, "SwiGLU pairs one gate and one up block");
    __shared__ int32_t red[SK_KS][SK_CB * 256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int M = p.M, N = p.N, K = p.K;
    const int NO = SWI ? N >> 1 : N;                       // output columns
    const int n0 = blockIdx.x * (SWI ? 16 : SK_CB * 16);  // first output column
    const int steps = K >> 6, per = (steps + SK_KS - 1) / SK_KS;
    const int s0 = wave * per, s1 = min(s0 + per, steps);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.A), 0, M * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.B), 0, N * K, 0x00020000);
    const int r16 = lane & 15, kq = (lane >> 4) * 16;
    v4i acc[SK_CB];
#pragma unroll
    for (int c = 0; c < SK_CB; ++c) acc[c] = v4i{0, 0, 0, 0};
    for (int s = s0; s < s1; s += SK_T) {
        v4i a[SK_T], b[SK_CB][SK_T];
#pragma unroll
        for (int t = 0; t < SK_T; ++t) {
            const bool ok = s + t < s1;  // steps past this wave's range read as zero
            const int k = (s + t) * 64 + kq;
#pragma unroll
            for (int c = 0; c < SK_CB; ++c)
                b[c][t] = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(
                             rb, ok ? ((SWI ? c * NO : 16 * c) + n0 + r16) * K + k : int(0x80000000u), 0, 2));
            a[t] = __builtin_bit_cast(
                v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? r16 * K + k : int(0x80000000u), 0, 0));
        }
#pragma unroll
        for (int t = 0; t < SK_T; ++t)
#pragma unroll
            for (int c = 0; c < SK_CB; ++c) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], b[c][t], acc[c], 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < SK_CB; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[wave][c * 256 + (4 * (lane >> 4) + v) * 16 + r16] = acc[c][v];
    __syncthreads();
    if constexpr (SWI) {
        for (int o = tid; o < 256; o += SK_KS * 64) {
            int32_t sg = 0, su = 0;
#pragma unroll
            for (int w = 0; w < SK_KS; ++w) {
                sg += red[w][o];
                su += red[w][256 + o];
            }
            const int m = o >> 4, n = n0 + (o & 15);
            if (m < M && n < NO) {
                const float sam = p.scale_a ? p.scale_a[m] : p.sa;
                const float yg = epilogue_value(static_cast<float>(sg), sam * (p.scale_b ? p.scale_b[n] : p.sb),
                                                p.bias, n);
                const float yu = epilogue_value(static_cast<float>(su),
                                                sam * (p.scale_b ? p.scale_b[NO + n] : p.sb), p.bias, NO + n);
                store_out<OUT>(p.C, static_cast<size_t>(m) * NO + n, swiglu_pair(yg, yu), 0);
            }
        }
        return;
    }
    for (int o = tid; o < SK_CB * 256; o += SK_KS * 64) {
        int32_t sum = 0;
#pragma unroll
        for (int w = 0; w < SK_KS; ++w) sum += red[w][o];
        const int m = (o >> 4) & 15, n = n0 + 16 * (o >> 8) + (o & 15);
        if (m < M && n < N) {
            const float sc = (p.scale_a ? p.scale_a[m] : p.sa) * (p.scale_b ? p.scale_b[n] : p.sb);
            store_out<OUT>(p.C, static_cast<size_t>(m) * N + n, epilogue_value(static_cast<float>(sum), sc, p.bias, n),
                           sum);
        }
    }
}

// gemv_lds_kernel (M <= 64 per workgroup): the weight panel streamed through LDS.  One
// workgroup per CU owns an even share of R = ceil(NO / G) weight rows
// (output columns), so every CU reads the same number of bytes, and keeps
// its HBM reads in flight from its first instruction to its last.
// The K bytes are cut into pieces of PIECE bytes; wave w owns pieces w, w+4,
// ...  An item is 16 rows x PIECE bytes of one piece: the wave copies it into
// LDS with buffer_load_dwordx4 ... lds instructions of 1 KiB each (one or two
// rows' contiguous bytes), keeps NS items in flight in a ring of NS slots, and
// multiplies a landed item from LDS with PIECE/64 v_mfma_i32_16x16x64_i8
// against the piece's activation rows.  Those arrive the same way (MB items
// of 16 activation rows, read into registers once per piece and tile chunk;
// each weight fragment then feeds MB MFMAs).  Batches past 16*MB rows run
// as more workgroups along y, one 16*MB-row chunk of A each: their copies of
// a weight share find it in the last-level cache.
// The wave walks its pieces for LK_TMAX tiles at a time (a tile chunk),
// accumulating each tile; as soon as every wave has summed its share of a
// tile, the four partial sums meet in LDS and the tile's outputs are computed
// (exact int32 sums, so any split is bit-exact), while later tiles stream in;
// the outputs are stored at the end of the chunk.
// k order: a dot product is a sum, so the MFMA's k positions may map to any
// permutation of a piece's bytes as long as both operands use the same one.
// With S = PIECE/64 steps, step s of lane group g = l/16 takes 16-byte chunk
// S*g + s; LDS row i of an item holds chunk c at slot c ^ z(i), z(i) =
// (i / (1024/PIECE)) mod S, so the 64 lanes of every ds_read_b128 touch 64
// distinct 16-byte slots of a 1 KiB span.  Activation rows >= M, bytes >= K
// and tile rows past the workgroup's share read as zero (offset 2^31 is
// outside every range); weight bytes past K in the last piece meet zero
// activations.
// SWI: B is [gate; up]; tile t of a chunk is gate tile t/2 (t even) or the
// matching up tile (t odd), and each output is swiglu_pair of the two.
// EL = ELEM_F8 (E4M3 codes, fp32 sums): v_mfma_scale_f32_16x16x128_f8f6f4
// takes 32 k bytes per lane, so each MFMA pairs two of the 16-byte reads
// (chunks 2t and 2t+1 of the lane's step sequence; both operands pair the
// same chunks, so the k permutation argument holds).  Codes 0x7F / 0xFF are
// NaN to the MFMA but 0.0 to the reference (src/quantized_gemm.cu:90-91).
// The stream runs on the raw codes: E4M3 has no infinity, every product of
// finite codes is finite and no sum of them can overflow fp32, so a NaN sum
// proves a NaN code in its activation row or weight row.  A workgroup that
// saw one replays its whole stream once with every fragment cleared of the
// codes on the VALU after its LDS read (clean tiles give the same bits
// either way, so the replay simply overwrites).  Inputs holding such codes
// take about twice the time; clearing every fragment on every call instead
// cost ~20 % of the decode.  Weight
// bytes past K in the last piece read as zero (they would be the next
// row's codes).  The four waves' partial sums meet in the fixed order
// w = 0..3.
constexpr int LK_TMAX = 4;    // tiles accumulated between two reductions
constexpr int LK_RMAX = 512;  // weight rows (of each half) of one workgroup

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Position in a wave's item sequence: tile chunk tc (nt tiles), the wave's
// j-th piece, and u < 0 (activation rows 16*(u+MB).. of the piece) or tile u
// of the chunk.
struct LkPos {
    int tc, nt, j, u;
};

// s_waitcnt vmcnt(n) / lgkmcnt(n) for an n known after unrolling; the lgkm
// form is tied to the register it guards so the consumer cannot move above it.
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<8>(); break;
        case 2: wait_vm<16>(); break;
        case 3: wait_vm<24>(); break;
        default: wait_vm<32>(); break;
    }
}
__device__ __forceinline__ void wait_lgkm_tied(int n, v4i& r) {
    switch (n) {
        case 0: asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r)); break;
        case 1: asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(r)); break;
        case 2: asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(r)); break;
        case 3: asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(r)); break;
        case 4: asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(r)); break;
        case 5: asm volatile("s_waitcnt lgkmcnt(5)" : "+v"(r)); break;
        case 6: asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(r)); break;
        default: asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(r)); break;
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));

// WNT: each weight byte is read by this launch's one workgroup row only, so the
// weight copies are non-temporal; with more rows (batches past 64 rows) the
// later rows find the share in cache and the copies keep the default policy
// (N = 14336, K = 4096: M = 64 19.5 against 20.5 us non-temporal; M = 512 119
// against 130 us with the default policy).
template <int OUT, bool SWI, int PIECE, int NS, int MB, int EL = ELEM_I8, bool WNT = true>
__global__ __launch_bounds__(256) void gemv_lds_kernel(GemmArgs p) {
    constexpr int H = SWI ? 2 : 1;
    constexpr int RPW = 1024 / PIECE;  // rows per 1 KiB copy instruction
    constexpr int DI = 16 / RPW;       // copy instructions per item
    constexpr int S = PIECE / 64;      // MFMA steps per item
    constexpr int LA = S < 8 ? S : 8;  // fragment reads ahead of their MFMA
    static_assert(PIECE == 512 || PIECE == 1024, "piece of 512 or 1024 bytes");
    static_assert(DI == 8 || DI == 16, "vmcnt steps of wait_vm_n are 8 copies");
    static_assert((NS - 1) * DI <= 32, "wait_vm_n covers up to 32 copies");
    static_assert(MB >= 1 && MB <= 4, "up to 64 activation rows per workgroup (esa, one dword copy per lane)");
    static_assert(EL == ELEM_I8 || (EL == ELEM_F8 && !SWI && OUT != FKE_OUT_I32 && S % 2 == 0),
                  "FP8: plain GEMM, fp32 or bf16 out, pairs of 16-byte reads");
    constexpr bool F8 = EL == ELEM_F8;
    using AccV = typename std::conditional<F8, v4f, v4i>::type;
    // Partial sums of the tiles being finished: all tiles of a chunk for one
    // activation block (no barrier between two finishes), or with more blocks
    // only the tile (SWI: pair) at hand, which leaves the LDS to a deeper ring.
    constexpr int NQ = SWI ? 2 : 1;  // tiles finished together
    constexpr int RT = MB == 1 ? LK_TMAX : NQ;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[NS][4][16 * PIECE];
    __shared__ __attribute__((aligned(16))) int32_t red[RT][4][MB * 256];
    __shared__ __attribute__((aligned(16))) float esb[H * LK_RMAX], ebias[H * LK_RMAX], esa[64];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = p.K;
    const int mc = blockIdx.y * 16 * MB;  // first activation row of this workgroup
    const int M = min(16 * MB, p.M - mc);
    const int NO = SWI ? p.N >> 1 : p.N;  // output columns
    const int R = (NO + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    const int r0 = blockIdx.x * R;
    if (r0 >= NO) return;  // uniform over the workgroup
    const int nr = min(R, NO - r0);  // rows of each half
    const int th = (nr + 15) >> 4;   // 16-row tiles of each half
    const int T = H * th;
    const int TC = (T + LK_TMAX - 1) / LK_TMAX;
    const int P = (K + PIECE - 1) / PIECE;  // >= 4
    const int np = (P - 1 - wave) / 4 + 1;  // pieces of this wave, >= 1
    // The wave walks its pieces starting at a different one in each
    // workgroup, so the CUs' concurrent reads spread over the whole K span
    // of their rows rather than all reading the same byte range at once.
    const int jo = static_cast<int>(blockIdx.x) % np;

    // Epilogue operands (scale_b and bias of the workgroup's rows, scale_a of
    // the activation rows) go straight to LDS with dword LDS-DMA copies issued
    // by wave 0 before its stream.  No register then holds a value loaded
    // outside the main loop, which would make the compiler drain every copy in
    // flight before entering it; being older than every item's copies, they
    // have landed once the first item has.
    if (wave == 0) {
        const int nq = (nr + 63) >> 6;  // 64 rows per copy instruction
#pragma unroll
        for (int h = 0; h < H; ++h) {
            if (p.scale_b) {
                const __amdgpu_buffer_rsrc_t r = make_rsrc(p.scale_b + h * NO + r0, nr * 4);
                for (int q = 0; q < nq; ++q)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_u8*)(esb + h * LK_RMAX + 64 * q), 4,
                                                             256 * q + 4 * lane, 0, 0, 0);
            }
            if (p.bias) {
                const __amdgpu_buffer_rsrc_t r = make_rsrc(p.bias + h * NO + r0, nr * 4);
                for (int q = 0; q < nq; ++q)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_u8*)(ebias + h * LK_RMAX + 64 * q), 4,
                                                             256 * q + 4 * lane, 0, 0, 0);
            }
        }
        if (p.scale_a)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(p.scale_a + mc, M * 4), (lds_u8*)esa, 4, 4 * lane, 0,
                                                     0, 0);
    }

    const int8_t* B = static_cast<const int8_t*>(p.B);
    const __amdgpu_buffer_rsrc_t rb0 = make_rsrc(B + static_cast<size_t>(r0) * K, nr * K);
    const __amdgpu_buffer_rsrc_t rb1 = make_rsrc(B + static_cast<size_t>(SWI ? NO + r0 : r0) * K, nr * K);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(static_cast<const int8_t*>(p.A) + static_cast<size_t>(mc) * K, M * K);
    lds_u8* const lring = (lds_u8*)(&ring[0][wave][0]);  // slot q at + q * 4 * 16 * PIECE

    // copy lanes: lane l fills slot l % (64/RPW) of row d*RPW + l / (64/RPW)
    const int crow = lane / (64 / RPW), cslot = lane % (64 / RPW);
    auto z = [](int i) __attribute__((always_inline)) { return (i / RPW) & (S - 1); };
    auto issue = [&](const LkPos& it, lds_u8* dst) __attribute__((always_inline)) {
        const int jr = it.j + jo < np ? it.j + jo : it.j + jo - np;
        const int pc = (wave + 4 * jr) * PIECE;  // first k byte of the piece
        if (it.u < 0) {
            const int a0 = 16 * (it.u + MB);  // first activation row of the item
#pragma unroll
            for (int d = 0; d < DI; ++d) {
                const int i = d * RPW + crow;
                const int k = pc + ((cslot ^ z(i)) << 4);
                const uint32_t off = a0 + i < M && k < K ? static_cast<uint32_t>((a0 + i) * K + k) : 0x80000000u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst + d * 1024, 16, static_cast<int>(off), 0, 0, 0);
            }
        } else {
            const int t = it.tc * LK_TMAX + it.u;
            const int row0 = 16 * (SWI ? t >> 1 : t);
            const __amdgpu_buffer_rsrc_t rb = SWI && (t & 1) ? rb1 : rb0;
#pragma unroll
            for (int d = 0; d < DI; ++d) {
                const int i = d * RPW + crow, r = row0 + i;
                const int k = pc + ((cslot ^ z(i)) << 4);
                // FP8: bytes past K read as zero (the next row's codes may be NaN codes)
                const uint32_t off = r < nr && (!F8 || k < K) ? static_cast<uint32_t>(r * K + k) : 0x80000000u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, dst + d * 1024, 16, static_cast<int>(off), 0, 0,
                                                         WNT ? 2 : 0);
            }
        }
    };
    // advance to the next item; false past the last one
    auto advance = [&](LkPos& it) __attribute__((always_inline)) {
        if (++it.u < it.nt) return true;
        it.u = -MB;
        if (++it.j < np) return true;
        it.j = 0;
        ++it.tc;
        it.nt = min(LK_TMAX, T - it.tc * LK_TMAX);
        return it.tc < TC;
    };

    // lane l = 16g + i reads row i, chunk S*g + s at slot (S*g + s) ^ z(i)
    const int li = lane & 15;
    const uint32_t lb = static_cast<uint32_t>(li * PIECE + (lane >> 4) * (PIECE / 4) + z(li) * 16);
    v4i act[MB][S];
    AccV acc[LK_TMAX][MB];
#pragma unroll
    for (int q = 0; q < LK_TMAX; ++q)
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[q][b] = AccV{0, 0, 0, 0};

    // Fragment reads are inline ds_read_b128: the compiler does not know
    // which ring slot an LDS-DMA copy writes, and before any LDS read it can
    // see it would wait for every copy in flight (the next items' too).  Each
    // wait below is tied to the registers it guards; LDS operations complete
    // in order, so lgkmcnt(n) means all but the last n reads have landed.
    auto rd = [&](const lds_u8* src, int s) __attribute__((always_inline)) {
        v4i r;
        asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(src + (lb ^ (s << 4))));
        return r;
    };
    // An item's fragments go to registers first, so its slot can be refilled
    // before the MFMAs run (the slot's copy is then in flight during them).
    // At most LA reads are in flight (lgkmcnt's field is 4 bits).
    auto read_all = [&](const lds_u8* src, v4i (&f)[S]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < LA; ++s) f[s] = rd(src, s);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            wait_lgkm_tied(min(S, s + LA) - s - 1, f[s]);
            if (s + LA < S) f[s + LA] = rd(src, s + LA);
        }
    };
    auto mma = [&](AccV (&c)[MB], const v4i (&w)[S]) __attribute__((always_inline)) {
        if constexpr (F8) {
#pragma unroll
            for (int t = 0; t < S / 2; ++t) {
                const v8i wv = __builtin_shufflevector(w[2 * t], w[2 * t + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int b = 0; b < MB; ++b)
                    c[b] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        __builtin_shufflevector(act[b][2 * t], act[b][2 * t + 1], 0, 1, 2, 3, 4, 5, 6, 7), wv, c[b],
                        0, 0, 0, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int b = 0; b < MB; ++b)
                    c[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(act[b][s], w[s], c[b], 0, 0, 0);
        }
    };

    // Lane l of a wave holds tile column l%16, rows 4*(l/16)+v of an MFMA
    // tile.  The LDS accesses of the reduction are inline for the reason
    // given at the fragment reads.
    auto ld = [](const void* a) __attribute__((always_inline)) {
        int v;
        asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"((lds_u8*)(const_cast<void*>(a))));
        return v;
    };
    // Finishing tile u of chunk tc (SWI: the pair u-1, u): the waves' partial
    // sums go to red, and after a barrier thread (m, nl) = (tid/16, tid%16)
    // computes output column nl of activation rows m + 16b into yv[u][b] /
    // sv[u][b].  Called by every wave once
    // its share of the tile is summed, so a chunk's early tiles are reduced
    // while the later tiles' copies stream in; the stores wait for the end of
    // the chunk (8 % faster at M = 4 than one reduction at the chunk's end).
    int nan_seen = 0;  // FP8: a NaN sum in this thread's outputs (a 0x7F / 0xFF code took part)
    float yv[LK_TMAX][MB];
    int32_t sv[LK_TMAX][MB];
    auto finish_tile = [&](int tc, int u) __attribute__((always_inline)) {
        // red slot of tile u - NQ + 1 + q
        auto rs = [&](int q) __attribute__((always_inline)) { return RT == LK_TMAX ? u - NQ + 1 + q : q; };
        if constexpr (RT < LK_TMAX) barrier();  // the previous finish has read red
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                // The MFMA result passes through a VALU move first: the
                // compiler puts the wait states an MFMA result needs before a
                // VALU reads it, but not before an inline-asm store does.
                // (The whole accumulator is reinterpreted as integers first:
                // a bit cast of one vector element reads element 0.)
                const v4i ai = __builtin_bit_cast(v4i, acc[u - NQ + 1 + q][b]);
                v4i a;
#pragma unroll
                for (int e = 0; e < 4; ++e) a[e] = __builtin_amdgcn_update_dpp(0, ai[e], 0xE4, 0xF, 0xF, false);
                asm volatile("ds_write_b128 %0, %1"
                             :
                             : "v"((lds_u8*)&red[rs(q)][wave][b * 256 + lane * 4]), "v"(a)
                             : "memory");
            }
        wait_lgkm0();
        barrier();
        const int m = tid >> 4, nl = tid & 15;
        if (m >= M) return;
        const int ri = ((m >> 2) * 16 + nl) * 4 + (m & 3);
        const int t = tc * LK_TMAX + u;  // SWI: the up tile of the pair
        const int r = 16 * (SWI ? t >> 1 : t) + nl;
        int b0 = ld(esb + r), c0 = ld(ebias + r);
        int b1 = SWI ? ld(esb + LK_RMAX + r) : 0, c1 = SWI ? ld(ebias + LK_RMAX + r) : 0;
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b0), "+v"(c0), "+v"(b1), "+v"(c1));
        const float sb0 = p.scale_b ? __int_as_float(b0) : p.sb, sb1 = p.scale_b ? __int_as_float(b1) : p.sb;
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            if (b > 0 && m + 16 * b >= M) break;
            // at most 4 * NQ + 1 reads in flight (lgkmcnt's field is 4 bits)
            int x[4 * NQ];
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int w = 0; w < 4; ++w) x[4 * q + w] = ld(&red[rs(q)][w][b * 256 + ri]);
            int xa = ld(esa + m + 16 * b);
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(xa));
#pragma unroll
            for (int q = 0; q < 4 * NQ; ++q) asm volatile("" : "+v"(x[q]));
            const float sam = p.scale_a ? __int_as_float(xa) : p.sa;
            int32_t s0 = 0;
            float v0;
            if constexpr (F8) {
                v0 = ((__int_as_float(x[0]) + __int_as_float(x[1])) + __int_as_float(x[2])) + __int_as_float(x[3]);
                if (v0 != v0 && r < nr) nan_seen = 1;  // rows of the share only (padding rows are not stored)
            } else {
                s0 = x[0] + x[1] + x[2] + x[3];
                v0 = static_cast<float>(s0);
            }
            const float sc0 = sam * sb0;
            const float y0 = p.bias ? __builtin_fmaf(v0, sc0, __int_as_float(c0)) : v0 * sc0;
            if constexpr (SWI) {
                const int32_t s1 = x[4] + x[5] + x[6] + x[7];
                const float sc1 = sam * sb1;
                const float y1 = p.bias ? __builtin_fmaf(static_cast<float>(s1), sc1, __int_as_float(c1))
                                        : static_cast<float>(s1) * sc1;
                yv[u][b] = swiglu_pair(y0, y1);
            } else {
                yv[u][b] = y0;
                sv[u][b] = s0;
            }
        }
    };
    // The chunk's stores: thread (m, nl) holds output column nl of each tile
    // for activation rows m + 16b.
    auto store_chunk = [&](int tc, int nt) __attribute__((always_inline)) {
        const int m = tid >> 4, nl = tid & 15;
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            if (m + 16 * b >= M) break;
#pragma unroll
            for (int u = SWI ? 1 : 0; u < LK_TMAX; u += SWI ? 2 : 1) {
                const int t = tc * LK_TMAX + u;
                const int r = 16 * (SWI ? t >> 1 : t) + nl;
                if (u < nt && r < nr)
                    store_out<OUT>(p.C, static_cast<size_t>(mc + m + 16 * b) * NO + r0 + r, yv[u][b], sv[u][b]);
            }
        }
    };

    auto san = [](v4i (&f)[S]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < S; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) f[q][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(f[q][e])));
    };
    // The whole stream; with clear_c true (the FP8 replay) every fragment is
    // cleared of the codes after its LDS read.
    auto stream = [&](auto clear_c) __attribute__((always_inline)) {
    constexpr bool clear = decltype(clear_c)::value;
    // Prologue: the first NS items in flight.
    LkPos pi{0, min(LK_TMAX, T), 0, -MB};
    int issued = 0;
    bool more = true;
#pragma unroll
    for (int q = 0; q < NS; ++q)
        if (more) {
            issue(pi, lring + q * (4 * 16 * PIECE));
            ++issued;
            more = advance(pi);
        }

    // Consumer: the same item order as the producer, spelled out as loops so
    // that every register array is indexed by constants.  Item c sits in
    // slot c % NS; once its fragments are in registers, item c + NS goes there.
    int c = 0;
    auto next_slot = [&]() __attribute__((always_inline)) {
        lds_u8* const slot = lring + (c % NS) * (4 * 16 * PIECE);
        wait_vm_n((issued - c - 1) * DI / 8);  // all but the later items' copies have landed
        return slot;
    };
    auto refill = [&](lds_u8* slot) __attribute__((always_inline)) {
        if (more) {
            issue(pi, slot);
            ++issued;
            more = advance(pi);
        }
        ++c;
    };
    for (int tc = 0; tc < TC; ++tc) {
        const int nt = min(LK_TMAX, T - tc * LK_TMAX);
        for (int j = 0; j < np; ++j) {
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                lds_u8* const slot = next_slot();
                read_all(slot, act[b]);
                refill(slot);
                if constexpr (clear) san(act[b]);
            }
#pragma unroll
            for (int u = 0; u < LK_TMAX; ++u) {
                if (u < nt) {
                    lds_u8* const slot = next_slot();
                    v4i w[S];
                    read_all(slot, w);
                    refill(slot);
                    if constexpr (clear) san(w);
                    mma(acc[u], w);
                    if (j == np - 1 && (!SWI || (u & 1))) finish_tile(tc, u);
                }
            }
        }
        store_chunk(tc, nt);
#pragma unroll
        for (int q = 0; q < LK_TMAX; ++q)
#pragma unroll
            for (int b = 0; b < MB; ++b) acc[q][b] = AccV{0, 0, 0, 0};
        barrier();  // every read of red for this chunk precedes the next chunk's writes
    }
    };
    // Raw codes first; FP8 only: a workgroup with a NaN output replays the
    // stream with the codes cleared (no copy is in flight between the two).
    stream(std::false_type{});
    if constexpr (F8)
        if (__syncthreads_or(nan_seen)) stream(std::true_type{});
}

hipError_t launch_mfma_skinny(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const void* f;
    if (p.swiglu) {
        const dim3 grid((p.N / 2 + 15) / 16);
        f = p.out_dtype == FKE_OUT_F32 ? reinterpret_cast<const void*>(&gemv_mfma_kernel<FKE_OUT_F32, true>)
                                       : reinterpret_cast<const void*>(&gemv_mfma_kernel<FKE_OUT_BF16, true>);
        return hipLaunchKernel(f, grid, dim3(SK_KS * 64), args, 0, stream);
    }
    const dim3 grid((p.N + SK_CB * 16 - 1) / (SK_CB * 16));
    switch (p.out_dtype) {
        case FKE_OUT_F32: f = reinterpret_cast<const void*>(&gemv_mfma_kernel<FKE_OUT_F32>); break;
        case FKE_OUT_BF16: f = reinterpret_cast<const void*>(&gemv_mfma_kernel<FKE_OUT_BF16>); break;
        default: f = reinterpret_cast<const void*>(&gemv_mfma_kernel<FKE_OUT_I32>); break;
    }
    return hipLaunchKernel(f, grid, dim3(SK_KS * 64), args, 0, stream);
}

bool pieces_even(int K, int piece) { return ((K + piece - 1) / piece) % 4 == 0; }

// The device's CU count, cached per device (device_cus).
int cu_count() { return device_cus(); }

// Workgroups of gemv_lds_kernel: one per CU, fewer when the rows run out
// (at least 16 rows each), more when a share would exceed LK_RMAX rows.
// (64-bit arithmetic: N may be anything up to INT32_MAX here.)
int lds_grid(const GemmArgs& p) {
    const int64_t cus = cu_count();
    const int64_t no = p.swiglu ? p.N / 2 : p.N;
    int64_t g = std::min(cus, (no + 15) / 16);
    if ((no + g - 1) / g > LK_RMAX) g = (no + LK_RMAX - 1) / LK_RMAX;
    return static_cast<int>(g);
}

template <int PIECE>
bool lds_fits(const GemmArgs& p) {
    // offsets within one workgroup's activation rows (at most 64) and weight rows
    if (p.K < 4 * PIECE || static_cast<int64_t>(min(p.M, 64)) * p.K > INT32_MAX) return false;
    const int64_t no = p.swiglu ? p.N / 2 : p.N;
    const int64_t g = lds_grid(p);
    const int64_t r = (no + g - 1) / g;
    return r * p.K + PIECE <= INT32_MAX;
}

// The kernel of one instantiation: non-temporal weight copies unless several
// workgroup rows share the weights (only the 4-block batches have more than
// one row: M > 64).
template <int OUT, bool SWI, int PIECE, int NS, int MB, int EL>
const void* lds_kernel_for(int rows) {
    if constexpr (MB == 4)
        if (rows > 1) return reinterpret_cast<const void*>(&gemv_lds_kernel<OUT, SWI, PIECE, NS, MB, EL, false>);
    return reinterpret_cast<const void*>(&gemv_lds_kernel<OUT, SWI, PIECE, NS, MB, EL, true>);
}

// grid.y: one workgroup row per 16*MB activation rows; NSW: ring slots of
// the SwiGLU instantiation (its two-tile reduction buffer takes LDS)
template <int PIECE, int NS, int MB, int NSW = NS>
hipError_t launch_lds_t(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const int rows = (p.M + 16 * MB - 1) / (16 * MB);
    const void* f;
    if (p.swiglu) {
        f = p.out_dtype == FKE_OUT_F32 ? lds_kernel_for<FKE_OUT_F32, true, PIECE, NSW, MB, ELEM_I8>(rows)
                                       : lds_kernel_for<FKE_OUT_BF16, true, PIECE, NSW, MB, ELEM_I8>(rows);
    } else {
        switch (p.out_dtype) {
            case FKE_OUT_F32: f = lds_kernel_for<FKE_OUT_F32, false, PIECE, NS, MB, ELEM_I8>(rows); break;
            case FKE_OUT_BF16: f = lds_kernel_for<FKE_OUT_BF16, false, PIECE, NS, MB, ELEM_I8>(rows); break;
            default: f = lds_kernel_for<FKE_OUT_I32, false, PIECE, NS, MB, ELEM_I8>(rows); break;
        }
    }
    return hipLaunchKernel(f, dim3(lds_grid(p), rows), dim3(256), args, 0, stream);
}

template <int PIECE, int NS, int MB>
hipError_t launch_lds_f8(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const int rows = (p.M + 16 * MB - 1) / (16 * MB);
    const void* f = p.out_dtype == FKE_OUT_F32 ? lds_kernel_for<FKE_OUT_F32, false, PIECE, NS, MB, ELEM_F8>(rows)
                                               : lds_kernel_for<FKE_OUT_BF16, false, PIECE, NS, MB, ELEM_F8>(rows);
    return hipLaunchKernel(f, dim3(lds_grid(p), rows), dim3(256), args, 0, stream);
}

template <int MT, bool FULLK, int NB = ROWS_NB, bool DW = false>
hipError_t launch_rows(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const void* f;
    if (p.swiglu) {
        const dim3 grid((p.N / 2 + ROWS_WAVES - 1) / ROWS_WAVES);
        f = p.out_dtype == FKE_OUT_F32
            ? reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_F32, FULLK, 2, true, ELEM_I8, DW>)
            : reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_BF16, FULLK, 2, true, ELEM_I8, DW>);
        return hipLaunchKernel(f, grid, dim3(ROWS_WAVES * 64), args, 0, stream);
    }
    const int units = (p.N + NB - 1) / NB;
    const dim3 grid((units + ROWS_WAVES - 1) / ROWS_WAVES);
    switch (p.out_dtype) {
        case FKE_OUT_F32:
            f = reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_F32, FULLK, NB, false, ELEM_I8, DW>);
            break;
        case FKE_OUT_BF16:
            f = reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_BF16, FULLK, NB, false, ELEM_I8, DW>);
            break;
        default:
            f = reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_I32, FULLK, NB, false, ELEM_I8, DW>);
            break;
    }
    return hipLaunchKernel(f, grid, dim3(ROWS_WAVES * 64), args, 0, stream);
}

// FP8 with 4-byte loads, 2..4 rows: two weight rows per wave, as for INT8.
template <int MT>
hipError_t launch_rows_f8_dw(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const dim3 grid(((p.N + 1) / 2 + ROWS_WAVES - 1) / ROWS_WAVES);
    const void* f = p.out_dtype == FKE_OUT_F32
        ? reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_F32, false, 2, false, ELEM_F8, true>)
        : reinterpret_cast<const void*>(&gemv_rows_kernel<MT, FKE_OUT_BF16, false, 2, false, ELEM_F8, true>);
    return hipLaunchKernel(f, grid, dim3(ROWS_WAVES * 64), args, 0, stream);
}

// FP8 at M = 1: the row kernel on E4M3 codes (one weight row per wave).
template <bool FULLK, bool DW = false>
hipError_t launch_rows_f8(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const dim3 grid((p.N + ROWS_WAVES - 1) / ROWS_WAVES);
    const void* f = p.out_dtype == FKE_OUT_F32
        ? reinterpret_cast<const void*>(&gemv_rows_kernel<1, FKE_OUT_F32, FULLK, 1, false, ELEM_F8, DW>)
        : reinterpret_cast<const void*>(&gemv_rows_kernel<1, FKE_OUT_BF16, FULLK, 1, false, ELEM_F8, DW>);
    return hipLaunchKernel(f, grid, dim3(ROWS_WAVES * 64), args, 0, stream);
}

template <int MT, int R>
hipError_t launch_t(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const dim3 grid((p.N + R - 1) / R);
    const void* f;
    switch (p.out_dtype) {
        case FKE_OUT_F32: f = reinterpret_cast<const void*>(&gemv_i8_kernel<MT, R, FKE_OUT_F32>); break;
        case FKE_OUT_BF16: f = reinterpret_cast<const void*>(&gemv_i8_kernel<MT, R, FKE_OUT_BF16>); break;
        default: f = reinterpret_cast<const void*>(&gemv_i8_kernel<MT, R, FKE_OUT_I32>); break;
    }
    return hipLaunchKernel(f, grid, dim3(256), args, 0, stream);
}

// The skinny MFMA kernel addresses A and B with 32-bit buffer offsets,
// computed for up to 16 activation rows and 32 weight rows past N.
bool skinny_offsets_fit(const GemmArgs& p) {
    return (static_cast<int64_t>(p.N < 16 ? 16 : p.N) + 32) * p.K <= INT32_MAX;
}

// M = 2..4 (and SwiGLU up to 4): the row kernel with two weight rows per
// wave, which reuses each activation chunk for both rows; measured 4-8 %
// faster than the split-K kernel at N = 14336, K = 4096.
template <bool FULLK, bool DW = false>
hipError_t launch_rows_m(const GemmArgs& p, hipStream_t s) {
    if (p.M <= 1) return launch_rows<1, FULLK, ROWS_NB, DW>(p, s);
    if (p.M <= 2) return launch_rows<2, FULLK, 2, DW>(p, s);
    return launch_rows<4, FULLK, 2, DW>(p, s);
}

// The row kernel's 4-byte form: B [N,K], up to 4 rows, K % 4 == 0 and
// 4-byte-aligned A / B where the 16-byte loads cannot run (K % 64 != 0 or
// rows not 16-byte aligned).
bool rows_dw_ok(const GemmArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (p.M < 1 || p.M > 4 || p.N < 1 || p.K < 4 || p.K % 4 != 0 || p.b_layout != FKE_B_NK) return false;
    if ((a | b) & 3) return false;
    return !(p.K % 64 == 0 && ((a | b) & 15) == 0);
}

}  // namespace

// Batches of 17..FKE_GEMV_MAX_M rows: whether the LDS-streamed kernel beats
// the MFMA GEMM, from cost models fitted to measurements on MI355X (N of 4096
// and 14336, K of 4096 and 14336, M of 17..512):
//  * streamed, per 64-row chunk of A: c0 + cw us per KiB of the workgroup's
//    weight share + ca us per KiB of the chunk's activation rows (L2 hits),
//    with (c0, cw, ca) = (4.0, 0.046, 0.004) for two 16-row blocks and
//    (5.2, 0.056, 0.0078) for four (each fit within 1 % of its three shapes;
//    chunks after the first measured up to 8 % faster): the weight stream
//    slows as more MFMAs and activation items sit between its items; the
//    workgroup rows of the chunks share the CUs, so small N runs several
//    chunks at once (N = 1792, M = 128: one chunk's 9.1 us);
//  * MFMA GEMM: mfma_time_estimate_us, by the tile it would run.  Up to a
//    few hundred rows it runs a 4-stage ring tile, one per CU, whose time
//    hardly depends on M, while the streamed kernel adds a chunk per 64 rows:
//    at N = 14336, K = 4096 the streamed kernel keeps M <= 32 (14.6 against
//    16.2 us on the 64x64 ring) and the MFMA GEMM takes M = 48..64 (16.2
//    against 19.3) and M = 65..128 on the 128x64 ring (20.3 against 36.7).
bool gemv_i8_batch_pays(const GemmArgs& p) {
    // The row kernel's 4-byte form past one row loses to the MFMA GEMM where
    // that GEMM can run (K % 16 == 0): 14336 x 4112, M = 4, 19.9 against
    // 15.4 us (M = 1: 13.7 against 15.2).
    if (p.M > 1 && rows_dw_ok(p)) return false;
    if (p.M <= 16 || p.M > FKE_GEMV_MAX_M) return p.M <= 16;
    const double kib = p.K / 1024.0;
    const int64_t g = lds_grid(p), no = p.swiglu ? p.N / 2 : p.N;
    const double share = static_cast<double>((no + g - 1) / g) * (p.swiglu ? 2 : 1) * kib;
    const bool four = p.M > 32;
    double chunk = (four ? 5.2 : 4.0) + (four ? 0.056 : 0.046) * share + (four ? 0.0078 : 0.004) * min(p.M, 64) * kib;
    // Shares past LK_TMAX 16-row tiles take several tile chunks, and with four
    // blocks each further chunk streams the 64 activation rows again at a CU's
    // ~44 KiB/us (64x16896x4096: 28.0 us, 22 without this term; two blocks
    // showed no such cost: 32x20480x4096, 19.7 us against 19.2).
    const int64_t th = ((no + g - 1) / g + 15) / 16 * (p.swiglu ? 2 : 1);
    if (four) chunk += static_cast<double>((th + LK_TMAX - 1) / LK_TMAX - 1) * 64.0 * kib / 44.0;
    // one row of g workgroups per 64 rows; rows share the CUs (one workgroup each)
    const int64_t waves = ((p.M + 63) / 64 * g + cu_count() - 1) / cu_count();
    const double t_lds = waves * chunk;
    return t_lds < mfma_time_estimate_us(p, cu_count());
}

bool gemv_i8_supports(const GemmArgs& p) {
    if (rows_dw_ok(p)) return true;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (!(p.M >= 1 && p.M <= FKE_GEMV_MAX_M && p.N >= 1 && p.K >= 64 && p.K % 64 == 0 &&
          p.b_layout == FKE_B_NK && ((a | b) & 15) == 0))
        return false;
    // batches past 16 rows: the LDS-streamed kernel only (K >= 2 KiB)
    if (p.M > 16) return lds_fits<512>(p);
    // SwiGLU pairs: the row kernel up to M = 4, the LDS-streamed kernel from
    // M = 3 when K >= 4 KiB, the skinny MFMA kernel otherwise
    return !p.swiglu || p.M <= 4 || lds_fits<1024>(p) || skinny_offsets_fit(p);
}


// The VALU dot-product decode kernels alone, with no MFMA: the row kernel
// (v_dot4 + DPP / ds_swizzle wave reduction) for M <= 4 and the split-K sdot
// kernel (LDS + group reduction) for 5 <= M <= 16.  The dispatcher prefers the
// MFMA kernels from M = 3 by measurement; this family stays selectable
// (FKE_PATH_GEMV_DOT) to cross-check and to measure that choice.
bool gemv_dot_supports(const GemmArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (!(p.M >= 1 && p.M <= 16 && p.N >= 1 && p.K >= 64 && p.K % 64 == 0 && p.b_layout == FKE_B_NK &&
          ((a | b) & 15) == 0))
        return false;
    return !p.swiglu || p.M <= 4;
}

hipError_t launch_gemv_dot(const GemmArgs& p, hipStream_t s) {
    if (p.M <= 4) return p.K % 4096 == 0 ? launch_rows_m<true>(p, s) : launch_rows_m<false>(p, s);
    if (p.M <= 8) return launch_t<8, 8>(p, s);
    return launch_t<16, 4>(p, s);
}

hipError_t launch_gemv_i8(const GemmArgs& p, hipStream_t s) {
    if (rows_dw_ok(p)) return launch_rows_m<false, true>(p, s);
    // M >= 3 with K >= 4 KiB: the LDS-streamed kernel (11.4-11.8 us at
    // N = 14336, K = 4096 for every M in 3..16, against 12.5-18.1 us for the
    // row and skinny kernels; SwiGLU 20.3-20.9 us against 21.5-34.3 us).  At
    // M = 1, 2 the row kernel is faster (9.8 / 11.0 us against 11.6 us).
    // Two activation blocks: 1 KiB pieces unless that leaves the four waves
    // uneven piece counts and 512 bytes does not (the workgroup waits for its
    // slowest wave: at K = 14336, 1 KiB pieces go 4/4/3/3 and took 8 % longer
    // at M = 17..32; at K = 4096 they are 4-6 % faster than 512).  One block
    // keeps 1 KiB pieces (512 at K = 14336 measured within 3 % either way).
    if (p.M > 32) return launch_lds_t<512, 4, 4, 3>(p, s);
    if (p.M > 16) {
        const bool big = lds_fits<1024>(p) && (pieces_even(p.K, 1024) || !pieces_even(p.K, 512));
        return big ? launch_lds_t<1024, 2, 2>(p, s) : launch_lds_t<512, 4, 2>(p, s);
    }
    if (p.M >= 3 && lds_fits<1024>(p)) return launch_lds_t<1024, 2, 1>(p, s);
    if (p.swiglu) {
        if (p.M <= 4) return p.K % 4096 == 0 ? launch_rows_m<true>(p, s) : launch_rows_m<false>(p, s);
        return launch_mfma_skinny(p, s);
    }
    if (p.M <= 4) return p.K % 4096 == 0 ? launch_rows_m<true>(p, s) : launch_rows_m<false>(p, s);
    if (skinny_offsets_fit(p)) return launch_mfma_skinny(p, s);
    if (p.M <= 8) return launch_t<8, 8>(p, s);
    return launch_t<16, 4>(p, s);
}

// FP8 decode and batches (B [N,K]): the row kernel at M = 1 (N = 14336,
// K = 4096: 10.3-10.5 us against 11.7 us on the LDS-streamed kernel; 4096 x
// 14336: 10.8 against 12.7), the LDS-streamed kernel on E4M3 codes above.
bool gemv_f8_supports(const GemmArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (rows_dw_ok(p)) return !p.swiglu && (p.out_dtype == FKE_OUT_F32 || p.out_dtype == FKE_OUT_BF16);
    return p.M >= 1 && p.M <= FKE_GEMV_MAX_M && p.N >= 1 && p.K % 64 == 0 && p.b_layout == FKE_B_NK &&
           !p.swiglu && (p.out_dtype == FKE_OUT_F32 || p.out_dtype == FKE_OUT_BF16) && ((a | b) & 15) == 0 &&
           (p.M == 1 || lds_fits<512>(p));
}

hipError_t launch_gemv_f8(const GemmArgs& p, hipStream_t s) {
    if (rows_dw_ok(p))
        return p.M == 1 ? launch_rows_f8<false, true>(p, s)
                        : p.M == 2 ? launch_rows_f8_dw<2>(p, s) : launch_rows_f8_dw<4>(p, s);
    if (p.M == 1) return p.K % 4096 == 0 ? launch_rows_f8<true>(p, s) : launch_rows_f8<false>(p, s);
    const bool big = lds_fits<1024>(p) && (pieces_even(p.K, 1024) || !pieces_even(p.K, 512));
    if (p.M > 32) return launch_lds_f8<512, 4, 4>(p, s);
    if (p.M > 16) return big ? launch_lds_f8<1024, 2, 2>(p, s) : launch_lds_f8<512, 4, 2>(p, s);
    return lds_fits<1024>(p) ? launch_lds_f8<1024, 2, 1>(p, s) : launch_lds_f8<512, 4, 1>(p, s);
}

}  // namespace fke
