// gemv_kn.hip — decode path (M <= 16) for B stored [K,N]: the layout the
// reference's FP8 launcher reads (src/quantized_gemm.cu:113, B[k*N + col]) and
// its Python op multiplies (python/flash_engine/ops.py:185, A @ B with B
// [K,N]).  Same arithmetic as src/quantized_gemm.cu:15-54 (INT8: exact int32
// sums) and :99-118 (FP8: fp32 sums of exact products, codes 0x7F / 0xFF
// counted as 0.0), with the fused epilogue of fke_qgemm_i8 / fke_qgemm_f8.
//
// HBM-bound: the weight panel is streamed once.  In [K,N] order a weight row
// is one k and an output column is a byte column, so the k bytes an MFMA
// lane needs for one column are N bytes apart in memory.  The kernel copies
// the panel into LDS as it lies and lets the LDS transpose it:
// ds_read_b64_tr_b8 gives each lane 8 consecutive k bytes of one column.
//
//  * Workgroup = 64 consecutive columns (64-byte row segments of B) over the
//    whole K; 4 waves split K: wave w takes the 128-row pieces w, w+4, ...
//    Grid = ceil(N / 64) workgroups; the two 64-column halves of each
//    128-byte line go to workgroups on one XCD.
//  * Bound by its access pattern, not by consumption: the same copies with
//    nothing consumed take as long (17 us at N = 14336, K = 4096).  Each CU
//    streams strided row segments at a rate that grows with the segment
//    width (64 / 128 / 256 / 512 bytes: 12 / 31 / 43 / 53 GB/s per CU), so
//    only a K split across workgroups (wider segments and every CU busy)
//    reaches the row-contiguous rate: copies of 512-byte segments in 8 K
//    ranges ran 9.8 us.  That needs a cross-workgroup reduction of the
//    partial sums, which this entry point (no workspace) cannot hold.
//  * Item = one piece: 128 k rows x 64 bytes of B (8 KiB, eight 1-KiB
//    buffer_load_dwordx4 ... lds copies of 16 rows each, four lanes per row)
//    plus the matching 128 k bytes of the 16 activation rows (2 KiB, two
//    copies; rows >= M and bytes >= K read as zero).  Each wave keeps NS
//    items in flight in its own ring slots.
//  * A landed item is read with ds_read_b128 (activations, in MFMA operand
//    order) and ds_read_b64_tr_b8 (weights): within each 16-lane group, lane
//    8h+i receives byte i of the 8 bytes addressed by lanes 2b+h (b = 0..7)
//    as its byte b, so lanes 2b+h addressing row k0+b at column c0+8h hand
//    lane j column c0+j with its k bytes in order - the MFMA's B operand.
//    INT8: v_mfma_i32_16x16x64_i8, two k steps per item; FP8:
//    v_mfma_scale_f32_16x16x128_f8f6f4, one step, fragments cleared of the
//    0x7F / 0xFF codes on the VALU (the MFMA reads them as NaN).
//  * The four waves' partial sums meet in LDS in the fixed order w = 0..3
//    (exact for INT8, deterministic for FP8), then the workgroup applies the
//    epilogue and stores 64 consecutive columns per activation row.
//
// LDS layouts (16-byte chunks, swizzled so that the 16-lane groups of one
// read instruction touch distinct banks whether the LDS serves 128 or 256
// bytes per cycle):
//  * weights: item row r (64 bytes, four chunks) keeps logical chunk c at
//    physical chunk c ^ kn_swz(r);
//  * activations: row m (128 bytes, eight chunks) keeps chunk c at
//    c ^ (m & 7) ^ ((m >> 3) & 1).
// The reads are inline ds_read instructions with lgkmcnt waits tied to their
// registers: the compiler cannot tell which ring slot an LDS-DMA copy
// writes, and before an LDS read it can see it would wait for every copy in
// flight.
#include "fke_internal.h"

#include <type_traits>

namespace fke {
namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr int KN_W = 64;                 // columns (bytes of a B row) per workgroup
constexpr int KN_ROWS = 128;             // k rows per item
constexpr int KN_BI = KN_ROWS * KN_W;    // weight bytes per item (8 KiB)
constexpr int KN_AI = 16 * KN_ROWS;      // activation bytes per item (2 KiB)
constexpr int KN_ITEM = KN_BI + KN_AI;   // 10 KiB
constexpr int KN_DB = KN_BI / 1024;      // weight copies per item
constexpr int KN_DA = KN_AI / 1024;      // activation copies per item
constexpr int KN_DI = KN_DB + KN_DA;     // copies per item
constexpr int KN_NS = 3;                 // ring slots per wave (120 KiB of LDS per workgroup)

// Physical chunk offset of item row r: bijective on r bits 1..2 within each
// 8-row group (a 16-lane group reads 8 rows x 16 bytes = 128 bytes), and
// with bit 4 ^ bit 5 flipping it, rows of the two 16-lane groups of a half
// wave that share r mod 4 land in different chunks too.
__device__ __forceinline__ int kn_swz(int r) { return ((r >> 1) & 3) ^ ((((r >> 4) ^ (r >> 5)) & 1) * 3); }
__device__ __forceinline__ int kn_aswz(int m) { return (m & 7) ^ ((m >> 3) & 1); }

__device__ __forceinline__ v4i rd128(const lds_u8* a) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ v2i rdtr(const lds_u8* a) {
    v2i r;
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
// Every LDS read has landed; the registers they wrote are tied to the wait,
// so nothing reads (or copies) them before it.
template <int N>
__device__ __forceinline__ void lgkm_wait_all(v4i (&a)[2], v2i (&t)[N]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    asm volatile("" : "+v"(a[0]), "+v"(a[1]));
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(t[i]));
}

// s_waitcnt vmcnt(KN_DI * n): every copy but those of the n latest items has landed.
__device__ __forceinline__ void wait_items(int n) {
    static_assert(KN_DI == 10, "vmcnt steps below are 10 copies");
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<10>(); break;
        default: wait_vm<20>(); break;
    }
}

template <int EL, int OUT>
__global__ __launch_bounds__(256) void gemv_kn_kernel(GemmArgs p) {
    constexpr bool F8 = EL == ELEM_F8;
    static_assert(EL == ELEM_I8 || (F8 && OUT != FKE_OUT_I32), "FP8: fp32 or bf16 out");
    static_assert(KN_NS == 3, "wait_items covers up to two later items");
    using AccV = typename std::conditional<F8, v4f, v4i>::type;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[KN_NS][4][KN_ITEM];
    __shared__ __attribute__((aligned(16))) float esb[KN_W], ebias[KN_W], esa[64];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, N = p.N, K = p.K;
    // Column block of this workgroup.  Workgroups are dispatched round robin
    // over the 8 XCDs (b on XCD b % 8); blocks 2j and 2j+1, the two 64-byte
    // halves of every 128-byte line of their rows, go to workgroups b and
    // b + 8, which run at the same time on one XCD, so each line is fetched
    // into that XCD's L2 once and both halves are used (23 -> 17 us at
    // N = 14336, K = 4096; wider groups of blocks per XCD measured no better).
    int blk = blockIdx.x;
    const int G16 = static_cast<int>(gridDim.x) / 16 * 16;
    if (blk < G16) blk = ((blk / 16) * 8 + (blk % 8)) * 2 + ((blk / 8) % 2);
    const int n0 = blk * KN_W;
    const int P = (K + KN_ROWS - 1) / KN_ROWS;         // pieces along K
    const int np = wave < P ? (P - 1 - wave) / 4 + 1 : 0;  // pieces of this wave

    // Epilogue operands straight to LDS (dword LDS-DMA by wave 0 before its
    // stream; older than every item's copies, so landed with the first item).
    if (wave == 0) {
        const int nc = min(KN_W, N - n0);
        if (p.scale_b)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(p.scale_b + n0, nc * 4), (lds_u8*)esb, 4, 4 * lane, 0,
                                                     0, 0);
        if (p.bias)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(p.bias + n0, nc * 4), (lds_u8*)ebias, 4, 4 * lane, 0,
                                                     0, 0);
        if (p.scale_a)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(p.scale_a, M * 4), (lds_u8*)esa, 4, 4 * lane, 0, 0,
                                                     0);
    }

    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, K * N);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, M * K);
    lds_u8* const lring = (lds_u8*)(&ring[0][wave][0]);  // slot q at + q * 4 * KN_ITEM
    constexpr int SLOT = 4 * KN_ITEM;

    // Copy geometry (k-independent part of each lane's source offsets).
    // Weights, copy d: row i = 16d + l/4 of the item, physical chunk l%4
    // holding logical chunk (l%4) ^ kn_swz(i).  Activations, copy d: row
    // m = 8d + l/8, physical chunk l%8 holding logical chunk (l%8) ^ kn_aswz(m).
    uint32_t boff[KN_DB];
    int brow[KN_DB];
#pragma unroll
    for (int d = 0; d < KN_DB; ++d) {
        const int i = 16 * d + (lane >> 2);
        brow[d] = i;
        boff[d] = static_cast<uint32_t>(i * N + n0 + 16 * ((lane & 3) ^ kn_swz(i)));
    }
    uint32_t aoff[KN_DA];
    int akb[KN_DA];
    bool arow[KN_DA];
#pragma unroll
    for (int d = 0; d < KN_DA; ++d) {
        const int m = 8 * d + (lane >> 3);
        const int c = (lane & 7) ^ kn_aswz(m);
        arow[d] = m < M;
        akb[d] = 16 * c;
        aoff[d] = static_cast<uint32_t>(m * K + 16 * c);
    }
    auto issue = [&](int j, lds_u8* dst) __attribute__((always_inline)) {
        const int k0 = (wave + 4 * j) * KN_ROWS;
#pragma unroll
        for (int d = 0; d < KN_DB; ++d) {
            const uint32_t off = k0 + brow[d] < K ? boff[d] + static_cast<uint32_t>(k0 * N) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, dst + d * 1024, 16, static_cast<int>(off), 0, 0, 2);
        }
#pragma unroll
        for (int d = 0; d < KN_DA; ++d) {
            const uint32_t off = arow[d] && k0 + akb[d] < K ? aoff[d] + static_cast<uint32_t>(k0) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst + KN_BI + d * 1024, 16, static_cast<int>(off), 0, 0, 0);
        }
    };

    // Read geometry.  Lane l = 16G + a, a = 2b + h: weight reads address item
    // row R0 + b (R0 = 16G (INT8) / 32G (FP8) plus the read's step and
    // eighth) at column block cb's 8-byte half h.  For INT8 the swizzle of
    // those rows does not depend on the step or eighth (bits 3 and 6), so each
    // column block needs one address plus immediates; for FP8 the eighth t
    // flips bit 4 for t >= 2, which equals block cb ^ 3's address.
    const int G = lane >> 4, b8 = (lane & 15) >> 1, hh = lane & 1;
    uint32_t wadr[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int r = (F8 ? 32 : 16) * G + b8;
        wadr[cb] = static_cast<uint32_t>(r * KN_W + 16 * (cb ^ kn_swz(r)) + 8 * hh);
    }
    // Activation reads: row m = l % 16, logical chunk (INT8) 4s + G for step
    // s, (FP8) 2G + e for half e.
    const int am = lane & 15;
    uint32_t aadr[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int c = F8 ? 2 * G + e : 4 * e + G;
        aadr[e] = static_cast<uint32_t>(KN_BI + am * KN_ROWS + 16 * (c ^ kn_aswz(am)));
    }

    AccV acc[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[cb] = AccV{0, 0, 0, 0};

    int issued = 0;
#pragma unroll
    for (int q = 0; q < KN_NS; ++q)
        if (issued < np) {
            issue(issued, lring + q * SLOT);
            ++issued;
        }
    for (int c = 0; c < np; ++c) {
        lds_u8* const slot = lring + (c % KN_NS) * SLOT;
        wait_items(issued - c - 1);
        // Fragments to registers, then the slot is refilled before the MFMAs.
        // 18 reads: at most 12 in flight (lgkmcnt's field is 4 bits).
        v4i af[2];
        v2i tr[16];  // INT8: [2 steps][4 blocks][2 eighths]; FP8: [4 blocks][4 eighths]
        af[0] = rd128(slot + aadr[0]);
        af[1] = rd128(slot + aadr[1]);
#pragma unroll
        for (int x = 0; x < 16; ++x) {
            uint32_t a;
            if constexpr (F8) {
                const int cb = x >> 2, t = x & 3;  // eighth t of block cb: rows 32G + 8t ..
                a = (t >= 2 ? wadr[cb ^ 3] : wadr[cb]) + (8 * t) * KN_W;
            } else {
                const int s = x >> 3, cb = (x >> 1) & 3, t = x & 1;  // rows 64s + 16G + 8t ..
                a = wadr[cb] + (64 * s + 8 * t) * KN_W;
            }
            if (x + 2 >= 12) asm volatile("s_waitcnt lgkmcnt(11)" ::: "memory");
            tr[x] = rdtr(slot + a);
        }
        lgkm_wait_all(af, tr);
        v4i wf[8];  // INT8: [2 steps][4 blocks] of 16 k bytes; FP8: [4 blocks][2 halves] of 16 k bytes
#pragma unroll
        for (int x = 0; x < 8; ++x) wf[x] = v4i{tr[2 * x][0], tr[2 * x][1], tr[2 * x + 1][0], tr[2 * x + 1][1]};
        if (issued < np) {
            issue(issued, slot);
            ++issued;
        }
        if constexpr (F8) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e) af[h][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(af[h][e])));
#pragma unroll
            for (int x = 0; x < 8; ++x)
#pragma unroll
                for (int e = 0; e < 4; ++e) wf[x][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(wf[x][e])));
            const v8i a8 = __builtin_shufflevector(af[0], af[1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
                acc[cb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    a8, __builtin_shufflevector(wf[2 * cb], wf[2 * cb + 1], 0, 1, 2, 3, 4, 5, 6, 7), acc[cb], 0, 0,
                    0, 0, 0, 0);
        } else {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)
                    acc[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[s], wf[4 * s + cb], acc[cb], 0, 0, 0);
        }
    }

    // Cross-wave reduction through LDS (the ring is free: every wave has
    // consumed its items and no copy is in flight).  Lane l of block cb holds
    // column 16cb + l%16, rows 4(l/16) + v.
    __syncthreads();
    using AccE = typename std::conditional<F8, float, int32_t>::type;
    AccE* red = reinterpret_cast<AccE*>(&ring[0][0][0]);  // [4 waves][4 blocks][64 lanes][4]
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[((wave * 4 + cb) * 64 + lane) * 4 + v] = acc[cb][v];
    __syncthreads();
    const int n = tid & 63, cb = n >> 4, j = n & 15;
    const float sbn = p.scale_b ? esb[n] : p.sb;
    const float bn = ebias[n];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = (tid >> 6) + 4 * q;
        if (m >= M || n0 + n >= N) continue;
        const int idx = (16 * (m >> 2) + j) * 4 + (m & 3);
        AccE s = red[(0 * 4 + cb) * 256 + idx];
#pragma unroll
        for (int w = 1; w < 4; ++w) s += red[(w * 4 + cb) * 256 + idx];
        const float sam = p.scale_a ? esa[m] : p.sa;
        float y;
        if constexpr (F8) y = p.bias ? __builtin_fmaf(s, p.sa * p.sb, bn) : s * (p.sa * p.sb);
        else y = p.bias ? __builtin_fmaf(static_cast<float>(s), sam * sbn, bn) : static_cast<float>(s) * (sam * sbn);
        int32_t si = 0;
        if constexpr (!F8) si = s;
        store_out<OUT>(p.C, static_cast<size_t>(m) * N + n0 + n, y, si);
    }
}

template <int EL>
hipError_t launch_kn(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const void* f;
    switch (p.out_dtype) {
        case FKE_OUT_F32: f = reinterpret_cast<const void*>(&gemv_kn_kernel<EL, FKE_OUT_F32>); break;
        case FKE_OUT_BF16: f = reinterpret_cast<const void*>(&gemv_kn_kernel<EL, FKE_OUT_BF16>); break;
        default:
            if constexpr (EL == ELEM_I8) {
                f = reinterpret_cast<const void*>(&gemv_kn_kernel<ELEM_I8, FKE_OUT_I32>);
                break;
            }
            return hipErrorInvalidValue;
    }
    return hipLaunchKernel(f, dim3((p.N + KN_W - 1) / KN_W), dim3(256), args, 0, stream);
}

}  // namespace

bool gemv_kn_supports(const GemmArgs& p, int elem) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (p.b_layout != FKE_B_KN || p.swiglu || p.M < 1 || p.M > 16 || p.N < 1 || p.K < 64) return false;
    if (elem != ELEM_I8 && elem != ELEM_F8) return false;
    if (elem == ELEM_F8 && p.out_dtype == FKE_OUT_I32) return false;
    // 16-byte copies: row starts (B: k*N + n, A: m*K + k) must stay 16-byte aligned
    if (p.N % 16 != 0 || p.K % 64 != 0 || ((a | b) & 15) != 0) return false;
    // 32-bit buffer offsets and ranges over all of B and A
    return static_cast<int64_t>(p.K) * p.N <= INT32_MAX && static_cast<int64_t>(p.M) * p.K <= INT32_MAX;
}

hipError_t launch_gemv_kn(const GemmArgs& p, int elem, hipStream_t stream) {
    return elem == ELEM_F8 ? launch_kn<ELEM_F8>(p, stream) : launch_kn<ELEM_I8>(p, stream);
}

}  // namespace fke
