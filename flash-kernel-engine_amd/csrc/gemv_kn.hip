// gemv_kn.hip — decode path (M <= 16) for B stored [K,N]: the layout the
// reference's FP8 launcher reads (src/quantized_gemm.cu:113, B[k*N + col]) and
// its Python op multiplies (python/flash_engine/ops.py:185, A @ B with B
// [K,N]).  Same arithmetic as src/quantized_gemm.cu:15-54 (INT8: exact int32
// sums) and :99-118 (FP8: fp32 sums of exact products, codes 0x7F / 0xFF
// counted as 0.0), with the fused epilogue of fke_qgemm_i8 / fke_qgemm_f8.
//
// HBM-bound: the weight panel is streamed once.  In [K,N] order a weight row
// is one k and an output column is a byte column, so the k bytes an MFMA
// lane needs for one column are N bytes apart in memory.  The kernels copy
// the panel into LDS as it lies and let the LDS transpose it:
// ds_read_b64_tr_b8 gives each lane 8 consecutive k bytes of one column.
// INT8 runs v_mfma_i32_16x16x64_i8 (two k steps per 128-row item); FP8
// v_mfma_scale_f32_16x16x128_f8f6f4 (one step) on the raw codes, and a wave
// whose sums came out NaN (a 0x7F / 0xFF code, NaN to the MFMA, 0.0 to the
// reference) streams its pieces again with those codes cleared on the VALU.
//
// A CU streams strided row segments at a rate that grows with the segment
// width, and the chip needs most CUs streaming, so the panel is cut along K
// as well as N when a workspace holds the partial sums:
//
//  * Split kernel (gemv_kn_split_kernel + kn_reduce_kernel).  Workgroup =
//    KW = 1, 2 or 4 waves of 128 consecutive columns each x one of S K ranges
//    (grid ceil(N/(128 KW)) x S, S <= 8; at N = 14336, K = 4096 two waves and
//    S = 4: 224 workgroups); wave w streams the 128-column block
//    KW*blockIdx/S + w over the range, so the workgroup reads 128 KW
//    contiguous bytes of every row it touches.  Each wave writes its block's
//    partial sums ([M][128], int32 / fp32) to the workspace; a second kernel
//    adds the S partials of each output in the fixed order s = 0..S-1 (exact
//    for INT8, deterministic for FP8) and applies the epilogue.  Summing in
//    the same kernel (the last split to arrive, counted by an atomic) cost
//    ~8 us more at that shape: its store / count / load round trips queue
//    behind the other workgroups' streams, where the second kernel's run
//    after them (13.2 against 19 us for M = 1).
//  * Row kernel (gemv_kn_row_kernel + kn_reduce_kernel), M = 1, and up to 32
//    rows with operands the 16-byte loads cannot take: workgroup = 1024
//    consecutive columns x one of S <= 64 K ranges x 1, 2 or 4 activation
//    rows, loaded straight into registers and summed on the VALU (no MFMA, no
//    LDS staging); its partial sums take the split kernel's layout and second
//    kernel.
//  * Full kernel (gemv_kn_full_kernel), when there is no workspace or K is
//    too short to split: one workgroup per 64-column block over all of K,
//    blocks 2j and 2j+1 (the two halves of each 128-byte line) on one XCD.
//
// Item = 128 k rows x the block's bytes of B plus the matching 128 k bytes
// of the 16 activation rows (rows >= M and bytes >= K read as zero), copied
// by buffer_load_dwordx4 ... lds; each wave keeps its items in flight in its
// own ring slots.  The reads are inline ds_read instructions with lgkmcnt
// waits tied to their registers: the compiler cannot tell which ring slot an
// LDS-DMA copy writes, and before an LDS read it can see it would wait for
// every copy in flight.
#include "fke_internal.h"

#include <type_traits>

namespace fke {
namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// ===========================================================================
// Split kernel: 128 columns per wave, four waves (512 columns) per workgroup.
// ===========================================================================
constexpr int KS_W = 128;                // columns (bytes of a B row) per wave
constexpr int KS_CB = KS_W / 16;         // 16-column MFMA blocks per wave
constexpr int KS_ROWS = 128;             // k rows per item
constexpr int KS_BI = KS_ROWS * KS_W;    // weight bytes per item (16 KiB)
constexpr int KS_AI = 16 * KS_ROWS;      // activation bytes per item and 16-row block (2 KiB)
constexpr int KS_DB = KS_BI / 1024;      // weight copies per item
constexpr int KS_DA = KS_AI / 1024;      // activation copies per item and block
constexpr int KS_NS = 2;                 // ring slots per wave (144 KiB of LDS per workgroup)
constexpr int KS_SMAX = 8;               // K splits at most
constexpr int KN_MAX_M = 32;             // rows at most (two 16-row activation blocks)

// LDS layouts (16-byte chunks, swizzled so that every 16-lane group of a read
// touches 32 distinct banks and every 32-lane half 64, whether the LDS serves
// 128 or 256 bytes per cycle):
//  * weights: item row r (128 bytes, eight chunks) keeps logical chunk c at
//    physical chunk c ^ ks_swz(r): bits 0..2 of r spread the eight rows a
//    16-lane group reads over eight chunks; bits 4 and 5 flip it between the
//    two 16-lane groups of a half wave (rows 16 apart for INT8, 32 apart for
//    FP8), whose rows share bit 0 and would otherwise meet mod 256 bytes;
//  * activations: row m (128 bytes) keeps chunk c at c ^ ks_aswz(m).
__device__ __forceinline__ int ks_swz(int r) { return (r & 7) ^ ((r >> 4) & 1) ^ ((r >> 5) & 1); }
__device__ __forceinline__ int ks_aswz(int m) { return (m & 7) ^ ((m >> 3) & 1); }

__device__ __forceinline__ v4i ks_rd128(const lds_u8* a) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
template <int OFF>
__device__ __forceinline__ v2i ks_rdtr(const lds_u8* a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
    v2i r;
    asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF));
    return r;
}
// Every LDS read has landed; the registers they wrote are tied to the wait,
// so nothing reads (or copies) them before it.
template <int MB>
__device__ __forceinline__ void ks_lgkm_wait_all(v4i (&a)[MB][2], v2i (&t)[32]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int b = 0; b < MB; ++b) asm volatile("" : "+v"(a[b][0]), "+v"(a[b][1]));
#pragma unroll
    for (int i = 0; i < 32; ++i) asm volatile("" : "+v"(t[i]));
}
// s_waitcnt vmcnt(DI * n) for DI copies per item: every copy but those of
// the n latest items has landed.
template <int DI>
__device__ __forceinline__ void ks_wait_items(int n) {
    static_assert(KS_NS == 2, "at most one later item");
    if (n == 0) wait_vm<0>();
    else wait_vm<DI>();
}

// Weight read of item fragment X (compile-time), at an immediate offset from
// the lane's column-block address wadr[]:
//  INT8: X = 16s + 2cb + t -> rows 64s + 16G + 8t + b of block cb;
//  FP8:  X = 4cb + t       -> rows 32G + 8t + b of block cb (the swizzle
//        flips bit 0 of the chunk for t >= 2, i.e. block cb ^ 1's address).
// At most 14 LDS reads are in flight when one is issued (lgkmcnt is 4 bits;
// the NA activation reads come first).
template <bool F8, int NA, int X>
__device__ __forceinline__ void ks_read_w(const lds_u8* slot, const uint32_t (&wadr)[KS_CB], v2i (&tr)[32]) {
    static_assert(NA <= 13, "the activation reads leave room for the weight reads");
    if constexpr (X < 32) {
        if constexpr (X + NA >= 14) asm volatile("s_waitcnt lgkmcnt(13)" ::: "memory");
        if constexpr (F8) {
            constexpr int cb = X >> 2, t = X & 3;
            tr[X] = ks_rdtr<8 * t * KS_W>(slot + wadr[t >= 2 ? (cb ^ 1) : cb]);
        } else {
            constexpr int s = X >> 4, cb = (X >> 1) & 7, t = X & 1;
            tr[X] = ks_rdtr<(64 * s + 8 * t) * KS_W>(slot + wadr[cb]);
        }
        ks_read_w<F8, NA, X + 1>(slot, wadr, tr);
    }
}

// Wave w of workgroup b streams column block KW*(b/S) + w (128 columns) over
// the 128-row pieces [s*PS, min(P, (s+1)*PS)) of split s = b % S and writes
// its sums to part[block][s][m][column] for m < M.
// NT: the weight copies are non-temporal.  At N = 14336, K = 4096 that is
// 13.0 against 14.9 us at M = 1 and still ahead at M = 12 (16.8 / 17.0), but
// behind from M = 14 (M = 16: 17.9 against 17.4 with the default policy).
constexpr int KS_NT_MAX_M = 12;
template <int EL, bool NT, int KW, int MB>
__global__ __launch_bounds__(KW * 64) void gemv_kn_split_kernel(GemmArgs p, KnSplit sp) {
    constexpr bool F8 = EL == ELEM_F8;
    constexpr int ITEM = KS_BI + MB * KS_AI;  // bytes per item: weights, then MB activation blocks
    constexpr int DA = MB * KS_DA;            // activation copies per item
    constexpr int DI = KS_DB + DA;            // copies per item
    static_assert(KS_NS * KW * ITEM <= 160 * 1024, "the ring fits the LDS");
    using AccV = typename std::conditional<F8, v4f, v4i>::type;
    using AccE = typename std::conditional<F8, float, int32_t>::type;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[KS_NS][KW][ITEM];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int M = p.M, N = p.N, K = p.K;
    const int S = sp.S;
    const int split = static_cast<int>(blockIdx.x) % S;
    const int cbg = KW * (static_cast<int>(blockIdx.x) / S) + wave;  // this wave's column block
    const int n0 = cbg * KS_W;
    if (n0 >= N) return;  // no barrier below: the other waves go on alone
    const int P = (K + KS_ROWS - 1) / KS_ROWS;
    const int pb = split * sp.PS, np = min(P, pb + sp.PS) - pb;

    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, K * N);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, M * K);
    lds_u8* const lring = (lds_u8*)(&ring[0][wave][0]);  // slot q at + q * SLOT
    constexpr int SLOT = KW * ITEM;

    // Copy geometry.  Weights, copy d: item row i = 8d + l/8 at physical
    // chunk l%8, holding logical chunk (l%8) ^ ks_swz(i); ks_swz(i) is
    // (l/8) ^ f(d) with f(d) = bit 1 ^ bit 2 of d, so two lane offsets serve
    // all sixteen copies.  Activations, copy d: row m = 8d + l/8, physical
    // chunk l%8 holding logical chunk (l%8) ^ ks_aswz(m).
    const int lr = lane >> 3, lc = lane & 7;
    const uint32_t bbase0 = static_cast<uint32_t>(lr * N + n0 + 16 * (lc ^ lr));
    const uint32_t bbase1 = static_cast<uint32_t>(lr * N + n0 + 16 * (lc ^ lr ^ 1));
    uint32_t aoff[DA];
    int akb[DA];
    bool arow[DA];
#pragma unroll
    for (int d = 0; d < DA; ++d) {
        const int m = 8 * d + lr;
        const int c = lc ^ ks_aswz(m);
        arow[d] = m < M;
        akb[d] = 16 * c;
        aoff[d] = static_cast<uint32_t>(m * K + 16 * c);
    }
    auto issue = [&](int j, lds_u8* dst) __attribute__((always_inline)) {
        const int k0 = (pb + j) * KS_ROWS;
#pragma unroll
        for (int d = 0; d < KS_DB; ++d) {
            const uint32_t base = (((d >> 1) ^ (d >> 2)) & 1) ? bbase1 : bbase0;
            const uint32_t off = k0 + 8 * d < K ? base + static_cast<uint32_t>((k0 + 8 * d) * N) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, dst + d * 1024, 16, static_cast<int>(off), 0, 0, NT ? 2 : 0);
        }
#pragma unroll
        for (int d = 0; d < DA; ++d) {
            const uint32_t off = arow[d] && k0 + akb[d] < K ? aoff[d] + static_cast<uint32_t>(k0) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst + KS_BI + d * 1024, 16, static_cast<int>(off), 0, 0, 0);
        }
    };

    // Read geometry.  Lane l = 16G + 2b + h addresses item row R0 + b at
    // column block cb's 8-byte half h; R0 = 16G (INT8) / 32G (FP8) plus the
    // read's immediate rows, which leave the row's swizzle unchanged.
    // Activation reads: row m = l % 16, logical chunk (INT8) 4s + G for step
    // s, (FP8) 2G + e for half e.
    const int G = lane >> 4, b8 = (lane & 15) >> 1, hh = lane & 1;
    uint32_t wadr[KS_CB];
#pragma unroll
    for (int cb = 0; cb < KS_CB; ++cb) {
        const int r = (F8 ? 32 : 16) * G + b8;
        wadr[cb] = static_cast<uint32_t>(r * KS_W + 16 * (cb ^ ks_swz(r)) + 8 * hh);
    }
    const int am = lane & 15;
    uint32_t aadr[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int c = F8 ? 2 * G + e : 4 * e + G;
        aadr[e] = static_cast<uint32_t>(KS_BI + am * KS_ROWS + 16 * (c ^ ks_aswz(am)));
    }

    AccV acc[MB][KS_CB];
    // The stream on raw codes (SAN false), or with FP8's 0x7F / 0xFF codes
    // cleared on the VALU (SAN true, FP8's replay).
    auto stream = [&](auto sanc) __attribute__((always_inline)) {
        constexpr bool SAN = decltype(sanc)::value;
        (void)SAN;
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int cb = 0; cb < KS_CB; ++cb) acc[b][cb] = AccV{0, 0, 0, 0};

        int issued = 0;
#pragma unroll
        for (int q = 0; q < KS_NS; ++q)
            if (issued < np) {
                issue(issued, lring + q * SLOT);
                ++issued;
            }
        for (int c = 0; c < np; ++c) {
            lds_u8* const slot = lring + (c % KS_NS) * SLOT;
            ks_wait_items<DI>(issued - c - 1);
            // Fragments to registers, then the slot is refilled before the MFMAs.
            v4i af[MB][2];
            v2i tr[32];
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                af[b][0] = ks_rd128(slot + aadr[0] + b * KS_AI);
                af[b][1] = ks_rd128(slot + aadr[1] + b * KS_AI);
            }
            ks_read_w<F8, 2 * MB, 0>(slot, wadr, tr);
            ks_lgkm_wait_all<MB>(af, tr);
            v4i wf[16];  // INT8: [2 steps][8 blocks] of 16 k bytes; FP8: [8 blocks][2 halves] of 16 k bytes
#pragma unroll
            for (int x = 0; x < 16; ++x) wf[x] = v4i{tr[2 * x][0], tr[2 * x][1], tr[2 * x + 1][0], tr[2 * x + 1][1]};
            if (issued < np) {
                issue(issued, slot);
                ++issued;
            }
            if constexpr (F8) {
                if constexpr (SAN) {
#pragma unroll
                    for (int b = 0; b < MB; ++b)
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                af[b][h][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(af[b][h][e])));
#pragma unroll
                    for (int x = 0; x < 16; ++x)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            wf[x][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(wf[x][e])));
                }
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    const v8i a8 = __builtin_shufflevector(af[b][0], af[b][1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                    for (int cb = 0; cb < KS_CB; ++cb)
                        acc[b][cb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            a8, __builtin_shufflevector(wf[2 * cb], wf[2 * cb + 1], 0, 1, 2, 3, 4, 5, 6, 7), acc[b][cb],
                            0, 0, 0, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int b = 0; b < MB; ++b)
#pragma unroll
                        for (int cb = 0; cb < KS_CB; ++cb)
                            acc[b][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[b][s], wf[8 * s + cb], acc[b][cb], 0,
                                                                               0, 0);
            }
        }
    };
    if constexpr (!F8) {
        stream(std::false_type{});
    } else {
        // E4M3 0x7F / 0xFF are NaN to the MFMA but 0.0 to the reference.
        // Real quantizers never emit them (they saturate at 448), and
        // clearing every fragment costs VALU work the stream cannot hide, so
        // the wave streams the raw codes first: every product of finite codes
        // is finite and no sum of them overflows, so a NaN sum proves a NaN
        // code in this wave's rows or columns, and only then does the wave
        // stream its pieces again with the codes cleared.  Its ring slots are
        // free (the stream ends with every copy landed) and the other waves
        // are not waited for, so the replay is the wave's own.
        stream(std::false_type{});
        bool bad = false;
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int cb = 0; cb < KS_CB; ++cb)
#pragma unroll
                for (int v = 0; v < 4; ++v) bad |= __builtin_isnan(acc[b][cb][v]);
        if (__builtin_amdgcn_ballot_w64(bad) != 0) stream(std::true_type{});
    }

    // Lane l of activation block b and column block cb holds column
    // 16cb + l%16, rows 16b + 4(l/16) + v.
    AccE* const part = static_cast<AccE*>(sp.part) + (static_cast<size_t>(cbg) * S + split) * M * KS_W;
    const int j = lane & 15;
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        const int mb = 16 * b + 4 * G;
#pragma unroll
        for (int cb = 0; cb < KS_CB; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (mb + v < M) part[(mb + v) * KS_W + 16 * cb + j] = acc[b][cb][v];
    }
}

// One thread per output (m, n): the S partials in split order, then the
// epilogue.  The kernel is latency-bound (every load is in flight at once):
// workgroups of 256 threads, or of 64 while that would leave CUs without one
// (M = 1: 224 workgroups).  Same box, N = 14336, K = 4096, bf16: M = 16
// 16.7 us for the call against 17.5 with four outputs per thread (16-byte
// loads, one 8-byte store) in 64-thread groups and 17.6 in 256-thread groups;
// M = 1 12.9 us with 64-thread groups, 13.0 with 256.
template <int EL, int OUT, int T, int SM>
__global__ __launch_bounds__(T) void kn_reduce_kernel(GemmArgs p, KnSplit sp) {
    constexpr bool F8 = EL == ELEM_F8;
    using AccE = typename std::conditional<F8, float, int32_t>::type;
    const int N = p.N, S = sp.S;
    const int m = blockIdx.y, n = blockIdx.x * T + threadIdx.x;  // grid: column blocks x M
    if (n >= N) return;
    const AccE* part = static_cast<const AccE*>(sp.part) + static_cast<size_t>(n / KS_W) * S * p.M * KS_W +
                       static_cast<size_t>(m) * KS_W + (n % KS_W);
    AccE v[SM];
#pragma unroll
    for (int t = 0; t < SM; ++t) v[t] = t < S ? part[static_cast<size_t>(t) * p.M * KS_W] : AccE(0);
    AccE s = v[0];
#pragma unroll
    for (int t = 1; t < SM; ++t)
        if (t < S) s += v[t];
    float y;
    int32_t si = 0;
    if constexpr (F8) {
        const float sab = p.sa * p.sb;
        y = p.bias ? __builtin_fmaf(s, sab, p.bias[n]) : s * sab;
    } else {
        si = s;
        const float sc = (p.scale_a ? p.scale_a[m] : p.sa) * (p.scale_b ? p.scale_b[n] : p.sb);
        y = p.bias ? __builtin_fmaf(static_cast<float>(s), sc, p.bias[n]) : static_cast<float>(s) * sc;
    }
    store_out<OUT>(p.C, static_cast<size_t>(m) * N + n, y, si);
}

// ===========================================================================
// Row kernel (M = 1; and 2..32 rows where the 16-byte loads cannot run):
// 1024 columns per workgroup, loaded from HBM straight into registers; no LDS
// staging and no MFMA.
// ===========================================================================
// One activation row leaves an MFMA nothing to share between its 16 rows, and
// the transposing LDS reads serve only to turn k rows into columns.  Here lane
// l loads bytes 16l..16l+15 (16 columns) of a 1 KiB row segment, one load
// instruction per k row; the workgroup's waves read the 128 consecutive rows
// of a piece over the same 1024 columns, a few rows per wave at a time (a
// batch).  A lane turns each 4 rows x 4 columns of a batch into four words of
// 4 k bytes (a byte transpose in eight v_perm_b32) and sums them with
// v_dot4_i32_i8 against the activation word of those 4 rows (INT8), or
// converts the codes with v_cvt_pk_f32_fp8 and adds the exact products with
// fma in k order (FP8), for each of the workgroup's activation rows.  The
// waves' sums meet in LDS in the order w = 0, 1, ... and go to the workspace
// in the split kernel's layout ([block of 128 columns][split][M][128]);
// kn_reduce_kernel finishes them.  More than four activation rows take
// workgroups of four rows each (grid y), each streaming the same weights.
// Why: 1024-column blocks take up to 64 K splits, where the split kernel's
// 512-column blocks take 8, so shapes with few column blocks still fill the
// CUs (N = 4096, K = 14336: 224 workgroups and 13.5 against 23.2 us); at
// N = 14336, K = 4096 both take 224 workgroups and the same time (12.9 us),
// although a plain read of this kernel's pattern is 1 us faster than of the
// split kernel's (10.3 against 11.3 us, back-to-back launches).
// Layout (N = 14336 / 4096 x K = 4096 / 14336, INT8 and FP8, one box, same
// A/B): 16 waves x 4-row batches x 2 in flight; 8 waves x 4 or 8 rows x 2,
// and 4 waves x 8 rows x 2, within 0.1 us of it; 16-row batches 0.8 us
// slower, three or four in flight 0.1-1.1 us slower: every load of a wave is
// issued early, so the arithmetic of its last batch runs after the stream,
// and short batches keep that tail short.
constexpr int KR_W = 1024;   // columns per workgroup
constexpr int KR_SMAX = 64;  // K splits at most
constexpr int KR_ROWS = 4;   // rows per wave per batch
constexpr int KR_D = 2;      // batches in flight per wave
static_assert(KR_ROWS == 4 || KR_ROWS == 8 || KR_ROWS == 16, "4, 8 or 16 activation bytes per batch");
static_assert(KR_D >= 2 && KR_D <= 4, "two to four batches in flight");
static_assert(KR_W % KS_W == 0, "workgroups cover whole 128-column blocks of the partial-sum layout");

// 4 x 4 byte transpose: byte j of r[i] is (row i, column j); byte i of c[j] becomes it.
__device__ __forceinline__ void kr_transpose4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t (&c)[4]) {
    const uint32_t lo01 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0.0 r1.0 r0.1 r1.1
    const uint32_t hi01 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0.2 r1.2 r0.3 r1.3
    const uint32_t lo23 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    c[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);  // r0.0 r1.0 r2.0 r3.0
    c[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
    c[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    c[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// MR activation rows per workgroup (1, 2 or 4): rows MR * blockIdx.y .. + MR -
// 1 of A, those past M read as zero and not stored.  Sixteen waves for one
// row; eight for more, whose 16 MR accumulators per lane need the registers
// of two waves per SIMD.
constexpr int kr_waves(int mr) { return mr == 1 ? 16 : 8; }
// The activation rows per workgroup for M rows.
constexpr int kr_rows(int M) { return M == 1 ? 1 : M == 2 ? 2 : 4; }

// DW: 4-byte loads (N % 4 == 0, K % 4 == 0, 4-byte-aligned operands: the
// shapes the 16-byte loads cannot take), four per lane and row, each word of
// 4 columns all in N or all out.  Load e of a row covers bytes 256e ..
// 256e + 255 of the block's segment (lane l's word at 256e + 4l), so each
// instruction reads whole cache lines; lane l then holds columns 256e + 4l +
// j (j < 4) where the 16-byte form holds 16l + 4e + j.
template <int EL, bool DW, int MR>
__global__ __launch_bounds__(kr_waves(MR) * 64) void gemv_kn_row_kernel(GemmArgs p, KnSplit sp) {
    constexpr bool F8 = EL == ELEM_F8;
    constexpr int WV = kr_waves(MR);
    constexpr int BP = KS_ROWS / (WV * KR_ROWS);  // batches per wave per 128-row piece
    constexpr int AW = KR_ROWS / 4;               // activation words per row and batch
    static_assert(KS_ROWS % (WV * KR_ROWS) == 0, "a 128-row piece is whole batches of every wave");
    using AccE = typename std::conditional<F8, float, int32_t>::type;
    __shared__ __attribute__((aligned(16))) AccE red[WV][KR_W];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = p.M, N = p.N, K = p.K, S = sp.S;
    const int cbg = blockIdx.x / S, split = blockIdx.x % S;
    const int c0 = cbg * KR_W, m0 = blockIdx.y * MR;
    const int P = (K + KS_ROWS - 1) / KS_ROWS;
    const int i0 = split * sp.PS, i1 = min(P, i0 + sp.PS);  // this split's pieces
    const int nb = (i1 - i0) * BP;                          // batches of each wave
    // 16-byte loads (N % 16 == 0): a lane's 16 columns are all in or all out;
    // DW: each of its four words is
    constexpr int LW = DW ? 4 : 1;
    // the block's column of word e of lane l (DW), or of its 16 bytes
    auto colw = [&](int e) __attribute__((always_inline)) { return DW ? 256 * e + 4 * lane : 16 * lane + 4 * e; };
    uint32_t lane_off[LW];
#pragma unroll
    for (int e = 0; e < LW; ++e) {
        const int col = c0 + colw(e);
        lane_off[e] = col < N ? static_cast<uint32_t>(col) : 0x80000000u;
    }
    // activation rows: m K, rows past M at bit 31
    uint32_t arow[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) arow[m] = m0 + m < M ? static_cast<uint32_t>((m0 + m) * K) : 0x80000000u;
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B, K * N);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A, M * K);

    // Batch j of the wave: sub-step h = j % BP of piece i0 + j / BP, rows
    // k0 .. k0 + KR_ROWS - 1 with k0 = 128 i + KR_ROWS (h * waves + w), so each
    // sub-step of the workgroup reads consecutive rows.  The activation bytes
    // of those rows come first (one load per activation row, the same address
    // in every lane, so that it counts with the batch), then those rows of the
    // lane's columns.  Batches past the split, rows past M and columns past N
    // read as zero; K % 4 == 0 (K % 64 == 0 with 16-byte loads), so a batch of
    // 4 rows is all in K or all out.
    auto load = [&](int j, v4i (&b)[KR_ROWS], int (&a)[MR][AW]) __attribute__((always_inline)) {
        const int k0 = (i0 + j / BP) * KS_ROWS + KR_ROWS * ((j % BP) * WV + wave);
        const bool on = j < nb && k0 < K;
        // Bit 31 set: outside every range.  Outside batches take row 0, so that
        // no offset (with the row's r * N added) passes 2^32: at most
        // 2^31 + K * N for an invalid column, 2^31 + 16 * N for a batch outside,
        // 2^31 + M * K for an activation row or batch outside.
        const int kk = on ? k0 : 0;
        const uint32_t off = on ? 0u : 0x80000000u;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int ao = static_cast<int>(off | (arow[m] + static_cast<uint32_t>(kk)));
            if constexpr (AW == 4) {
                const v4i av = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, ao, 0, 0));
#pragma unroll
                for (int q = 0; q < 4; ++q) a[m][q] = av[q];
            } else if constexpr (AW == 2) {
                const v2i av = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(ra, ao, 0, 0));
                a[m][0] = av[0];
                a[m][1] = av[1];
            } else {
                a[m][0] = __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(ra, ao, 0, 0));
            }
        }
        if constexpr (DW) {
#pragma unroll
            for (int r = 0; r < KR_ROWS; ++r)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    b[r][e] = __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(
                                                          rb, static_cast<int>(off | (lane_off[e] + static_cast<uint32_t>(kk * N))),
                                                          r * N, 2));
        } else {
            const uint32_t base = off | (lane_off[0] + static_cast<uint32_t>(kk * N));
#pragma unroll
            for (int r = 0; r < KR_ROWS; ++r)
                b[r] = __builtin_bit_cast(v4i,
                                          __builtin_amdgcn_raw_buffer_load_b128(rb, static_cast<int>(base), r * N, 2));
        }
    };

    AccE acc[MR][16];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[m][j] = AccE(0);

    auto consume = [&](const v4i (&b)[KR_ROWS], const int (&a)[MR][AW], auto san) __attribute__((always_inline)) {
        if constexpr (F8) {
            constexpr bool SAN = decltype(san)::value;
            float af[MR][KR_ROWS];
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int q = 0; q < AW; ++q) {
                    const uint32_t w =
                        SAN ? e4m3_sanitize(static_cast<uint32_t>(a[m][q])) : static_cast<uint32_t>(a[m][q]);
                    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
                    const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
                    af[m][4 * q] = lo.x;
                    af[m][4 * q + 1] = lo.y;
                    af[m][4 * q + 2] = hi.x;
                    af[m][4 * q + 3] = hi.y;
                }
#pragma unroll
            for (int r = 0; r < KR_ROWS; ++r) {
                v4i w = b[r];
                if constexpr (SAN) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(w[e])));
                }
                float bf[16];
                e4m3_chunk_to_f32(w, bf);
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[m][j] = __builtin_fmaf(af[m][r], bf[j], acc[m][j]);
            }
        } else {
#pragma unroll
            for (int q = 0; q < AW; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    uint32_t c[4];
                    kr_transpose4(static_cast<uint32_t>(b[4 * q][e]), static_cast<uint32_t>(b[4 * q + 1][e]),
                                  static_cast<uint32_t>(b[4 * q + 2][e]), static_cast<uint32_t>(b[4 * q + 3][e]), c);
#pragma unroll
                    for (int m = 0; m < MR; ++m)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[m][4 * e + j] =
                                __builtin_amdgcn_sdot4(static_cast<int>(c[j]), a[m][q], acc[m][4 * e + j], false);
                }
        }
    };
    // KR_D batches in flight in KR_D buffers, KR_D batches per iteration.  The
    // loads are issued unconditionally (a batch past the split reads nothing),
    // so the compiler's wait before each batch's use counts only the later
    // batches' loads; only the arithmetic of batches past the split is
    // skipped.  The scheduling barriers keep each batch's loads ahead of the
    // previous batch's arithmetic.
    auto stream = [&](auto san) __attribute__((always_inline)) {
        v4i b[KR_D][KR_ROWS];
        int a[KR_D][MR][AW];
#pragma unroll
        for (int d = 0; d < KR_D - 1; ++d) load(d, b[d], a[d]);
        for (int j = 0; j < nb; j += KR_D) {
#pragma unroll
            for (int d = 0; d < KR_D; ++d) {
                fence();
                load(j + d + KR_D - 1, b[(d + KR_D - 1) % KR_D], a[(d + KR_D - 1) % KR_D]);
                fence();
                if (j + d < nb) consume(b[d], a[d], san);
            }
        }
        fence();
    };
    if constexpr (!F8) {
        stream(std::false_type{});
    } else {
        // E4M3 0x7F / 0xFF: NaN to v_cvt_pk_f32_fp8, 0.0 to the reference.  The
        // stream runs on the raw codes; every product of finite codes is finite
        // and no sum of them overflows fp32, so a NaN sum proves a NaN code in
        // the wave's rows, and only then does the wave stream them again with
        // the codes cleared.
        stream(std::false_type{});
        bool bad = false;
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int j = 0; j < 16; ++j) bad |= __builtin_isnan(acc[m][j]);
        if (__builtin_amdgcn_ballot_w64(bad) != 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[m][j] = 0.0f;
            stream(std::true_type{});
        }
    }

    // The waves' sums, one activation row at a time, in the order w = 0, 1,
    // ...: lane l of wave w holds columns colw(e) + j of the workgroup's block
    // in acc[m][4e + j]; thread t finishes columns CT t .. CT t + CT - 1.
    constexpr int CT = KR_W / (WV * 64);
    AccE* const part = static_cast<AccE*>(sp.part);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if (m > 0) __syncthreads();  // every thread has read the previous row's sums
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            AccE* d = &red[wave][colw(e)];
            d[0] = acc[m][4 * e];
            d[1] = acc[m][4 * e + 1];
            d[2] = acc[m][4 * e + 2];
            d[3] = acc[m][4 * e + 3];
        }
        __syncthreads();
        if (m0 + m >= M) continue;  // the same for the whole workgroup
#pragma unroll
        for (int h = 0; h < CT; ++h) {
            const int col = CT * tid + h, n = c0 + col;
            AccE s = red[0][col];
#pragma unroll
            for (int w = 1; w < WV; ++w) s += red[w][col];
            if (n < N) part[((static_cast<size_t>(n / KS_W) * S + split) * M + m0 + m) * KS_W + n % KS_W] = s;
        }
    }
}

// The split kernel for M rows on kw-wave workgroups: 16-row activation blocks
// MB = 1 or 2 (M <= 16 / 32), non-temporal weight copies up to KS_NT_MAX_M
// rows; four waves only with one block.  (Four blocks, M <= 64, measured
// slower than the MFMA GEMM's 64x64 ring past 32 rows: N = 14336, K = 4096,
// M = 48 / 64 21.8 / 23.2 us on two-wave workgroups and 25.5 / 26.4 on one-wave
// ones against 21.4 / 21.8.)
template <int EL>
const void* ks_kernel(int M, int kw) {
    if (M <= 16) {
        const bool nt = M <= KS_NT_MAX_M;
        switch (kw) {
            case 1: return nt ? reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, true, 1, 1>)
                              : reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, false, 1, 1>);
            case 2: return nt ? reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, true, 2, 1>)
                              : reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, false, 2, 1>);
            case 4: return nt ? reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, true, 4, 1>)
                              : reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, false, 4, 1>);
            default: return nullptr;
        }
    }
    if ((kw != 1 && kw != 2) || M > KN_MAX_M) return nullptr;
    return kw == 1 ? reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, false, 1, 2>)
                   : reinterpret_cast<const void*>(&gemv_kn_split_kernel<EL, false, 2, 2>);
}

template <int EL, bool DW>
const void* kr_kernel(int mr) {
    return mr == 1   ? reinterpret_cast<const void*>(&gemv_kn_row_kernel<EL, DW, 1>)
           : mr == 2 ? reinterpret_cast<const void*>(&gemv_kn_row_kernel<EL, DW, 2>)
                     : reinterpret_cast<const void*>(&gemv_kn_row_kernel<EL, DW, 4>);
}

template <int EL, int OUT>
hipError_t launch_kn_split_out(const GemmArgs& p, const KnSplit& sp, hipStream_t stream) {
    GemmArgs a = p;
    KnSplit s = sp;
    void* args[] = {&a, &s};
    hipError_t e;
    if (sp.rowk) {
        const int nblk = (p.N + KR_W - 1) / KR_W, mr = kr_rows(p.M);
        const void* row = sp.dw ? kr_kernel<EL, true>(mr) : kr_kernel<EL, false>(mr);
        e = hipLaunchKernel(row, dim3(nblk * sp.S, (p.M + mr - 1) / mr), dim3(kr_waves(mr) * 64), args, 0, stream);
    } else {
        const int nblk = (p.N + sp.kw * KS_W - 1) / (sp.kw * KS_W);
        const void* split = ks_kernel<EL>(p.M, sp.kw);
        if (!split) return hipErrorInvalidValue;
        e = hipLaunchKernel(split, dim3(nblk * sp.S), dim3(sp.kw * 64), args, 0, stream);
    }
    if (e != hipSuccess) return e;
    // the split count bounds the partial sums each thread loads at once
    const void* red;
    if (static_cast<int64_t>(p.M) * p.N >= 256 * 256) {
        red = sp.S <= 8    ? reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 256, 8>)
              : sp.S <= 16 ? reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 256, 16>)
              : sp.S <= 32 ? reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 256, 32>)
                           : reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 256, KR_SMAX>);
        return hipLaunchKernel(red, dim3((p.N + 255) / 256, p.M), dim3(256), args, 0, stream);
    }
    red = sp.S <= 8    ? reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 64, 8>)
          : sp.S <= 16 ? reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 64, 16>)
          : sp.S <= 32 ? reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 64, 32>)
                       : reinterpret_cast<const void*>(&kn_reduce_kernel<EL, OUT, 64, KR_SMAX>);
    return hipLaunchKernel(red, dim3((p.N + 63) / 64, p.M), dim3(64), args, 0, stream);
}

template <int EL>
hipError_t launch_kn_split(const GemmArgs& p, const KnSplit& sp, hipStream_t stream) {
    switch (p.out_dtype) {
        case FKE_OUT_F32: return launch_kn_split_out<EL, FKE_OUT_F32>(p, sp, stream);
        case FKE_OUT_BF16: return launch_kn_split_out<EL, FKE_OUT_BF16>(p, sp, stream);
        default:
            if constexpr (EL == ELEM_I8) return launch_kn_split_out<ELEM_I8, FKE_OUT_I32>(p, sp, stream);
            return hipErrorInvalidValue;
    }
}

// ===========================================================================
// Full kernel: one workgroup per 64-column block over all of K (no workspace).
// Four waves split K: wave w takes the 128-row pieces w, w+4, ...; items of
// 128 rows x 64 bytes (8 KiB, sixteen rows per 1-KiB copy, four lanes per
// row) plus 2 KiB of activations, three ring slots per wave (120 KiB); the
// four waves' sums meet in LDS in the fixed order w = 0..3.
// ===========================================================================
constexpr int KF_W = 64;                 // columns (bytes of a B row) per workgroup
constexpr int KF_ROWS = 128;             // k rows per item
constexpr int KF_BI = KF_ROWS * KF_W;    // weight bytes per item (8 KiB)
constexpr int KF_AI = 16 * KF_ROWS;      // activation bytes per item (2 KiB)
constexpr int KF_ITEM = KF_BI + KF_AI;   // 10 KiB
constexpr int KF_DB = KF_BI / 1024;      // weight copies per item
constexpr int KF_DA = KF_AI / 1024;      // activation copies per item
constexpr int KF_DI = KF_DB + KF_DA;     // copies per item
constexpr int KF_NS = 3;                 // ring slots per wave (120 KiB of LDS per workgroup)

// Physical chunk offset of item row r: bijective on r bits 1..2 within each
// 8-row group (a 16-lane group reads 8 rows x 16 bytes = 128 bytes), and
// with bit 4 ^ bit 5 flipping it, rows of the two 16-lane groups of a half
// wave that share r mod 4 land in different chunks too.
__device__ __forceinline__ int kf_swz(int r) { return ((r >> 1) & 3) ^ ((((r >> 4) ^ (r >> 5)) & 1) * 3); }
__device__ __forceinline__ int kf_aswz(int m) { return (m & 7) ^ ((m >> 3) & 1); }

__device__ __forceinline__ v4i kf_rd128(const lds_u8* a) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ v2i kf_rdtr(const lds_u8* a) {
    v2i r;
    asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
// Every LDS read has landed; the registers they wrote are tied to the wait,
// so nothing reads (or copies) them before it.
template <int N>
__device__ __forceinline__ void kf_lgkm_wait_all(v4i (&a)[2], v2i (&t)[N]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    asm volatile("" : "+v"(a[0]), "+v"(a[1]));
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(t[i]));
}

// s_waitcnt vmcnt(KF_DI * n): every copy but those of the n latest items has landed.
__device__ __forceinline__ void kf_wait_items(int n) {
    static_assert(KF_DI == 10, "vmcnt steps below are 10 copies");
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<10>(); break;
        default: wait_vm<20>(); break;
    }
}

template <int EL, int OUT>
__global__ __launch_bounds__(256) void gemv_kn_full_kernel(GemmArgs p) {
    constexpr bool F8 = EL == ELEM_F8;
    static_assert(EL == ELEM_I8 || (F8 && OUT != FKE_OUT_I32), "FP8: fp32 or bf16 out");
    static_assert(KF_NS == 3, "kf_wait_items covers up to two later items");
    using AccV = typename std::conditional<F8, v4f, v4i>::type;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[KF_NS][4][KF_ITEM];
    __shared__ __attribute__((aligned(16))) float esb[KF_W], ebias[KF_W], esa[64];

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
    const int n0 = blk * KF_W;
    const int P = (K + KF_ROWS - 1) / KF_ROWS;         // pieces along K
    const int np = wave < P ? (P - 1 - wave) / 4 + 1 : 0;  // pieces of this wave

    // Epilogue operands straight to LDS (dword LDS-DMA by wave 0 before its
    // stream; older than every item's copies, so landed with the first item).
    if (wave == 0) {
        const int nc = min(KF_W, N - n0);
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
    lds_u8* const lring = (lds_u8*)(&ring[0][wave][0]);  // slot q at + q * 4 * KF_ITEM
    constexpr int SLOT = 4 * KF_ITEM;

    // Copy geometry (k-independent part of each lane's source offsets).
    // Weights, copy d: row i = 16d + l/4 of the item, physical chunk l%4
    // holding logical chunk (l%4) ^ kf_swz(i).  Activations, copy d: row
    // m = 8d + l/8, physical chunk l%8 holding logical chunk (l%8) ^ kf_aswz(m).
    uint32_t boff[KF_DB];
    int brow[KF_DB];
#pragma unroll
    for (int d = 0; d < KF_DB; ++d) {
        const int i = 16 * d + (lane >> 2);
        brow[d] = i;
        boff[d] = static_cast<uint32_t>(i * N + n0 + 16 * ((lane & 3) ^ kf_swz(i)));
    }
    uint32_t aoff[KF_DA];
    int akb[KF_DA];
    bool arow[KF_DA];
#pragma unroll
    for (int d = 0; d < KF_DA; ++d) {
        const int m = 8 * d + (lane >> 3);
        const int c = (lane & 7) ^ kf_aswz(m);
        arow[d] = m < M;
        akb[d] = 16 * c;
        aoff[d] = static_cast<uint32_t>(m * K + 16 * c);
    }
    auto issue = [&](int j, lds_u8* dst) __attribute__((always_inline)) {
        const int k0 = (wave + 4 * j) * KF_ROWS;
#pragma unroll
        for (int d = 0; d < KF_DB; ++d) {
            const uint32_t off = k0 + brow[d] < K ? boff[d] + static_cast<uint32_t>(k0 * N) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, dst + d * 1024, 16, static_cast<int>(off), 0, 0, 2);
        }
#pragma unroll
        for (int d = 0; d < KF_DA; ++d) {
            const uint32_t off = arow[d] && k0 + akb[d] < K ? aoff[d] + static_cast<uint32_t>(k0) : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst + KF_BI + d * 1024, 16, static_cast<int>(off), 0, 0, 0);
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
        wadr[cb] = static_cast<uint32_t>(r * KF_W + 16 * (cb ^ kf_swz(r)) + 8 * hh);
    }
    // Activation reads: row m = l % 16, logical chunk (INT8) 4s + G for step
    // s, (FP8) 2G + e for half e.
    const int am = lane & 15;
    uint32_t aadr[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int c = F8 ? 2 * G + e : 4 * e + G;
        aadr[e] = static_cast<uint32_t>(KF_BI + am * KF_ROWS + 16 * (c ^ kf_aswz(am)));
    }

    AccV acc[4];
    // The stream on raw codes (SAN false), or with FP8's 0x7F / 0xFF codes
    // cleared on the VALU (SAN true, FP8's replay).
    auto stream = [&](auto sanc) __attribute__((always_inline)) {
        constexpr bool SAN = decltype(sanc)::value;
        (void)SAN;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[cb] = AccV{0, 0, 0, 0};

        int issued = 0;
#pragma unroll
        for (int q = 0; q < KF_NS; ++q)
            if (issued < np) {
                issue(issued, lring + q * SLOT);
                ++issued;
            }
        for (int c = 0; c < np; ++c) {
            lds_u8* const slot = lring + (c % KF_NS) * SLOT;
            kf_wait_items(issued - c - 1);
            // Fragments to registers, then the slot is refilled before the MFMAs.
            // 18 reads: at most 12 in flight (lgkmcnt's field is 4 bits).
            v4i af[2];
            v2i tr[16];  // INT8: [2 steps][4 blocks][2 eighths]; FP8: [4 blocks][4 eighths]
            af[0] = kf_rd128(slot + aadr[0]);
            af[1] = kf_rd128(slot + aadr[1]);
#pragma unroll
            for (int x = 0; x < 16; ++x) {
                uint32_t a;
                if constexpr (F8) {
                    const int cb = x >> 2, t = x & 3;  // eighth t of block cb: rows 32G + 8t ..
                    a = (t >= 2 ? wadr[cb ^ 3] : wadr[cb]) + (8 * t) * KF_W;
                } else {
                    const int s = x >> 3, cb = (x >> 1) & 3, t = x & 1;  // rows 64s + 16G + 8t ..
                    a = wadr[cb] + (64 * s + 8 * t) * KF_W;
                }
                if (x + 2 >= 12) asm volatile("s_waitcnt lgkmcnt(11)" ::: "memory");
                tr[x] = kf_rdtr(slot + a);
            }
            kf_lgkm_wait_all(af, tr);
            v4i wf[8];  // INT8: [2 steps][4 blocks] of 16 k bytes; FP8: [4 blocks][2 halves] of 16 k bytes
#pragma unroll
            for (int x = 0; x < 8; ++x) wf[x] = v4i{tr[2 * x][0], tr[2 * x][1], tr[2 * x + 1][0], tr[2 * x + 1][1]};
            if (issued < np) {
                issue(issued, slot);
                ++issued;
            }
            if constexpr (F8) {
                if constexpr (SAN) {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            af[h][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(af[h][e])));
#pragma unroll
                    for (int x = 0; x < 8; ++x)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            wf[x][e] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(wf[x][e])));
                }
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
    };
    if constexpr (!F8) {
        stream(std::false_type{});
    } else {
        // E4M3 0x7F / 0xFF are NaN to the MFMA but 0.0 to the reference.
        // Real quantizers never emit them (they saturate at 448), and
        // clearing every fragment costs VALU work the stream cannot hide, so
        // the wave streams the raw codes first: every product of finite codes
        // is finite and no sum of them overflows, so a NaN sum proves a NaN
        // code in this wave's rows or columns, and only then does the wave
        // stream its pieces again with the codes cleared.  Its ring slots are
        // free (the stream ends with every copy landed) and the other waves
        // are not waited for, so the replay is the wave's own.
        stream(std::false_type{});
        bool bad = false;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int v = 0; v < 4; ++v) bad |= __builtin_isnan(acc[cb][v]);
        if (__builtin_amdgcn_ballot_w64(bad) != 0) stream(std::true_type{});
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
hipError_t launch_kn_full(const GemmArgs& p, hipStream_t stream) {
    GemmArgs a = p;
    void* args[] = {&a};
    const void* f;
    switch (p.out_dtype) {
        case FKE_OUT_F32: f = reinterpret_cast<const void*>(&gemv_kn_full_kernel<EL, FKE_OUT_F32>); break;
        case FKE_OUT_BF16: f = reinterpret_cast<const void*>(&gemv_kn_full_kernel<EL, FKE_OUT_BF16>); break;
        default:
            if constexpr (EL == ELEM_I8) {
                f = reinterpret_cast<const void*>(&gemv_kn_full_kernel<ELEM_I8, FKE_OUT_I32>);
                break;
            }
            return hipErrorInvalidValue;
    }
    return hipLaunchKernel(f, dim3((p.N + KF_W - 1) / KF_W), dim3(256), args, 0, stream);
}

}  // namespace

// Layout, operand types and 32-bit offsets common to every [K,N] kernel.
static bool kn_common_ok(const GemmArgs& p, int elem) {
    if (p.b_layout != FKE_B_KN || p.swiglu || p.M < 1 || p.M > KN_MAX_M || p.N < 1 || p.K < 4) return false;
    if (elem != ELEM_I8 && elem != ELEM_F8) return false;
    if (elem == ELEM_F8 && p.out_dtype == FKE_OUT_I32) return false;
    return static_cast<int64_t>(p.K) * p.N <= INT32_MAX && static_cast<int64_t>(p.M) * p.K <= INT32_MAX;
}
// 16-byte copies: row starts (B: k*N + n, A: m*K + k) stay 16-byte aligned (every kernel).
static bool kn_aligned16(const GemmArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    return p.K >= 64 && p.N % 16 == 0 && p.K % 64 == 0 && ((a | b) & 15) == 0;
}
// 4-byte loads: the row kernel's dword form (any M to 32), which a workspace
// of one split's partial sums or more lets run.
static bool kn_aligned4(const GemmArgs& p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    return p.N % 4 == 0 && p.K % 4 == 0 && ((a | b) & 3) == 0;
}
static bool kn_shape_ok(const GemmArgs& p, int elem) {
    return kn_common_ok(p, elem) && (kn_aligned16(p) || kn_aligned4(p));
}

// Partial sums of the split kernel: [ceil(N/128)][S][M][128], 4 bytes each.
static size_t kn_ws_bytes(int M, int N, int S) {
    return static_cast<size_t>((N + KS_W - 1) / KS_W) * static_cast<size_t>(S) * static_cast<size_t>(M) * KS_W * 4;
}

// K splits of the split kernel for workgroups of kw waves (128 columns each):
// as many as fill the device's CUs with one workgroup each (S <= 8, at least
// one 128-row piece per split, and no more than a workspace of ws_bytes, or a
// split-pool slot, holds), with no empty split; grid 0 and S = 1: the full kernel.
// Past CUs / 2 blocks the workgroups take several rounds, and S in 2..4 is the
// one with the fewest rounds per split (ties: the smaller): at N = 81920 /
// 98304 / 128256, K = 4096, M = 1, four-wave workgroups with S = 3 / 4 / 2 ran
// 54 / 64 / 79 us against 88 / 107 / 108 us for the full kernel.
struct KsPlan {
    int S, PS, grid;
};
static KsPlan ks_plan(const GemmArgs& p, int kw, int kCUs, size_t ws_bytes) {
    const int P = (p.K + KS_ROWS - 1) / KS_ROWS;
    const int nblk = (p.N + kw * KS_W - 1) / (kw * KS_W);
    int S = kCUs / nblk;
    if (S < 2) {
        double best = 0.0;
        for (int s = 2; s <= 4; ++s) {
            const double per = static_cast<double>((static_cast<int64_t>(nblk) * s + kCUs - 1) / kCUs) / s;
            if (s == 2 || per < best - 1e-9) {
                best = per;
                S = s;
            }
        }
    }
    if (S > KS_SMAX) S = KS_SMAX;
    if (S > P) S = P;
    while (S > 1 && kn_ws_bytes(p.M, p.N, S) > ws_bytes) --S;
    if (S < 2) return KsPlan{1, P, 0};
    const int PS = (P + S - 1) / S;
    S = (P + PS - 1) / PS;
    return KsPlan{S, PS, nblk * S};
}

// The plan: M = 1 takes the row kernel whenever two or more splits of its
// 1024-column workgroups fit: S = CUs / blocks (at most 64, whole 128-row
// pieces, none empty; 16 at N = 14336, K = 4096: 224 workgroups).  So does
// any M (to 32) that the 16-byte loads cannot take, with blocks counted once
// per workgroup of activation rows and one split when no more fit.  Otherwise
// the split kernel, on workgroups of two waves (256 columns; four splits at
// N = 14336), of four when two-wave blocks outnumber half the CUs (N > 32768
// on 256 CUs: fewer, wider workgroups over several rounds), and of one when
// two-wave workgroups, their splits capped, fill less than 7/8 of the CUs and
// one-wave ones fill more (few column blocks, long K), or past 13 rows when
// one-wave ones fill 7/8 with fewer splits (fewer partial sums).  Same-box A/B
// (HIP graphs, K = 4096 unless noted, INT8 bf16 out, us): N = 14336, M = 4 /
// 8 / 10 / 12 / 14 / 16: two waves 13.8 / 14.2 / 14.5 / 14.5 / 15.9 / 16.2,
// one 14.8 / 15.0 / 15.1 / 15.2 / 15.9 / 16.0, four 14.1 / 15.1 / 15.5 /
// 16.0 / 16.5 / 16.8; N = 4096, K = 14336, M = 4 / 16: one 13.5 / 15.0, two
// 17.2 / 18.5, four 24.0 / 25.8; N = 128256, M = 16: four 98.4, two 100.7,
// one 103.1.
static void kn_splits(const GemmArgs& p, size_t ws_bytes, KnSplit* sp) {
    const int kCUs = device_cus();
    if (ws_bytes > FKE_SPLIT_SLOT_BYTES) ws_bytes = FKE_SPLIT_SLOT_BYTES;
    const int P = (p.K + KS_ROWS - 1) / KS_ROWS;
    sp->rowk = 0;
    sp->dw = !kn_aligned16(p);
    if (p.M == 1 || sp->dw) {
        const int mr = kr_rows(p.M);
        int S = kCUs / ((p.N + KR_W - 1) / KR_W * ((p.M + mr - 1) / mr));
        if (S > KR_SMAX) S = KR_SMAX;
        if (S > P) S = P;
        if (S < 1) S = 1;
        while (S > 1 && kn_ws_bytes(p.M, p.N, S) > ws_bytes) --S;
        // the dword form has no other kernel: one split will do
        if (S >= 2 || (sp->dw && kn_ws_bytes(p.M, p.N, 1) <= ws_bytes)) {
            const int PS = (P + S - 1) / S;
            sp->S = (P + PS - 1) / PS;
            sp->PS = PS;
            sp->rowk = 1;
            sp->kw = 0;
            return;
        }
    }
    if (sp->dw) {  // no kernel without its workspace: gemv_kn_plan_runs says no
        sp->S = 1;
        sp->PS = P;
        sp->kw = 0;
        return;
    }
    const int fill = kCUs - kCUs / 8;
    int kw = 2;
    KsPlan pl;
    if ((p.N + 2 * KS_W - 1) / (2 * KS_W) > kCUs / 2) {
        kw = 4;
        pl = ks_plan(p, 4, kCUs, ws_bytes);
    } else {
        pl = ks_plan(p, 2, kCUs, ws_bytes);
        const KsPlan p1 = ks_plan(p, 1, kCUs, ws_bytes);
        if (p1.S > 1 && ((pl.grid < fill && p1.grid > pl.grid) || (p.M > 13 && p1.S < pl.S && p1.grid >= fill))) {
            kw = 1;
            pl = p1;
        }
    }
    sp->S = pl.S;
    sp->PS = pl.PS;
    sp->kw = kw;
}

// 17..32 rows (two activation blocks per item) only where the split
// plan, at a pool slot's size, fills 7/8 of the CUs or more in one round on
// one- or two-wave workgroups; other batches go to the MFMA GEMM's tiles.
bool gemv_kn_supports(const GemmArgs& p, int elem) {
    if (!kn_shape_ok(p, elem)) return false;
    KnSplit sp;
    if (!kn_aligned16(p)) {  // the row kernel's dword form
        kn_splits(p, SIZE_MAX, &sp);
        return sp.rowk != 0;
    }
    if (p.M <= 16) return true;
    kn_splits(p, SIZE_MAX, &sp);
    if (sp.S < 2 || sp.rowk || sp.kw == 4) return false;
    const int kCUs = device_cus();
    const int grid = (p.N + sp.kw * KS_W - 1) / (sp.kw * KS_W) * sp.S;
    return grid <= kCUs && grid >= kCUs - kCUs / 8;
}

// Same box, N = 14336, K = 4000, B [K,N], INT8 bf16 out: M = 4 16.2 us on
// the row kernel against 19.4 on the MFMA GEMM; M = 16 27.8 against 20.3.
bool gemv_kn_yields_to_mfma(const GemmArgs& p) { return p.M > 4 && !kn_aligned16(p); }

size_t gemv_kn_workspace_bytes(const GemmArgs& p) {
    KnSplit sp;
    kn_splits(p, SIZE_MAX, &sp);
    return sp.S > 1 || sp.rowk ? kn_ws_bytes(p.M, p.N, sp.S) : 0;
}

bool gemv_kn_plan_runs(const GemmArgs& p, const KnSplit& sp) {
    return sp.rowk || (!sp.dw && (sp.S > 1 || p.M <= 16));
}

// No split (S = 1) without a workspace, or with one not 16-byte aligned (the
// second kernel reads the partial sums 16 bytes at a time).
KnSplit gemv_kn_plan(const GemmArgs& p, void* ws, size_t ws_bytes) {
    KnSplit sp;
    const bool usable = ws && (reinterpret_cast<uintptr_t>(ws) & 15) == 0;
    kn_splits(p, usable ? ws_bytes : 0, &sp);
    sp.part = sp.S > 1 || sp.rowk ? ws : nullptr;
    return sp;
}

hipError_t launch_gemv_kn(const GemmArgs& p, int elem, const KnSplit& sp, hipStream_t stream) {
    if (!gemv_kn_plan_runs(p, sp)) return hipErrorInvalidValue;  // the full kernel: 16 rows, 16-byte loads
    if (sp.S > 1 || sp.rowk) {
        if (!sp.part) return hipErrorInvalidValue;
        return elem == ELEM_F8 ? launch_kn_split<ELEM_F8>(p, sp, stream) : launch_kn_split<ELEM_I8>(p, sp, stream);
    }
    return elem == ELEM_F8 ? launch_kn_full<ELEM_F8>(p, stream) : launch_kn_full<ELEM_I8>(p, stream);
}

}  // namespace fke
