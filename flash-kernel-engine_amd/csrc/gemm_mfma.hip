// gemm_mfma.hip — LDS-staged MFMA GEMM for the large-M (prefill) shapes.
//
// Replaces the arithmetic of reference src/quantized_gemm.cu:15-54 (INT8,
// int8_gemm_dp4a_kernel) and :99-118 (FP8, fp8_gemm_scaled_kernel) for M > 16.
//
// Workgroup tile 256x256 with 8 waves (two per SIMD): wave w owns rows
// 128*((w>>1)&1) .. +128 and columns 64*((w&1) + 2*(w>>2)) .. +64, i.e. 4x2
// MFMA blocks of 32x32 held in 128 AGPRs.  Two waves per SIMD let one wave
// issue MFMAs while the other waits on LDS or memory.
//   INT8: v_mfma_i32_32x32x32_i8   (exact int32 accumulation)
//   FP8 : v_mfma_f32_32x32x64_f8f6f4 with E4M3 operands (fp32 accumulation)
// K advances 128 bytes per stage; two LDS stages of (256+256)x128 bytes
// (128 KiB of the CU's 160 KiB).  A (and B when stored [N,K]) is copied
// global->LDS with 128-bit direct-to-LDS loads (global_load_lds_dwordx4),
// eight lanes per 128-byte row segment, from per-lane 32-bit offsets computed
// once.  B stored [K,N] goes through registers and is byte-transposed with
// v_perm_b32 before a ds_write_b64.
//
// LDS layout of a stage: row r (an M row of A or an N row of B) holds its 128
// K-bytes as eight 16-byte chunks; logical chunk c is stored at physical
// chunk c ^ swz(r), swz(r) = (q ^ (q >> 3)) & 7 with q = r mod 32.  A 128-bit
// fragment read by 8 (or 16) consecutive lanes of consecutive rows then
// touches every LDS bank once, whether the LDS serves 8 lanes x 16 B or 16
// lanes x 16 B per cycle; and because the swizzle repeats every 32 rows, all
// fragments of a k step share one address register plus immediate offsets.
//
// The per-row / per-column epilogue operands of the tile (scale_a, scale_b,
// bias) are staged once in LDS beside the two stages.
#include "fke_internal.h"

namespace fke {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 128;           // bytes of K per stage
constexpr int NWAVES = 8;
constexpr int NTHREADS = NWAVES * 64;
constexpr int STAGE_A = BM * BK;  // 32 KiB
constexpr int STAGE_B = BN * BK;  // 32 KiB
constexpr int PW = BM * BK / 1024 / NWAVES;  // DMA loads per wave per panel (4)

__device__ __forceinline__ int swz(int r) { return ((r & 31) ^ ((r & 31) >> 3)) & 7; }

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without the LDS fence of __syncthreads: every LDS write a
// stage depends on comes from LDS-DMA (ordered by the explicit vmcnt wait
// before the barrier) or from ds_writes followed by an explicit lgkmcnt wait.
// The empty asm statements keep the compiler from moving memory operations
// across the barrier.
__device__ __forceinline__ void barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void dma16(const int8_t* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}

// Workgroup -> output tile.  Consecutive workgroup ids are dispatched round
// robin over the 8 XCDs; give each XCD a contiguous range of tile ids and walk
// that range in groups of GROUP_M tile rows so the workgroups an XCD runs at
// once share A and B panels in its L2.
constexpr int GROUP_M = 4;
constexpr int NXCD = 8;

__device__ __forceinline__ void tile_of(int bid, int gm, int gn, int& tm, int& tn) {
    const int nwg = gm * gn;
    const int q = nwg / NXCD, rem = nwg % NXCD;
    const int xcd = bid % NXCD, local = bid / NXCD;
    const int tile = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + local;
    const int per_group = GROUP_M * gn;
    const int group = tile / per_group;
    const int first_m = group * GROUP_M;
    const int gsize = min(gm - first_m, GROUP_M);
    const int in_group = tile % per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Direct-to-LDS copy plan of one 256-row x 128-byte K-contiguous panel (A, or
// B in [N,K] order).  Each wave issues PW loads of 1 KiB (8 rows x 128 B);
// lane l lands at byte 16*l of its KiB, so it fetches the logical chunk that
// the swizzle assigns to that physical slot.  Rows past `rows` re-read the
// last valid row (their outputs are never stored).
struct Panel {
    int off[PW];  // byte offset of this lane's 16-byte source at k = 0
    __device__ void init(int ld, int row0, int rows, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int seg = wave * PW + i;
            const int r = seg * 8 + (lane >> 3);
            const int lc = (lane & 7) ^ swz(r);
            off[i] = min(row0 + r, rows - 1) * ld + lc * 16;
        }
    }
    // gk: uniform panel base at this stage's k; wave: uniform wave index.
    __device__ __forceinline__ void issue(const int8_t* gk, uint8_t* lds, int wave) const {
#pragma unroll
        for (int i = 0; i < PW; ++i)
            dma16(gk + static_cast<uint32_t>(off[i]), lds + (wave * PW + i) * 1024);
    }
};

// B stored [K,N]: each thread owns an 8(k) x 8(n) byte block of the 128 x 256
// stage tile (thread t: n group t%32, k group t/32), loaded as eight 8-byte
// rows so that 32 lanes read 256 contiguous bytes of one k row.
struct KNPlan {
    const int8_t* base;  // B + n (column group start, clamped) at k = 8*(t/32)
    int N;
    __device__ void init(const int8_t* B, int N_, int n0, int tid) {
        N = N_;
        const int n = min(n0 + (tid & 31) * 8, N_ - 8);  // ragged N: re-read the last group
        base = B + n + static_cast<size_t>(tid >> 5) * 8 * N_;
    }
    __device__ __forceinline__ void load(int k0, uint2 (&r)[8]) const {
        const int8_t* q = base + static_cast<size_t>(k0) * N;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = *reinterpret_cast<const uint2*>(q + static_cast<size_t>(i) * N);
    }
};

// 4x4 byte transpose of (x0..x3) rows -> columns with v_perm_b32.
__device__ __forceinline__ void t4x4(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                     uint32_t& y0, uint32_t& y1, uint32_t& y2, uint32_t& y3) {
    const uint32_t t0 = __builtin_amdgcn_perm(x1, x0, 0x05010400u);  // a0 b0 a1 b1
    const uint32_t t1 = __builtin_amdgcn_perm(x1, x0, 0x07030602u);  // a2 b2 a3 b3
    const uint32_t t2 = __builtin_amdgcn_perm(x3, x2, 0x05010400u);  // c0 d0 c1 d1
    const uint32_t t3 = __builtin_amdgcn_perm(x3, x2, 0x07030602u);  // c2 d2 c3 d3
    y0 = __builtin_amdgcn_perm(t2, t0, 0x05040100u);                 // a0 b0 c0 d0
    y1 = __builtin_amdgcn_perm(t2, t0, 0x07060302u);                 // a1 b1 c1 d1
    y2 = __builtin_amdgcn_perm(t3, t1, 0x05040100u);                 // a2 b2 c2 d2
    y3 = __builtin_amdgcn_perm(t3, t1, 0x07060302u);                 // a3 b3 c3 d3
}

// Transpose the thread's 8x8 block and store it as 8 bytes (k = 8*kg..+8) of
// eight B^T rows (n = 8*ng + c).
template <int ELEM>
__device__ __forceinline__ void kn_store(const uint2 (&r)[8], uint8_t* lds_b, int tid) {
    const int ng = tid & 31, kg = tid >> 5;
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // column halves: bytes 0..3 (.x) and 4..7 (.y)
        uint32_t lo[4], hi[4];
        if (h == 0) {
            t4x4(r[0].x, r[1].x, r[2].x, r[3].x, lo[0], lo[1], lo[2], lo[3]);
            t4x4(r[4].x, r[5].x, r[6].x, r[7].x, hi[0], hi[1], hi[2], hi[3]);
        } else {
            t4x4(r[0].y, r[1].y, r[2].y, r[3].y, lo[0], lo[1], lo[2], lo[3]);
            t4x4(r[4].y, r[5].y, r[6].y, r[7].y, hi[0], hi[1], hi[2], hi[3]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int n = ng * 8 + h * 4 + c;
            uint32_t w0 = lo[c], w1 = hi[c];
            if constexpr (ELEM == ELEM_F8) {
                w0 = e4m3_sanitize(w0);
                w1 = e4m3_sanitize(w1);
            }
            const int chunk = (kg >> 1) ^ swz(n);
            *reinterpret_cast<uint2*>(lds_b + n * BK + chunk * 16 + (kg & 1) * 8) = make_uint2(w0, w1);
        }
    }
}

// FP8 operands staged by DMA cannot be rewritten on the way in; sanitize the
// 0x7F/0xFF codes in the fragment registers instead.
__device__ __forceinline__ v8i sanitize8(v8i x) {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = static_cast<int>(e4m3_sanitize(static_cast<uint32_t>(x[i])));
    return x;
}

template <int ELEM>
struct Acc;
template <>
struct Acc<ELEM_I8> {
    using T = v16i;
};
template <>
struct Acc<ELEM_F8> {
    using T = v16f;
};

// One stage of MFMAs for this wave's 128x64 block: rows r0.. of the stage's A
// rows (As) and columns c0.. of its B^T rows (Bs).  `live` false zeroes the B
// fragments (a phantom stage that must add nothing).
template <int ELEM, int BL>
__device__ __forceinline__ void stage_compute(const uint8_t* As, const uint8_t* Bs,
                                              typename Acc<ELEM>::T (&acc)[4][2], int r0, int c0,
                                              int lane, bool live) {
    const int lr = lane & 31;
    const int lh = lane >> 5;
    // Rows r0 + 32*i + lr share swz(lr): one base address per operand and k
    // step, the 32-row blocks at immediate offsets of 32*BK bytes.
    const int sw = swz(lr);
    const uint8_t* Ab = As + (r0 + lr) * BK;
    const uint8_t* Bb = Bs + (c0 + lr) * BK;
    if constexpr (ELEM == ELEM_I8) {
        // Fragments of k step ks+1 are read while the MFMAs of step ks run.
        auto rd = [&](int ks, v4i (&a)[4], v4i (&b)[2]) {
            const int co = ((ks * 2 + lh) ^ sw) << 4;  // this lane's 16-byte chunk of the 32-byte step
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const v4i*>(Ab + i * 32 * BK + co);
#pragma unroll
            for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const v4i*>(Bb + j * 32 * BK + co);
        };
        v4i a0[4], b0[2], a1[4], b1[2];
        auto mm = [&](const v4i (&a)[4], const v4i (&b)[2]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], live ? b[j] : v4i{0, 0, 0, 0},
                                                                      acc[i][j], 0, 0, 0);
        };
        // Program order per step: reads of step ks+1, then the MFMAs of step
        // ks (fenced, so the MFMAs only wait on reads issued a block earlier).
        rd(0, a0, b0);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks += 2) {
            rd(ks + 1, a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            mm(a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 2 < BK / 32) rd(ks + 2, a0, b0);
            __builtin_amdgcn_sched_barrier(0);
            mm(a1, b1);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < BK / 64; ++ks) {
            const int cx = ((ks * 4 + lh * 2) ^ sw) << 4;      // two 16-byte chunks = 32 k codes per lane
            const int cy = ((ks * 4 + lh * 2 + 1) ^ sw) << 4;
            v8i a[4], b[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v4i x = *reinterpret_cast<const v4i*>(Ab + i * 32 * BK + cx);
                const v4i y = *reinterpret_cast<const v4i*>(Ab + i * 32 * BK + cy);
                a[i] = sanitize8(v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]});
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const v4i x = *reinterpret_cast<const v4i*>(Bb + j * 32 * BK + cx);
                const v4i y = *reinterpret_cast<const v4i*>(Bb + j * 32 * BK + cy);
                b[j] = v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                if constexpr (BL == FKE_B_NK) b[j] = sanitize8(b[j]);  // KN was sanitized at staging
                if (!live) b[j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        a[i], b[j], acc[i][j], 0, 0, 0, 0, 0, 0);
        }
    }
}

template <int ELEM, int BL, int OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_mfma_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[STAGE_A + STAGE_B];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[STAGE_A + STAGE_B];
    __shared__ __attribute__((aligned(16))) float epi_sa[BM];    // scale of each tile row
    __shared__ __attribute__((aligned(16))) float epi_sb[BN];    // scale of each tile column
    __shared__ __attribute__((aligned(16))) float epi_bias[BN];  // bias of each tile column

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS/M0 math
    const int r0 = ((wave >> 1) & 1) * 128;             // wave's rows within the tile
    const int c0 = ((wave & 1) + 2 * (wave >> 2)) * 64;  // wave's columns within the tile

    const int M = p.M, N = p.N, K = p.K;
    const int gm = (M + BM - 1) / BM, gn = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gm, gn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int8_t* A = static_cast<const int8_t*>(p.A);
    const int8_t* B = static_cast<const int8_t*>(p.B);

    // epilogue operands -> LDS (visible after the first barrier below)
    if (tid < BM) {
        const int m = min(m0 + tid, M - 1);
        epi_sa[tid] = p.scale_a ? p.scale_a[m] : p.sa;
    } else {
        const int c = tid - BM;
        const int n = min(n0 + c, N - 1);
        epi_sb[c] = p.scale_b ? p.scale_b[n] : p.sb;
        epi_bias[c] = p.bias ? p.bias[n] : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the epilogue-operand ds_writes are done

    typename Acc<ELEM>::T acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    const int KT = K / BK;
    Panel pa, pb;
    pa.init(K, m0, M, wave, lane);
    KNPlan kp;
    if constexpr (BL == FKE_B_NK) pb.init(K, n0, N, wave, lane);
    else kp.init(B, N, n0, tid);
    uint2 knr[8];

    // Stage kt -> buffer: DMA for A (and B in NK order); B in KN order is
    // loaded into registers here and transposed into LDS by finish().
    // The DMA block is fenced on both sides: each global_load_lds needs its own
    // M0 value, and an M0 write that the scheduler hoists into the MFMA stream
    // costs an lgkmcnt(0) wait there.
    auto issue = [&](int kt, uint8_t* buf) {
        __builtin_amdgcn_sched_barrier(0);
        pa.issue(A + kt * BK, buf, wave);
        if constexpr (BL == FKE_B_NK) pb.issue(B + kt * BK, buf + STAGE_A, wave);
        else kp.load(kt * BK, knr);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto finish = [&](uint8_t* buf) {
        if constexpr (BL == FKE_B_KN) {
            kn_store<ELEM>(knr, buf + STAGE_A, tid);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): own ds_writes done
        }
        wait_vm<0>();
        barrier();
    };

    // Two-stage pipeline with static buffer roles (lds0 / lds1 are distinct
    // objects, so the compiler can see that a stage's LDS DMA never aliases
    // the other stage's fragment reads and need not wait on it early).  The
    // sched_barrier after each issue keeps the loads ahead of the stage's
    // MFMAs (the scheduler would otherwise sink them below), and the body has
    // no data-dependent branches, so the accumulators stay in AGPRs.
    issue(0, lds0);
    finish(lds0);
    int kt = 0;
    for (; kt + 2 < KT; kt += 2) {
        issue(kt + 1, lds1);
        __builtin_amdgcn_sched_barrier(0);
        stage_compute<ELEM, BL>(lds0, lds0 + STAGE_A, acc, r0, c0, lane, true);
        finish(lds1);
        issue(kt + 2, lds0);
        __builtin_amdgcn_sched_barrier(0);
        stage_compute<ELEM, BL>(lds1, lds1 + STAGE_A, acc, r0, c0, lane, true);
        finish(lds0);
    }
    // Tail: one or two stages remain, stage kt is in lds0.  With one left, the
    // lds1 stage re-reads stage kt (a valid address) and its B fragments are
    // zeroed, so it adds nothing.
    issue(min(kt + 1, KT - 1), lds1);
    __builtin_amdgcn_sched_barrier(0);
    stage_compute<ELEM, BL>(lds0, lds0 + STAGE_A, acc, r0, c0, lane, true);
    finish(lds1);
    stage_compute<ELEM, BL>(lds1, lds1 + STAGE_A, acc, r0, c0, lane, kt + 1 < KT);

    // Fused epilogue.  32x32 block layout of the accumulator: lane l holds
    // column l%32 and rows 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.
    const int lr = lane & 31, lh = lane >> 5;
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int cn = c0 + j * 32 + lr;  // column within the tile
        const int n = n0 + cn;
        const float sbn = epi_sb[cn];
        const float bn = epi_bias[cn];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int rm = r0 + i * 32 + 8 * g + 4 * lh;  // first of 4 consecutive tile rows
                const float4 sa4 = *reinterpret_cast<const float4*>(&epi_sa[rm]);
                const float sav[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = 4 * g + e;
                    const int m = m0 + rm + e;
                    if (m >= M || n >= N) continue;
                    const size_t idx = static_cast<size_t>(m) * N + n;
                    if constexpr (ELEM == ELEM_I8) {
                        const int32_t a = acc[i][j][v];
                        const float s = sav[e] * sbn;
                        const float y = has_bias ? __builtin_fmaf(static_cast<float>(a), s, bn)
                                                 : static_cast<float>(a) * s;
                        store_out<OUT>(p.C, idx, y, a);
                    } else {
                        const float s = p.sa * p.sb;
                        const float y = has_bias ? __builtin_fmaf(acc[i][j][v], s, bn) : acc[i][j][v] * s;
                        store_out<OUT>(p.C, idx, y, 0);
                    }
                }
            }
        }
    }
}

template <int ELEM, int BL, int OUT>
hipError_t launch_t(const GemmArgs& p, hipStream_t stream) {
    const int gm = (p.M + BM - 1) / BM, gn = (p.N + BN - 1) / BN;
    GemmArgs a = p;
    void* args[] = {&a};
    return hipLaunchKernel(reinterpret_cast<const void*>(&gemm_mfma_kernel<ELEM, BL, OUT>),
                           dim3(gm * gn), dim3(NTHREADS), args, 0, stream);
}

template <int ELEM, int BL>
hipError_t launch_out(const GemmArgs& p, hipStream_t s) {
    switch (p.out_dtype) {
        case FKE_OUT_F32: return launch_t<ELEM, BL, FKE_OUT_F32>(p, s);
        case FKE_OUT_BF16: return launch_t<ELEM, BL, FKE_OUT_BF16>(p, s);
        default:
            if constexpr (ELEM == ELEM_I8) return launch_t<ELEM, BL, FKE_OUT_I32>(p, s);
            return hipErrorInvalidValue;
    }
}

}  // namespace

bool mfma_supports(const GemmArgs& p, int elem) {
    (void)elem;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p.A), b = reinterpret_cast<uintptr_t>(p.B);
    if (p.M < 1 || p.N < 1 || p.K < BK || p.K % BK != 0) return false;
    if ((a | b) & 15) return false;
    // per-lane DMA offsets are 32-bit: (rows - 1) * K + K must fit
    if (static_cast<int64_t>(p.M) * p.K > INT32_MAX) return false;
    if (p.b_layout == FKE_B_NK && static_cast<int64_t>(p.N) * p.K > INT32_MAX) return false;
    if (p.b_layout == FKE_B_KN && (p.N % 16 != 0)) return false;
    return true;
}

hipError_t launch_mfma(const GemmArgs& p, int elem, hipStream_t s) {
    if (elem == ELEM_I8)
        return p.b_layout == FKE_B_NK ? launch_out<ELEM_I8, FKE_B_NK>(p, s)
                                      : launch_out<ELEM_I8, FKE_B_KN>(p, s);
    return p.b_layout == FKE_B_NK ? launch_out<ELEM_F8, FKE_B_NK>(p, s)
                                  : launch_out<ELEM_F8, FKE_B_KN>(p, s);
}

}  // namespace fke
