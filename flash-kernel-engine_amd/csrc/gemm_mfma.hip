// gemm_mfma.hip — LDS-staged MFMA GEMM for the large-M (prefill) shapes.
//
// Replaces the arithmetic of reference src/quantized_gemm.cu:15-54 (INT8,
// int8_gemm_dp4a_kernel) and :99-118 (FP8, fp8_gemm_scaled_kernel) for M > 16.
//
// Workgroup tile 256x256, 4 waves in a 2x2 grid, each wave owns 128x128 outputs
// as 4x4 MFMA blocks of 32x32:
//   INT8: v_mfma_i32_32x32x32_i8   (exact int32 accumulation)
//   FP8 : v_mfma_f32_32x32x64_f8f6f4 with E4M3 operands (fp32 accumulation)
// K advances 128 bytes per stage; two LDS stages of (256+256)x128 bytes
// (128 KiB of the CU's 160 KiB).  A (and B when stored [N,K]) is copied
// global->LDS with 128-bit direct-to-LDS loads (global_load_lds_dwordx4),
// eight lanes per 128-byte row segment.  B stored [K,N] goes through
// registers and is byte-transposed with v_perm_b32 before a ds_write_b64.
//
// LDS layout of a stage: row r (an M row of A or an N row of B) holds its 128
// K-bytes as eight 16-byte chunks; logical chunk c is stored at physical
// chunk c ^ swz(r), swz(r) = (r ^ (r >> 3)) & 7.  A 128-bit fragment read by
// 8 (or 16) consecutive lanes of consecutive rows then touches every LDS bank
// once, whether the LDS serves 8 lanes x 16 B or 16 lanes x 16 B per cycle.
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
constexpr int NTHREADS = 256;
constexpr int STAGE_A = BM * BK;  // 32 KiB
constexpr int STAGE_B = BN * BK;  // 32 KiB

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// s_waitcnt vmcnt(0) with expcnt/lgkmcnt left unconstrained (gfx9 encoding).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup -> output tile.  Consecutive workgroup ids are dispatched round
// robin over the 8 XCDs; give each XCD a contiguous range of tile ids and walk
// that range in groups of GROUP_M tile rows so the ~32 workgroups an XCD runs
// at once share A and B tiles in its L2.
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

// Direct-to-LDS copy of one 256-row x 128-byte K-contiguous panel (A, or B in
// [N,K] order).  Each wave issues 8 loads of 1 KiB (8 rows x 128 B); lane l
// lands at byte 16*l of its KiB, so the lane fetches the logical chunk that
// the swizzle assigns to that physical slot.  Rows past `rows` re-read the
// last valid row (their outputs are never stored).
__device__ __forceinline__ void panel_dma(const int8_t* __restrict__ g, int ld, int row0, int rows,
                                          int k0, uint8_t* lds, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int seg = wave * 8 + i;
        const int r = seg * 8 + (lane >> 3);
        const int lc = (lane & 7) ^ swz(r);
        const int gr = min(row0 + r, rows - 1);
        const int8_t* src = g + static_cast<size_t>(gr) * ld + k0 + lc * 16;
        __builtin_amdgcn_global_load_lds(src, lds + seg * 1024, 16, 0, 0);
    }
}

// B stored [K,N]: each thread owns an 8(k) x 16(n) byte block of the 128 x 256
// stage tile (thread t: n block t%16, k block t/16), loaded as eight 16-byte
// rows so that 16 lanes read 256 contiguous bytes of one k row.
struct KNRegs {
    v4i r[8];
};

__device__ __forceinline__ void kn_load(const int8_t* __restrict__ B, int N, int K, int n0, int k0,
                                        int tid, KNRegs& st) {
    const int nb = tid & 15, kb = tid >> 4;
    const int n = n0 + nb * 16;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int k = k0 + kb * 8 + i;
        if (n + 16 <= N) {
            st.r[i] = *reinterpret_cast<const v4i*>(B + static_cast<size_t>(k) * N + n);
        } else {
            // ragged N edge: columns past N are never stored; read the clamped
            // last 16-byte group so every load stays inside the row.
            const int nn = max(N - 16, 0);
            st.r[i] = *reinterpret_cast<const v4i*>(B + static_cast<size_t>(k) * N + nn);
        }
    }
    (void)K;
}

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

template <int ELEM>
__device__ __forceinline__ void kn_store(const KNRegs& st, uint8_t* lds_b, int tid) {
    const int nb = tid & 15, kb = tid >> 4;
    // rows k = 8*kb + i (i = 0..7); columns n = 16*nb + j (j = 0..15).
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // 4-column group: bytes 4q..4q+3 of each row word q
        uint32_t lo[4], hi[4];
        t4x4(st.r[0][q], st.r[1][q], st.r[2][q], st.r[3][q], lo[0], lo[1], lo[2], lo[3]);
        t4x4(st.r[4][q], st.r[5][q], st.r[6][q], st.r[7][q], hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int n = nb * 16 + q * 4 + c;
            uint32_t w0 = lo[c], w1 = hi[c];
            if constexpr (ELEM == ELEM_F8) {
                w0 = e4m3_sanitize(w0);
                w1 = e4m3_sanitize(w1);
            }
            const int chunk = (kb >> 1) ^ swz(n);
            uint2* dst = reinterpret_cast<uint2*>(lds_b + n * BK + chunk * 16 + (kb & 1) * 8);
            *dst = make_uint2(w0, w1);
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

// One stage of MFMAs on LDS buffers As (rows of A) / Bs (rows of B^T).
template <int ELEM, int BL>
__device__ __forceinline__ void stage_compute(const uint8_t* As, const uint8_t* Bs,
                                              typename Acc<ELEM>::T (&acc)[4][4], int wm, int wn,
                                              int lane, bool live) {
    const int lr = lane & 31;
    const int lh = lane >> 5;
    if constexpr (ELEM == ELEM_I8) {
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int c = ks * 2 + lh;  // this lane's 16-byte chunk of the 32-byte k step
            v4i a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wm * 128 + i * 32 + lr;
                a[i] = *reinterpret_cast<const v4i*>(As + r * BK + ((c ^ swz(r)) << 4));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = wn * 128 + j * 32 + lr;
                b[j] = *reinterpret_cast<const v4i*>(Bs + r * BK + ((c ^ swz(r)) << 4));
                if (!live) b[j] = v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < BK / 64; ++ks) {
            const int c0 = ks * 4 + lh * 2;  // two 16-byte chunks = 32 k codes per lane
            v8i a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wm * 128 + i * 32 + lr;
                const v4i x = *reinterpret_cast<const v4i*>(As + r * BK + ((c0 ^ swz(r)) << 4));
                const v4i y = *reinterpret_cast<const v4i*>(As + r * BK + (((c0 + 1) ^ swz(r)) << 4));
                a[i] = sanitize8(v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]});
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = wn * 128 + j * 32 + lr;
                const v4i x = *reinterpret_cast<const v4i*>(Bs + r * BK + ((c0 ^ swz(r)) << 4));
                const v4i y = *reinterpret_cast<const v4i*>(Bs + r * BK + (((c0 + 1) ^ swz(r)) << 4));
                b[j] = v8i{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                if constexpr (BL == FKE_B_NK) b[j] = sanitize8(b[j]);  // KN was sanitized at staging
                if (!live) b[j] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        a[i], b[j], acc[i][j], 0, 0, 0, 0, 0, 0);
        }
    }
}

template <int ELEM, int BL, int OUT>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_mfma_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[STAGE_A + STAGE_B];
    __shared__ __attribute__((aligned(1024))) uint8_t lds1[STAGE_A + STAGE_B];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int M = p.M, N = p.N, K = p.K;
    const int gm = (M + BM - 1) / BM, gn = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, gm, gn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int8_t* A = static_cast<const int8_t*>(p.A);
    const int8_t* B = static_cast<const int8_t*>(p.B);

    typename Acc<ELEM>::T acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    const int KT = K / BK;
    KNRegs kn;

    auto issue = [&](int kt, uint8_t* buf) {
        panel_dma(A, K, m0, M, kt * BK, buf, wave, lane);
        if constexpr (BL == FKE_B_NK) {
            panel_dma(B, K, n0, N, kt * BK, buf + STAGE_A, wave, lane);
        } else {
            kn_load(B, N, K, n0, kt * BK, tid, kn);
        }
    };
    auto finish = [&](uint8_t* buf) {
        if constexpr (BL == FKE_B_KN) kn_store<ELEM>(kn, buf + STAGE_A, tid);
        wait_vm0();
        __syncthreads();
    };

    // Two-stage pipeline with static buffer roles (lds0 / lds1 are distinct
    // objects, so the compiler can see that a stage's LDS DMA never aliases the
    // other stage's fragment reads and need not wait on it early).  The body
    // has no data-dependent branches, so the 256 accumulators stay in AGPRs.
    issue(0, lds0);
    finish(lds0);
    int kt = 0;
    // sched_barrier after each issue: without it the scheduler sinks the
    // loads below the stage's MFMAs, so they never overlap with compute.
    for (; kt + 2 < KT; kt += 2) {
        issue(kt + 1, lds1);
        __builtin_amdgcn_sched_barrier(0);
        stage_compute<ELEM, BL>(lds0, lds0 + STAGE_A, acc, wm, wn, lane, true);
        finish(lds1);
        issue(kt + 2, lds0);
        __builtin_amdgcn_sched_barrier(0);
        stage_compute<ELEM, BL>(lds1, lds1 + STAGE_A, acc, wm, wn, lane, true);
        finish(lds0);
    }
    // Tail: one or two stages remain, stage kt is in lds0.  With one left, the
    // lds1 stage re-reads stage kt (a valid address) and its B fragments are
    // zeroed, so it adds nothing.
    issue(min(kt + 1, KT - 1), lds1);
    __builtin_amdgcn_sched_barrier(0);
    stage_compute<ELEM, BL>(lds0, lds0 + STAGE_A, acc, wm, wn, lane, true);
    finish(lds1);
    stage_compute<ELEM, BL>(lds1, lds1 + STAGE_A, acc, wm, wn, lane, kt + 1 < KT);

    // Fused epilogue.  32x32 block layout of the accumulator: lane l holds
    // column l%32 and rows 8*(v/4) + 4*(l/32) + v%4 for v = 0..15.
    const int lr = lane & 31, lh = lane >> 5;
    const float* bias = p.bias;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 128 + j * 32 + lr;
        if (n >= N) continue;
        float sbn;
        if constexpr (ELEM == ELEM_I8) sbn = p.scale_b ? p.scale_b[n] : p.sb;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (m >= M) continue;
                const size_t idx = static_cast<size_t>(m) * N + n;
                if constexpr (ELEM == ELEM_I8) {
                    const int32_t a = acc[i][j][v];
                    const float s = (p.scale_a ? p.scale_a[m] : p.sa) * sbn;
                    store_out<OUT>(p.C, idx, epilogue_value(static_cast<float>(a), s, bias, n), a);
                } else {
                    const float s = p.sa * p.sb;
                    store_out<OUT>(p.C, idx, epilogue_value(acc[i][j][v], s, bias, n), 0);
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
