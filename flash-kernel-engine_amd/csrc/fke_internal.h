// fke_internal.h — shared definitions of the gfx950 quantized GEMM kernels.
//
// Device code here is written for CDNA4 (gfx950) only: 64-lane wavefronts,
// MFMA matrix cores, 160 KiB of LDS per CU.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fke_qgemm.h"

namespace fke {

// Arguments of one GEMM call, passed by value to every kernel.
struct GemmArgs {
    const void* A;        // [M,K] int8 / e4m3 codes
    const void* B;        // [N,K] (NK) or [K,N] (KN)
    void* C;              // [M,N] fp32 / bf16 / int32
    int M, N, K;
    const float* scale_a; // [M] or null (then sa)
    const float* scale_b; // [N] or null (then sb)
    float sa, sb;
    const float* bias;    // [N] or null
    int out_dtype;        // FKE_OUT_*
    int b_layout;         // FKE_B_*
    int swiglu;           // 1: B is [gate; up] (N = 2I rows, NK), C is [M, I] = SwiGLU of the pairs
};

// Operand element types.  ELEM_F16 / ELEM_BF16: GemmArgs::K counts elements
// at the C ABI; the MFMA kernel works on K bytes (2K).
enum Elem { ELEM_I8 = 0, ELEM_F8 = 1, ELEM_F16 = 2, ELEM_BF16 = 3 };
constexpr int elem_bytes(int elem) { return elem >= ELEM_F16 ? 2 : 1; }

// Launchers (return this launch's status; arguments already validated).
hipError_t launch_generic(const GemmArgs& p, int elem, hipStream_t stream);
// INT8 / FP8 on the matrix cores with K % 4 == 0, 4-byte-aligned A / B and,
// for B [K,N], N % 4 == 0 (the shapes the MFMA GEMM's 16-byte copies cannot
// take); the SwiGLU GEMM too (INT8, B [N,K], float out).
bool words_supports(const GemmArgs& p, int elem);
hipError_t launch_words(const GemmArgs& p, int elem, hipStream_t stream);
hipError_t launch_gemv_i8(const GemmArgs& p, hipStream_t stream);
// MFMA GEMM workgroup tile: AUTO = chosen by tile count (mfma_pick_tile).
enum MfmaTile {
    MFMA_TILE_AUTO = 0,
    MFMA_TILE_256x256 = 1,
    MFMA_TILE_128x128 = 2,
    MFMA_TILE_128x128_RING4 = 3,
    MFMA_TILE_128x64_RING4 = 4,  // not for SwiGLU
    MFMA_TILE_64x64_RING4 = 5    // not for SwiGLU
};
// K split of the MFMA GEMM: S ranges of KS stages (128 K bytes each); split s
// writes its raw sums (int32 for INT8, fp32 for FP8) to part[s][M][N], and a
// second kernel adds the S sums of each output in the order s = 0..S-1 and
// applies the epilogue.  S = 1: no split, the fused epilogue.
struct SplitK {
    int S = 1;
    int KS = 0;
    void* part = nullptr;
};
// Tile and K split the MFMA GEMM runs with on `cus` CUs (S = 1: none).
struct MfmaPlan {
    int tile;
    int S;
    int KS;
};
MfmaPlan mfma_plan(const GemmArgs& p, int elem, int cus);
// Bytes of the partial sums of an S-way split (S * M * N * 4).
size_t mfma_split_bytes(const GemmArgs& p, int S);
hipError_t launch_mfma(const GemmArgs& p, int elem, hipStream_t stream, int tile = MFMA_TILE_AUTO,
                       const SplitK& sk = SplitK{});
int mfma_pick_tile(const GemmArgs& p, int cus);
// Estimated time (us) of the MFMA GEMM on an 8-bit B [N,K] shape.
double mfma_time_estimate_us(const GemmArgs& p, int cus);
// CUs of the current device (256 without one).
int device_cus();
hipError_t launch_quant_rows(const void* X, int in_dtype, int M, int K, int8_t* Q, float* S,
                             hipStream_t stream);
hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype,
                         hipStream_t stream);

// Largest batch the decode family takes: past 16 rows only its LDS-streamed
// kernel, 64 activation rows per workgroup and more workgroups beyond that.
constexpr int FKE_GEMV_MAX_M = 512;

// Shape/alignment predicates of the fast families (host side).
bool gemv_i8_supports(const GemmArgs& p);
bool gemv_i8_batch_pays(const GemmArgs& p);  // M > 16: the decode family beats the MFMA GEMM
bool gemv_f8_supports(const GemmArgs& p);
hipError_t launch_gemv_f8(const GemmArgs& p, hipStream_t stream);
bool mfma_supports(const GemmArgs& p, int elem);
// The VALU dot-product decode kernels (no MFMA), M <= 16, INT8, B [N,K].
bool gemv_dot_supports(const GemmArgs& p);
hipError_t launch_gemv_dot(const GemmArgs& p, hipStream_t stream);
// Decode (M <= 16) with B stored [K,N], INT8 or FP8 (gemv_kn.hip): with a
// workspace for partial sums, S K splits of 128- to 512-column workgroups
// (M = 1: 1024-column workgroups of the row kernel) and a second kernel that
// adds the splits; without one (S = 1), one workgroup per 64-column block over
// all of K.
struct KnSplit {
    int S;       // K splits (1: no workspace)
    int PS;      // 128-row pieces per split
    void* part;  // [ceil(N/128)][S][M][128] partial sums (int32 / fp32)
    int rowk;    // 1: the row kernel writes them (1024-column workgroups), 0: the split kernel
    int kw;      // the split kernel's waves per workgroup (1, 2 or 4 blocks of 128 columns)
    int dw;      // 1: 4-byte loads (the row kernel's form for operands the 16-byte loads cannot take)
};
bool gemv_kn_supports(const GemmArgs& p, int elem);
// Whether the MFMA GEMM should take the shape where it can: past 4 rows with
// 4-byte operands (the row kernel streams the weights once per 4 rows).
bool gemv_kn_yields_to_mfma(const GemmArgs& p);
size_t gemv_kn_workspace_bytes(const GemmArgs& p);  // 0: runs unsplit
KnSplit gemv_kn_plan(const GemmArgs& p, void* ws, size_t ws_bytes);
// Whether the plan has a kernel (past 16 rows, or with 4-byte operands, the decode needs its workspace).
bool gemv_kn_plan_runs(const GemmArgs& p, const KnSplit& sp);
hipError_t launch_gemv_kn(const GemmArgs& p, int elem, const KnSplit& sp, hipStream_t stream);

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

// fp32 -> bf16 bits, round to nearest even; a NaN keeps its sign and upper
// payload bits and is made quiet (((bits >> 16) | 0x40)).  gfx950 converts in
// one instruction (v_cvt_pk_bf16_f32, two values at a time), which was checked
// against that definition, computed in software, on 2.2 M fp32 bit patterns
// (random, every NaN class of either sign, infinities, denormals, ties): every
// result identical.  The software form branched on the NaN test for every
// element of a bf16 epilogue.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float y) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(y));
}

// E4M3 code -> fp32 following reference src/quantized_gemm.cu:81-97, built
// from IEEE bits: exp==0 -> m*2^-9; 0x7F/0xFF -> +0.0; else
// (1+m/8)*2^(e-7), i.e. fp32 exponent field e+120 and mantissa m<<20.
__device__ __forceinline__ float e4m3_decode(uint32_t x) {
    const uint32_t e = (x >> 3) & 0xFu;
    const uint32_t m = x & 7u;
    float v;
    if (e == 0) {
        v = static_cast<float>(m) * 0.001953125f;
    } else if (e == 15 && m == 7) {
        return 0.0f;
    } else {
        v = __uint_as_float(((e + 120u) << 23) | (m << 20));
    }
    return (x & 0x80u) ? -v : v;
}

// Replace every 0x7F / 0xFF byte of a packed word by 0x00, so that the MFMA
// (which reads those codes as NaN) sees the reference's 0.0.
// (w & 0x7F..) + 0x01.. sets bit 7 of a byte exactly when its low 7 bits are
// all ones (no carry can cross bytes); that bit, moved to bit 2, turns the
// byte's v_perm selector i into 4+i, which selects a byte of the zero operand.
__device__ __forceinline__ uint32_t e4m3_sanitize(uint32_t w) {
    const uint32_t hi = (w & 0x7F7F7F7Fu) + 0x01010101u;
    const uint32_t sel = ((hi >> 5) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(0u, w, sel);
}

typedef float v2f __attribute__((ext_vector_type(2)));

// E4M3 codes -> fp32 with gfx950's v_cvt_pk_f32_fp8 (two codes per
// instruction; checked against the reference's decode, src/quantized_gemm.cu:
// 81-97, on all 256 codes: identical, except 0x7F / 0xFF, which it turns into
// NaN where the reference reads 0.0 - see e4m3_sanitize).  16 codes of one
// 16-byte chunk (a vector of four 32-bit words), in byte order.
template <typename V4>
__device__ __forceinline__ void e4m3_chunk_to_f32(V4 c, float (&f)[16]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8(c[e], false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(c[e], true);
        f[4 * e] = lo.x;
        f[4 * e + 1] = lo.y;
        f[4 * e + 2] = hi.x;
        f[4 * e + 3] = hi.y;
    }
}

// Canonical fused epilogue: s = fp32(sa_m*sb_n); y = bias ? fma(v,s,bias) : v*s.
__device__ __forceinline__ float epilogue_value(float v, float s, const float* bias, int n) {
    return bias ? __builtin_fmaf(v, s, bias[n]) : v * s;
}

// SwiGLU of one (gate, up) pair: (g * sigmoid(g)) * u with sigmoid(g) =
// 1 / (1 + exp(-g)), in that order (reference src/fused_activations.cu:9-11,
// :30-33).  exp is the device library's expf (within 1 ulp; the reference
// uses the fast __expf) and the reciprocal is v_rcp_f32 (1 ulp).  exp(-g)
// overflows to +inf for g < -88.7, which gives sigmoid = 0 and h = +-0.
__device__ __forceinline__ float swiglu_pair(float g, float u) {
    const float s = __builtin_amdgcn_rcpf(1.0f + expf(-g));
    return (g * s) * u;
}

// ---- memory-pipeline helpers shared by the LDS-staged kernels ----

// s_waitcnt vmcnt(N) with the other counters unconstrained (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_vm0() { wait_vm<0>(); }
// s_waitcnt lgkmcnt(0), the other counters unconstrained.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier without the LDS fence of __syncthreads: every LDS write a
// stage depends on comes from LDS-DMA (ordered by an explicit vmcnt wait
// before the barrier) or from ds_writes followed by an explicit lgkmcnt wait.
// The empty asm statements keep the compiler from moving memory operations
// across the barrier.
__device__ __forceinline__ void barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// Buffer resource over `bytes` bytes at `base` (raw buffer: stride 0, bounds
// checked against num_records; gfx9 dword3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// 16 bytes per lane, buffer -> LDS (buffer_load_dwordx4 ... lds): lane l's
// bytes land at lds + 16*l.  The MUBUF form rather than global_load_lds: the
// compiler treats a FLAT-encoded LDS DMA as a pending access of both memory
// kinds and then waits for every outstanding LDS read (lgkmcnt(0)) wherever
// one result is needed, which would serialise the fragment reads.
// aux = 2 marks the load non-temporal (a stream read once).
template <int AUX = 0>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff, uint8_t* l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(l)), 16,
        static_cast<int>(voff), soff, 0, AUX);
}
// 4 bytes per lane, buffer -> LDS (buffer_load_dword ... lds): lane l's word
// lands at lds + 4*l.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff, void* l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(l)), 4,
        static_cast<int>(voff), soff, 0, 0);
}

// ---- per-token INT8 quantisation (quant_i8.hip) ----

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 1));
    v = fmaxf(v, __shfl_xor(v, 2));
    v = fmaxf(v, __shfl_xor(v, 4));
    v = fmaxf(v, __shfl_xor(v, 8));
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

// Row scale s (stored / applied in the epilogue), the reciprocal r applied to
// the elements, and the power of two f the elements are multiplied by first:
//   amax == 0: s = r = f = 1
//   otherwise: s = fp32(amax/127), f = 2^64 if amax < 2^-64 else 1,
//              r = fp32(127/(amax*f))
// f keeps r finite for rows whose maximum is below 127/FLT_MAX (x*f and
// amax*f are exact); wherever 127/amax is finite the codes equal those of
// f = 1.  amax = +inf gives s = inf, r = 0.
struct RowScale {
    float s, r, f;
};
__device__ __forceinline__ RowScale scale_of(float amax) {
    if (amax == 0.0f) return {1.0f, 1.0f, 1.0f};
    const float f = amax < 0x1p-64f ? 0x1p64f : 1.0f;
    return {amax / 127.0f, 127.0f / (amax * f), f};
}

// Code of x (already multiplied by the row's f), clamp(rne(fp32(x * r)),
// -127, 127), in the low byte of the result, in a few VALU operations: the
// product p is finite or NaN (|x| <= amax*f and r = fp32(127/(amax*f)), or
// r = 0 for an infinite amax), and a finite |p| <= 127*(1+2^-23) < 2^22, so
// adding 1.5*2^23 (a separate, correctly rounded fp32 add - the product is
// rounded first) rounds p to an integer half to even and leaves it, two's
// complement, in the low mantissa bits; it never reaches +-128, so no clamp
// is needed.  A NaN product (NaN x, or inf * 0) selects 0.
__device__ __forceinline__ uint32_t q8_bits(float x, float r) {
#pragma clang fp contract(off)  // the product must be rounded before the add
    const float p = x * r;
    const uint32_t t = __float_as_uint(p + 12582912.0f);
    return p != p ? 0u : t;
}

// Low bytes of t0..t3 -> bytes 0..3 of one word.
__device__ __forceinline__ uint32_t pack_q8(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    return __builtin_amdgcn_perm(__builtin_amdgcn_perm(t3, t2, 0x0C0C0400u), __builtin_amdgcn_perm(t1, t0, 0x0C0C0400u),
                                 0x05040100u);
}

template <int OUT>
__device__ __forceinline__ void store_out(void* C, size_t idx, float y, int32_t acc) {
    if constexpr (OUT == FKE_OUT_F32) {
        static_cast<float*>(C)[idx] = y;
    } else if constexpr (OUT == FKE_OUT_BF16) {
        static_cast<uint16_t*>(C)[idx] = f32_to_bf16_rne(y);
    } else {
        static_cast<int32_t*>(C)[idx] = acc;
    }
}

}  // namespace fke
