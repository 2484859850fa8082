/*
 * fke_oracle.h — CPU restatement of flash-kernel-engine's quantized GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links or calls this
 * code; it is the checker used by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py.  Every function names the reference file:line
 * it restates (paths relative to the reference repository root).
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   fko_ref_host_gemm_i8      KAT64 golden values from the reference test's
 *                             closed-form inputs; brute force vs double math.
 *   fko_ref_kernel_gemm_i8    equals fko_ref_host_gemm_i8 for K%4==0 (closed
 *                             form); K%4!=0 truncation/misalignment by a
 *                             hand-derived tiny case.
 *   fko_e4m3_decode           exhaustive 256-code table vs the OCP E4M3 closed
 *                             form (exact powers of two) incl. 0x7F/0xFF -> 0.
 *   fko_ref_kernel_gemm_f8    brute force with exact (double) products, order
 *                             check against a hand-computed rounding case.
 *   fko_ref_py_gemm_i8        numpy int32 matmul closed form.
 *   fko_w8a8_*                reduction to the reference when scales are
 *                             uniform / bias absent / fp32 out; bf16 RNE known
 *                             answers; exact-integer checksums.
 *   generators                fixed known-answer streams (SplitMix64 KAT).
 *   fko_quantize_rows_i8      hand-derived rows (ties to even, exact scales),
 *                             invariants (the amax element maps to +-127,
 *                             |q*s - x| <= s/2), brute force in exact rationals.
 *   fko_swiglu1 / _f32        the reference test's vector (python/tests/
 *                             test_correctness.py:166-176), float64 closed
 *                             form over a sweep, silu(g) - silu(-g) = g,
 *                             exact special values (g = 0, saturation).
 *   fko_w8a8_swiglu           equals fko_w8a8_gemm on the gate rows and on the
 *                             up rows followed by fko_swiglu_f32, bit for bit.
 *   fko_f16_to_f32            exhaustive 65536 codes vs numpy's float16 cast.
 *   fko_gemm_half             exact small-integer products vs int64 matmul;
 *                             float64 matmul within the sequential-sum error
 *                             bound; a hand case whose value depends on the
 *                             summation order (pins k ascending).
 */
#ifndef FKE_ORACLE_H
#define FKE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded generators (synthetic inputs; no reference counterpart) ---- */
uint64_t fko_splitmix64(uint64_t* state);
void fko_gen_i8_uniform(int8_t* dst, size_t n, uint64_t seed);            /* (u%255)-127        */
void fko_gen_i8_clipped_normal(int8_t* dst, size_t n, uint64_t seed,
                               double sigma);                              /* clamp(rint(s*z))   */
void fko_gen_f32_uniform(float* dst, size_t n, uint64_t seed, double lo, double hi);
void fko_gen_f32_normal(float* dst, size_t n, uint64_t seed, double mu, double sigma);

/* ---- reference restatements ---- */
/* tests/test_quantized_gemm.cu:39-48 — full-K int32 triple loop, B is [N,K]. */
void fko_ref_host_gemm_i8(const int8_t* A, const int8_t* B, float* C,
                          int M, int N, int K, float scale_a, float scale_b);
/* src/quantized_gemm.cu:15-54,68 — the device kernel's arithmetic, including
 * its K/4 word truncation and int32 row reinterpretation. */
void fko_ref_kernel_gemm_i8(const int8_t* A, const int8_t* B, float* C,
                            int M, int N, int K, float scale_a, float scale_b);
/* src/quantized_gemm.cu:81-97 */
float fko_e4m3_decode(uint8_t x);
/* src/quantized_gemm.cu:99-118,132 — sequential-k fp32 sum, B is [K,N]. */
void fko_ref_kernel_gemm_f8(const uint8_t* A, const uint8_t* B, float* C,
                            int M, int N, int K, float scale_a, float scale_b);
/* python/flash_engine/ops.py:180-186 — B is [K,N]; scale product in double. */
void fko_ref_py_gemm_i8(const int8_t* A, const int8_t* B, float* C,
                        int M, int N, int K, double scale_a, double scale_b);

/* ---- extended W8A8 path (per-token x per-channel scales, bias, out dtype) ---- */
enum { FKO_OUT_F32 = 0, FKO_OUT_BF16 = 1, FKO_OUT_I32 = 2 };
enum { FKO_B_NK = 0, FKO_B_KN = 1 };

/* exact int32 accumulators acc[m,n] = sum_k A[m,k]*B(n,k) for the listed rows
 * (rows==NULL -> all M rows, nrows ignored).  acc is [nrows or M, N]. */
void fko_w8a8_acc(const int8_t* A, const int8_t* B, int32_t* acc,
                  int M, int N, int K, int b_layout,
                  const int* rows, int nrows, int nthreads);
/* canonical epilogue: s = fp32(sa_m*sb_n); y = bias ? fmaf(fp32(acc),s,bias_n)
 * : fp32(acc)*s; out = y (f32) | bf16_rne(y) | acc (i32).  scale_a/scale_b may
 * be NULL (then the scalars sa/sb are used for every row/column). `rows`
 * maps acc row r to problem row rows[r] for scale_a lookup (NULL: identity). */
void fko_w8a8_epilogue(const int32_t* acc, void* out, int R, int N,
                       const float* scale_a, const float* scale_b, float sa, float sb,
                       const float* bias, int out_dtype, const int* rows);
/* fp8 with the same epilogue over the reference's sequential fp32 sum:
 * y = sum*fp32(sa*sb) (+bias via fmaf), out f32|bf16. */
void fko_f8_gemm(const uint8_t* A, const uint8_t* B, void* out, int M, int N, int K,
                 float sa, float sb, const float* bias, int out_dtype, int b_layout,
                 const int* rows, int nrows, int nthreads);

uint16_t fko_f32_to_bf16_rne(float x);
float fko_bf16_to_f32(uint16_t h);
/* saturating round-to-nearest-even fp32 -> OCP E4M3 (never emits 0x7F/0xFF) */
uint8_t fko_f32_to_e4m3_sat(float x);
/* per-tensor quantiser of the FP8 config: s = amax/448, q = e4m3_sat(x/s). */
float fko_quantize_e4m3(const float* x, uint8_t* q, size_t n);
/* per-token INT8 activation quantiser (no reference counterpart; the step in
 * front of the W8A8 GEMM): per row m, amax = max|x| over non-NaN elements,
 * s = fp32(amax/127), f = 2^64 if amax < 2^-64 else 1, r = fp32(127/(amax*f))
 * (s = r = 1 when amax == 0), p = fp32(fp32(x*f)*r),
 * q = NaN(p) ? 0 : clamp(rne(p), -127, 127); scale[m] = s.
 * x is fp32 (in_dtype 0) or bf16 bits (in_dtype 1), [M,K]. */
void fko_quantize_rows_i8(const void* x, int in_dtype, int M, int K, int8_t* q, float* scale);

/* IEEE binary16 -> fp32 (exact): e = 0 -> m * 2^-24; e = 31 -> inf / NaN;
 * else (1 + m/1024) * 2^(e-15).  The operand type of the reference's WMMA
 * GEMM (src/tensor_core_attention.cu:13-18, half). */
float fko_f16_to_f32(uint16_t h);
/* fp16 / bf16 GEMM (extends src/tensor_core_attention.cu:13-66, which
 * accumulates fp16 products into fp32 with alpha applied at the end):
 * acc = sum over k = 0..K-1, in order, of the exact fp32 products; then the
 * W8A8 canonical epilogue (s = fp32(sa_m*sb_n), fmaf with bias) and f32 /
 * bf16 output.  A, B are raw 16-bit codes; in_dtype 2 = fp16, 1 = bf16. */
void fko_gemm_half(const uint16_t* A, const uint16_t* B, void* out, int M, int N, int K, int in_dtype,
                   const float* scale_a, const float* scale_b, float sa, float sb, const float* bias,
                   int out_dtype, int b_layout, const int* rows, int nrows, int nthreads);

/* SwiGLU of one pair, src/fused_activations.cu:9-11,30-33:
 * (g * sigmoid(g)) * u with sigmoid(g) = 1 / (1 + exp(-g)), fp32, in that
 * order (the reference's __expf is a fast approximation; here expf and the
 * division are the C library's / IEEE, so this is the function's value within
 * about one ulp). */
float fko_swiglu1(float g, float u);
/* elementwise over n fp32 pairs (src/fused_activations.cu:17-83) */
void fko_swiglu_f32(const float* g, const float* u, float* h, size_t n);
/* W8A8 gate/up GEMM with SwiGLU (no reference counterpart as one call): W is
 * [2I, K] (rows 0..I-1 gate, I..2I-1 up); g, u = canonical epilogue values of
 * rows n and I+n (scale_b / bias indexed the same way, [2I] or NULL);
 * out[r, n] = fko_swiglu1(g, u) as f32 or bf16_rne, [nrows or M, I]. */
void fko_w8a8_swiglu(const int8_t* A, const int8_t* W, void* out, int M, int I, int K,
                     const float* scale_a, const float* scale_b, float sa, float sb,
                     const float* bias, int out_dtype, const int* rows, int nrows, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
