/*
 * fke_oracle.c — CPU restatement of flash-kernel-engine's quantized GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg.  It is never linked into or called by the
 * shipped library.  Built with -O3 -ffp-contract=off so every fp32 operation
 * rounds exactly once, as written.  Reference paths are relative to the
 * flash-kernel-engine repository root.
 */
#include "fke_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Generators                                                                */
/* ------------------------------------------------------------------------- */

/* SplitMix64 (Steele, Lea, Flood 2014), the public 64-bit mixing generator. */
uint64_t fko_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double u01_open0(uint64_t u) { return (double)((u >> 11) + 1) * 0x1.0p-53; } /* (0,1] */
static double u01(uint64_t u) { return (double)(u >> 11) * 0x1.0p-53; }            /* [0,1) */

void fko_gen_i8_uniform(int8_t* dst, size_t n, uint64_t seed) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) dst[i] = (int8_t)((int)(fko_splitmix64(&s) % 255u) - 127);
}

/* Box-Muller, cosine branch only: z = sqrt(-2 ln u1) cos(2 pi u2). */
static double next_normal(uint64_t* s) {
    double u1 = u01_open0(fko_splitmix64(s));
    double u2 = u01(fko_splitmix64(s));
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
}

void fko_gen_i8_clipped_normal(int8_t* dst, size_t n, uint64_t seed, double sigma) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        double v = rint(sigma * next_normal(&s)); /* round half to even */
        if (v > 127.0) v = 127.0;
        if (v < -127.0) v = -127.0;
        dst[i] = (int8_t)v;
    }
}

void fko_gen_f32_uniform(float* dst, size_t n, uint64_t seed, double lo, double hi) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) dst[i] = (float)(lo + (hi - lo) * u01(fko_splitmix64(&s)));
}

void fko_gen_f32_normal(float* dst, size_t n, uint64_t seed, double mu, double sigma) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) dst[i] = (float)(mu + sigma * next_normal(&s));
}

/* ------------------------------------------------------------------------- */
/* Reference restatements                                                    */
/* ------------------------------------------------------------------------- */

/* tests/test_quantized_gemm.cu:39-48: int32 acc over the full K, B row n at
 * B[n*K + k]; h_ref = float(acc) * (scale_a * scale_b) with the product taken
 * in fp32. */
void fko_ref_host_gemm_i8(const int8_t* A, const int8_t* B, float* C,
                          int M, int N, int K, float scale_a, float scale_b) {
    const float alpha = scale_a * scale_b;
    for (int m = 0; m < M; ++m) {
        for (int n = 0; n < N; ++n) {
            int32_t acc = 0;
            for (int k = 0; k < K; ++k)
                acc += (int32_t)A[(size_t)m * K + k] * (int32_t)B[(size_t)n * K + k];
            C[(size_t)m * N + n] = (float)acc * alpha;
        }
    }
}

/* One __dp4a: four signed byte products added to acc (wrapping int32). */
static int32_t dp4a_s8(uint32_t a, uint32_t b, int32_t acc) {
    uint32_t r = (uint32_t)acc;
    for (int i = 0; i < 4; ++i) {
        int32_t x = (int8_t)(a >> (8 * i));
        int32_t y = (int8_t)(b >> (8 * i));
        r += (uint32_t)(x * y);
    }
    return (int32_t)r;
}

static uint32_t load_word(const int8_t* p) {
    uint32_t w;
    memcpy(&w, p, 4); /* little-endian int32 reinterpretation, as on the GPU */
    return w;
}

/* src/quantized_gemm.cu:22-52 and :68: k_packed = K/4 words per row; row r of A
 * starts at word r*k_packed (byte 4*r*(K/4)), column c of B at word c*k_packed;
 * acc += dp4a(...) for k < K/4; C = float(acc) * alpha, alpha = sa*sb (fp32). */
void fko_ref_kernel_gemm_i8(const int8_t* A, const int8_t* B, float* C,
                            int M, int N, int K, float scale_a, float scale_b) {
    const float alpha = scale_a * scale_b;
    const int kp = K / 4;
    for (int row = 0; row < M; ++row) {
        for (int col = 0; col < N; ++col) {
            int32_t acc = 0;
            for (int k = 0; k < kp; ++k) {
                uint32_t a = load_word(A + 4 * ((size_t)row * kp + k));
                uint32_t b = load_word(B + 4 * ((size_t)col * kp + k));
                acc = dp4a_s8(a, b, acc);
            }
            C[(size_t)row * N + col] = (float)acc * alpha;
        }
    }
}

/* src/quantized_gemm.cu:81-97, with exact powers of two:
 *   exp==0            -> mant/8 * 2^-6           (subnormal)
 *   exp==15 && mant==7 -> 0.0                    (0x7F / 0xFF: the reference's
 *                                                 NaN clamp, not OCP NaN)
 *   otherwise         -> (1 + mant/8) * 2^(exp-7)                             */
float fko_e4m3_decode(uint8_t x) {
    int sign = (x >> 7) & 1;
    int e = (x >> 3) & 0xF;
    int m = x & 7;
    float v;
    if (e == 0) {
        v = (float)m / 8.0f * (1.0f / 64.0f);
    } else if (e == 15 && m == 7) {
        return 0.0f;
    } else {
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    }
    return sign ? -v : v;
}

/* src/quantized_gemm.cu:106-116 and :132: sum over k = 0..K-1 in order of
 * dec(A[row*K+k]) * dec(B[k*N+col]) in fp32, C = sum * (sa*sb). */
void fko_ref_kernel_gemm_f8(const uint8_t* A, const uint8_t* B, float* C,
                            int M, int N, int K, float scale_a, float scale_b) {
    const float alpha = scale_a * scale_b;
    for (int row = 0; row < M; ++row) {
        for (int col = 0; col < N; ++col) {
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) {
                float a = fko_e4m3_decode(A[(size_t)row * K + k]);
                float b = fko_e4m3_decode(B[(size_t)k * N + col]);
                sum += a * b; /* each product is exact in fp32 */
            }
            C[(size_t)row * N + col] = sum * alpha;
        }
    }
}

/* python/flash_engine/ops.py:180-186: int32(A) @ int32(B) with B [K,N], then
 * .astype(float32) * (scale_a*scale_b): the scale product is a Python float
 * (double), which numpy (NEP 50) casts to float32 before the multiply. */
void fko_ref_py_gemm_i8(const int8_t* A, const int8_t* B, float* C,
                        int M, int N, int K, double scale_a, double scale_b) {
    const float alpha = (float)(scale_a * scale_b);
    for (int m = 0; m < M; ++m) {
        for (int n = 0; n < N; ++n) {
            uint32_t acc = 0;
            for (int k = 0; k < K; ++k)
                acc += (uint32_t)((int32_t)A[(size_t)m * K + k] * (int32_t)B[(size_t)k * N + n]);
            C[(size_t)m * N + n] = (float)(int32_t)acc * alpha;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Extended W8A8 path                                                        */
/* ------------------------------------------------------------------------- */

void fko_w8a8_acc(const int8_t* A, const int8_t* B, int32_t* acc,
                  int M, int N, int K, int b_layout,
                  const int* rows, int nrows, int nthreads) {
    const int R = rows ? nrows : M;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int r = 0; r < R; ++r) {
        const int m = rows ? rows[r] : r;
        const int8_t* a = A + (size_t)m * K;
        int32_t* out = acc + (size_t)r * N;
        if (b_layout == FKO_B_NK) {
            for (int n = 0; n < N; ++n) {
                const int8_t* b = B + (size_t)n * K;
                int32_t s = 0;
                for (int k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
                out[n] = s;
            }
        } else {
            for (int n = 0; n < N; ++n) out[n] = 0;
            for (int k = 0; k < K; ++k) {
                const int32_t av = a[k];
                const int8_t* b = B + (size_t)k * N;
                for (int n = 0; n < N; ++n) out[n] += av * (int32_t)b[n];
            }
        }
    }
}

uint16_t fko_f32_to_bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float fko_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float epi(float v, float s, const float* bias, int n) {
    return bias ? fmaf(v, s, bias[n]) : v * s;
}

static void store_out(void* out, size_t idx, int out_dtype, float y, int32_t acc) {
    if (out_dtype == FKO_OUT_F32) ((float*)out)[idx] = y;
    else if (out_dtype == FKO_OUT_BF16) ((uint16_t*)out)[idx] = fko_f32_to_bf16_rne(y);
    else ((int32_t*)out)[idx] = acc;
}

void fko_w8a8_epilogue(const int32_t* acc, void* out, int R, int N,
                       const float* scale_a, const float* scale_b, float sa, float sb,
                       const float* bias, int out_dtype, const int* rows) {
    for (int r = 0; r < R; ++r) {
        const int m = rows ? rows[r] : r;
        const float am = scale_a ? scale_a[m] : sa;
        for (int n = 0; n < N; ++n) {
            const size_t i = (size_t)r * N + n;
            const float s = am * (scale_b ? scale_b[n] : sb);
            store_out(out, i, out_dtype, epi((float)acc[i], s, bias, n), acc[i]);
        }
    }
}

void fko_f8_gemm(const uint8_t* A, const uint8_t* B, void* out, int M, int N, int K,
                 float sa, float sb, const float* bias, int out_dtype, int b_layout,
                 const int* rows, int nrows, int nthreads) {
    const int R = rows ? nrows : M;
    const float alpha = sa * sb;
    float dec[256];
    for (int i = 0; i < 256; ++i) dec[i] = fko_e4m3_decode((uint8_t)i);
    if (nthreads < 1) nthreads = 1;
    if (b_layout == FKO_B_KN) {
        /* B decoded once; rows in blocks of RB, k outer and n inner, so each
         * decoded B row serves RB rows from cache.  Every sums[i][n] still
         * adds k = 0..K-1 in order, one product and one sum per step. */
        enum { RB = 8 };
        float* bf = (float*)malloc(sizeof(float) * (size_t)K * N);
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (int k = 0; k < K; ++k)
            for (int n = 0; n < N; ++n) bf[(size_t)k * N + n] = dec[B[(size_t)k * N + n]];
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
        for (int r0 = 0; r0 < R; r0 += RB) {
            const int nr = R - r0 < RB ? R - r0 : RB;
            float* sums = (float*)malloc(sizeof(float) * (size_t)RB * N);
            for (size_t i = 0; i < (size_t)RB * N; ++i) sums[i] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float* b = bf + (size_t)k * N;
                for (int i = 0; i < nr; ++i) {
                    const int m = rows ? rows[r0 + i] : r0 + i;
                    const float av = dec[A[(size_t)m * K + k]];
                    float* s = sums + (size_t)i * N;
                    for (int n = 0; n < N; ++n) s[n] += av * b[n];
                }
            }
            for (int i = 0; i < nr; ++i)
                for (int n = 0; n < N; ++n)
                    store_out(out, (size_t)(r0 + i) * N + n, out_dtype, epi(sums[(size_t)i * N + n], alpha, bias, n),
                              0);
            free(sums);
        }
        free(bf);
        return;
    }
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int r = 0; r < R; ++r) {
        const int m = rows ? rows[r] : r;
        const uint8_t* a = A + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const uint8_t* b = B + (size_t)n * K;
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) sum += dec[a[k]] * dec[b[k]];
            store_out(out, (size_t)r * N + n, out_dtype, epi(sum, alpha, bias, n), 0);
        }
    }
}

/* Saturating RNE quantiser to OCP E4M3 (bias 7, max finite 448 = 0x7E).
 * All steps are exact in double: |x| is an fp32 value, scalings are by powers
 * of two and nearbyint rounds half to even in the default rounding mode. */
uint8_t fko_f32_to_e4m3_sat(float x) {
    if (x != x) return 0x00; /* NaN input: no NaN output from this quantiser */
    uint8_t sign = signbit(x) ? 0x80 : 0x00;
    double a = fabs((double)x);
    if (a >= 448.0) return sign | 0x7E;
    if (a < 0x1.0p-6) { /* subnormal range: step 2^-9, m in 0..8 (8 == min normal) */
        int m = (int)nearbyint(a * 512.0);
        return sign | (uint8_t)m;
    }
    int e2;
    double fr = frexp(a, &e2); /* a = fr * 2^e2, fr in [0.5,1) */
    int e = e2 - 1;            /* a = (2*fr) * 2^e, 2*fr in [1,2) */
    int m = (int)nearbyint((2.0 * fr - 1.0) * 8.0);
    if (m == 8) { m = 0; e += 1; }
    int be = e + 7;
    if (be > 15 || (be == 15 && m == 7)) return sign | 0x7E;
    return sign | (uint8_t)((be << 3) | m);
}

float fko_quantize_e4m3(const float* x, uint8_t* q, size_t n) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float v = fabsf(x[i]);
        if (v > amax) amax = v;
    }
    float s = amax / 448.0f;
    if (s == 0.0f) s = 1.0f;
    for (size_t i = 0; i < n; ++i) q[i] = fko_f32_to_e4m3_sat(x[i] / s);
    return s;
}

/* Per-token INT8 quantiser (no reference counterpart).  fp32 arithmetic as the
 * kernel does it: the scale and its reciprocal are single correctly rounded
 * fp32 divisions, each code one fp32 product (the file is built with
 * -ffp-contract=off); nearbyintf rounds half to even in the default mode.
 *   amax = max |x| over the row's non-NaN elements (+inf included)
 *   amax == 0:  s = r = 1, f = 1
 *   otherwise:  s = fp32(amax / 127); f = 2^64 if amax < 2^-64 else 1;
 *               r = fp32(127 / (amax * f))
 *   p = fp32(fp32(x * f) * r);  q = NaN(p) ? 0 : clamp(rne(p), -127, 127)
 * f keeps 127/amax finite for rows whose maximum is below 127/FLT_MAX: x * f
 * and amax * f are exact (a power of two, no overflow), and for every row
 * where 127/amax is finite the result equals that of f = 1.  A row holding
 * +-inf has s = inf and r = 0, so every code is 0 (inf * 0 is NaN); NaN
 * elements give 0. */
void fko_quantize_rows_i8(const void* x, int in_dtype, int M, int K, int8_t* q, float* scale) {
    for (int m = 0; m < M; ++m) {
        float amax = 0.0f;
        for (int k = 0; k < K; ++k) {
            const size_t i = (size_t)m * K + k;
            const float v = in_dtype == 0 ? ((const float*)x)[i] : fko_bf16_to_f32(((const uint16_t*)x)[i]);
            const float a = fabsf(v);
            if (a > amax) amax = a;
        }
        const float f = (amax > 0.0f && amax < 0x1p-64f) ? 0x1p64f : 1.0f;
        const float s = amax == 0.0f ? 1.0f : amax / 127.0f;
        const float r = amax == 0.0f ? 1.0f : 127.0f / (amax * f);
        scale[m] = s;
        for (int k = 0; k < K; ++k) {
            const size_t i = (size_t)m * K + k;
            const float v = in_dtype == 0 ? ((const float*)x)[i] : fko_bf16_to_f32(((const uint16_t*)x)[i]);
            const float p = (v * f) * r;
            if (p != p) { q[i] = 0; continue; }
            float t = nearbyintf(p);
            if (t > 127.0f) t = 127.0f;
            if (t < -127.0f) t = -127.0f;
            q[i] = (int8_t)t;
        }
    }
}

/* src/fused_activations.cu:9-11 (fast_sigmoid) and :30-33 / :48 (the pair).
 * Built with -ffp-contract=off: every operation rounds once, as written. */
float fko_swiglu1(float g, float u) {
    const float s = 1.0f / (1.0f + expf(-g));
    return (g * s) * u;
}

void fko_swiglu_f32(const float* g, const float* u, float* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = fko_swiglu1(g[i], u[i]);
}

void fko_w8a8_swiglu(const int8_t* A, const int8_t* W, void* out, int M, int I, int K,
                     const float* scale_a, const float* scale_b, float sa, float sb,
                     const float* bias, int out_dtype, const int* rows, int nrows, int nthreads) {
    const int R = rows ? nrows : M;
    const int N = 2 * I;
    int32_t* acc = (int32_t*)malloc((size_t)R * N * sizeof(int32_t));
    if (!acc) return;
    fko_w8a8_acc(A, W, acc, M, N, K, FKO_B_NK, rows, nrows, nthreads);
    for (int r = 0; r < R; ++r) {
        const int m = rows ? rows[r] : r;
        const float am = scale_a ? scale_a[m] : sa;
        for (int n = 0; n < I; ++n) {
            const int32_t* a = acc + (size_t)r * N;
            const float g = epi((float)a[n], am * (scale_b ? scale_b[n] : sb), bias, n);
            const float u = epi((float)a[I + n], am * (scale_b ? scale_b[I + n] : sb), bias, I + n);
            store_out(out, (size_t)r * I + n, out_dtype, fko_swiglu1(g, u), 0);
        }
    }
    free(acc);
}

/* IEEE binary16 -> fp32, exact, from the bit fields. */
float fko_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        float v = ldexpf((float)m, -24);
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void fko_gemm_half(const uint16_t* A, const uint16_t* B, void* out, int M, int N, int K, int in_dtype,
                   const float* scale_a, const float* scale_b, float sa, float sb, const float* bias,
                   int out_dtype, int b_layout, const int* rows, int nrows, int nthreads) {
    const int R = rows ? nrows : M;
    float* dec = (float*)malloc(sizeof(float) * 65536);
    if (!dec) return;
    for (uint32_t i = 0; i < 65536; ++i) dec[i] = in_dtype == 2 ? fko_f16_to_f32((uint16_t)i) : fko_bf16_to_f32((uint16_t)i);
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int r = 0; r < R; ++r) {
        const int m = rows ? rows[r] : r;
        const uint16_t* a = A + (size_t)m * K;
        const float am = scale_a ? scale_a[m] : sa;
        float* sums = (float*)malloc(sizeof(float) * (size_t)N);
        for (int n = 0; n < N; ++n) sums[n] = 0.0f;
        if (b_layout == FKO_B_KN) {
            for (int k = 0; k < K; ++k) { /* each sums[n] still adds k = 0..K-1 in order */
                const float av = dec[a[k]];
                const uint16_t* b = B + (size_t)k * N;
                for (int n = 0; n < N; ++n) sums[n] += av * dec[b[n]];
            }
        } else {
            for (int n = 0; n < N; ++n) {
                const uint16_t* b = B + (size_t)n * K;
                float sum = 0.0f;
                for (int k = 0; k < K; ++k) sum += dec[a[k]] * dec[b[k]];
                sums[n] = sum;
            }
        }
        for (int n = 0; n < N; ++n) {
            const float s = am * (scale_b ? scale_b[n] : sb);
            store_out(out, (size_t)r * N + n, out_dtype, epi(sums[n], s, bias, n), 0);
        }
        free(sums);
    }
    free(dec);
}
