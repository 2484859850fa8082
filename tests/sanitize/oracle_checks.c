/* CPU sanitizer run of the oracle (oracle/fke_oracle.c): every function on
 * small inputs that include the edge values the tests use - NaN, +-inf,
 * subnormals, tiny row maxima, all E4M3 / fp16 codes, K tails, row subsets,
 * both B layouts, several thread counts.  Built with AddressSanitizer and
 * UndefinedBehaviorSanitizer (float-cast-overflow included) by
 * tests/sanitize/Makefile; any report aborts the run.  The numerics are
 * pinned elsewhere (tests/test_oracle.py); the checks here are loose sanity
 * checks so that every call's result is used. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fke_oracle.h"

static int failures = 0;
#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            ++failures;                                                 \
        }                                                               \
    } while (0)

static void gemms(void) {
    enum { M = 7, N = 9, K = 37 };
    int8_t A[M * K], B[N * K], Bkn[K * N];
    fko_gen_i8_uniform(A, M * K, 1);
    fko_gen_i8_uniform(B, N * K, 2);
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) Bkn[k * N + n] = B[n * K + k];
    float C[M * N], C2[M * N];
    fko_ref_host_gemm_i8(A, B, C, M, N, K, 0.01f, 0.02f);
    fko_ref_kernel_gemm_i8(A, B, C2, M, N, 36, 0.01f, 0.02f); /* K % 4 == 0 prefix of the same rows */
    fko_ref_py_gemm_i8(A, Bkn, C2, M, N, K, 0.5, 0.25);
    int32_t acc[M * N], acc2[M * N];
    fko_w8a8_acc(A, B, acc, M, N, K, FKO_B_NK, NULL, 0, 1);
    fko_w8a8_acc(A, Bkn, acc2, M, N, K, FKO_B_KN, NULL, 0, 3);
    CHECK(memcmp(acc, acc2, sizeof acc) == 0);
    for (int i = 0; i < M * N; ++i) CHECK((float)acc[i] * (0.01f * 0.02f) == C[i]);
    const int rows[3] = {6, 0, 3};
    int32_t accr[3 * N];
    fko_w8a8_acc(A, B, accr, M, N, K, FKO_B_NK, rows, 3, 2);
    CHECK(memcmp(accr, acc + 6 * N, N * sizeof(int32_t)) == 0);
    float sa[M], sb[N], bias[N];
    fko_gen_f32_uniform(sa, M, 3, 0.001, 0.02);
    fko_gen_f32_uniform(sb, N, 4, 0.001, 0.02);
    fko_gen_f32_normal(bias, N, 5, 0.0, 0.02);
    float yf[M * N];
    uint16_t yb[M * N];
    int32_t yi[M * N];
    fko_w8a8_epilogue(acc, yf, M, N, sa, sb, 1.f, 1.f, bias, FKO_OUT_F32, NULL);
    fko_w8a8_epilogue(acc, yb, M, N, NULL, NULL, 0.5f, 0.25f, NULL, FKO_OUT_BF16, NULL);
    fko_w8a8_epilogue(accr, yi, 3, N, sa, sb, 1.f, 1.f, bias, FKO_OUT_I32, rows);
    CHECK(yi[0] == accr[0]);
    /* SwiGLU GEMM: W = [gate; up] with I = 4 */
    int8_t W[8 * K];
    fko_gen_i8_uniform(W, 8 * K, 6);
    float h[M * 4];
    fko_w8a8_swiglu(A, W, h, M, 4, K, sa, sb, 1.f, 1.f, bias, FKO_OUT_F32, NULL, 0, 2);
    for (int i = 0; i < M * 4; ++i) CHECK(isfinite(h[i]));
}

static void fp8(void) {
    enum { M = 5, N = 11, K = 129 };
    float xa[M * K], xb[K * N];
    fko_gen_f32_normal(xa, M * K, 7, 0.0, 1.0);
    fko_gen_f32_normal(xb, K * N, 8, 0.0, 1.0);
    uint8_t qa[M * K], qb[K * N], qbnk[N * K];
    const float sa = fko_quantize_e4m3(xa, qa, M * K), sb = fko_quantize_e4m3(xb, qb, K * N);
    qa[3] = 0x7F;
    qb[10] = 0xFF; /* the reference decodes these to 0.0 */
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n) qbnk[n * K + k] = qb[k * N + n];
    float C[M * N], Cr[M * N], Cn[M * N];
    fko_ref_kernel_gemm_f8(qa, qb, Cr, M, N, K, sa, sb);
    fko_f8_gemm(qa, qb, C, M, N, K, sa, sb, NULL, FKO_OUT_F32, FKO_B_KN, NULL, 0, 3);
    fko_f8_gemm(qa, qbnk, Cn, M, N, K, sa, sb, NULL, FKO_OUT_F32, FKO_B_NK, NULL, 0, 1);
    CHECK(memcmp(C, Cr, sizeof C) == 0 && memcmp(Cn, Cr, sizeof C) == 0);
    const int rows[2] = {4, 1};
    uint16_t Cb[2 * N];
    fko_f8_gemm(qa, qb, Cb, M, N, K, sa, sb, NULL, FKO_OUT_BF16, FKO_B_KN, rows, 2, 2);
    const float special[] = {0.f, -0.f, 1.f, -1.f, 448.f, 449.f, 464.f, 1e30f, -1e30f, INFINITY, -INFINITY, NAN,
                             1e-30f, 0.001953125f, 0.0009765625f, 0.00146484375f, 240.f, -300.f};
    for (size_t i = 0; i < sizeof special / sizeof *special; ++i) {
        const uint8_t q = fko_f32_to_e4m3_sat(special[i]);
        CHECK((q & 0x7F) != 0x7F);
    }
    for (int c = 0; c < 256; ++c) CHECK(isfinite(fko_e4m3_decode((uint8_t)c)));
    float zeros[4] = {0, 0, 0, 0};
    uint8_t qz[4];
    CHECK(fko_quantize_e4m3(zeros, qz, 4) == 1.0f);
}

static void quantiser(void) {
    enum { M = 8, K = 40 };
    float x[M * K];
    fko_gen_f32_normal(x, M * K, 9, 0.0, 1.0);
    for (int k = 0; k < K; ++k) {
        x[1 * K + k] = 0.0f;                 /* all-zero row */
        x[2 * K + k] *= 1e-38f;              /* 127/amax overflows without the prescale */
        x[3 * K + k] *= 1e-44f;              /* subnormal maximum */
        x[7 * K + k] = NAN;                  /* all-NaN row */
    }
    x[4 * K + 5] = INFINITY;                 /* a row holding +inf: scale inf, codes 0 */
    x[5 * K + 0] = -INFINITY;
    x[6 * K + 3] = NAN;
    int8_t q[M * K];
    float s[M];
    fko_quantize_rows_i8(x, 0, M, K, q, s);
    CHECK(s[1] == 1.0f && isinf(s[4]) && isinf(s[5]) && s[7] == 1.0f);
    int has127 = 0;
    for (int k = 0; k < K; ++k) has127 |= q[2 * K + k] == 127 || q[2 * K + k] == -127;
    CHECK(has127);
    uint16_t xb[M * K];
    for (int i = 0; i < M * K; ++i) xb[i] = fko_f32_to_bf16_rne(x[i]);
    fko_quantize_rows_i8(xb, 1, M, K, q, s);
    CHECK(isinf(s[4]));
}

static void halves_and_swiglu(void) {
    for (int c = 0; c < 65536; ++c) {
        const float f = fko_f16_to_f32((uint16_t)c);
        CHECK(f == f || ((c >> 10) & 31) == 31);
        const uint16_t b = fko_f32_to_bf16_rne(fko_bf16_to_f32((uint16_t)c));
        CHECK(b == (uint16_t)c || ((c >> 7) & 0xFF) == 0xFF);
    }
    enum { M = 3, N = 5, K = 19 };
    uint16_t A[M * K], B[N * K];
    for (int i = 0; i < M * K; ++i) A[i] = (uint16_t)(0x3C00 + i);   /* fp16 values near 1 */
    for (int i = 0; i < N * K; ++i) B[i] = (uint16_t)(0x3F80 + i);   /* bf16 values near 1 */
    float out[M * M];
    uint16_t outb[N * N];
    fko_gemm_half(A, A, out, M, M, K, 2, NULL, NULL, 1.f, 1.f, NULL, FKO_OUT_F32, FKO_B_NK, NULL, 0, 1);
    fko_gemm_half(B, B, outb, N, N, K, 1, NULL, NULL, 2.f, 1.f, NULL, FKO_OUT_BF16, FKO_B_KN, NULL, 0, 2);
    const float g[6] = {0.f, 1.f, -100.f, 100.f, -90.f, NAN}, u[6] = {1.f, 2.f, 3.f, -1.f, 1.f, 1.f};
    float hh[6];
    fko_swiglu_f32(g, u, hh, 6);
    CHECK(hh[0] == 0.0f && fabsf(hh[2]) == 0.0f);
}

static void generators(void) {
    uint64_t st = 1234567;
    CHECK(fko_splitmix64(&st) != 0);
    int8_t a[1];
    fko_gen_i8_uniform(a, 0, 1);
    int8_t c[1000];
    fko_gen_i8_clipped_normal(c, 1000, 2, 30.0);
    float f[1000];
    fko_gen_f32_uniform(f, 1000, 3, 0.001, 0.02);
    fko_gen_f32_normal(f, 1000, 4, 0.0, 1e3);
}

int main(void) {
    generators();
    gemms();
    fp8();
    quantiser();
    halves_and_swiglu();
    if (failures) {
        printf("[FAIL] %d checks\n", failures);
        return 1;
    }
    printf("[PASS] oracle under AddressSanitizer + UndefinedBehaviorSanitizer\n");
    return 0;
}
