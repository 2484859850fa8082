/* CPU sanitizer run of the library's host code (include/fke_qgemm.h): every
 * entry point with arguments it must reject, the dispatch queries over a grid
 * of shapes up to INT32_MAX (signed overflow in the size arithmetic would be
 * reported), and the workspace sizing.  No GPU is touched: rejected calls
 * return before any HIP call, and the dispatch queries only read the device's
 * CU count (256 when there is no device).  Built with AddressSanitizer and
 * UndefinedBehaviorSanitizer by tests/sanitize/Makefile. */
#include <limits.h>
#include <stdint.h>
#include <stdio.h>

#include "fke_qgemm.h"

#define INVALID 1
static int failures = 0;
#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            ++failures;                                                 \
        }                                                               \
    } while (0)

int main(void) {
    /* a fake, 16-byte aligned device address: never dereferenced (rejected first) */
    void* P = (void*)(uintptr_t)4096;
    const int bad_sizes[][3] = {{0, 1, 1}, {1, 0, 1}, {1, 1, 0}, {-1, 8, 8}, {8, -5, 8}, {8, 8, INT_MIN}};
    for (int i = 0; i < 6; ++i) {
        const int M = bad_sizes[i][0], N = bad_sizes[i][1], K = bad_sizes[i][2];
        CHECK(fke_qgemm_i8(P, P, P, M, N, K, NULL, NULL, 1.f, 1.f, NULL, FKE_OUT_F32, FKE_B_NK, NULL) == INVALID);
        CHECK(fke_qgemm_f8(P, P, P, M, N, K, 1.f, 1.f, NULL, FKE_OUT_F32, FKE_B_KN, NULL) == INVALID);
        CHECK(fke_gemm_half(P, P, P, M, N, K, FKE_IN_BF16, NULL, NULL, 1.f, 1.f, NULL, FKE_OUT_F32, FKE_B_NK,
                            NULL) == INVALID);
        CHECK(fke_qgemm_i8_swiglu(P, P, P, M, N, K, NULL, NULL, 1.f, 1.f, NULL, FKE_OUT_BF16, NULL) == INVALID);
        CHECK(fke_quantize_rows_i8(P, FKE_IN_F32, M, K, P, P, NULL) == INVALID || (M > 0 && K > 0));
        CHECK(fke_w8a8_linear_noalloc(P, FKE_IN_BF16, P, P, M, N, K, NULL, 1.f, NULL, FKE_OUT_BF16, NULL) == INVALID);
    }
    CHECK(fke_qgemm_i8(NULL, P, P, 8, 8, 8, NULL, NULL, 1.f, 1.f, NULL, 0, 0, NULL) == INVALID);
    CHECK(fke_qgemm_i8(P, P, P, 8, 8, 8, NULL, NULL, 1.f, 1.f, NULL, 7, 0, NULL) == INVALID);
    CHECK(fke_qgemm_i8(P, P, P, 8, 8, 8, NULL, NULL, 1.f, 1.f, NULL, 0, 9, NULL) == INVALID);
    CHECK(fke_qgemm_f8(P, P, P, 8, 8, 8, 1.f, 1.f, NULL, FKE_OUT_I32, 0, NULL) == INVALID);
    CHECK(fke_launch_int8_gemm_dp4a(P, P, P, 1.f, 1.f, 8, 8, 6, NULL) == INVALID);
    CHECK(fke_launch_fp8_gemm_scaled(P, NULL, P, 1.f, 1.f, 8, 8, 8, NULL) == INVALID);
    CHECK(fke_launch_wmma_gemm_fp16(P, P, NULL, 8, 8, 8, 1.f, 0.f, NULL) == INVALID);
    CHECK(fke_swiglu(P, P, P, -1, FKE_IN_F32, NULL) == INVALID);
    CHECK(fke_swiglu(P, P, P, 0, FKE_IN_F32, NULL) == 0);     /* nothing to do, nothing launched */
    CHECK(fke_swiglu(P, P, NULL, 8, FKE_IN_F32, NULL) == INVALID);
    CHECK(fke_qgemm_i8_swiglu(P, P, P, 8, INT_MAX, 64, NULL, NULL, 1.f, 1.f, NULL, FKE_OUT_BF16, NULL) == INVALID);
    CHECK(fke_qgemm_i8_on_path(17, P, P, P, 8, 8, 64, NULL, NULL, 1.f, 1.f, NULL, 0, 0, NULL) == INVALID);
    CHECK(fke_qgemm_i8_on_path(FKE_PATH_GEMV, P, P, P, 513, 64, 4096, NULL, NULL, 1.f, 1.f, NULL, 0, 0, NULL) ==
          INVALID);
    /* workspace sizing and the workspace-taking entry points */
    CHECK(fke_w8a8_linear_workspace_size(0, 5) == 0 && fke_w8a8_linear_workspace_size(5, -1) == 0);
    CHECK(fke_w8a8_linear_workspace_size(INT_MAX, INT_MAX) > (size_t)INT_MAX);
    const size_t need = fke_w8a8_linear_workspace_size(8, 4096);
    CHECK(fke_w8a8_linear(P, FKE_IN_BF16, P, P, 8, 64, 4096, NULL, 1.f, NULL, FKE_OUT_BF16, P, need - 1, NULL) ==
          INVALID);
    CHECK(fke_w8a8_linear(P, FKE_IN_BF16, P, P, 8, 64, 4096, NULL, 1.f, NULL, FKE_OUT_BF16, NULL, need, NULL) ==
          INVALID);
    CHECK(fke_w8a8_linear_noalloc(P, FKE_IN_BF16, P, P, INT_MAX, 64, INT_MAX, NULL, 1.f, NULL, FKE_OUT_BF16,
                                  NULL) == INVALID);
    CHECK(fke_w8a8_linear_noalloc(P, FKE_IN_BF16, P, P, 4096, 64, 8192, NULL, 1.f, NULL, FKE_OUT_BF16, NULL) ==
          INVALID);
    /* dispatch queries over a grid of shapes, both layouts, every output type */
    const int dims[] = {1, 2, 3, 15, 16, 17, 63, 64, 65, 127, 128, 129, 512, 513, 2047, 2048, 4095, 4096,
                        4104, 8192, 14336, 65536, 1 << 20, (1 << 20) + 16, 1 << 24, INT_MAX / 2, INT_MAX};
    const int nd = (int)(sizeof dims / sizeof *dims);
    long n_paths[5] = {0}, n_ws = 0, n_tiles[5] = {0}, n_split = 0;
    for (int a = 0; a < nd; ++a)
        for (int b = 0; b < nd; ++b)
            for (int c = 0; c < nd; ++c)
                for (int lay = 0; lay < 2; ++lay) {
                    const int M = dims[a], N = dims[b], K = dims[c];
                    for (int out = 0; out < 3; ++out) {
                        const int p8 = fke_select_path_i8(P, P, P, M, N, K, out, lay);
                        CHECK(p8 >= FKE_PATH_GEMV && p8 <= FKE_PATH_GENERIC);
                        ++n_paths[p8 + 1];
                    }
                    for (int out = 0; out < 2; ++out) {
                        const int pf = fke_select_path_f8(P, P, P, M, N, K, out, lay);
                        CHECK(pf >= FKE_PATH_GEMV && pf <= FKE_PATH_GENERIC);
                        const int ph = fke_select_path_half(P, P, P, M, N, K, FKE_IN_F16, out, lay);
                        CHECK(ph == FKE_PATH_MFMA || ph == FKE_PATH_GENERIC);
                    }
                    const int ps = fke_select_path_i8_swiglu(P, P, P, M, N, K, FKE_OUT_BF16);
                    CHECK(ps == -1 || (ps >= FKE_PATH_GEMV && ps <= FKE_PATH_GENERIC));
                    /* B [K,N] decode workspace (M <= 32): M*N*4 bytes per split (N rounded to 128),
                       2..8 splits (the row kernel, M = 1 or N, K not multiples of 16 / 64: 1..64) */
                    const size_t ws = fke_qgemm_workspace_size(M, N, K, lay);
                    const size_t row = (size_t)((N + 127LL) / 128) * 128 * 4 * (size_t)M;
                    const int rowk = M == 1 || N % 16 != 0 || K % 64 != 0;
                    /* or the MFMA GEMM's K split: S * M * N * 4 bytes, 2 <= S <= 8 */
                    int tp = -1;
                    const int S = fke_select_mfma_split(M, N, K, lay, 256, &tp);
                    CHECK(S >= 1 && S <= 8 && (tp == FKE_PATH_MFMA_256x256 ||
                                               (tp >= FKE_PATH_MFMA_128x128 && tp <= FKE_PATH_MFMA_64x64_RING4)));
                    CHECK(S == 1 || tp >= FKE_PATH_MFMA_128x128_RING4);
                    const size_t split = S > 1 ? (size_t)S * (size_t)M * (size_t)N * 4 : 0;
                    CHECK(ws == 0 || ws == split ||
                          (lay == FKE_B_KN && M <= 32 && ws % row == 0 && ws / row >= (rowk ? 1 : 2) &&
                           ws / row <= (rowk ? 64 : 8)));
                    n_split += S > 1;
                    ++n_ws;
                    /* MFMA tile: the narrow rings not for SwiGLU; -1 only for an odd SwiGLU N */
                    for (int sw = 0; sw < 2; ++sw) {
                        const int t = fke_select_mfma_tile(M, N, K, lay, sw, 256);
                        CHECK(t == -1 ? (sw && N % 2)
                                      : (t == FKE_PATH_MFMA_256x256 ||
                                         (t >= FKE_PATH_MFMA_128x128 && t <= FKE_PATH_MFMA_64x64_RING4 &&
                                          !(sw && t >= FKE_PATH_MFMA_128x64_RING4))));
                        if (t >= 0) ++n_tiles[t - FKE_PATH_MFMA_256x256];
                    }
                }
    CHECK(n_paths[FKE_PATH_GEMV + 1] > 0 && n_paths[FKE_PATH_MFMA + 1] > 0 && n_paths[FKE_PATH_GENERIC + 1] > 0);
    for (int t = 0; t < 5; ++t) CHECK(n_tiles[t] > 0);
    CHECK(n_split > 0);
    CHECK(fke_select_mfma_split(0, 64, 64, 0, 256, NULL) == -1 && fke_select_mfma_split(64, 64, 64, 2, 256, NULL) == -1);
    CHECK(fke_select_path_i8(NULL, P, P, 8, 8, 8, 0, 0) == -1);
    CHECK(fke_select_path_f8(P, P, P, 8, 8, 8, FKE_OUT_I32, 0) == -1);
    CHECK(fke_status_string(1) != NULL && fke_version() != NULL);
    if (failures) {
        printf("[FAIL] %d checks\n", failures);
        return 1;
    }
    printf("[PASS] C ABI host code under AddressSanitizer + UndefinedBehaviorSanitizer (%ld dispatch queries, "
           "%ld workspace sizes)\n", n_paths[1] + n_paths[2] + n_paths[3] + n_paths[4], n_ws);
    return 0;
}
