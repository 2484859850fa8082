/*
 * fke_qgemm.h — C ABI of the MI355X (gfx950) quantized GEMM library
 * (libfke_qgemm.so).  Plain pointers, sizes and an opaque stream; no C++ or
 * torch types.  Every entry point returns a hipError_t value as int:
 * 0 = hipSuccess, 1 = hipErrorInvalidValue (argument rejected before any HIP
 * call), otherwise the status of this call's kernel launch.
 *
 * Conventions shared by all GEMM entry points (reference:
 * flash-kernel-engine include/quantized_gemm.cuh:6-41, src/quantized_gemm.cu):
 *   - A, B, C, scale and bias pointers are caller-owned DEVICE buffers.  C is
 *     fully overwritten.  No entry point allocates or frees device memory
 *     (as the reference launchers, src/quantized_gemm.cu:56-75, :120-139).
 *     The K splits' partial sums go to the caller's workspace (the _ws entry
 *     points, fke_w8a8_linear) or to device memory the library reserves
 *     with its code object (FKE_SPLIT_SLOTS slots of FKE_SPLIT_SLOT_BYTES per
 *     GPU, one per stream; see fke_qgemm_workspace_size).
 *   - All matrices are row-major.  A is [M,K].  B is [N,K] (FKE_B_NK,
 *     K-contiguous per output column) or [K,N] (FKE_B_KN).  C is [M,N].
 *   - The call is asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronises.  Calls are re-entrant from any host
 *     thread.  Global state: the stream-to-slot table of the split pool
 *     (calls on one stream share its slot; different streams never do), and
 *     the device scratch of fke_w8a8_linear_noalloc with the event that
 *     orders its calls.
  */
#ifndef FKE_QGEMM_H
#define FKE_QGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Output element type of the fused epilogue. */
enum fke_out_dtype {
    FKE_OUT_F32 = 0,  /* fp32 y                                  */
    FKE_OUT_BF16 = 1, /* bf16, round-to-nearest-even of fp32 y   */
    FKE_OUT_I32 = 2   /* raw int32 accumulator (INT8 GEMM only)  */
};

/* Storage order of B. */
enum fke_b_layout {
    FKE_B_NK = 0, /* B[n*K + k] */
    FKE_B_KN = 1  /* B[k*N + n] */
};

/* Element type of floating-point activations (quantiser input: F32, BF16;
 * elementwise SwiGLU: all three). */
enum fke_in_dtype {
    FKE_IN_F32 = 0,  /* fp32 */
    FKE_IN_BF16 = 1, /* bf16 */
    FKE_IN_F16 = 2   /* IEEE fp16 */
};

/* Kernel family used by a call (for tests and benchmarks). */
enum fke_path {
    FKE_PATH_AUTO = 0,    /* dispatcher's choice                                */
    FKE_PATH_GEMV = 1,    /* decode family, M<=512 (INT8, NK): weight streamed  */
    FKE_PATH_MFMA = 2,    /* LDS-staged MFMA GEMM (INT8 i32 / FP8 f32 acc); for */
                          /* K % 4 == 0, 4-byte-aligned A/B (B [K,N]: N % 4 ==  */
                          /* 0) but not 16, the word kernel, also on the MFMAs  */
    FKE_PATH_GENERIC = 3, /* any-shape tiled fallback (exact reference order)   */
    FKE_PATH_GEMV_DOT = 4, /* decode, VALU dot products only (no MFMA): INT8,   */
                           /* B [N,K], M <= 16, K % 64 == 0 (fke_qgemm_i8*_on_path) */
    /* The MFMA GEMM with its workgroup tile pinned (FKE_PATH_MFMA picks a
     * smaller tile where 256x256 tiles would leave CUs idle, see
     * fke_select_mfma_tile).  Same results bit for bit, both B layouts; the
     * 64-column tiles reject the SwiGLU GEMM (hipErrorInvalidValue). */
    FKE_PATH_MFMA_256x256 = 5,
    FKE_PATH_MFMA_128x128 = 6,
    FKE_PATH_MFMA_128x128_RING4 = 7, /* 128x128, one workgroup per CU, four LDS stages */
    FKE_PATH_MFMA_128x64_RING4 = 8,  /* 128x64 (rows x columns), the same; not SwiGLU  */
    FKE_PATH_MFMA_64x64_RING4 = 9    /* 64x64, the same; not SwiGLU                    */
};

/*
 * Drop-in for flash_engine::quantized::launch_int8_gemm_dp4a
 * (reference include/quantized_gemm.cuh:19-27, src/quantized_gemm.cu:56-75):
 * C[m,n] = float(sum_k A[m,k]*B[n,k]) * fp32(scale_a*scale_b); B is [N,K]; C fp32.
 * Rejects M,N,K <= 0, K % 4 != 0 (where the reference kernel truncates K and
 * misaligns rows) and NULL pointers with hipErrorInvalidValue.
 */
int fke_launch_int8_gemm_dp4a(const int8_t* d_A, const int8_t* d_B, float* d_C,
                              float scale_a, float scale_b, int M, int N, int K,
                              void* stream);

/*
 * Drop-in for flash_engine::quantized::launch_fp8_gemm_scaled
 * (reference include/quantized_gemm.cuh:30-38, src/quantized_gemm.cu:120-139):
 * C[m,n] = (sum_k dec(A[m,k])*dec(B[k,n])) * fp32(scale_a*scale_b) with OCP
 * E4M3 decode and the reference's 0x7F/0xFF -> 0.0 rule; B is [K,N]; C fp32;
 * fp32 accumulation.
 */
int fke_launch_fp8_gemm_scaled(const uint8_t* d_A, const uint8_t* d_B, float* d_C,
                               float scale_a, float scale_b, int M, int N, int K,
                               void* stream);

/*
 * W8A8 INT8 GEMM with the fused epilogue (extends reference
 * src/quantized_gemm.cu:15-75; per-row/per-column scales, bias and the bf16/i32
 * outputs have no reference counterpart and reduce to it when uniform):
 *   acc[m,n] = sum_{k<K} A[m,k]*B(n,k)                  (exact int32)
 *   s        = fp32(sa_m * sb_n)   sa_m = scale_a ? scale_a[m] : sa
 *                                  sb_n = scale_b ? scale_b[n] : sb
 *   y        = bias ? fmaf(fp32(acc), s, bias[n]) : fp32(acc) * s
 *   C        = y (F32) | bf16_rne(y) (BF16) | acc (I32)
 * Any K >= 1.  scale_a is [M], scale_b and bias are [N] (fp32, device).
 */
int fke_qgemm_i8(const int8_t* A, const int8_t* B, void* C, int M, int N, int K,
                 const float* scale_a, const float* scale_b, float sa, float sb,
                 const float* bias, int out_dtype, int b_layout, void* stream);

/* Same as fke_qgemm_i8 on an explicit kernel family (enum fke_path).  Returns
 * hipErrorInvalidValue when that family cannot run the given shape/layout/
 * alignment.  Used by tests to cross-check kernel families. */
int fke_qgemm_i8_on_path(int path, const int8_t* A, const int8_t* B, void* C,
                         int M, int N, int K, const float* scale_a, const float* scale_b,
                         float sa, float sb, const float* bias, int out_dtype,
                         int b_layout, void* stream);

/*
 * Scaled FP8 E4M3 GEMM with the fused epilogue (extends reference
 * src/quantized_gemm.cu:99-139): sum = sum_k dec(A[m,k])*dec(B(k,n)) in fp32,
 * y = bias ? fmaf(sum, fp32(sa*sb), bias[n]) : sum * fp32(sa*sb);
 * C = y (F32) | bf16_rne(y) (BF16).  Codes 0x7F/0xFF decode to 0.0 as in the
 * reference.  The MFMA family and the decode family (B [N,K], M <= 512, K >= 2048,
 * picked for decode and small batches) sum in a different order than the
 * reference's sequential loop (each product is exact; only fp32 rounding of the
 * sum differs); the GENERIC family keeps the reference's sequential k order.
 */
int fke_qgemm_f8(const uint8_t* A, const uint8_t* B, void* C, int M, int N, int K,
                 float sa, float sb, const float* bias, int out_dtype, int b_layout,
                 void* stream);

int fke_qgemm_f8_on_path(int path, const uint8_t* A, const uint8_t* B, void* C,
                         int M, int N, int K, float sa, float sb, const float* bias,
                         int out_dtype, int b_layout, void* stream);

/*
 * Workspace of the B [K,N] decode (M <= 16, and 17..32 where its split fills
 * the CUs; M <= 32 also with N and K only multiples of 4 and 4-byte-aligned
 * operands, which need it; INT8 and FP8; no reference counterpart: the reference kernels sum
 * all of K in one thread, src/quantized_gemm.cu:29-37, :106-116).  The decode
 * splits K over workgroups of 128 to 1024 columns (up to 8 splits; M = 1 up to
 * 64) and adds the splits' partial sums in a second kernel, in split order
 * (exact for INT8, deterministic for FP8).  Past 16 rows the decode needs its
 * split: a workspace without room for it runs the MFMA GEMM instead.  The
 * MFMA GEMM's K split (fke_select_mfma_split) uses the same workspace.  The
 * partial sums need fke_qgemm_workspace_size(M, N, K, b_layout) bytes of
 * device memory (0 for shapes that neither the decode nor the MFMA GEMM
 * splits; the larger of the two needs otherwise; never more than
 * FKE_SPLIT_SLOT_BYTES: the split plans are capped to one slot).
 * fke_qgemm_i8 / fke_qgemm_f8 and the drop-in launchers put them in the
 * stream's slot of the library's split pool: a stream is given one of the
 * FKE_SPLIT_SLOTS slots of its GPU on its first split call (also while it
 * is being captured into a graph, whose kernels then keep that slot's
 * address) and keeps it; the next FKE_SPLIT_SMALL_SLOTS streams on that GPU
 * get slots of FKE_SPLIT_SMALL_SLOT_BYTES, on which plans that need more run
 * with fewer splits (the B [K,N] decode) or unsplit (the MFMA GEMM); past
 * both, and on hipStreamPerThread, calls run unsplit.  A graph captured on a stream must
 * not be replayed while other work that uses the capture stream's slot (calls
 * on that stream, other graphs captured on it) can run at the same time.
 * fke_qgemm_i8_ws / fke_qgemm_f8_ws are the same calls on the caller's
 * workspace (16-byte aligned), taken as given: NULL, fewer bytes or an
 * unaligned pointer run with fewer splits or unsplit.  INT8 results are the
 * same bits whatever the workspace.  FP8 sums each split in fp32 and adds the
 * splits in order, so the bits depend on the number of splits: a workspace of
 * at least fke_qgemm_workspace_size bytes gives the bits of fke_qgemm_f8
 * (eager or captured) on a stream holding a large pool slot, a smaller one
 * other bits (within the same FP8 error bounds, and the same from call to
 * call); on a stream holding a small slot fke_qgemm_f8 gives the bits of a
 * FKE_SPLIT_SMALL_SLOT_BYTES workspace, eager or captured alike.  Calls that can overlap in time
 * must not share a workspace.  Other kernel families ignore it.
 */
#define FKE_SPLIT_SLOTS 16
#define FKE_SPLIT_SLOT_BYTES (16u << 20)
#define FKE_SPLIT_SMALL_SLOTS 48
#define FKE_SPLIT_SMALL_SLOT_BYTES (2u << 20)
size_t fke_qgemm_workspace_size(int M, int N, int K, int b_layout);
/* Slots of the current GPU's split pool that streams hold (0..FKE_SPLIT_SLOTS
 * + FKE_SPLIT_SMALL_SLOTS; the first FKE_SPLIT_SLOTS are the large ones), or
 * -1 without a device.  Host logic only; launches nothing. */
int fke_split_slots_in_use(void);
int fke_qgemm_i8_ws(const int8_t* A, const int8_t* B, void* C, int M, int N, int K,
                    const float* scale_a, const float* scale_b, float sa, float sb,
                    const float* bias, int out_dtype, int b_layout,
                    void* workspace, size_t workspace_bytes, void* stream);
int fke_qgemm_f8_ws(const uint8_t* A, const uint8_t* B, void* C, int M, int N, int K,
                    float sa, float sb, const float* bias, int out_dtype, int b_layout,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-token (per-row) symmetric INT8 quantiser: the step that produces A and
 * scale_a for fke_qgemm_i8 from fp32 or bf16 activations X [M,K].  No
 * reference counterpart (the reference GEMMs take int8 inputs and scalar
 * scales, src/quantized_gemm.cu:56-75):
 *   amax_m = max_k |X[m,k]|             (NaN elements ignored, +-inf counted)
 *   s_m    = fp32(amax_m / 127) -> scale[m]
 *   f_m    = 2^64 if amax_m < 2^-64 else 1;  r_m = fp32(127 / (amax_m * f_m))
 *            (s_m = r_m = 1 when amax_m == 0)
 *   p      = fp32(fp32(X[m,k] * f_m) * r_m)
 *   Q[m,k] = NaN(p) ? 0 : clamp(rne(p), -127, 127)
 * f_m (exact) keeps r_m finite when 127/amax_m would overflow fp32 and changes
 * no code where it would not.  A row holding +-inf gets scale inf and all
 * codes 0; NaN elements give 0.
 * The divisions are IEEE fp32, correctly rounded.  Q is int8 [M,K] row-major,
 * scale fp32 [M]; device buffers.  Rejects NULL pointers, M,K <= 0 and bad
 * dtypes with hipErrorInvalidValue.
 */
int fke_quantize_rows_i8(const void* X, int in_dtype, int M, int K, int8_t* Q, float* scale,
                         void* stream);

/*
 * Elementwise SwiGLU, drop-in for flash_engine::activation::launch_fused_swiglu_fp32
 * / _fp16 (reference include/fused_activations.cuh:11-25, src/fused_activations.cu:17-118),
 * with bf16 added:
 *   out[i] = (g * sigmoid(g)) * u,  sigmoid(g) = 1 / (1 + exp(-g)),
 * computed in fp32 from g = gate[i], u = up[i] and rounded to the element type
 * (dtype: enum fke_in_dtype) to nearest even.  n elements, device buffers (out
 * may alias gate or up).  exp within 1 ulp, reciprocal within 1 ulp.  Rejects
 * NULL pointers, n < 0 and bad dtypes; n == 0 launches nothing.
 */
int fke_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/*
 * W8A8 gate/up projection with SwiGLU fused into the GEMM epilogue (fuses
 * reference src/fused_activations.cu:17-35 behind the quantized GEMM; no
 * single reference call).  W is the merged weight [2I, K] int8 row-major (the
 * B [N,K] layout): rows 0..I-1 are the gate projection, rows I..2I-1 the up
 * projection.  With epi() the fke_qgemm_i8 epilogue (fp32 y):
 *   g = epi(A . W[n]),   using scale_b[n],   bias[n]
 *   u = epi(A . W[I+n]), using scale_b[I+n], bias[I+n]
 *   H[m,n] = (g * sigmoid(g)) * u   as in fke_swiglu, for n < I
 * H is [M, I], fp32 or bf16 (out_dtype).  scale_b and bias are [2I] or NULL;
 * scale_a [M] or NULL.  Equals fke_swiglu applied to the two fp32 GEMM
 * outputs, bit for bit.  Rejects I < 1, 2I > INT32_MAX and FKE_OUT_I32.
 */
int fke_qgemm_i8_swiglu(const int8_t* A, const int8_t* W, void* H, int M, int I, int K,
                        const float* scale_a, const float* scale_b, float sa, float sb,
                        const float* bias, int out_dtype, void* stream);

int fke_qgemm_i8_swiglu_on_path(int path, const int8_t* A, const int8_t* W, void* H, int M, int I,
                                int K, const float* scale_a, const float* scale_b, float sa,
                                float sb, const float* bias, int out_dtype, void* stream);

/*
 * fp16 / bf16 GEMM on the MFMA tile engine (extends reference
 * src/tensor_core_attention.cu:13-86, whose WMMA kernel computes fp16 A [M,K]
 * times B stored [N,K] into fp32; per-row/per-column scales, bias and the
 * bf16 operands and output have no reference counterpart):
 *   acc[m,n] = sum_k A[m,k]*B(n,k) in fp32       (each product exact in fp32)
 *   y        = bias ? fmaf(acc, s, bias[n]) : acc * s,  s = fp32(sa_m * sb_n)
 *   C        = y (F32) | bf16_rne(y) (BF16)
 * in_dtype: FKE_IN_F16 or FKE_IN_BF16 (A and B alike); K counts elements.
 * The MFMA family (K % 64 == 0, B [N,K], 16-byte aligned) sums in its own
 * order; the GENERIC family sums k = 0..K-1 in order.  Any M, N, K >= 1.
 */
int fke_gemm_half(const void* A, const void* B, void* C, int M, int N, int K, int in_dtype,
                  const float* scale_a, const float* scale_b, float sa, float sb,
                  const float* bias, int out_dtype, int b_layout, void* stream);

int fke_gemm_half_on_path(int path, const void* A, const void* B, void* C, int M, int N, int K,
                          int in_dtype, const float* scale_a, const float* scale_b, float sa,
                          float sb, const float* bias, int out_dtype, int b_layout, void* stream);

/*
 * Drop-in for flash_engine::tensor_core::launch_wmma_gemm_fp16 (reference
 * include/tensor_core_gemm.cuh:27-35, src/tensor_core_attention.cu:68-86):
 * C[m,n] = alpha * sum_k A[m,k]*B[n*K+k], A and B fp16, C fp32 [M,N].  beta
 * is accepted and unused, as in the reference (C is overwritten).  Any M, N,
 * K >= 1 (the reference kernel needs multiples of 16).
 */
int fke_launch_wmma_gemm_fp16(const void* d_A, const void* d_B, float* d_C, int M, int N, int K,
                              float alpha, float beta, void* stream);

/*
 * W8A8 linear layer from float activations in one call: the per-token
 * quantisation of fke_quantize_rows_i8 applied to X [M,K] (fp32 or bf16,
 * in_dtype), then the fke_qgemm_i8 GEMM with B = W [N,K] int8, scale_a = the
 * row scales, scale_b = w_scale ([N] or NULL for the scalar sb) and bias:
 *   Y = fke_qgemm_i8(quantize(X), W, ...)   bit for bit, fp32 or bf16 [M,N].
 * No reference counterpart (its GEMMs take int8 inputs).  Two launches on
 * `stream`: the quantiser writes the codes and scales into the caller's
 * device `workspace` (at least fke_w8a8_linear_workspace_size(M, K) bytes,
 * else hipErrorInvalidValue), the GEMM reads them there; calls that share a
 * workspace must be ordered (same stream).  A K split's partial sums go to
 * the workspace past the row scales (from the next 256-byte boundary) when it
 * holds fke_qgemm_workspace_size(M, N, K, FKE_B_NK) bytes there, else to the
 * stream's slot of the split pool.
 */
size_t fke_w8a8_linear_workspace_size(int M, int K);
int fke_w8a8_linear(const void* X, int in_dtype, const int8_t* W, void* Y, int M, int N, int K,
                    const float* w_scale, float sb, const float* bias, int out_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * fke_w8a8_linear without the caller's workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments and result as fke_w8a8_linear, bit for bit; the quantised
 * activations and row scales go to a library-owned device array of
 * FKE_W8A8_NOALLOC_SCRATCH_BYTES bytes per GPU (held until the process ends;
 * its address is looked up once per device); a K split's partial sums go
 * to the same array, past the codes and scales, with as many splits as fit.
 * The call allocates nothing.
 * Rejects, with hipErrorInvalidValue, shapes whose workspace
 * (fke_w8a8_linear_workspace_size(M, K)) exceeds the array, and a stream of a
 * device other than the current one.  Every call on one GPU shares that GPU's
 * array.  Calls made outside graph capture are ordered: a call on a stream
 * other than the previous call's first makes its stream wait (on the
 * device's event, recorded after every such call) for the work queued
 * before the previous call ended, so calls from several streams or host
 * threads never overlap.  Work captured into a graph is not ordered: a
 * replay that can overlap another call on the same GPU races.  Nothing in
 * the array needs to start at zero (each call writes what it reads).
 */
#define FKE_W8A8_NOALLOC_SCRATCH_BYTES (32u << 20)
int fke_w8a8_linear_noalloc(const void* X, int in_dtype, const int8_t* W, void* Y, int M, int N, int K,
                            const float* w_scale, float sb, const float* bias, int out_dtype,
                            void* stream);

/* The same with the fused SwiGLU gate/up GEMM (fke_qgemm_i8_swiglu): W is
 * [2I, K], w_scale and bias [2I], H [M, I]. */
int fke_w8a8_swiglu_linear(const void* X, int in_dtype, const int8_t* W, void* H, int M, int I,
                           int K, const float* w_scale, float sb, const float* bias,
                           int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* The family fke_qgemm_i8 / fke_qgemm_f8 would pick (enum fke_path), or -1
 * for arguments they would reject.  Host logic only: launches nothing; the
 * batch cost model reads the current device's CU count (256 without a device). */
int fke_select_path_i8(const void* A, const void* B, const void* C, int M, int N, int K,
                       int out_dtype, int b_layout);
int fke_select_path_f8(const void* A, const void* B, const void* C, int M, int N, int K,
                       int out_dtype, int b_layout);
int fke_select_path_i8_swiglu(const void* A, const void* W, const void* H, int M, int I, int K,
                              int out_dtype);
int fke_select_path_half(const void* A, const void* B, const void* C, int M, int N, int K,
                         int in_dtype, int out_dtype, int b_layout);
/* The workgroup tile FKE_PATH_MFMA runs for this shape (any operand type) on
 * a GPU of `cus` CUs (<= 0: the current device's, 256 without a device), as
 * the FKE_PATH_MFMA_* value that pins it, or -1 for bad arguments; swiglu !=
 * 0 for the fused SwiGLU GEMM with N = 2I.  From the shape alone: where the
 * MFMA GEMM cannot run the call (K, or N with B [K,N], not a multiple of 16
 * bytes, or operands not 16-byte aligned), FKE_PATH_MFMA runs the word
 * kernel instead (128x128 or 128x64 tiles, no K split) or refuses it, and
 * neither this tile nor fke_select_mfma_split's plan applies.  Host logic
 * only; launches nothing. */
int fke_select_mfma_tile(int M, int N, int K, int b_layout, int swiglu, int cus);
/* The K split FKE_PATH_MFMA takes for an 8-bit GEMM of this shape (INT8 and
 * FP8, not SwiGLU) on `cus` CUs (<= 0: the current device's): the number of
 * splits S (1 = unsplit, on fke_select_mfma_tile's tile; -1 for bad
 * arguments) and, in *tile_path when not NULL, the FKE_PATH_MFMA_* tile it
 * runs on.  No reference counterpart (the reference has one GEMM launch per
 * call, src/quantized_gemm.cu:70-72, :134-136): with few output tiles and a long K,
 * S ring-tile workgroups per output tile each sum a contiguous 1/S of K, and
 * a second kernel adds the S partial sums in split order (exact for INT8,
 * deterministic for FP8) and applies the epilogue.  The partial sums,
 * S * M * N * 4 bytes (at most FKE_SPLIT_SLOT_BYTES), live in the workspace
 * described at fke_qgemm_workspace_size; without room the GEMM runs unsplit.  Host logic
 * only; launches nothing. */
int fke_select_mfma_split(int M, int N, int K, int b_layout, int cus, int* tile_path);

/* Replaces flash_engine::print_device_info (reference include/flash_engine.h:29,
 * src/flash_engine_api.cu:7-27): prints the device's properties to stdout. */
int fke_print_device_info(int device_id);

/* Replaces flash_engine::get_version (reference include/flash_engine.h:24-26). */
const char* fke_version(void);

/* Human-readable name for a status returned above. */
const char* fke_status_string(int status);

#ifdef __cplusplus
}
#endif
#endif /* FKE_QGEMM_H */
