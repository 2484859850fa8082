// capi.hip — extern "C" boundary of libfke_qgemm.so: argument validation,
// kernel-family dispatch and the drop-in entry points.
//
// Error contract: arguments are validated first and rejected with
// hipErrorInvalidValue before any HIP runtime call, so the checks run (and are
// tested) without a GPU.  Otherwise the return value is the status of this
// call's hipLaunchKernel (the reference returned cudaGetLastError() after its
// launch, src/quantized_gemm.cu:74,138, which could also surface an earlier
// sticky error).  No call path allocates device memory.  State kept between
// calls: the per-device addresses of the two static device arrays below (set
// once), the stream-to-slot table of the K splits' pool, and the event and
// last stream that order fke_w8a8_linear_noalloc calls across streams.
#include <cstdio>
#include <mutex>

#include "fke_internal.h"

// Device scratch of fke_w8a8_linear_noalloc: the quantised activations and
// their row scales between its two launches (the layout of the workspace of
// fke_w8a8_linear).  Each GPU the library runs on holds its own copy for the
// life of the process.  In host code `scratch` is only a handle: its device
// address on the current device comes from hipGetSymbolAddress (below).
static __device__ __align__(256) uint8_t scratch[FKE_W8A8_NOALLOC_SCRATCH_BYTES];

// Partial sums of the K splits (the [K,N] decode's and the MFMA GEMM's),
// FKE_SPLIT_SLOTS slots of FKE_SPLIT_SLOT_BYTES per GPU, then
// FKE_SPLIT_SMALL_SLOTS of FKE_SPLIT_SMALL_SLOT_BYTES, reserved with the code
// object: no call path allocates device memory.  A stream gets a slot the
// first time one of its calls splits K (a large one while any is free) and
// keeps it for the life of the process: calls on one stream run in order and
// share it, calls on different streams never do.  No split plan needs more
// than one large slot; plans adapt to a small one (the [K,N] decode with
// fewer splits, the MFMA GEMM unsplit where its plan does not fit).  The
// small slots keep the splits for the many streams a framework may cycle
// through (torch's pool holds 32 per device and priority) at 2 MiB each: the
// [K,N] decode at N = 14336, K = 4096 needs 0.9 / 1.75 MiB at M = 1 / 16.
static __device__ __align__(256) uint8_t split_pool[size_t{FKE_SPLIT_SLOTS} * FKE_SPLIT_SLOT_BYTES];
static __device__ __align__(256) uint8_t split_pool_small[size_t{FKE_SPLIT_SMALL_SLOTS} * FKE_SPLIT_SMALL_SLOT_BYTES];

namespace {

using fke::GemmArgs;

constexpr int kMaxDevices = 64;

// Per-device set-up, done once per device with that device current (the
// first call on it that needs it) and immutable afterwards: the addresses of
// `scratch` and `split_pool` on that device, and the event that orders
// fke_w8a8_linear_noalloc calls across streams.
struct DeviceSetup {
    std::once_flag once;
    hipError_t status = hipSuccess;
    uint8_t* scratch = nullptr;
    uint8_t* pool = nullptr;
    uint8_t* pool_small = nullptr;
    hipEvent_t noalloc_done = nullptr;
};
DeviceSetup g_dev[kMaxDevices];

hipError_t device_setup(int dev, DeviceSetup** out) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    DeviceSetup& d = g_dev[dev];
    std::call_once(d.once, [&d] {
        void* a = nullptr;
        void* b = nullptr;
        void* c = nullptr;
        d.status = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
        if (d.status == hipSuccess) d.status = hipGetSymbolAddress(&b, HIP_SYMBOL(split_pool));
        if (d.status == hipSuccess) d.status = hipGetSymbolAddress(&c, HIP_SYMBOL(split_pool_small));
        if (d.status == hipSuccess) d.status = hipEventCreateWithFlags(&d.noalloc_done, hipEventDisableTiming);
        d.scratch = static_cast<uint8_t*>(a);
        d.pool = static_cast<uint8_t*>(b);
        d.pool_small = static_cast<uint8_t*>(c);
    });
    if (d.status != hipSuccess) return d.status;
    *out = &d;
    return hipSuccess;
}

// The current device, and a check that stream `s` belongs to it (device
// memory looked up here must be the copy on the stream's device).
hipError_t current_device_of(hipStream_t s, int* dev) {
    hipError_t st = hipGetDevice(dev);
    if (st != hipSuccess) return st;
    if (s && s != hipStreamPerThread) {
        hipDevice_t sdev = 0;
        st = hipStreamGetDevice(s, &sdev);
        if (st != hipSuccess) return st;
        if (sdev != *dev) return hipErrorInvalidValue;
    }
    return hipSuccess;
}

// Device memory for a K split's partial sums.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};

// Slot table of the split pool: slot i of device d (split_pool for i <
// FKE_SPLIT_SLOTS, split_pool_small after) belongs to g_slot_stream[d][i].
std::mutex g_slot_mu;
constexpr int kSlots = FKE_SPLIT_SLOTS + FKE_SPLIT_SMALL_SLOTS;
hipStream_t g_slot_stream[kMaxDevices][kSlots];
int g_slot_count[kMaxDevices];

// The pool slot of stream `s` on the current device, assigned on first use.
// Empty (the call then runs unsplit) when every slot belongs to another
// stream, for hipStreamPerThread (one handle for many streams) and for a
// stream of another device.  Under graph capture the capturing stream's slot
// is used like any other: the graph's kernels keep its address.
Workspace stream_slot(hipStream_t s) {
    if (s == hipStreamPerThread) return {};
    int dev = 0;
    DeviceSetup* d = nullptr;
    if (current_device_of(s, &dev) != hipSuccess || device_setup(dev, &d) != hipSuccess) return {};
    std::lock_guard<std::mutex> lock(g_slot_mu);
    int i = 0;
    while (i < g_slot_count[dev] && g_slot_stream[dev][i] != s) ++i;
    if (i == g_slot_count[dev]) {
        if (i == kSlots) return {};
        g_slot_stream[dev][i] = s;
        g_slot_count[dev] = i + 1;
    }
    Workspace w;
    if (i < FKE_SPLIT_SLOTS) {
        w.ptr = d->pool + static_cast<size_t>(i) * FKE_SPLIT_SLOT_BYTES;
        w.bytes = FKE_SPLIT_SLOT_BYTES;
    } else {
        w.ptr = d->pool_small + static_cast<size_t>(i - FKE_SPLIT_SLOTS) * FKE_SPLIT_SMALL_SLOT_BYTES;
        w.bytes = FKE_SPLIT_SMALL_SLOT_BYTES;
    }
    return w;
}

// Where a call's K-split partial sums go.  POOL: the stream's slot (the
// plain entry points).  CALLER: the caller's workspace exactly as given (a
// NULL, short or unaligned one gives fewer splits or none: the _ws entry
// points, and the allocation-free linear's scratch).  CALLER_OR_POOL: the
// caller's when it holds the whole plan, else the stream's slot
// (fke_w8a8_linear's workspace past its codes and scales).
enum WsMode { WS_POOL, WS_CALLER, WS_CALLER_OR_POOL };
struct WsChoice {
    WsMode mode = WS_POOL;
    Workspace caller;
};

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

Workspace split_workspace(hipStream_t s, size_t need, const WsChoice& wc) {
    if (need == 0) return {};
    if (wc.mode == WS_CALLER) return wc.caller;
    if (wc.mode == WS_CALLER_OR_POOL && wc.caller.ptr && wc.caller.bytes >= need && aligned16(wc.caller.ptr))
        return wc.caller;
    return stream_slot(s);
}

// The caller's workspace of a _ws entry point, taken as given.
WsChoice caller_ws(void* workspace, size_t workspace_bytes) {
    WsChoice wc;
    wc.mode = WS_CALLER;
    wc.caller.ptr = workspace;
    wc.caller.bytes = workspace ? workspace_bytes : 0;
    return wc;
}

// Cross-stream order of fke_w8a8_linear_noalloc calls on each device: the
// stream of the last call made outside graph capture, and whether it
// recorded DeviceSetup::noalloc_done.
std::mutex g_noalloc_mu[kMaxDevices];
hipStream_t g_noalloc_last[kMaxDevices];
bool g_noalloc_recorded[kMaxDevices];

int run_mfma(int path, const GemmArgs& p, int elem, hipStream_t s, const WsChoice& wc = WsChoice{});

// The [K,N] decode, split over the workspace `wc` gives.  Past 16 rows it
// needs its split (the one-kernel decode takes 16 rows), and with operands
// only 4-byte aligned (N or K not a multiple of 16 / 64) a workspace of one
// split at least; without it the MFMA GEMM runs, or the generic kernel.
hipError_t run_kn(const GemmArgs& p, int elem, hipStream_t s, const WsChoice& wc) {
    const Workspace ws = split_workspace(s, fke::gemv_kn_workspace_bytes(p), wc);
    const fke::KnSplit sp = fke::gemv_kn_plan(p, ws.ptr, ws.bytes);
    if (!fke::gemv_kn_plan_runs(p, sp)) {
        if (fke::mfma_supports(p, elem) || fke::words_supports(p, elem))
            return static_cast<hipError_t>(run_mfma(FKE_PATH_MFMA, p, elem, s, wc));
        return fke::launch_generic(p, elem, s);
    }
    return fke::launch_gemv_kn(p, elem, sp, s);
}

int run_i8(int path, const GemmArgs& p, void* stream, const WsChoice& wc = WsChoice{});

bool common_args_ok(const void* A, const void* B, const void* C, int M, int N, int K,
                    int b_layout) {
    if (!A || !B || !C) return false;
    if (M < 1 || N < 1 || K < 1) return false;
    if (b_layout != FKE_B_NK && b_layout != FKE_B_KN) return false;
    return true;
}

bool i8_args_ok(const void* A, const void* B, const void* C, int M, int N, int K, int out_dtype,
                int b_layout) {
    return common_args_ok(A, B, C, M, N, K, b_layout) && out_dtype >= FKE_OUT_F32 &&
           out_dtype <= FKE_OUT_I32;
}

bool f8_args_ok(const void* A, const void* B, const void* C, int M, int N, int K, int out_dtype,
                int b_layout) {
    return common_args_ok(A, B, C, M, N, K, b_layout) &&
           (out_dtype == FKE_OUT_F32 || out_dtype == FKE_OUT_BF16);
}

GemmArgs make_args(const void* A, const void* B, void* C, int M, int N, int K, const float* scale_a,
                   const float* scale_b, float sa, float sb, const float* bias, int out_dtype,
                   int b_layout) {
    GemmArgs p;
    p.A = A;
    p.B = B;
    p.C = C;
    p.M = M;
    p.N = N;
    p.K = K;
    p.scale_a = scale_a;
    p.scale_b = scale_b;
    p.sa = sa;
    p.sb = sb;
    p.bias = bias;
    p.out_dtype = out_dtype;
    p.b_layout = b_layout;
    p.swiglu = 0;
    return p;
}

// Workspace of the unfused W8A8 linear: int8 codes [M,K] at offset 0, then the
// fp32 row scales [M] at the next 256-byte boundary.
size_t w8a8_ws_scale_offset(int M, int K) {
    return (static_cast<size_t>(M) * static_cast<size_t>(K) + 255) & ~static_cast<size_t>(255);
}
size_t w8a8_ws_bytes(int M, int K) { return w8a8_ws_scale_offset(M, K) + 4 * static_cast<size_t>(M); }

// Shared body of fke_w8a8_linear / fke_w8a8_swiglu_linear.  p describes the
// GEMM on the int8 codes with A = X: the quantiser writes X's codes and row
// scales into the workspace, then the GEMM reads them there.  The workspace
// past the row scales (from the next 256-byte boundary) holds a K split's
// partial sums: as a whole plan's, or else the stream's pool slot takes them
// (`mode` WS_CALLER_OR_POOL), or as many splits as it holds (WS_CALLER).
int run_w8a8_from_float(GemmArgs p, int in_dtype, void* workspace, size_t workspace_bytes, void* stream,
                        WsMode mode) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!workspace || workspace_bytes < w8a8_ws_bytes(p.M, p.K)) return hipErrorInvalidValue;
    int8_t* Q = static_cast<int8_t*>(workspace);
    float* S = reinterpret_cast<float*>(static_cast<char*>(workspace) + w8a8_ws_scale_offset(p.M, p.K));
    const hipError_t st = fke::launch_quant_rows(p.A, in_dtype, p.M, p.K, Q, S, s);
    if (st != hipSuccess) return st;
    p.A = Q;
    p.scale_a = S;
    const size_t used = (w8a8_ws_bytes(p.M, p.K) + 255) & ~static_cast<size_t>(255);
    WsChoice wc;
    wc.mode = mode;
    if (workspace_bytes > used) {
        wc.caller.ptr = static_cast<char*>(workspace) + used;
        wc.caller.bytes = workspace_bytes - used;
    }
    return run_i8(FKE_PATH_AUTO, p, stream, wc);
}

// SwiGLU GEMM: B is the merged [2I, K] weight; the kernels see N = 2I.
bool swiglu_args_ok(const void* A, const void* W, const void* H, int M, int I, int K, int out_dtype) {
    if (I < 1 || I > INT32_MAX / 2) return false;
    return common_args_ok(A, W, H, M, 2 * I, K, FKE_B_NK) &&
           (out_dtype == FKE_OUT_F32 || out_dtype == FKE_OUT_BF16);
}

GemmArgs make_swiglu_args(const void* A, const void* W, void* H, int M, int I, int K, const float* scale_a,
                          const float* scale_b, float sa, float sb, const float* bias, int out_dtype) {
    GemmArgs p = make_args(A, W, H, M, 2 * I, K, scale_a, scale_b, sa, sb, bias, out_dtype, FKE_B_NK);
    p.swiglu = 1;
    return p;
}

// Decode with B [K,N]: the transposing kernels, but where the row kernel's
// 4-byte form would stream the weights more than once (past 4 rows) the MFMA
// GEMM if it takes the shape, and past 8 rows the word kernel.  Same box,
// N = 14340, K = 4096, bf16 out: row kernel / word kernel M = 8 23.7 / 36.0
// us, M = 12 40.3 / 36.1, M = 16 39.9 / 36.0 (FP8 26.7 / 40.3 and 43.7 /
// 40.3).
bool kn_decode_pays(const GemmArgs& p, int elem) {
    if (!fke::gemv_kn_supports(p, elem)) return false;
    if (!fke::gemv_kn_yields_to_mfma(p)) return true;
    return !(fke::mfma_supports(p, elem) || (p.M > 8 && fke::words_supports(p, elem)));
}

int pick_i8(const GemmArgs& p) {
    if (kn_decode_pays(p, fke::ELEM_I8)) return FKE_PATH_GEMV;
    // decode and batches up to FKE_GEMV_MAX_M rows: the decode family where
    // its cost model beats the MFMA GEMM's, or where that GEMM cannot run
    if (fke::gemv_i8_supports(p) && (fke::gemv_i8_batch_pays(p) || !fke::mfma_supports(p, fke::ELEM_I8)))
        return FKE_PATH_GEMV;
    if (fke::mfma_supports(p, fke::ELEM_I8)) return FKE_PATH_MFMA;
    if (fke::words_supports(p, fke::ELEM_I8)) return FKE_PATH_MFMA;  // the word kernel's matrix cores
    return FKE_PATH_GENERIC;
}

int pick_f8(const GemmArgs& p) {
    if (kn_decode_pays(p, fke::ELEM_F8)) return FKE_PATH_GEMV;
    // decode and small batches (B [N,K]): the streamed kernel, by the same cost model as INT8
    if (fke::gemv_f8_supports(p) && (fke::gemv_i8_batch_pays(p) || !fke::mfma_supports(p, fke::ELEM_F8)))
        return FKE_PATH_GEMV;
    if (fke::mfma_supports(p, fke::ELEM_F8)) return FKE_PATH_MFMA;
    if (fke::words_supports(p, fke::ELEM_F8)) return FKE_PATH_MFMA;  // the word kernel's matrix cores
    return FKE_PATH_GENERIC;
}

// FKE_PATH_MFMA_* -> the kernel's tile (the 64-column rings: not SwiGLU);
// -1 for any other path, -2 for a tile the call cannot take.
int mfma_tile_of_path(int path, const GemmArgs& p) {
    switch (path) {
        case FKE_PATH_MFMA: return fke::MFMA_TILE_AUTO;
        case FKE_PATH_MFMA_256x256: return fke::MFMA_TILE_256x256;
        case FKE_PATH_MFMA_128x128: return fke::MFMA_TILE_128x128;
        case FKE_PATH_MFMA_128x128_RING4: return fke::MFMA_TILE_128x128_RING4;
        case FKE_PATH_MFMA_128x64_RING4: return p.swiglu ? -2 : fke::MFMA_TILE_128x64_RING4;
        case FKE_PATH_MFMA_64x64_RING4: return p.swiglu ? -2 : fke::MFMA_TILE_64x64_RING4;
        default: return -1;
    }
}

// The MFMA GEMM with the tile `path` names, after its shape check.  The
// automatic tile also takes the K split the plan gives (8-bit shapes with few
// tiles and a long K), on the workspace `wc` gives; unsplit, on the tile
// rule's tile, when that does not hold the partial sums.
int run_mfma(int path, const GemmArgs& p, int elem, hipStream_t s, const WsChoice& wc) {
    const int tile = mfma_tile_of_path(path, p);
    if (tile < 0) return hipErrorInvalidValue;
    if (!fke::mfma_supports(p, elem)) {
        // K % 4 == 0 (and N % 4 == 0 with B [K,N]), 4-byte-aligned operands: the word kernel
        if (tile == fke::MFMA_TILE_AUTO && fke::words_supports(p, elem)) return fke::launch_words(p, elem, s);
        return hipErrorInvalidValue;
    }
    if (tile == fke::MFMA_TILE_AUTO) {
        const fke::MfmaPlan pl = fke::mfma_plan(p, elem, fke::device_cus());
        if (pl.S > 1) {
            const size_t need = fke::mfma_split_bytes(p, pl.S);
            const Workspace ws = split_workspace(s, need, wc);
            if (ws.ptr && ws.bytes >= need && aligned16(ws.ptr))
                return fke::launch_mfma(p, elem, s, pl.tile, fke::SplitK{pl.S, pl.KS, ws.ptr});
        }
    }
    return fke::launch_mfma(p, elem, s, tile);
}

int run_i8(int path, const GemmArgs& p, void* stream, const WsChoice& wc) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (path == FKE_PATH_AUTO) path = pick_i8(p);
    switch (path) {
        case FKE_PATH_GEMV:
            if (fke::gemv_kn_supports(p, fke::ELEM_I8)) return run_kn(p, fke::ELEM_I8, s, wc);
            if (!fke::gemv_i8_supports(p)) return hipErrorInvalidValue;
            return fke::launch_gemv_i8(p, s);
        case FKE_PATH_MFMA:
        case FKE_PATH_MFMA_256x256:
        case FKE_PATH_MFMA_128x128:
        case FKE_PATH_MFMA_128x128_RING4:
        case FKE_PATH_MFMA_128x64_RING4:
        case FKE_PATH_MFMA_64x64_RING4: return run_mfma(path, p, fke::ELEM_I8, s, wc);
        case FKE_PATH_GENERIC: return fke::launch_generic(p, fke::ELEM_I8, s);
        case FKE_PATH_GEMV_DOT:
            if (!fke::gemv_dot_supports(p)) return hipErrorInvalidValue;
            return fke::launch_gemv_dot(p, s);
        default: return hipErrorInvalidValue;
    }
}

bool half_args_ok(const void* A, const void* B, const void* C, int M, int N, int K, int in_dtype, int out_dtype,
                  int b_layout) {
    return common_args_ok(A, B, C, M, N, K, b_layout) && (in_dtype == FKE_IN_F16 || in_dtype == FKE_IN_BF16) &&
           (out_dtype == FKE_OUT_F32 || out_dtype == FKE_OUT_BF16);
}

int half_elem(int in_dtype) { return in_dtype == FKE_IN_F16 ? fke::ELEM_F16 : fke::ELEM_BF16; }

int pick_half(const GemmArgs& p, int elem) {
    if (fke::mfma_supports(p, elem)) return FKE_PATH_MFMA;
    return FKE_PATH_GENERIC;
}

int run_half(int path, const GemmArgs& p, int elem, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (path == FKE_PATH_AUTO) path = pick_half(p, elem);
    switch (path) {
        case FKE_PATH_MFMA:
        case FKE_PATH_MFMA_256x256:
        case FKE_PATH_MFMA_128x128:
        case FKE_PATH_MFMA_128x128_RING4:
        case FKE_PATH_MFMA_128x64_RING4:
        case FKE_PATH_MFMA_64x64_RING4: return run_mfma(path, p, elem, s);
        case FKE_PATH_GENERIC: return fke::launch_generic(p, elem, s);
        default: return hipErrorInvalidValue;
    }
}

int run_f8(int path, const GemmArgs& p, void* stream, const WsChoice& wc = WsChoice{}) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (path == FKE_PATH_AUTO) path = pick_f8(p);
    switch (path) {
        case FKE_PATH_GEMV:
            if (fke::gemv_kn_supports(p, fke::ELEM_F8)) return run_kn(p, fke::ELEM_F8, s, wc);
            if (!fke::gemv_f8_supports(p)) return hipErrorInvalidValue;
            return fke::launch_gemv_f8(p, s);
        case FKE_PATH_MFMA:
        case FKE_PATH_MFMA_256x256:
        case FKE_PATH_MFMA_128x128:
        case FKE_PATH_MFMA_128x128_RING4:
        case FKE_PATH_MFMA_128x64_RING4:
        case FKE_PATH_MFMA_64x64_RING4: return run_mfma(path, p, fke::ELEM_F8, s, wc);
        case FKE_PATH_GENERIC: return fke::launch_generic(p, fke::ELEM_F8, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

extern "C" {

int fke_qgemm_i8_on_path(int path, const int8_t* A, const int8_t* B, void* C, int M, int N, int K,
                         const float* scale_a, const float* scale_b, float sa, float sb,
                         const float* bias, int out_dtype, int b_layout, void* stream) {
    if (!i8_args_ok(A, B, C, M, N, K, out_dtype, b_layout)) return hipErrorInvalidValue;
    return run_i8(path, make_args(A, B, C, M, N, K, scale_a, scale_b, sa, sb, bias, out_dtype, b_layout),
                  stream);
}

int fke_qgemm_i8(const int8_t* A, const int8_t* B, void* C, int M, int N, int K, const float* scale_a,
                 const float* scale_b, float sa, float sb, const float* bias, int out_dtype,
                 int b_layout, void* stream) {
    return fke_qgemm_i8_on_path(FKE_PATH_AUTO, A, B, C, M, N, K, scale_a, scale_b, sa, sb, bias,
                                out_dtype, b_layout, stream);
}

int fke_qgemm_f8_on_path(int path, const uint8_t* A, const uint8_t* B, void* C, int M, int N, int K,
                         float sa, float sb, const float* bias, int out_dtype, int b_layout,
                         void* stream) {
    if (!f8_args_ok(A, B, C, M, N, K, out_dtype, b_layout)) return hipErrorInvalidValue;
    return run_f8(path, make_args(A, B, C, M, N, K, nullptr, nullptr, sa, sb, bias, out_dtype, b_layout),
                  stream);
}

int fke_qgemm_f8(const uint8_t* A, const uint8_t* B, void* C, int M, int N, int K, float sa, float sb,
                 const float* bias, int out_dtype, int b_layout, void* stream) {
    return fke_qgemm_f8_on_path(FKE_PATH_AUTO, A, B, C, M, N, K, sa, sb, bias, out_dtype, b_layout,
                                stream);
}

size_t fke_qgemm_workspace_size(int M, int N, int K, int b_layout) {
    if (M < 1 || N < 1 || K < 1 || (b_layout != FKE_B_NK && b_layout != FKE_B_KN)) return 0;
    // alignment-independent: the decode's shape rules with aligned stand-in pointers
    const void* a = reinterpret_cast<const void*>(uintptr_t{4096});
    const GemmArgs p = make_args(a, a, const_cast<void*>(a), M, N, K, nullptr, nullptr, 1.f, 1.f, nullptr, FKE_OUT_F32,
                                 b_layout);
    const size_t kn = fke::gemv_kn_supports(p, fke::ELEM_I8) ? fke::gemv_kn_workspace_bytes(p) : 0;
    const fke::MfmaPlan pl = fke::mfma_plan(p, fke::ELEM_I8, fke::device_cus());
    const size_t split = pl.S > 1 && fke::mfma_supports(p, fke::ELEM_I8) ? fke::mfma_split_bytes(p, pl.S) : 0;
    return kn > split ? kn : split;
}

int fke_split_slots_in_use(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
    std::lock_guard<std::mutex> lock(g_slot_mu);
    return g_slot_count[dev];
}

int fke_qgemm_i8_ws(const int8_t* A, const int8_t* B, void* C, int M, int N, int K, const float* scale_a,
                    const float* scale_b, float sa, float sb, const float* bias, int out_dtype, int b_layout,
                    void* workspace, size_t workspace_bytes, void* stream) {
    if (!i8_args_ok(A, B, C, M, N, K, out_dtype, b_layout)) return hipErrorInvalidValue;
    return run_i8(FKE_PATH_AUTO, make_args(A, B, C, M, N, K, scale_a, scale_b, sa, sb, bias, out_dtype, b_layout),
                  stream, caller_ws(workspace, workspace_bytes));
}

int fke_qgemm_f8_ws(const uint8_t* A, const uint8_t* B, void* C, int M, int N, int K, float sa, float sb,
                    const float* bias, int out_dtype, int b_layout, void* workspace, size_t workspace_bytes,
                    void* stream) {
    if (!f8_args_ok(A, B, C, M, N, K, out_dtype, b_layout)) return hipErrorInvalidValue;
    return run_f8(FKE_PATH_AUTO, make_args(A, B, C, M, N, K, nullptr, nullptr, sa, sb, bias, out_dtype, b_layout),
                  stream, caller_ws(workspace, workspace_bytes));
}

int fke_qgemm_i8_swiglu_on_path(int path, const int8_t* A, const int8_t* W, void* H, int M, int I, int K,
                                const float* scale_a, const float* scale_b, float sa, float sb,
                                const float* bias, int out_dtype, void* stream) {
    if (!swiglu_args_ok(A, W, H, M, I, K, out_dtype)) return hipErrorInvalidValue;
    return run_i8(path, make_swiglu_args(A, W, H, M, I, K, scale_a, scale_b, sa, sb, bias, out_dtype), stream);
}

int fke_qgemm_i8_swiglu(const int8_t* A, const int8_t* W, void* H, int M, int I, int K, const float* scale_a,
                        const float* scale_b, float sa, float sb, const float* bias, int out_dtype,
                        void* stream) {
    return fke_qgemm_i8_swiglu_on_path(FKE_PATH_AUTO, A, W, H, M, I, K, scale_a, scale_b, sa, sb, bias,
                                       out_dtype, stream);
}

int fke_select_path_i8_swiglu(const void* A, const void* W, const void* H, int M, int I, int K,
                              int out_dtype) {
    if (!swiglu_args_ok(A, W, H, M, I, K, out_dtype)) return -1;
    return pick_i8(make_swiglu_args(A, W, const_cast<void*>(H), M, I, K, nullptr, nullptr, 1.f, 1.f, nullptr,
                                    out_dtype));
}

size_t fke_w8a8_linear_workspace_size(int M, int K) {
    if (M < 1 || K < 1) return 0;
    return w8a8_ws_bytes(M, K);
}

int fke_w8a8_linear(const void* X, int in_dtype, const int8_t* W, void* Y, int M, int N, int K, const float* w_scale,
                    float sb, const float* bias, int out_dtype, void* workspace, size_t workspace_bytes,
                    void* stream) {
    if (!common_args_ok(X, W, Y, M, N, K, FKE_B_NK)) return hipErrorInvalidValue;
    if (in_dtype != FKE_IN_F32 && in_dtype != FKE_IN_BF16) return hipErrorInvalidValue;
    if (out_dtype != FKE_OUT_F32 && out_dtype != FKE_OUT_BF16) return hipErrorInvalidValue;
    return run_w8a8_from_float(make_args(X, W, Y, M, N, K, nullptr, w_scale, 1.0f, sb, bias, out_dtype, FKE_B_NK),
                               in_dtype, workspace, workspace_bytes, stream, WS_CALLER_OR_POOL);
}

int fke_w8a8_linear_noalloc(const void* X, int in_dtype, const int8_t* W, void* Y, int M, int N, int K,
                            const float* w_scale, float sb, const float* bias, int out_dtype, void* stream) {
    if (!common_args_ok(X, W, Y, M, N, K, FKE_B_NK)) return hipErrorInvalidValue;
    if (in_dtype != FKE_IN_F32 && in_dtype != FKE_IN_BF16) return hipErrorInvalidValue;
    if (out_dtype != FKE_OUT_F32 && out_dtype != FKE_OUT_BF16) return hipErrorInvalidValue;
    if (w8a8_ws_bytes(M, K) > FKE_W8A8_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
    // The scratch must be the copy on the stream's device, looked up with
    // that device current: a stream of another device is refused.
    hipStream_t s = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t st = current_device_of(s, &dev);
    if (st != hipSuccess) return st;
    DeviceSetup* d = nullptr;
    st = device_setup(dev, &d);
    if (st != hipSuccess) return st;
    // Calls made outside graph capture are ordered on the device's event: a
    // call on another stream than the last one's (or on hipStreamPerThread,
    // whose one handle names a stream per host thread) first waits for the
    // work queued before that event was recorded, and every such call
    // records it after its own launches.  Under capture neither happens.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    st = hipStreamIsCapturing(s, &cs);
    if (st != hipSuccess) return st;
    const bool eager = cs == hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(g_noalloc_mu[dev]);
    if (eager && g_noalloc_recorded[dev] && (g_noalloc_last[dev] != s || s == hipStreamPerThread)) {
        st = hipStreamWaitEvent(s, d->noalloc_done, 0);
        if (st != hipSuccess) return st;
    }
    st = static_cast<hipError_t>(
        run_w8a8_from_float(make_args(X, W, Y, M, N, K, nullptr, w_scale, 1.0f, sb, bias, out_dtype, FKE_B_NK),
                            in_dtype, d->scratch, FKE_W8A8_NOALLOC_SCRATCH_BYTES, stream, WS_CALLER));
    if (st != hipSuccess || !eager) return st;
    st = hipEventRecord(d->noalloc_done, s);
    if (st != hipSuccess) return st;
    g_noalloc_last[dev] = s;
    g_noalloc_recorded[dev] = true;
    return hipSuccess;
}

int fke_w8a8_swiglu_linear(const void* X, int in_dtype, const int8_t* W, void* H, int M, int I, int K,
                           const float* w_scale, float sb, const float* bias, int out_dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
    if (!swiglu_args_ok(X, W, H, M, I, K, out_dtype)) return hipErrorInvalidValue;
    if (in_dtype != FKE_IN_F32 && in_dtype != FKE_IN_BF16) return hipErrorInvalidValue;
    return run_w8a8_from_float(make_swiglu_args(X, W, H, M, I, K, nullptr, w_scale, 1.0f, sb, bias, out_dtype),
                               in_dtype, workspace, workspace_bytes, stream, WS_CALLER_OR_POOL);
}

int fke_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
    if (!gate || !up || !out || n < 0) return hipErrorInvalidValue;
    if (dtype != FKE_IN_F32 && dtype != FKE_IN_BF16 && dtype != FKE_IN_F16) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    return fke::launch_swiglu(gate, up, out, n, dtype, static_cast<hipStream_t>(stream));
}

int fke_gemm_half_on_path(int path, const void* A, const void* B, void* C, int M, int N, int K, int in_dtype,
                          const float* scale_a, const float* scale_b, float sa, float sb, const float* bias,
                          int out_dtype, int b_layout, void* stream) {
    if (!half_args_ok(A, B, C, M, N, K, in_dtype, out_dtype, b_layout)) return hipErrorInvalidValue;
    return run_half(path, make_args(A, B, C, M, N, K, scale_a, scale_b, sa, sb, bias, out_dtype, b_layout),
                    half_elem(in_dtype), stream);
}

int fke_gemm_half(const void* A, const void* B, void* C, int M, int N, int K, int in_dtype, const float* scale_a,
                  const float* scale_b, float sa, float sb, const float* bias, int out_dtype, int b_layout,
                  void* stream) {
    return fke_gemm_half_on_path(FKE_PATH_AUTO, A, B, C, M, N, K, in_dtype, scale_a, scale_b, sa, sb, bias,
                                 out_dtype, b_layout, stream);
}

int fke_select_path_half(const void* A, const void* B, const void* C, int M, int N, int K, int in_dtype,
                         int out_dtype, int b_layout) {
    if (!half_args_ok(A, B, C, M, N, K, in_dtype, out_dtype, b_layout)) return -1;
    return pick_half(make_args(A, B, const_cast<void*>(C), M, N, K, nullptr, nullptr, 1.f, 1.f, nullptr, out_dtype,
                               b_layout),
                     half_elem(in_dtype));
}

int fke_select_mfma_tile(int M, int N, int K, int b_layout, int swiglu, int cus) {
    if (M < 1 || N < 1 || K < 1 || (b_layout != FKE_B_NK && b_layout != FKE_B_KN) || (swiglu && N % 2)) return -1;
    GemmArgs p = make_args(nullptr, nullptr, nullptr, M, N, K, nullptr, nullptr, 1.f, 1.f, nullptr, FKE_OUT_F32,
                           b_layout);
    p.swiglu = swiglu ? 1 : 0;
    if (cus <= 0) cus = fke::device_cus();
    switch (fke::mfma_pick_tile(p, cus)) {
        case fke::MFMA_TILE_128x128: return FKE_PATH_MFMA_128x128;
        case fke::MFMA_TILE_128x128_RING4: return FKE_PATH_MFMA_128x128_RING4;
        case fke::MFMA_TILE_128x64_RING4: return FKE_PATH_MFMA_128x64_RING4;
        case fke::MFMA_TILE_64x64_RING4: return FKE_PATH_MFMA_64x64_RING4;
        default: return FKE_PATH_MFMA_256x256;
    }
}

int fke_select_mfma_split(int M, int N, int K, int b_layout, int cus, int* tile_path) {
    if (M < 1 || N < 1 || K < 1 || (b_layout != FKE_B_NK && b_layout != FKE_B_KN)) return -1;
    const GemmArgs p = make_args(nullptr, nullptr, nullptr, M, N, K, nullptr, nullptr, 1.f, 1.f, nullptr,
                                 FKE_OUT_BF16, b_layout);
    if (cus <= 0) cus = fke::device_cus();
    const fke::MfmaPlan pl = fke::mfma_plan(p, fke::ELEM_I8, cus);
    if (tile_path) {
        switch (pl.tile) {
            case fke::MFMA_TILE_128x128: *tile_path = FKE_PATH_MFMA_128x128; break;
            case fke::MFMA_TILE_128x128_RING4: *tile_path = FKE_PATH_MFMA_128x128_RING4; break;
            case fke::MFMA_TILE_128x64_RING4: *tile_path = FKE_PATH_MFMA_128x64_RING4; break;
            case fke::MFMA_TILE_64x64_RING4: *tile_path = FKE_PATH_MFMA_64x64_RING4; break;
            default: *tile_path = FKE_PATH_MFMA_256x256;
        }
    }
    return pl.S;
}

// Reference src/tensor_core_attention.cu:13-86 (launch_wmma_gemm_fp16): A fp16
// [M,K], B fp16 [N,K] ("column-major K x N"), C fp32 = alpha * A.B^T; beta is
// accepted and, as there, unused (C is overwritten).
int fke_launch_wmma_gemm_fp16(const void* d_A, const void* d_B, float* d_C, int M, int N, int K, float alpha,
                              float beta, void* stream) {
    (void)beta;
    return fke_gemm_half(d_A, d_B, d_C, M, N, K, FKE_IN_F16, nullptr, nullptr, alpha, 1.0f, nullptr, FKE_OUT_F32,
                         FKE_B_NK, stream);
}

int fke_select_path_i8(const void* A, const void* B, const void* C, int M, int N, int K,
                       int out_dtype, int b_layout) {
    if (!i8_args_ok(A, B, C, M, N, K, out_dtype, b_layout)) return -1;
    return pick_i8(make_args(A, B, const_cast<void*>(C), M, N, K, nullptr, nullptr, 1.f, 1.f, nullptr,
                             out_dtype, b_layout));
}

int fke_select_path_f8(const void* A, const void* B, const void* C, int M, int N, int K,
                       int out_dtype, int b_layout) {
    if (!f8_args_ok(A, B, C, M, N, K, out_dtype, b_layout)) return -1;
    return pick_f8(make_args(A, B, const_cast<void*>(C), M, N, K, nullptr, nullptr, 1.f, 1.f, nullptr,
                             out_dtype, b_layout));
}

int fke_quantize_rows_i8(const void* X, int in_dtype, int M, int K, int8_t* Q, float* scale,
                         void* stream) {
    if (!X || !Q || !scale || M < 1 || K < 1) return hipErrorInvalidValue;
    if (in_dtype != FKE_IN_F32 && in_dtype != FKE_IN_BF16) return hipErrorInvalidValue;
    return fke::launch_quant_rows(X, in_dtype, M, K, Q, scale, static_cast<hipStream_t>(stream));
}

// Reference src/quantized_gemm.cu:56-75: B [N,K], fp32 out, alpha = sa*sb.
int fke_launch_int8_gemm_dp4a(const int8_t* d_A, const int8_t* d_B, float* d_C, float scale_a,
                              float scale_b, int M, int N, int K, void* stream) {
    if (K % 4 != 0) return hipErrorInvalidValue;
    return fke_qgemm_i8(d_A, d_B, d_C, M, N, K, nullptr, nullptr, scale_a, scale_b, nullptr,
                        FKE_OUT_F32, FKE_B_NK, stream);
}

// Reference src/quantized_gemm.cu:120-139: B [K,N], fp32 out, alpha = sa*sb.
int fke_launch_fp8_gemm_scaled(const uint8_t* d_A, const uint8_t* d_B, float* d_C, float scale_a,
                               float scale_b, int M, int N, int K, void* stream) {
    return fke_qgemm_f8(d_A, d_B, d_C, M, N, K, scale_a, scale_b, nullptr, FKE_OUT_F32, FKE_B_KN,
                        stream);
}

// Reference src/flash_engine_api.cu:7-27, with the properties that matter on
// CDNA (architecture name, CUs, wavefront size, LDS).
int fke_print_device_info(int device_id) {
    hipDeviceProp_t prop;
    hipError_t err = hipGetDeviceProperties(&prop, device_id);
    if (err != hipSuccess) return err;
    printf("========================================================\n");
    printf(" FlashKernel-Engine (MI355X build) GPU Diagnostics\n");
    printf("========================================================\n");
    printf(" Device:                        %s\n", prop.name);
    printf(" Architecture:                  %s\n", prop.gcnArchName);
    printf(" Compute Units:                 %d\n", prop.multiProcessorCount);
    printf(" Wavefront Size:                %d\n", prop.warpSize);
    printf(" Max Threads Per CU:            %d\n", prop.maxThreadsPerMultiProcessor);
    printf(" Max Threads Per Block:         %d\n", prop.maxThreadsPerBlock);
    printf(" LDS Per Block:                 %.1f KB\n", prop.sharedMemPerBlock / 1024.0);
    printf(" LDS Per CU:                    %.1f KB\n", prop.maxSharedMemoryPerMultiProcessor / 1024.0);
    printf(" Total Global Memory:           %.2f GB\n", prop.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
    printf(" Memory Bus Width:              %d bits\n", prop.memoryBusWidth);
    printf(" Peak Memory Clock:             %.1f MHz\n", prop.memoryClockRate * 1e-3);
    printf(" Peak Engine Clock:             %.1f MHz\n", prop.clockRate * 1e-3);
    printf("========================================================\n");
    fflush(stdout);
    return hipSuccess;
}

const char* fke_version(void) { return "1.2.0"; }

const char* fke_status_string(int status) {
    return hipGetErrorString(static_cast<hipError_t>(status));
}

}  // extern "C"
