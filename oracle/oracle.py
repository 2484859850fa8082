"""numpy front end for the CPU oracle (liboracle.so, built from fke_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The shipped library never
imports this module.  Each wrapper names the reference file:line its C
function restates.
"""
from __future__ import annotations

import ctypes as ct
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")

OUT_F32, OUT_BF16, OUT_I32 = 0, 1, 2
B_NK, B_KN = 0, 1
HALF_BF16, HALF_F16 = 1, 2  # in_dtype codes of gemm_half (fke_in_dtype values)

_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = ct.CDLL(_SO)
        _declare(_lib)
    return _lib


_p = ct.c_void_p
_i = ct.c_int
_f = ct.c_float
_d = ct.c_double
_sz = ct.c_size_t
_u64 = ct.c_uint64


def _declare(L):
    L.fko_splitmix64.argtypes = [ct.POINTER(_u64)]
    L.fko_splitmix64.restype = _u64
    L.fko_gen_i8_uniform.argtypes = [_p, _sz, _u64]
    L.fko_gen_i8_clipped_normal.argtypes = [_p, _sz, _u64, _d]
    L.fko_gen_f32_uniform.argtypes = [_p, _sz, _u64, _d, _d]
    L.fko_gen_f32_normal.argtypes = [_p, _sz, _u64, _d, _d]
    L.fko_ref_host_gemm_i8.argtypes = [_p, _p, _p, _i, _i, _i, _f, _f]
    L.fko_ref_kernel_gemm_i8.argtypes = [_p, _p, _p, _i, _i, _i, _f, _f]
    L.fko_e4m3_decode.argtypes = [ct.c_uint8]
    L.fko_e4m3_decode.restype = _f
    L.fko_ref_kernel_gemm_f8.argtypes = [_p, _p, _p, _i, _i, _i, _f, _f]
    L.fko_ref_py_gemm_i8.argtypes = [_p, _p, _p, _i, _i, _i, _d, _d]
    L.fko_w8a8_acc.argtypes = [_p, _p, _p, _i, _i, _i, _i, _p, _i, _i]
    L.fko_w8a8_epilogue.argtypes = [_p, _p, _i, _i, _p, _p, _f, _f, _p, _i, _p]
    L.fko_f8_gemm.argtypes = [_p, _p, _p, _i, _i, _i, _f, _f, _p, _i, _i, _p, _i, _i]
    L.fko_f32_to_bf16_rne.argtypes = [_f]
    L.fko_f32_to_bf16_rne.restype = ct.c_uint16
    L.fko_f32_to_e4m3_sat.argtypes = [_f]
    L.fko_f32_to_e4m3_sat.restype = ct.c_uint8
    L.fko_quantize_e4m3.argtypes = [_p, _p, _sz]
    L.fko_quantize_rows_i8.argtypes = [_p, _i, _i, _i, _p, _p]
    L.fko_quantize_rows_i8.restype = None
    L.fko_quantize_e4m3.restype = _f
    L.fko_swiglu1.argtypes = [_f, _f]
    L.fko_swiglu1.restype = _f
    L.fko_swiglu_f32.argtypes = [_p, _p, _p, _sz]
    L.fko_swiglu_f32.restype = None
    L.fko_w8a8_swiglu.argtypes = [_p, _p, _p, _i, _i, _i, _p, _p, _f, _f, _p, _i, _p, _i, _i]
    L.fko_w8a8_swiglu.restype = None
    L.fko_f16_to_f32.argtypes = [ct.c_uint16]
    L.fko_f16_to_f32.restype = _f
    L.fko_gemm_half.argtypes = [_p, _p, _p, _i, _i, _i, _i, _p, _p, _f, _f, _p, _i, _i, _p, _i, _i]
    L.fko_gemm_half.restype = None


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---- generators -----------------------------------------------------------

def splitmix64_stream(seed: int, n: int) -> list[int]:
    s = _u64(seed)
    return [int(lib().fko_splitmix64(ct.byref(s))) for _ in range(n)]


def gen_i8_uniform(shape, seed: int) -> np.ndarray:
    out = np.empty(shape, dtype=np.int8)
    lib().fko_gen_i8_uniform(_ptr(out), out.size, seed)
    return out


def gen_i8_clipped_normal(shape, seed: int, sigma: float = 30.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.int8)
    lib().fko_gen_i8_clipped_normal(_ptr(out), out.size, seed, sigma)
    return out


def gen_f32_uniform(shape, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().fko_gen_f32_uniform(_ptr(out), out.size, seed, lo, hi)
    return out


def gen_f32_normal(shape, seed: int, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().fko_gen_f32_normal(_ptr(out), out.size, seed, mu, sigma)
    return out


# ---- reference restatements ------------------------------------------------

def ref_host_gemm_i8(A, B_nk, scale_a: float, scale_b: float) -> np.ndarray:
    """tests/test_quantized_gemm.cu:39-48 (B is [N,K])."""
    A = _c(A, np.int8); B_nk = _c(B_nk, np.int8)
    M, K = A.shape; N = B_nk.shape[0]
    C = np.empty((M, N), dtype=np.float32)
    lib().fko_ref_host_gemm_i8(_ptr(A), _ptr(B_nk), _ptr(C), M, N, K, scale_a, scale_b)
    return C


def ref_kernel_gemm_i8(A, B_nk, scale_a: float, scale_b: float) -> np.ndarray:
    """src/quantized_gemm.cu:15-54 (K/4 word truncation included)."""
    A = _c(A, np.int8); B_nk = _c(B_nk, np.int8)
    M, K = A.shape; N = B_nk.shape[0]
    C = np.empty((M, N), dtype=np.float32)
    lib().fko_ref_kernel_gemm_i8(_ptr(A), _ptr(B_nk), _ptr(C), M, N, K, scale_a, scale_b)
    return C


def e4m3_decode(code: int) -> float:
    """src/quantized_gemm.cu:81-97."""
    return float(lib().fko_e4m3_decode(code))


def e4m3_decode_table() -> np.ndarray:
    return np.array([e4m3_decode(i) for i in range(256)], dtype=np.float32)


def ref_kernel_gemm_f8(A, B_kn, scale_a: float, scale_b: float) -> np.ndarray:
    """src/quantized_gemm.cu:99-118 (B is [K,N], sequential fp32 sum)."""
    A = _c(A, np.uint8); B_kn = _c(B_kn, np.uint8)
    M, K = A.shape; N = B_kn.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    lib().fko_ref_kernel_gemm_f8(_ptr(A), _ptr(B_kn), _ptr(C), M, N, K, scale_a, scale_b)
    return C


def ref_py_gemm_i8(A, B_kn, scale_a: float = 1.0, scale_b: float = 1.0) -> np.ndarray:
    """python/flash_engine/ops.py:180-186 (B is [K,N])."""
    A = _c(A, np.int8); B_kn = _c(B_kn, np.int8)
    M, K = A.shape; N = B_kn.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    lib().fko_ref_py_gemm_i8(_ptr(A), _ptr(B_kn), _ptr(C), M, N, K, scale_a, scale_b)
    return C


# ---- extended W8A8 / FP8 -----------------------------------------------------

def w8a8_acc(A, B, b_layout: int = B_NK, rows=None, nthreads: int = 0) -> np.ndarray:
    A = _c(A, np.int8); B = _c(B, np.int8)
    M, K = A.shape
    N = B.shape[0] if b_layout == B_NK else B.shape[1]
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    R = M if r is None else r.size
    acc = np.empty((R, N), dtype=np.int32)
    nt = nthreads or (os.cpu_count() or 1)
    lib().fko_w8a8_acc(_ptr(A), _ptr(B), _ptr(acc), M, N, K, b_layout, _ptr(r),
                       0 if r is None else r.size, nt)
    return acc


def w8a8_epilogue(acc, scale_a=None, scale_b=None, sa: float = 1.0, sb: float = 1.0,
                  bias=None, out_dtype: int = OUT_F32, rows=None) -> np.ndarray:
    acc = _c(acc, np.int32)
    R, N = acc.shape
    dt = {OUT_F32: np.float32, OUT_BF16: np.uint16, OUT_I32: np.int32}[out_dtype]
    out = np.empty((R, N), dtype=dt)
    sa_arr, sb_arr, b_arr = _c(scale_a, np.float32), _c(scale_b, np.float32), _c(bias, np.float32)
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    lib().fko_w8a8_epilogue(_ptr(acc), _ptr(out), R, N, _ptr(sa_arr), _ptr(sb_arr), sa, sb,
                            _ptr(b_arr), out_dtype, _ptr(r))
    return out


def w8a8_gemm(A, B, scale_a=None, scale_b=None, sa: float = 1.0, sb: float = 1.0, bias=None,
              out_dtype: int = OUT_F32, b_layout: int = B_NK, rows=None, nthreads: int = 0):
    acc = w8a8_acc(A, B, b_layout, rows, nthreads)
    return w8a8_epilogue(acc, scale_a, scale_b, sa, sb, bias, out_dtype, rows)


def f8_gemm(A, B, sa: float, sb: float, bias=None, out_dtype: int = OUT_F32,
            b_layout: int = B_KN, rows=None, nthreads: int = 0) -> np.ndarray:
    A = _c(A, np.uint8); B = _c(B, np.uint8)
    M, K = A.shape
    N = B.shape[0] if b_layout == B_NK else B.shape[1]
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    R = M if r is None else r.size
    dt = {OUT_F32: np.float32, OUT_BF16: np.uint16}[out_dtype]
    out = np.empty((R, N), dtype=dt)
    b_arr = _c(bias, np.float32)
    nt = nthreads or (os.cpu_count() or 1)
    lib().fko_f8_gemm(_ptr(A), _ptr(B), _ptr(out), M, N, K, sa, sb, _ptr(b_arr), out_dtype,
                      b_layout, _ptr(r), 0 if r is None else r.size, nt)
    return out


def f32_to_bf16_rne(x: float) -> int:
    return int(lib().fko_f32_to_bf16_rne(x))


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_e4m3_sat(x: float) -> int:
    return int(lib().fko_f32_to_e4m3_sat(x))


def quantize_e4m3(x) -> tuple[np.ndarray, float]:
    x = _c(x, np.float32)
    q = np.empty(x.shape, dtype=np.uint8)
    s = lib().fko_quantize_e4m3(_ptr(x), _ptr(q), x.size)
    return q, float(s)


IN_F32, IN_BF16 = 0, 1


def quantize_rows_i8(x, in_dtype: int = IN_F32) -> tuple[np.ndarray, np.ndarray]:
    """Per-token INT8 quantiser: x [M,K] fp32 (IN_F32) or bf16 bits as uint16
    (IN_BF16) -> (q int8 [M,K], scale fp32 [M])."""
    x = _c(x, np.float32 if in_dtype == IN_F32 else np.uint16)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.int8)
    s = np.empty(M, dtype=np.float32)
    lib().fko_quantize_rows_i8(_ptr(x), in_dtype, M, K, _ptr(q), _ptr(s))
    return q, s


# ---- SwiGLU --------------------------------------------------------------------

def swiglu_f32(gate, up) -> np.ndarray:
    """src/fused_activations.cu:9-35: (g * sigmoid(g)) * u elementwise, fp32."""
    g = _c(gate, np.float32); u = _c(up, np.float32)
    assert g.shape == u.shape
    h = np.empty_like(g)
    lib().fko_swiglu_f32(_ptr(g), _ptr(u), _ptr(h), g.size)
    return h


def w8a8_swiglu(A, W, scale_a=None, scale_b=None, sa: float = 1.0, sb: float = 1.0, bias=None,
                out_dtype: int = OUT_F32, rows=None, nthreads: int = 0) -> np.ndarray:
    """W8A8 gate/up GEMM + SwiGLU: W is [2I, K] (gate rows, then up rows); out [R, I]."""
    A = _c(A, np.int8); W = _c(W, np.int8)
    M, K = A.shape
    I = W.shape[0] // 2
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    R = M if r is None else r.size
    out = np.empty((R, I), dtype=np.float32 if out_dtype == OUT_F32 else np.uint16)
    sa_arr, sb_arr, b_arr = _c(scale_a, np.float32), _c(scale_b, np.float32), _c(bias, np.float32)
    nt = nthreads or (os.cpu_count() or 1)
    lib().fko_w8a8_swiglu(_ptr(A), _ptr(W), _ptr(out), M, I, K, _ptr(sa_arr), _ptr(sb_arr), sa, sb,
                          _ptr(b_arr), out_dtype, _ptr(r), 0 if r is None else r.size, nt)
    return out


# ---- fp16 / bf16 GEMM ------------------------------------------------------------

def f16_to_f32(bits) -> np.ndarray:
    """IEEE binary16 codes -> fp32 (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return np.array([lib().fko_f16_to_f32(int(v)) for v in b.ravel()], dtype=np.float32).reshape(b.shape)


def gemm_half(A, B, in_dtype: int, scale_a=None, scale_b=None, sa: float = 1.0, sb: float = 1.0, bias=None,
              out_dtype: int = OUT_F32, b_layout: int = B_NK, rows=None, nthreads: int = 0) -> np.ndarray:
    """fp16 (in_dtype HALF_F16) / bf16 (HALF_BF16) GEMM on raw uint16 codes,
    sequential fp32 sum (src/tensor_core_attention.cu:13-66 restated)."""
    A = _c(A, np.uint16); B = _c(B, np.uint16)
    M, K = A.shape
    N = B.shape[0] if b_layout == B_NK else B.shape[1]
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    R = M if r is None else r.size
    out = np.empty((R, N), dtype=np.float32 if out_dtype == OUT_F32 else np.uint16)
    sa_arr, sb_arr, b_arr = _c(scale_a, np.float32), _c(scale_b, np.float32), _c(bias, np.float32)
    nt = nthreads or (os.cpu_count() or 1)
    lib().fko_gemm_half(_ptr(A), _ptr(B), _ptr(out), M, N, K, in_dtype, _ptr(sa_arr), _ptr(sb_arr), sa, sb,
                        _ptr(b_arr), out_dtype, b_layout, _ptr(r), 0 if r is None else r.size, nt)
    return out
