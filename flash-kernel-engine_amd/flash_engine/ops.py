"""Quantized GEMM operations of the MI355X build (torch tensors on a ROCm GPU).

`quantized_gemm_int8` keeps the signature and the arithmetic of reference
python/flash_engine/ops.py:180-186 (C = (A_int8 @ B_int8) * (scale_a*scale_b),
B stored [K,N], fp32 result) but runs the HIP kernels of libfke_qgemm.so
through its C ABI; host (numpy) inputs are copied to the GPU and the result
copied back.  The checks before each call follow the reference binding idiom
(python/bindings.cpp:101-133: device/shape checks, a fresh output tensor, the
current stream).  Every op runs the HIP kernels; without the built library the
load of the library raises.  The one host computation is the reference op's
own numpy arithmetic in `quantized_gemm_int8`, taken only for numpy inputs on
a machine with no visible GPU.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _ext, _lib
from ._lib import (B_KN, B_NK, OUT_BF16, OUT_F32, OUT_I32, PATH_AUTO, PATH_GEMV, PATH_GEMV_DOT, PATH_GENERIC,
                   PATH_MFMA, PATH_MFMA_64x64_RING4, PATH_MFMA_128x64_RING4, PATH_MFMA_128x128,
                   PATH_MFMA_128x128_RING4, PATH_MFMA_256x256)

_OUT_CODES = {torch.float32: OUT_F32, torch.bfloat16: OUT_BF16, torch.int32: OUT_I32}
_LAYOUTS = {"nk": B_NK, "kn": B_KN}
_PATHS = {"auto": PATH_AUTO, "gemv": PATH_GEMV, "mfma": PATH_MFMA, "generic": PATH_GENERIC,
          "gemv_dot": PATH_GEMV_DOT, "mfma_256x256": PATH_MFMA_256x256, "mfma_128x128": PATH_MFMA_128x128,
          "mfma_128x128_ring4": PATH_MFMA_128x128_RING4, "mfma_128x64_ring4": PATH_MFMA_128x64_RING4,
          "mfma_64x64_ring4": PATH_MFMA_64x64_RING4}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check_dev(name: str, t: torch.Tensor, dtype, device) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _check_vec(name: str, t, n: int, device) -> None:
    if t is None:
        return
    _check_dev(name, t, torch.float32, device)
    if t.numel() != n:
        raise ValueError(f"{name} must have {n} elements, got {t.numel()}")


def w8a8_gemm(A: torch.Tensor, B: torch.Tensor, scale_a=None, scale_b=None, bias=None,
              out_dtype=torch.bfloat16, b_layout: str = "nk", sa: float = 1.0, sb: float = 1.0,
              path: str = "auto", out: torch.Tensor | None = None) -> torch.Tensor:
    """W8A8 INT8 GEMM with the fused epilogue.

    acc = A[M,K] . B  (exact int32; B is [N,K] for b_layout="nk", [K,N] for "kn")
    y   = fp32(acc) * fp32(scale_a[m] * scale_b[n])  (+ bias[n] via one fma)
    out = y as fp32 / bf16 (round to nearest even), or acc as int32.
    scale_a [M], scale_b [N], bias [N] are fp32 GPU tensors or None (then the
    scalars sa / sb apply to every row / column).
    """
    dev = A.device
    _check_dev("A", A, torch.int8, dev)
    _check_dev("B", B, torch.int8, dev)
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("A and B must be 2-D")
    layout = _LAYOUTS[b_layout]
    M, K = A.shape
    N, KB = (B.shape[0], B.shape[1]) if layout == B_NK else (B.shape[1], B.shape[0])
    if KB != K:
        raise ValueError(f"K mismatch: A has {K}, B has {KB}")
    _check_vec("scale_a", scale_a, M, dev)
    _check_vec("scale_b", scale_b, N, dev)
    _check_vec("bias", bias, N, dev)
    code = _OUT_CODES[out_dtype]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    else:
        _check_dev("out", out, out_dtype, dev)
        if tuple(out.shape) != (M, N):
            raise ValueError("out has the wrong shape")
    st = _lib.lib().fke_qgemm_i8_on_path(
        _PATHS[path], A.data_ptr(), B.data_ptr(), out.data_ptr(), M, N, K, _ptr(scale_a),
        _ptr(scale_b), sa, sb, _ptr(bias), code, layout, _stream(A))
    _lib.check(st, "fke_qgemm_i8")
    return out


def fp8_gemm_scaled(A: torch.Tensor, B: torch.Tensor, scale_a: float, scale_b: float, bias=None,
                    out_dtype=torch.float32, b_layout: str = "kn", path: str = "auto",
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Scaled FP8 E4M3 GEMM (reference src/quantized_gemm.cu:99-139).

    sum = sum_k dec(A[m,k]) * dec(B(k,n)) in fp32, y = sum * fp32(scale_a*scale_b)
    (+ bias[n] via one fma); codes 0x7F/0xFF decode to 0.0 like the reference.
    A is [M,K] and B is [K,N] ("kn", the reference layout) or [N,K] ("nk"),
    as torch.uint8 codes or torch.float8_e4m3fn.
    """
    dev = A.device
    if A.dtype == torch.float8_e4m3fn:
        A = A.view(torch.uint8)
    if B.dtype == torch.float8_e4m3fn:
        B = B.view(torch.uint8)
    _check_dev("A", A, torch.uint8, dev)
    _check_dev("B", B, torch.uint8, dev)
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("A and B must be 2-D")
    layout = _LAYOUTS[b_layout]
    M, K = A.shape
    N, KB = (B.shape[0], B.shape[1]) if layout == B_NK else (B.shape[1], B.shape[0])
    if KB != K:
        raise ValueError(f"K mismatch: A has {K}, B has {KB}")
    _check_vec("bias", bias, N, dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("FP8 GEMM writes fp32 or bf16")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    else:
        _check_dev("out", out, out_dtype, dev)
        if tuple(out.shape) != (M, N):
            raise ValueError(f"out must be [{M}, {N}], got {tuple(out.shape)}")
    st = _lib.lib().fke_qgemm_f8_on_path(
        _PATHS[path], A.data_ptr(), B.data_ptr(), out.data_ptr(), M, N, K, scale_a, scale_b,
        _ptr(bias), _OUT_CODES[out_dtype], layout, _stream(A))
    _lib.check(st, "fke_qgemm_f8")
    return out


def quantize_per_token(x: torch.Tensor, q: torch.Tensor | None = None,
                       scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token symmetric INT8 quantisation of activations x [M,K] (fp32 or bf16).

    scale[m] = fp32(max_k |x[m,k]| / 127), r = fp32(127 / max_k |x[m,k]|) (both 1
    for an all-zero row) and q[m,k] = clamp(round_half_even(fp32(x[m,k] * r)), -127, 127),
    so x ~= q * scale.
    Returns (q int8 [M,K], scale fp32 [M]) on x's device, ready to be the A and
    scale_a of `w8a8_gemm`.  No reference counterpart: the reference's quantized
    GEMMs take int8 inputs with scalar scales.
    """
    dev = x.device
    codes = {torch.float32: _lib.IN_F32, torch.bfloat16: _lib.IN_BF16}
    if x.dtype not in codes:
        raise TypeError(f"x must be float32 or bfloat16, got {x.dtype}")
    _check_dev("x", x, x.dtype, dev)
    if x.dim() != 2:
        raise ValueError("x must be 2-D [M,K]")
    M, K = x.shape
    if q is None:
        q = torch.empty((M, K), dtype=torch.int8, device=dev)
    else:
        _check_dev("q", q, torch.int8, dev)
        if tuple(q.shape) != (M, K):
            raise ValueError(f"q must be [{M}, {K}], got {tuple(q.shape)}")
    if scale is None:
        scale = torch.empty(M, dtype=torch.float32, device=dev)
    else:
        _check_vec("scale", scale, M, dev)
    st = _lib.lib().fke_quantize_rows_i8(x.data_ptr(), codes[x.dtype], M, K, q.data_ptr(),
                                         scale.data_ptr(), _stream(x))
    _lib.check(st, "fke_quantize_rows_i8")
    return q, scale


_IN_CODES = {torch.float32: _lib.IN_F32, torch.bfloat16: _lib.IN_BF16}


def _float_linear(fn: str, x, weight, weight_scale, bias, out_dtype, n_vec: int, out_cols: int) -> torch.Tensor:
    """Shared body of w8a8_linear / w8a8_gate_up_swiglu: one C call
    (fke_w8a8_linear / fke_w8a8_swiglu_linear) that quantises x per token into
    a workspace and runs the W8A8 GEMM on it."""
    dev = x.device
    if x.dtype not in _IN_CODES:
        raise TypeError(f"x must be float32 or bfloat16, got {x.dtype}")
    _check_dev("x", x, x.dtype, dev)
    _check_dev("weight", weight, torch.int8, dev)
    if x.dim() != 2 or weight.dim() != 2 or weight.shape[1] != x.shape[1]:
        raise ValueError("x must be [M,K] and weight [N,K]")
    _check_vec("weight_scale", weight_scale, n_vec, dev)
    _check_vec("bias", bias, n_vec, dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("out_dtype must be float32 or bfloat16")
    M, K = x.shape
    L = _lib.lib()
    out = torch.empty((M, out_cols), dtype=out_dtype, device=dev)
    ws = torch.empty(L.fke_w8a8_linear_workspace_size(M, K), dtype=torch.uint8, device=dev)
    st = getattr(L, fn)(x.data_ptr(), _IN_CODES[x.dtype], weight.data_ptr(), out.data_ptr(), M, out_cols, K,
                        _ptr(weight_scale), 1.0, _ptr(bias), _OUT_CODES[out_dtype], ws.data_ptr(), ws.numel(),
                        _stream(x))
    _lib.check(st, fn)
    return out


def w8a8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, bias=None,
                out_dtype=torch.bfloat16) -> torch.Tensor:
    """y = x . W^T with W8A8 quantisation: x [M,K] fp32/bf16 activations are
    quantised per token (as `quantize_per_token`), weight [N,K] int8 carries
    per-channel scales weight_scale [N]; bias [N] fp32 optional.  Equal, bit for
    bit, to `w8a8_gemm(*quantize_per_token(x), ...)`: the quantiser and the GEMM,
    two launches on the current stream through one C call."""
    return _float_linear("fke_w8a8_linear", x, weight, weight_scale, bias, out_dtype, weight.shape[0],
                         weight.shape[0])


def w8a8_swiglu(A: torch.Tensor, W: torch.Tensor, scale_a=None, scale_b=None, bias=None,
                out_dtype=torch.bfloat16, sa: float = 1.0, sb: float = 1.0, path: str = "auto",
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Gate/up projection with SwiGLU fused into the GEMM epilogue.

    W is the merged int8 weight [2I, K]: rows 0..I-1 project the gate, rows
    I..2I-1 the up branch (nn.Linear layout).  With the `w8a8_gemm` epilogue
    g = y(A, W[n]) and u = y(A, W[I+n]) (scale_b / bias [2I], indexed by
    weight row), out[m, n] = (g * sigmoid(g)) * u for n < I, fp32 or bf16
    [M, I]; equal to `fused_swiglu` of the two fp32 GEMM outputs.
    """
    dev = A.device
    _check_dev("A", A, torch.int8, dev)
    _check_dev("W", W, torch.int8, dev)
    if A.dim() != 2 or W.dim() != 2:
        raise ValueError("A and W must be 2-D")
    M, K = A.shape
    if W.shape[1] != K or W.shape[0] % 2:
        raise ValueError(f"W must be [2I, {K}], got {tuple(W.shape)}")
    I = W.shape[0] // 2
    _check_vec("scale_a", scale_a, M, dev)
    _check_vec("scale_b", scale_b, 2 * I, dev)
    _check_vec("bias", bias, 2 * I, dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("the SwiGLU GEMM writes fp32 or bf16")
    if out is None:
        out = torch.empty((M, I), dtype=out_dtype, device=dev)
    else:
        _check_dev("out", out, out_dtype, dev)
        if tuple(out.shape) != (M, I):
            raise ValueError("out has the wrong shape")
    st = _lib.lib().fke_qgemm_i8_swiglu_on_path(
        _PATHS[path], A.data_ptr(), W.data_ptr(), out.data_ptr(), M, I, K, _ptr(scale_a), _ptr(scale_b),
        sa, sb, _ptr(bias), _OUT_CODES[out_dtype], _stream(A))
    _lib.check(st, "fke_qgemm_i8_swiglu")
    return out


def w8a8_gate_up_swiglu(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, bias=None,
                        out_dtype=torch.bfloat16) -> torch.Tensor:
    """The gate/up half of a SwiGLU MLP in W8A8: x [M,K] fp32/bf16 is quantised
    per token and silu(x W_gate^T) * (x W_up^T) is computed from the merged
    weight [2I, K] with per-channel scales weight_scale [2I]: the quantiser, then
    the fused gate/up GEMM."""
    if weight.dim() != 2 or weight.shape[0] % 2:
        raise ValueError("weight must be [2I, K]")
    return _float_linear("fke_w8a8_swiglu_linear", x, weight, weight_scale, bias, out_dtype, weight.shape[0],
                         weight.shape[0] // 2)


def gemm_half(A: torch.Tensor, B: torch.Tensor, scale_a=None, scale_b=None, bias=None,
              out_dtype=torch.float32, b_layout: str = "nk", sa: float = 1.0, sb: float = 1.0,
              path: str = "auto", out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 / bf16 GEMM on the MFMA tile engine (extends reference
    src/tensor_core_attention.cu:13-86, launch_wmma_gemm_fp16).

    acc = A[M,K] . B in fp32 (B [N,K] for "nk", [K,N] for "kn"; A and B both
    float16 or both bfloat16), y = acc * fp32(scale_a[m] * scale_b[n]) (+ bias[n]
    via one fma), out fp32 or bf16 [M,N].  With sa = alpha and no vectors this is
    the reference's C = alpha * A B^T.
    """
    dev = A.device
    codes = {torch.float16: _lib.IN_F16, torch.bfloat16: _lib.IN_BF16}
    if A.dtype not in codes:
        raise TypeError(f"A must be float16 or bfloat16, got {A.dtype}")
    _check_dev("A", A, A.dtype, dev)
    _check_dev("B", B, A.dtype, dev)
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("A and B must be 2-D")
    layout = _LAYOUTS[b_layout]
    M, K = A.shape
    N, KB = (B.shape[0], B.shape[1]) if layout == B_NK else (B.shape[1], B.shape[0])
    if KB != K:
        raise ValueError(f"K mismatch: A has {K}, B has {KB}")
    _check_vec("scale_a", scale_a, M, dev)
    _check_vec("scale_b", scale_b, N, dev)
    _check_vec("bias", bias, N, dev)
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("the half GEMM writes fp32 or bf16")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    else:
        _check_dev("out", out, out_dtype, dev)
        if tuple(out.shape) != (M, N):
            raise ValueError("out has the wrong shape")
    st = _lib.lib().fke_gemm_half_on_path(
        _PATHS[path], A.data_ptr(), B.data_ptr(), out.data_ptr(), M, N, K, codes[A.dtype], _ptr(scale_a),
        _ptr(scale_b), sa, sb, _ptr(bias), _OUT_CODES[out_dtype], layout, _stream(A))
    _lib.check(st, "fke_gemm_half")
    return out


def fused_swiglu(gate, up):
    """(gate * sigmoid(gate)) * up, elementwise (reference python/flash_engine/ops.py:218-230,
    src/fused_activations.cu).  float32, float16 or bfloat16 GPU tensors of one
    shape; computed in fp32 and rounded once to the input type.  numpy inputs
    are copied to cuda:0 and the result returned as numpy."""
    host = isinstance(gate, np.ndarray)
    if host:
        gate = torch.from_numpy(np.ascontiguousarray(gate)).cuda()
        up = torch.from_numpy(np.ascontiguousarray(up)).cuda()
    out = _ext.ext().fused_swiglu_forward(gate.contiguous(), up.contiguous())
    return out.cpu().numpy() if host else out


def _host_int8(x, name: str) -> np.ndarray:
    """A numpy operand as contiguous int8 for the GPU path.  The reference
    widens its inputs with astype(np.int32) (python/flash_engine/ops.py:184), so
    an integer array whose values lie outside [-128, 127] would give a
    different product after a narrowing cast: it is rejected instead."""
    x = np.asarray(x)
    if x.dtype == np.int8:
        return np.ascontiguousarray(x)
    if not np.issubdtype(x.dtype, np.integer):
        raise TypeError(f"{name} must hold integers (int8 values), got {x.dtype}")
    if x.size and (int(x.min()) < -128 or int(x.max()) > 127):
        raise ValueError(f"{name} has values outside the int8 range [-128, 127]")
    return np.ascontiguousarray(x, dtype=np.int8)


def quantized_gemm_int8(A, B, scale_a: float = 1.0, scale_b: float = 1.0):
    """C = (A_int8 @ B_int8) * (scale_a * scale_b), B stored [K,N], fp32 out.

    Same signature and result as reference python/flash_engine/ops.py:180-186:
    the scale product is formed in double (Python floats) and applied as fp32,
    the int32 product is exact.  GPU tensors stay on the GPU and run the HIP
    kernels.  numpy arrays are copied to cuda:0 and the result is returned as a
    numpy array.  Only on a machine where no GPU is visible at all do numpy
    inputs take the reference op's own host arithmetic (an int32 numpy matmul,
    as there), so CPU-only callers of the reference op keep working; wherever a
    GPU is visible the HIP path runs, and a missing HIP library raises.
    """
    host = isinstance(A, np.ndarray) or isinstance(B, np.ndarray)
    if host and not torch.cuda.is_available():
        acc = np.asarray(A).astype(np.int32) @ np.asarray(B).astype(np.int32)
        return acc.astype(np.float32) * (scale_a * scale_b)
    if host:
        A = torch.from_numpy(_host_int8(A, "A")).cuda()
        B = torch.from_numpy(_host_int8(B, "B")).cuda()
    alpha = float(np.float32(float(scale_a) * float(scale_b)))
    # the compiled binding, as the reference op calls its extension (ops.py:10-13)
    out = _ext.ext().quantized_gemm_int8_forward(A.contiguous(), B.contiguous(), None, None, None,
                                                 torch.float32, "kn", alpha, 1.0)
    if host:
        return out.cpu().numpy()
    return out


def print_device_info(device_id: int = 0) -> None:
    _lib.check(_lib.lib().fke_print_device_info(device_id), "fke_print_device_info")
