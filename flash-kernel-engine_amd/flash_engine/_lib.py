"""ctypes binding of libfke_qgemm.so (the C ABI declared in include/fke_qgemm.h).

This is the Python side of the drop-in boundary: plain pointers, sizes and a
stream handle cross it, nothing else.  Loading fails loudly if the HIP library
has not been built; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as ct
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "lib", "libfke_qgemm.so")

# enum values of include/fke_qgemm.h
OUT_F32, OUT_BF16, OUT_I32 = 0, 1, 2
B_NK, B_KN = 0, 1
PATH_AUTO, PATH_GEMV, PATH_MFMA, PATH_GENERIC, PATH_GEMV_DOT = 0, 1, 2, 3, 4
PATH_MFMA_256x256, PATH_MFMA_128x128, PATH_MFMA_128x128_RING4 = 5, 6, 7
PATH_MFMA_128x64_RING4, PATH_MFMA_64x64_RING4 = 8, 9
IN_F32, IN_BF16, IN_F16 = 0, 1, 2
HIP_SUCCESS, HIP_ERROR_INVALID_VALUE = 0, 1
W8A8_NOALLOC_SCRATCH_BYTES = 32 << 20  # FKE_W8A8_NOALLOC_SCRATCH_BYTES
SPLIT_SLOTS, SPLIT_SLOT_BYTES = 16, 16 << 20  # FKE_SPLIT_SLOTS, FKE_SPLIT_SLOT_BYTES
SPLIT_SMALL_SLOTS, SPLIT_SMALL_SLOT_BYTES = 48, 2 << 20  # FKE_SPLIT_SMALL_SLOTS, FKE_SPLIT_SMALL_SLOT_BYTES

# Every exported symbol with its (argtypes, restype).
_p, _i, _f = ct.c_void_p, ct.c_int, ct.c_float
SIGNATURES = {
    "fke_launch_int8_gemm_dp4a": ([_p, _p, _p, _f, _f, _i, _i, _i, _p], _i),
    "fke_launch_fp8_gemm_scaled": ([_p, _p, _p, _f, _f, _i, _i, _i, _p], _i),
    "fke_qgemm_i8": ([_p, _p, _p, _i, _i, _i, _p, _p, _f, _f, _p, _i, _i, _p], _i),
    "fke_qgemm_i8_on_path": ([_i, _p, _p, _p, _i, _i, _i, _p, _p, _f, _f, _p, _i, _i, _p], _i),
    "fke_qgemm_f8": ([_p, _p, _p, _i, _i, _i, _f, _f, _p, _i, _i, _p], _i),
    "fke_qgemm_f8_on_path": ([_i, _p, _p, _p, _i, _i, _i, _f, _f, _p, _i, _i, _p], _i),
    "fke_qgemm_workspace_size": ([_i, _i, _i, _i], ct.c_size_t),
    "fke_split_slots_in_use": ([], _i),
    "fke_qgemm_i8_ws": ([_p, _p, _p, _i, _i, _i, _p, _p, _f, _f, _p, _i, _i, _p, ct.c_size_t, _p], _i),
    "fke_qgemm_f8_ws": ([_p, _p, _p, _i, _i, _i, _f, _f, _p, _i, _i, _p, ct.c_size_t, _p], _i),
    "fke_quantize_rows_i8": ([_p, _i, _i, _i, _p, _p, _p], _i),
    "fke_swiglu": ([_p, _p, _p, ct.c_int64, _i, _p], _i),
    "fke_qgemm_i8_swiglu": ([_p, _p, _p, _i, _i, _i, _p, _p, _f, _f, _p, _i, _p], _i),
    "fke_qgemm_i8_swiglu_on_path": ([_i, _p, _p, _p, _i, _i, _i, _p, _p, _f, _f, _p, _i, _p], _i),
    "fke_select_path_i8_swiglu": ([_p, _p, _p, _i, _i, _i, _i], _i),
    "fke_gemm_half": ([_p, _p, _p, _i, _i, _i, _i, _p, _p, _f, _f, _p, _i, _i, _p], _i),
    "fke_gemm_half_on_path": ([_i, _p, _p, _p, _i, _i, _i, _i, _p, _p, _f, _f, _p, _i, _i, _p], _i),
    "fke_launch_wmma_gemm_fp16": ([_p, _p, _p, _i, _i, _i, _f, _f, _p], _i),
    "fke_select_path_half": ([_p, _p, _p, _i, _i, _i, _i, _i, _i], _i),
    "fke_select_mfma_tile": ([_i, _i, _i, _i, _i, _i], _i),
    "fke_select_mfma_split": ([_i, _i, _i, _i, _i, ct.POINTER(ct.c_int)], _i),
    "fke_w8a8_linear_workspace_size": ([_i, _i], ct.c_size_t),
    "fke_w8a8_linear": ([_p, _i, _p, _p, _i, _i, _i, _p, _f, _p, _i, _p, ct.c_size_t, _p], _i),
    "fke_w8a8_linear_noalloc": ([_p, _i, _p, _p, _i, _i, _i, _p, _f, _p, _i, _p], _i),
    "fke_w8a8_swiglu_linear": ([_p, _i, _p, _p, _i, _i, _i, _p, _f, _p, _i, _p, ct.c_size_t, _p], _i),
    "fke_select_path_i8": ([_p, _p, _p, _i, _i, _i, _i, _i], _i),
    "fke_select_path_f8": ([_p, _p, _p, _i, _i, _i, _i, _i], _i),
    "fke_print_device_info": ([_i], _i),
    "fke_version": ([], ct.c_char_p),
    "fke_status_string": ([_i], ct.c_char_p),
}

_lib = None


class FkeError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: status {status} ({status_string(status)})")


def lib() -> ct.CDLL:
    """Load libfke_qgemm.so once; raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libfke_qgemm.so not found at {LIB_PATH}; build it with "
                "`make -C flash-kernel-engine_amd/csrc` or __graft_entry__.build()")
        L = ct.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def status_string(status: int) -> str:
    s = lib().fke_status_string(status)
    return s.decode() if s else "unknown"


def check(status: int, what: str) -> None:
    if status != HIP_SUCCESS:
        raise FkeError(status, what)


def version() -> str:
    return lib().fke_version().decode()
