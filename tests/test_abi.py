"""CPU tests of the C-ABI boundary (libfke_qgemm.so): it loads, exports every
symbol include/fke_qgemm.h declares, rejects bad arguments with
hipErrorInvalidValue before any HIP call, and dispatches shapes to the
expected kernel family.  No GPU compute is issued here."""
import ctypes as ct
import os
import re
import subprocess

import pytest

from flash_engine import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fke_qgemm.h")
DROPIN = os.path.join(REPO, "flash-kernel-engine_amd", "_build", "test_quantized_gemm_dropin")
INVALID = _lib.HIP_ERROR_INVALID_VALUE


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fke_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_header_symbols():
    L = _lib.lib()
    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(L, s), f"missing export {s}"
    assert set(syms) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (fke_\w+)", out))
    assert set(syms) <= exported


def test_version_and_status_strings():
    assert _lib.version() == "1.2.0"
    assert "invalid" in _lib.status_string(INVALID).lower()


P = 4096  # a fake, 16-byte aligned "device" address: never dereferenced here


@pytest.mark.parametrize("M,N,K", [(0, 8, 8), (8, 0, 8), (8, 8, 0), (-1, 8, 8), (8, -3, 8)])
def test_rejects_bad_sizes(M, N, K):
    L = _lib.lib()
    assert L.fke_qgemm_i8(P, P, P, M, N, K, None, None, 1.0, 1.0, None, 0, 0, None) == INVALID
    assert L.fke_qgemm_f8(P, P, P, M, N, K, 1.0, 1.0, None, 0, 1, None) == INVALID
    assert L.fke_launch_int8_gemm_dp4a(P, P, P, 1.0, 1.0, M, N, K, None) == INVALID
    assert L.fke_launch_fp8_gemm_scaled(P, P, P, 1.0, 1.0, M, N, K, None) == INVALID


def test_rejects_null_pointers_and_bad_enums():
    L = _lib.lib()
    for a, b, c in [(None, P, P), (P, None, P), (P, P, None)]:
        assert L.fke_qgemm_i8(a, b, c, 8, 8, 8, None, None, 1.0, 1.0, None, 0, 0, None) == INVALID
        assert L.fke_qgemm_f8(a, b, c, 8, 8, 8, 1.0, 1.0, None, 0, 0, None) == INVALID
    assert L.fke_qgemm_i8(P, P, P, 8, 8, 8, None, None, 1.0, 1.0, None, 3, 0, None) == INVALID
    assert L.fke_qgemm_i8(P, P, P, 8, 8, 8, None, None, 1.0, 1.0, None, 0, 2, None) == INVALID
    assert L.fke_qgemm_f8(P, P, P, 8, 8, 8, 1.0, 1.0, None, _lib.OUT_I32, 0, None) == INVALID
    assert L.fke_qgemm_i8_on_path(9, P, P, P, 8, 8, 8, None, None, 1.0, 1.0, None, 0, 0, None) == INVALID


def test_workspace_entry_points_reject_bad_arguments():
    L = _lib.lib()
    for a, b, c in [(None, P, P), (P, None, P), (P, P, None)]:
        assert L.fke_qgemm_i8_ws(a, b, c, 1, 16, 64, None, None, 1.0, 1.0, None, 0, 1, P, 1 << 20, None) == INVALID
        assert L.fke_qgemm_f8_ws(a, b, c, 1, 16, 64, 1.0, 1.0, None, 0, 1, P, 1 << 20, None) == INVALID
    for M, N, K in [(0, 16, 64), (1, 0, 64), (1, 16, 0)]:
        assert L.fke_qgemm_i8_ws(P, P, P, M, N, K, None, None, 1.0, 1.0, None, 0, 1, None, 0, None) == INVALID
        assert L.fke_qgemm_f8_ws(P, P, P, M, N, K, 1.0, 1.0, None, 0, 1, None, 0, None) == INVALID
    assert L.fke_qgemm_i8_ws(P, P, P, 1, 16, 64, None, None, 1.0, 1.0, None, 3, 1, None, 0, None) == INVALID
    assert L.fke_qgemm_f8_ws(P, P, P, 1, 16, 64, 1.0, 1.0, None, _lib.OUT_I32, 1, None, 0, None) == INVALID
    assert L.fke_qgemm_f8_ws(P, P, P, 1, 16, 64, 1.0, 1.0, None, 0, 2, None, 0, None) == INVALID


@pytest.mark.parametrize("M,N,K,layout,expect", [
    # C2 with B [K,N], [M][N] int32 partials per split: M = 1 on the row kernel, 14 workgroups
    # of 1024 columns x 16 splits; M = 16 on one-wave workgroups, 112 of 128 columns x 2
    # splits; M = 4 on two-wave workgroups, 56 of 256 columns x 4 splits
    (1, 14336, 4096, 1, 16 * 1 * 14336 * 4),
    (16, 14336, 4096, 1, 2 * 16 * 14336 * 4),
    (4, 14336, 4096, 1, 4 * 4 * 14336 * 4),
    # row kernel: 4 blocks -> 64 splits at most, 112 pieces in 56 splits of 2;
    # 126 blocks -> 2 splits
    (1, 4096, 14336, 1, 56 * 1 * 4096 * 4),
    (1, 128256, 4096, 1, 2 * 1 * 128256 * 4),
    # splits capped by the 128-row pieces of K: K = 512 -> 4 splits
    (4, 14336, 512, 1, 4 * 4 * 14336 * 4),
    # N = 2^16: four-wave workgroups, 128 blocks of 512 columns -> 2 splits
    (2, 65536, 4096, 1, 2 * 2 * 65536 * 4),
    # N rounded up to 128-column blocks (one-wave workgroups: 9 blocks x 8 splits)
    (3, 1040, 4096, 1, 8 * 3 * 1152 * 4),
    # M = 16, N = 20016, K = 2048: two-wave workgroups x 3 splits (one-wave ones split as often)
    (16, 20016, 2048, 1, 3 * 16 * 20096 * 4),
    # 17..32 rows on the split decode: one-wave workgroups x 2 splits at N = 14336
    (17, 14336, 4096, 1, 2 * 17 * 14336 * 4), (32, 14336, 4096, 1, 2 * 32 * 14336 * 4),
    # unsplit: K of one piece, the decode not taken (M > 16, B [N,K], N % 16 != 0, K % 64 != 0)
    (1, 14336, 128, 1, 0), (33, 14336, 4096, 1, 0), (1, 14336, 4096, 0, 0), (1, 1002, 4096, 1, 0),
    (1, 14336, 4002, 1, 0), (0, 14336, 4096, 1, 0), (1, 14336, 4096, 2, 0),
    # N or K only a multiple of 4: the row kernel's 4-byte form (8 blocks of 128 x 32 splits;
    # 112 blocks x 16 splits); past one row, 1024-column blocks x row groups of 2 / 4 rows
    # (M = 3: 15 blocks -> 16 splits of 2 pieces; M = 16: 60 -> 4 splits; M = 32: 120 -> 2)
    (1, 1000, 4096, 1, 32 * 1 * 1024 * 4), (1, 14336, 4000, 1, 16 * 1 * 14336 * 4),
    (4, 1000, 4096, 1, 32 * 4 * 1024 * 4), (3, 14340, 4096, 1, 16 * 3 * 14464 * 4),
    (16, 14340, 4096, 1, 4 * 16 * 14464 * 4), (32, 14340, 4096, 1, 2 * 32 * 14464 * 4),
])
def test_workspace_size(M, N, K, layout, expect):
    assert _lib.lib().fke_qgemm_workspace_size(M, N, K, layout) == expect


def test_quantizer_rejects_bad_arguments():
    L = _lib.lib()
    q = L.fke_quantize_rows_i8
    assert q(None, 0, 4, 8, P, P, None) == INVALID
    assert q(P, 0, 4, 8, None, P, None) == INVALID
    assert q(P, 0, 4, 8, P, None, None) == INVALID
    for M, K in [(0, 8), (4, 0), (-1, 8)]:
        assert q(P, 0, M, K, P, P, None) == INVALID
    for dt in (-1, 2):
        assert q(P, dt, 4, 8, P, P, None) == INVALID


def test_swiglu_rejects_bad_arguments():
    L = _lib.lib()
    sw = L.fke_swiglu
    assert sw(None, P, P, 16, 0, None) == INVALID
    assert sw(P, None, P, 16, 0, None) == INVALID
    assert sw(P, P, None, 16, 0, None) == INVALID
    assert sw(P, P, P, -1, 0, None) == INVALID
    for dt in (-1, 3):
        assert sw(P, P, P, 16, dt, None) == INVALID
    assert sw(P, P, P, 0, 0, None) == _lib.HIP_SUCCESS  # nothing to do, nothing launched
    g = L.fke_qgemm_i8_swiglu
    assert g(None, P, P, 4, 8, 64, None, None, 1.0, 1.0, None, 0, None) == INVALID
    assert g(P, P, None, 4, 8, 64, None, None, 1.0, 1.0, None, 0, None) == INVALID
    for M, I, K in [(0, 8, 64), (4, 0, 64), (4, 8, 0), (4, 1 << 30, 64)]:
        assert g(P, P, P, M, I, K, None, None, 1.0, 1.0, None, 0, None) == INVALID
    assert g(P, P, P, 4, 8, 64, None, None, 1.0, 1.0, None, _lib.OUT_I32, None) == INVALID
    # past 16 rows the decode family needs K >= 2048 and at most 512 rows
    assert L.fke_qgemm_i8_swiglu_on_path(_lib.PATH_GEMV, P, P, P, 17, 64, 1024, None, None, 1.0, 1.0,
                                         None, 0, None) == INVALID
    assert L.fke_qgemm_i8_swiglu_on_path(_lib.PATH_GEMV, P, P, P, 513, 64, 4096, None, None, 1.0, 1.0,
                                         None, 0, None) == INVALID
    assert L.fke_qgemm_i8_swiglu_on_path(_lib.PATH_MFMA, P, P, P, 64, 64, 102, None, None, 1.0, 1.0,
                                         None, 0, None) == INVALID


@pytest.mark.parametrize("M,I,K,expect", [
    (1, 14336, 4096, _lib.PATH_GEMV),
    (3, 14336, 4096, _lib.PATH_GEMV),
    (16, 14336, 4096, _lib.PATH_GEMV),
    (17, 14336, 4096, _lib.PATH_GEMV),     # batches: the LDS-streamed kernel while its cost model wins
    (32, 14336, 4096, _lib.PATH_GEMV),
    (64, 14336, 4096, _lib.PATH_MFMA),     # the 128x128 ring (SwiGLU pairs need 128 columns)
    (128, 14336, 4096, _lib.PATH_MFMA),
    (4096, 14336, 4096, _lib.PATH_MFMA),
    (64, 64, 100, _lib.PATH_MFMA),         # K % 16 != 0, K % 4 == 0: the word kernel's SwiGLU form
    (64, 64, 102, _lib.PATH_GENERIC),      # K % 4 != 0
    (4, 64, 100, _lib.PATH_GEMV),          # up to 4 rows: the row kernel's 4-byte form
    (2, 300000, 4096, _lib.PATH_GEMV),     # row kernel: 64-bit row bases
    (8, 300000, 4096, _lib.PATH_GEMV),     # LDS-streamed kernel: buffer bases per workgroup
    (8, 600000, 2048, _lib.PATH_GENERIC),  # K < 4096 and 2I*K past the skinny kernel's 32-bit offsets
])
def test_dispatch_i8_swiglu(M, I, K, expect):
    assert _lib.lib().fke_select_path_i8_swiglu(P, P, P, M, I, K, 0) == expect


def test_half_gemm_rejects_bad_arguments_and_dispatch():
    L = _lib.lib()
    g = L.fke_gemm_half
    F16, BF16 = _lib.IN_F16, _lib.IN_BF16
    assert g(None, P, P, 4, 4, 64, F16, None, None, 1.0, 1.0, None, 0, 0, None) == INVALID
    for dt in (_lib.IN_F32, -1, 3):
        assert g(P, P, P, 4, 4, 64, dt, None, None, 1.0, 1.0, None, 0, 0, None) == INVALID
    assert g(P, P, P, 4, 4, 64, F16, None, None, 1.0, 1.0, None, _lib.OUT_I32, 0, None) == INVALID
    for M, N, K in [(0, 4, 64), (4, 0, 64), (4, 4, 0)]:
        assert g(P, P, P, M, N, K, BF16, None, None, 1.0, 1.0, None, 0, 0, None) == INVALID
    assert L.fke_launch_wmma_gemm_fp16(P, P, None, 4, 4, 64, 1.0, 0.0, None) == INVALID
    sel = L.fke_select_path_half
    assert sel(P, P, P, 8192, 8192, 8192, BF16, 0, 0) == _lib.PATH_MFMA
    assert sel(P, P, P, 1, 4096, 4096, F16, 1, 0) == _lib.PATH_MFMA
    assert sel(P, P, P, 256, 256, 96, F16, 0, 0) == _lib.PATH_MFMA         # 192 K bytes: a partial last stage
    assert sel(P, P, P, 256, 256, 100, F16, 0, 0) == _lib.PATH_GENERIC     # 200 K bytes: K % 8 != 0
    assert sel(P, P, P, 256, 256, 256, F16, 0, 1) == _lib.PATH_GENERIC     # B [K,N]
    assert sel(P + 2, P, P, 256, 256, 256, F16, 0, 0) == _lib.PATH_GENERIC
    assert L.fke_gemm_half_on_path(_lib.PATH_MFMA, P, P, P, 64, 64, 100, F16, None, None, 1.0, 1.0, None, 0, 0,
                                   None) == INVALID
    assert L.fke_gemm_half_on_path(_lib.PATH_GEMV, P, P, P, 1, 64, 64, F16, None, None, 1.0, 1.0, None, 0, 0,
                                   None) == INVALID


def test_w8a8_linear_from_float_arguments():
    L = _lib.lib()
    F32, BF16 = _lib.IN_F32, _lib.IN_BF16
    lin = L.fke_w8a8_linear
    need = L.fke_w8a8_linear_workspace_size(8, 4096)
    assert need == 8 * 4096 + 4 * 8
    assert L.fke_w8a8_linear_workspace_size(3, 100) == 512 + 12   # codes padded to 256 bytes
    assert L.fke_w8a8_linear_workspace_size(0, 100) == 0
    assert lin(None, BF16, P, P, 1, 64, 4096, None, 1.0, None, 1, P, need, None) == INVALID
    for dt in (-1, _lib.IN_F16, 5):
        assert lin(P, dt, P, P, 1, 64, 4096, None, 1.0, None, 1, P, need, None) == INVALID
    assert lin(P, BF16, P, P, 1, 64, 4096, None, 1.0, None, _lib.OUT_I32, P, need, None) == INVALID
    # the workspace is required and must be large enough: rejected before any launch
    assert lin(P, BF16, P, P, 8, 64, 4096, None, 1.0, None, 1, None, 0, None) == INVALID
    assert lin(P, BF16, P, P, 8, 64, 4096, None, 1.0, None, 1, P, need - 1, None) == INVALID
    assert lin(P, BF16, P, P, 1, 64, 4096, None, 1.0, None, 1, None, 0, None) == INVALID
    assert L.fke_w8a8_swiglu_linear(P, F32, P, P, 9, 64, 4096, None, 1.0, None, 1, None, 0, None) == INVALID
    assert L.fke_w8a8_swiglu_linear(P, F32, P, P, 9, 64, 4096, None, 1.0, None, 2, P, 1 << 20, None) == INVALID


def test_w8a8_linear_noalloc_arguments():
    """The allocation-free linear takes no workspace and rejects, before any
    HIP call, shapes whose workspace would not fit its device scratch, as well
    as everything fke_w8a8_linear rejects."""
    L = _lib.lib()
    BF16 = _lib.IN_BF16
    na = L.fke_w8a8_linear_noalloc
    cap = _lib.W8A8_NOALLOC_SCRATCH_BYTES
    assert cap == 32 << 20
    M, K = 4096, 8192                       # codes exactly fill the array: the scales do not fit
    assert L.fke_w8a8_linear_workspace_size(M, K) > cap
    assert na(P, BF16, P, P, M, 64, K, None, 1.0, None, 1, None) == INVALID
    assert na(P, BF16, P, P, 1, 64, cap, None, 1.0, None, 1, None) == INVALID
    assert L.fke_w8a8_linear_workspace_size(4096, 8000) <= cap   # fits (checked on the GPU)
    assert na(None, BF16, P, P, 1, 64, 4096, None, 1.0, None, 1, None) == INVALID
    assert na(P, _lib.IN_F16, P, P, 1, 64, 4096, None, 1.0, None, 1, None) == INVALID
    assert na(P, BF16, P, P, 1, 64, 4096, None, 1.0, None, _lib.OUT_I32, None) == INVALID
    assert na(P, BF16, P, P, 0, 64, 4096, None, 1.0, None, 1, None) == INVALID


def test_dropin_int8_rejects_k_not_multiple_of_4():
    """The reference kernel silently drops the K tail and misaligns rows when
    K % 4 != 0 (src/quantized_gemm.cu:28-30); the drop-in rejects it."""
    L = _lib.lib()
    for K in (1, 2, 3, 5, 4097):
        assert L.fke_launch_int8_gemm_dp4a(P, P, P, 1.0, 1.0, 8, 8, K, None) == INVALID


def test_path_unavailable_for_shape_is_rejected():
    L = _lib.lib()
    # GEMV needs M <= 512 (K >= 2048 past 16 rows), K % 64 == 0, B [N,K]; MFMA needs K % 16 == 0 (INT8 with B [N,K]: K % 4 == 0, the word kernel)
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV, P, P, P, 17, 64, 1024, None, None, 1.0, 1.0, None,
                                  0, 0, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV, P, P, P, 513, 64, 4096, None, None, 1.0, 1.0, None,
                                  0, 0, None) == INVALID
    # the dot-product decode family: INT8, B [N,K], M <= 16, K % 64 == 0
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV_DOT, P, P, P, 17, 64, 4096, None, None, 1.0, 1.0, None,
                                  0, 0, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV_DOT, P, P, P, 4, 64, 4096, None, None, 1.0, 1.0, None,
                                  0, 1, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV_DOT, P, P, P, 4, 64, 4000, None, None, 1.0, 1.0, None,
                                  0, 0, None) == INVALID
    assert L.fke_qgemm_i8_swiglu_on_path(_lib.PATH_GEMV_DOT, P, P, P, 5, 64, 4096, None, None, 1.0, 1.0, None,
                                         1, None) == INVALID
    # GEMV with B [K,N]: M <= 16 (to 32 where the split fills the CUs) with N % 16 == 0 and
    # K % 64 == 0, or M <= 32 with N % 4 == 0 and K % 4 == 0 (the row kernel's 4-byte form)
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV, P, P, P, 17, 64, 4096, None, None, 1.0, 1.0, None,
                                  0, 1, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV, P, P, P, 4, 70, 4096, None, None, 1.0, 1.0, None,
                                  0, 1, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV, P, P, P, 4, 64, 4002, None, None, 1.0, 1.0, None,
                                  0, 1, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_GEMV, P, P, P, 33, 72, 4096, None, None, 1.0, 1.0, None,
                                  0, 1, None) == INVALID
    assert L.fke_qgemm_i8_on_path(_lib.PATH_MFMA, P, P, P, 64, 64, 102, None, None, 1.0, 1.0, None,
                                  0, 0, None) == INVALID
    # the word kernel (K % 4 == 0) only on the automatic tile
    assert L.fke_qgemm_i8_on_path(_lib.PATH_MFMA_128x128, P, P, P, 64, 64, 100, None, None, 1.0, 1.0, None,
                                  0, 0, None) == INVALID
    # FP8 decode family: B [N,K] with K >= 2048, or B [K,N] as for INT8; fp32 / bf16 out
    assert L.fke_qgemm_f8_on_path(_lib.PATH_GEMV, P, P, P, 17, 64, 4096, 1.0, 1.0, None, 0, 1,
                                  None) == INVALID
    assert L.fke_qgemm_f8_on_path(_lib.PATH_GEMV, P, P, P, 4, 70, 4096, 1.0, 1.0, None, 0, 1,
                                  None) == INVALID
    assert L.fke_qgemm_f8_on_path(_lib.PATH_GEMV, P, P, P, 33, 72, 4096, 1.0, 1.0, None, 0, 1,
                                  None) == INVALID
    assert L.fke_qgemm_f8_on_path(_lib.PATH_GEMV, P, P, P, 4, 64, 1024, 1.0, 1.0, None, 0, 0,
                                  None) == INVALID
    assert L.fke_qgemm_f8_on_path(_lib.PATH_GEMV, P, P, P, 4, 64, 4096, 1.0, 1.0, None, _lib.OUT_I32, 0,
                                  None) == INVALID


@pytest.mark.parametrize("M,N,K,layout,expect", [
    (1, 14336, 4096, 0, _lib.PATH_GEMV),
    (4, 14336, 4096, 0, _lib.PATH_GEMV),
    (16, 14336, 4096, 0, _lib.PATH_GEMV),
    (17, 14336, 4096, 0, _lib.PATH_GEMV),    # batches: LDS-streamed kernel against the MFMA GEMM's cost
    (32, 14336, 4096, 0, _lib.PATH_GEMV),
    (48, 14336, 4096, 0, _lib.PATH_MFMA),    # four activation blocks: the MFMA GEMM's 64x64 ring is faster
    (32, 65536, 4096, 0, _lib.PATH_GEMV),    # large N: streamed 51.6 against 57.2 us on four 64x64 rounds
    (48, 65536, 4096, 0, _lib.PATH_MFMA),    # 59.3 on four 64x64 rounds against 70.5 streamed
    (64, 16896, 4096, 0, _lib.PATH_MFMA),    # two tile chunks streamed (28.0 us) against the 128x128 ring (23.4)
    (32, 20480, 4096, 0, _lib.PATH_GEMV),    # two chunks with two blocks: streamed 19.7 against 24.6
    (64, 14336, 4096, 0, _lib.PATH_MFMA),
    (128, 14336, 4096, 0, _lib.PATH_MFMA),   # 128x64 ring
    (192, 14336, 4096, 0, _lib.PATH_MFMA),
    (64, 4096, 4096, 0, _lib.PATH_GEMV),
    (128, 4096, 4096, 0, _lib.PATH_MFMA),
    (384, 4096, 4096, 0, _lib.PATH_MFMA),
    (128, 1792, 4096, 0, _lib.PATH_GEMV),    # small N: the streamed kernel's chunks run side by side
    (512, 1792, 4096, 0, _lib.PATH_MFMA),
    (384, 4096, 14336, 0, _lib.PATH_MFMA),
    (512, 4096, 14336, 0, _lib.PATH_MFMA),
    (17, 14336, 1024, 0, _lib.PATH_MFMA),    # K < 2048: no streamed batch kernel
    (100, 4096, 2112, 0, _lib.PATH_MFMA),    # K % 128 != 0: the MFMA GEMM, its last K stage cleared past K
    (17, 14336, 4096, 1, _lib.PATH_GEMV),    # B [K,N] to 32 rows: the split decode while its plan fills the CUs
    (32, 14336, 4096, 1, _lib.PATH_GEMV),
    (33, 14336, 4096, 1, _lib.PATH_MFMA),
    (32, 131072, 4096, 1, _lib.PATH_MFMA),   # four-wave workgroups over several rounds: the MFMA GEMM
    (4096, 11008, 4096, 0, _lib.PATH_MFMA),
    (8192, 8192, 8192, 0, _lib.PATH_MFMA),
    (8192, 8192, 8192, 1, _lib.PATH_MFMA),
    (1, 14336, 4096, 1, _lib.PATH_GEMV),     # B [K,N] decode: the transposing streamed kernel
    (16, 14336, 4096, 1, _lib.PATH_GEMV),
    (4, 4096, 64, 1, _lib.PATH_GEMV),
    (4, 4104, 4096, 1, _lib.PATH_GEMV),      # B [K,N] with N % 16 != 0: the row kernel's 4-byte form
    (1, 4104, 4096, 1, _lib.PATH_GEMV),
    (8, 4104, 4096, 1, _lib.PATH_GEMV),
    (9, 4104, 4096, 1, _lib.PATH_MFMA),      # past 8 rows the word kernel
    (5, 14336, 4000, 1, _lib.PATH_MFMA),     # past 4 rows the MFMA GEMM where it can (K % 16 == 0, N % 16 == 0)
    (4, 14336, 4000, 1, _lib.PATH_GEMV),     # one row group: the 4-byte form
    (33, 4104, 4096, 1, _lib.PATH_MFMA),     # past 32 rows: the word kernel (N % 4 == 0, K % 4 == 0)
    (33, 4102, 4096, 1, _lib.PATH_GENERIC),  # N % 4 != 0
    (1, 1002, 4096, 1, _lib.PATH_GENERIC),   # N % 4 != 0
    (17, 4096, 4096, 1, _lib.PATH_GEMV),
    (64, 64, 100, 0, _lib.PATH_MFMA),        # K % 16 != 0, K % 4 == 0: the word kernel (B [N,K])
    (64, 64, 4, 0, _lib.PATH_MFMA),
    (64, 64, 102, 0, _lib.PATH_GENERIC),     # K % 4 != 0
    (1, 14336, 4100, 0, _lib.PATH_GEMV),     # up to 4 rows: the [N,K] row kernel's 4-byte form
    (1, 14336, 4112, 0, _lib.PATH_GEMV),     # (one row also where K % 16 == 0, K % 64 != 0)
    (4, 14336, 4112, 0, _lib.PATH_MFMA),     # past one row the MFMA GEMM where it can run
    (4, 14336, 4108, 0, _lib.PATH_GEMV),
    (5, 14336, 4100, 0, _lib.PATH_MFMA),     # past 4 rows: the word kernel
    (8, 64, 96, 0, _lib.PATH_MFMA),          # K of 6 16-byte chunks: one partial stage
    (8, 64, 104, 0, _lib.PATH_MFMA),         # K % 16 != 0: rows not 16-byte aligned, the word kernel
    (300, 520, 4104, 0, _lib.PATH_MFMA),
    (300, 520, 4106, 0, _lib.PATH_GENERIC),
    (300, 520, 4104, 1, _lib.PATH_MFMA),     # B [K,N] past 32 rows: the word kernel too
    (300, 522, 4104, 1, _lib.PATH_GENERIC),
    (300, 520, 4112, 0, _lib.PATH_MFMA),
])
def test_dispatch_i8(M, N, K, layout, expect):
    assert _lib.lib().fke_select_path_i8(P, P, P, M, N, K, 0, layout) == expect


def test_dispatch_unaligned_pointer_falls_back():
    L = _lib.lib()
    assert L.fke_select_path_i8(P + 1, P, P, 1, 4096, 4096, 0, 0) == _lib.PATH_GENERIC
    assert L.fke_select_path_i8(P, P + 4, P, 256, 4096, 4096, 0, 0) == _lib.PATH_MFMA  # the word kernel
    assert L.fke_select_path_i8(P, P + 2, P, 256, 4096, 4096, 0, 0) == _lib.PATH_GENERIC
    assert L.fke_select_path_f8(P + 2, P, P, 256, 256, 256, 0, 1) == _lib.PATH_GENERIC
    assert L.fke_select_path_f8(P, P, P, 8192, 8192, 8192, 1, 1) == _lib.PATH_MFMA
    assert L.fke_select_path_i8(None, P, P, 8, 8, 8, 0, 0) == -1


@pytest.mark.parametrize("M,N,K,layout,expect", [
    (1, 14336, 4096, 0, _lib.PATH_GEMV),      # FP8 decode: the row kernel at M = 1, the LDS-streamed kernel above
    (1, 14336, 1024, 0, _lib.PATH_GEMV),      # the row kernel takes any K % 64 == 0
    (16, 14336, 4096, 0, _lib.PATH_GEMV),
    (32, 14336, 4096, 0, _lib.PATH_GEMV),
    (64, 14336, 4096, 0, _lib.PATH_MFMA),     # batches past 32 rows: the MFMA GEMM's 64x64 ring
    (1, 14336, 4096, 1, _lib.PATH_GEMV),      # B [K,N] (the reference layout): transposing decode kernel
    (16, 14336, 4096, 1, _lib.PATH_GEMV),
    (17, 14336, 4096, 1, _lib.PATH_GEMV),
    (33, 14336, 4096, 1, _lib.PATH_MFMA),
    (4, 14336, 4000, 1, _lib.PATH_GEMV),      # K % 64 != 0: the row kernel's 4-byte form (K % 4 == 0)
    (4, 14336, 4004, 1, _lib.PATH_GEMV),      # K % 16 != 0 (K % 4 == 0): the 4-byte form too
    (16, 14336, 4000, 1, _lib.PATH_MFMA),     # past 4 rows the MFMA GEMM where it can
    (8, 14336, 4004, 1, _lib.PATH_GEMV),      # and the 4-byte form where it cannot, to 8 rows
    (16, 14336, 4004, 1, _lib.PATH_MFMA),     # then the word kernel
    (4, 14336, 4002, 1, _lib.PATH_GENERIC),   # K % 4 != 0
    (64, 14336, 4100, 1, _lib.PATH_MFMA),     # past 32 rows, K % 16 != 0: the word kernel (both layouts)
    (1, 14336, 4100, 0, _lib.PATH_GEMV),      # up to 4 rows, B [N,K]: the row kernel's 4-byte form
    (4, 14336, 4100, 0, _lib.PATH_GEMV),
    (4, 14336, 4112, 0, _lib.PATH_MFMA),      # past one row the MFMA GEMM where it can run
    (5, 14336, 4100, 0, _lib.PATH_MFMA),      # past 4 rows the word kernel
    (64, 14336, 4100, 0, _lib.PATH_MFMA),
    (64, 14338, 4100, 1, _lib.PATH_GENERIC),  # N % 4 != 0 with B [K,N]
    (8192, 8192, 8192, 0, _lib.PATH_MFMA),
    (4, 14336, 1024, 0, _lib.PATH_MFMA),      # K < 2048
    (4, 300, 2112, 0, _lib.PATH_GEMV),        # K % 128 != 0: no MFMA GEMM
])
def test_dispatch_f8(M, N, K, layout, expect):
    assert _lib.lib().fke_select_path_f8(P, P, P, M, N, K, 0, layout) == expect


def test_dropin_header_program_host_checks():
    """The drop-in C++ program (built by g++ against include/quantized_gemm.cuh)
    passes its argument-validation checks without a GPU."""
    assert os.path.exists(DROPIN), "build first: make -C flash-kernel-engine_amd/csrc"
    r = subprocess.run([DROPIN, "--host-only"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "[PASS]" in r.stdout


def test_torch_extension_loads_and_binds_the_ops():
    """The torch extension (bindings.cpp idiom) imports and exposes its
    entries; it links libfke_qgemm.so, whose exports are checked above."""
    from flash_engine import _ext
    m = _ext.ext()
    for name in ("quantized_gemm_int8_forward", "fp8_gemm_scaled_forward", "quantize_per_token_forward",
                 "quantized_gemm_int8_swiglu_forward", "fused_swiglu_forward"):
        assert hasattr(m, name), name


def test_torch_extension_rejects_host_tensors():
    import torch
    from flash_engine import _ext
    m = _ext.ext()
    a = torch.zeros((4, 8), dtype=torch.int8)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        m.quantized_gemm_int8_forward(a, a)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        m.quantize_per_token_forward(torch.zeros((4, 8)))
    with pytest.raises(RuntimeError, match="GPU tensors"):
        m.fused_swiglu_forward(torch.zeros(8), torch.zeros(8))
    with pytest.raises(RuntimeError, match="GPU tensor"):
        m.quantized_gemm_int8_swiglu_forward(a, a)


@pytest.mark.parametrize("M,N,K,layout,swiglu,cus,want", [
    (8192, 8192, 8192, 0, 0, 256, _lib.PATH_MFMA_256x256),       # 1024 tiles of 256x256
    (4096, 11008, 4096, 0, 0, 256, _lib.PATH_MFMA_256x256),      # 688
    (3072, 4096, 4096, 0, 0, 256, _lib.PATH_MFMA_256x256),       # 192 / 768 of 128x128: a partial second round
    (1024, 14336, 4096, 0, 0, 256, _lib.PATH_MFMA_256x256),      # 224 / 896
    (8192, 8192, 1024, 0, 0, 256, _lib.PATH_MFMA_256x256),       # short K, many tiles
    (4096, 1376, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128),       # 96 / 352: one round of two per CU
    (8192, 1024, 8192, 0, 0, 256, _lib.PATH_MFMA_128x128),       # 128 / 512
    (512, 14336, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128),       # 112 / 448
    (64, 14336, 4096, 0, 0, 256, _lib.PATH_MFMA_64x64_RING4),    # 224 tiles of 64x64: one per CU at most
    (256, 4096, 1024, 0, 0, 256, _lib.PATH_MFMA_64x64_RING4),    # 256
    (512, 1792, 4096, 0, 0, 256, _lib.PATH_MFMA_64x64_RING4),    # 224
    (128, 14336, 4096, 0, 0, 256, _lib.PATH_MFMA_128x64_RING4),  # 448 of 64x64, 224 of 128x64
    (512, 4096, 4096, 0, 0, 256, _lib.PATH_MFMA_128x64_RING4),   # 512 / 256
    (1024, 4096, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128_RING4), # 1024 / 512 / 256 of 128x128
    (256, 14336, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128_RING4), # 224 of 128x128
    (4096, 1376, 4096, 1, 0, 256, _lib.PATH_MFMA_128x128),       # B [K,N]: the same rule
    (128, 4096, 1024, 1, 0, 256, _lib.PATH_MFMA_64x64_RING4),
    (4096, 1376, 4096, 0, 1, 256, _lib.PATH_MFMA_128x128),       # SwiGLU, 688 outputs: 96 / 352
    (128, 28672, 4096, 0, 1, 256, _lib.PATH_MFMA_128x128_RING4), # SwiGLU, 14336 outputs: 224 tiles of 64
    (4096, 2752, 4096, 0, 1, 256, _lib.PATH_MFMA_256x256),       # SwiGLU, 1376 outputs: 176 / 704
    (4096, 1376, 4096, 0, 0, 80, _lib.PATH_MFMA_256x256),        # fills 80 CUs
    # one row of tiles, more tiles than CUs (decode batches against a large N)
    (64, 65536, 4096, 0, 0, 256, _lib.PATH_MFMA_64x64_RING4),    # 1024 tiles of 64x64: four rounds
    (64, 128256, 4096, 1, 0, 256, _lib.PATH_MFMA_64x64_RING4),   # B [K,N]: the same rule
    (48, 32768, 4096, 0, 0, 256, _lib.PATH_MFMA_64x64_RING4),    # 256 of 128x128 would leave no CU idle
    (64, 16896, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128_RING4),  # 132 of 128x128: one round, half the CUs
    (64, 28672, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128_RING4),  # 224 = 7/8 of the CUs
    (64, 28800, 4096, 0, 0, 256, _lib.PATH_MFMA_64x64_RING4),    # 225
    (128, 65536, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128),       # 512 of 128x128: two per CU
    (96, 131072, 4096, 0, 0, 256, _lib.PATH_MFMA_128x128),       # 1024 of 128x128: four rounds
    (256, 65536, 4096, 0, 0, 256, _lib.PATH_MFMA_256x256),       # past 128 rows: 256x256
    (128, 65536, 4096, 0, 1, 256, _lib.PATH_MFMA_256x256),       # SwiGLU keeps the previous rule
])
def test_mfma_tile_choice(M, N, K, layout, swiglu, cus, want):
    assert _lib.lib().fke_select_mfma_tile(M, N, K, layout, swiglu, cus) == want


@pytest.mark.parametrize("M,N,K,layout,want_s,want_tile", [
    (64, 4096, 14336, 0, 4, _lib.PATH_MFMA_64x64_RING4),     # one tile row: 64 tiles, 28 stages a split
    (100, 1000, 14720, 0, 7, _lib.PATH_MFMA_64x64_RING4),    # 115 stages: 6 splits of 17 and one of 13
    (200, 2000, 8192, 1, 4, _lib.PATH_MFMA_128x64_RING4),    # B [K,N] (slower unsplit)
    (128, 8192, 28672, 0, 4, _lib.PATH_MFMA_128x128_RING4),  # 64 tiles of 128x128: one tile row
    (120, 2000, 28672, 0, 8, _lib.PATH_MFMA_128x64_RING4),
    (128, 4096, 14336, 0, 1, _lib.PATH_MFMA_64x64_RING4),    # two tile rows share B: unsplit is as fast
    (200, 2000, 8192, 0, 1, _lib.PATH_MFMA_64x64_RING4),     # the same with B [N,K]
    (128, 14336, 4096, 0, 1, _lib.PATH_MFMA_128x64_RING4),   # 224 tiles: no room to split
    (512, 4096, 14336, 0, 1, _lib.PATH_MFMA_128x64_RING4),   # 256 tiles
    (128, 4096, 384, 0, 1, _lib.PATH_MFMA_64x64_RING4),      # three stages: too short to split
    (4096, 4096, 4096, 0, 1, _lib.PATH_MFMA_256x256),
])
def test_mfma_split_choice(M, N, K, layout, want_s, want_tile):
    t = ct.c_int(-1)
    L = _lib.lib()
    assert L.fke_select_mfma_split(M, N, K, layout, 256, ct.byref(t)) == want_s
    assert t.value == want_tile
    assert L.fke_select_mfma_split(M, N, K, layout, 256, None) == want_s
    if want_s == 1:
        assert want_tile == L.fke_select_mfma_tile(M, N, K, layout, 0, 256)
    if not (layout == _lib.B_KN and M <= 16):
        assert L.fke_qgemm_workspace_size(M, N, K, layout) == (want_s * M * N * 4 if want_s > 1 else 0)


def test_mfma_split_rejects_bad_arguments():
    L = _lib.lib()
    assert L.fke_select_mfma_split(0, 64, 64, 0, 256, None) == -1
    assert L.fke_select_mfma_split(64, 64, 64, 2, 256, None) == -1


def test_mfma_tile_choice_rejects_bad_arguments():
    L = _lib.lib()
    assert L.fke_select_mfma_tile(0, 64, 64, 0, 0, 256) == -1
    assert L.fke_select_mfma_tile(64, 64, 64, 2, 0, 256) == -1
    assert L.fke_select_mfma_tile(64, 63, 64, 0, 1, 256) == -1


def test_narrow_ring_tiles_reject_swiglu_before_any_launch():
    L = _lib.lib()
    for path in (_lib.PATH_MFMA_128x64_RING4, _lib.PATH_MFMA_64x64_RING4):
        assert L.fke_qgemm_i8_swiglu_on_path(path, P, P, P, 64, 64, 256, None, None, 1.0, 1.0, None,
                                             _lib.OUT_BF16, None) == _lib.HIP_ERROR_INVALID_VALUE


def test_library_imports_no_device_allocator():
    """No entry point can allocate or free device memory: the library does not
    even import an allocation routine (the K splits' partial sums go to the
    caller's workspace or to the static split pool)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    imported = set(re.findall(r"\bU (hip\w+)", out))
    assert "hipLaunchKernel" in imported
    alloc = {s for s in imported if re.match(r"hip(Ext)?(Malloc|Free|MemPool|HostAlloc|HostMalloc|MemAlloc)", s)}
    assert not alloc, f"allocation routines imported: {sorted(alloc)}"


def test_split_pool_constants_match_header():
    text = open(HEADER).read()
    slots = int(re.search(r"#define FKE_SPLIT_SLOTS (\d+)", text).group(1))
    slot = re.search(r"#define FKE_SPLIT_SLOT_BYTES \((\d+)u << (\d+)\)", text)
    scratch = re.search(r"#define FKE_W8A8_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert slots == _lib.SPLIT_SLOTS
    assert int(slot.group(1)) << int(slot.group(2)) == _lib.SPLIT_SLOT_BYTES
    small = int(re.search(r"#define FKE_SPLIT_SMALL_SLOTS (\d+)", text).group(1))
    small_b = re.search(r"#define FKE_SPLIT_SMALL_SLOT_BYTES \((\d+)u << (\d+)\)", text)
    assert small == _lib.SPLIT_SMALL_SLOTS
    assert int(small_b.group(1)) << int(small_b.group(2)) == _lib.SPLIT_SMALL_SLOT_BYTES
    assert int(scratch.group(1)) << int(scratch.group(2)) == _lib.W8A8_NOALLOC_SCRATCH_BYTES
    assert _lib.lib().fke_split_slots_in_use() == -1  # no device here


@pytest.mark.parametrize("layout", [0, 1])
def test_split_plans_fit_one_pool_slot(layout):
    """Every split plan, decode and MFMA, fits one slot of the split pool,
    including shapes whose uncapped plan would not (M = 16 against an LM head
    of 262144 columns, a long-K batch against 16384 columns)."""
    L = _lib.lib()
    cap = _lib.SPLIT_SLOT_BYTES
    seen_cap = False
    for M in (1, 4, 16, 64, 128, 200, 256):
        for N in (1024, 8192, 14336, 16384, 65536, 128256, 262144):
            for K in (1024, 4096, 14336, 28672):
                ws = L.fke_qgemm_workspace_size(M, N, K, layout)
                assert ws <= cap, (M, N, K, layout, ws)
                seen_cap |= ws > cap // 2
    assert seen_cap


def test_probe_library_exports_and_argument_checks():
    """The measurement probes bench.py loads (libfke_probe.so, not part of the
    C ABI) export their entry points, and the read probe turns bad arguments
    into hipErrorInvalidValue before any launch."""
    path = os.path.join(os.path.dirname(_lib.LIB_PATH), "libfke_probe.so")
    probe = ct.CDLL(path)
    for name in ("fke_probe_mfma_i8", "fke_probe_mfma_src_bytes", "fke_probe_mfma_out_elems", "fke_probe_read",
                 "fke_probe_read_out_elems"):
        assert hasattr(probe, name), name
    probe.fke_probe_read.argtypes = [ct.c_void_p, ct.c_int64, ct.c_void_p, ct.c_int, ct.c_int, ct.c_int, ct.c_int32,
                                 ct.c_void_p]
    probe.fke_probe_read.restype = ct.c_int
    probe.fke_probe_read_out_elems.argtypes = [ct.c_int, ct.c_int]
    probe.fke_probe_read_out_elems.restype = ct.c_size_t
    assert probe.fke_probe_read_out_elems(256, 4) == 1024
    bad = [(None, 4096, P, 1, 1, 4), (P, 4096, None, 1, 1, 4), (P, 4096, P, 0, 1, 4), (P, 4096, P, 1, 9, 4),
           (P, 4096, P, 1, 1, 2), (P, 4096 + 16, P, 1, 1, 4), (P, 1 << 31, P, 1, 1, 8), (P, 0, P, 1, 1, 4)]
    for src, n, out, grid, waves, unit in bad:
        assert probe.fke_probe_read(src, n, out, grid, waves, unit, 0, None) == _lib.HIP_ERROR_INVALID_VALUE
