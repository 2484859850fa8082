"""CPU tests of the Python surface: the reference module name, the reference
op's host arithmetic where no GPU is visible, and argument checks that must
fire before any launch (no GPU needed: a launch would fail these tests)."""
import os
import subprocess
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
from flash_engine import _lib, ops  # noqa: E402

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "flash-kernel-engine_amd")


def test_extension_imports_by_the_reference_module_name():
    """`import flash_engine_cuda` (reference python/flash_engine/ops.py:9-13,
    setup.py:51) works from a fresh interpreter with the package directory on
    the path, and carries fused_swiglu_forward (which the reference op calls,
    ops.py:222-223) and the GEMM entries."""
    code = ("import sys; sys.path.insert(0, %r); import torch; import flash_engine_cuda as m; "
            "names = ['fused_swiglu_forward', 'quantized_gemm_int8_forward', 'fp8_gemm_scaled_forward', "
            "'quantize_per_token_forward', 'quantized_gemm_int8_swiglu_forward']; "
            "missing = [n for n in names if not hasattr(m, n)]; "
            "assert not missing, missing; print(m.__file__)" % PKG)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("flash_engine_cuda.so")


def test_loader_and_plain_import_share_one_module():
    from flash_engine import _ext
    m = _ext.ext()
    import flash_engine_cuda
    assert flash_engine_cuda is m


@pytest.mark.skipif(torch.cuda.is_available(), reason="the host arithmetic is taken only without a GPU")
def test_quantized_gemm_int8_host_arithmetic_without_gpu(oracle):
    """numpy inputs on a machine with no GPU: the reference op's result
    (python/flash_engine/ops.py:180-186, restated by the oracle), bit for bit,
    including operands held in wider integer types with values past int8
    (the reference widens with astype(np.int32))."""
    r = np.random.default_rng(3)
    A = r.integers(-127, 128, (33, 70), dtype=np.int8)
    B = r.integers(-127, 128, (70, 41), dtype=np.int8)
    for sa, sb in [(1.0, 1.0), (0.01, 0.02), (0.0123, 0.0456)]:
        got = ops.quantized_gemm_int8(A, B, sa, sb)
        assert got.dtype == np.float32
        assert np.array_equal(got.view(np.uint32), oracle.ref_py_gemm_i8(A, B, sa, sb).view(np.uint32))
    Aw = r.integers(-1000, 1000, (5, 9)).astype(np.int32)
    Bw = r.integers(-1000, 1000, (9, 4)).astype(np.int32)
    expect = (Aw.astype(np.int64) @ Bw.astype(np.int64)).astype(np.float32) * np.float32(0.5)
    assert np.array_equal(ops.quantized_gemm_int8(Aw, Bw, 0.5, 1.0), expect)


def test_gpu_path_operand_conversion():
    """numpy operands bound for the GPU: int8 passes through, other integer
    types are narrowed only when every value fits int8, floats are refused."""
    a = np.arange(-4, 4, dtype=np.int64).reshape(2, 4)
    c = ops._host_int8(a, "A")
    assert c.dtype == np.int8 and c.flags.c_contiguous and np.array_equal(c, a)
    with pytest.raises(ValueError, match="int8 range"):
        ops._host_int8(np.array([[0, 128]], dtype=np.int32), "A")
    with pytest.raises(ValueError, match="int8 range"):
        ops._host_int8(np.array([[-129]], dtype=np.int16), "B")
    with pytest.raises(TypeError, match="integers"):
        ops._host_int8(np.zeros((2, 2), dtype=np.float32), "A")


@pytest.fixture
def no_launch(monkeypatch):
    """Host tensors accepted as if they were on the GPU, and any use of the C
    library fails the test: a check that raises first fired before a launch."""
    class NoLaunch:
        def __getattr__(self, name):
            raise AssertionError(f"{name} reached the C library")
    monkeypatch.setattr(ops, "_check_dev", lambda *a, **k: None)
    monkeypatch.setattr(_lib, "lib", lambda: NoLaunch())


def test_fp8_gemm_rejects_wrong_out_and_rank_before_launch(no_launch):
    A = torch.zeros((4, 64), dtype=torch.uint8)
    B = torch.zeros((64, 8), dtype=torch.uint8)
    for bad in [(4, 7), (8, 4), (32,), (4, 8, 1)]:
        with pytest.raises(ValueError, match="out must be"):
            ops.fp8_gemm_scaled(A, B, 1.0, 1.0, out=torch.empty(bad))
    with pytest.raises(ValueError, match="2-D"):
        ops.fp8_gemm_scaled(A.view(-1), B, 1.0, 1.0)
    with pytest.raises(ValueError, match="2-D"):
        ops.fp8_gemm_scaled(A, B.view(1, 64, 8), 1.0, 1.0)
    with pytest.raises(AssertionError, match="reached the C library"):  # a good call gets that far
        ops.fp8_gemm_scaled(A, B, 1.0, 1.0, out=torch.empty((4, 8)))


def test_quantize_per_token_rejects_wrong_q_before_launch(no_launch):
    x = torch.zeros((4, 64))
    for bad in [(4, 63), (3, 64), (256,)]:
        with pytest.raises(ValueError, match="q must be"):
            ops.quantize_per_token(x, q=torch.empty(bad, dtype=torch.int8))
    with pytest.raises(ValueError, match="scale must have"):
        ops.quantize_per_token(x, scale=torch.empty(3))
    with pytest.raises(AssertionError, match="reached the C library"):
        ops.quantize_per_token(x, q=torch.empty((4, 64), dtype=torch.int8))


def test_other_ops_reject_wrong_out_before_launch(no_launch):
    A = torch.zeros((4, 64), dtype=torch.int8)
    B = torch.zeros((8, 64), dtype=torch.int8)
    with pytest.raises(ValueError, match="wrong shape"):
        ops.w8a8_gemm(A, B, out_dtype=torch.float32, out=torch.empty((4, 7)))
    W = torch.zeros((16, 64), dtype=torch.int8)
    with pytest.raises(ValueError, match="wrong shape"):
        ops.w8a8_swiglu(A, W, out_dtype=torch.float32, out=torch.empty((4, 16)))
    H = torch.zeros((4, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="wrong shape"):
        ops.gemm_half(H, H.clone(), out=torch.empty((4, 5)))
