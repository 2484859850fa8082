"""GPU tests of the W8A8 linear layer from float activations in one call
(fke_w8a8_linear, fke_w8a8_swiglu_linear: the per-token quantiser into a
caller workspace, then the GEMM on its codes).  Bar: bit-exact against the
oracle's quantiser followed by its W8A8 GEMM (fko_quantize_rows_i8 +
fko_w8a8_*), and against the separate GPU calls (fke_quantize_rows_i8 +
fke_qgemm_i8); the SwiGLU variant bit-exact against the separate GPU calls and
within the SwiGLU tolerance (1e-6 relative) of the oracle.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _lib, ops  # noqa: E402

NTH = 16


def say(*a):
    print("[case]", *a, flush=True)


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def same(got, ref, what):
    g = got.view(np.uint32) if got.dtype == np.float32 else got
    r = ref.view(np.uint32) if ref.dtype == np.float32 else ref
    bad = g != r
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} mismatches, first at {i}: {got[i]!r} vs {ref[i]!r}")


def activations(M, K, seed, dtype):
    r = np.random.default_rng(seed)
    x = (r.standard_normal((M, K)) * r.uniform(0.1, 4, (M, 1))).astype(np.float32)
    if M >= 2:
        x[1, :] = 0.0                         # all-zero row: scale 1, codes 0
    x[0, K // 3] = np.nan                     # NaN element: ignored by the maximum, code 0
    t = dev_t(x)
    if dtype == "bf16":
        t = t.to(torch.bfloat16)
    return t


def host_bits(t):
    """Activations as the oracle takes them: fp32 values, or bf16 bit patterns."""
    return t.view(torch.int16).cpu().numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.cpu().numpy()


def weights(oracle, N, K, seed):
    W = oracle.gen_i8_uniform((N, K), seed)
    sb = oracle.gen_f32_uniform((N,), seed + 1, 0.001, 0.02)
    bias = oracle.gen_f32_normal((N,), seed + 2, 0.0, 0.5)
    return W, sb, bias


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K", [4096, 8192, 4160, 64, 100, 4100])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_decode_linear_from_float(oracle, dev, M, K, xdt):
    N = 333
    say("decode linear from float", M, K, xdt)
    x = activations(M, K, 10 * M + K, xdt)
    W, sb, bias = weights(oracle, N, K, 7 + K)
    code = oracle.IN_F32 if xdt == "f32" else oracle.IN_BF16
    q, s = oracle.quantize_rows_i8(host_bits(x), code)
    for out, odt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        for b in (None, bias):
            y = ops.w8a8_linear(x, dev_t(W), dev_t(sb), None if b is None else dev_t(b), out_dtype=odt)
            ref = oracle.w8a8_gemm(q, W, s, sb, bias=b, out_dtype=oracle.OUT_F32 if out == "f32" else oracle.OUT_BF16)
            q2, s2 = ops.quantize_per_token(x)
            y2 = ops.w8a8_gemm(q2, dev_t(W), s2, dev_t(sb), None if b is None else dev_t(b), out_dtype=odt)
            torch.cuda.synchronize()
            same(host(y), ref, f"one call vs oracle M={M} K={K} {xdt}->{out} bias={b is not None}")
            same(host(y), host(y2), f"one call vs separate calls M={M} K={K} {xdt}->{out}")


@pytest.mark.parametrize("M,K", [(40, 100), (300, 4100)])
def test_linear_odd_k(oracle, dev, M, K):
    """K a multiple of 4 only: the codes' rows are 4-byte aligned and the GEMM
    is the word kernel; bit-exact against the oracle and the separate calls."""
    N = 520
    say("linear, odd K", M, K)
    x = activations(M, K, 500 + M + K, "f32")
    W, sb, bias = weights(oracle, N, K, 13 + K)
    assert _lib.lib().fke_select_path_i8(4096, 4096, 4096, M, N, K, _lib.OUT_F32, _lib.B_NK) == _lib.PATH_MFMA
    y = ops.w8a8_linear(x, dev_t(W), dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    q2, s2 = ops.quantize_per_token(x)
    y2 = ops.w8a8_gemm(q2, dev_t(W), s2, dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    torch.cuda.synchronize()
    q, s = oracle.quantize_rows_i8(host_bits(x), oracle.IN_F32)
    same(host(y), oracle.w8a8_gemm(q, W, s, sb, bias=bias), f"odd K M={M} K={K} vs oracle")
    same(host(y), host(y2), f"odd K M={M} K={K} vs separate calls")


@pytest.mark.parametrize("M", [5, 17, 300])
def test_linear_through_workspace(oracle, dev, M):
    """Larger M: the GEMM after the quantiser is the skinny MFMA or the tiled
    MFMA kernel."""
    N, K = 520, 1024
    say("linear through workspace", M)
    x = activations(M, K, 300 + M, "bf16")
    W, sb, bias = weights(oracle, N, K, 11)
    L = _lib.lib()
    y = ops.w8a8_linear(x, dev_t(W), dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    torch.cuda.synchronize()
    q, s = oracle.quantize_rows_i8(host_bits(x), oracle.IN_BF16)
    same(host(y), oracle.w8a8_gemm(q, W, s, sb, bias=bias), f"workspace M={M}")
    # the C entry point refuses to run without the workspace
    yy = torch.empty((M, N), dtype=torch.float32, device=dev)
    Wt = dev_t(W)
    assert L.fke_w8a8_linear(x.data_ptr(), _lib.IN_BF16, Wt.data_ptr(), yy.data_ptr(), M, N, K, None, 1.0, None,
                             0, None, 0, None) == _lib.HIP_ERROR_INVALID_VALUE


def test_decode_linear_full_shape(oracle, dev):
    """Decode M = 1, N = 14336, K = 4096 from bf16 activations, bf16 out."""
    M, N, K = 1, 14336, 4096
    say("decode linear full shape")
    x = activations(M, K, 5, "bf16")
    W, sb, bias = weights(oracle, N, K, 99)
    y = ops.w8a8_linear(x, dev_t(W), dev_t(sb), dev_t(bias), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    q, s = oracle.quantize_rows_i8(host_bits(x), oracle.IN_BF16)
    same(host(y), oracle.w8a8_gemm(q, W, s, sb, bias=bias, out_dtype=oracle.OUT_BF16, nthreads=NTH), "full shape")


@pytest.mark.parametrize("M", [1, 3, 4, 9])
def test_swiglu_linear_from_float(oracle, dev, M):
    I, K = 200, 4096
    say("swiglu linear from float", M)
    x = activations(M, K, 40 + M, "bf16")
    W, sb, bias = weights(oracle, 2 * I, K, 21)
    h = ops.w8a8_gate_up_swiglu(x, dev_t(W), dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    q2, s2 = ops.quantize_per_token(x)
    h2 = ops.w8a8_swiglu(q2, dev_t(W), s2, dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    torch.cuda.synchronize()
    same(host(h), host(h2), f"one call vs separate calls M={M}")
    q, s = oracle.quantize_rows_i8(host_bits(x), oracle.IN_BF16)
    ref = oracle.w8a8_swiglu(q, W, s, sb, bias=bias)
    got = host(h).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-6 * np.abs(ref) + 1e-33), "swiglu linear vs oracle"
