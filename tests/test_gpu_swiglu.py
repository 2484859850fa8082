"""GPU tests of SwiGLU: the elementwise op (reference src/fused_activations.cu,
python/flash_engine/ops.py:218-230) and the W8A8 gate/up GEMM with SwiGLU fused
into its epilogue, through the C ABI and the torch extension, against the CPU
oracle (oracle/fke_oracle.c: fko_swiglu1, fko_w8a8_swiglu).

Bars:
  * fp32: |gpu - oracle| <= 1e-6 * |oracle| + 1e-33.  The kernel's expf and
    reciprocal are each within 1 ulp and the oracle's within half an ulp, so
    the two differ by a few ulps (2^-23 ~ 1.2e-7 relative each).  The
    absolute term covers g < -87, where sigmoid(g) < 2^-125 leaves the normal
    range (the reciprocal flushes it to zero) and |h| < |g*u| * 2^-125.
  * bf16 / fp16: the oracle's fp32 value rounded to nearest even, or one unit
    of the output type away from it (the fp32 values may straddle a rounding
    boundary); at least 99 % identical.
  * the fused GEMM equals the unfused pipeline (fp32 GEMM of all 2I weight
    rows, then the elementwise op on the gate and up halves) bit for bit, and
    its bf16 output is the bf16 rounding of its fp32 output.
  * the reference's own SwiGLU test vector: max abs difference < 1e-6.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _ext, _lib, ops  # noqa: E402

NTH = 16


def say(*a):
    print("[case]", *a, flush=True)


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def bf16_bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def f32_to_bf16_np(x):
    """round-to-nearest-even fp32 -> bf16 bits (NaN-free inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def check_f32(got, ref, what):
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    tol = 1e-6 * np.abs(ref.astype(np.float64)) + 1e-33
    bad = err > tol
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} outside tolerance, first at {i}: {got[i]!r} vs {ref[i]!r}")


def check_rounded(got_bits, ref_bits, what, kind, got_f32, ref_f32):
    """got / ref are uint16 bit patterns of bf16 or fp16 values: equal, or
    adjacent; got_f32 / ref_f32 are the same values widened to fp32, used for
    the absolute term of the fp32 bar (|h| < 1e-33 where sigmoid underflows)."""
    g = got_bits.astype(np.int64)
    r = ref_bits.astype(np.int64)
    # adjacent representable values of one sign differ by 1 in the bit pattern
    same_sign = (g >> 15) == (r >> 15)
    adj = same_sign & (np.abs(g - r) <= 1)
    both_zero = ((g & 0x7FFF) == 0) & ((r & 0x7FFF) <= 1) | ((r & 0x7FFF) == 0) & ((g & 0x7FFF) <= 1)
    underflow = (np.abs(ref_f32) < 1e-33) & (np.abs(got_f32) < 1e-33)
    ok = adj | both_zero | underflow
    assert ok.all(), f"{what}: {int((~ok).sum())} {kind} values more than one unit apart"
    assert (g == r).mean() >= 0.99, f"{what}: only {(g == r).mean():.4f} identical"


# ------------------------------------------------------------- elementwise

def test_swiglu_reference_test_vector(dev):
    """python/tests/test_correctness.py:166-176, through the Python op."""
    say("fused_swiglu reference vector")
    gate = np.array([-2.0, -0.5, 0.0, 0.5, 2.0], dtype=np.float32)
    up = np.array([1.0, 2.0, 3.0, 4.0, 5.0], dtype=np.float32)
    out = ops.fused_swiglu(gate, up)
    ref = (gate / (np.float32(1.0) + np.exp(-gate))) * up
    assert isinstance(out, np.ndarray) and out.dtype == np.float32
    assert np.max(np.abs(out - ref)) < 1e-6


def swiglu_inputs(n, seed):
    r = np.random.default_rng(seed)
    g = (r.standard_normal(n) * 4).astype(np.float32)
    if n >= 64:  # a sweep over the whole range, saturation included
        g[: n // 8] = np.linspace(-100, 100, n // 8, dtype=np.float32)
    u = (r.standard_normal(n) * 2).astype(np.float32)
    return g, u


@pytest.mark.parametrize("n", [1, 3, 5, 8, 4099, (1 << 20) + 3])
@pytest.mark.parametrize("aligned", [True, False])
def test_swiglu_f32(oracle, dev, n, aligned):
    say("swiglu f32", n, "aligned" if aligned else "offset by one element")
    g, u = swiglu_inputs(n, 40 + n)
    ref = oracle.swiglu_f32(g, u)
    off = 0 if aligned else 1
    gb = torch.zeros(n + off, dtype=torch.float32, device=dev)
    ub = torch.zeros(n + off, dtype=torch.float32, device=dev)
    gb[off:] = dev_t(g)
    ub[off:] = dev_t(u)
    out = torch.full((n + off,), float("nan"), dtype=torch.float32, device=dev)
    st = _lib.lib().fke_swiglu(gb[off:].data_ptr(), ub[off:].data_ptr(), out[off:].data_ptr(), n,
                               _lib.IN_F32, torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "fke_swiglu")
    torch.cuda.synchronize()
    h = out.cpu().numpy()
    check_f32(h[off:], ref, f"swiglu f32 n={n}")
    if off:
        assert np.isnan(h[0]), "wrote before the output"


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("n", [7, 4096 + 5, 1 << 18])
def test_swiglu_16bit(oracle, dev, dtype, n):
    say("swiglu", dtype, n)
    g, u = swiglu_inputs(n, 60 + n)
    if dtype == "bf16":
        gt = dev_t(g).to(torch.bfloat16)
        ut = dev_t(u).to(torch.bfloat16)
    else:
        g = np.clip(g, -60000, 60000)
        gt = dev_t(g).to(torch.float16)
        ut = dev_t(u).to(torch.float16)
    ref32 = oracle.swiglu_f32(gt.float().cpu().numpy(), ut.float().cpu().numpy())
    out = ops.fused_swiglu(gt, ut)
    torch.cuda.synchronize()
    assert out.dtype == gt.dtype and out.shape == gt.shape
    got32 = out.float().cpu().numpy()
    if dtype == "bf16":
        check_rounded(bf16_bits(out), f32_to_bf16_np(ref32), f"swiglu bf16 n={n}", "bf16", got32, ref32)
    else:
        ref16 = np.clip(ref32, -65504, 65504).astype(np.float16).view(np.uint16)
        check_rounded(out.view(torch.int16).cpu().numpy().view(np.uint16), ref16, f"swiglu f16 n={n}", "fp16",
                      got32, ref32)


def test_swiglu_extension_shapes_and_in_place(oracle, dev):
    """Any shape (numel elements) through the reference binding name; out may
    alias an input at the C ABI."""
    say("swiglu 3-D through fused_swiglu_forward, then in place")
    g, u = swiglu_inputs(3 * 5 * 67, 81)
    gt, ut = dev_t(g.reshape(3, 5, 67)), dev_t(u.reshape(3, 5, 67))
    out = _ext.ext().fused_swiglu_forward(gt, ut)
    torch.cuda.synchronize()
    ref = oracle.swiglu_f32(g, u).reshape(3, 5, 67)
    check_f32(out.cpu().numpy(), ref, "3-D")
    st = _lib.lib().fke_swiglu(gt.data_ptr(), ut.data_ptr(), gt.data_ptr(), gt.numel(), _lib.IN_F32,
                               torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "fke_swiglu")
    torch.cuda.synchronize()
    assert torch.equal(gt, out)


# ------------------------------------------------------------- fused GEMM

def swiglu_gemm_inputs(oracle, M, I, K, seed):
    A = oracle.gen_i8_clipped_normal((M, K), seed, 30.0)
    W = oracle.gen_i8_uniform((2 * I, K), seed + 1)
    sa = oracle.gen_f32_uniform((M,), seed + 2, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((2 * I,), seed + 3, 0.0005, 0.005)
    bias = oracle.gen_f32_normal((2 * I,), seed + 4, 0.0, 0.5)
    return A, W, sa, sb, bias


CASES = [
    # (M, I, K, path)
    (1, 200, 4096, "gemv"), (1, 130, 192, "gemv"), (2, 77, 320, "gemv"), (3, 64, 4096, "gemv"),
    (4, 33, 128, "gemv"), (2, 77, 100, "gemv"), (4, 50, 68, "gemv"), (5, 100, 256, "gemv"), (9, 300, 1024, "gemv"), (16, 47, 4096, "gemv"),
    (17, 130, 2048, "gemv"), (40, 300, 4096, "gemv"), (64, 100, 2048, "gemv"), (100, 77, 4096, "gemv"),
    (200, 513, 2048, "gemv"),
    (17, 130, 256, "mfma"), (300, 200, 512, "mfma"), (256, 128, 128, "mfma"), (513, 333, 384, "mfma"),
    (300, 200, 512, "mfma_256x256"), (513, 333, 384, "mfma_256x256"),
    (17, 130, 256, "mfma_128x128"), (256, 128, 128, "mfma_128x128"), (513, 333, 384, "mfma_128x128"),
    (17, 130, 256, "mfma_128x128_ring4"), (300, 200, 640, "mfma_128x128_ring4"), (513, 333, 384, "mfma_128x128_ring4"),
    (33, 40, 100, "generic"), (7, 9, 77, "generic"), (1, 5, 3, "generic"), (70, 100, 256, "generic"),
    # K % 16 != 0 (K % 4 == 0): the word kernel's SwiGLU form, 128x64 tiles and (I = 1100, M = 1024) 128x128
    (9, 300, 100, "mfma"), (70, 100, 1028, "mfma"), (300, 200, 68, "mfma"), (1024, 1100, 100, "mfma"),
]


@pytest.mark.parametrize("M,I,K,path", CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_w8a8_swiglu_vs_oracle_and_unfused(oracle, dev, M, I, K, path, with_bias):
    say("w8a8_swiglu", M, I, K, path, "bias" if with_bias else "no bias")
    A, W, sa, sb, bias = swiglu_gemm_inputs(oracle, M, I, K, 1000 + M * 7 + I + K)
    b = bias if with_bias else None
    At, Wt, sat, sbt = dev_t(A), dev_t(W), dev_t(sa), dev_t(sb)
    bt = None if b is None else dev_t(b)
    h32 = ops.w8a8_swiglu(At, Wt, sat, sbt, bt, out_dtype=torch.float32, path=path)
    h16 = ops.w8a8_swiglu(At, Wt, sat, sbt, bt, out_dtype=torch.bfloat16, path=path)
    # unfused: one fp32 GEMM over all 2I rows, then the elementwise op
    y = ops.w8a8_gemm(At, Wt, sat, sbt, bt, out_dtype=torch.float32)
    hu = ops.fused_swiglu(y[:, :I].contiguous(), y[:, I:].contiguous())
    torch.cuda.synchronize()
    ref = oracle.w8a8_swiglu(A, W, sa, sb, bias=b, nthreads=NTH)
    h32n = h32.cpu().numpy()
    check_f32(h32n, ref, "fused f32 vs oracle")
    assert np.array_equal(h32n.view(np.uint32), hu.cpu().numpy().view(np.uint32)), "fused != unfused"
    assert np.array_equal(bf16_bits(h16), f32_to_bf16_np(h32n)), "bf16 output != bf16(fp32 output)"


def test_w8a8_swiglu_scalar_scales_and_extension(oracle, dev):
    say("w8a8_swiglu scalar scales, torch extension")
    M, I, K = 40, 96, 256
    A, W, _, _, _ = swiglu_gemm_inputs(oracle, M, I, K, 77)
    out = _ext.ext().quantized_gemm_int8_swiglu_forward(dev_t(A), dev_t(W), None, None, None, torch.float32,
                                                        0.01, 0.002)
    torch.cuda.synchronize()
    check_f32(out.cpu().numpy(), oracle.w8a8_swiglu(A, W, sa=0.01, sb=0.002, nthreads=NTH), "scalar scales")


@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_w8a8_swiglu_decode_full(oracle, dev, M):
    """Llama-3-8B MLP gate/up at decode: K = 4096, I = 14336 (W is 112 MiB)."""
    say("w8a8_swiglu decode full", M)
    A, W, sa, sb, bias = swiglu_gemm_inputs(oracle, M, 14336, 4096, 90 + M)
    h = ops.w8a8_swiglu(dev_t(A), dev_t(W), dev_t(sa), dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    torch.cuda.synchronize()
    check_f32(h.cpu().numpy(), oracle.w8a8_swiglu(A, W, sa, sb, bias=bias, nthreads=NTH), f"decode M={M}")


def test_w8a8_swiglu_decode_weight_past_2gib(oracle, dev):
    """M = 8, I = 300000, K = 4096: the [gate; up] weight is 2.46 GB, past
    32-bit offsets from its base; the LDS-streamed kernel addresses each
    workgroup's rows from their own base.  Sampled output columns (both ends,
    the middle) against the oracle on host copies of their gate and up rows."""
    M, I, K = 8, 300000, 4096
    say("w8a8_swiglu decode, weight past 2 GiB", M, I, K)
    assert _lib.lib().fke_select_path_i8_swiglu(4096, 4096, 4096, M, I, K, 0) == _lib.PATH_GEMV
    g = torch.Generator(device=dev)
    g.manual_seed(31337)
    Wd = torch.randint(-127, 128, (2 * I, K), dtype=torch.int8, device=dev, generator=g)
    A = oracle.gen_i8_clipped_normal((M, K), 31338, 30.0)
    sa = oracle.gen_f32_uniform((M,), 31339, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((2 * I,), 31340, 0.0005, 0.005)
    bias = oracle.gen_f32_normal((2 * I,), 31341, 0.0, 0.5)
    h = ops.w8a8_swiglu(dev_t(A), Wd, dev_t(sa), dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    torch.cuda.synchronize()
    cols = np.concatenate([np.arange(0, 300), np.arange(I // 2 - 150, I // 2 + 150), np.arange(I - 300, I)])
    rows = np.concatenate([cols, I + cols])
    Ws = Wd[torch.from_numpy(rows).long().cuda()].cpu().numpy()
    del Wd
    ns = len(cols)
    ref = oracle.w8a8_swiglu(A, Ws, sa, np.concatenate([sb[cols], sb[I + cols]]),
                             bias=np.concatenate([bias[cols], bias[I + cols]]), nthreads=NTH)
    check_f32(h[:, torch.from_numpy(cols).long().cuda()].cpu().numpy(), ref, "decode past 2 GiB")
    assert ref.shape == (M, ns)


def test_w8a8_swiglu_prefill_full(oracle, dev):
    """M = 4096 tokens, I = 14336, K = 4096: all rows against the unfused GPU
    pipeline (bit for bit), sampled rows against the oracle."""
    say("w8a8_swiglu prefill full 4096x14336x4096")
    M, I, K = 4096, 14336, 4096
    A, W, sa, sb, bias = swiglu_gemm_inputs(oracle, M, I, K, 123)
    At, Wt, sat, sbt, bt = dev_t(A), dev_t(W), dev_t(sa), dev_t(sb), dev_t(bias)
    h = ops.w8a8_swiglu(At, Wt, sat, sbt, bt, out_dtype=torch.float32)
    y = ops.w8a8_gemm(At, Wt, sat, sbt, bt, out_dtype=torch.float32)
    hu = ops.fused_swiglu(y[:, :I].contiguous(), y[:, I:].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), hu.view(torch.int32)), "fused != unfused"
    del y, hu
    rows = np.array([0, 1, 255, 256, 2047, 4095], dtype=np.int32)
    ref = oracle.w8a8_swiglu(A, W, sa, sb, bias=bias, rows=rows, nthreads=NTH)
    check_f32(h[torch.from_numpy(rows).long().cuda()].cpu().numpy(), ref, "prefill sampled rows")


@pytest.mark.parametrize("M", [1, 300])
def test_w8a8_gate_up_swiglu_end_to_end(oracle, dev, M):
    """bf16 activations -> per-token quantiser -> fused gate/up SwiGLU, against
    the oracle's quantiser followed by its fused GEMM."""
    say("w8a8_gate_up_swiglu", M)
    I, K = 256, 512
    r = np.random.default_rng(5 + M)
    x = torch.from_numpy(r.standard_normal((M, K)).astype(np.float32)).cuda().to(torch.bfloat16)
    _, W, _, sb, bias = swiglu_gemm_inputs(oracle, 1, I, K, 500)
    h = ops.w8a8_gate_up_swiglu(x, dev_t(W), dev_t(sb), dev_t(bias), out_dtype=torch.float32)
    torch.cuda.synchronize()
    q, s = oracle.quantize_rows_i8(bf16_bits(x), oracle.IN_BF16)
    check_f32(h.cpu().numpy(), oracle.w8a8_swiglu(q, W, s, sb, bias=bias, nthreads=NTH), "end to end")
