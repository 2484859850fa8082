"""GPU tests of the fp16 / bf16 GEMM (fke_gemm_half, the drop-in
fke_launch_wmma_gemm_fp16 for reference src/tensor_core_attention.cu:13-86)
against the CPU oracle (oracle/fke_oracle.c: fko_gemm_half).

Bars:
  * operands that are small integers (or integers times a power of two,
    fp16 subnormals included): every partial sum is exact in fp32, so both
    families must equal the oracle bit for bit, epilogue included;
  * GENERIC family: bit-exact on any data (it sums k = 0..K-1 in order, as
    the oracle does);
  * MFMA family on random data: |gpu - oracle| <= 2 * K * 2^-24 * sum_k |a b|
    per element, the sum of the two results' fp32 summation-error bounds
    (each is within K * 2^-24 * sum|a b| of the exact value whatever the
    order); bf16 output = bf16 rounding of the fp32 output.
The reference ships no test of its WMMA GEMM; these closed-form checks pin it.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _lib, ops  # noqa: E402

NTH = 16
TD = {"f16": torch.float16, "bf16": torch.bfloat16}


def say(*a):
    print("[case]", *a, flush=True)


def enc(x, dt):
    """fp32 numpy -> raw uint16 codes of fp16 / bf16 (round to nearest even)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dt == "f16":
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def dev_codes(bits, dt):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(TD[dt])


def dev_f32(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def code(dt, oracle):
    return oracle.HALF_F16 if dt == "f16" else oracle.HALF_BF16


def host(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def run(A, B, dt, layout="nk", path="auto", sa=None, sb=None, bias=None, out="f32", alpha=1.0):
    r = ops.gemm_half(dev_codes(A, dt), dev_codes(B, dt), dev_f32(sa), dev_f32(sb), dev_f32(bias),
                      out_dtype=torch.float32 if out == "f32" else torch.bfloat16, b_layout=layout, sa=alpha,
                      path=path)
    torch.cuda.synchronize()
    return host(r)


def same_bits(got, ref, what):
    g = got.view(np.uint32) if got.dtype == np.float32 else got
    r = ref.view(np.uint32) if ref.dtype == np.float32 else ref
    bad = g != r
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} mismatches, first at {i}: {got[i]!r} vs {ref[i]!r}")


def int_operands(M, N, K, seed, lo=-8, hi=8):
    r = np.random.default_rng(seed)
    return r.integers(lo, hi + 1, (M, K)).astype(np.float32), r.integers(lo, hi + 1, (N, K)).astype(np.float32)


def epi_vectors(M, N, seed):
    r = np.random.default_rng(seed)
    return (r.uniform(0.5, 2, M).astype(np.float32), r.uniform(0.01, 0.1, N).astype(np.float32),
            r.standard_normal(N).astype(np.float32))


MFMA_SHAPES = [(256, 256, 64), (300, 200, 512), (513, 333, 384), (1, 100, 128), (40, 1000, 64),
               # K % 64 != 0 (K % 8 == 0): a partial last stage, cleared past K
               (129, 70, 8), (256, 256, 72), (300, 200, 1000)]


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("shape", MFMA_SHAPES)
@pytest.mark.parametrize("tile", ["mfma_256x256", "mfma_128x128", "mfma_128x128_ring4", "mfma_128x64_ring4",
                                  "mfma_64x64_ring4"])
def test_mfma_integer_operands_bit_exact(oracle, dev, dt, shape, tile):
    M, N, K = shape
    say("half gemm mfma integers", dt, shape, tile)
    a, b = int_operands(M, N, K, 100 + M + N + K)
    A, B = enc(a, dt), enc(b, dt)
    sa, sb, bias = epi_vectors(M, N, 7)
    got = run(A, B, dt, path=tile, sa=sa, sb=sb, bias=bias)
    ref = oracle.gemm_half(A, B, code(dt, oracle), sa, sb, bias=bias, nthreads=NTH)
    same_bits(got, ref, f"{dt} {shape}")
    gotb = run(A, B, dt, path=tile, sa=sa, sb=sb, bias=bias, out="bf16")
    same_bits(gotb, enc(ref, "bf16"), f"{dt} {shape} bf16 out")


def test_mfma_f16_subnormal_operands(oracle, dev):
    """fp16 subnormals (multiples of 2^-24) times small integers: exact sums
    of multiples of 2^-24, so the MFMA must keep subnormal inputs."""
    say("half gemm mfma fp16 subnormals")
    M, N, K = 64, 64, 256
    r = np.random.default_rng(3)
    a = (r.integers(-1023, 1024, (M, K)) * 2.0**-24).astype(np.float32)   # |a| < 2^-14: subnormal fp16
    b = r.integers(-8, 9, (N, K)).astype(np.float32)
    A, B = enc(a, "f16"), enc(b, "f16")
    assert np.array_equal(A.view(np.float16).astype(np.float32), a)
    got = run(A, B, "f16", path="mfma")
    ref = oracle.gemm_half(A, B, oracle.HALF_F16, nthreads=NTH)
    same_bits(got, ref, "fp16 subnormal operands")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(300, 200, 512), (129, 257, 1024)])
def test_mfma_random_within_bound(oracle, dev, dt, shape):
    M, N, K = shape
    say("half gemm mfma random", dt, shape)
    r = np.random.default_rng(200 + K)
    A, B = enc(r.standard_normal((M, K)), dt), enc(r.standard_normal((N, K)), dt)
    got = run(A, B, dt, path="mfma")
    ref = oracle.gemm_half(A, B, code(dt, oracle), nthreads=NTH)
    dec = (lambda c: c.view(np.float16).astype(np.float64)) if dt == "f16" else \
        (lambda c: (c.astype(np.uint32) << 16).view(np.float32).astype(np.float64))
    bound = 2 * K * 2.0**-24 * (np.abs(dec(A)) @ np.abs(dec(B)).T)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= bound), f"max err/bound {np.max(err / np.maximum(bound, 1e-30)):.3f}"
    gotb = run(A, B, dt, path="mfma", out="bf16")
    same_bits(gotb, enc(got, "bf16"), "bf16 out = bf16(fp32 out)")
    for tile in ("mfma_256x256", "mfma_128x128", "mfma_128x128_ring4", "mfma_128x64_ring4", "mfma_64x64_ring4"):
        same_bits(run(A, B, dt, path=tile), got, f"{tile} vs auto")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (7, 13, 77), (65, 70, 129), (33, 40, 300)])
def test_generic_bit_exact(oracle, dev, dt, layout, shape):
    M, N, K = shape
    say("half gemm generic", dt, layout, shape)
    r = np.random.default_rng(300 + M + K)
    A = enc(r.standard_normal((M, K)), dt)
    Bnk = enc(r.standard_normal((N, K)), dt)
    B = Bnk if layout == "nk" else np.ascontiguousarray(Bnk.T)
    sa, sb, bias = epi_vectors(M, N, 9)
    lay = oracle.B_NK if layout == "nk" else oracle.B_KN
    got = run(A, B, dt, layout=layout, path="generic", sa=sa, sb=sb, bias=bias)
    ref = oracle.gemm_half(A, B, code(dt, oracle), sa, sb, bias=bias, b_layout=lay, nthreads=NTH)
    same_bits(got, ref, f"{dt} {layout} {shape}")


def test_dropin_wmma_gemm_fp16(oracle, dev):
    """fke_launch_wmma_gemm_fp16: C = alpha * A B^T over fp16 A [M,K], B [N,K];
    beta is ignored and C is overwritten (reference src/tensor_core_attention.cu:57-65)."""
    say("drop-in launch_wmma_gemm_fp16")
    M, N, K = 128, 192, 256
    a, b = int_operands(M, N, K, 11)
    A, B = enc(a, "f16"), enc(b, "f16")
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    At, Bt = dev_codes(A, "f16"), dev_codes(B, "f16")  # held: the call takes raw pointers
    st = _lib.lib().fke_launch_wmma_gemm_fp16(At.data_ptr(), Bt.data_ptr(), C.data_ptr(), M, N, K, 0.5, 3.0,
                                              torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "fke_launch_wmma_gemm_fp16")
    torch.cuda.synchronize()
    want = (a.astype(np.int64) @ b.astype(np.int64).T).astype(np.float32) * np.float32(0.5)
    same_bits(C.cpu().numpy(), want, "alpha * A B^T")


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_full_8192_cubed_sampled_rows(oracle, dev, dt):
    """8192^3 on the MFMA path: integer operands (exact), all outputs against the
    int64 matmul of sampled rows and the oracle on those rows."""
    say("half gemm 8192^3", dt)
    M = N = K = 8192
    r = np.random.default_rng(17)
    a = r.integers(-4, 5, (M, K)).astype(np.float32)
    b = r.integers(-4, 5, (N, K)).astype(np.float32)
    A, B = enc(a, dt), enc(b, dt)
    C = ops.gemm_half(dev_codes(A, dt), dev_codes(B, dt), out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 4095, 8191], dtype=np.int32)
    ref = oracle.gemm_half(A, B, code(dt, oracle), rows=rows, nthreads=NTH)
    same_bits(C[torch.from_numpy(rows).long().cuda()].cpu().numpy(), ref, f"{dt} 8192^3 sampled rows")


def _device_int_codes(shape, dt, seed, dev):
    """Small-integer operands made on the device (exact in fp16 and bf16)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randint(-4, 5, shape, dtype=torch.int8, device=dev, generator=g).to(TD[dt])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("M,want_path", [((1 << 31) // 16384 - 1, "mfma"), ((1 << 31) // 16384 + 1, "generic")])
def test_largest_activation_panel(oracle, dev, dt, M, want_path):
    """M * 2K at the MFMA kernel's 32-bit byte-offset limit (2 GiB of A), and
    just past it, where the dispatcher sends the call to the generic kernel:
    sampled rows against the oracle (integer operands: exact)."""
    N, K = 128, 8192
    say("half gemm largest A", dt, M, want_path)
    path = {"mfma": _lib.PATH_MFMA, "generic": _lib.PATH_GENERIC}[want_path]
    Ad = _device_int_codes((M, K), dt, 21, dev)
    B = enc(int_operands(1, N, K, 22)[1], dt)
    Bd = dev_codes(B, dt)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    sel = _lib.lib().fke_select_path_half(Ad.data_ptr(), Bd.data_ptr(), C.data_ptr(), M, N, K,
                                         _lib.IN_F16 if dt == "f16" else _lib.IN_BF16, _lib.OUT_F32, _lib.B_NK)
    assert sel == path
    C = ops.gemm_half(Ad, Bd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 255, 256, M // 2, M - 257, M - 2, M - 1], device=dev)
    A = host(Ad[rows]).view(np.uint16)
    ref = oracle.gemm_half(A, B, code(dt, oracle), nthreads=NTH)
    same_bits(C[rows].cpu().numpy(), ref, f"{dt} M={M}")
