"""CPU tests that pin the oracle (oracle/fke_oracle.c) before it is trusted.

Each oracle function is checked against the reference's own known answers
(the KAT64 case of tests/test_quantized_gemm.cu), against fixtures
(tests/golden/golden.json), and against what the mathematics fixes: numpy
int64 matmuls, exact rational arithmetic, torch's float8/bfloat16 casts
(library routines), closed forms and hand-derived tiny cases.  Each check is
chosen so that a plausible slip (transposed B, dropped K tail, wrong bias
rounding, wrong decode exponent) fails it.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "golden.json")))


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- generators

def test_splitmix64_published_vector(oracle):
    g = GOLDEN["splitmix64"]
    assert oracle.splitmix64_stream(g["seed"], 5) == g["first5"]


def test_generators_ranges_and_moments(oracle):
    a = oracle.gen_i8_uniform((1 << 16,), 1)
    assert a.min() == -127 and a.max() == 127
    assert abs(a.astype(np.float64).mean()) < 1.5
    s = oracle.gen_f32_uniform((1 << 16,), 2, 0.001, 0.02)
    assert s.min() >= 0.001 and s.max() < 0.02
    z = oracle.gen_f32_normal((1 << 16,), 3, 0.0, 0.02)
    assert abs(z.mean()) < 1e-3 and abs(z.std() - 0.02) < 1e-3
    c = oracle.gen_i8_clipped_normal((1 << 16,), 4, 30.0)
    assert c.min() >= -127 and c.max() <= 127 and abs(c.std() - 30.0) < 1.0
    # deterministic per seed, different across seeds
    assert np.array_equal(oracle.gen_i8_uniform((64,), 9), oracle.gen_i8_uniform((64,), 9))
    assert not np.array_equal(oracle.gen_i8_uniform((64,), 9), oracle.gen_i8_uniform((64,), 10))


# ------------------------------------------------------- INT8 reference GEMM

def kat64_inputs():
    M = N = K = 64
    A = (np.arange(M * K) % 7 - 3).astype(np.int8).reshape(M, K)
    B = (np.arange(N * K) % 5 - 2).astype(np.int8).reshape(N, K)
    return A, B


def test_kat64_reference_case(oracle):
    """The reference test's closed-form case (tests/test_quantized_gemm.cu:19-48)."""
    g = GOLDEN["kat64"]
    A, B = kat64_inputs()
    acc = oracle.w8a8_acc(A, B)
    assert int(acc.sum()) == g["acc_sum"]
    assert int(acc.min()) == g["acc_min"] and int(acc.max()) == g["acc_max"]
    assert int((acc != 0).sum()) == g["acc_nonzero"]
    assert acc[0, :8].tolist() == g["acc_row0_first8"]
    assert int(acc[63, 63]) == g["acc_63_63"]
    C = oracle.ref_host_gemm_i8(A, B, 0.05, 0.02)
    alpha = np.array(g["alpha_bits"], dtype=np.uint32).view(np.float32)
    assert np.array_equal(C, acc.astype(np.float32) * alpha)
    assert C[0, 0] == np.float32(-6.0) * alpha


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 5, 7), (17, 9, 64), (8, 33, 130), (8, 8, 8)])
def test_ref_host_gemm_vs_numpy(oracle, shape):
    M, N, K = shape
    r = rng(sum(shape))
    A = r.integers(-127, 128, (M, K), dtype=np.int8)
    B = r.integers(-127, 128, (N, K), dtype=np.int8)
    sa, sb = np.float32(0.013), np.float32(0.0071)
    C = oracle.ref_host_gemm_i8(A, B, float(sa), float(sb))
    acc = A.astype(np.int64) @ B.astype(np.int64).T  # B is [N,K]: transposed here
    assert np.array_equal(C, acc.astype(np.float32) * (sa * sb))
    # a transposed-B mistake would not pass: B is not symmetric in these cases
    if M == N == K and M > 1:
        assert not np.array_equal(acc, A.astype(np.int64) @ B.astype(np.int64))


def test_ref_kernel_equals_host_for_k_multiple_of_4(oracle):
    r = rng(5)
    A = r.integers(-127, 128, (13, 96), dtype=np.int8)
    B = r.integers(-127, 128, (11, 96), dtype=np.int8)
    assert np.array_equal(oracle.ref_kernel_gemm_i8(A, B, 0.5, 0.25),
                          oracle.ref_host_gemm_i8(A, B, 0.5, 0.25))


def test_ref_kernel_k_tail_truncation_hand_case(oracle):
    """src/quantized_gemm.cu:28-35 with K=5: one int32 word per row, row r starting
    at byte 4*r.  Row 0 sums bytes 0..3, row 1 bytes 4..7 (misaligned)."""
    A = np.arange(1, 11, dtype=np.int8).reshape(2, 5)
    B = np.ones((1, 5), dtype=np.int8)
    C = oracle.ref_kernel_gemm_i8(A, B, 1.0, 1.0)
    assert C.ravel().tolist() == [1 + 2 + 3 + 4, 5 + 6 + 7 + 8]
    # the host loop of the reference test uses the full K instead
    assert oracle.ref_host_gemm_i8(A, B, 1.0, 1.0).ravel().tolist() == [15, 40]


def test_ref_py_gemm_matches_numpy_expression(oracle):
    """python/flash_engine/ops.py:180-186, evaluated by numpy itself."""
    r = rng(11)
    A = r.integers(-127, 127, (32, 64), dtype=np.int8)
    B = r.integers(-127, 127, (64, 32), dtype=np.int8)
    for sa, sb in [(1.0, 1.0), (0.01, 0.02), (0.0123, 0.0456)]:
        expect = np.matmul(A.astype(np.int32), B.astype(np.int32)).astype(np.float32) * (sa * sb)
        got = oracle.ref_py_gemm_i8(A, B, sa, sb)
        assert got.dtype == np.float32 and np.array_equal(got, expect)


@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_w8a8_acc_vs_numpy(oracle, layout):
    r = rng(21)
    M, N, K = 19, 37, 200
    A = r.integers(-127, 128, (M, K), dtype=np.int8)
    Bnk = r.integers(-127, 128, (N, K), dtype=np.int8)
    B = Bnk if layout == "nk" else np.ascontiguousarray(Bnk.T)
    code = oracle.B_NK if layout == "nk" else oracle.B_KN
    acc = oracle.w8a8_acc(A, B, code, nthreads=3)
    assert np.array_equal(acc, (A.astype(np.int64) @ Bnk.astype(np.int64).T).astype(np.int32))
    rows = np.array([18, 0, 7], dtype=np.int32)
    assert np.array_equal(oracle.w8a8_acc(A, B, code, rows=rows), acc[rows])


def test_w8a8_full_range_extremes(oracle):
    """|acc| = K*127^2 at K=8192 (1.32e8) stays exact (no overflow)."""
    K = 8192
    A = np.full((2, K), -127, dtype=np.int8)
    B = np.stack([np.full(K, -127, np.int8), np.full(K, 127, np.int8)])
    acc = oracle.w8a8_acc(A, B)
    assert acc[0].tolist() == [K * 127 * 127, -K * 127 * 127]


# ------------------------------------------------------------------ epilogue

def f32_rne(x: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to fp32 (no double rounding)."""
    c = np.float32(float(x))
    cands = {c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))}
    best = sorted(cands, key=lambda v: (abs(Fraction(float(v)) - x),
                                        int(np.array(v, np.float32).view(np.uint32)) & 1))
    return best[0]


def test_epilogue_reduces_to_reference(oracle):
    """Uniform scales, no bias, fp32 out == tests/test_quantized_gemm.cu:46."""
    r = rng(31)
    A = r.integers(-127, 128, (24, 64), dtype=np.int8)
    B = r.integers(-127, 128, (40, 64), dtype=np.int8)
    acc = oracle.w8a8_acc(A, B)
    ref = oracle.ref_host_gemm_i8(A, B, 0.05, 0.02)
    y_scalar = oracle.w8a8_epilogue(acc, sa=0.05, sb=0.02)
    y_vec = oracle.w8a8_epilogue(acc, np.full(24, 0.05, np.float32), np.full(40, 0.02, np.float32))
    assert np.array_equal(y_scalar, ref) and np.array_equal(y_vec, ref)


def test_epilogue_bias_is_one_rounding(oracle):
    """y = round_f32(fp32(acc) * s + bias) exactly (fmaf), checked with exact
    rationals; a two-rounding mul-then-add differs on some of these."""
    r = rng(41)
    acc = r.integers(-2_000_000, 2_000_000, (8, 64)).astype(np.int32)
    sa = oracle.gen_f32_uniform((8,), 5, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((64,), 6, 0.001, 0.02)
    bias = oracle.gen_f32_normal((64,), 7, 0.0, 0.02)
    y = oracle.w8a8_epilogue(acc, sa, sb, bias=bias)
    differs_from_two_roundings = 0
    for m in range(8):
        for n in range(64):
            s = np.float32(sa[m] * sb[n])
            exact = Fraction(float(np.float32(acc[m, n]))) * Fraction(float(s)) + Fraction(float(bias[n]))
            assert y[m, n] == f32_rne(exact), (m, n)
            two = np.float32(np.float32(np.float32(acc[m, n]) * s) + bias[n])
            differs_from_two_roundings += int(two != y[m, n])
    assert differs_from_two_roundings > 0


def test_bf16_rne_known_answers(oracle):
    assert oracle.f32_to_bf16_rne(1.0) == 0x3F80
    assert oracle.f32_to_bf16_rne(1.0 + 2.0 ** -8) == 0x3F80       # tie -> even
    assert oracle.f32_to_bf16_rne(1.0 + 3 * 2.0 ** -8) == 0x3F82   # tie -> even (up)
    assert oracle.f32_to_bf16_rne(1.0 + 2.0 ** -8 + 2.0 ** -20) == 0x3F81
    assert oracle.f32_to_bf16_rne(-2.5) == 0xC020
    assert oracle.f32_to_bf16_rne(float("inf")) == 0x7F80


def test_bf16_rne_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    x = np.concatenate([oracle.gen_f32_normal((4096,), 8, 0, 3.0),
                        oracle.gen_f32_uniform((4096,), 9, -1e-3, 1e-3)]).astype(np.float32)
    acc = np.zeros((1, x.size), np.int32)
    # route through the epilogue's bf16 store: acc=0 with bias=x gives y=x
    got = oracle.w8a8_epilogue(acc, sa=1.0, sb=1.0, bias=x, out_dtype=oracle.OUT_BF16)[0]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


# ----------------------------------------------------------------------- FP8

def test_e4m3_decode_exhaustive(oracle):
    table = oracle.e4m3_decode_table()
    golden = np.array(GOLDEN["e4m3"], dtype=np.uint32).view(np.float32)
    assert np.array_equal(table.view(np.uint32), golden.view(np.uint32))
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e, m = (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            assert table[code] == 0.0  # the reference's NaN clamp
        elif e == 0:
            assert table[code] == s * m / 512.0
        else:
            assert table[code] == s * (1 + m / 8) * 2.0 ** (e - 7)
    assert table[0x7E] == 448.0 and table[0xFE] == -448.0 and table[0x01] == 2.0 ** -9


def test_e4m3_decode_matches_torch_float8(oracle):
    torch = pytest.importorskip("torch")
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(oracle.e4m3_decode_table()[codes], ref)


def test_e4m3_quantizer(oracle):
    torch = pytest.importorskip("torch")
    x = oracle.gen_f32_normal((1 << 15,), 12, 0.0, 1.0)
    q, s = oracle.quantize_e4m3(x)
    assert s == np.float32(np.abs(x).max()) / np.float32(448.0)
    assert not np.isin(q, [0x7F, 0xFF]).any()
    v = (x / np.float32(s)).astype(np.float32)
    ref = torch.from_numpy(np.clip(v, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)
    # saturation instead of NaN, RNE ties to even, subnormals
    assert oracle.f32_to_e4m3_sat(1e9) == 0x7E and oracle.f32_to_e4m3_sat(-500.0) == 0xFE
    assert oracle.f32_to_e4m3_sat(1.0625) == 0x38   # 1 + 1/16: tie -> 1.0 (even)
    assert oracle.f32_to_e4m3_sat(1.1875) == 0x3A   # 1 + 3/16: tie -> 1.25 (even)
    assert oracle.f32_to_e4m3_sat(2.0 ** -9) == 0x01
    assert oracle.f32_to_e4m3_sat(2.0 ** -10) == 0x00  # tie -> 0 (even)


def f8_sequential(A, B_kn, table, alpha):
    """Python float32 restatement of src/quantized_gemm.cu:109-116 (k in order)."""
    M, K = A.shape
    N = B_kn.shape[1]
    C = np.zeros((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            s = np.float32(0.0)
            for k in range(K):
                s = np.float32(s + table[A[m, k]] * table[B_kn[k, n]])
            C[m, n] = np.float32(s * alpha)
    return C


def test_f8_reference_sequential_order(oracle):
    r = rng(51)
    A = r.integers(0, 256, (5, 70), dtype=np.uint8)
    B = r.integers(0, 256, (70, 6), dtype=np.uint8)
    table = oracle.e4m3_decode_table()
    alpha = np.float32(np.float32(0.3) * np.float32(0.7))
    ref = f8_sequential(A, B, table, alpha)
    assert np.array_equal(oracle.ref_kernel_gemm_f8(A, B, 0.3, 0.7), ref)
    assert np.array_equal(oracle.f8_gemm(A, B, 0.3, 0.7, b_layout=oracle.B_KN), ref)
    assert np.array_equal(oracle.f8_gemm(A, np.ascontiguousarray(B.T), 0.3, 0.7,
                                         b_layout=oracle.B_NK), ref)
    # exact double-precision sum differs only by fp32 rounding of the partial sums
    exact = (table[A].astype(np.float64) @ table[B].astype(np.float64)) * float(alpha)
    assert np.allclose(ref, exact, rtol=1e-5, atol=1e-6 * np.abs(exact).max())


def _round_to_bits(q, bits):
    """Nearest-even binary float with `bits` significand bits of the exact
    rational q (normal range), as a Python float."""
    from fractions import Fraction
    if q == 0:
        return 0.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    scaled = a * Fraction(2) ** (bits - 1 - e)   # in [2^(bits-1), 2^bits)
    n = round(scaled)                             # Fraction rounds half to even
    return float((1 if q > 0 else -1) * n * Fraction(2) ** (e - bits + 1))


def test_f8_bias_and_bf16_epilogue(oracle):
    """fko_f8_gemm's bias and bf16 arm on its own: y = fmaf(s, fp32(sa*sb),
    bias[n]) with s the sequential fp32 sum, rounded once (checked with exact
    rationals), then bf16 = nearest-even of that fp32 y to 8 significand bits.
    Bias magnitudes span the sums' so that a separate multiply-then-add (two
    roundings) would differ somewhere."""
    from fractions import Fraction
    r = rng(53)
    M, K, N = 6, 90, 7
    A = r.integers(0, 256, (M, K), dtype=np.uint8)
    B = r.integers(0, 256, (K, N), dtype=np.uint8)
    table = oracle.e4m3_decode_table()
    sa, sb = 0.3, 0.7
    alpha = np.float32(np.float32(sa) * np.float32(sb))
    bias = (r.standard_normal(N) * np.array([1e-3, 1e-1, 1, 10, 100, 1e3, 1e4])).astype(np.float32)
    y32 = oracle.f8_gemm(A, B, sa, sb, bias=bias, b_layout=oracle.B_KN)
    y16 = oracle.f8_gemm(A, B, sa, sb, bias=bias, out_dtype=oracle.OUT_BF16, b_layout=oracle.B_KN)
    y16_nk = oracle.f8_gemm(A, np.ascontiguousarray(B.T), sa, sb, bias=bias, out_dtype=oracle.OUT_BF16,
                            b_layout=oracle.B_NK)
    two_roundings = 0
    for m in range(M):
        for n in range(N):
            s = np.float32(0.0)
            for k in range(K):
                s = np.float32(s + table[A[m, k]] * table[B[k, n]])
            exact = Fraction(float(s)) * Fraction(float(alpha)) + Fraction(float(bias[n]))
            want = np.float32(_round_to_bits(exact, 24))
            assert y32[m, n].view(np.uint32) == want.view(np.uint32), (m, n, y32[m, n], want)
            want16 = np.float32(_round_to_bits(Fraction(float(want)), 8))
            assert y16[m, n] == (want16.view(np.uint32) >> 16), (m, n)
            two_roundings += np.float32(np.float32(s * alpha) + bias[n]) != want
    assert np.array_equal(y16_nk, y16)
    assert two_roundings > 0, "no case separates the fused multiply-add from two roundings"


def test_f8_order_matters_case(oracle):
    """A case where the sequential order is observable: 448*448 = 200704 has an
    fp32 ulp of 2^-6, so each following 1.0 * 2^-9 product is rounded away one
    at a time, while the exact (or a pairwise) sum of the eight keeps 2^-6."""
    A = np.array([[0x7E] + [0x38] * 8], dtype=np.uint8)        # 448, then 1.0 x8
    B = np.array([[0x7E]] + [[0x01]] * 8, dtype=np.uint8)      # 448, then 2^-9 x8
    got = oracle.ref_kernel_gemm_f8(A, B, 1.0, 1.0)[0, 0]
    assert got == np.float32(200704.0)
    assert np.float32(200704.0 + 8 * 2.0 ** -9) == np.float32(200704.015625) != got


# ------------------------------------------------------------------ fixtures

def test_c1_golden_fixture(oracle):
    import hashlib
    g = GOLDEN["c1"]
    M, N, K = g["M"], g["N"], g["K"]
    A = oracle.gen_i8_uniform((M, K), g["seed_A"])
    B = oracle.gen_i8_uniform((N, K), g["seed_B"])
    sa = oracle.gen_f32_uniform((M,), g["seed_sa"], 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), g["seed_sb"], 0.001, 0.02)

    def sha(a):
        return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()

    assert [sha(A), sha(B), sha(sa), sha(sb)] == [g["sha256"][k] for k in ("A", "B", "scale_a", "scale_b")]
    acc = oracle.w8a8_acc(A, B)
    assert np.array_equal(acc, (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32))
    f32 = oracle.w8a8_epilogue(acc, sa, sb)
    bf16 = oracle.w8a8_epilogue(acc, sa, sb, out_dtype=oracle.OUT_BF16)
    assert sha(acc) == g["sha256"]["acc"]
    assert sha(f32) == g["sha256"]["f32"]
    assert sha(bf16) == g["sha256"]["bf16"]
    for m, n, a, fbits, h in g["samples"]:
        assert acc[m, n] == a and f32[m:m + 1, n].view(np.uint32)[0] == fbits and bf16[m, n] == h


# ------------------------------------------------- per-token INT8 quantiser

def test_quantize_rows_known_answers(oracle):
    """Hand-derived rows.  Row 1 has amax 127, so r = 1 exactly and x*r = x:
    2.5 -> 2 and 3.5 -> 4 (ties to even), -2.5 -> -2.  Row 0: r = 127/2 = 63.5
    exactly, so 1 -> 63.5 -> 64 (tie to even), 0.5 -> 31.75 -> 32, and the amax
    element -2 -> -127.  An all-zero row gets scale 1 and zero codes."""
    x = np.array([[1.0, -2.0, 0.5, 0.0],
                  [127.0, 2.5, 3.5, -2.5],
                  [0.0, 0.0, 0.0, 0.0],
                  [-0.25, 0.125, 0.0625, 1e-9]], dtype=np.float32)
    q, s = oracle.quantize_rows_i8(x)
    assert s[0] == np.float32(2.0) / np.float32(127.0)
    assert s[1] == 1.0 and s[2] == 1.0
    assert s[3] == np.float32(0.25) / np.float32(127.0)
    assert q[0].tolist() == [64, -127, 32, 0]
    assert q[1].tolist() == [127, 2, 4, -2]
    assert q[2].tolist() == [0, 0, 0, 0]
    assert q[3].tolist() == [-127, 64, 32, 0]     # r = 508: 0.125 -> 63.5 -> 64, 0.0625 -> 31.75


def test_quantize_rows_invariants(oracle):
    """On random rows: the scale is fp32(amax/127); the amax element maps to
    +-127; every code is within [-127, 127]; and the dequantised value is within
    half a step of x (plus the one rounding of the quotient), checked in exact
    rationals."""
    r = rng(21)
    x = (r.standard_normal((64, 300)) * r.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    q, s = oracle.quantize_rows_i8(x)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(s, amax / np.float32(127.0))
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    for m in range(x.shape[0]):
        k = int(np.argmax(np.abs(x[m])))
        assert q[m, k] == (127 if x[m, k] > 0 else -127)
        sm = Fraction(float(s[m]))
        for k in range(0, x.shape[1], 7):
            err = abs(Fraction(int(q[m, k])) * sm - Fraction(float(x[m, k])))
            assert err <= sm / 2 * Fraction(1 + 2**-20), (m, k)


def test_quantize_rows_matches_numpy_fp32_semantics(oracle):
    """numpy's float32 division and product are IEEE correctly rounded and
    np.rint rounds half to even: an independent evaluation of the same fp32
    arithmetic.  A C slip such as a double-precision product, dividing by s
    instead of multiplying by r, or truncation instead of rint fails."""
    r = rng(22)
    x = (r.standard_normal((40, 1000)) * 3).astype(np.float32)
    x[5, :] = 0.0
    x[6, ::3] = np.float32(1.5)     # exact ties once s is a power of two
    x[6, 0] = np.float32(127.0)
    q, s = oracle.quantize_rows_i8(x)
    amax = np.abs(x).max(axis=1)
    zero = amax == 0
    s_np = np.where(zero, np.float32(1.0), amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        r_np = np.where(zero, np.float32(1.0), np.float32(127.0) / amax).astype(np.float32)
    q_np = np.clip(np.rint(x * r_np[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(s, s_np)
    assert np.array_equal(q, q_np)
    assert q[6, 3] == 2                # 1.5 with s = 1 -> 2 (even)


def _quantize_rows_numpy(x, f=None):
    """The quantiser evaluated by numpy's IEEE float32 arithmetic with the
    row factor f given (None: 2^64 below a 2^-64 maximum, else 1)."""
    amax = np.max(np.where(np.isnan(x), np.float32(0), np.abs(x)), axis=1).astype(np.float32)
    if f is None:
        f = np.where((amax > 0) & (amax < np.float32(2.0**-64)), np.float32(2.0**64), np.float32(1.0))
    f = np.asarray(f, dtype=np.float32) * np.ones_like(amax)
    zero = amax == 0
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        s = np.where(zero, np.float32(1), amax / np.float32(127)).astype(np.float32)
        r = np.where(zero, np.float32(1), np.float32(127) / (amax * f)).astype(np.float32)
        p = (x * f[:, None]).astype(np.float32) * r[:, None]
        q = np.where(np.isnan(p), 0, np.clip(np.rint(np.nan_to_num(p, nan=0.0)), -127, 127)).astype(np.int8)
    return q, s


def test_quantize_rows_tiny_row_maxima(oracle):
    """Rows whose maximum is below 127/FLT_MAX (~3.7e-37), where fp32(127/amax)
    overflows: the power-of-two prescale keeps the amax element at +-127 and
    every code equal to the exact-rational rounding of x*127/amax (to within
    the one rounding of r).  Rows with a maximum in [2^-121, 2^-64) take the
    prescale too, and there the codes equal the f = 1 evaluation: the
    prescale changes no row where 127/amax is finite."""
    r = rng(24)
    base = r.standard_normal((6, 64)).astype(np.float32)
    mags = np.array([1e-38, 2e-40, 1e-44, 3e-37, 1e-30, 2.0**-70], dtype=np.float32)
    x = (base / np.abs(base).max(axis=1, keepdims=True) * mags[:, None]).astype(np.float32)
    x[2, 5] = np.float32(1e-45)            # the smallest subnormal scale of values
    q, s = oracle.quantize_rows_i8(x)
    q_np, s_np = _quantize_rows_numpy(x)
    assert np.array_equal(q, q_np) and np.array_equal(s, s_np)
    amax = np.abs(x).max(axis=1)
    for m in range(x.shape[0]):
        k = int(np.argmax(np.abs(x[m])))
        assert q[m, k] == (127 if x[m, k] > 0 else -127), m
        for kk in range(x.shape[1]):          # |q - x*127/amax| <= 1/2 (+ the rounding of r)
            ideal = Fraction(float(x[m, kk])) * 127 / Fraction(float(amax[m]))
            assert abs(Fraction(int(q[m, kk])) - ideal) <= Fraction(1, 2) + Fraction(1, 2**16), (m, kk)
    with np.errstate(over="ignore", divide="ignore"):
        finite = np.float32(127) / amax < np.float32(np.inf)
    q1, _ = _quantize_rows_numpy(x[finite], f=1.0)
    assert finite.sum() >= 2 and np.array_equal(q[finite], q1)


def test_quantize_rows_non_finite(oracle):
    """NaN elements give code 0 and do not enter the maximum; a row holding
    +-inf has scale inf and r = 0, so every code is 0 (inf * 0 is NaN, finite *
    0 is 0); the other rows are untouched."""
    x = np.array([[1.0, np.inf, -3.0, 0.5],
                  [-np.inf, 2.0, np.nan, 0.0],
                  [np.nan, 2.0, -4.0, 1.0],
                  [np.nan, np.nan, np.nan, np.nan],
                  [np.inf, -np.inf, 0.0, 1e-45]], dtype=np.float32)
    q, s = oracle.quantize_rows_i8(x)
    assert np.isinf(s[0]) and np.isinf(s[1]) and np.isinf(s[4])
    assert q[0].tolist() == [0, 0, 0, 0] and q[1].tolist() == [0, 0, 0, 0] and q[4].tolist() == [0, 0, 0, 0]
    assert s[2] == np.float32(4.0) / np.float32(127.0)
    assert q[2].tolist() == [0, 64, -127, 32]       # r = 31.75: 2 -> 63.5 -> 64
    assert s[3] == 1.0 and q[3].tolist() == [0, 0, 0, 0]
    q_np, s_np = _quantize_rows_numpy(x)
    assert np.array_equal(q, q_np) and np.array_equal(s, s_np)


def test_quantize_rows_bf16_input(oracle):
    """bf16 inputs quantise exactly like their fp32 values (bf16 -> fp32 is
    exact: the bits shifted left by 16)."""
    r = rng(23)
    x32 = r.standard_normal((8, 256)).astype(np.float32)
    bits = np.array([oracle.f32_to_bf16_rne(float(v)) for v in x32.ravel()], dtype=np.uint16).reshape(x32.shape)
    xb = oracle.bf16_to_f32(bits)
    qb, sb = oracle.quantize_rows_i8(bits, oracle.IN_BF16)
    qf, sf = oracle.quantize_rows_i8(xb)
    assert np.array_equal(qb, qf) and np.array_equal(sb, sf)


# ---------------------------------------------------------------- SwiGLU

def test_swiglu_reference_test_vector(oracle):
    """The reference's own check (python/tests/test_correctness.py:166-176):
    gate [-2,-0.5,0,0.5,2], up [1..5], against numpy fp32
    (gate / (1 + exp(-gate))) * up, max abs difference < 1e-6."""
    gate = np.array([-2.0, -0.5, 0.0, 0.5, 2.0], dtype=np.float32)
    up = np.array([1.0, 2.0, 3.0, 4.0, 5.0], dtype=np.float32)
    ref = (gate / (np.float32(1.0) + np.exp(-gate))) * up
    out = oracle.swiglu_f32(gate, up)
    assert np.max(np.abs(out - ref)) < 1e-6


def test_swiglu_float64_closed_form_sweep(oracle):
    """Against g*u/(1+e^-g) in float64 over g in [-90, 90]: within 4 fp32 ulps
    of the exact value wherever sigmoid(g) and the result are normal numbers
    (g > -87: below that 1/(1+e^-g) leaves the normal range and e^-g overflows
    fp32 past -88.7, so the fp32 formula flushes towards zero - there |h| is
    checked to be tiny).  A sign slip (e^+g), a dropped factor (silu without
    u, sigmoid without g) or a wrong operand order is off by far more."""
    r = rng(31)
    g = np.concatenate([np.linspace(-90, 90, 20001), r.standard_normal(5000) * 4]).astype(np.float32)
    u = (r.standard_normal(g.size) * 2).astype(np.float32)
    h = oracle.swiglu_f32(g, u).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    exact = g64 * u64 / (1.0 + np.exp(-g64))
    tiny = float(np.finfo(np.float32).tiny)
    inr = g > -87.0
    normal = inr & (np.abs(exact) >= tiny)
    ulp = np.spacing(np.abs(exact[normal]).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(h[normal] - exact[normal]) <= 4 * ulp)
    sub = inr & ~normal  # subnormal results: a few steps of 2^-149
    assert np.all(np.abs(h[sub] - exact[sub]) <= 8 * 2.0**-149 + 4 * 2.0**-23 * np.abs(exact[sub]))
    low = ~inr           # sigmoid(g) <= e^g < 2^-125
    assert np.all(np.abs(h[low]) <= np.abs(g64 * u64)[low] * 2.0**-124)


def test_swiglu_odd_part_identity(oracle):
    """silu(g) - silu(-g) = g(sigmoid(g) + sigmoid(-g)) = g exactly in real
    arithmetic; with u = 1 the fp32 values agree to a few ulps of |g|."""
    g = np.linspace(-20, 20, 4001).astype(np.float32)
    one = np.ones_like(g)
    d = oracle.swiglu_f32(g, one).astype(np.float64) - oracle.swiglu_f32(-g, one).astype(np.float64)
    assert np.all(np.abs(d - g.astype(np.float64)) <= 4 * np.spacing(np.abs(g)).astype(np.float64) + 1e-30)


def test_swiglu_special_values(oracle):
    """g = 0 gives 0 (sigmoid(0) = 1/2 exactly); g = 100 gives g*u exactly
    (e^-100 < 2^-24, so 1 + e^-100 rounds to 1); g = -100 overflows e^100 to
    inf and gives a signed zero; the pair order is (gate, up): swapping them
    changes the value."""
    assert oracle.lib().fko_swiglu1(0.0, 7.0) == 0.0
    assert oracle.lib().fko_swiglu1(1.0, 0.0) == 0.0
    assert oracle.lib().fko_swiglu1(100.0, 3.0) == 300.0
    v = oracle.lib().fko_swiglu1(-100.0, 3.0)
    assert v == 0.0 and math.copysign(1.0, v) == -1.0
    # sigmoid(ln 3) = 3/4: h = 0.75 * ln3 * u up to the rounding of ln 3 itself
    g = np.float32(math.log(3.0))
    assert abs(oracle.lib().fko_swiglu1(float(g), 2.0) - 1.5 * float(g)) <= 2e-7 * 1.5 * float(g)
    assert oracle.lib().fko_swiglu1(2.0, 0.5) != oracle.lib().fko_swiglu1(0.5, 2.0)


def test_w8a8_swiglu_is_gemm_then_swiglu(oracle):
    """The fused oracle equals the pinned GEMM oracle on W's gate rows
    (0..I-1) and up rows (I..2I-1), each with its own slice of scale_b and
    bias, followed by the pinned elementwise SwiGLU: bit for bit, in fp32 and
    bf16, for all rows and a row subset.  Swapping the halves, indexing
    scale_b / bias by the output column for the up rows, or applying SwiGLU
    to bf16-rounded values fails."""
    r = rng(32)
    M, I, K = 9, 37, 72
    A = r.integers(-127, 128, (M, K), dtype=np.int8)
    W = r.integers(-127, 128, (2 * I, K), dtype=np.int8)
    sa = r.uniform(0.001, 0.02, M).astype(np.float32)
    sb = r.uniform(0.001, 0.02, 2 * I).astype(np.float32)
    bias = (r.standard_normal(2 * I) * 0.5).astype(np.float32)
    for b in (None, bias):
        g = oracle.w8a8_gemm(A, W[:I], sa, sb[:I], bias=None if b is None else b[:I])
        u = oracle.w8a8_gemm(A, W[I:], sa, sb[I:], bias=None if b is None else b[I:])
        h = oracle.swiglu_f32(g, u)
        fused = oracle.w8a8_swiglu(A, W, sa, sb, bias=b)
        assert np.array_equal(fused.view(np.uint32), h.view(np.uint32))
        fb = oracle.w8a8_swiglu(A, W, sa, sb, bias=b, out_dtype=oracle.OUT_BF16)
        hb = np.array([oracle.f32_to_bf16_rne(float(v)) for v in h.ravel()], dtype=np.uint16).reshape(h.shape)
        assert np.array_equal(fb, hb)
        rows = np.array([8, 0, 3], dtype=np.int32)
        assert np.array_equal(oracle.w8a8_swiglu(A, W, sa, sb, bias=b, rows=rows), fused[rows])
    # scalar scales
    g = oracle.w8a8_gemm(A, W[:I], sa=0.5, sb=0.25)
    u = oracle.w8a8_gemm(A, W[I:], sa=0.5, sb=0.25)
    assert np.array_equal(oracle.w8a8_swiglu(A, W, sa=0.5, sb=0.25), oracle.swiglu_f32(g, u))


# ---------------------------------------------------------------- fp16 / bf16 GEMM

def f16_bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits_np(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_f16_decode_exhaustive(oracle):
    """All 65536 binary16 codes against numpy's float16 -> float32 cast (a
    library routine): same bits, NaN for NaN codes."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(codes)
    want = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert oracle.lib().fko_f16_to_f32(0x0001) == 2.0**-24   # smallest subnormal
    assert oracle.lib().fko_f16_to_f32(0x7BFF) == 65504.0    # largest finite


@pytest.mark.parametrize("in_dtype", ["f16", "bf16"])
@pytest.mark.parametrize("layout", [0, 1])
def test_gemm_half_small_integers_exact(oracle, in_dtype, layout):
    """Integer operands in [-8, 8] are exact in both formats and every partial
    sum is an integer below 2^24, so any summation order gives the int64
    matmul exactly.  A transposed B, a dropped K tail or a decode slip fails."""
    r = rng(41)
    M, N, K = 13, 21, 300
    a = r.integers(-8, 9, (M, K)).astype(np.float32)
    b = r.integers(-8, 9, (N, K)).astype(np.float32)
    enc = f16_bits if in_dtype == "f16" else bf16_bits_np
    code = oracle.HALF_F16 if in_dtype == "f16" else oracle.HALF_BF16
    B = enc(b) if layout == 0 else np.ascontiguousarray(enc(b).T)
    got = oracle.gemm_half(enc(a), B, code, b_layout=layout)
    want = a.astype(np.int64) @ b.astype(np.int64).T
    assert np.array_equal(got, want.astype(np.float32))


def test_gemm_half_float64_bound_and_epilogue(oracle):
    """Random fp16 operands: within the sequential-sum bound K * 2^-24 *
    sum|a b| of the float64 product; with scales and bias, each output is
    fmaf(acc, fp32(sa_m * sb_n), bias_n) of the unscaled result."""
    r = rng(42)
    M, N, K = 17, 29, 1000
    a = f16_bits(r.standard_normal((M, K)))
    b = f16_bits(r.standard_normal((N, K)))
    af, bf = a.view(np.float16).astype(np.float64), b.view(np.float16).astype(np.float64)
    acc = oracle.gemm_half(a, b, oracle.HALF_F16)
    exact = af @ bf.T
    bound = K * 2.0**-24 * (np.abs(af) @ np.abs(bf).T)
    assert np.all(np.abs(acc - exact) <= bound)
    sa = r.uniform(0.5, 2, M).astype(np.float32)
    sb = r.uniform(0.5, 2, N).astype(np.float32)
    bias = r.standard_normal(N).astype(np.float32)
    y = oracle.gemm_half(a, b, oracle.HALF_F16, sa, sb, bias=bias)
    s = (sa[:, None] * sb[None, :]).astype(np.float32)
    want = (acc.astype(np.float64) * s.astype(np.float64) + bias.astype(np.float64)).astype(np.float32)
    assert np.array_equal(y, want)
    yb = oracle.gemm_half(a, b, oracle.HALF_F16, sa, sb, bias=bias, out_dtype=oracle.OUT_BF16)
    assert np.array_equal(yb, bf16_bits_np(y))


def test_gemm_half_sequential_order_case(oracle):
    """Products 1, 2^24, -2^24 summed k = 0, 1, 2: 1 + 2^24 rounds to 2^24
    (ties to even), so the sequential fp32 sum is 0 (any order that adds the
    two large products first gives 1).  Pins the oracle's k-ascending order."""
    a = f16_bits(np.array([[1.0, 4096.0, -4096.0]]))
    b = f16_bits(np.array([[1.0, 4096.0, 4096.0]]))
    assert oracle.gemm_half(a, b, oracle.HALF_F16)[0, 0] == 0.0
    a2 = f16_bits(np.array([[4096.0, -4096.0, 1.0]]))
    b2 = f16_bits(np.array([[4096.0, 4096.0, 1.0]]))
    assert oracle.gemm_half(a2, b2, oracle.HALF_F16)[0, 0] == 1.0
