"""GPU parity tests: the HIP kernels, called through the C ABI, against the CPU
oracle on the same seeded inputs.

Bars: int32 accumulators bit-exact; the fp32 and bf16 epilogue outputs
bit-exact against the oracle's canonical epilogue (which is the reference's
float(acc)*fp32(sa*sb) when scales are uniform and there is no bias); FP8 on the
MFMA family within 2e-2 max-norm relative error of the reference's sequential
fp32 sum (and bit-exact on the GENERIC family, which keeps that order).
Every test prints the case it is about to run before touching the GPU.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _lib, ops  # noqa: E402

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(REPO, "flash-kernel-engine_amd", "_build", "test_quantized_gemm_dropin")
NTH = min(16, os.cpu_count() or 1)

OUT_T = {"f32": torch.float32, "bf16": torch.bfloat16, "i32": torch.int32}


def say(*a):
    print("[case]", *a, flush=True)


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def oracle_out(oracle, acc, sa_vec, sb_vec, sa, sb, bias, out):
    code = {"f32": oracle.OUT_F32, "bf16": oracle.OUT_BF16, "i32": oracle.OUT_I32}[out]
    return oracle.w8a8_epilogue(acc, sa_vec, sb_vec, sa, sb, bias, code)


def inputs_i8(oracle, M, N, K, seed, layout="nk", act="uniform"):
    A = (oracle.gen_i8_uniform((M, K), seed) if act == "uniform"
         else oracle.gen_i8_clipped_normal((M, K), seed, 30.0))
    Bnk = oracle.gen_i8_uniform((N, K), seed + 1)
    B = Bnk if layout == "nk" else np.ascontiguousarray(Bnk.T)
    sa = oracle.gen_f32_uniform((M,), seed + 2, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), seed + 3, 0.001, 0.02)
    bias = oracle.gen_f32_normal((N,), seed + 4, 0.0, 0.02)
    return A, B, sa, sb, bias


def gpu_i8(A, B, layout, out, path="auto", sa_vec=None, sb_vec=None, sa=1.0, sb=1.0, bias=None):
    r = ops.w8a8_gemm(dev_t(A), dev_t(B), None if sa_vec is None else dev_t(sa_vec),
                      None if sb_vec is None else dev_t(sb_vec),
                      None if bias is None else dev_t(bias), out_dtype=OUT_T[out],
                      b_layout=layout, sa=sa, sb=sb, path=path)
    torch.cuda.synchronize()
    return host(r)


def assert_same(got, ref, what):
    if got.dtype == np.float32:
        bad = got.view(np.uint32) != ref.view(np.uint32)
    else:
        bad = got != ref
    n = int(bad.sum())
    if n:
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {n} mismatches, first at {tuple(i)}: {got[tuple(i)]} vs {ref[tuple(i)]}")


# ------------------------------------------------------------- reference KAT

def test_kat64_dropin_entry(oracle, dev):
    """The reference test's own case through fke_launch_int8_gemm_dp4a."""
    say("kat64 via fke_launch_int8_gemm_dp4a")
    M = N = K = 64
    A = (np.arange(M * K) % 7 - 3).astype(np.int8).reshape(M, K)
    B = (np.arange(N * K) % 5 - 2).astype(np.int8).reshape(N, K)
    dA, dB = dev_t(A), dev_t(B)
    dC = torch.empty((M, N), dtype=torch.float32, device=dev)
    st = _lib.lib().fke_launch_int8_gemm_dp4a(dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), 0.05, 0.02,
                                              M, N, K, None)
    assert st == 0
    torch.cuda.synchronize()
    assert_same(host(dC), oracle.ref_host_gemm_i8(A, B, 0.05, 0.02), "kat64")


def test_dropin_program_full(dev):
    say("drop-in C++ program (reference test restated on the HIP API)")
    r = subprocess.run([DROPIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


# ------------------------------------------------------------ C1 (the CPU-sized config)

@pytest.mark.parametrize("path", ["auto", "mfma", "generic"])
def test_c1_golden(oracle, dev, path):
    import json
    g = json.load(open(os.path.join(REPO, "tests", "golden", "golden.json")))["c1"]
    say("c1 golden", path)
    M, N, K = g["M"], g["N"], g["K"]
    A = oracle.gen_i8_uniform((M, K), g["seed_A"])
    B = oracle.gen_i8_uniform((N, K), g["seed_B"])
    sa = oracle.gen_f32_uniform((M,), g["seed_sa"], 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), g["seed_sb"], 0.001, 0.02)
    acc = oracle.w8a8_acc(A, B)
    for out in ("i32", "f32", "bf16"):
        got = gpu_i8(A, B, "nk", out, path, sa, sb)
        assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, None, out), f"c1 {path} {out}")
    for m, n, a, _, _ in g["samples"]:
        assert acc[m, n] == a


# ------------------------------------------------------- kernel families x options

# Every MFMA tile, pinned (the dispatcher would pick a small one for shapes
# this size), and the generic kernel, both B layouts.
SMALL_TILES = ["mfma_128x128", "mfma_128x128_ring4", "mfma_128x64_ring4", "mfma_64x64_ring4"]
I8_FAMILIES = ["mfma_256x256"] + SMALL_TILES + ["generic"]


@pytest.mark.parametrize("path", I8_FAMILIES)
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("out", ["f32", "bf16", "i32"])
@pytest.mark.parametrize("opts", ["vec_bias", "scalar"])
def test_i8_families_ragged(oracle, dev, path, layout, out, opts):
    M, N, K = 300, 528, 384  # ragged in M and N against every tile
    say("i8", path, layout, out, opts, (M, N, K))
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 100, layout)
    acc = oracle.w8a8_acc(A, B, oracle.B_NK if layout == "nk" else oracle.B_KN)
    if opts == "vec_bias":
        got = gpu_i8(A, B, layout, out, path, sa, sb, bias=bias)
        ref = oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
    else:
        got = gpu_i8(A, B, layout, out, path, sa=0.05, sb=0.02)
        ref = oracle_out(oracle, acc, None, None, 0.05, 0.02, None, out)
    assert_same(got, ref, f"{path} {layout} {out} {opts}")


@pytest.mark.parametrize("M", list(range(1, 17)))
def test_gemv_every_m(oracle, dev, M):
    N, K = 1000, 1024  # N ragged against every row-block size
    say("gemv", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 200 + M, act="normal")
    acc = oracle.w8a8_acc(A, B)
    assert_same(gpu_i8(A, B, "nk", "i32", "gemv"), acc, f"gemv M={M} i32")
    got = gpu_i8(A, B, "nk", "bf16", "gemv", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"gemv M={M} bf16")


@pytest.mark.parametrize("K", [64, 128, 4096 + 64, 14336])
@pytest.mark.parametrize("M", [1, 3, 9])  # row kernel, sdot split-K kernel, MFMA skinny kernel
def test_gemv_k_variants(oracle, dev, M, K):
    N = 300
    say("gemv K", M, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 300 + K)
    acc = oracle.w8a8_acc(A, B)
    assert_same(gpu_i8(A, B, "nk", "i32", "gemv"), acc, f"gemv K={K}")


# The LDS-streamed decode kernel (3 <= M <= 16, K >= 4096): small N (fewer
# workgroups than CUs), N not a multiple of 16, K with a partial last 1 KiB
# piece, K = 14336 (waves own 4 or 3 pieces), several tile chunks per
# workgroup (N = 20000), every output type, scales as vectors or scalars,
# with and without bias.
STREAM_SHAPES = [(100, 4096), (1000, 4160), (777, 5056), (4096, 14336), (20000, 4096), (129, 8192)]


@pytest.mark.parametrize("shape", STREAM_SHAPES)
@pytest.mark.parametrize("M", [3, 8, 16])
def test_gemv_streamed_shapes(oracle, dev, M, shape):
    N, K = shape
    say("gemv streamed", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 700 + M + N + K, act="normal")
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    assert_same(gpu_i8(A, B, "nk", "i32", "gemv"), acc, f"streamed M={M} {shape} i32")
    got = gpu_i8(A, B, "nk", "bf16", "gemv", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"streamed M={M} {shape} bf16")
    got = gpu_i8(A, B, "nk", "f32", "gemv", sa=0.013, sb=0.007)
    assert_same(got, oracle_out(oracle, acc, None, None, 0.013, 0.007, None, "f32"), f"streamed M={M} {shape} f32")
    got = gpu_i8(A, B, "nk", "f32", "gemv", sa_vec=sa, sb=0.007, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, None, 1.0, 0.007, bias, "f32"), f"streamed M={M} {shape} mixed")


MID_SHAPES = [(100, 4096), (777, 5056), (1000, 2048), (4096, 14336), (129, 8192)]


@pytest.mark.parametrize("shape", MID_SHAPES)
@pytest.mark.parametrize("M", [17, 32, 33, 64, 65, 130, 200])
def test_gemv_streamed_batches(oracle, dev, M, shape):
    """Batches past 16 rows on the LDS-streamed kernel: 2 or 4 activation
    blocks per workgroup, and workgroup rows along y past 64 rows (ragged
    last chunk at 65, 130, 200)."""
    N, K = shape
    say("gemv streamed batch", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 900 + M + N + K, act="normal")
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    assert_same(gpu_i8(A, B, "nk", "i32", "gemv"), acc, f"batch M={M} {shape} i32")
    got = gpu_i8(A, B, "nk", "bf16", "gemv", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"batch M={M} {shape} bf16")
    got = gpu_i8(A, B, "nk", "f32", "gemv", sa=0.013, sb=0.007)
    assert_same(got, oracle_out(oracle, acc, None, None, 0.013, 0.007, None, "f32"), f"batch M={M} {shape} f32")
    got = gpu_i8(A, B, "nk", "f32", "gemv", sa_vec=sa, sb=0.007, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, None, 1.0, 0.007, bias, "f32"), f"batch M={M} {shape} mixed")


@pytest.mark.parametrize("M,N,K", [(512, 300, 2048), (449, 1000, 4096), (257, 70, 14336)])
def test_gemv_streamed_batch_largest(oracle, dev, M, N, K):
    """The largest batches the decode family takes (up to 512 rows: 8 workgroup
    rows of 64 activation rows), ragged last chunks, 512-byte and 1 KiB pieces."""
    say("gemv streamed largest batch", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 950 + M + N + K, act="normal")
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    assert_same(gpu_i8(A, B, "nk", "i32", "gemv"), acc, f"batch M={M} i32")
    got = gpu_i8(A, B, "nk", "bf16", "gemv", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"batch M={M} bf16")


def test_gemv_streamed_more_workgroups_than_cus(oracle, dev):
    """N = 140000 rows: a share would pass 512 rows per CU, so the launch takes
    more workgroups than CUs; sampled columns against the oracle."""
    M, N, K = 5, 140000, 4096
    say("gemv streamed, N > 512 rows per CU", M, N, K)
    g = torch.Generator(device=dev)
    g.manual_seed(4242)
    Bd = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    A = oracle.gen_i8_clipped_normal((M, K), 4243, 30.0)
    sa = oracle.gen_f32_uniform((M,), 4244, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), 4245, 0.001, 0.02)
    bias = oracle.gen_f32_normal((N,), 4246, 0.0, 0.02)
    out = ops.w8a8_gemm(dev_t(A), Bd, dev_t(sa), dev_t(sb), dev_t(bias), out_dtype=torch.float32, path="gemv")
    torch.cuda.synchronize()
    cols = np.concatenate([np.arange(0, 600), np.arange(N // 2 - 300, N // 2 + 300), np.arange(N - 600, N)])
    Bs = Bd[torch.from_numpy(cols).long().cuda()].cpu().numpy()
    acc = oracle.w8a8_acc(A, Bs, nthreads=NTH)
    ref = oracle.w8a8_epilogue(acc, sa, sb[cols], 1.0, 1.0, bias[cols], oracle.OUT_F32)
    assert_same(out[:, torch.from_numpy(cols).long().cuda()].cpu().numpy(), ref, "streamed N=140000")


@pytest.mark.parametrize("shape", [(1, 1, 1), (7, 13, 77), (65, 3, 5), (33, 70, 129), (2, 5, 4)])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_generic_odd_shapes(oracle, dev, shape, layout):
    M, N, K = shape
    say("generic odd", shape, layout)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 400 + sum(shape), layout)
    acc = oracle.w8a8_acc(A, B, oracle.B_NK if layout == "nk" else oracle.B_KN)
    got = gpu_i8(A, B, layout, "f32", "auto", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "f32"), f"generic {shape}")


def test_unaligned_pointers_use_generic(oracle, dev):
    M, N, K = 40, 256, 256
    say("unaligned A")
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 500)
    buf = torch.zeros(M * K + 1, dtype=torch.int8, device=dev)
    buf[1:] = dev_t(A.ravel())
    dA = buf[1:].view(M, K)
    assert dA.data_ptr() % 16 == 1
    assert _lib.lib().fke_select_path_i8(dA.data_ptr(), 4096, 4096, M, N, K, 0, 0) == _lib.PATH_GENERIC
    r = ops.w8a8_gemm(dA, dev_t(B), dev_t(sa), dev_t(sb), None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_same(host(r), oracle_out(oracle, oracle.w8a8_acc(A, B), sa, sb, 1., 1., None, "f32"), "unaligned")


# ------------------------------------------------------ full-size workloads

@pytest.mark.parametrize("M", [1, 4, 16])
def test_c2_decode_full(oracle, dev, M):
    """Decode: M in {1,4,16}, N=14336, K=4096, clipped N(0,30^2) activations,
    per-channel scales, fused bias, bf16 out; checked in full."""
    N, K = 14336, 4096
    say("c2 decode", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 1000 + M, act="normal")
    assert _lib.lib().fke_select_path_i8(4096, 4096, 4096, M, N, K, 1, 0) == _lib.PATH_GEMV
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    got = gpu_i8(A, B, "nk", "bf16", "auto", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"c2 M={M}")


@pytest.mark.parametrize("M", [1, 4, 16])
def test_c2_decode_full_b_kn(oracle, dev, M):
    """C2 with B stored [K,N] (the layout of the reference's Python op and FP8
    launcher): the transposing decode kernel, checked in full."""
    N, K = 14336, 4096
    say("c2 decode B [K,N]", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 1000 + M, layout="kn", act="normal")
    assert _lib.lib().fke_select_path_i8(4096, 4096, 4096, M, N, K, 1, 1) == _lib.PATH_GEMV
    acc = oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH)
    got = gpu_i8(A, B, "kn", "bf16", "auto", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"c2 kn M={M}")


# (M, N, K): one 64-column block and a ragged last block (N % 64 != 0), a K
# that ends in half an item (K % 128 == 64), K below one item per wave (waves
# without items), K = 14336 (28 items per wave), more blocks than CUs, and N
# past 65536 (K splits over several rounds of workgroups: S = 3 with splits of
# 3 / 3 / 2 items, S = 2).  M = 1 runs the row kernel: 1024-column blocks, one
# block with 16 valid columns (32 splits), 56 splits of K = 14336, 17 splits
# of which the last has one 128-row piece (K = 4160), and 81 blocks x 3.
# 17..32 rows: two activation blocks on one-wave workgroups (rows 29..31 of
# the second empty in one) and on two-wave workgroups.
KN_SHAPES = [(1, 16, 4096), (3, 304, 1024), (16, 1040, 192), (5, 4096, 64), (2, 4096, 14336),
             (16, 20016, 2048), (8, 1008, 4160), (1, 82000, 1024), (9, 100000, 512),
             (1, 4096, 14336), (1, 14352, 4160), (17, 14336, 4096), (32, 20016, 2048), (29, 4096, 4096)]


@pytest.mark.parametrize("M,N,K", KN_SHAPES)
@pytest.mark.parametrize("out,opts", [("i32", "none"), ("f32", "vec"), ("bf16", "vec"), ("f32", "scalar")])
def test_gemv_kn_i8_bit_exact(oracle, dev, M, N, K, out, opts):
    """INT8 decode with B [K,N] on the transposing kernel: every output type,
    per-row / per-column scales with bias and scalar scales, bit-exact."""
    say("gemv kn i8", M, N, K, out, opts)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 7000 + M + N + K, layout="kn")
    acc = oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH)
    if out == "i32":
        assert_same(gpu_i8(A, B, "kn", "i32", "gemv"), acc, f"kn i32 {M, N, K}")
    elif opts == "vec":
        got = gpu_i8(A, B, "kn", out, "gemv", sa, sb, bias=bias)
        assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out), f"kn {out} {M, N, K}")
    else:
        got = gpu_i8(A, B, "kn", out, "gemv", sa=0.013, sb=0.021)
        assert_same(got, oracle_out(oracle, acc, None, None, 0.013, 0.021, None, out), f"kn scalar {M, N, K}")


@pytest.mark.parametrize("M,N,K", KN_SHAPES + [(16, 14336, 4096), (1, 14336, 4096)])
@pytest.mark.parametrize("nan_codes", [False, True])
def test_gemv_kn_f8_tolerance(oracle, dev, M, N, K, nan_codes):
    """FP8 decode with B [K,N] (the reference launcher's layout) on the
    transposing kernel: fp32 sums in another order than the reference's
    sequential loop, codes 0x7F / 0xFF counted as 0.0."""
    say("gemv kn f8", M, N, K, nan_codes)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 7500 + M + N + K, "kn", with_nan_codes=nan_codes)
    bias = oracle.gen_f32_normal((N,), 7501 + N, 0.0, 0.02)
    ref = oracle.f8_gemm(A, B, sa, sb, bias=bias, b_layout=oracle.B_KN, nthreads=NTH)
    for out in ("f32", "bf16"):
        got = gpu_f8(A, B, sa, sb, "kn", out, "gemv", bias=bias)
        if out == "bf16":
            got = oracle.bf16_to_f32(got)
        assert_fp8_close(got, ref, out, f"kn {M, N, K} nan={nan_codes}")


def kn_i8_ws(A, B, sa, sb, bias, out, ws, ws_bytes, stream=None, ws_shift=0, c_shift=0):
    """fke_qgemm_i8_ws (B [K,N]) on device inputs, with the caller's workspace
    (ws_shift bytes past its start) and C c_shift elements into a buffer."""
    M, K = A.shape
    N = B.shape[1]
    Cbuf = torch.empty(M * N + c_shift, dtype=OUT_T[out], device=A.device)
    C = Cbuf[c_shift:].view(M, N)
    st = _lib.lib().fke_qgemm_i8_ws(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(),
                                    sb.data_ptr(), 1.0, 1.0, bias.data_ptr(),
                                    {"f32": _lib.OUT_F32, "bf16": _lib.OUT_BF16, "i32": _lib.OUT_I32}[out],
                                    _lib.B_KN, None if ws is None else ws.data_ptr() + ws_shift, ws_bytes,
                                    stream if stream is not None else torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "fke_qgemm_i8_ws")
    return C


@pytest.mark.parametrize("M", [1, 16, 24])
def test_gemv_kn_split_full_and_fewer_splits(oracle, dev, M):
    """C2 with B [K,N] through fke_qgemm_i8_ws: the K-split kernels on a
    workspace of fke_qgemm_workspace_size bytes, on a third of it (fewer
    splits) and on none (the one-kernel full-K decode; past 16 rows the MFMA
    GEMM), every output dtype bit-exact against the oracle."""
    N, K = 14336, 4096
    say("c2 kn split/full", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9100 + M, layout="kn", act="normal")
    acc = oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH)
    need = _lib.lib().fke_qgemm_workspace_size(M, N, K, _lib.B_KN)
    # [M][N] int32 partial sums per split: 16 on the M = 1 row kernel, 2 on the one-wave split
    # workgroups at M = 16 and 24 (past 16 rows a workspace without room for the split, or one
    # not 16-byte aligned, gives the MFMA GEMM)
    assert need == 4 * {1: 16, 16: 2, 24: 2}[M] * M * N
    dA, dB, dsa, dsb, dbias = dev_t(A), dev_t(B), dev_t(sa), dev_t(sb), dev_t(bias)
    for nbytes in (need, need // 3, 0):
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev) if nbytes else None
        for out in ("i32", "f32", "bf16"):
            got = kn_i8_ws(dA, dB, dsa, dsb, dbias, out, ws, nbytes)
            torch.cuda.synchronize()
            assert_same(host(got), oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out),
                        f"kn ws={nbytes} {out} M={M}")
    # an output not aligned for the reduction's vector stores (element stores), and a
    # workspace not 16-byte aligned (run unsplit)
    ws = torch.empty(need + 16, dtype=torch.uint8, device=dev)
    for out in ("f32", "bf16"):
        got = kn_i8_ws(dA, dB, dsa, dsb, dbias, out, ws, need, c_shift=1)
        torch.cuda.synchronize()
        assert_same(host(got), oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out), f"kn C+1 {out} M={M}")
    got = kn_i8_ws(dA, dB, dsa, dsb, dbias, "i32", ws, need, ws_shift=4)
    torch.cuda.synchronize()
    assert_same(host(got), acc, f"kn ws+4 M={M}")


def dev_at(x, shift):
    """A device copy of array x placed `shift` bytes into a uint8 buffer (an
    operand only `shift`-aligned); returns (buffer, pointer)."""
    raw = np.ascontiguousarray(x).view(np.uint8).reshape(-1)
    buf = torch.zeros(raw.size + shift, dtype=torch.uint8, device="cuda")
    buf[shift:].copy_(torch.from_numpy(raw))
    return buf, buf.data_ptr() + shift


# B [K,N] whose N or K is only a multiple of 4, or whose operands are only
# 4-byte aligned: the row kernel's 4-byte form (one split when the plan gives
# one, a ragged last 1024-column block, K not a multiple of 128; past one row,
# workgroups of 2 or 4 activation rows, the last group part empty; past 8
# rows the word kernel takes these shapes).
KN_DW_CASES = [(1, 1000, 4096, 0), (1, 14340, 4096, 0), (1, 4100, 4100, 0), (1, 2052, 100, 0), (1, 14336, 4000, 0),
               (1, 14336, 4096, 4), (1, 1024, 4, 4), (2, 14340, 4096, 0), (3, 4100, 4100, 4), (4, 1000, 4096, 0),
               (5, 2052, 100, 0), (8, 14336, 4096, 4), (6, 14340, 4096, 0), (7, 4100, 1028, 4),
               (8, 14340, 4096, 0)]


@pytest.mark.parametrize("M,N,K,shift", KN_DW_CASES)
def test_gemv_kn_row_kernel_dword_form(oracle, dev, M, N, K, shift):
    """INT8 bit-exact on every output type, and FP8 (0x7F / 0xFF codes
    included) within the bounds of the sequential sum, through fke_qgemm_i8 /
    fke_qgemm_f8 with A and B `shift` bytes past 16-byte alignment."""
    say("kn row kernel, 4-byte loads", M, N, K, shift)
    L = _lib.lib()
    assert L.fke_select_path_i8(4096 + shift, 4096 + shift, 4096, M, N, K, _lib.OUT_BF16, _lib.B_KN) == _lib.PATH_GEMV
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9700 + 31 * M + N + K, layout="kn", act="normal")
    acc = oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH)
    (ba, pa), (bb, pb) = dev_at(A, shift), dev_at(B, shift)
    dsa, dsb, dbias = dev_t(sa), dev_t(sb), dev_t(bias)
    for out in ("i32", "f32", "bf16"):
        C = torch.empty((M, N), dtype=OUT_T[out], device=dev)
        _lib.check(L.fke_qgemm_i8(pa, pb, C.data_ptr(), M, N, K, dsa.data_ptr(), dsb.data_ptr(), 1.0, 1.0,
                                  dbias.data_ptr(), {"f32": _lib.OUT_F32, "bf16": _lib.OUT_BF16, "i32": _lib.OUT_I32}[out],
                                  _lib.B_KN, torch.cuda.current_stream().cuda_stream), "fke_qgemm_i8")
        torch.cuda.synchronize()
        want = acc if out == "i32" else oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
        assert_same(host(C), want, f"kn dword {out} M={M} N={N} K={K} shift={shift}")
    A8, B8, fa, fb = f8_inputs(oracle, M, N, K, 9800 + 31 * M + N + K, "kn", with_nan_codes=True)
    ref = oracle.f8_gemm(A8, B8, fa, fb, b_layout=oracle.B_KN, nthreads=NTH)
    (ba, pa), (bb, pb) = dev_at(A8, shift), dev_at(B8, shift)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.check(L.fke_qgemm_f8(pa, pb, C.data_ptr(), M, N, K, fa, fb, None, _lib.OUT_F32, _lib.B_KN,
                              torch.cuda.current_stream().cuda_stream), "fke_qgemm_f8")
    torch.cuda.synchronize()
    assert_fp8_close(host(C), ref, "f32", f"kn dword fp8 M={M} N={N} K={K} shift={shift}")


def test_gemv_kn_graph_replays(oracle, dev):
    """The split [K,N] decode captured into a HIP graph (on the stream's slot
    of the split pool, and on a caller's workspace): three replays with other
    [K,N] decodes run eagerly between them, each replay bit-exact."""
    M, N, K = 4, 14336, 4096
    say("kn graph replays", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9200, layout="kn", act="normal")
    ref = oracle_out(oracle, oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH), sa, sb, 1.0, 1.0, bias, "bf16")
    A2, B2, sa2, sb2, bias2 = inputs_i8(oracle, M, N, K, 9300, layout="kn", act="normal")
    dA, dB, dsa, dsb, dbias = dev_t(A), dev_t(B), dev_t(sa), dev_t(sb), dev_t(bias)
    d2 = [dev_t(x) for x in (A2, B2, sa2, sb2, bias2)]
    s = torch.cuda.Stream()
    ws = torch.empty(_lib.lib().fke_qgemm_workspace_size(M, N, K, _lib.B_KN), dtype=torch.uint8, device=dev)
    with torch.cuda.stream(s):  # an eager call on the stream first: the capture reuses its slot
        ops.w8a8_gemm(dA, dB, dsa, dsb, dbias, out_dtype=torch.bfloat16, b_layout="kn")
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out_a = ops.w8a8_gemm(dA, dB, dsa, dsb, dbias, out_dtype=torch.bfloat16, b_layout="kn")
        out_b = kn_i8_ws(dA, dB, dsa, dsb, dbias, "bf16", ws, ws.numel(), stream=s.cuda_stream)
    for r in range(3):
        out_a.zero_()
        out_b.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_same(host(out_a), ref, f"replay {r} (stream workspace)")
        assert_same(host(out_b), ref, f"replay {r} (caller workspace)")
        other = ops.w8a8_gemm(*d2[:2], d2[2], d2[3], d2[4], out_dtype=torch.bfloat16, b_layout="kn")
        other2 = kn_i8_ws(*d2, "bf16", ws, ws.numel())
        torch.cuda.synchronize()
        assert torch.equal(other, other2)


def test_graph_replays_every_nk_family(oracle, dev):
    """One HIP graph holding, with B [N,K], the row kernel (M = 1), the
    LDS-streamed decode (M = 16), the MFMA GEMM, its K split (first kernel and
    the kernel that adds the splits, on the stream's pool slot) and the FP8
    decode: three replays with eager calls on other inputs between them, every
    replay checked against the oracle (INT8 bit-exact; FP8 within the FP8 bar
    and bit-identical from replay to replay)."""
    L = _lib.lib()
    tile = ctypes.c_int(0)
    assert L.fke_select_mfma_split(100, 1000, 14720, _lib.B_NK, 0, ctypes.byref(tile)) > 1  # the K split shape
    cases = [(1, 4096, 4096, "bf16"), (16, 4096, 4096, "bf16"), (300, 512, 1024, "f32"), (100, 1000, 14720, "bf16")]
    data, refs, others = [], [], []
    for i, (M, N, K, out) in enumerate(cases):
        say("graph replays", M, N, K, out)
        A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9400 + 10 * i, act="normal")
        refs.append(oracle_out(oracle, oracle.w8a8_acc(A, B, oracle.B_NK, nthreads=NTH), sa, sb, 1.0, 1.0, bias, out))
        data.append([dev_t(x) for x in (A, B, sa, sb, bias)])
        A2, B2, sa2, sb2, bias2 = inputs_i8(oracle, M, N, K, 9405 + 10 * i, act="normal")
        others.append([dev_t(x) for x in (A2, B2, sa2, sb2, bias2)])
    qa, qb, fsa, fsb = f8_inputs(oracle, 8, 2048, 4096, 9480, layout="nk")
    f8_ref = oracle.f8_gemm(qa, qb, fsa, fsb, None, oracle.OUT_F32, oracle.B_NK, nthreads=NTH)
    dqa, dqb = dev_t(qa), dev_t(qb)

    def run_all(ins):
        outs = [ops.w8a8_gemm(*d[:2], d[2], d[3], d[4], out_dtype=OUT_T[c[3]]) for d, c in zip(ins, cases)]
        outs.append(ops.fp8_gemm_scaled(dqa, dqb, fsa, fsb, None, out_dtype=torch.float32, b_layout="nk"))
        return outs

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):  # eager first: the stream takes its pool slot, the capture reuses it
        run_all(data)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = run_all(data)
    f8_first = None
    for r in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, ref, c in zip(outs, refs, cases):
            assert_same(host(o), ref, f"replay {r} {c}")
        f8 = host(outs[-1])
        assert_fp8_close(f8, f8_ref, "f32", f"replay {r} fp8 decode")
        if f8_first is None:
            f8_first = f8
        assert np.array_equal(f8.view(np.uint32), f8_first.view(np.uint32)), f"replay {r}: fp8 bits changed"
        eager = run_all(others)  # other inputs, eagerly, on the current stream
        torch.cuda.synchronize()
        again = run_all(others)
        torch.cuda.synchronize()
        for a, b in zip(eager[:-1], again[:-1]):
            assert torch.equal(a, b)


def test_gemv_kn_two_streams(oracle, dev):
    """[K,N] decodes of different inputs on two streams at once, each on its
    stream's slot of the split pool: both bit-exact."""
    M, N, K = 8, 14336, 4096
    say("kn two streams", M, N, K)
    ins = [inputs_i8(oracle, M, N, K, 9400 + 10 * i, layout="kn", act="normal") for i in range(2)]
    refs = [oracle_out(oracle, oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH), sa, sb, 1.0, 1.0, bias, "bf16")
            for A, B, sa, sb, bias in ins]
    dins = [[dev_t(x) for x in t] for t in ins]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[], []]
    for _ in range(20):
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                A, B, sa, sb, bias = dins[i]
                outs[i].append(ops.w8a8_gemm(A, B, sa, sb, bias, out_dtype=torch.bfloat16, b_layout="kn"))
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert_same(host(o), refs[i], f"stream {i}")


def test_host_threads_each_on_own_stream(oracle, dev):
    """Four host threads call the library at once, each on a stream of its own
    (the C ABI is stateless apart from the stream-to-slot table of the split
    pool, filled on a stream's first split call under a mutex, and ctypes
    releases the GIL around each call): per thread, the [K,N] INT8
    decode, the [N,K] MFMA GEMM and the [K,N] FP8 decode, twelve times over.
    INT8 results bit-exact against the oracle; FP8 results bit-identical to
    the same call made alone before the threads start (and that one within
    the FP8 bar)."""
    import threading

    T, ITERS = 4, 12
    cases = []
    for t in range(T):
        M, N, K = 1 + 5 * t, 4096, 2048  # M = 1, 6, 11, 16
        A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9700 + 10 * t, layout="kn", act="normal")
        ref_kn = oracle_out(oracle, oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH), sa, sb, 1.0, 1.0, bias, "bf16")
        M2, N2, K2 = 256 + 64 * t, 1024, 1024
        A2, B2, sa2, sb2, bias2 = inputs_i8(oracle, M2, N2, K2, 9800 + 10 * t)
        ref_nk = oracle_out(oracle, oracle.w8a8_acc(A2, B2, nthreads=NTH), sa2, sb2, 1.0, 1.0, bias2, "f32")
        A3, B3, s3a, s3b = f8_inputs(oracle, M, N, K, 9900 + 10 * t, "kn")
        ref_f8 = oracle.f8_gemm(A3, B3, s3a, s3b, b_layout=oracle.B_KN, nthreads=NTH)
        cases.append(dict(kn=[dev_t(x) for x in (A, B, sa, sb, bias)], ref_kn=ref_kn,
                          nk=[dev_t(x) for x in (A2, B2, sa2, sb2, bias2)], ref_nk=ref_nk,
                          f8=(dev_t(A3), dev_t(B3), float(s3a), float(s3b)), ref_f8=ref_f8))
    say("host threads", T, "x", ITERS, "iterations")
    solo = []
    for c in cases:  # FP8 references: the same calls, one at a time
        A3, B3, s3a, s3b = c["f8"]
        r = ops.fp8_gemm_scaled(A3, B3, s3a, s3b, out_dtype=torch.float32, b_layout="kn")
        torch.cuda.synchronize()
        assert_fp8_close(host(r), c["ref_f8"], "f32", "threads: solo fp8 kn")
        solo.append(host(r))

    errors = []
    start = threading.Barrier(T)

    def work(t):
        try:
            c = cases[t]
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                start.wait(timeout=60)
                for i in range(ITERS):
                    y1 = ops.w8a8_gemm(*c["kn"], out_dtype=torch.bfloat16, b_layout="kn")
                    y2 = ops.w8a8_gemm(*c["nk"], out_dtype=torch.float32, b_layout="nk")
                    A3, B3, s3a, s3b = c["f8"]
                    y3 = ops.fp8_gemm_scaled(A3, B3, s3a, s3b, out_dtype=torch.float32, b_layout="kn")
                    s.synchronize()
                    assert_same(host(y1), c["ref_kn"], f"thread {t} iteration {i}: i8 kn")
                    assert_same(host(y2), c["ref_nk"], f"thread {t} iteration {i}: i8 nk")
                    assert_same(host(y3), solo[t], f"thread {t} iteration {i}: f8 kn against the solo call")
        except BaseException as e:  # reported below, from the test's own thread
            errors.append((t, repr(e)))

    threads = [threading.Thread(target=work, args=(t,)) for t in range(T)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a host thread did not finish"
    assert not errors, errors


@pytest.mark.parametrize("M", [1, 16])
def test_gemv_kn_f8_split_deterministic(oracle, dev, M):
    """FP8 decode with B [K,N] at the C2 shape on the K-split kernels and on
    the full-K kernel (no workspace): each within the FP8 bars of the
    reference's sequential sum, and each bit-identical from call to call (the
    splits are added in a fixed order)."""
    N, K = 14336, 4096
    say("kn f8 split determinism", M, N, K)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 9500 + M, "kn")
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_KN, nthreads=NTH)
    dA, dB = dev_t(A), dev_t(B)
    need = _lib.lib().fke_qgemm_workspace_size(M, N, K, _lib.B_KN)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    for wsp, nbytes in ((ws, need), (None, 0)):
        runs = []
        for _ in range(2):
            C = torch.empty((M, N), dtype=torch.float32, device=dev)
            st = _lib.lib().fke_qgemm_f8_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, sa, sb, None,
                                            _lib.OUT_F32, _lib.B_KN, None if wsp is None else wsp.data_ptr(),
                                            nbytes, torch.cuda.current_stream().cuda_stream)
            _lib.check(st, "fke_qgemm_f8_ws")
            torch.cuda.synchronize()
            runs.append(host(C))
        assert_same(runs[1], runs[0], f"fp8 kn ws={nbytes} run to run")
        assert_fp8_close(runs[0], ref, "f32", f"kn ws={nbytes} M={M}")


@pytest.mark.parametrize("M", [1, 7, 16])
def test_fp8_dropin_launcher_decode(oracle, dev, M):
    """The drop-in fke_launch_fp8_gemm_scaled (B [K,N], fp32 out, alpha =
    sa*sb; src/quantized_gemm.cu:120-139) at decode shapes, against the
    reference's own sequential loop."""
    N, K = 2048, 4096
    say("fp8 drop-in decode", M, N, K)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 7600 + M, "kn", with_nan_codes=True)
    ref = oracle.ref_kernel_gemm_f8(A, B, sa, sb)
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    dA, dB = dev_t(A), dev_t(B)  # held: a temporary's memory could be reused for the next operand
    st = _lib.lib().fke_launch_fp8_gemm_scaled(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), sa, sb,
                                               M, N, K, None)
    _lib.check(st, "fke_launch_fp8_gemm_scaled")
    torch.cuda.synchronize()
    assert_fp8_close(C.cpu().numpy(), ref, "f32", f"drop-in M={M}")


def test_fp8_dropin_launcher_batch_on_the_split_decode(oracle, dev):
    """The drop-in fke_launch_fp8_gemm_scaled (B [K,N]) with a 24-row batch at
    the decode weights' shape, which the dispatcher gives to the [K,N] split
    decode (two activation blocks per item), against the reference's
    sequential sum (the threaded restatement), 0x7F / 0xFF codes included."""
    M, N, K = 24, 14336, 4096
    say("fp8 drop-in batch", M, N, K)
    L = _lib.lib()
    assert L.fke_select_path_f8(4096, 4096, 4096, M, N, K, _lib.OUT_F32, _lib.B_KN) == _lib.PATH_GEMV
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 7700, "kn", with_nan_codes=True)
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_KN, nthreads=NTH)  # the sequential sum, threaded
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    dA, dB = dev_t(A), dev_t(B)  # held: a temporary's memory could be reused for the next operand
    _lib.check(L.fke_launch_fp8_gemm_scaled(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), sa, sb, M, N, K,
                                            None), "fke_launch_fp8_gemm_scaled")
    torch.cuda.synchronize()
    assert_fp8_close(C.cpu().numpy(), ref, "f32", f"drop-in batch M={M}")


@pytest.mark.parametrize("M,N,K,want", [(1, 1000, 100, "gemv"), (7, 4100, 1028, "gemv"), (64, 1000, 100, "mfma"),
                                        (300, 4100, 4100, "mfma"), (37, 50, 131, "generic")])
def test_fp8_dropin_launcher_odd_shapes(oracle, dev, M, N, K, want):
    """The drop-in fke_launch_fp8_gemm_scaled (B [K,N]: the reference
    launcher, which takes any shape) where N or K is only a multiple of 4
    (the [K,N] decode's 4-byte form up to 8 rows, the word kernel above) or
    neither (the generic kernel), against the reference's sequential sum with
    0x7F / 0xFF codes."""
    say("fp8 drop-in odd shape", M, N, K, want)
    L = _lib.lib()
    path = {"gemv": _lib.PATH_GEMV, "mfma": _lib.PATH_MFMA, "generic": _lib.PATH_GENERIC}[want]
    assert L.fke_select_path_f8(4096, 4096, 4096, M, N, K, _lib.OUT_F32, _lib.B_KN) == path
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 7800 + M + N + K, "kn", with_nan_codes=True)
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_KN, nthreads=NTH)
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    dA, dB = dev_t(A), dev_t(B)  # held: a temporary's memory could be reused for the next operand
    _lib.check(L.fke_launch_fp8_gemm_scaled(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), sa, sb, M, N, K,
                                            None), "fke_launch_fp8_gemm_scaled")
    torch.cuda.synchronize()
    if want == "generic":  # the reference's own order: the same bits
        assert np.array_equal(C.cpu().numpy().view(np.uint32), ref.view(np.uint32)), "generic FP8 not bit-exact"
    else:
        assert_fp8_close(C.cpu().numpy(), ref, "f32", f"drop-in odd M={M} N={N} K={K}")


@pytest.mark.parametrize("M", list(range(1, 17)))
def test_gemv_dot_family_bit_exact(oracle, dev, M):
    """The VALU dot-product decode kernels (row kernel for M <= 4, split-K sdot
    kernel above; FKE_PATH_GEMV_DOT) at every M up to 16: bit-exact, and equal
    to the dispatcher's (MFMA) choice."""
    N, K = 1000, 4096
    say("gemv dot family", M, N, K)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 7800 + M, act="normal")
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    got = gpu_i8(A, B, "nk", "bf16", "gemv_dot", sa, sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"dot M={M}")
    assert_same(gpu_i8(A, B, "nk", "i32", "gemv_dot"), acc, f"dot i32 M={M}")
    assert_same(got, gpu_i8(A, B, "nk", "bf16", "auto", sa, sb, bias=bias), f"dot vs auto M={M}")


@pytest.mark.parametrize("M", [6, 9])
def test_decode_weight_past_2gib(oracle, dev, M):
    """A 2.1 GB weight (N*K > 2^31): the skinny MFMA kernel's 32-bit offsets do
    not reach, so 5 <= M <= 16 runs the split-K sdot kernel (64-bit row bases).
    The weight is generated on the device; sampled output columns (both ends and
    the middle) are checked against the oracle on host copies of those rows."""
    N, K = (1 << 31) // 4096 + 64, 4096
    say("decode weight past 2 GiB", M, N, K)
    assert _lib.lib().fke_select_path_i8(4096, 4096, 4096, M, N, K, 1, 0) == _lib.PATH_GEMV
    g = torch.Generator(device=dev)
    g.manual_seed(77 + M)
    Bd = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    A = oracle.gen_i8_clipped_normal((M, K), 500 + M, 30.0)
    sa = oracle.gen_f32_uniform((M,), 501, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), 502, 0.001, 0.02)
    bias = oracle.gen_f32_normal((N,), 503, 0.0, 0.02)
    out = ops.w8a8_gemm(dev_t(A), Bd, dev_t(sa), dev_t(sb), dev_t(bias), out_dtype=torch.float32, path="gemv")
    torch.cuda.synchronize()
    cols = np.concatenate([np.arange(0, 64), np.arange(N // 2, N // 2 + 64), np.arange(N - 64, N)])
    Bs = Bd[torch.from_numpy(cols).long().cuda()].cpu().numpy()
    del Bd
    acc = oracle.w8a8_acc(A, Bs, nthreads=NTH)
    ref = oracle.w8a8_epilogue(acc, sa, sb[cols], 1.0, 1.0, bias[cols], oracle.OUT_F32)
    got = out[:, torch.from_numpy(cols).long().cuda()].cpu().numpy()
    assert_same(got, ref, f"decode past 2 GiB M={M}")


def _sampled_rows_check(oracle, A_dev, B_dev, sa, sb, rows, what):
    """Oracle check of the listed output rows of C = A . B^T (B [N,K] on the device)."""
    out = ops.w8a8_gemm(A_dev, B_dev, dev_t(sa), dev_t(sb), None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    Ah = A_dev[torch.from_numpy(rows).long().cuda()].cpu().numpy()
    acc = oracle.w8a8_acc(Ah, B_dev.cpu().numpy(), nthreads=NTH)
    ref = oracle.w8a8_epilogue(acc, sa[rows], sb, 1.0, 1.0, None, oracle.OUT_F32)
    assert_same(out[torch.from_numpy(rows).long().cuda()].cpu().numpy(), ref, what)


def test_mfma_largest_activation_panel(oracle, dev):
    """M*K = 2^31 - 8192, the largest A the MFMA kernel's 32-bit offsets take
    (2 GiB of activations): first, middle and last rows against the oracle."""
    M, N, K = (1 << 31) // 8192 - 1, 256, 8192
    say("mfma largest A", M, N, K)
    L = _lib.lib()
    assert L.fke_select_path_i8(4096, 4096, 4096, M, N, K, 0, 0) == _lib.PATH_MFMA
    assert L.fke_select_path_i8(4096, 4096, 4096, M + 2, N, K, 0, 0) == _lib.PATH_GENERIC
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    B = dev_t(oracle.gen_i8_uniform((N, K), 6))
    sa = oracle.gen_f32_uniform((M,), 7, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), 8, 0.001, 0.02)
    rows = np.array([0, 1, 255, 256, M // 2, M - 257, M - 2, M - 1], dtype=np.int32)
    _sampled_rows_check(oracle, A, B, sa, sb, rows, "largest A panel")


def test_generic_past_the_mfma_offsets(oracle, dev):
    """M*K just above 2^31: the dispatcher sends it to the generic kernel
    (64-bit indexing), which must give the same exact results."""
    M, N, K = (1 << 31) // 8192 + 1, 64, 8192
    say("generic past the MFMA offsets", M, N, K)
    assert _lib.lib().fke_select_path_i8(4096, 4096, 4096, M, N, K, 0, 0) == _lib.PATH_GENERIC
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    B = dev_t(oracle.gen_i8_uniform((N, K), 10))
    sa = oracle.gen_f32_uniform((M,), 11, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), 12, 0.001, 0.02)
    rows = np.array([0, 63, 64, M // 2, M - 65, M - 1], dtype=np.int32)
    _sampled_rows_check(oracle, A, B, sa, sb, rows, "generic past 2^31")


def test_mfma_largest_weight_panel(oracle, dev):
    """N*K = 2^31 - 8192 (2 GiB of weights, B [N,K]): sampled output columns
    against the oracle on host copies of those weight rows."""
    M, N, K = 300, (1 << 31) // 8192 - 1, 8192
    say("mfma largest B", M, N, K)
    assert _lib.lib().fke_select_path_i8(4096, 4096, 4096, M, N, K, 0, 0) == _lib.PATH_MFMA
    g = torch.Generator(device=dev)
    g.manual_seed(13)
    Bd = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    A = oracle.gen_i8_uniform((M, K), 14)
    sa = oracle.gen_f32_uniform((M,), 15, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), 16, 0.001, 0.02)
    out = ops.w8a8_gemm(dev_t(A), Bd, dev_t(sa), dev_t(sb), None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    cols = np.array([0, 1, 255, 256, N // 2, N - 257, N - 2, N - 1])
    Bs = Bd[torch.from_numpy(cols).long().cuda()].cpu().numpy()
    del Bd
    acc = oracle.w8a8_acc(A, Bs, nthreads=NTH)
    ref = oracle.w8a8_epilogue(acc, sa, sb[cols], 1.0, 1.0, None, oracle.OUT_F32)
    assert_same(out[:, torch.from_numpy(cols).long().cuda()].cpu().numpy(), ref, "largest B panel")


def test_c3_prefill_full(oracle, dev):
    """Prefill: 4096x11008x4096, bf16 out: every output checked."""
    M, N, K = 4096, 11008, 4096
    say("c3 prefill", M, N, K)
    A, B, sa, sb, _ = inputs_i8(oracle, M, N, K, 2000)
    acc_ref = oracle.w8a8_acc(A, B, nthreads=NTH)
    got = gpu_i8(A, B, "nk", "bf16", "auto", sa, sb)
    assert_same(got, oracle_out(oracle, acc_ref, sa, sb, 1.0, 1.0, None, "bf16"), "c3 bf16")


def test_c4_square_full(oracle, dev):
    """Config 3: 8192^3; the i32 result bit-exact in full against the oracle,
    the fp32 output bit-exact against the epilogue of that i32, plus exact
    int64 row/column checksums (a size-independent property)."""
    M = N = K = 8192
    say("c4 square", M, N, K)
    A, B, sa, sb, _ = inputs_i8(oracle, M, N, K, 3000)
    acc = gpu_i8(A, B, "nk", "i32", "auto")
    colsum = acc.astype(np.int64).sum(0)
    rowsum = acc.astype(np.int64).sum(1)
    assert np.array_equal(colsum, B.astype(np.int64) @ A.astype(np.int64).sum(0))
    assert np.array_equal(rowsum, A.astype(np.int64) @ B.astype(np.int64).sum(0))
    acc_ref = oracle.w8a8_acc(A, B, nthreads=NTH)
    assert_same(acc, acc_ref, "c4 i32")
    f32 = gpu_i8(A, B, "nk", "f32", "auto", sa, sb)
    assert_same(f32, oracle_out(oracle, acc_ref, sa, sb, 1.0, 1.0, None, "f32"), "c4 f32")


@pytest.mark.parametrize("tile", SMALL_TILES + ["mfma_256x256"])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("shape", [(1, 1, 128), (129, 65, 256), (256, 128, 128), (257, 129, 640),
                                   (513, 1000, 1152), (64, 4000, 256), (100, 300, 384), (130, 200, 512),
                                   (300, 2000, 1664)])
def test_mfma_tiles_ragged_shapes(oracle, dev, tile, layout, shape):
    """Every tile against the oracle, bit-exact, on shapes ragged in M and N
    against each tile (and exactly one 128x128 tile), K of 1 to 13 stages
    (every remainder of the 4-stage ring's unrolling), both B layouts, every
    output type, per-row / per-column scales with bias."""
    M, N, K = shape
    if layout == "kn":  # the MFMA kernel takes B [K,N] with N % 16 == 0
        N = max(16, (N + 15) // 16 * 16)
    say("i8 small tile", tile, layout, (M, N, K))
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 900 + M + N, layout, act="normal")
    acc = oracle.w8a8_acc(A, B, oracle.B_NK if layout == "nk" else oracle.B_KN)
    for out in ("i32", "f32", "bf16"):
        got = gpu_i8(A, B, layout, out, tile, sa, sb, bias=bias)
        assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out), f"{tile} {layout} {(M, N, K)} {out}")


@pytest.mark.parametrize("M,N,K,layout,want", [
    (48, 33024, 1024, "nk", _lib.PATH_MFMA_64x64_RING4),    # 516 tiles of 64x64: three rounds, one tile row
    (64, 65536, 512, "kn", _lib.PATH_MFMA_64x64_RING4),     # 1024 tiles, B [K,N]
    (100, 70000, 512, "nk", _lib.PATH_MFMA_128x128),        # 547 of 128x128, ragged rows and columns
])
def test_single_tile_row_many_rounds(oracle, dev, M, N, K, layout, want):
    """One row of tiles with more tiles than CUs (decode batches against a large
    N): the dispatcher's tile (several rounds per workgroup, B copied
    non-temporally), int32 and bf16 outputs bit-exact against the oracle."""
    say("single tile row", M, N, K, layout)
    code = _lib.B_KN if layout == "kn" else _lib.B_NK
    assert _lib.lib().fke_select_mfma_tile(M, N, K, code, 0, 0) == want
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 13000 + M, layout=layout)
    acc = oracle.w8a8_acc(A, B, oracle.B_KN if layout == "kn" else oracle.B_NK, nthreads=NTH)
    assert_same(gpu_i8(A, B, layout, "i32", path="mfma"), acc, f"single row {(M, N, K)} i32")
    got = gpu_i8(A, B, layout, "bf16", path="mfma", sa_vec=sa, sb_vec=sb, bias=bias)
    assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16"), f"single row {(M, N, K)} bf16")


@pytest.mark.parametrize("M,N,K,out,want", [
    (4096, 1376, 4096, "bf16", _lib.PATH_MFMA_128x128),   # 8-way column shard of 11008
    (8192, 1024, 8192, "f32", _lib.PATH_MFMA_128x128),    # 8-way column shard of 8192
    (512, 4096, 4096, "bf16", _lib.PATH_MFMA_128x64_RING4),   # a short prefill: one tile per CU at most
    (128, 14336, 4096, "bf16", _lib.PATH_MFMA_128x64_RING4),  # a decode batch of 128 rows
    (64, 14336, 4096, "bf16", _lib.PATH_MFMA_64x64_RING4),    # a decode batch of 64 rows
    (500, 1792, 4096, "f32", _lib.PATH_MFMA_64x64_RING4),     # ragged rows, 224 tiles
    (2048, 1376, 4096, "f32", _lib.PATH_MFMA_128x128_RING4),  # 176 tiles
])
def test_mfma_few_tile_shapes_full(oracle, dev, M, N, K, out, want):
    """Shapes the dispatcher gives a smaller tile (fewer 256x256 tiles than
    CUs): the tile it picks on this GPU, every output against the oracle, and
    the same outputs from every pinned tile with B in either layout (and from
    the streamed decode kernel where it takes the shape)."""
    L = _lib.lib()
    pick = L.fke_select_mfma_tile(M, N, K, 0, 0, 0)
    say("few-tile shape", M, N, K, out, "tile path", pick)
    assert L.fke_select_mfma_tile(M, N, K, 0, 0, 256) == want
    assert torch.cuda.get_device_properties(0).multi_processor_count != 256 or pick == want
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 4000 + N)
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    ref = oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
    got = gpu_i8(A, B, "nk", out, "auto", sa, sb, bias=bias)
    assert_same(got, ref, f"auto {M}x{N}x{K}")
    for tile in ["mfma_256x256"] + SMALL_TILES:
        assert_same(gpu_i8(A, B, "nk", out, tile, sa, sb, bias=bias), ref, f"{tile} {M}x{N}x{K}")
    Bkn = np.ascontiguousarray(B.T)
    assert L.fke_select_mfma_tile(M, N, K, 1, 0, 256) == want  # the same rule for B [K,N]
    for tile in ["auto", "mfma_256x256"] + SMALL_TILES:
        assert_same(gpu_i8(A, Bkn, "kn", out, tile, sa, sb, bias=bias), ref, f"B [K,N] {tile} {M}x{N}x{K}")
    if M <= 512:  # the streamed decode kernel gives the same bits
        assert_same(gpu_i8(A, B, "nk", out, "gemv", sa, sb, bias=bias), ref, f"gemv {M}x{N}x{K}")


# K % 128 != 0 on the MFMA GEMM (K a multiple of 16): the last stage is
# partial and its chunks past K are cleared in LDS.  One and several stages,
# ragged M and N, both layouts.
PARTIAL_K_SHAPES = [(129, 65, 16), (257, 129, 144), (64, 4000, 2880), (300, 520, 4160), (513, 1040, 1040)]


@pytest.mark.parametrize("tile", SMALL_TILES + ["mfma_256x256", "mfma"])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("shape", PARTIAL_K_SHAPES)
def test_mfma_partial_last_stage_i8(oracle, dev, tile, layout, shape):
    """INT8 with K % 128 != 0 on every MFMA tile: int32, fp32 and bf16
    outputs bit-exact against the oracle."""
    M, N, K = shape
    if layout == "kn":
        N = (N + 15) // 16 * 16
    say("i8 partial last stage", tile, layout, (M, N, K))
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 17000 + K, layout, act="normal")
    acc = oracle.w8a8_acc(A, B, oracle.B_NK if layout == "nk" else oracle.B_KN, nthreads=NTH)
    for out in ("i32", "f32", "bf16"):
        got = gpu_i8(A, B, layout, out, tile, sa, sb, bias=bias)
        assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out), f"{tile} {layout} {(M, N, K)} {out}")


@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("shape", PARTIAL_K_SHAPES)
def test_mfma_partial_last_stage_fp8(oracle, dev, layout, shape):
    """FP8 with K % 128 != 0 (0x7F / 0xFF codes included): every pinned tile
    gives the same bits (they sum K in the same stages and steps), within the
    FP8 bars of the reference's sequential sum, as is the dispatcher's choice
    (which may split K, and so add in another order)."""
    M, N, K = shape
    if layout == "kn":
        N = (N + 15) // 16 * 16
    say("f8 partial last stage", layout, (M, N, K))
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 17500 + K, layout, with_nan_codes=True)
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_KN if layout == "kn" else oracle.B_NK, nthreads=NTH)
    first = gpu_f8(A, B, sa, sb, layout, "f32", "mfma_256x256")
    assert_fp8_close(first, ref, "f32", f"partial stage {layout} {(M, N, K)}")
    for tile in SMALL_TILES:
        assert_same(gpu_f8(A, B, sa, sb, layout, "f32", tile), first, f"{tile} {layout} {(M, N, K)}")
    assert_fp8_close(gpu_f8(A, B, sa, sb, layout, "f32", "mfma"), ref, "f32", f"auto {layout} {(M, N, K)}")


@pytest.mark.parametrize("M,N,K,layout", [(64, 4096, 14352, "nk"), (100, 1000, 14736, "nk"),
                                          (200, 2000, 8208, "kn")])
def test_mfma_k_split_partial_last_stage(oracle, dev, M, N, K, layout):
    """A K split whose last split ends in the partial stage: int32 and bf16
    bit-exact against the oracle; FP8 within its bars and the same bits on
    every call."""
    S, tile = mfma_split_of(M, N, K, layout)
    say("mfma k split, partial last stage", M, N, K, layout, "splits", S)
    assert S > 1
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 17800 + M, layout=layout)
    acc = oracle.w8a8_acc(A, B, oracle.B_KN if layout == "kn" else oracle.B_NK, nthreads=NTH)
    assert_same(gpu_i8(A, B, layout, "i32", path="mfma"), acc, f"split {(M, N, K)} i32")
    ref = oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16")
    assert_same(gpu_i8(A, B, layout, "bf16", "mfma", sa, sb, bias=bias), ref, f"split {(M, N, K)} bf16")
    A8, B8, s8a, s8b = f8_inputs(oracle, M, N, K, 17900 + M, layout, with_nan_codes=True)
    ref8 = oracle.f8_gemm(A8, B8, s8a, s8b, b_layout=oracle.B_KN if layout == "kn" else oracle.B_NK, nthreads=NTH)
    got8 = gpu_f8(A8, B8, s8a, s8b, layout, "f32", "mfma")
    assert_fp8_close(got8, ref8, "f32", f"split fp8 {(M, N, K)}")
    assert_same(gpu_f8(A8, B8, s8a, s8b, layout, "f32", "mfma"), got8, "split fp8 repeat")


@pytest.mark.parametrize("path", ["mfma", "gemv", "generic"])
def test_bf16_rounding_of_epilogue_values(oracle, dev, path):
    """The bf16 output's rounding on chosen fp32 values: with A all zero the
    epilogue value is fmaf(0, s, bias[n]) = bias[n] exactly, so the bias
    carries the patterns (halfway cases of both parities, values just off
    them, fp32 denormals and the largest finite values, both signs, and 4096
    random finite patterns); every output equals the oracle's round to
    nearest even, bit for bit, on each kernel family."""
    r = np.random.default_rng(21)
    pats = []
    for hi in (0x3F80, 0x3F81, 0x4B7F, 0x0001, 0x007F, 0x7F7F, 0x0080):
        for lo in (0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF):
            pats.append((hi << 16) | lo)
    pats += [1, 2, 0x7FFFFF, 0x7F7FFFFF, 0x00800000]
    pats = np.array(pats, dtype=np.uint32)
    pats = np.concatenate([pats, pats | 0x80000000])
    rnd = r.integers(0, 2**32, 4096, dtype=np.uint64).astype(np.uint32)
    rnd = rnd[(rnd & 0x7F800000) != 0x7F800000]  # finite
    bias = np.concatenate([pats, rnd]).view(np.float32)
    M, K = (4, 4096) if path == "gemv" else (40, 512)
    N = (bias.size + 15) // 16 * 16
    bias = np.concatenate([bias, np.zeros(N - bias.size, np.float32)])
    say("bf16 rounding", path, M, N, K)
    A = np.zeros((M, K), np.int8)
    B = oracle.gen_i8_uniform((N, K), 22)
    sa = oracle.gen_f32_uniform((M,), 23, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), 24, 0.001, 0.02)
    acc = np.zeros((M, N), np.int32)
    ref = oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16")
    assert_same(gpu_i8(A, B, "nk", "bf16", path, sa, sb, bias=bias), ref, f"bf16 rounding {path}")


def mfma_split_of(M, N, K, layout):
    t = ctypes.c_int(0)
    S = _lib.lib().fke_select_mfma_split(M, N, K, _lib.B_KN if layout == "kn" else _lib.B_NK, 256,
                                         ctypes.byref(t))
    return S, t.value


# The automatic MFMA path splits K on these (checked on 256 CUs): a few output
# tiles with a long K, a split count that does not divide the stages, ragged
# rows and columns, and both B layouts.
SPLIT_CASES = [
    (64, 4096, 14336, "nk"),    # 64 tiles of 64x64, 4 splits of 28 stages
    (100, 1000, 14720, "nk"),   # 32 tiles of 64x64, 7 splits: 6 of 17 stages and one of 13
    (200, 2000, 8192, "kn"),    # B [K,N], 64 tiles of 128x64, 4 splits
    (120, 2000, 28672, "nk"),   # ragged rows and columns, 32 tiles of 128x64, 8 splits
    (256, 2048, 28672, "nk"),   # 32 tiles of 128x128 over two tile rows, 7 splits
]


@pytest.mark.parametrize("M,N,K,layout", SPLIT_CASES)
def test_mfma_k_split_int8_exact(oracle, dev, M, N, K, layout):
    """The K split of the MFMA GEMM (the split items' int32 partial sums added
    in split order, then the epilogue): int32, bf16 and f32 outputs bit-exact
    against the oracle, and equal to the unsplit kernel on the same tile."""
    S, tile = mfma_split_of(M, N, K, layout)
    say("mfma k split", M, N, K, layout, "splits", S, "tile path", tile)
    assert S > 1
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 14000 + M, layout=layout)
    acc = oracle.w8a8_acc(A, B, oracle.B_KN if layout == "kn" else oracle.B_NK, nthreads=NTH)
    assert_same(gpu_i8(A, B, layout, "i32", path="mfma"), acc, f"split {(M, N, K)} i32")
    for out in ("bf16", "f32"):
        ref = oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
        assert_same(gpu_i8(A, B, layout, out, path="mfma", sa_vec=sa, sb_vec=sb, bias=bias), ref,
                    f"split {(M, N, K)} {out}")
    name = {_lib.PATH_MFMA_64x64_RING4: "mfma_64x64_ring4", _lib.PATH_MFMA_128x64_RING4: "mfma_128x64_ring4",
            _lib.PATH_MFMA_128x128_RING4: "mfma_128x128_ring4"}[tile]
    ref = oracle_out(oracle, acc, None, None, 0.5, 0.25, None, "f32")
    assert_same(gpu_i8(A, B, layout, "f32", path=name, sa=0.5, sb=0.25), ref, f"unsplit {name} {(M, N, K)}")
    assert_same(gpu_i8(A, B, layout, "f32", path="mfma", sa=0.5, sb=0.25), ref, f"split scalar scales {(M, N, K)}")


def test_mfma_k_split_workspace(oracle, dev):
    """fke_qgemm_i8_ws on a split shape: the caller's workspace when it holds the
    partial sums (fke_qgemm_workspace_size bytes), unsplit when it is too small,
    NULL or unaligned; every result bit-exact."""
    M, N, K = 64, 4096, 14336
    S, _ = mfma_split_of(M, N, K, "nk")
    need = _lib.lib().fke_qgemm_workspace_size(M, N, K, _lib.B_NK)
    say("mfma k split workspace", S, need)
    assert S > 1 and need == S * M * N * 4
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 15000)
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    ref = oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, "bf16")
    Ad, Bd, sad, sbd, biasd = dev_t(A), dev_t(B), dev_t(sa), dev_t(sb), dev_t(bias)
    ws = torch.empty(need + 64, dtype=torch.uint8, device=dev)
    for ptr, nbytes in ((ws.data_ptr(), need), (ws.data_ptr(), need - 4), (None, 0), (ws.data_ptr() + 4, need)):
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        st = _lib.lib().fke_qgemm_i8_ws(Ad.data_ptr(), Bd.data_ptr(), C.data_ptr(), M, N, K, sad.data_ptr(),
                                        sbd.data_ptr(), 1.0, 1.0, biasd.data_ptr(), _lib.OUT_BF16, _lib.B_NK,
                                        ptr, nbytes, torch.cuda.current_stream().cuda_stream)
        _lib.check(st, "fke_qgemm_i8_ws")
        torch.cuda.synchronize()
        assert_same(host(C), ref, f"workspace {nbytes} bytes at offset {0 if ptr is None else ptr - ws.data_ptr()}")


@pytest.mark.parametrize("nan_codes", [False, True])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_mfma_k_split_fp8(oracle, dev, layout, nan_codes):
    """FP8 on a split shape: within the FP8 bounds of the reference's sequential
    sum, and the same bits on every call (the partial sums are added in split
    order).  With 0x7F / 0xFF codes in both operands every split item's sums
    come out NaN on the MFMA and are replayed with those codes cleared (the
    reference reads them as 0.0)."""
    M, N, K = 64, 4096, 14336
    S, _ = mfma_split_of(M, N, K, layout)
    say("mfma k split fp8", layout, S, "nan codes" if nan_codes else "")
    assert S > 1
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 16000, layout, with_nan_codes=nan_codes)
    bias = oracle.gen_f32_normal((N,), 16001, 0.0, 0.02)
    ref = oracle.f8_gemm(A, B, sa, sb, bias=bias, b_layout=oracle.B_KN if layout == "kn" else oracle.B_NK,
                         nthreads=NTH)
    got = gpu_f8(A, B, sa, sb, layout, "f32", "mfma", bias=bias)
    assert_fp8_close(got, ref, "f32", f"split {layout}")
    assert_same(gpu_f8(A, B, sa, sb, layout, "f32", "mfma", bias=bias), got, "split fp8 repeat")


# ---------------------------------------------------------------------- FP8

def f8_inputs(oracle, M, N, K, seed, layout="kn", with_nan_codes=False):
    xa = oracle.gen_f32_normal((M, K), seed)
    xb = oracle.gen_f32_normal((K, N), seed + 1)
    qa, sa = oracle.quantize_e4m3(xa)
    qb, sb = oracle.quantize_e4m3(xb)
    if with_nan_codes:  # the reference decodes these to 0.0
        qa.ravel()[::97] = 0x7F
        qb.ravel()[::89] = 0xFF
    B = qb if layout == "kn" else np.ascontiguousarray(qb.T)
    return qa, B, sa, sb


def gpu_f8(A, B, sa, sb, layout, out="f32", path="auto", bias=None):
    r = ops.fp8_gemm_scaled(dev_t(A), dev_t(B), sa, sb, None if bias is None else dev_t(bias),
                            out_dtype=OUT_T[out], b_layout=layout, path=path)
    torch.cuda.synchronize()
    return host(r)


def rel_errors(got, ref):
    d = got.astype(np.float64) - ref.astype(np.float64)
    return (np.abs(d).max() / max(np.abs(ref).max(), 1e-30),
            np.linalg.norm(d) / max(np.linalg.norm(ref.astype(np.float64)), 1e-30))


# Measured-level bounds beside the FP8 bar (2e-2, max-norm and Frobenius
# relative to the reference's sequential fp32 sum).  Another fp32 summation
# order moves a sum by a few units of fp32 rounding of its partial sums: fp32
# outputs measured 1e-5..3e-5 (max-norm) and ~1.5e-5 (Frobenius), held to
# 2e-4 / 1e-4.  A bf16 output is the rounding of such a sum, so each element
# must lie within bf16's half unit (at most 2^-8 of the element) plus 2e-4 of
# the largest element.  A regression to a lower-precision accumulation fails
# these long before it reaches 2e-2.
FP8_F32_TIGHT = (2e-4, 1e-4)


def assert_fp8_close(got, ref, out, what=""):
    mx, fro = rel_errors(got, ref)
    print(f"[fp8 error] {what} {out}: max-norm {mx:.3e} frobenius {fro:.3e}", flush=True)
    assert np.isfinite(got).all(), f"{what} {out}: non-finite output"
    assert mx <= 2e-2 and fro <= 2e-2, (what, out, mx, fro)
    if out == "f32":
        assert mx <= FP8_F32_TIGHT[0] and fro <= FP8_F32_TIGHT[1], ("measured-level bound", what, mx, fro)
    else:
        r = ref.astype(np.float64)
        allowed = 2.0**-8 * np.abs(r) + 2e-4 * max(np.abs(r).max(), 1e-30)
        bad = np.abs(got.astype(np.float64) - r) > allowed
        assert not bad.any(), ("bf16 beyond its rounding of an fp32-level sum", what, int(bad.sum()))


@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("shape", [(64, 64, 256), (37, 50, 131), (300, 272, 384)])
def test_fp8_generic_bit_exact(oracle, dev, layout, shape):
    M, N, K = shape
    say("fp8 generic", shape, layout)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 600 + K, layout, with_nan_codes=True)
    code = oracle.B_KN if layout == "kn" else oracle.B_NK
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=code)
    assert_same(gpu_f8(A, B, sa, sb, layout, "f32", "generic"), ref, "fp8 generic")
    if layout == "kn":
        assert_same(ref, oracle.ref_kernel_gemm_f8(A, B, sa, sb), "oracle vs reference loop")


@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("out", ["f32", "bf16"])
@pytest.mark.parametrize("nan_codes", [False, True])
def test_fp8_mfma_tolerance(oracle, dev, layout, out, nan_codes):
    """The 256x256 tile within the FP8 bounds, and every smaller tile equal to
    it bit for bit, both B layouts: each output is summed over K in the same
    order whatever the tile."""
    M, N, K = 300, 528, 1024
    say("fp8 mfma", layout, out, nan_codes)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 700, layout, with_nan_codes=nan_codes)
    bias = oracle.gen_f32_normal((N,), 701, 0.0, 0.02)
    code = oracle.B_KN if layout == "kn" else oracle.B_NK
    ref = oracle.f8_gemm(A, B, sa, sb, bias=bias, b_layout=code)
    big = gpu_f8(A, B, sa, sb, layout, out, "mfma_256x256", bias=bias)
    got = oracle.bf16_to_f32(big) if out == "bf16" else big
    assert_fp8_close(got, ref, out, f"mfma 256x256 {layout} nan={nan_codes}")
    for tile in SMALL_TILES:
        assert_same(gpu_f8(A, B, sa, sb, layout, out, tile, bias=bias), big, f"fp8 {tile} {layout} vs 256x256")


@pytest.mark.parametrize("M,N,K", [(1, 300, 4096), (1, 14336, 4096), (1, 777, 4160), (1, 1001, 1984), (3, 1000, 2048),
                                   (16, 777, 5056),
                                   (16, 4096, 14336), (17, 129, 4096), (40, 500, 2048), (64, 1000, 14336),
                                   (130, 300, 8192)])
@pytest.mark.parametrize("nan_codes", [False, True])
def test_fp8_streamed_tolerance(oracle, dev, M, N, K, nan_codes):
    """FP8 decode and batches (B [N,K]) on the row kernel (M = 1, K a multiple
    of 4096 or not) and the LDS-streamed kernel: fp32 sums in another order than
    the reference's sequential loop, so the FP8 bar (2e-2 relative); codes 0x7F
    / 0xFF count as 0.0 like the reference."""
    say("fp8 streamed", M, N, K, nan_codes)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 800 + M + K, "nk", with_nan_codes=nan_codes)
    bias = oracle.gen_f32_normal((N,), 801 + N, 0.0, 0.02)
    ref = oracle.f8_gemm(A, B, sa, sb, bias=bias, b_layout=oracle.B_NK, nthreads=NTH)
    for out in ("f32", "bf16"):
        got = gpu_f8(A, B, sa, sb, "nk", out, "gemv", bias=bias)
        if out == "bf16":
            got = oracle.bf16_to_f32(got)
        assert_fp8_close(got, ref, out, f"streamed {M, N, K} nan={nan_codes}")


@pytest.mark.parametrize("M", [1, 16, 64])
def test_fp8_streamed_isolated_nan_codes(oracle, dev, M):
    """One weight row and one activation element hold NaN codes: only the
    workgroups whose outputs come out NaN replay their stream with the codes
    cleared; every output still matches the reference (codes as 0.0)."""
    N, K = 5000, 4096
    say("fp8 streamed isolated NaN codes", M, N, K)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 870 + M, "nk")
    B[1234, 77] = 0x7F
    B[4999, K - 1] = 0xFF
    A[M - 1, 300] = 0xFF
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_NK, nthreads=NTH)
    got = gpu_f8(A, B, sa, sb, "nk", "f32", "gemv")
    assert_fp8_close(got, ref, "f32", f"streamed isolated NaN codes M={M}")


# Extreme operands on every family, both layouts.  INT8: -128 (the generators
# never emit it), +-127, at K = 8192, where |acc| reaches 8192 * 128^2 =
# 1.34e8; compared as int32.  FP8: codes 0x7E / 0xFE only (+-448, the largest
# finite E4M3): every product is +-49 * 2^12 and every partial sum over
# K = 8192 an integer multiple of 2^12 below 2^24 * 2^12, so each is exact in
# fp32 in any order and the MFMA and streamed families must match the
# reference's sequential sum bit for bit.
EXTREME_CASES = (
    [(1, 4096, 8192, "nk", "gemv"), (2, 4096, 8192, "nk", "gemv"), (16, 4096, 8192, "nk", "gemv"),
     (16, 4096, 8192, "nk", "gemv_dot"), (40, 4096, 8192, "nk", "gemv"), (100, 4096, 8192, "nk", "gemv"),
     (1, 4096, 8192, "kn", "gemv"), (16, 4096, 8192, "kn", "gemv"), (24, 4096, 8192, "kn", "gemv"),
     (37, 50, 8192, "nk", "generic"), (37, 48, 8192, "kn", "generic")]
    + [(300, 528, 8192, lay, "mfma_" + t) for lay in ("nk", "kn")
       for t in ("256x256", "128x128", "128x128_ring4", "128x64_ring4", "64x64_ring4")]
    + [(300, 528, 8192, lay, "mfma") for lay in ("nk", "kn")])  # the automatic tile: a K split


def extreme_i8(M, N, K, layout, seed):
    r = np.random.default_rng(seed)
    A = np.where(r.random((M, K)) < 0.5, -128, 127).astype(np.int8)
    A[0] = -128  # one row of -128 only
    Bnk = np.where(r.random((N, K)) < 0.5, -128, -127).astype(np.int8)
    Bnk[1] = 127
    return A, (Bnk if layout == "nk" else np.ascontiguousarray(Bnk.T))


@pytest.mark.parametrize("M,N,K,layout,path", EXTREME_CASES)
def test_extreme_int8_operands(oracle, dev, M, N, K, layout, path):
    say("extreme int8", M, N, K, layout, path)
    A, B = extreme_i8(M, N, K, layout, 11000 + M + N)
    code = oracle.B_KN if layout == "kn" else oracle.B_NK
    acc = oracle.w8a8_acc(A, B, code, nthreads=NTH)
    assert np.abs(acc.astype(np.int64)).max() >= 8192 * 127 * 127  # the case reaches the large sums
    assert_same(gpu_i8(A, B, layout, "i32", path=path), acc, f"extreme int8 {path} {layout}")


@pytest.mark.parametrize("M,N,K,layout,path",
                         [c for c in EXTREME_CASES if c[4] != "gemv_dot" and not (c[4] == "gemv" and c[0] > 32 and c[3] == "kn")])
def test_extreme_fp8_codes_exact(oracle, dev, M, N, K, layout, path):
    say("extreme fp8", M, N, K, layout, path)
    r = np.random.default_rng(12000 + M + N)
    A = np.where(r.random((M, K)) < 0.5, 0x7E, 0xFE).astype(np.uint8)
    Bkn = np.where(r.random((K, N)) < 0.5, 0x7E, 0xFE).astype(np.uint8)
    Bkn[:, 0] = 0x7E  # a column of +448 only: with row 0 below, the sum K * 448^2
    A[0] = 0x7E
    B = Bkn if layout == "kn" else np.ascontiguousarray(Bkn.T)
    sa, sb = 0.5, 0.25
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_KN if layout == "kn" else oracle.B_NK, nthreads=NTH)
    assert ref[0, 0] == np.float32(K * 448.0 * 448.0 * sa * sb)
    assert_same(gpu_f8(A, B, sa, sb, layout, "f32", path=path), ref, f"extreme fp8 {path} {layout}")


def test_c5_fp8_full(oracle, dev):
    """FP8 square: 8192^3 e4m3 (per-tensor amax/448 scales, B [K,N]), bf16 out,
    against the reference's sequential fp32 sum on 1024 rows spread over M
    (every 8th row: each of the 32 row tiles contributes 32 rows)."""
    M = N = K = 8192
    say("c5 fp8", M, N, K)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 4000, "kn")
    got = oracle.bf16_to_f32(gpu_f8(A, B, sa, sb, "kn", "bf16"))
    rows = np.arange(3, M, 8, dtype=np.int32)
    assert rows.size == 1024
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_KN, rows=rows, nthreads=NTH)
    assert_fp8_close(got[rows], ref, "bf16", "c5 1024 rows")


# --------------------------------------------------------------- python op

def test_python_op_matches_reference_numpy_op(oracle, dev):
    """flash_engine.quantized_gemm_int8 == reference python/flash_engine/ops.py:180-186."""
    say("python op")
    r = np.random.default_rng(5)
    for (M, N, K) in [(32, 32, 64), (300, 256, 512)]:
        A = r.integers(-127, 127, (M, K), dtype=np.int8)
        B = r.integers(-127, 127, (K, N), dtype=np.int8)
        for sa, sb in [(1.0, 1.0), (0.01, 0.02), (0.0123, 0.0456)]:
            ref = oracle.ref_py_gemm_i8(A, B, sa, sb)
            got_np = ops.quantized_gemm_int8(A, B, scale_a=sa, scale_b=sb)
            assert isinstance(got_np, np.ndarray)
            assert_same(got_np, ref, "python op (numpy in)")
            got_t = ops.quantized_gemm_int8(dev_t(A), dev_t(B), sa, sb)
            assert_same(host(got_t), ref, "python op (torch in)")


def test_python_op_host_operands_with_a_gpu(oracle, dev):
    """numpy operands where a GPU is visible run the HIP kernels: held in a
    wider integer type with every value in [-128, 127] they give the
    reference op's result (its astype(np.int32) widening changes nothing
    there, python/flash_engine/ops.py:184); values past int8 raise ValueError
    and float arrays TypeError, where the reference op would widen them (the
    int8 kernels cannot take them), before anything is launched."""
    say("python op, host operands of other types")
    r = np.random.default_rng(6)
    A = r.integers(-128, 128, (20, 96)).astype(np.int16)
    B = r.integers(-128, 128, (96, 48)).astype(np.int64)
    ref = oracle.ref_py_gemm_i8(A.astype(np.int8), B.astype(np.int8), 0.01, 0.02)
    expr = (A.astype(np.int32) @ B.astype(np.int32)).astype(np.float32) * (0.01 * 0.02)  # the reference's line
    assert_same(ref, expr, "oracle against the reference expression")
    assert_same(ops.quantized_gemm_int8(A, B, 0.01, 0.02), ref, "int16 / int64 operands")
    with pytest.raises(ValueError, match="int8 range"):
        ops.quantized_gemm_int8(A * 2, B, 0.01, 0.02)
    with pytest.raises(TypeError, match="integers"):
        ops.quantized_gemm_int8(A.astype(np.float32), B, 0.01, 0.02)


# ------------------------------------------------- per-token INT8 quantiser

def quant_inputs(oracle, M, K, seed, dtype):
    x = oracle.gen_f32_normal((M, K), seed, 0.0, 1.0)
    x *= oracle.gen_f32_uniform((M, 1), seed + 1, 0.01, 100.0)   # row scales over four decades
    if M > 2:
        x[1, :] = 0.0                                            # an all-zero row
        x[2, ::5] = np.float32(x[2, 0])                          # repeated values, ties
    if dtype == "bf16":
        bits = (torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
        return bits, oracle.IN_BF16
    return x, oracle.IN_F32


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("M,K", [(1, 4096), (16, 4096), (300, 1024), (7, 10000), (33, 8 * 1337), (5, 100), (3, 1)])
def test_quantize_rows_bit_exact(oracle, dev, M, K, dtype):
    """Chunked kernel (K % 8 == 0), rows longer than the register cache
    (K = 10000, 10696) and the element-wise kernel (K = 100, K = 1) against the
    oracle: codes and scales bit-exact."""
    say("quantize rows", M, K, dtype)
    x, code = quant_inputs(oracle, M, K, 900 + M + K, dtype)
    q_ref, s_ref = oracle.quantize_rows_i8(x, code)
    xt = dev_t(x) if dtype == "f32" else dev_t(x.view(np.int16)).view(torch.bfloat16)
    q, s = ops.quantize_per_token(xt)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_quantize_rows_unaligned_input(oracle, dev):
    """A row base that is not 16-byte aligned takes the element-wise kernel."""
    M, K = 9, 512
    say("quantize rows unaligned", M, K)
    x, _ = quant_inputs(oracle, M, K + 1, 950, "f32")
    xs = np.ascontiguousarray(x.reshape(-1)[1:1 + M * K].reshape(M, K))
    q_ref, s_ref = oracle.quantize_rows_i8(xs)
    big = dev_t(x.reshape(-1))
    xt = big[1:1 + M * K].view(M, K)            # 4-byte offset from the allocation
    assert xt.data_ptr() % 16 != 0
    q, s = ops.quantize_per_token(xt)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy(), s_ref) and np.array_equal(q.cpu().numpy(), q_ref)


def edge_rows(K):
    """Rows with tiny maxima (127/amax overflows fp32 below ~3.7e-37), +-inf,
    NaN and all-NaN, beside ordinary rows, for the quantiser's edge cases."""
    r = np.random.default_rng(K)
    base = r.standard_normal((10, K)).astype(np.float32)
    mags = np.array([1.0, 1e-38, 2e-40, 1e-44, 2.0**-70, 3e-37, 5.0, 1.0, 1.0, 1.0], dtype=np.float32)
    x = (base / np.abs(base).max(axis=1, keepdims=True) * mags[:, None]).astype(np.float32)
    x[6, K // 3] = np.inf
    x[7, 0] = -np.inf
    x[7, K - 1] = np.nan
    x[8, ::7] = np.nan
    x[9, :] = np.nan
    return x


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("K", [4096, 100])
def test_quantize_rows_edge_values(oracle, dev, K, dtype):
    """Tiny row maxima (the power-of-two prescale), +-inf rows (scale inf, all
    codes 0), NaN elements and all-NaN rows, on the chunked kernel (K = 4096)
    and the element-wise kernel (K = 100): codes and scales bit-exact against
    the oracle."""
    say("quantize rows edge values", K, dtype)
    x = edge_rows(K)
    if dtype == "bf16":
        bits = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        q_ref, s_ref = oracle.quantize_rows_i8(bits, oracle.IN_BF16)
        xt = dev_t(bits.view(np.int16)).view(torch.bfloat16)
    else:
        q_ref, s_ref = oracle.quantize_rows_i8(x)
        xt = dev_t(x)
    q, s = ops.quantize_per_token(xt)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.isinf(s_ref[6]) and not q_ref[6].any()


@pytest.mark.parametrize("M", [1, 9, 300])
def test_w8a8_linear_end_to_end(oracle, dev, M):
    """bf16 activations -> per-token quantiser -> W8A8 GEMM with per-channel
    weight scales and bias, bf16 out: bit-exact against the oracle's quantiser
    followed by the oracle's GEMM (exercises GEMV, MFMA-skinny and MFMA GEMM)."""
    N, K = 640, 4096
    say("w8a8_linear", M, N, K)
    x, code = quant_inputs(oracle, M, K, 970 + M, "bf16")
    W = oracle.gen_i8_uniform((N, K), 971)
    ws = oracle.gen_f32_uniform((N,), 972, 0.001, 0.02)
    bias = oracle.gen_f32_normal((N,), 973, 0.0, 0.02)
    q_ref, s_ref = oracle.quantize_rows_i8(x, code)
    acc = oracle.w8a8_acc(q_ref, W)
    ref = oracle.w8a8_epilogue(acc, s_ref, ws, 1.0, 1.0, bias, oracle.OUT_BF16)
    xt = dev_t(x.view(np.int16)).view(torch.bfloat16)
    y = ops.w8a8_linear(xt, dev_t(W), dev_t(ws), dev_t(bias), out_dtype=torch.bfloat16)
    assert_same(host(y), ref, f"w8a8_linear M={M}")


# ------------------------------------------------- torch extension binding

@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_torch_extension_i8_bit_exact(oracle, dev, layout):
    """flash_engine_cuda.quantized_gemm_int8_forward (bindings.cpp idiom) on the
    MFMA and decode families, every output type, against the oracle."""
    from flash_engine import _ext
    m = _ext.ext()
    for (M, N, K) in [(300, 528, 384), (3, 300, 1024)]:
        if layout == "kn" and M <= 16:
            continue  # the decode family takes [N,K] only (the generic family covers it)
        say("torch ext i8", layout, M, N, K)
        A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 990 + M, layout)
        acc = oracle.w8a8_acc(A, B, oracle.B_NK if layout == "nk" else oracle.B_KN)
        for out in ("f32", "bf16", "i32"):
            y = m.quantized_gemm_int8_forward(dev_t(A), dev_t(B), dev_t(sa), dev_t(sb), dev_t(bias),
                                              OUT_T[out], layout, 1.0, 1.0)
            assert_same(host(y), oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out), f"ext {layout} {out}")


def test_torch_extension_f8_and_quantizer(oracle, dev):
    from flash_engine import _ext
    m = _ext.ext()
    M, N, K = 256, 256, 512
    say("torch ext f8 + quantizer", M, N, K)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 995, "kn")
    y = m.fp8_gemm_scaled_forward(dev_t(A), dev_t(B), sa, sb, None, torch.float32, "kn")
    ref = oracle.f8_gemm(A, B, sa, sb, None, oracle.OUT_F32, oracle.B_KN, nthreads=NTH)
    assert_fp8_close(y.cpu().numpy(), ref, "f32", "torch ext")
    x, code = quant_inputs(oracle, 20, 4096, 996, "f32")
    q, s = m.quantize_per_token_forward(dev_t(x))
    q_ref, s_ref = oracle.quantize_rows_i8(x, code)
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        M = int(rng.choice([1, 2, 3, 5, 15, 16, 17, 31, 32, 33, 47, 63, 64, 65, 100, 129, 200, 300]))
        N = int(rng.integers(1, 1500))
        K = int(rng.choice([64, 192, 1024, 1984, 2048, 2112, 3008, 4096, 4160, 6144]))
        layout = str(rng.choice(["nk", "nk", "kn"]))
        out = str(rng.choice(["i32", "bf16", "f32"]))
        cases.append((M, N, K, layout, out))
    return cases


@pytest.mark.parametrize("M,N,K,layout,out", _random_cases(40, 20261201))
def test_auto_dispatch_random_shapes(oracle, dev, M, N, K, layout, out):
    """Seeded random shapes through the automatic dispatch (every family and
    block-count boundary of the decode, batch, MFMA and generic paths),
    bit-exact against the oracle."""
    say("auto random", M, N, K, layout, out)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 5000 + M + N + K, layout)
    acc = oracle.w8a8_acc(A, B, oracle.B_NK if layout == "nk" else oracle.B_KN, nthreads=NTH)
    if out == "i32":
        assert_same(gpu_i8(A, B, layout, "i32"), acc, f"auto {M, N, K, layout} i32")
    else:
        got = gpu_i8(A, B, layout, out, "auto", sa, sb, bias=bias)
        assert_same(got, oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out), f"auto {M, N, K, layout} {out}")


@pytest.mark.parametrize("M,N,K,layout,out", _random_cases(20, 20261202))
def test_fp8_auto_dispatch_random_shapes(oracle, dev, M, N, K, layout, out):
    """Seeded random shapes through the FP8 automatic dispatch (decode family
    for B [N,K], MFMA and generic families), within the FP8 bar of the
    reference's sequential sum, with a few NaN codes."""
    out = "f32" if out == "i32" else out
    say("fp8 auto random", M, N, K, layout, out)
    A, B, sa, sb = f8_inputs(oracle, M, N, K, 6000 + M + N + K, layout, with_nan_codes=(M + N) % 3 == 0)
    ref = oracle.f8_gemm(A, B, sa, sb, b_layout=oracle.B_NK if layout == "nk" else oracle.B_KN, nthreads=NTH)
    got = gpu_f8(A, B, sa, sb, layout, out)
    if out == "bf16":
        got = oracle.bf16_to_f32(got)
    assert_fp8_close(got, ref, out, f"auto {M, N, K, layout}")


# B [N,K] up to 4 rows whose K is a multiple of 4 but not of 64, or whose
# operands are only 4-byte aligned: the row kernel's 4-byte form (past one
# row only where the MFMA GEMM cannot run: K % 16 != 0 or unaligned).
ROWS_DW_CASES = [(1, 14336, 4100, 0), (2, 1000, 68, 0), (3, 4100, 4, 4), (4, 14336, 4108, 0), (1, 4096, 4096, 4),
                 (4, 2048, 1028, 4), (1, 14336, 4000, 0)]


@pytest.mark.parametrize("M,N,K,shift", ROWS_DW_CASES)
def test_gemv_rows_dword_form(oracle, dev, M, N, K, shift):
    """INT8 bit-exact on every output type; FP8 (0x7F / 0xFF codes included)
    within the bounds of the sequential sum; A and B `shift` bytes past
    16-byte alignment."""
    say("gemv rows, 4-byte loads", M, N, K, shift)
    L = _lib.lib()
    assert L.fke_select_path_i8(4096 + shift, 4096 + shift, 4096, M, N, K, _lib.OUT_BF16, _lib.B_NK) == _lib.PATH_GEMV
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9600 + 5 * M + N + K, act="normal")
    acc = oracle.w8a8_acc(A, B, nthreads=NTH)
    (ba, pa), (bb, pb) = dev_at(A, shift), dev_at(B, shift)
    dsa, dsb, dbias = dev_t(sa), dev_t(sb), dev_t(bias)
    for out in ("i32", "f32", "bf16"):
        C = torch.empty((M, N), dtype=OUT_T[out], device=dev)
        _lib.check(L.fke_qgemm_i8(pa, pb, C.data_ptr(), M, N, K, dsa.data_ptr(), dsb.data_ptr(), 1.0, 1.0,
                                  dbias.data_ptr(), {"f32": _lib.OUT_F32, "bf16": _lib.OUT_BF16, "i32": _lib.OUT_I32}[out],
                                  _lib.B_NK, torch.cuda.current_stream().cuda_stream), "fke_qgemm_i8")
        torch.cuda.synchronize()
        want = acc if out == "i32" else oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
        assert_same(host(C), want, f"rows dword {out} M={M} N={N} K={K} shift={shift}")
    assert L.fke_select_path_f8(4096 + shift, 4096 + shift, 4096, M, N, K, _lib.OUT_BF16, _lib.B_NK) == _lib.PATH_GEMV
    A8, B8, fa, fb = f8_inputs(oracle, M, N, K, 9650 + 3 * M + N + K, "nk", with_nan_codes=True)
    ref = oracle.f8_gemm(A8, B8, fa, fb, b_layout=oracle.B_NK, nthreads=NTH)
    (ba, pa), (bb, pb) = dev_at(A8, shift), dev_at(B8, shift)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.check(L.fke_qgemm_f8(pa, pb, C.data_ptr(), M, N, K, fa, fb, None, _lib.OUT_F32, _lib.B_NK,
                              torch.cuda.current_stream().cuda_stream), "fke_qgemm_f8")
    torch.cuda.synchronize()
    assert_fp8_close(host(C), ref, "f32", f"rows dword fp8 M={M} N={N} K={K} shift={shift}")


# INT8 and FP8 whose K (and N, for B [K,N]) is a multiple of 4 but not of 16,
# or whose operands are only 4-byte aligned: the word kernel (128x128 tiles,
# 128x64 where those number at most half the CUs, on the matrix cores, 4-byte
# copies), through the automatic path.  B [K,N]
# from 33 rows (below, the [K,N] decode's 4-byte form takes such shapes).
WORDS_CASES = [(5, 14336, 4100, 0, "nk"), (6, 1000, 68, 0, "nk"), (64, 64, 100, 0, "nk"), (129, 257, 4, 0, "nk"),
               (300, 520, 4104, 0, "nk"), (256, 4096, 4096, 4, "nk"), (200, 1030, 1028, 4, "nk"),
               (1024, 1024, 4100, 0, "nk"), (33, 4100, 4100, 0, "kn"), (64, 64, 100, 0, "kn"),
               (129, 260, 4, 0, "kn"), (300, 520, 4104, 0, "kn"), (256, 4096, 4096, 4, "kn"),
               (200, 1028, 1028, 4, "kn"), (1024, 1024, 4100, 0, "kn"),
               # 256 tiles of 128x128: the wide tile (128 or fewer take 128x64 tiles)
               (2048, 2048, 100, 0, "nk"), (2048, 2064, 68, 4, "nk"), (2048, 2048, 100, 0, "kn"),
               (2048, 2064, 132, 4, "kn")]


def _words_path(L, M, N, K, shift, layout, f8=False):
    sel = L.fke_select_path_f8 if f8 else L.fke_select_path_i8
    return sel(4096 + shift, 4096 + shift, 4096, M, N, K, _lib.OUT_BF16, _lib.B_KN if layout == "kn" else _lib.B_NK)


@pytest.mark.parametrize("M,N,K,shift,layout", WORDS_CASES)
def test_words_kernel_bit_exact(oracle, dev, M, N, K, shift, layout):
    """INT8: every output type bit-exact against the oracle, with A and B
    `shift` bytes past 16-byte alignment; the call goes to FKE_PATH_MFMA."""
    say("int8 word kernel", M, N, K, shift, layout)
    L = _lib.lib()
    assert _words_path(L, M, N, K, shift, layout) == _lib.PATH_MFMA
    bl, obl = (_lib.B_KN, oracle.B_KN) if layout == "kn" else (_lib.B_NK, oracle.B_NK)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 9900 + 7 * M + N + K, layout=layout, act="normal")
    acc = oracle.w8a8_acc(A, B, obl, nthreads=NTH)
    (ba, pa), (bb, pb) = dev_at(A, shift), dev_at(B, shift)
    dsa, dsb, dbias = dev_t(sa), dev_t(sb), dev_t(bias)
    for out in ("i32", "f32", "bf16"):
        C = torch.empty((M, N), dtype=OUT_T[out], device=dev)
        _lib.check(L.fke_qgemm_i8(pa, pb, C.data_ptr(), M, N, K, dsa.data_ptr(), dsb.data_ptr(), 1.0, 1.0,
                                  dbias.data_ptr(), {"f32": _lib.OUT_F32, "bf16": _lib.OUT_BF16, "i32": _lib.OUT_I32}[out],
                                  bl, torch.cuda.current_stream().cuda_stream), "fke_qgemm_i8")
        torch.cuda.synchronize()
        want = acc if out == "i32" else oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
        assert_same(host(C), want, f"words {out} M={M} N={N} K={K} shift={shift} {layout}")
    # scalar scales and no bias (the reference launcher's form)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.check(L.fke_qgemm_i8(pa, pb, C.data_ptr(), M, N, K, None, None, 0.05, 0.02, None, _lib.OUT_F32, bl,
                              torch.cuda.current_stream().cuda_stream), "fke_qgemm_i8")
    torch.cuda.synchronize()
    assert_same(host(C), oracle_out(oracle, acc, None, None, 0.05, 0.02, None, "f32"), f"words scalar M={M} {layout}")


@pytest.mark.parametrize("nan_codes", [False, True])
@pytest.mark.parametrize("M,N,K,shift,layout", WORDS_CASES)
def test_words_kernel_fp8(oracle, dev, M, N, K, shift, layout, nan_codes):
    """FP8 within the bounds of the sequential fp32 sum (codes 0x7F / 0xFF
    counted as 0.0: the workgroup's replay), bf16 and fp32 out with bias."""
    say("fp8 word kernel", M, N, K, shift, layout, nan_codes)
    L = _lib.lib()
    assert _words_path(L, M, N, K, shift, layout, f8=True) == _lib.PATH_MFMA
    bl, obl = (_lib.B_KN, oracle.B_KN) if layout == "kn" else (_lib.B_NK, oracle.B_NK)
    A8, B8, fa, fb = f8_inputs(oracle, M, N, K, 9950 + 7 * M + N + K, layout, with_nan_codes=nan_codes)
    bias = oracle.gen_f32_normal((N,), 9951 + M + N, 0.0, 0.02)
    (ba, pa), (bb, pb) = dev_at(A8, shift), dev_at(B8, shift)
    dbias = dev_t(bias)
    ref = oracle.f8_gemm(A8, B8, fa, fb, bias=bias, b_layout=obl, nthreads=NTH)
    for out in ("f32", "bf16"):
        C = torch.empty((M, N), dtype=OUT_T[out], device=dev)
        _lib.check(L.fke_qgemm_f8(pa, pb, C.data_ptr(), M, N, K, fa, fb, dbias.data_ptr(),
                                  _lib.OUT_F32 if out == "f32" else _lib.OUT_BF16, bl,
                                  torch.cuda.current_stream().cuda_stream), "fke_qgemm_f8")
        torch.cuda.synchronize()
        got = host(C) if out == "f32" else oracle.bf16_to_f32(host(C))
        assert_fp8_close(got, ref, out, f"words fp8 M={M} N={N} K={K} shift={shift} {layout} nan={nan_codes}")


def _random_word_cases(n, seed):
    """Shapes whose N and K are multiples of 4 only (now and then of 16),
    with operands 0, 4, 8 or 12 bytes past 16-byte alignment: the 4-byte
    forms of the decode kernels, the word kernel and, where aligned, the
    16-byte families."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        M = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 20, 21, 32, 33, 64, 100, 129, 200]))
        N = 4 * int(rng.integers(1, 600))
        K = 4 * int(rng.integers(1, 650))
        layout = str(rng.choice(["nk", "kn"]))
        shift = int(rng.choice([0, 4, 8, 12]))
        cases.append((M, N, K, layout, shift))
    return cases


@pytest.mark.parametrize("M,N,K,layout,shift", _random_word_cases(30, 20261203))
def test_auto_dispatch_random_word_shapes(oracle, dev, M, N, K, layout, shift):
    """Seeded shapes of 4-byte multiples through the automatic dispatch: INT8
    bit-exact (bf16 out with bias, and int32), FP8 (0x7F / 0xFF codes in one
    case of three) within the bounds of the sequential sum."""
    say("auto random, 4-byte shapes", M, N, K, layout, shift)
    L = _lib.lib()
    bl, obl = (_lib.B_KN, oracle.B_KN) if layout == "kn" else (_lib.B_NK, oracle.B_NK)
    A, B, sa, sb, bias = inputs_i8(oracle, M, N, K, 5200 + M + N + K, layout)
    acc = oracle.w8a8_acc(A, B, obl, nthreads=NTH)
    (ba, pa), (bb, pb) = dev_at(A, shift), dev_at(B, shift)
    dsa, dsb, dbias = dev_t(sa), dev_t(sb), dev_t(bias)
    for out, code in (("bf16", _lib.OUT_BF16), ("i32", _lib.OUT_I32)):
        C = torch.empty((M, N), dtype=OUT_T[out], device=dev)
        _lib.check(L.fke_qgemm_i8(pa, pb, C.data_ptr(), M, N, K, dsa.data_ptr(), dsb.data_ptr(), 1.0, 1.0,
                                  dbias.data_ptr(), code, bl, torch.cuda.current_stream().cuda_stream), "fke_qgemm_i8")
        torch.cuda.synchronize()
        want = acc if out == "i32" else oracle_out(oracle, acc, sa, sb, 1.0, 1.0, bias, out)
        assert_same(host(C), want, f"random words {out} {M, N, K, layout, shift}")
    A8, B8, fa, fb = f8_inputs(oracle, M, N, K, 5300 + M + N + K, layout, with_nan_codes=(M + N) % 3 == 0)
    ref = oracle.f8_gemm(A8, B8, fa, fb, b_layout=obl, nthreads=NTH)
    (ba8, pa8), (bb8, pb8) = dev_at(A8, shift), dev_at(B8, shift)
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    _lib.check(L.fke_qgemm_f8(pa8, pb8, C.data_ptr(), M, N, K, fa, fb, None, _lib.OUT_F32, bl,
                              torch.cuda.current_stream().cuda_stream), "fke_qgemm_f8")
    torch.cuda.synchronize()
    assert_fp8_close(host(C), ref, "f32", f"random words fp8 {M, N, K, layout, shift}")
