"""The allocation-free W8A8 linear (fke_w8a8_linear_noalloc), through the C
ABI: bit-identical to fke_w8a8_linear with a caller workspace, on two calls in
a row (the second smaller, so it reads only what it wrote over the first
call's leftovers in the shared device scratch), on a shape whose workspace
fills most of the scratch, on a shape whose GEMM splits K (partial sums in
the scratch past the codes and scales), and on two streams whose calls the
library orders."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _lib  # noqa: E402


def say(*a):
    print("[case]", *a, flush=True)


def _inputs(M, N, K, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = (torch.randn((M, K), device=dev, generator=g) * 3).to(torch.bfloat16)
    W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    ws = torch.rand(N, device=dev, generator=g) * 0.019 + 0.001
    bias = torch.randn(N, device=dev, generator=g) * 0.02
    return x, W, ws, bias


def _with_workspace(L, x, W, ws, bias, out_code, out_dtype, stream):
    M, K = x.shape
    N = W.shape[0]
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    work = torch.empty(L.fke_w8a8_linear_workspace_size(M, K), dtype=torch.uint8, device=x.device)
    st = L.fke_w8a8_linear(x.data_ptr(), _lib.IN_BF16, W.data_ptr(), y.data_ptr(), M, N, K, ws.data_ptr(), 1.0,
                           bias.data_ptr(), out_code, work.data_ptr(), work.numel(), stream)
    _lib.check(st, "fke_w8a8_linear")
    return y


def _noalloc(L, x, W, ws, bias, out_code, out_dtype, stream):
    M, K = x.shape
    N = W.shape[0]
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    st = L.fke_w8a8_linear_noalloc(x.data_ptr(), _lib.IN_BF16, W.data_ptr(), y.data_ptr(), M, N, K,
                                   ws.data_ptr(), 1.0, bias.data_ptr(), out_code, stream)
    _lib.check(st, "fke_w8a8_linear_noalloc")
    return y


def _same(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))


@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_noalloc_matches_workspace_entry_two_calls(out):
    assert torch.cuda.is_available()
    dev = torch.device("cuda:0")
    L = _lib.lib()
    code, dt = (_lib.OUT_BF16, torch.bfloat16) if out == "bf16" else (_lib.OUT_F32, torch.float32)
    sh = torch.cuda.current_stream(dev).cuda_stream
    # first a prefill-sized call (MFMA GEMM), then a smaller decode call (row kernel)
    for (M, N, K), seed in (((300, 640, 4096), 11), ((3, 1000, 2048), 12)):
        say("noalloc linear", M, N, K, out)
        x, W, ws, bias = _inputs(M, N, K, seed, dev)
        ref = _with_workspace(L, x, W, ws, bias, code, dt, sh)
        got = _noalloc(L, x, W, ws, bias, code, dt, sh)
        torch.cuda.synchronize()
        assert _same(got, ref), f"noalloc differs at {(M, N, K)}"


def test_noalloc_near_the_scratch_limit():
    """M*K close to the 32 MiB scratch (4096 x 8000 codes plus the scales at
    the next 256-byte boundary), then a one-row call that leaves the rest of
    the previous contents in place."""
    dev = torch.device("cuda:0")
    L = _lib.lib()
    sh = torch.cuda.current_stream(dev).cuda_stream
    for (M, N, K), seed in (((4096, 256, 8000), 21), ((1, 256, 8000), 22)):
        assert L.fke_w8a8_linear_workspace_size(M, K) <= _lib.W8A8_NOALLOC_SCRATCH_BYTES
        say("noalloc linear near limit", M, N, K)
        x, W, ws, bias = _inputs(M, N, K, seed, dev)
        ref = _with_workspace(L, x, W, ws, bias, _lib.OUT_BF16, torch.bfloat16, sh)
        got = _noalloc(L, x, W, ws, bias, _lib.OUT_BF16, torch.bfloat16, sh)
        torch.cuda.synchronize()
        assert _same(got, ref), f"noalloc differs at {(M, N, K)}"
    x, W, ws, bias = _inputs(4096, 256, 8192, 23, dev)
    y = torch.empty((4096, 256), dtype=torch.bfloat16, device=dev)
    st = L.fke_w8a8_linear_noalloc(x.data_ptr(), _lib.IN_BF16, W.data_ptr(), y.data_ptr(), 4096, 256, 8192,
                                   ws.data_ptr(), 1.0, bias.data_ptr(), _lib.OUT_BF16, sh)
    assert st == _lib.HIP_ERROR_INVALID_VALUE   # past the scratch: refused before any launch


def test_noalloc_k_split_and_two_streams():
    """64x4096x14336 splits K four ways on the MFMA ring tiles: the partial sums
    go to the scratch past the codes and scales.  Then calls alternate between
    two streams with no host synchronisation, on inputs of different shapes
    (the split shape and a decode shape): the library orders them, and every
    output equals its workspace-entry reference."""
    dev = torch.device("cuda:0")
    L = _lib.lib()
    sh = torch.cuda.current_stream(dev).cuda_stream
    M, N, K = 64, 4096, 14336
    assert L.fke_select_mfma_split(M, N, K, _lib.B_NK, 0, None) == 4
    say("noalloc linear k split", M, N, K)
    cases = [_inputs(M, N, K, 31, dev), _inputs(2, 2048, 14336, 32, dev)]
    refs = [_with_workspace(L, *c, _lib.OUT_BF16, torch.bfloat16, sh) for c in cases]
    got = _noalloc(L, *cases[0], _lib.OUT_BF16, torch.bfloat16, sh)
    torch.cuda.synchronize()
    assert _same(got, refs[0]), "noalloc differs on the split shape"
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    say("noalloc linear two streams, 8 calls each")
    outs = []
    for i in range(16):
        c = i % 2
        outs.append((c, _noalloc(L, *cases[c], _lib.OUT_BF16, torch.bfloat16, streams[c].cuda_stream)))
    torch.cuda.synchronize()
    for i, (c, y) in enumerate(outs):
        assert _same(y, refs[c]), f"call {i} on stream {c} differs"
