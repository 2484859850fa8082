"""The K splits' partial sums on the library's static split pool (no call
allocates device memory): a stream never used before, captured into a HIP
graph, gets a pool slot and the same two-kernel split plan as an eager call;
INT8 results stay bit-exact against the oracle on every replay, FP8 results
are bit-identical to the eager call's; and a run of split calls on fresh
streams leaves the device's free memory unchanged.  Graphs are captured and
replayed through the HIP runtime itself (ctypes), so their kernel nodes can
be counted."""
import ctypes as ct
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _lib  # noqa: E402

NTH = min(16, os.cpu_count() or 1)
M16, N, K = 16, 14336, 4096          # C2's decode shape, B [K,N]: 2 K splits
GRAPH_NODE_KERNEL = 0                 # hipGraphNodeTypeKernel
CAPTURE_GLOBAL = 0                    # hipStreamCaptureModeGlobal


def say(*a):
    print("[case]", *a, flush=True)


class Hip:
    """The HIP runtime this process already loaded (torch's), for raw streams
    and graphs."""

    def __init__(self):
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        assert path, "libamdhip64 not loaded"
        self.h = ct.CDLL(path)
        v = ct.c_void_p
        for name, args in {
            "hipStreamCreate": [ct.POINTER(v)], "hipStreamDestroy": [v], "hipStreamSynchronize": [v],
            "hipStreamBeginCapture": [v, ct.c_int], "hipStreamEndCapture": [v, ct.POINTER(v)],
            "hipGraphGetNodes": [v, ct.POINTER(v), ct.POINTER(ct.c_size_t)],
            "hipGraphNodeGetType": [v, ct.POINTER(ct.c_int)],
            "hipGraphInstantiate": [ct.POINTER(v), v, ct.POINTER(v), ct.c_char_p, ct.c_size_t],
            "hipGraphLaunch": [v, v], "hipGraphExecDestroy": [v], "hipGraphDestroy": [v],
        }.items():
            fn = getattr(self.h, name)
            fn.argtypes = args
            fn.restype = ct.c_int

    def ok(self, st, what):
        assert st == 0, f"{what}: hip status {st}"

    def stream(self):
        s = ct.c_void_p()
        self.ok(self.h.hipStreamCreate(ct.byref(s)), "hipStreamCreate")
        return s.value

    def capture(self, s, body):
        """Capture body(s) on stream s; returns the graph."""
        self.ok(self.h.hipStreamBeginCapture(s, CAPTURE_GLOBAL), "hipStreamBeginCapture")
        try:
            body(s)
        finally:
            g = ct.c_void_p()
            st = self.h.hipStreamEndCapture(s, ct.byref(g))
        self.ok(st, "hipStreamEndCapture")
        return g.value

    def node_types(self, g):
        n = ct.c_size_t(0)
        self.ok(self.h.hipGraphGetNodes(g, None, ct.byref(n)), "hipGraphGetNodes")
        nodes = (ct.c_void_p * n.value)()
        self.ok(self.h.hipGraphGetNodes(g, nodes, ct.byref(n)), "hipGraphGetNodes")
        kinds = []
        for i in range(n.value):
            t = ct.c_int(-1)
            self.ok(self.h.hipGraphNodeGetType(nodes[i], ct.byref(t)), "hipGraphNodeGetType")
            kinds.append(t.value)
        return kinds

    def instantiate(self, g):
        e = ct.c_void_p()
        self.ok(self.h.hipGraphInstantiate(ct.byref(e), g, None, None, 0), "hipGraphInstantiate")
        return e.value

    def replay(self, e, s):
        self.ok(self.h.hipGraphLaunch(e, s), "hipGraphLaunch")
        self.ok(self.h.hipStreamSynchronize(s), "hipStreamSynchronize")


@pytest.fixture(scope="module")
def hip(dev):
    torch.zeros(1, device=dev)  # the runtime and device 0 are initialised
    return Hip()


def dev_t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def assert_same(got, ref, what):
    bad = (got.view(np.uint32) != ref.view(np.uint32)) if got.dtype == np.float32 else (got != ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} mismatches"


def i8_case(oracle, M, seed):
    A = oracle.gen_i8_clipped_normal((M, K), seed, 30.0)
    B = np.ascontiguousarray(oracle.gen_i8_uniform((N, K), seed + 1).T)
    sa = oracle.gen_f32_uniform((M,), seed + 2, 0.001, 0.02)
    sb = oracle.gen_f32_uniform((N,), seed + 3, 0.001, 0.02)
    bias = oracle.gen_f32_normal((N,), seed + 4, 0.0, 0.02)
    acc = oracle.w8a8_acc(A, B, oracle.B_KN, nthreads=NTH)
    ref = oracle.w8a8_epilogue(acc, sa, sb, 1.0, 1.0, bias, oracle.OUT_BF16)
    return [dev_t(x) for x in (A, B, sa, sb, bias)], ref


def i8_call(L, d, C, s):
    A, B, sa, sb, bias = d
    M = A.shape[0]
    _lib.check(L.fke_qgemm_i8(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, sa.data_ptr(), sb.data_ptr(),
                              1.0, 1.0, bias.data_ptr(), _lib.OUT_BF16, _lib.B_KN, s), "fke_qgemm_i8")


def test_capture_on_a_never_used_stream_keeps_the_split(oracle, dev, hip):
    """INT8 [K,N] decode at M = 16, N = 14336, K = 4096 captured on a stream
    created for the test: the capture takes a pool slot, the graph holds the
    split kernel and the kernel that adds the splits, and three replays are
    bit-exact against the oracle."""
    say("capture never-used stream: i8 kn decode", M16, N, K)
    L = _lib.lib()
    assert L.fke_qgemm_workspace_size(M16, N, K, _lib.B_KN) == 2 * M16 * N * 4  # a 2-way split
    d, ref = i8_case(oracle, M16, 31000)
    C = torch.empty((M16, N), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    s = hip.stream()
    used = L.fke_split_slots_in_use()
    assert 0 <= used < _lib.SPLIT_SLOTS + _lib.SPLIT_SMALL_SLOTS, used
    g = hip.capture(s, lambda st: i8_call(L, d, C, st))
    assert L.fke_split_slots_in_use() == used + 1, "the capture did not take a pool slot"
    assert hip.node_types(g) == [GRAPH_NODE_KERNEL] * 2, hip.node_types(g)
    e = hip.instantiate(g)
    for r in range(3):
        C.zero_()
        torch.cuda.synchronize()
        hip.replay(e, s)
        assert_same(host(C), ref, f"replay {r}")
        i8_call(L, d, C, torch.cuda.current_stream().cuda_stream)  # eager, on another stream's slot
        torch.cuda.synchronize()
        assert_same(host(C), ref, f"eager after replay {r}")
    hip.ok(hip.h.hipGraphExecDestroy(e), "hipGraphExecDestroy")
    hip.ok(hip.h.hipGraphDestroy(g), "hipGraphDestroy")


def test_captured_fp8_decode_has_the_eager_bits(oracle, dev, hip):
    """FP8 [K,N] decode (codes 0x7F / 0xFF included) at the same shape: the
    eager call, the call on a caller workspace of fke_qgemm_workspace_size
    bytes and the graph captured on a new stream give the same bits (one split
    plan for all three), within the FP8 bars of the reference's sequential
    sum."""
    say("capture never-used stream: f8 kn decode", M16, N, K)
    L = _lib.lib()
    xa = oracle.gen_f32_normal((M16, K), 32000)
    xb = oracle.gen_f32_normal((K, N), 32001)
    qa, sa = oracle.quantize_e4m3(xa)
    qb, sb = oracle.quantize_e4m3(xb)
    qa.ravel()[::97] = 0x7F
    qb.ravel()[::89] = 0xFF
    ref = oracle.f8_gemm(qa, qb, sa, sb, b_layout=oracle.B_KN, nthreads=NTH)
    dA, dB = dev_t(qa), dev_t(qb)
    need = L.fke_qgemm_workspace_size(M16, N, K, _lib.B_KN)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    outs = [torch.empty((M16, N), dtype=torch.float32, device=dev) for _ in range(3)]

    def eager(C, s):
        _lib.check(L.fke_qgemm_f8(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M16, N, K, float(sa), float(sb), None,
                                  _lib.OUT_F32, _lib.B_KN, s), "fke_qgemm_f8")

    cur = torch.cuda.current_stream().cuda_stream
    eager(outs[0], cur)
    _lib.check(L.fke_qgemm_f8_ws(dA.data_ptr(), dB.data_ptr(), outs[1].data_ptr(), M16, N, K, float(sa), float(sb),
                                 None, _lib.OUT_F32, _lib.B_KN, ws.data_ptr(), need, cur), "fke_qgemm_f8_ws")
    torch.cuda.synchronize()
    s = hip.stream()
    g = hip.capture(s, lambda st: eager(outs[2], st))
    assert hip.node_types(g) == [GRAPH_NODE_KERNEL] * 2
    e = hip.instantiate(g)
    hip.replay(e, s)
    got = [host(c) for c in outs]
    assert np.isfinite(got[0]).all()
    d = got[0].astype(np.float64) - ref.astype(np.float64)
    rel = np.abs(d).max() / np.abs(ref).max()
    print(f"[fp8 error] captured decode max-norm {rel:.3e}", flush=True)
    assert rel <= 2e-2
    assert_same(got[1], got[0], "caller workspace against eager")
    assert_same(got[2], got[0], "graph replay against eager")
    hip.ok(hip.h.hipGraphExecDestroy(e), "hipGraphExecDestroy")
    hip.ok(hip.h.hipGraphDestroy(g), "hipGraphDestroy")


def test_split_calls_allocate_no_device_memory(oracle, dev, hip):
    """Split calls of every kind on two streams that have never run one (each
    takes a new pool slot) leave the device's free memory unchanged: the INT8
    and FP8 [K,N] decodes, the drop-in FP8 launcher at a decode shape, the
    MFMA GEMM's K split (64x4096x14336, B [N,K]) and the W8A8 linear on a
    workspace that holds only its codes and scales.  Outputs are checked."""
    L = _lib.lib()
    say("no device allocation: split calls on fresh streams")
    d, ref = i8_case(oracle, M16, 33000)
    C = torch.empty((M16, N), dtype=torch.bfloat16, device=dev)
    Mm, Nm, Km = 64, 4096, 14336
    assert L.fke_select_mfma_split(Mm, Nm, Km, _lib.B_NK, 0, None) > 1
    Am = dev_t(oracle.gen_i8_uniform((Mm, Km), 33100))
    Bm = dev_t(oracle.gen_i8_uniform((Nm, Km), 33101))
    acc_m = oracle.w8a8_acc(Am.cpu().numpy(), Bm.cpu().numpy(), nthreads=NTH)
    Cm = torch.empty((Mm, Nm), dtype=torch.int32, device=dev)
    qa = dev_t(np.full((7, K), 0x38, np.uint8))     # 1.0 in e4m3
    qb = dev_t(np.full((K, 2048), 0x30, np.uint8))  # 0.5
    Cf = torch.empty((7, 2048), dtype=torch.float32, device=dev)
    X = torch.randn((Mm, Km), device=dev).to(torch.bfloat16)
    Y = torch.empty((Mm, Nm), dtype=torch.bfloat16, device=dev)
    Y_ref = torch.empty_like(Y)
    work = torch.empty(L.fke_w8a8_linear_workspace_size(Mm, Km), dtype=torch.uint8, device=dev)
    big = torch.empty(work.numel() + 256 + L.fke_qgemm_workspace_size(Mm, Nm, Km, _lib.B_NK), dtype=torch.uint8,
                      device=dev)

    def calls(s):
        i8_call(L, d, C, s)
        _lib.check(L.fke_qgemm_i8(Am.data_ptr(), Bm.data_ptr(), Cm.data_ptr(), Mm, Nm, Km, None, None, 1.0, 1.0,
                                  None, _lib.OUT_I32, _lib.B_NK, s), "fke_qgemm_i8 split")
        _lib.check(L.fke_launch_fp8_gemm_scaled(qa.data_ptr(), qb.data_ptr(), Cf.data_ptr(), 0.5, 2.0, 7, 2048, K, s),
                   "fke_launch_fp8_gemm_scaled")
        _lib.check(L.fke_w8a8_linear(X.data_ptr(), _lib.IN_BF16, Bm.data_ptr(), Y.data_ptr(), Mm, Nm, Km, None, 0.01,
                                     None, _lib.OUT_BF16, work.data_ptr(), work.numel(), s), "fke_w8a8_linear")

    def check(what):
        torch.cuda.synchronize()
        assert_same(host(C), ref, f"{what}: i8 kn decode")
        assert_same(host(Cm), acc_m, f"{what}: mfma k split")
        assert (Cf == 0.5 * K).all(), f"{what}: fp8 drop-in"   # sum of K products 1.0 * 0.5, times 0.5 * 2.0
        assert torch.equal(Y.view(torch.int16), Y_ref.view(torch.int16)), f"{what}: w8a8 linear"

    # the reference of the linear: its whole split plan on the caller's workspace
    _lib.check(L.fke_w8a8_linear(X.data_ptr(), _lib.IN_BF16, Bm.data_ptr(), Y_ref.data_ptr(), Mm, Nm, Km, None, 0.01,
                                 None, _lib.OUT_BF16, big.data_ptr(), big.numel(), None), "fke_w8a8_linear (big)")
    calls(torch.cuda.current_stream().cuda_stream)  # code object loaded, the current stream's slot taken
    check("current stream")
    streams = [hip.stream() for _ in range(2)]
    for s in streams:  # each stream's own first work (its hardware queue) before the measurement
        with torch.cuda.stream(torch.cuda.ExternalStream(s)):
            C.zero_()
    torch.cuda.synchronize()
    used = L.fke_split_slots_in_use()
    free0 = torch.cuda.mem_get_info()[0]
    for s in streams:
        calls(s)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert L.fke_split_slots_in_use() == used + 2
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
    check("fresh streams")
