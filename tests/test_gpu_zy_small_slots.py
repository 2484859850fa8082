"""GPU test of the split pool's small slots (capi.hip, stream_slot): past the
FKE_SPLIT_SLOTS large slots of a GPU, the next FKE_SPLIT_SMALL_SLOTS streams
get slots of FKE_SPLIT_SMALL_SLOT_BYTES, and a split whose partial sums fit
one still runs (captured or eager, the same plan, bit-exact).  A stream keeps
its slot for the life of the process, so this test hands out every large slot
of the pytest process: the file is collected after the other GPU test files
(only the no-allocation test, which does not use the pool, comes later)."""
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from flash_engine import _lib  # noqa: E402
from test_gpu_split_pool import (GRAPH_NODE_KERNEL, N, Hip, assert_same, host, i8_call,  # noqa: E402
                                 i8_case)


def test_small_slot_keeps_the_split(oracle, dev):
    torch.zeros(1, device=dev)
    hip = Hip()
    L = _lib.lib()
    d1, ref1 = i8_case(oracle, 1, 41000)
    C1 = torch.empty((1, N), dtype=torch.bfloat16, device=dev)
    print("[case] taking the large slots", flush=True)
    for _ in range(_lib.SPLIT_SLOTS):
        if L.fke_split_slots_in_use() >= _lib.SPLIT_SLOTS:
            break
        s = hip.stream()
        i8_call(L, d1, C1, s)  # M = 1 with B [K,N]: the row kernel's split takes the stream's slot
        hip.ok(hip.h.hipStreamSynchronize(s), "hipStreamSynchronize")
    used = L.fke_split_slots_in_use()
    assert _lib.SPLIT_SLOTS <= used < _lib.SPLIT_SLOTS + _lib.SPLIT_SMALL_SLOTS, used
    assert_same(host(C1), ref1, "M = 1 on the last large slot")

    # M = 16 needs 2 * 16 * N * 4 bytes (1.75 MiB at N = 14336): it fits a small slot
    M16 = 16
    need = L.fke_qgemm_workspace_size(M16, N, 4096, _lib.B_KN)
    assert 0 < need <= _lib.SPLIT_SMALL_SLOT_BYTES, need
    print("[case] capture on a small slot, M = 16", flush=True)
    d, ref = i8_case(oracle, M16, 42000)
    C = torch.empty((M16, N), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    s = hip.stream()
    g = hip.capture(s, lambda st: i8_call(L, d, C, st))
    assert L.fke_split_slots_in_use() == used + 1, "the capture did not take a small slot"
    assert hip.node_types(g) == [GRAPH_NODE_KERNEL] * 2, hip.node_types(g)  # the split and its sum
    e = hip.instantiate(g)
    for r in range(3):
        C.zero_()
        torch.cuda.synchronize()
        hip.replay(e, s)
        assert_same(host(C), ref, f"replay {r} on a small slot")
    C.zero_()
    torch.cuda.synchronize()
    i8_call(L, d, C, s)
    hip.ok(hip.h.hipStreamSynchronize(s), "hipStreamSynchronize")
    assert_same(host(C), ref, "eager on the small slot")
    assert L.fke_split_slots_in_use() == used + 1
