"""Host-side pieces of bench.py that a GPU run depends on: the tile names it
prints cover every pinned MFMA tile path of the C ABI, and the kernel label of
each batch line resolves for every batch size the dispatcher takes (host-only
dispatch queries, no GPU)."""
import os
import re
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "flash-kernel-engine_amd"))

import bench  # noqa: E402
from flash_engine import _lib  # noqa: E402


def test_tile_labels_cover_every_pinned_tile_path():
    hdr = open(os.path.join(REPO, "include", "fke_qgemm.h")).read()
    values = {int(v) for v in re.findall(r"FKE_PATH_MFMA_\w+\s*=\s*(\d+)", hdr)}
    assert values and values == set(bench.TILE_LABELS)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 4096), (1792, 4096), (14336, 14336)])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_batch_kernel_label_for_every_m(N, K, layout):
    L = _lib.lib()
    for M in range(1, 513):
        label = bench.gemv_kernel(L, _lib, M, N, K, layout)
        assert label.startswith(("gemv_rows_kernel", "gemv_lds_kernel", "gemv_kn_split_kernel", "gemv_kn_row_kernel",
                                 f"gemm_mfma_kernel<i8,{layout.upper()},bf16,"))
        assert label.startswith("gemv_kn_row_kernel") == (layout == "kn" and M == 1)
        assert (label.startswith("gemv_kn") or label.startswith("gemm_mfma")) if layout == "kn" else True
