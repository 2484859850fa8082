"""CPU sanitizer runs (tests/sanitize): the oracle under gcc's AddressSanitizer
and UndefinedBehaviorSanitizer (float-cast-overflow included), and the C ABI's
host code (validation, dispatch over shapes up to INT32_MAX, workspace sizing)
under clang's, without a GPU.  The binaries are built by
`make -C tests/sanitize` (part of __graft_entry__.build())."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "sanitize", "_build")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


@pytest.mark.parametrize("prog", ["oracle_san", "abi_san"])
def test_sanitizer_run_is_clean(prog):
    path = os.path.join(BUILD, prog)
    assert os.path.exists(path), f"{path} not built: make -C tests/sanitize (or __graft_entry__.build())"
    r = subprocess.run([path], capture_output=True, text=True, timeout=600, env=ENV)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "[PASS]" in r.stdout
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr
