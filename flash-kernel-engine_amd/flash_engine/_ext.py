"""Loader of the torch extension `flash_engine_hip` (csrc/torch_ext.cpp), the
binding in the idiom of reference python/bindings.cpp.  It is built in-tree
next to libfke_qgemm.so (flash-kernel-engine_amd/lib/flash_engine_hip.so) by
csrc/build_torch_ext.py; loading fails loudly when it has not been built.
"""
from __future__ import annotations

import importlib.util
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXT_PATH = os.path.join(_PKG, "lib", "flash_engine_hip.so")

_mod = None


def ext():
    """The loaded extension module (import torch first; it links against it)."""
    global _mod
    if _mod is None:
        import torch  # noqa: F401  (the extension's torch symbols come from here)

        if not os.path.exists(EXT_PATH):
            raise ImportError(f"flash_engine_hip not built at {EXT_PATH}; run __graft_entry__.build() or "
                              "python flash-kernel-engine_amd/csrc/build_torch_ext.py")
        spec = importlib.util.spec_from_file_location("flash_engine_hip", EXT_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _mod = mod
    return _mod
