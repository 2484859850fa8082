"""Loader of the torch extension `flash_engine_cuda` (csrc/torch_ext.cpp), the
binding in the idiom of reference python/bindings.cpp under the module name the
reference builds and imports (setup.py:51, python/flash_engine/ops.py:9-13).
It is built in-tree by csrc/build_torch_ext.py into
flash-kernel-engine_amd/flash_engine_cuda.so, beside this package, so `import
flash_engine_cuda` finds it wherever `flash_engine` is importable; loading fails
loudly when it has not been built.
"""
from __future__ import annotations

import importlib.util
import os
import sys

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXT_PATH = os.path.join(_PKG, "flash_engine_cuda.so")
NAME = "flash_engine_cuda"

_mod = None


def ext():
    """The loaded extension module (import torch first; it links against it)."""
    global _mod
    if _mod is None:
        import torch  # noqa: F401  (the extension's torch symbols come from here)

        mod = sys.modules.get(NAME)
        if mod is None:
            if not os.path.exists(EXT_PATH):
                raise ImportError(f"{NAME} not built at {EXT_PATH}; run __graft_entry__.build() or "
                                  "python flash-kernel-engine_amd/csrc/build_torch_ext.py")
            spec = importlib.util.spec_from_file_location(NAME, EXT_PATH)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            sys.modules[NAME] = mod
        _mod = mod
    return _mod
