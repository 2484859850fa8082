"""Build step of the torch extension `flash_engine_cuda` (csrc/torch_ext.cpp).

The module keeps the name the reference builds (setup.py:51, CUDAExtension
"flash_engine_cuda") and imports (python/flash_engine/ops.py:9-13), so a
caller written against the reference finds it by that name.  Compiles the
binding with torch.utils.cpp_extension (host C++ only: it calls the C ABI of
libfke_qgemm.so, which `make -C flash-kernel-engine_amd/csrc` builds first) and
places it at flash-kernel-engine_amd/flash_engine_cuda.so, beside the
flash_engine package as a setup.py install would, with an rpath to lib/.
"""
from __future__ import annotations

import os
import shutil

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
REPO = os.path.dirname(PKG)
LIB_DIR = os.path.join(PKG, "lib")
OUT = os.path.join(PKG, "flash_engine_cuda.so")


def build(verbose: bool = False) -> str:
    from torch.utils import cpp_extension

    bdir = os.path.join(PKG, "_build", "torch_ext")
    os.makedirs(bdir, exist_ok=True)
    mod = cpp_extension.load(
        name="flash_engine_cuda",
        sources=[os.path.join(HERE, "torch_ext.cpp")],
        extra_include_paths=[os.path.join(REPO, "include"), "/opt/rocm/include"],
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__"],
        # $ORIGIN: ninja unescapes $$ and the shell must not expand the rest
        extra_ldflags=[f"-L{LIB_DIR}", "-lfke_qgemm", "-L/opt/rocm/lib", "-lamdhip64", "-lc10_hip",
                       "-Wl,-rpath,\\$$ORIGIN/lib", f"-Wl,-rpath,{LIB_DIR}"],
        build_directory=bdir,
        with_cuda=False,
        verbose=verbose,
    )
    shutil.copy2(mod.__file__, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
