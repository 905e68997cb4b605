"""``pip install .`` for the MI355X FlashAttention (counterpart of the reference's
setup.py:20-47, which builds the ``flash_attn_turing`` CUDA extension).

Builds, with hipcc for gfx950 and the flags of flash-attention-turing_amd/build.py:
  * libfa_mi355x.so   - the HIP kernels behind the C ABI of include/fa_mi355x.h;
  * flash_attn_turing - the PyTorch extension (host layer), linked against it;
and installs both as top-level modules next to ``flash_attention_interface``
(the reference's public Python API, imported the same way) and ``fa_capi``
(the ctypes binding of the C ABI).  The extension finds libfa_mi355x.so next
to itself (rpath $ORIGIN), and fa_capi loads it from its own directory.

There is no CUDA source, CUTLASS submodule or nvcc flag: the build needs only
ROCm (``ROCM_PATH``, default /opt/rocm) and PyTorch-ROCm.  Build in place
instead with ``python flash-attention-turing_amd/build.py``.
"""

import os
import sys

from setuptools import Extension, setup
from setuptools.command.build_ext import build_ext

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = "flash-attention-turing_amd"


class HipBuild(build_ext):
    """Builds the HIP library and the extension with build.py instead of
    setuptools' compiler driver (the kernels need hipcc and gfx950 flags)."""

    def build_extension(self, ext):
        sys.path.insert(0, os.path.join(HERE, PKG_DIR))
        import build as fa_build

        out_dir = os.path.dirname(os.path.abspath(self.get_ext_fullpath(ext.name)))
        os.makedirs(out_dir, exist_ok=True)
        jobs = int(os.environ.get("MAX_JOBS", "4"))
        fa_build.build_library(jobs, out_dir=out_dir, obj_dir=os.path.join(os.path.abspath(self.build_temp), "hip"))
        fa_build.build_extension(out_dir=out_dir)


setup(
    name="flash_attn_turing",
    version="0.1.0",
    description="FlashAttention forward, backward and KV-cache decode for AMD MI355X (gfx950)",
    package_dir={"": PKG_DIR},
    py_modules=["flash_attention_interface", "fa_capi"],
    # The sources list is informational: HipBuild compiles them with hipcc.
    ext_modules=[
        Extension(
            "flash_attn_turing",
            sources=[f"{PKG_DIR}/csrc/flash_api.cpp"]
            + [f"{PKG_DIR}/csrc/{f}" for f in ("fa_abi.hip", "fa_fwd.hip", "fa_bwd.hip", "fa_kvcache.hip")],
        )
    ],
    cmdclass={"build_ext": HipBuild},
    install_requires=["torch"],
    python_requires=">=3.10",
)
