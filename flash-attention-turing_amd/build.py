"""Build the MI355X FlashAttention library and its PyTorch extension in-tree.

Outputs (next to this file):
  * libfa_mi355x.so   - the HIP kernels behind the C ABI of include/fa_mi355x.h
                        (hipcc --offload-arch=gfx950)
  * flash_attn_turing.<ext>.so - the Python extension module (host layer)
  * probes/ceiling_probe - the hardware-ceiling probe (MFMA rate and clock, LDS
                        instruction costs, HBM read rates) behind the rooflines

Usage:  python build.py [--jobs N]
"""

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

KERNEL_SOURCES = ["fa_abi.hip", "fa_fwd.hip", "fa_bwd.hip", "fa_kvcache.hip"]
LIB_NAME = "libfa_mi355x.so"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    # Packed fp32 VALU ops stay off (they have given wrong results on this pool).
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# Per-source additions to HIP_FLAGS (none at present).
FILE_FLAGS = {}


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_library(jobs: int, out_dir: str = HERE, obj_dir: str = None) -> str:
    objdir = obj_dir or os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = []

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, KERNEL_SOURCES))
    lib = os.path.join(out_dir, LIB_NAME)
    tmp = lib + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, lib)
    return lib


def build_extension(out_dir: str = HERE) -> str:
    """Link the extension against the libfa_mi355x.so already built in out_dir;
    it finds that library at run time next to itself (rpath $ORIGIN)."""
    import torch
    from torch.utils import cpp_extension

    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(out_dir, "flash_attn_turing" + ext_suffix)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = cpp_extension.include_paths() + [sysconfig.get_paths()["include"], f"{ROCM}/include", INCLUDE]
    libdirs = cpp_extension.library_paths()
    cmd = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=flash_attn_turing",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        *[f"-I{p}" for p in incs],
        os.path.join(CSRC, "flash_api.cpp"),
        "-o",
        out + ".tmp",
        *[f"-L{p}" for p in libdirs],
        f"-L{out_dir}",
        "-lfa_mi355x",
        "-lc10",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_python",
        "-lc10_hip",
        "-ltorch_hip",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        *[f"-Wl,-rpath,{p}" for p in libdirs],
    ]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build_probe() -> str:
    src = os.path.join(HERE, "probes", "ceiling_probe.hip")
    out = os.path.join(HERE, "probes", "ceiling_probe")
    _run([HIPCC, *HIP_FLAGS, src, "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build(jobs: int = 4) -> None:
    build_library(jobs)
    build_extension()
    build_probe()


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--lib-only", action="store_true")
    args = ap.parse_args()
    print("built", build_library(args.jobs))
    if not args.lib_only:
        print("built", build_extension())
        print("built", build_probe())
    sys.exit(0)
