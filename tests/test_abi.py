"""The C-ABI library loads and exports every entry point include/fa_mi355x.h
declares (CPU only: no compute calls), and argument errors come back as codes."""

import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fa_mi355x.h")
LIB = os.path.join(REPO, "flash-attention-turing_amd", "libfa_mi355x.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_]+\s*\*?\s*(fa_[a-z0-9_]+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (HIP runtime first, as in every product import)

    assert os.path.exists(LIB), "libfa_mi355x.so is not built (python __graft_entry__.py / build.py)"
    return ctypes.CDLL(LIB)


def test_header_declares_the_abi():
    names = declared_functions()
    for required in ("fa_fwd", "fa_bwd_preprocess", "fa_bwd_dq", "fa_bwd_dkdv", "fa_bwd", "fa_kv_append",
                     "fa_kv_splitkv", "fa_kv_combine", "fa_fwd_kvcache", "fa_kv_num_splits",
                     "fa_kv_workspace_bytes", "fa_error_string"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in fa_mi355x.h but not exported"


def test_abi_version_matches_the_header(lib):
    want = int(re.search(r"#define FA_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    lib.fa_abi_version.restype = ctypes.c_int
    assert lib.fa_abi_version() == want
    import fa_capi

    assert fa_capi.ABI_VERSION == want, "fa_capi.py's struct mirrors are for another layout version"


def test_argument_errors_are_codes(lib):
    lib.fa_error_string.restype = ctypes.c_char_p
    assert lib.fa_fwd(None, None) == -1
    assert lib.fa_bwd(None, None) == -1
    assert lib.fa_fwd_kvcache(None, None) == -1
    assert b"invalid argument" in lib.fa_error_string(-1)
    assert b"head_dim" in lib.fa_error_string(-2)


def test_num_splits_heuristic(lib):
    f = lib.fa_kv_num_splits
    assert f(7, 100000, 128, 1, 64, 32, 8, 256) == 7  # explicit requests are kept
    assert f(0, 256, 128, 1, 1, 8, 8, 256) == 1  # too short to split
    s = f(0, 32768, 128, 1, 4, 32, 8, 256)
    assert 1 < s <= 64
    assert f(0, 1 << 20, 128, 1, 1, 8, 1, 256) <= 128
    # The split counts measured best on MI355X (256 CUs) for these decode shapes:
    # (capacity, head_dim, seqlen_q, batch, heads, kv heads) -> splits
    measured_best = {
        (32768 + 256, 128, 1, 64, 32, 8): 4,   # c4: paged, lengths 1k-32k
        (32768 + 256, 128, 1, 8, 32, 8): 4,    # 8 x 32k
        (131072 + 256, 128, 1, 1, 32, 8): 32,  # 1 x 128k
        (131072, 64, 4, 4, 16, 16): 16,        # c5: 4 query tokens, 65k-131k
        (8192, 128, 1, 16, 32, 8): 2,          # 16 x 8k
        (2048, 128, 1, 1, 32, 8): 16,          # short caches on few sequences: down to 64-128 positions
        (1024, 128, 1, 1, 32, 8): 16,
        (512, 128, 1, 1, 32, 8): 8,
        (2048, 128, 1, 4, 32, 8): 8,
    }
    for (cap, d, sq, b, h, hk), best in measured_best.items():
        assert f(0, cap, d, sq, b, h, hk, 256) == best
    assert f(0, 4096, 128, 1, 256, 32, 8, 256) == 1  # large batches fill the chip unsplit


def test_ctypes_structs_match_the_c_layout(tmp_path):
    """fa_capi's ctypes structs have the size and field offsets gcc gives the
    structs of include/fa_mi355x.h (a mismatch would pass garbage to kernels)."""
    import shutil
    import subprocess

    import fa_capi

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    structs = {"fa_tensor": fa_capi.FaTensor, "fa_fwd_args": fa_capi.FaFwdArgs, "fa_bwd_args": fa_capi.FaBwdArgs,
               "fa_kvcache_args": fa_capi.FaKvcacheArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "fa_mi355x.h"', "int main(void) {"]
    for cname, st in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in st._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, got):
        cname, field, value = line.split()
        st = structs[cname]
        expect = ctypes.sizeof(st) if field == "size" else getattr(st, field).offset
        assert int(value) == expect, f"{cname}.{field}: C {value} vs ctypes {expect}"


def test_c_program_links_the_library(tmp_path):
    """A plain C caller: compiled against include/fa_mi355x.h with gcc, linked
    with -lfa_mi355x, it calls the host-only entry points (argument checks,
    sizes, the split heuristic, error texts) with no GPU work."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    src = tmp_path / "caller.c"
    src.write_text(r"""
#include <stdio.h>
#include <string.h>
#include "fa_mi355x.h"
int main(void) {
    fa_kvcache_args kv;
    memset(&kv, 0, sizeof kv);
    kv.batch = 2; kv.seqlen_q = 20; kv.nheads = 4; kv.nheads_k = 2; kv.head_dim = 128; kv.num_splits = 3;
    printf("%d %d %d\n", fa_fwd(NULL, NULL), fa_bwd(NULL, NULL), fa_fwd_kvcache(NULL, NULL));
    printf("%zu %zu\n", fa_kv_workspace_bytes(&kv), fa_kv_split_count_len(&kv));
    printf("%d\n", fa_kv_num_splits(0, 32768 + 256, 128, 1, 64, 32, 8, 256));
    printf("%s\n", fa_error_string(FA_ERR_WORKSPACE));
    return 0;
}
""")
    exe = tmp_path / "caller"
    libdir = os.path.dirname(LIB)
    rocm_lib = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe), f"-L{libdir}",
                    "-lfa_mi355x", f"-Wl,-rpath,{libdir}", f"-Wl,-rpath,{rocm_lib}"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    assert out[0].split() == ["-1", "-1", "-1"]
    assert out[1].split() == [str(3 * 2 * 4 * 20 * 129 * 4), str(2 * 2 * 2)]
    assert out[2] == "4"
    assert "workspace" in out[3]


def _capi():
    import sys

    sys.path.insert(0, os.path.join(REPO, "flash-attention-turing_amd"))
    import fa_capi

    return fa_capi


def test_validation_errors_before_any_launch(lib):
    # Each entry point checks its arguments before touching the device, so
    # these calls return codes on a machine without a GPU.  Pointers are fake
    # but 16-byte aligned; nothing is dereferenced.
    fa_capi = _capi()
    T = fa_capi.FaTensor
    P = 1 << 20  # an aligned fake device address

    def tensor(ptr=P, rs=1024, hs=128):
        return T(ptr, 0, rs, hs)

    f = fa_capi.FaFwdArgs()
    f.q = f.k = f.v = f.o = tensor()
    f.lse = P
    f.batch, f.seqlen_q, f.seqlen_k, f.nheads, f.nheads_k, f.head_dim, f.lse_seqlen = 1, 8, 8, 4, 2, 96, 8
    fwd = lib.fa_fwd
    fwd.argtypes = [ctypes.POINTER(fa_capi.FaFwdArgs), ctypes.c_void_p]
    assert fwd(ctypes.byref(f), None) == -2  # head_dim 96: unsupported
    f.head_dim, f.nheads_k = 128, 3
    assert fwd(ctypes.byref(f), None) == -1  # 4 q-heads over 3 kv heads
    f.nheads_k, f.lse_seqlen = 2, 4
    assert fwd(ctypes.byref(f), None) == -1  # LSE rows shorter than seqlen_q
    f.lse_seqlen = 8
    f.q = tensor(P + 8)
    assert fwd(ctypes.byref(f), None) == -1  # q not 16-byte aligned
    f.q = tensor(rs=1020)
    assert fwd(ctypes.byref(f), None) == -1  # row stride not a multiple of 8 elements

    kv = fa_capi.FaKvcacheArgs()
    kv.q = kv.k_cache = kv.v_cache = kv.o = tensor()
    kv.lse = kv.cache_seqlens = P
    kv.batch, kv.seqlen_q, kv.nheads, kv.nheads_k, kv.head_dim = 2, 1, 4, 2, 128
    kv.num_splits = 4  # needs the split accumulators
    split = lib.fa_kv_splitkv
    split.argtypes = [ctypes.POINTER(fa_capi.FaKvcacheArgs), ctypes.c_void_p]
    assert split(ctypes.byref(kv), None) == -3
    kv.out_accum, kv.lse_accum = P + 4, P  # 4-byte aligned accumulators: the combine reads 64-bit words
    assert split(ctypes.byref(kv), None) == -1
    kv.out_accum = kv.lse_accum = None
    kv.num_splits = 0
    assert split(ctypes.byref(kv), None) == -1  # num_splits must be >= 1 here
    kv.num_splits, kv.block_table, kv.page_block_size = 1, P, 100
    assert split(ctypes.byref(kv), None) == -1  # page size not a multiple of the 32-key tile
    kv.page_block_size, kv.cache_batch_idx = 256, P
    assert split(ctypes.byref(kv), None) == -1  # paged and remapped at once
    ws = lib.fa_kv_workspace_bytes
    ws.argtypes = [ctypes.POINTER(fa_capi.FaKvcacheArgs)]
    ws.restype = ctypes.c_size_t
    kv.num_splits = 3
    assert ws(ctypes.byref(kv)) == 3 * 2 * 4 * 1 * (128 + 1) * 4
    kv.num_splits = 1
    assert ws(ctypes.byref(kv)) == 0
    # Split counts: one per (batch, kv head, 32-row tile of the GQA group x query rows), with splits only.
    cl = lib.fa_kv_split_count_len
    cl.argtypes = [ctypes.POINTER(fa_capi.FaKvcacheArgs)]
    cl.restype = ctypes.c_size_t
    assert cl(ctypes.byref(kv)) == 0
    kv.num_splits = 3
    assert cl(ctypes.byref(kv)) == 2 * 2 * 1
    kv.seqlen_q = 20  # 2 q-heads per kv head x 20 rows = 40 rows: two tiles
    assert cl(ctypes.byref(kv)) == 2 * 2 * 2
    kv.seqlen_q, kv.num_splits = 1, 1
    # Rotary: rotary_dim a multiple of 16 up to head_dim, both aligned tables,
    # at least one row, and new keys to rotate.
    kv.block_table, kv.page_block_size, kv.cache_batch_idx = None, 0, None
    kv.rotary_cos = kv.rotary_sin = P
    kv.rotary_dim, kv.rotary_seqlen = 64, 16
    assert split(ctypes.byref(kv), None) == -1  # no k_new
    kv.k_new = kv.v_new = tensor()
    kv.rotary_dim = 40
    assert split(ctypes.byref(kv), None) == -1  # not a multiple of 16
    kv.rotary_dim = 144
    assert split(ctypes.byref(kv), None) == -1  # wider than head_dim
    kv.rotary_dim, kv.rotary_sin = 64, P + 8
    assert split(ctypes.byref(kv), None) == -1  # misaligned sin table
    kv.rotary_sin, kv.rotary_seqlen = P, 0
    assert split(ctypes.byref(kv), None) == -1  # empty table
