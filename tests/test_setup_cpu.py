"""setup.py (the `pip install .` path): its metadata names the reference's module,
and every module and source it lists exists.  The compile itself is what
__graft_entry__.build() runs through the same build.py functions."""

import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _setup_query(*args):
    out = subprocess.run([sys.executable, "setup.py", *args], cwd=REPO, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return out.stdout.split()


def test_setup_metadata_names_the_reference_module():
    assert _setup_query("--name") == ["flash_attn_turing"]


def test_setup_lists_existing_modules_and_sources():
    import ast

    tree = ast.parse(open(os.path.join(REPO, "setup.py")).read())
    strings = {n.value for n in ast.walk(tree) if isinstance(n, ast.Constant) and isinstance(n.value, str)}
    pkg = os.path.join(REPO, "flash-attention-turing_amd")
    for mod in ("flash_attention_interface", "fa_capi"):
        assert mod in strings and os.path.isfile(os.path.join(pkg, mod + ".py"))
    for src in ("fa_abi.hip", "fa_fwd.hip", "fa_bwd.hip", "fa_kvcache.hip"):
        assert src in strings and os.path.isfile(os.path.join(pkg, "csrc", src))
    assert os.path.isfile(os.path.join(pkg, "csrc", "flash_api.cpp"))
