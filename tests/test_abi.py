"""The C ABI library loads and exports every entry point include/zkie_hip.h
declares (no compute calls: runs without a GPU)."""
import ctypes
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zkie_hip.h")
LIB = os.path.join(ROOT, "zkie_amd", "libzkie_hip.so")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\bint\s+(zkie_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    for must in ("zkie_ntt_forward_goldilocks", "zkie_p2_upload_constants", "zkie_p2_leaf_batch",
                 "zkie_p2_leaf_scalar", "zkie_p2_compress_batch", "zkie_p2_compress_scalar",
                 "zkie_lde_batch", "zkie_merkle_commit", "zkie_merkle_open_batch",
                 "zkie_merkle_open_pruned", "zkie_fold_rows", "zkie_dft_batch"):
        assert must in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build with python -m zkie_amd.build"
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (zkie_\w+)", out))
    assert set(declared_symbols()) <= exported


def test_python_binding_covers_header():
    from zkie_amd import _native as N

    assert set(declared_symbols()) == set(N.SIGNATURES)


def test_no_cpu_fallback_in_product():
    # The product package never imports the oracle.
    for dirpath, _, files in os.walk(os.path.join(ROOT, "zkie_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in src.replace("oracle/", ""), f
