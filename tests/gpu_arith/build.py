"""Build and load the device-arithmetic test kernels (tests/gpu_arith/arith.hip):
test infrastructure for the GPU tests, built for gfx950 beside the tests."""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libzkie_arith_test.so")
SRC = os.path.join(HERE, "arith.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
_u64, _u64p = ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)
_lib = None


def build() -> str:
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", SRC, "-o", LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC}:\n{r.stderr}")
    return LIB


def load():
    """The prebuilt library (built by __graft_entry__.build()); a missing one
    is an error, not a skip."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise FileNotFoundError(f"{LIB} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB)
        L.arith_ops.restype = ctypes.c_int
        L.arith_binary.argtypes = [_u64p, _u64p, _u64p, _u64]
        L.arith_binary.restype = ctypes.c_int
        L.arith_states.argtypes = [_u64p, _u64, ctypes.c_int, _u64, _u64p, _u64p, _u64]
        L.arith_states.restype = ctypes.c_int
        _lib = L
    return _lib
