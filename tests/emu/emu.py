"""Loader of the host emulation of the device code (test infrastructure)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libzkie_emu.so")
SRC = os.path.join(HERE, "emu.cpp")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
_u64, _u64p = ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)
_lib = None


def build() -> str:
    deps = [SRC] + [os.path.join(HERE, "..", "..", "zkie_amd", "csrc", f)
                    for f in ("gl64.hpp", "poseidon2.hpp", "ntt_pass.hpp", "ntt_plan.hpp", "last_leaf.hpp")]
    if os.path.exists(LIB) and all(os.path.getmtime(LIB) >= os.path.getmtime(d) for d in deps):
        return LIB
    cmd = [HIPCC, "--offload-host-only", "-O2", "-fPIC", "-shared", "-std=c++17",
           "-DZK_LIMB_MUL_ON_HOST", "-DZK_EMU_BOUNDS", SRC, "-o", LIB]
    subprocess.run(cmd, check=True, capture_output=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(build())
        for n in ("emu_gl_add", "emu_gl_sub", "emu_gl_mul"):
            getattr(L, n).restype = _u64
            getattr(L, n).argtypes = [_u64, _u64]
        for n in ("emu_gl_add_small",):
            getattr(L, n).restype = _u64
            getattr(L, n).argtypes = [_u64, _u64]
        L.emu_gl_shl.restype = _u64
        L.emu_gl_shl.argtypes = [_u64, ctypes.c_int]
        L.emu_gl_add_shl.restype = _u64
        L.emu_gl_add_shl.argtypes = [_u64, _u64, ctypes.c_int]
        for n in ("emu_gl_sqr", "emu_gl_halve", "emu_gl_canon", "emu_gl_canon_fast"):
            getattr(L, n).restype = _u64
            getattr(L, n).argtypes = [_u64]
        L.emu_gl_inv_pow2.restype = _u64
        L.emu_gl_inv_pow2.argtypes = [_u64, ctypes.c_int]
        L.emu_dot.restype = _u64
        L.emu_dot.argtypes = [_u64p, _u64p, _u64]
        L.emu_acc_sum.restype = _u64
        L.emu_acc_sum.argtypes = [_u64p, _u64]
        L.emu_p2_permute.argtypes = [_u64p, _u64p, _u64p, _u64p, _u64, ctypes.c_int]
        L.emu_p2_internal_round.argtypes = [_u64p, _u64, _u64, ctypes.c_int]
        L.emu_p2_mds_light.argtypes = [_u64p]
        L.emu_dft.argtypes = [_u64p, ctypes.c_uint32, _u64, ctypes.c_int, ctypes.c_uint32]
        L.emu_dft.restype = ctypes.c_int
        L.emu_lde.argtypes = [_u64p, _u64, _u64, ctypes.c_uint32, _u64p, ctypes.c_uint32]
        L.emu_lde.restype = ctypes.c_int
        L.emu_lde_rows.argtypes = [_u64p, _u64, _u64, _u64, ctypes.c_uint32, _u64p, ctypes.c_uint32]
        L.emu_lde_rows.restype = ctypes.c_int
        L.emu_prefix_source.argtypes = [_u64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.emu_prefix_source.restype = _u64
        L.emu_lde_leaf.argtypes = [_u64p, _u64, _u64, ctypes.c_uint32, _u64p, _u64p, _u64p, _u64p, _u64p,
                                   _u64, ctypes.c_int]
        L.emu_lde_leaf.restype = ctypes.c_int
        _lib = L
    return _lib


def ptr(a: np.ndarray):
    assert a.dtype == np.uint64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_u64p)
