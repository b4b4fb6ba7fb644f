"""Loader of the CPU baseline of bench.py (oracle/cpu_baseline.c): a fast
AVX2/OpenMP port of the reference CPU commit path, timed beside the GPU.

TEST INFRASTRUCTURE ONLY: used by bench.py's cpu_baseline leg and by
tests/test_cpu_baseline.py, which proves it bit-identical to the oracle. The
product path never loads it."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libzkie_cpu_baseline.so")
_u64, _u64p, _u32 = ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64), ctypes.c_uint32
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            subprocess.run(["make", "-s", "-C", HERE, "libzkie_cpu_baseline.so"], check=True)
        L = ctypes.CDLL(LIB)
        L.cb_p2_set_constants.argtypes = [_u64p, _u64p, _u64p, _u64]
        L.cb_merkle_layer_lens.argtypes = [_u64, _u64p]
        L.cb_merkle_layer_lens.restype = _u32
        L.cb_merkle_commit.argtypes = [_u64p, _u64, _u64, _u64p, _u64p]
        L.cb_lde.argtypes = [_u64p, _u64, _u64, _u32, _u64p]
        L.cb_fold_rows.argtypes = [_u64p, _u64, _u32, _u64p, _u64p]
        L.cb_set_threads.argtypes = [ctypes.c_int]
        L.cb_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a):
    assert a.dtype == np.uint64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_u64p)


def set_constants(rc_init, rc_final, rc_internal, diag15):
    """Poseidon2 constants (layout of zkie_p2_upload_constants)."""
    a, b, c = (np.ascontiguousarray(x, np.uint64) for x in (rc_init, rc_final, rc_internal))
    lib().cb_p2_set_constants(_p(a), _p(b), _p(c), int(diag15))


def set_threads(n: int):
    lib().cb_set_threads(int(n))


def max_threads() -> int:
    return int(lib().cb_max_threads())


def lde_batch(mat: np.ndarray, log_blowup: int) -> np.ndarray:
    m = np.ascontiguousarray(mat, np.uint64)
    h, w = m.shape
    out = np.empty((h << log_blowup, w), np.uint64)
    lib().cb_lde(_p(m), h, w, log_blowup, _p(out))
    return out


def merkle_commit(mat: np.ndarray):
    """(list of layers as (len, 8) arrays, root)."""
    m = np.ascontiguousarray(mat, np.uint64)
    h, w = m.shape
    lens = np.zeros(66, np.uint64)
    nl = lib().cb_merkle_layer_lens(h, _p(lens))
    lens = [int(x) for x in lens[:nl]]
    layers = np.empty(sum(lens) * 8, np.uint64)
    root = np.empty(8, np.uint64)
    lib().cb_merkle_commit(_p(m), h, w, _p(layers), _p(root))
    out, off = [], 0
    for n in lens:
        out.append(layers[off * 8:(off + n) * 8].reshape(n, 8))
        off += n
    return out, root


def fold_rows(mat: np.ndarray, k: int, r) -> np.ndarray:
    """Row fold of base rows of 2^k entries with k EF challenges: (h, 2)."""
    m = np.ascontiguousarray(mat, np.uint64).reshape(-1, 1 << k)
    rr = np.ascontiguousarray(r, np.uint64).reshape(-1)
    out = np.empty((m.shape[0], 2), np.uint64)
    lib().cb_fold_rows(_p(m), m.shape[0], k, _p(rr), _p(out))
    return out
