"""ctypes binding of libzkie_hip.so (the C ABI declared in include/zkie_hip.h).

The shared library is the product: there is no CPU fallback. Loading fails
loudly when the library has not been built or no HIP device is usable.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libzkie_hip.so")

_u64p = ctypes.POINTER(ctypes.c_uint64)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p
_u64, _u32, _int, _sz = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t

# name: (argtypes); every function returns int except zkie_device_count (int too)
SIGNATURES = {
    "zkie_device_count": [],
    "zkie_dev_alloc": [ctypes.POINTER(_vp), _sz],
    "zkie_dev_free": [_vp],
    "zkie_memcpy_htod": [_vp, _vp, _sz],
    "zkie_memcpy_dtoh": [_vp, _vp, _sz],
    "zkie_memcpy_dtod": [_vp, _vp, _sz, _vp],
    "zkie_memset": [_vp, _int, _sz],
    "zkie_device_synchronize": [],
    "zkie_stream_synchronize": [_vp],
    "zkie_stream_create": [ctypes.POINTER(_vp)],
    "zkie_stream_destroy": [_vp],
    "zkie_stream_wait": [_vp, _vp],
    "zkie_ntt_forward_goldilocks": [_vp, _vp, _u32, _u64, _vp],
    "zkie_p2_upload_constants": [_u64p, _u64p, _u64p, _u64],
    "zkie_p2_leaf_batch": [_vp, _vp, _u32, _u32],
    "zkie_p2_leaf_scalar": [_vp, _vp, _u32, _u32, _u32],
    "zkie_p2_compress_batch": [_vp, _vp, _u32, _u32],
    "zkie_p2_compress_scalar": [_vp, _vp, _u32, _u32, _u32],
    "zkie_p2_default_constants": [_u64p, _u64p, _u64p, _u64p],
    "zkie_dft_batch": [_vp, _u32, _u64, _vp],
    "zkie_idft_batch": [_vp, _u32, _u64, _vp],
    "zkie_lde_batch": [_vp, _u64, _u64, _u32, _u64, _vp, _vp],
    "zkie_lde_batch_noalloc": [_vp, _u64, _u64, _u32, _u64, _vp, _vp],
    "zkie_merkle_layout": [_u64, _u32p, _u64p],
    "zkie_merkle_commit": [_vp, _u64, _u64, _vp, _u64p, _vp],
    "zkie_lde_commit": [_vp, _u64, _u64, _u32, _u64, _vp, _vp, _u64p, _vp],
    "zkie_commit_batch": [_u64p, _u32, _u32, _u32, _u32, _vp, _vp, _vp, _u64p, _vp],
    "zkie_merkle_open_batch": [_vp, _u64, _u64, _vp, _u64p, _u64, _u64p, _u64p, _vp],
    "zkie_merkle_open_pruned": [_vp, _u64, _u64, _vp, _u64p, _u64, _u64p, _u64p, _u64, _u64p, _vp],
    "zkie_fold_rows": [_vp, _u64, _u32, _int, _u64p, _vp, _vp],
    "zkie_fold_rows_at": [_vp, _u64, _u32, _int, _u64p, _u64, _u64p, _u64p, _vp],
    "zkie_mle_eval": [_vp, _u32, _int, _u64p, _u64p, _vp],
    "zkie_whir_encode": [_vp, _u32, _int, _u32, _u32, _int, _vp, _vp],
    "zkie_sumcheck_round": [_vp, _int, _vp, _u32, _u64p, _vp],
    "zkie_eq_table": [_u64p, _u32, _vp, _vp],
    "zkie_constraint_weights": [_u64p, _u32, _u64p, _u32, _u64p, _u32, _int, _vp, _vp],
    "zkie_sumcheck_fold": [_vp, _int, _vp, _u32, _u64p, _vp, _vp, _u64p, _vp],
    "zkie_sumcheck_prove": [_vp, _int, _vp, _u32, _u32, _u64p, _u64p, _vp, _vp, _vp],
    "zkie_prover_data_size": [_u64, _u64, _u64p],
    "zkie_prover_data_write": [_vp, _u64, _u64, _vp, _vp, _vp, _vp],
    "zkie_prover_data_read": [_vp, _vp, _u64, _u64, _vp, _vp, _u64p, _vp],
    "zkie_gen_inputs": [_u64, _u64, _int, _u64p],
    "zkie_profile_enable": [_int],
    "zkie_profile_reset": [],
    "zkie_profile_query": [ctypes.c_char_p, _u64p, ctypes.POINTER(ctypes.c_double)],
    "zkie_profile_names": [ctypes.c_char_p, _sz],
}

_lib = None


class ZkieError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load the library (no fallback: raises if it is missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise ImportError(
                f"{path} is missing: build it with `python -m zkie_amd.build` "
                "(the HIP library is required; there is no CPU path)")
        L = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _int
        _lib = L
    return _lib


def check(rc: int, what: str):
    if rc != 0:
        raise ZkieError(f"{what} failed with status {rc}")


def p(a: np.ndarray):
    assert a.dtype == np.uint64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_u64p)


class DeviceBuffer:
    """A device allocation of u64 elements owned by this object."""

    def __init__(self, n_elems: int):
        self.n = int(n_elems)
        self.ptr = _vp()
        check(load().zkie_dev_alloc(ctypes.byref(self.ptr), max(self.n, 1) * 8), "zkie_dev_alloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a, dtype=np.uint64)
        b = cls(a.size)
        b.upload(a)
        return b

    @property
    def addr(self) -> int:
        return self.ptr.value or 0

    def upload(self, a: np.ndarray, offset_elems: int = 0):
        a = np.ascontiguousarray(a, dtype=np.uint64)
        assert offset_elems + a.size <= self.n
        check(load().zkie_memcpy_htod(self.addr + 8 * offset_elems, a.ctypes.data, a.size * 8),
              "zkie_memcpy_htod")

    def download(self, n: int | None = None, offset_elems: int = 0) -> np.ndarray:
        n = self.n - offset_elems if n is None else n
        assert offset_elems + n <= self.n
        out = np.empty(n, np.uint64)
        check(load().zkie_memcpy_dtoh(out.ctypes.data, self.addr + 8 * offset_elems, n * 8),
              "zkie_memcpy_dtoh")
        return out

    def free(self):
        if self.ptr is not None and self.ptr.value:
            load().zkie_dev_free(self.ptr)
            self.ptr = _vp()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_count() -> int:
    return load().zkie_device_count()


def p2_default_constants():
    a, b, c, d = (np.zeros(64, np.uint64), np.zeros(64, np.uint64), np.zeros(22, np.uint64),
                  np.zeros(1, np.uint64))
    check(load().zkie_p2_default_constants(p(a), p(b), p(c), p(d)), "zkie_p2_default_constants")
    return a, b, c, int(d[0])


def merkle_layout(h: int):
    nl = ctypes.c_uint32()
    lens = np.zeros(65, np.uint64)
    check(load().zkie_merkle_layout(h, ctypes.byref(nl), p(lens)), "zkie_merkle_layout")
    return [int(x) for x in lens[: nl.value]]


# zkie_write_fn / zkie_read_fn: int (*)(void* ctx, void* bytes, uint64_t len)
IO_FN = ctypes.CFUNCTYPE(_int, _vp, _vp, _u64)


def prover_data_size(h: int, w: int) -> int:
    n = ctypes.c_uint64()
    check(load().zkie_prover_data_size(h, w, ctypes.byref(n)), "zkie_prover_data_size")
    return int(n.value)


def _view(ptr: int, n: int) -> memoryview:
    return memoryview((ctypes.c_char * n).from_address(ptr)).cast("B")


def prover_data_write(d_mat: int, h: int, w: int, d_layers: int, sink, stream=None) -> None:
    """Stream the prover data to sink(view) piece by piece; each view is only
    valid during its call. An exception raised by sink propagates."""
    err = []

    def cb(_ctx, ptr, n):
        try:
            sink(_view(ptr, n))
            return 0
        except BaseException as e:  # noqa: BLE001 - re-raised below
            err.append(e)
            return 1

    fn = IO_FN(cb)
    rc = load().zkie_prover_data_write(d_mat, h, w, d_layers, ctypes.cast(fn, _vp), None, stream)
    if err:
        raise err[0]
    check(rc, "zkie_prover_data_write")


def prover_data_read(source, h: int, w: int, d_mat: int, d_layers: int, stream=None) -> np.ndarray:
    """Fill the device matrix and layers from source(view), which must fill the
    whole view (a short fill or an exception stops the call). Returns the root."""
    err = []

    def cb(_ctx, ptr, n):
        try:
            source(_view(ptr, n))
            return 0
        except BaseException as e:  # noqa: BLE001 - re-raised below
            err.append(e)
            return 1

    fn = IO_FN(cb)
    root = np.zeros(8, np.uint64)
    rc = load().zkie_prover_data_read(ctypes.cast(fn, _vp), None, h, w, d_mat, d_layers, p(root),
                                      stream)
    if err:
        raise err[0]
    check(rc, "zkie_prover_data_read")
    return root


GEN_UNIFORM, GEN_I16, GEN_I8, GEN_GAUSS_I16 = 0, 1, 2, 3


def gen_inputs(seed: int, n: int, kind: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    check(load().zkie_gen_inputs(seed, n, kind, p(out)), "zkie_gen_inputs")
    return out


def profile_enable(on: bool = True):
    check(load().zkie_profile_enable(1 if on else 0), "zkie_profile_enable")


def profile_reset():
    check(load().zkie_profile_reset(), "zkie_profile_reset")


def profile_query(kernel: str):
    n = ctypes.c_uint64()
    ms = ctypes.c_double()
    check(load().zkie_profile_query(kernel.encode(), ctypes.byref(n), ctypes.byref(ms)),
          "zkie_profile_query")
    return int(n.value), float(ms.value)


def profile_names():
    buf = ctypes.create_string_buffer(1 << 16)
    check(load().zkie_profile_names(buf, len(buf)), "zkie_profile_names")
    return [x for x in buf.value.decode().split("\n") if x]


class Stream:
    """A non-blocking HIP stream of the default priority owned by this object."""

    def __init__(self):
        self.ptr = _vp()
        check(load().zkie_stream_create(ctypes.byref(self.ptr)), "zkie_stream_create")

    @property
    def handle(self):
        return self.ptr.value

    def wait(self, other: "Stream") -> None:
        """Later work on self waits for the work queued on `other` so far."""
        check(load().zkie_stream_wait(self.handle, other.handle), "zkie_stream_wait")

    def synchronize(self) -> None:
        check(load().zkie_stream_synchronize(self.handle), "zkie_stream_synchronize")

    def __del__(self):
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            load().zkie_stream_destroy(self.ptr)
            self.ptr = _vp()
