"""zkie_lde_batch_noalloc (the LDE whose work buffers live in a fixed device
array of the library, for callers that cannot allocate) against
zkie_lde_batch and the oracle, bit for bit: two calls in a row, the second
with a smaller input, then a coset LDE on a stream; sizes beyond the fixed
array are refused before any device work."""
import numpy as np
import pytest

from zkie_amd._native import DeviceBuffer, check

pytestmark = pytest.mark.gpu

ZKIE_ERR_SCRATCH_LIMIT = -5


def _lde_both(native, x, h, w, lb, shift, stream=None):
    L = native.load()
    d_in = DeviceBuffer.from_array(x)
    d_ref, d_na = DeviceBuffer((h << lb) * w), DeviceBuffer((h << lb) * w)
    check(L.zkie_lde_batch(d_in.addr, h, w, lb, shift, d_ref.addr, stream), "zkie_lde_batch")
    check(L.zkie_lde_batch_noalloc(d_in.addr, h, w, lb, shift, d_na.addr, stream), "zkie_lde_batch_noalloc")
    check(L.zkie_device_synchronize(), "sync")
    return d_ref.download().reshape(h << lb, w), d_na.download().reshape(h << lb, w)


def test_noalloc_lde_matches_lde(native, oracle):
    # the first call fills the whole intermediate (n w = 2^23 u64, the
    # maximum); the second is smaller and uses a coset shift, so it reads
    # only what it wrote itself after the first call
    for h, w, lb, shift in [(1 << 17, 16, 2, 1), (1 << 10, 8, 2, 7)]:
        print("CASE noalloc lde", h, w, lb, shift, flush=True)
        x = oracle.gen_uniform(h + w + lb, h * w).reshape(h, w)
        ref, got = _lde_both(native, x, h, w, lb, shift)
        assert (got == ref).all(), (h, w, lb, shift)
        assert (got == oracle.lde_batch(x, lb, shift)).all(), (h, w, lb, shift)


def test_noalloc_lde_on_stream_and_single_pass(native, oracle):
    s = native.Stream()
    for h, w, lb, shift in [(1 << 14, 16, 3, 0xFEDCBA9876543210 % 0xFFFFFFFF00000001), (64, 4, 2, 1)]:
        print("CASE noalloc lde stream", h, w, lb, shift, flush=True)
        x = oracle.gen_uniform(h * 3 + w, h * w).reshape(h, w)
        ref, got = _lde_both(native, x, h, w, lb, shift, stream=s.handle)
        assert (got == ref).all(), (h, w, lb, shift)


def test_noalloc_lde_refuses_beyond_its_scratch(native):
    print("CASE noalloc lde limit", flush=True)
    L = native.load()
    d = DeviceBuffer(16)
    # (2^18 << 2) x 16 = 2^24 u64 > 2^23: refused before any device work
    assert L.zkie_lde_batch_noalloc(d.addr, 1 << 18, 16, 2, 1, d.addr, None) == ZKIE_ERR_SCRATCH_LIMIT
    assert L.zkie_lde_batch_noalloc(d.addr, 1 << 20, 1 << 10, 0, 1, d.addr, None) == ZKIE_ERR_SCRATCH_LIMIT
    assert L.zkie_lde_batch_noalloc(d.addr, 3, 16, 2, 1, d.addr, None) == -1  # height not a power of two
