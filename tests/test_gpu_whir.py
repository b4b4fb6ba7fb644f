"""GPU parity of the WHIR round pieces around the commitment (bit-exact
against the oracle): out-of-domain multilinear evaluation on the device
table, the queried-row fold, and commit_extension's encoding in both
variable orders."""
import numpy as np
import pytest

P = 0xFFFFFFFF00000001
pytestmark = pytest.mark.gpu


def _r(oracle, seed, t):
    return (oracle.gen_uniform(seed, 2 * t) % np.uint64(P)).reshape(t, 2)


@pytest.mark.parametrize("is_ext", [False, True])
@pytest.mark.parametrize("t", [0, 1, 5, 6, 7, 12, 13, 18])
def test_mle_eval_matches_oracle(native, oracle, is_ext, t):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE mle_eval t={t} ext={is_ext}", flush=True)
    E = 2 if is_ext else 1
    vals = oracle.gen_uniform(100 + t, E << t)
    r = _r(oracle, 200 + t, t)
    got = pcs.mle_eval(DeviceBuffer.from_array(vals), t, is_ext, r)
    want = oracle.mle_eval(vals, r, is_ext) if t else (
        np.array([vals[0], vals[1] if is_ext else 0], np.uint64))
    assert (got == want).all()


@pytest.mark.parametrize("is_ext", [False, True])
@pytest.mark.parametrize("k", [1, 3, 4, 5])
def test_fold_rows_at_matches_oracle(native, oracle, is_ext, k):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE fold_rows_at k={k} ext={is_ext}", flush=True)
    h = 3000
    E = 2 if is_ext else 1
    mat = oracle.gen_uniform(7 + k, h * (E << k)).reshape(h, E << k)
    r = _r(oracle, 8 + k, k)
    idx = np.array([2999, 0, 17, 17, 1024, 5, 2047], np.uint64)  # unsorted, repeated
    got = pcs.fold_rows_at(DeviceBuffer.from_array(mat), h, k, is_ext, idx, r)
    want = oracle.fold_rows(mat[idx.astype(np.int64)], k, r, is_ext)
    assert (got == want).all()


def test_fold_rows_at_rejects_index_out_of_range(native, oracle):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer, ZkieError

    mat = oracle.gen_uniform(1, 64 * 16).reshape(64, 16)
    with pytest.raises(ZkieError):
        pcs.fold_rows_at(DeviceBuffer.from_array(mat), 64, 4, False, [3, 64], _r(oracle, 2, 4))


@pytest.mark.parametrize("prefix", [False, True])
@pytest.mark.parametrize("is_ext", [False, True])
@pytest.mark.parametrize("n,k,lr", [(6, 1, 1), (10, 4, 3), (14, 4, 2), (17, 4, 3)])
def test_whir_encode_matches_oracle(native, oracle, prefix, is_ext, n, k, lr):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE whir_encode n={n} k={k} lr={lr} ext={is_ext} prefix={prefix}", flush=True)
    E = 2 if is_ext else 1
    poly = oracle.gen_uniform(50 + n, E << n)
    out = DeviceBuffer(E << (n + lr))
    pcs.whir_encode(DeviceBuffer.from_array(poly), n, is_ext, k, lr, prefix, out)
    want = oracle.whir_encode(poly, n, is_ext, k, lr, prefix)
    assert (out.download().reshape(want.shape) == want).all()


def test_whir_encode_prefix_rejects_overlap(native, oracle):
    from zkie_amd import _native as N
    from zkie_amd._native import DeviceBuffer

    buf = DeviceBuffer(1 << 12)
    rc = N.load().zkie_whir_encode(buf.addr, 8, 0, 2, 2, 1, buf.addr, None)
    assert rc == -1


def test_streams_order_dependent_work(native, oracle):
    """A fold queued on a second stream after zkie_stream_wait sees the LDE
    queued before it on the first stream (the stream plumbing of the ABI)."""
    from zkie_amd import _native as N
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print("CASE streams", flush=True)
    h, w, lb = 1 << 12, 16, 2
    data = oracle.gen_uniform(77, h * w).reshape(h, w)
    d_in, d_cw, d_f = DeviceBuffer.from_array(data), DeviceBuffer(h * w << lb), DeviceBuffer(2 * (h << lb))
    a, b = N.Stream(), N.Stream()
    r = _r(oracle, 78, 4)
    pcs.lde_device(d_in, h, w, lb, d_cw, stream=a.handle)
    b.wait(a)
    pcs.fold_rows_device(d_cw, h << lb, 4, r, False, d_f, stream=b.handle)
    b.synchronize()
    want = oracle.fold_rows(oracle.lde_batch(data, lb), 4, r, False)
    assert (d_f.download().reshape(-1, 2) == want).all()
