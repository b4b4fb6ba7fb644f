"""GPU tests of the library's shared scratch under concurrent use: calls
queued on several streams without any ordering between them, and calls made
from several host threads at once, each give the oracle's result bit for bit
(the scratch leases order every buffer's users on the GPU)."""
import threading

import numpy as np
import pytest

P = 0xFFFFFFFF00000001
pytestmark = pytest.mark.gpu


def test_ldes_on_unordered_streams(native, oracle):
    """Three LDEs and an inverse DFT, all needing the multi-pass NTT scratch,
    queued back to back on four streams with no waits between them; the last
    LDE is larger, so the scratch also grows while the others are queued."""
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer, Stream

    print("CASE ldes on unordered streams", flush=True)
    shapes = [(1 << 17, 16, 2), (1 << 17, 16, 2), (1 << 18, 16, 2)]
    inputs = [oracle.gen_uniform(300 + i, h * w).reshape(h, w) for i, (h, w, _) in enumerate(shapes)]
    d_in = [DeviceBuffer.from_array(x) for x in inputs]
    d_out = [DeviceBuffer((h << lb) * w) for h, w, lb in shapes]
    lg_i = 17
    x_i = oracle.gen_uniform(399, (1 << lg_i) * 16).reshape(1 << lg_i, 16)
    d_i = DeviceBuffer.from_array(x_i)
    streams = [Stream() for _ in range(4)]
    for k, (h, w, lb) in enumerate(shapes):
        pcs.lde_device(d_in[k], h, w, lb, d_out[k], stream=streams[k].handle)
    from zkie_amd._native import check, load

    check(load().zkie_idft_batch(d_i.addr, lg_i, 16, streams[3].handle), "zkie_idft_batch")
    for s in streams:
        s.synchronize()
    for k, (h, w, lb) in enumerate(shapes):
        assert (d_out[k].download().reshape(h << lb, w) == oracle.lde_batch(inputs[k], lb)).all(), k
    assert (oracle.dft_batch(d_i.download().reshape(x_i.shape)) == x_i).all()


def test_host_threads_share_the_library(native, oracle):
    """Four host threads, each on its own stream, run LDE, commitment,
    openings and queried-row folds (all four scratch users) concurrently."""
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer, Stream

    print("CASE host threads", flush=True)
    h, w, lb, k = 1 << 14, 16, 2, 4
    n = h << lb
    jobs = []
    for t in range(4):
        data = oracle.gen_uniform(500 + t, h * w).reshape(h, w)
        cw = oracle.lde_batch(data, lb)
        layers, root = oracle.merkle_commit(cw)
        idx = np.sort(oracle.gen_uniform(600 + t, 64) % np.uint64(n))
        r = (oracle.gen_uniform(700 + t, 2 * k) % np.uint64(P)).reshape(k, 2)
        fold = oracle.fold_rows(cw, k, r, False)[idx.astype(np.int64)]
        jobs.append((data, cw, root, idx, r, fold))
    errors = []

    def work(t):
        try:
            data, cw, root, idx, r, fold = jobs[t]
            s = Stream()
            d_in, d_cw = DeviceBuffer.from_array(data), DeviceBuffer(n * w)
            mmcs = pcs.HipMerkleTreeMmcs()
            for _ in range(3):
                pcs.lde_device(d_in, h, w, lb, d_cw, stream=s.handle)
                tree = mmcs.commit_device(d_cw, n, w, stream=s.handle)
                rows, sib = mmcs.open_batches(idx, tree, stream=s.handle)
                got = pcs.fold_rows_at(d_cw, n, k, False, idx, r, stream=s.handle)
                assert (tree.root == root).all(), f"thread {t}: root"
                assert (rows == cw[idx.astype(np.int64)]).all(), f"thread {t}: rows"
                for j in range(0, idx.size, 16):
                    assert oracle.merkle_verify(root, n, int(idx[j]), rows[j], sib[j]), f"thread {t}: path"
                assert (got == fold).all(), f"thread {t}: fold"
            s.synchronize()
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors


def test_coset_ldes_on_unordered_streams(native, oracle):
    """Coset LDEs (shift != 1) queued on two streams with no waits between
    them and no host synchronisation inside the calls: the coset powers are
    formed on the device in the leased table of each call's stream."""
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer, Stream

    print("CASE coset ldes on unordered streams", flush=True)
    cases = [(1 << 12, 16, 2, 7), (1 << 13, 8, 1, 0x1234567890ABCDEF), (1 << 16, 1, 2, 11)]
    streams = [Stream(), Stream()]
    inputs, outs = [], []
    for i, (h, w, lb, shift) in enumerate(cases):
        x = oracle.gen_uniform(800 + i, h * w).reshape(h, w)
        d_in, d_out = DeviceBuffer.from_array(x), DeviceBuffer((h << lb) * w)
        pcs.lde_device(d_in, h, w, lb, d_out, shift=shift, stream=streams[i % 2].handle)
        inputs.append((x, d_in))
        outs.append(d_out)
    for s in streams:
        s.synchronize()
    for (h, w, lb, shift), (x, _), d_out in zip(cases, inputs, outs):
        got = d_out.download().reshape(h << lb, w)
        assert (got == oracle.lde_batch(x, lb, shift % P)).all(), (h, w, lb, shift)
