"""GPU parity of zkie_commit_batch (Whir::commit_batch, whir.rs:476-525)
against the oracle's stack + encode + commit: the stacked witness, the
codeword, every digest layer and the root, bit-exact. Cases: a power-of-two
and a ragged table count (zero padding rows neither written nor read), tables
smaller than a row, no blowup (the padding written out), tables that already
sit in their place in the stack, a fused 16-wide commit, and the refusals."""
from types import SimpleNamespace

import numpy as np
import pytest

from zkie_amd import pcs
from zkie_amd._native import DeviceBuffer, check, p

pytestmark = pytest.mark.gpu


def _case(*a):
    print("CASE", *a, flush=True)


@pytest.mark.parametrize("count,arity,k,lb", [(1, 10, 2, 2), (4, 8, 2, 1), (3, 9, 3, 2), (5, 2, 3, 1),
                                              (6, 7, 4, 0), (7, 16, 4, 2), (16, 12, 4, 3), (3, 14, 1, 1)])
def test_commit_batch(native, oracle, count, arity, k, lb):
    _case("commit_batch", count, arity, k, lb)
    ts = [oracle.gen_uniform(1000 * count + 10 * arity + i, 1 << arity) for i in range(count)]
    stack, cw, layers, root = oracle.commit_batch(ts, k, lb)
    mmcs = pcs.HipMerkleTreeMmcs()
    tree, d_stack = mmcs.commit_batch_device([DeviceBuffer.from_array(t) for t in ts], arity, k, lb)
    total = count << arity
    got_stack = d_stack.download()
    assert (got_stack[:total] == stack.reshape(-1)[:total]).all()
    if lb == 0:
        assert (got_stack[total:] == 0).all()
    assert (tree.d_mat.download().reshape(cw.shape) == cw).all()
    got = tree.layers()
    assert len(got) == len(layers)
    for a, b in zip(got, layers):
        assert (a == b).all()
    assert (tree.root == root).all()


def test_tables_already_in_the_stack(native, oracle):
    _case("commit_batch in place")
    count, arity, k, lb = 3, 11, 4, 2
    ts = [oracle.gen_uniform(77 + i, 1 << arity) for i in range(count)]
    _, _, _, root = oracle.commit_batch(ts, k, lb)
    d_stack = DeviceBuffer(1 << 13)
    d_stack.upload(np.concatenate(ts))
    views = [SimpleNamespace(addr=d_stack.addr + 8 * (i << arity)) for i in range(count)]
    tree, _ = pcs.HipMerkleTreeMmcs().commit_batch_device(views, arity, k, lb, d_stack=d_stack)
    assert (tree.root == root).all()


def test_refusals(native):
    _case("commit_batch refusals")
    L = native.load()
    a, s, cw, lay = DeviceBuffer(1 << 10), DeviceBuffer(1 << 12), DeviceBuffer(1 << 14), DeviceBuffer(1 << 12)
    root = np.zeros(8, np.uint64)

    def call(ptrs, count, arity, k, lb, stack=s):
        arr = np.array(ptrs, np.uint64)
        return L.zkie_commit_batch(p(arr), count, arity, k, lb, stack.addr, cw.addr, lay.addr, p(root), None)

    assert call([a.addr], 0, 4, 2, 1) != 0                      # empty batch
    assert call([a.addr], 1, 2, 3, 1) != 0                      # fills no row
    assert call([0], 1, 4, 2, 1) != 0                           # null table
    assert call([s.addr + 8, a.addr], 2, 4, 2, 1) != 0          # overlaps the stack, not its slot
    assert call([a.addr], 1, 41, 2, 1) != 0                     # arity beyond the limit
    big = [a.addr] * 512
    assert call(big, 512, 40, 16, 0) != 0                       # 2^9 x 2^40 entries: beyond 2^48
