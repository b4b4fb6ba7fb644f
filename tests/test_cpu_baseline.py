"""The CPU baseline of bench.py (oracle/cpu_baseline.c, the AVX2 port of the
reference CPU commit path that is timed beside the GPU) is bit-identical to
the oracle: LDE codewords, every digest layer and root, and row folds, on
widths that take its vector and scalar paths, odd heights and edge values."""
import numpy as np
import pytest

from oracle import cpu_baseline as CB

P = 0xFFFFFFFF00000001


@pytest.fixture(scope="module")
def cb(oracle):
    CB.set_constants(*oracle.p2_constants())
    return CB


@pytest.mark.parametrize("lg,w,lb", [(0, 4, 0), (0, 16, 2), (3, 1, 2), (6, 16, 2), (9, 3, 1), (10, 16, 2),
                                     (12, 16, 3), (11, 32, 1), (8, 128, 1), (13, 8, 2)])
def test_lde_matches_oracle(cb, oracle, lg, w, lb):
    x = oracle.gen_uniform(lg * 31 + w, (1 << lg) * w).reshape(1 << lg, w)
    assert (cb.lde_batch(x, lb) == oracle.lde_batch(x, lb)).all()


def test_lde_edge_values(cb, oracle):
    x = np.array([[0, 1, P - 1, P - 2], [P - 1, P - 1, 0, 2**63], [1, 2**32, 2**32 - 1, P - 2**32]] * 4,
                 np.uint64)
    x = x.reshape(-1, 4)[:8]
    assert (cb.lde_batch(x, 2) == oracle.lde_batch(x, 2)).all()


@pytest.mark.parametrize("h,w", [(1, 1), (1, 16), (2, 8), (3, 5), (7, 16), (100, 3), (513, 16), (1000, 32),
                                 (256, 128), (1 << 12, 16), (4097, 1)])
def test_merkle_matches_oracle(cb, oracle, h, w):
    m = oracle.gen_uniform(h * 7 + w, h * w).reshape(h, w)
    layers, root = cb.merkle_commit(m)
    olayers, oroot = oracle.merkle_commit(m)
    assert len(layers) == len(olayers)
    for a, b in zip(layers, olayers):
        assert (a.reshape(-1) == b.reshape(-1)).all()
    assert (root == oroot).all()


def test_permutation_edge_states(cb, oracle):
    # rows of p - 1 and zeros exercise every wrap of the canonical adds
    for row in (np.full(16, P - 1, np.uint64), np.zeros(16, np.uint64),
                np.array([P - 1, 0] * 8, np.uint64), np.array([2**63] * 16, np.uint64)):
        m = np.stack([row] * 5)
        layers, root = cb.merkle_commit(m)
        olayers, oroot = oracle.merkle_commit(m)
        assert (root == oroot).all()


@pytest.mark.parametrize("k", [0, 1, 2, 4, 6])
def test_fold_matches_oracle(cb, oracle, k):
    m = oracle.gen_uniform(50 + k, 333 * (1 << k)).reshape(333, 1 << k)
    r = (oracle.gen_uniform(60 + k, 2 * k) % np.uint64(P)).reshape(k, 2) if k else np.zeros((0, 2), np.uint64)
    assert (cb.fold_rows(m, k, r) == oracle.fold_rows(m, k, r, False)).all()
    edge = np.full((5, 1 << k), P - 1, np.uint64)
    rr = np.full((k, 2), P - 1, np.uint64)
    assert (cb.fold_rows(edge, k, rr) == oracle.fold_rows(edge, k, rr, False)).all()


def test_results_do_not_depend_on_threads(cb, oracle):
    x = oracle.gen_uniform(77, (1 << 11) * 16).reshape(1 << 11, 16)
    outs = []
    for t in (1, 3, 8):
        cb.set_threads(t)
        cw = cb.lde_batch(x, 2)
        outs.append((cw, cb.merkle_commit(cw)[1]))
    cb.set_threads(8)
    for cw, root in outs[1:]:
        assert (cw == outs[0][0]).all() and (root == outs[0][1]).all()
