"""Pins of the oracle Merkle tree: the vendored p3-merkle-tree tests restated
(padded_len tables, XOR dummy compressor layers, structural commits, the
pruning doc example) plus an independent python build of the layers and
open/verify round trips."""
import numpy as np
import pytest

from oracle import pyref


def test_padded_len_tables(oracle):
    # merkle_tree.rs:756-815
    n2 = {0: 0, 1: 1, 2: 2, 3: 4, 4: 4, 5: 6, 7: 8, 8: 8, 9: 10, 15: 16, 16: 16}
    n4 = {0: 0, 1: 1, 2: 4, 3: 4, 4: 4, 5: 8, 7: 8, 8: 8, 9: 12}
    n8 = {0: 0, 1: 1, 2: 8, 3: 8, 5: 8, 7: 8, 8: 8, 9: 16, 15: 16, 16: 16}
    for n, table in ((2, n2), (4, n4), (8, n8)):
        for raw, exp in table.items():
            assert oracle.padded_len(raw, n) == exp
    for n in (2, 4, 8):
        for raw in range(2, 129):
            pl = oracle.padded_len(raw, n)
            assert pl >= n and pl % n == 0


def _d(b):
    return np.full(8, int.from_bytes(bytes([b]) * 8, "little"), np.uint64)


def _layer(*bs):
    return np.stack([_d(b) for b in bs])


def test_compress_layer_with_xor_dummy(oracle):
    # merkle_tree.rs:675-756 (DummyCompressionFunction = XOR)
    assert (oracle.compress_layer(_layer(1, 2, 3, 4), 1) == _layer(3, 7)).all()
    assert (oracle.compress_layer(_layer(5, 6, 7), 1) == _layer(3)).all()
    assert (oracle.compress_layer(_layer(0xAA, 0x55), 1) == _layer(0xFF)).all()
    out = oracle.compress_layer(_layer(1, 2, 3, 4, 5, 6), 1)
    assert out.shape[0] == 4
    assert (out == np.stack([_d(3), _d(7), _d(3), _d(0)])).all()


def test_layer_lengths(oracle):
    for h, exp in [(1, [1]), (2, [2, 1]), (3, [4, 2, 1]), (5, [6, 4, 2, 1]), (8, [8, 4, 2, 1]),
                   (9, [10, 6, 4, 2, 1])]:
        assert oracle.layer_lens(h) == exp


def test_commit_structure(oracle):
    perm = pyref.Poseidon2()
    H = lambda row: perm.hash_row(row)
    C = perm.compress
    # mmcs/batch.rs:336-367 commit_single_1x8: v = [2,1,2,2,0,0,1,0] as an 8x1 matrix
    v = [2, 1, 2, 2, 0, 0, 1, 0]
    _, root = oracle.merkle_commit(np.array(v, np.uint64).reshape(8, 1))
    exp = C(C(C(H([v[0]]), H([v[1]])), C(H([v[2]]), H([v[3]]))),
            C(C(H([v[4]]), H([v[5]])), C(H([v[6]]), H([v[7]]))))
    assert [int(x) for x in root] == exp
    # :417-429 commit_single_8x1: one row of 8 -> root = hash(row)
    row = [int(x) for x in oracle.gen_uniform(1, 8)]
    _, root = oracle.merkle_commit(np.array(row, np.uint64).reshape(1, 8))
    assert [int(x) for x in root] == H(row)
    # :431-453 commit_single_2x2
    _, root = oracle.merkle_commit(np.array([[0, 1], [2, 1]], np.uint64))
    assert [int(x) for x in root] == C(H([0, 1]), H([2, 1]))


@pytest.mark.parametrize("h,w", [(1, 3), (2, 1), (3, 2), (5, 8), (6, 16), (7, 9), (16, 1), (33, 4)])
def test_layers_match_python_build(oracle, h, w):
    perm = pyref.Poseidon2()
    m = oracle.gen_uniform(h * 100 + w, h * w).reshape(h, w)
    layers, root = oracle.merkle_commit(m)
    py = pyref.merkle_layers(m.tolist(), perm)
    assert len(py) == len(layers)
    for a, b in zip(layers, py):
        assert a.tolist() == b
    assert root.tolist() == py[-1][0]


@pytest.mark.parametrize("h", [1, 2, 3, 5, 8, 13])
def test_open_verify_roundtrip(oracle, h):
    m = oracle.gen_uniform(h, h * 4).reshape(h, 4)
    layers, root = oracle.merkle_commit(m)
    for i in range(h):
        sib = oracle.merkle_open(layers, h, i)
        assert sib.shape[0] == len(layers) - 1
        assert oracle.merkle_verify(root, h, i, m[i], sib)
        if sib.shape[0]:
            bad = sib.copy()
            bad[0, 0] ^= np.uint64(1)
            assert not oracle.merkle_verify(root, h, i, m[i], bad)
        row = m[i].copy()
        row[0] ^= np.uint64(1)
        assert not oracle.merkle_verify(root, h, i, row, sib)


def test_pruning_doc_example(oracle):
    # pruning.rs:22-45: leaves {1, 2, 5} of 8 -> send 0, 3, 4 at level 0 and F at level 1.
    m = oracle.gen_uniform(0, 8).reshape(8, 1)
    layers, _ = oracle.merkle_commit(m)
    pr = oracle.merkle_open_pruned(layers, 8, [5, 1, 2, 2])
    exp = np.stack([layers[0][0], layers[0][3], layers[0][4], layers[1][3]])
    assert (pr == exp).all()
    # pruning.rs:504-525 counts
    assert oracle.merkle_open_pruned(layers, 8, list(range(8))).shape[0] == 0
    assert oracle.merkle_open_pruned(layers, 8, [5]).shape[0] == 3
    assert (oracle.merkle_open_pruned(layers, 8, [5]) == oracle.merkle_open(layers, 8, 5)).all()


def test_pruned_never_exceeds_unpruned(oracle):
    m = oracle.gen_uniform(0, 32).reshape(32, 1)
    layers, _ = oracle.merkle_commit(m)
    for end in range(1, 33):
        idx = sorted({(i * 13) % 32 for i in range(end)})
        assert oracle.merkle_open_pruned(layers, 32, idx).shape[0] <= len(idx) * 5
