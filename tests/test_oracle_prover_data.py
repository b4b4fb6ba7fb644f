"""Oracle checks for the prover-data cache stream (whir.rs:542-602 with
merkle_tree.rs:223-276). Pins that do not restate the writer: byte strings
spelled out field by field with struct for small trees, the parser reading
back what the writer produced (two independent walks of the format), the
stream length from the tree geometry, and rejection of truncated or padded
streams."""
import struct

import numpy as np
import pytest


def q(*xs):
    return struct.pack("<" + "Q" * len(xs), *xs)


def test_single_row_tree_bytes(oracle):
    mat = np.array([[5]], np.uint64)
    layers, root = oracle.merkle_commit(mat)
    assert [l.shape[0] for l in layers] == [1]
    want = q(1, 1, 1) + q(5) + q(1, 1) + q(*[int(x) for x in root])
    assert oracle.prover_data_bytes(mat, layers) == want


def test_three_row_tree_bytes(oracle):
    mat = np.arange(6, dtype=np.uint64).reshape(3, 2) + np.uint64(100)
    layers, root = oracle.merkle_commit(mat)
    lens = [l.shape[0] for l in layers]
    assert lens == [4, 2, 1]  # padded_len ladder of merkle_tree.rs:577-585
    want = q(1, 2, 6) + q(100, 101, 102, 103, 104, 105) + q(3, 4, 2, 1, 2, 2)
    for l in layers:
        want += b"".join(q(*[int(x) for x in d]) for d in l)
    got = oracle.prover_data_bytes(mat, layers)
    assert got == want
    assert got[-64:] == q(*[int(x) for x in root])


@pytest.mark.parametrize("h,w", [(1, 3), (2, 1), (5, 8), (64, 16), (100, 9)])
def test_parse_inverts_write(oracle, h, w):
    mat = oracle.gen_uniform(h * 31 + w, h * w).reshape(h, w)
    layers, _ = oracle.merkle_commit(mat)
    buf = oracle.prover_data_bytes(mat, layers)
    lens = oracle.layer_lens(h)
    assert len(buf) == 8 * (3 + h * w + 2 * len(lens)) + 64 * sum(lens)
    mats, got_layers, arities = oracle.parse_prover_data(buf)
    assert len(mats) == 1 and (mats[0] == mat).all()
    assert [l.shape[0] for l in got_layers] == lens
    assert all((a == b).all() for a, b in zip(got_layers, layers))
    assert arities == [2] * (len(lens) - 1)


def test_parse_rejects_truncated_and_padded(oracle):
    mat = oracle.gen_uniform(3, 40).reshape(10, 4)
    layers, _ = oracle.merkle_commit(mat)
    buf = oracle.prover_data_bytes(mat, layers)
    for cut in (8, 30, len(buf) - 64, len(buf) - 1):
        with pytest.raises(ValueError):
            oracle.parse_prover_data(buf[:cut])
    with pytest.raises(ValueError):
        oracle.parse_prover_data(buf + q(0))
