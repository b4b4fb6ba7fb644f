"""Pins of the oracle DFT / LDE: the O(n^2) definition, an independent
python-integer restatement and the invariants the transform must satisfy."""
import numpy as np
import pytest

from oracle import pyref

P = 0xFFFFFFFF00000001


@pytest.mark.parametrize("lg,w", [(0, 3), (1, 1), (2, 3), (4, 1), (5, 4), (7, 2), (8, 1)])
def test_dft_matches_definition(oracle, lg, w):
    x = oracle.gen_uniform(lg * 10 + w, (1 << lg) * w).reshape(1 << lg, w)
    assert (oracle.dft_batch(x) == oracle.dft_naive(x)).all()


def test_dft_matches_python_integers(oracle):
    for lg in (3, 6):
        col = oracle.gen_uniform(5, 1 << lg)
        assert oracle.dft_batch(col.reshape(-1, 1))[:, 0].tolist() == pyref.dft(col.tolist())


def test_impulse_probes(oracle):
    # goldilocks_ntt.cu:11-15: impulse at 0 -> all ones, at 1 -> powers of w.
    lg = 6
    n = 1 << lg
    e0 = np.zeros((n, 1), np.uint64)
    e0[0] = 1
    assert (oracle.dft_batch(e0) == 1).all()
    e1 = np.zeros((n, 1), np.uint64)
    e1[1] = 1
    g = oracle.two_adic_generator(lg)
    assert oracle.dft_batch(e1)[:, 0].tolist() == [pow(g, i, P) for i in range(n)]


def test_inverse_and_linearity(oracle):
    x = oracle.gen_uniform(1, 1024 * 3).reshape(1024, 3)
    y = oracle.gen_uniform(2, 1024 * 3).reshape(1024, 3)
    X, Y = oracle.dft_batch(x), oracle.dft_batch(y)
    assert (oracle.idft_batch(X) == x).all()
    s = ((x.astype(object) + y.astype(object)) % P).astype(np.uint64)
    assert (oracle.dft_batch(s) == ((X.astype(object) + Y.astype(object)) % P).astype(np.uint64)).all()


def test_convolution_theorem(oracle):
    n = 64
    a = [int(v) for v in oracle.gen_uniform(3, n)]
    b = [int(v) for v in oracle.gen_uniform(4, n)]
    conv = [sum(a[j] * b[(i - j) % n] for j in range(n)) % P for i in range(n)]
    A = oracle.dft_batch(np.array(a, np.uint64).reshape(n, 1))[:, 0]
    B = oracle.dft_batch(np.array(b, np.uint64).reshape(n, 1))[:, 0]
    C = oracle.dft_batch(np.array(conv, np.uint64).reshape(n, 1))[:, 0]
    assert [int(c) for c in C] == [int(x) * int(y) % P for x, y in zip(A, B)]


@pytest.mark.parametrize("lg,w,lb", [(4, 1, 2), (6, 16, 2), (5, 3, 3), (8, 2, 1)])
def test_lde_restricts_to_subgroup_dft(oracle, lg, w, lb):
    # The codeword rows t = 0 mod 2^lb evaluate on the subgroup of size h:
    # they equal the unpadded DFT (writer.rs:73-81 encoding).
    x = oracle.gen_uniform(9, (1 << lg) * w).reshape(1 << lg, w)
    cw = oracle.lde_batch(x, lb)
    assert cw.shape == ((1 << lg) << lb, w)
    assert (cw[:: 1 << lb] == oracle.dft_batch(x)).all()


def test_coset_lde_is_polynomial_evaluation(oracle):
    h, lb, shift = 16, 2, 7
    x = oracle.gen_uniform(11, h * 2).reshape(h, 2)
    cw = oracle.lde_batch(x, lb, shift)
    n = h << lb
    g = oracle.two_adic_generator(n.bit_length() - 1)
    for t in (0, 1, 5, n - 1):
        pt = shift * pow(g, t, P) % P
        for c in range(2):
            acc = 0
            for j in reversed(range(h)):
                acc = (acc * pt + int(x[j, c])) % P
            assert int(cw[t, c]) == acc
