"""Pins of the oracle row fold: mle::eval semantics (common/mle.rs), the eq
expansion, special points, and the fold / encode commutation that links the
codeword fold to the table fold of the next WHIR round."""
import random

import numpy as np

from oracle import pyref

P = 0xFFFFFFFF00000001


def _rand_ef(rng, k):
    return [(rng.randrange(P), rng.randrange(P)) for _ in range(k)]


def test_partial_then_full_matches_full(oracle):
    # mle.rs:71-82 restated: fold the first 2 of 4 variables, then the rest.
    vals = oracle.gen_uniform(2, 16)
    pt = [int(x) for x in oracle.gen_uniform(3, 4)]
    full = oracle.mle_eval_base(vals, pt)
    r01 = np.array([[pt[0], 0], [pt[1], 0]], np.uint64)
    rest = oracle.fold_rows(vals.reshape(4, 4), 2, r01, False)
    assert (rest[:, 1] == 0).all()
    assert oracle.mle_eval_base(rest[:, 0].copy(), pt[2:]) == full


def test_fold_matches_python_and_eq_expansion(oracle):
    rng = random.Random(4)
    for k, ext in [(1, False), (3, False), (4, False), (2, True), (4, True)]:
        h = 5
        width = 1 << k
        r = _rand_ef(rng, k)
        if ext:
            m = oracle.gen_uniform(k, h * 2 * width).reshape(h, 2 * width)
            rows = [[(int(m[t, 2 * j]), int(m[t, 2 * j + 1])) for j in range(width)] for t in range(h)]
        else:
            m = oracle.gen_uniform(k, h * width).reshape(h, width)
            rows = [[(int(m[t, j]), 0) for j in range(width)] for t in range(h)]
        out = oracle.fold_rows(m, k, np.array(r, np.uint64), ext)
        for t in range(h):
            assert tuple(int(x) for x in out[t]) == pyref.mle_eval_ef(rows[t], r)
            # sum_j eq(r, j) row[j], eq over bits with bit 0 the LSB (mle.rs:44-56)
            acc = (0, 0)
            for j in range(width):
                e = (1, 0)
                for b in range(k):
                    rb = r[b] if (j >> b) & 1 else ((1 - r[b][0]) % P, (-r[b][1]) % P)
                    e = pyref.ef_mul(e, rb)
                pr = pyref.ef_mul(e, rows[t][j])
                acc = ((acc[0] + pr[0]) % P, (acc[1] + pr[1]) % P)
            assert tuple(int(x) for x in out[t]) == acc


def test_boolean_point_selects_entry(oracle):
    m = oracle.gen_uniform(8, 3 * 16).reshape(3, 16)
    for j in (0, 5, 15):
        r = np.array([[(j >> b) & 1, 0] for b in range(4)], np.uint64)
        out = oracle.fold_rows(m, 4, r, False)
        assert (out[:, 0] == m[:, j]).all() and (out[:, 1] == 0).all()


def test_fold_commutes_with_encode(oracle):
    # fold_rows(encode(T)) = encode(fold_table(T)): the row fold of the codeword
    # is the codeword of the folded table (same height, blowup kept).
    rng = random.Random(9)
    k, rows, lb = 4, 64, 2
    T = oracle.gen_uniform(21, rows * 16).reshape(rows, 16)
    r = np.array(_rand_ef(rng, k), np.uint64)
    cw = oracle.lde_batch(T, lb)
    lhs = oracle.fold_rows(cw, k, r, False)
    folded_table = oracle.fold_rows(T, k, r, False)  # (rows, 2): EF table of the next round
    rhs = oracle.lde_batch(folded_table, lb)  # EF column = two base columns
    assert (lhs == rhs).all()
