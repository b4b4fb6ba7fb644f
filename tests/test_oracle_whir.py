"""Oracle checks for the WHIR round pieces around the commitment: the
multilinear evaluation (out-of-domain answers) and commit_extension's
encoding in both variable orders. Pins that do not restate the formula:
Boolean points select table entries, the pairwise fold (mle.rs:12-20)
agrees with the eq-weight row fold of or_fold_rows, and a hand-computed
2 x 2 Prefix encoding fixes the transposition of writer.rs:43-71."""
import numpy as np
import pytest

P = 0xFFFFFFFF00000001


def ef_point(bits):
    return np.array([[b, 0] for b in bits], np.uint64)


@pytest.mark.parametrize("is_ext", [False, True])
def test_mle_eval_boolean_points_select_entries(oracle, is_ext):
    t = 5
    vals = oracle.gen_uniform(11, (2 if is_ext else 1) << t)
    v = vals.reshape(-1, 2) if is_ext else vals
    for idx in (0, 1, 6, 17, 31):
        bits = [(idx >> b) & 1 for b in range(t)]  # variable 0 = least-significant bit
        got = oracle.mle_eval(vals, ef_point(bits), is_ext)
        want = [int(v[idx][0]), int(v[idx][1])] if is_ext else [int(v[idx]), 0]
        assert [int(x) for x in got] == want


@pytest.mark.parametrize("is_ext", [False, True])
@pytest.mark.parametrize("t,k", [(4, 1), (7, 3), (9, 4)])
def test_mle_eval_equals_row_fold_then_eval(oracle, is_ext, t, k):
    E = 2 if is_ext else 1
    vals = oracle.gen_uniform(20 + t, E << t)
    r = oracle.gen_uniform(30 + t, 2 * t).reshape(t, 2) % np.uint64(P)
    direct = oracle.mle_eval(vals, r, is_ext)
    folded = oracle.fold_rows(vals.reshape(1 << (t - k), E << k), k, r[:k], is_ext)
    assert (oracle.mle_eval(folded.reshape(-1), r[k:], True) == direct).all()


def test_mle_eval_base_point_matches_base_routine(oracle):
    t = 6
    vals = oracle.gen_uniform(5, 1 << t)
    pt = oracle.gen_uniform(6, t)
    got = oracle.mle_eval(vals, np.stack([pt, np.zeros(t, np.uint64)], 1), False)
    assert int(got[1]) == 0 and int(got[0]) == oracle.mle_eval_base(vals, pt)


def test_whir_encode_prefix_known_answer(oracle):
    a, b, c, d = 3, 5, 11, 1000
    # Prefix, n = 2, k = 1: entry (i, j) = T[2 j + i] -> rows [a, c], [b, d];
    # no padding, 2-point DFT per column: [x0 + x1, x0 - x1].
    got = oracle.whir_encode(np.array([a, b, c, d], np.uint64), 2, False, 1, 0, True)
    assert got.tolist() == [[a + b, c + d], [(a - b) % P, (c - d) % P]]
    got = oracle.whir_encode(np.array([a, b, c, d], np.uint64), 2, False, 1, 0, False)
    assert got.tolist() == [[a + c, b + d], [(a - c) % P, (b - d) % P]]


@pytest.mark.parametrize("is_ext", [False, True])
def test_whir_encode_rows_at_stride_blowup_are_the_unpadded_dft(oracle, is_ext):
    n, k, lr = 8, 2, 2
    E = 2 if is_ext else 1
    poly = oracle.gen_uniform(40, E << n)
    for prefix in (False, True):
        cw = oracle.whir_encode(poly, n, is_ext, k, lr, prefix)
        base = oracle.whir_encode(poly, n, is_ext, k, 0, prefix)
        assert cw.shape == ((1 << (n - k + lr)), E << k)
        assert (cw[:: 1 << lr] == base).all()
