"""Oracle checks for the sumcheck rounds of a product of two multilinear
tables (common/sumcheck.rs:33-89, the round polynomials the WHIR prover
sends before each fold). Pins that do not restate the oracle's formulas:

* the base-field case equals a line-by-line pure-Python restatement of
  sumcheck::prove with Python integers;
* in EF, each round polynomial agrees with the sums it must interpolate at
  X = 0, 1, 2 and 3 (sums of f(X, b) h(X, b) with f(X, b) = (1 - X) f0 + X f1,
  so the degree-2 claim is checked at a fourth point);
* the protocol identities of sumcheck::verify (sumcheck.rs:91-111): p_1(0) +
  p_1(1) is the hypercube sum, p_{i+1}(0) + p_{i+1}(1) = p_i(r_i), and after
  all rounds p_t(r_t) = f(r) h(r) with f(r) from the multilinear evaluation
  (mle.rs:8-22); a tampered coefficient breaks it (the soundness test of
  sumcheck.rs:317-336);
* k rounds leave the table fold over the low k variables (or_fold_rows with
  the table as rows of 2^k entries)."""
import numpy as np
import pytest

P = 0xFFFFFFFF00000001
W = 7
INV2 = (P + 1) // 2


def ef_mul(a, b):
    return ((a[0] * b[0] + W * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def ef_add(a, b):
    return ((a[0] + b[0]) % P, (a[1] + b[1]) % P)


def ef_sub(a, b):
    return ((a[0] - b[0]) % P, (a[1] - b[1]) % P)


def ef_scale(a, k):
    return (a[0] * k % P, a[1] * k % P)


def poly_at(c, x):
    """c0 + c1 x + c2 x^2 in EF at an EF point x."""
    c0, c1, c2 = (tuple(int(v) for v in ci) for ci in c)
    return ef_add(ef_add(c0, ef_mul(c1, x)), ef_mul(c2, ef_mul(x, x)))


def prove_base_literal(f, h, challenges):
    """common/sumcheck.rs:33-89 over Goldilocks, line by line."""
    f_buf, h_buf, rounds = list(f), list(h), []
    for r in challenges:
        half = len(f_buf) // 2
        y0 = y1 = y2 = 0
        for s in range(half):
            f0, f1, h0, h1 = f_buf[2 * s], f_buf[2 * s + 1], h_buf[2 * s], h_buf[2 * s + 1]
            y0 = (y0 + f0 * h0) % P
            y1 = (y1 + f1 * h1) % P
            y2 = (y2 + ((2 * f1 - f0) % P) * ((2 * h1 - h0) % P)) % P
        c0 = y0
        c1 = ((4 * y1 - y2 - 3 * y0) * INV2) % P
        c2 = ((y2 - 2 * y1 + y0) * INV2) % P
        rounds.append((c0, c1, c2))
        for buf in (f_buf, h_buf):
            for i in range(half):
                a, b = buf[2 * i], buf[2 * i + 1]
                buf[i] = (a + r * (b - a)) % P
            del buf[half:]
    return rounds, f_buf, h_buf


def _tables(oracle, seed, t, f_ext):
    f = oracle.gen_uniform(seed, (2 if f_ext else 1) << t)
    h = oracle.gen_uniform(seed + 1, 2 << t)
    r = (oracle.gen_uniform(seed + 2, 2 * t) % np.uint64(P)).reshape(t, 2)
    return f, h, r


@pytest.mark.parametrize("t", [1, 2, 5, 8])
def test_base_case_matches_literal_restatement(oracle, t):
    f = [int(x) % P for x in oracle.gen_uniform(40 + t, 1 << t)]
    h = [int(x) % P for x in oracle.gen_uniform(50 + t, 1 << t)]
    ch = [int(x) % P for x in oracle.gen_uniform(60 + t, t)]
    want, fe, he = prove_base_literal(f, h, ch)
    h_ef = np.array([[x, 0] for x in h], np.uint64)
    r = np.array([[x, 0] for x in ch], np.uint64)
    polys, fo, ho = oracle.sumcheck_prove(np.array(f, np.uint64), False, h_ef, r)
    for i, (c0, c1, c2) in enumerate(want):
        assert [int(v) for v in polys[i][:, 0]] == [c0, c1, c2]
        assert (polys[i][:, 1] == 0).all()
    assert [int(fo[0][0]), int(ho[0][0])] == [fe[0], he[0]] and int(fo[0][1]) == int(ho[0][1]) == 0


@pytest.mark.parametrize("f_ext", [False, True])
@pytest.mark.parametrize("t", [1, 3, 6])
def test_round_polys_interpolate_the_sums(oracle, t, f_ext):
    f, h, r = _tables(oracle, 70 + t, t, f_ext)
    fv = f.reshape(-1, 2) if f_ext else np.stack([f, np.zeros_like(f)], 1)
    fb = [(int(a) % P, int(b) % P) for a, b in fv]
    hb = [(int(a) % P, int(b) % P) for a, b in h.reshape(-1, 2)]
    polys, _, _ = oracle.sumcheck_prove(f, f_ext, h, r)
    for i in range(t):
        for X in (0, 1, 2, 3):
            s = (0, 0)
            for j in range(len(fb) // 2):
                fx = ef_add(ef_scale(fb[2 * j], (1 - X) % P), ef_scale(fb[2 * j + 1], X))
                hx = ef_add(ef_scale(hb[2 * j], (1 - X) % P), ef_scale(hb[2 * j + 1], X))
                s = ef_add(s, ef_mul(fx, hx))
            assert poly_at(polys[i], (X, 0)) == s, (i, X)
        ri = (int(r[i][0]), int(r[i][1]))
        fb = [ef_add(fb[2 * j], ef_mul(ri, ef_sub(fb[2 * j + 1], fb[2 * j]))) for j in range(len(fb) // 2)]
        hb = [ef_add(hb[2 * j], ef_mul(ri, ef_sub(hb[2 * j + 1], hb[2 * j]))) for j in range(len(hb) // 2)]


@pytest.mark.parametrize("f_ext", [False, True])
@pytest.mark.parametrize("t", [1, 4, 10])
def test_verifier_identities(oracle, t, f_ext):
    f, h, r = _tables(oracle, 90 + t, t, f_ext)
    polys, fo, ho = oracle.sumcheck_prove(f, f_ext, h, r)
    fv = f.reshape(-1, 2) if f_ext else np.stack([f, np.zeros_like(f)], 1)
    claim = (0, 0)
    for a, b in zip(fv, h.reshape(-1, 2)):
        claim = ef_add(claim, ef_mul((int(a[0]), int(a[1])), (int(b[0]), int(b[1]))))

    def verify(ps):
        prev = claim
        for i in range(t):
            if ef_add(poly_at(ps[i], (0, 0)), poly_at(ps[i], (1, 0))) != prev:
                return False
            prev = poly_at(ps[i], (int(r[i][0]), int(r[i][1])))
        f_r = oracle.mle_eval(f, r, f_ext)
        h_r = oracle.mle_eval(h, r, True)
        want = ef_mul((int(f_r[0]), int(f_r[1])), (int(h_r[0]), int(h_r[1])))
        return prev == want and want == ef_mul((int(fo[0][0]), int(fo[0][1])), (int(ho[0][0]), int(ho[0][1])))

    assert verify(polys)
    bad = polys.copy()
    bad[t // 2][0][0] = (int(bad[t // 2][0][0]) + 1) % P
    assert not verify(bad)


@pytest.mark.parametrize("f_ext", [False, True])
@pytest.mark.parametrize("t,k", [(6, 1), (8, 4), (12, 4), (9, 3)])
def test_rounds_leave_the_table_fold(oracle, t, k, f_ext):
    f, h, r = _tables(oracle, 110 + t, t, f_ext)
    _, fo, ho = oracle.sumcheck_prove(f, f_ext, h, r[:k])
    E = 2 if f_ext else 1
    assert (fo == oracle.fold_rows(f.reshape(-1, E << k), k, r[:k], f_ext)).all()
    assert (ho == oracle.fold_rows(h.reshape(-1, 2 << k), k, r[:k], True)).all()


@pytest.mark.parametrize("t", [0, 1, 3, 7])
def test_eq_table_is_the_product_formula(oracle, t):
    """Each entry against the product over its bits, written per entry
    (mle.rs:44-56 states the same table by doubling)."""
    pt = (oracle.gen_uniform(130 + t, 2 * t) % np.uint64(P)).reshape(t, 2)
    got = oracle.eq_table(pt)
    for x in range(1 << t):
        e = (1, 0)
        for b in range(t):
            z = (int(pt[b][0]), int(pt[b][1]))
            e = ef_mul(e, z if (x >> b) & 1 else ((1 - z[0]) % P, (-z[1]) % P))
        assert (int(got[x][0]), int(got[x][1])) == e


@pytest.mark.parametrize("f_ext", [False, True])
@pytest.mark.parametrize("t", [1, 6, 10])
def test_eq_table_weights_evaluate(oracle, t, f_ext):
    """sum_x eq(p, x) f(x) = f(p), the multilinear evaluation (mle.rs:8-22)."""
    pt = (oracle.gen_uniform(140 + t, 2 * t) % np.uint64(P)).reshape(t, 2)
    f = oracle.gen_uniform(150 + t, (2 if f_ext else 1) << t)
    fv = f.reshape(-1, 2) if f_ext else np.stack([f, np.zeros_like(f)], 1)
    eq = oracle.eq_table(pt)
    s = (0, 0)
    for a, b in zip(eq, fv):
        s = ef_add(s, ef_mul((int(a[0]), int(a[1])), (int(b[0]) % P, int(b[1]) % P)))
    want = oracle.mle_eval(f, pt, f_ext)
    assert s == (int(want[0]), int(want[1]))
