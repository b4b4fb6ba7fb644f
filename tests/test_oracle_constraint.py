"""The oracle's batched constraint weights of a WHIR round (p3-whir
src/pcs/prover/mod.rs:228-314; or_constraint_weights), pinned against what
the mathematics fixes, computed independently in Python integers:
  * with gamma = 0 only the first constraint remains: the eq table of p_0, or
    the power table z^x of the first selection point;
  * a selection constraint's weights are the powers z^x (bit b of x standing
    for z^(2^b));
  * the weighted sum over the hypercube is the batched claim:
    sum_x f(x) w(x) = sum_j gamma^j f(p_j) + sum_k gamma^(m+k) F(z_k), with
    f(p) the multilinear evaluation (mle.rs:8-22) and F(z) the polynomial
    whose coefficients are the table, at z (Horner);
  * as a polynomial in gamma, coefficient c is constraint c's table.
The order of the gamma powers (the Eq group first, from gamma^0) restates
Constraint::new of the external p3-sumcheck crate and is parity unpinned."""
import numpy as np
import pytest

P = 0xFFFFFFFF00000001


def ef_mul(a, b):
    return ((a[0] * b[0] + 7 * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def ef_add(a, b):
    return ((a[0] + b[0]) % P, (a[1] + b[1]) % P)


def ef_pow(a, e):
    r = (1, 0)
    while e:
        if e & 1:
            r = ef_mul(r, a)
        a = ef_mul(a, a)
        e >>= 1
    return r


def rand_ef(oracle, seed, count):
    v = oracle.gen_uniform(seed, 2 * count) % np.uint64(P)
    return [(int(v[2 * i]), int(v[2 * i + 1])) for i in range(count)]


def horner(table, z):
    acc = (0, 0)
    for x in reversed(range(len(table))):
        acc = ef_add(ef_mul(acc, z), table[x])
    return acc


@pytest.mark.parametrize("n,m,q", [(1, 1, 0), (3, 0, 2), (5, 2, 3), (8, 2, 6), (10, 1, 4)])
def test_gamma_zero_keeps_the_first_constraint(oracle, n, m, q):
    pts = np.array(rand_ef(oracle, 10 + n, m * n), np.uint64).reshape(m, n, 2) if m else []
    sel = np.array(rand_ef(oracle, 20 + n, q), np.uint64) if q else []
    w = oracle.constraint_weights(pts, sel, [0, 0], n)
    if m:
        assert (w == oracle.eq_table(pts[0])).all()
    else:
        z = (int(sel[0][0]), int(sel[0][1]))
        assert all(tuple(int(v) for v in w[x]) == ef_pow(z, x) for x in range(1 << n))


@pytest.mark.parametrize("n", [1, 4, 9])
def test_select_weights_are_powers(oracle, n):
    z = rand_ef(oracle, 30 + n, 1)[0]
    w = oracle.constraint_weights([], np.array([z], np.uint64), [5, 9], n)
    for x in range(1 << n):
        # z^x from the bits of x: bit b contributes z^(2^b)
        e = (1, 0)
        for b in range(n):
            if x >> b & 1:
                e = ef_mul(e, ef_pow(z, 1 << b))
        assert tuple(int(v) for v in w[x]) == e


@pytest.mark.parametrize("n,m,q", [(4, 2, 3), (7, 2, 5), (9, 3, 8)])
def test_weighted_sum_is_the_batched_claim(oracle, n, m, q):
    f = rand_ef(oracle, 40 + n, 1 << n)
    pts = np.array(rand_ef(oracle, 50 + n, m * n), np.uint64).reshape(m, n, 2)
    sel = rand_ef(oracle, 60 + n, q)
    gamma = rand_ef(oracle, 70 + n, 1)[0]
    w = oracle.constraint_weights(pts, np.array(sel, np.uint64), np.array(gamma, np.uint64), n)
    lhs = (0, 0)
    for x in range(1 << n):
        lhs = ef_add(lhs, ef_mul(f[x], (int(w[x][0]), int(w[x][1]))))
    fa = np.array(f, np.uint64).reshape(-1)
    rhs, g = (0, 0), (1, 0)
    for j in range(m):
        ans = oracle.mle_eval(fa, pts[j], True)
        rhs = ef_add(rhs, ef_mul(g, (int(ans[0]), int(ans[1]))))
        g = ef_mul(g, gamma)
    for z in sel:
        rhs = ef_add(rhs, ef_mul(g, horner(f, z)))
        g = ef_mul(g, gamma)
    assert lhs == rhs


def test_polynomial_in_gamma(oracle):
    # w(gamma) = sum_c gamma^c T_c: recover T_0..T_2 from three gammas (Vandermonde)
    n, m, q = 5, 1, 2
    pts = np.array(rand_ef(oracle, 80, m * n), np.uint64).reshape(m, n, 2)
    sel = rand_ef(oracle, 81, q)
    gs = [(2, 0), (3, 0), (5, 0)]
    ws = [oracle.constraint_weights(pts, np.array(sel, np.uint64), np.array(g, np.uint64), n) for g in gs]
    t0 = oracle.eq_table(pts[0])
    for x in (0, 1, 7, 31):
        # T_c(x) for the three constraints, then each w at x is sum_c g^c T_c(x)
        T = [(int(t0[x][0]), int(t0[x][1])), ef_pow(sel[0], x), ef_pow(sel[1], x)]
        for g, w in zip(gs, ws):
            exp = (0, 0)
            for c, tc in enumerate(T):
                exp = ef_add(exp, ef_mul(ef_pow(g, c), tc))
            assert tuple(int(v) for v in w[x]) == exp
