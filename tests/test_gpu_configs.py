"""The five workloads on the GPU against the oracle.

Configs 1, 2 and 5 are compared bit for bit at their full sizes (codewords,
every digest layer, roots, folded tables, openings). Configs 3 and 4 are
compared bit for bit on scaled-down shapes that take the same kernel paths,
and at full size through size-independent properties: the inverse DFT of the
codeword returns the zero-padded input, sampled codeword entries equal direct
polynomial evaluation, sampled digests equal the oracle hash of their
children, sampled opening paths verify against the root, and sampled folded
entries equal the oracle fold of their rows."""
import numpy as np
import pytest

from zkie_amd import configs as C
from zkie_amd import pipeline as PL
from zkie_amd._native import DeviceBuffer, check, p

pytestmark = pytest.mark.gpu

P = 0xFFFFFFFF00000001


def _case(*a):
    print("CASE", *a, flush=True)


def oracle_workload(O, wl: C.Workload, data: np.ndarray):
    """The same pipeline composed from oracle functions."""
    res = {"rounds": [], "fold": None, "tables": []}
    cw = O.lde_batch(data, wl.log_blowup)
    layers, root = O.merkle_commit(cw)
    res["rounds"].append((cw, layers, root))
    k = wl.fold_k
    if k and wl.rounds == 0:
        res["fold"] = O.fold_rows(cw, k, C.challenges(k), False)
    if wl.rounds:
        ch = C.challenges(k * wl.rounds)
        table, ext = data, False
        for r in range(wl.rounds):
            folded = O.fold_rows(table, k, ch[k * r:k * (r + 1)], ext)  # (rows, 2)
            res["tables"].append(folded)
            coeff = folded.reshape(-1, 2 << k)
            cw = O.lde_batch(coeff, wl.log_blowup)
            layers, root = O.merkle_commit(cw)
            res["rounds"].append((cw, layers, root))
            table, ext = coeff, True
    return res


def compare_full(O, wl, data, out, ref):
    assert len(out.rounds) == len(ref["rounds"])
    g = C.XorShift64(C.SEED_QUERIES)
    for rnd, (cw, layers, root) in zip(out.rounds, ref["rounds"]):
        assert (rnd.codeword.download().reshape(cw.shape) == cw).all()
        got = rnd.tree.layers()
        assert len(got) == len(layers)
        for a, b in zip(got, layers):
            assert (a == b).all()
        assert (rnd.tree.root == root).all()
        if wl.queries:
            idx = C.query_indices(wl.queries, rnd.rows, g)
            assert (rnd.queries == idx).all()
            assert (rnd.opened_rows == cw[idx.astype(np.int64)]).all()
            for k, i in enumerate(idx):
                assert (rnd.paths[k] == O.merkle_open(layers, rnd.rows, int(i))).all()
                assert O.merkle_verify(root, rnd.rows, int(i), rnd.opened_rows[k], rnd.paths[k])
            assert (rnd.pruned == O.merkle_open_pruned(layers, rnd.rows, idx)).all()
    if ref["fold"] is not None:
        assert (out.fold.download().reshape(-1, 2) == ref["fold"]).all()
    for (buf, n), t in zip(out.tables, ref["tables"]):
        assert (buf.download().reshape(-1, 2) == t).all()


@pytest.mark.parametrize("number,rows", [(1, None), (2, None), (5, None), (3, 1 << 18), (3, 1 << 10),
                                         (4, 1 << 12), (5, 1 << 12)])
def test_workload_bit_exact(native, oracle, number, rows):
    wl = C.CONFIGS[number] if rows is None else C.CONFIGS[number].scaled(rows)
    _case("workload", wl.name)
    data = PL.workload_inputs(wl)
    assert (data.reshape(-1) == {0: oracle.gen_uniform, 1: oracle.gen_i16, 2: oracle.gen_i8,
                                 3: oracle.gen_gauss_i16}[wl.kind](C.SEED_DATA, wl.elems)).all()
    d_in = DeviceBuffer.from_array(data)
    out = PL.run_workload(wl, d_in)
    ref = oracle_workload(oracle, wl, data)
    compare_full(oracle, wl, data, out, ref)


def property_checks(native, oracle, wl, data, out, rng, samples=24):
    rnd = out.rounds[0]
    n, w = rnd.rows, rnd.width
    # 1) the inverse DFT of the whole codeword is the zero-padded input
    lg = n.bit_length() - 1
    chk = DeviceBuffer(n * w)
    check(native.load().zkie_memcpy_dtod(chk.addr, rnd.codeword.addr, n * w * 8, None), "copy")
    check(native.load().zkie_idft_batch(chk.addr, lg, w, None), "idft")
    back = chk.download().reshape(n, w)
    assert (back[: wl.rows] == data).all()
    assert not back[wl.rows:].any()
    del back, chk
    # 2) sampled codeword entries = direct evaluation at w_n^t
    g = oracle.two_adic_generator(lg)
    for _ in range(3):
        t, c = int(rng.integers(n)), int(rng.integers(w))
        val = rnd.codeword.download(1, t * w + c)[0]
        assert int(val) == oracle.poly_eval(data, c, pow(g, t, P))
    # 3) sampled leaves and internal nodes against the oracle hash
    offs, acc = [], 0
    for ln in rnd.tree.layer_lens:
        offs.append(acc)
        acc += ln * 8
    for _ in range(samples):
        i = int(rng.integers(n))
        row = rnd.codeword.download(w, i * w)
        assert (rnd.tree.d_layers.download(8, offs[0] + 8 * i) == oracle.leaf_hash(row)).all()
    for lvl in range(1, len(rnd.tree.layer_lens)):
        for _ in range(4):
            j = int(rng.integers(rnd.tree.layer_lens[lvl]))
            kids = rnd.tree.d_layers.download(16, offs[lvl - 1] + 16 * j)
            par = rnd.tree.d_layers.download(8, offs[lvl] + 8 * j)
            assert (par == oracle.compress(kids[:8], kids[8:])).all()
    # 4) opening paths verify against the root
    idx = np.unique(rng.integers(0, n, size=samples).astype(np.uint64))
    from zkie_amd.pcs import HipMerkleTreeMmcs
    rows, paths = HipMerkleTreeMmcs().open_batches(idx, rnd.tree)
    for k, i in enumerate(idx):
        assert oracle.merkle_verify(rnd.tree.root, n, int(i), rows[k], paths[k])
    # 5) sampled fold entries
    if out.fold is not None:
        ch = C.challenges(wl.fold_k)
        for k, i in enumerate(idx[:8]):
            got = out.fold.download(2, 2 * int(i))
            assert (got == oracle.fold_rows(rows[k:k + 1], wl.fold_k, ch, False)[0]).all()


@pytest.mark.parametrize("number", [3, 4])
def test_workload_full_size_properties(native, oracle, number):
    wl = C.CONFIGS[number]
    _case("full-size properties", wl.name)
    data = PL.workload_inputs(wl)
    d_in = DeviceBuffer.from_array(data)
    out = PL.run_workload(wl, d_in, with_openings=False)
    property_checks(native, oracle, wl, data, out, np.random.default_rng(number))


def test_largest_fused_commit_properties(native, oracle):
    """Configuration 3's pipeline at twice its rows (2^25 x 16, codeword
    2^27 x 16 = 16 GiB): the transform splits into three 9-bit passes, so the
    last one is fused with the leaf hash in 512-thread workgroups (one per
    2^9-row tile, 2^18 of them), checked through the same size-independent
    properties."""
    wl = C.CONFIGS[3].scaled(1 << 25)
    _case("full-size properties", wl.name)
    data = PL.workload_inputs(wl)
    d_in = DeviceBuffer.from_array(data)
    out = PL.run_workload(wl, d_in, with_openings=False)
    property_checks(native, oracle, wl, data, out, np.random.default_rng(25))


@pytest.mark.gpu
def test_whir_rounds_ood_and_stir_full_size(native, oracle):
    """The WHIR-shaped workload at full size: every round's sumcheck weights
    (the initial evaluation constraint, then the folded weights plus each
    round's batched OOD + STIR constraint) and round polynomials equal the
    oracle's, every round's out-of-domain
    answers equal the oracle's multilinear evaluation of the folded table,
    the STIR row folds equal the oracle's fold of the opened rows, and each
    row fold agrees with the next codeword (FRI/STIR consistency): the fold
    of row t of a codeword with N rows is sum_c w_N^(c t) C'[t mod N/2^k][c]."""
    wl = C.CONFIGS[5]
    print("CASE whir rounds OOD + STIR + batched constraints", wl.name, flush=True)
    k = wl.fold_k
    out = PL.run_workload(wl, DeviceBuffer.from_array(PL.workload_inputs(wl)), with_openings=False)
    assert len(out.rounds) == wl.rounds + 1
    weights = None
    for r in range(1, len(out.rounds)):
        prev, rnd = out.rounds[r - 1], out.rounds[r]
        table, t_entries = out.tables[r - 1]
        tab = table.download()
        n_vars = t_entries.bit_length() - 1
        for z, ans in zip(rnd.ood_points, rnd.ood_answers):
            assert (ans == oracle.mle_eval(tab, C.ef_pow2_chain(z, n_vars), True)).all()
        # the sumcheck rounds that folded the previous table, with the running
        # weights: the initial evaluation constraint, then after every round
        # the folded weights plus that round's batched constraint
        ch = C.challenges(k * wl.rounds)[k * (r - 1):k * r]
        prev_tab = (PL.workload_inputs(wl).reshape(-1) if r == 1 else out.tables[r - 2][0].download())
        if r == 1:
            weights = oracle.eq_table(rnd.weight_point)
        polys, f_out, h_out = oracle.sumcheck_prove(prev_tab, r > 1, weights, ch)
        assert (rnd.sumcheck_polys == polys).all()
        assert (tab.reshape(-1, 2) == f_out).all()
        eq_pts = np.array([C.ef_pow2_chain(z, n_vars) for z in rnd.ood_points], np.uint64)
        w_c = oracle.constraint_weights(eq_pts, rnd.stir_points, rnd.gamma, n_vars)
        weights = ((h_out.astype(object) + w_c.astype(object)) % C.P).astype(np.uint64)
        assert (rnd.weights.download().reshape(-1, 2) == weights).all()
        idx = rnd.stir_indices.astype(np.int64)
        prev_cw = prev.codeword.download().reshape(prev.rows, prev.width)
        ch = C.challenges(k * wl.rounds)[k * (r - 1):k * r]
        assert (rnd.stir_folds == oracle.fold_rows(prev_cw[idx], k, ch, r > 1)).all()
        # consistency with the next codeword (EF rows of 2^k entries)
        N, M = prev.rows, rnd.rows
        cw = rnd.codeword.download().reshape(M, 1 << k, 2)
        w_n = pow(7, (C.P - 1) // N, C.P)
        for t, f in zip(idx[:16], rnd.stir_folds[:16]):
            acc0 = acc1 = 0
            for c in range(1 << k):
                wc = pow(w_n, int(c * t), C.P)
                acc0 = (acc0 + wc * int(cw[t % M, c, 0])) % C.P
                acc1 = (acc1 + wc * int(cw[t % M, c, 1])) % C.P
            assert [acc0, acc1] == [int(f[0]), int(f[1])]


def _ef_mul(a, b):
    return ((a[0] * b[0] + 7 * a[1] * b[1]) % C.P, (a[0] * b[1] + a[1] * b[0]) % C.P)


def _poly_at(poly, x):
    """c0 + c1 x + c2 x^2 in EF."""
    c = [(int(poly[i][0]), int(poly[i][1])) for i in range(3)]
    x = (int(x[0]), int(x[1]))
    acc = c[2]
    for i in (1, 0):
        acc = _ef_mul(acc, x)
        acc = ((acc[0] + c[i][0]) % C.P, (acc[1] + c[i][1]) % C.P)
    return acc


def test_whir_batched_constraints_full_size(native, oracle):
    """The WHIR-shaped workload at full size, checked the way its verifier
    combines the claims (p3-whir verifier/mod.rs:158-180): the sum over the
    round table of table x batched weights equals the batched claim
    sum_j gamma^j ood_j + sum_k gamma^(m+k) stir_k (the STIR claims are the
    queried-row folds, the values of the table's polynomial at w_N^index), and
    each round's first sumcheck polynomial sums over {0, 1} to the previous
    sumcheck's final claim plus that batched claim."""
    from zkie_amd import pcs

    wl = C.CONFIGS[5]
    print("CASE whir batched constraints", wl.name, flush=True)
    k = wl.fold_k
    out = PL.run_workload(wl, DeviceBuffer.from_array(PL.workload_inputs(wl)), with_openings=False)
    ch = C.challenges(k * wl.rounds)
    for r in range(1, len(out.rounds)):
        rnd = out.rounds[r]
        table, t_entries = out.tables[r - 1]
        n_vars = t_entries.bit_length() - 1
        eq_pts = np.array([C.ef_pow2_chain(z, n_vars) for z in rnd.ood_points], np.uint64)
        w = pcs.constraint_weights(eq_pts, rnd.stir_points, rnd.gamma, n_vars)
        y = np.zeros(6, np.uint64)
        check(native.load().zkie_sumcheck_round(table.addr, 1, w.addr, n_vars, p(y), None), "round")
        c0, c1, c2 = (int(y[0]), int(y[1])), (int(y[2]), int(y[3])), (int(y[4]), int(y[5]))
        # p(0) + p(1) = 2 c0 + c1 + c2
        total = ((2 * c0[0] + c1[0] + c2[0]) % C.P, (2 * c0[1] + c1[1] + c2[1]) % C.P)
        assert total == (int(rnd.claim[0]), int(rnd.claim[1])), r
        if r + 1 < len(out.rounds):
            # next round's sumcheck: its first polynomial sums to the claim
            # left by this round's sumcheck plus this round's batched claim
            last = _poly_at(rnd.sumcheck_polys[-1], ch[k * (r - 1) + k - 1])
            nxt = out.rounds[r + 1].sumcheck_polys[0]
            s0 = _poly_at(nxt, (0, 0))
            s1 = _poly_at(nxt, (1, 0))
            got = ((s0[0] + s1[0]) % C.P, (s0[1] + s1[1]) % C.P)
            want = ((last[0] + int(rnd.claim[0])) % C.P, (last[1] + int(rnd.claim[1])) % C.P)
            assert got == want, r
