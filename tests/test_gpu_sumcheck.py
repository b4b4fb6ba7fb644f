"""GPU parity of the sumcheck rounds (common/sumcheck.rs:33-89 with EF
tables, the round polynomials of a WHIR round): the device round
polynomials and folded tables equal the oracle's bit for bit, the
round-by-round entry points compose to the all-rounds one, k rounds leave
the device table fold (zkie_fold_rows) over the low k variables, and
overlapping buffers are refused."""
import numpy as np
import pytest

P = 0xFFFFFFFF00000001
pytestmark = pytest.mark.gpu


def _tables(oracle, seed, t, f_ext):
    f = oracle.gen_uniform(seed, (2 if f_ext else 1) << t)
    h = oracle.gen_uniform(seed + 1, 2 << t)
    r = (oracle.gen_uniform(seed + 2, 2 * t) % np.uint64(P)).reshape(t, 2)
    return f, h, r


@pytest.mark.parametrize("f_ext", [False, True])
@pytest.mark.parametrize("t,rounds", [(1, 1), (2, 2), (5, 1), (5, 5), (9, 4), (13, 13), (18, 4),
                                      (20, 20), (22, 4)])
def test_prove_matches_oracle(native, oracle, t, rounds, f_ext):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE sumcheck_prove t={t} rounds={rounds} ext={f_ext}", flush=True)
    f, h, r = _tables(oracle, 1000 + 3 * t, t, f_ext)
    polys, f_out, h_out = pcs.sumcheck_prove(DeviceBuffer.from_array(f), f_ext, DeviceBuffer.from_array(h), t,
                                             r[:rounds])
    wp, wf, wh = oracle.sumcheck_prove(f, f_ext, h, r[:rounds])
    assert (polys == wp).all()
    assert (f_out.download().reshape(-1, 2) == wf).all()
    assert (h_out.download().reshape(-1, 2) == wh).all()


@pytest.mark.parametrize("f_ext", [False, True])
def test_round_entries_compose(native, oracle, f_ext):
    """zkie_sumcheck_round + zkie_sumcheck_fold round by round, as a prover
    whose challenges come from its transcript calls them."""
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE sumcheck rounds ext={f_ext}", flush=True)
    t = 11
    f, h, r = _tables(oracle, 1200, t, f_ext)
    wp, wf, wh = oracle.sumcheck_prove(f, f_ext, h, r)
    d_f, d_h, ext = DeviceBuffer.from_array(f), DeviceBuffer.from_array(h), f_ext
    for i in range(t):
        assert (pcs.sumcheck_round(d_f, ext, d_h, t - i) == wp[i]).all(), i
        d_f, d_h = pcs.sumcheck_fold(d_f, ext, d_h, t - i, r[i])
        ext = True
    assert (d_f.download().reshape(-1, 2) == wf).all() and (d_h.download().reshape(-1, 2) == wh).all()
    # the fold that also forms the next round's polynomial in the same pass
    d_f, d_h, ext = DeviceBuffer.from_array(f), DeviceBuffer.from_array(h), f_ext
    assert (pcs.sumcheck_round(d_f, ext, d_h, t) == wp[0]).all()
    for i in range(t - 1):
        d_f, d_h, poly = pcs.sumcheck_fold(d_f, ext, d_h, t - i, r[i], next_poly=True)
        assert (poly == wp[i + 1]).all(), i
        ext = True
    d_f, d_h = pcs.sumcheck_fold(d_f, ext, d_h, 1, r[t - 1])
    assert (d_f.download().reshape(-1, 2) == wf).all() and (d_h.download().reshape(-1, 2) == wh).all()


@pytest.mark.parametrize("f_ext", [False, True])
def test_rounds_leave_the_device_table_fold(native, oracle, f_ext):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE sumcheck vs fold_rows ext={f_ext}", flush=True)
    t, k = 16, 4
    f, h, r = _tables(oracle, 1300, t, f_ext)
    d_f = DeviceBuffer.from_array(f)
    _, f_out, _ = pcs.sumcheck_prove(d_f, f_ext, DeviceBuffer.from_array(h), t, r[:k])
    folded = DeviceBuffer(2 << (t - k))
    pcs.fold_rows_device(d_f, 1 << (t - k), k, r[:k], f_ext, folded)
    assert (f_out.download() == folded.download()).all()


def test_rejects_overlap_and_bad_sizes(native, oracle):
    from zkie_amd._native import DeviceBuffer, load

    print("CASE sumcheck arguments", flush=True)
    L = load()
    t = 6
    f, h, r = _tables(oracle, 1400, t, True)
    d_f, d_h = DeviceBuffer.from_array(f), DeviceBuffer.from_array(h)
    out = DeviceBuffer(2 << t)
    rr = np.ascontiguousarray(r[0])
    polys = np.zeros(6 * t, np.uint64)
    p = native.p
    assert L.zkie_sumcheck_fold(d_f.addr, 1, d_h.addr, t, p(rr), d_f.addr, out.addr, None, None) == -1
    assert L.zkie_sumcheck_fold(d_f.addr, 1, d_h.addr, t, p(rr), out.addr, out.addr + 8, None, None) == -1
    assert L.zkie_sumcheck_fold(d_f.addr, 1, d_h.addr, 1, p(rr), out.addr, out.addr + 64, p(polys),
                                None) == -1
    assert L.zkie_sumcheck_round(d_f.addr, 1, d_h.addr, 0, p(polys), None) == -1
    rs = np.ascontiguousarray(r.reshape(-1))
    assert L.zkie_sumcheck_prove(d_f.addr, 1, d_h.addr, t, t + 1, p(rs), p(polys), out.addr,
                                 out.addr + 2, None) == -1


@pytest.mark.parametrize("t", [0, 1, 2, 7, 16, 22])
def test_eq_table_matches_oracle(native, oracle, t):
    from zkie_amd import pcs

    print(f"CASE eq_table t={t}", flush=True)
    pt = (oracle.gen_uniform(1500 + t, 2 * t) % np.uint64(P)).reshape(t, 2)
    assert (pcs.eq_table(pt).download().reshape(-1, 2) == oracle.eq_table(pt)).all()


@pytest.mark.parametrize("n,m,q,acc", [(0, 1, 0, False), (3, 1, 2, False), (7, 0, 3, True), (8, 2, 5, True),
                                       (9, 2, 0, False), (12, 2, 100, False), (16, 5, 30, True),
                                       (18, 2, 128, True), (11, 0, 0, False), (11, 0, 0, True), (0, 150, 60, False),
                                       (0, 40, 200, True), (2, 60, 10, False)])
def test_constraint_weights_match_oracle(native, oracle, n, m, q, acc):
    """zkie_constraint_weights (the batched constraint of a WHIR round) equals
    the oracle bit for bit: tables split at 8 or more low bits, several
    launches when the points exceed one launch's arguments (m n + q > 96),
    added to or overwriting the running weights."""
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    print(f"CASE constraint_weights n={n} m={m} q={q} acc={acc}", flush=True)
    pts = (oracle.gen_uniform(3000 + n, 2 * m * n) % np.uint64(P)).reshape(m, n, 2)
    sel = (oracle.gen_uniform(3100 + n, 2 * q) % np.uint64(P)).reshape(q, 2)
    gamma = oracle.gen_uniform(3200 + n, 2) % np.uint64(P)
    base = oracle.gen_uniform(3300 + n, 2 << n) % np.uint64(P)
    d_w = DeviceBuffer.from_array(base)
    pcs.constraint_weights(pts, sel, gamma, n, d_w=d_w, accumulate=acc)
    exp = oracle.constraint_weights(pts if m else [], sel if q else [], gamma, n)
    if acc:
        exp = ((exp.astype(object) + base.reshape(-1, 2).astype(object)) % P).astype(np.uint64)
    assert (d_w.download().reshape(-1, 2) == exp).all()


def test_constraint_weights_on_a_stream(native, oracle):
    """Queued on a non-null stream after a kernel that writes the running
    weights, with nothing waiting for the host in between."""
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer, Stream

    print("CASE constraint_weights stream", flush=True)
    s = Stream()
    n = 14
    pt = (oracle.gen_uniform(3400, 2 * n) % np.uint64(P)).reshape(n, 2)
    sel = (oracle.gen_uniform(3401, 40) % np.uint64(P)).reshape(20, 2)
    gamma = np.array([3, 4], np.uint64)
    d_w = pcs.eq_table(pt, s.handle)
    pcs.constraint_weights([], sel, gamma, n, d_w=d_w, accumulate=True, stream=s.handle)
    s.synchronize()
    exp = (oracle.eq_table(pt).astype(object) + oracle.constraint_weights([], sel, gamma, n).astype(object)) % P
    assert (d_w.download().reshape(-1, 2) == exp.astype(np.uint64)).all()
