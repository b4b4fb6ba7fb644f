"""The device code of libzkie_hip.so, built for the host (tests/emu/emu.cpp),
checked against the oracle: the 32-bit-limb Goldilocks arithmetic on edge
and non-canonical values, the permutation in both diagonal modes, and the NTT
pass kernels (every workgroup and thread executed with bounds checks)."""
import random

import numpy as np
import pytest

from tests.emu.emu import ptr

P = 0xFFFFFFFF00000001
M = (1 << 64) - 1
EDGE = [0, 1, 2, P - 1, P, P + 1, M, M - 1, 2**32 - 1, 2**32, 2**63, P - 2**32, 2**64 - 2**32]


def test_arithmetic(emu):
    rng = random.Random(1)
    vals = EDGE + [rng.getrandbits(64) for _ in range(4000)]
    for a in vals:
        b = rng.choice(vals)
        assert emu.emu_gl_canon(emu.emu_gl_add(a, b)) == (a + b) % P
        assert emu.emu_gl_canon(emu.emu_gl_sub(a, b)) == (a - b) % P
        assert emu.emu_gl_canon(emu.emu_gl_mul(a, b)) == (a * b) % P
        assert emu.emu_gl_canon(emu.emu_gl_sqr(a)) == (a * a) % P
        assert emu.emu_gl_canon(emu.emu_gl_halve(a)) == a * pow(2, P - 2, P) % P
        for k in (3, 4, 5, 32):
            assert emu.emu_gl_canon(emu.emu_gl_inv_pow2(a, k)) == a * pow(2**k, P - 2, P) % P
        assert emu.emu_gl_canon_fast(a) == a % P
        for sh in (1, 2):
            assert emu.emu_gl_canon(emu.emu_gl_shl(a, sh)) == (a << sh) % P
            assert emu.emu_gl_canon(emu.emu_gl_add_shl(b, a, sh)) == (b + (a << sh)) % P
        if b < P:
            assert emu.emu_gl_canon(emu.emu_gl_add_small(a, b)) == (a + b) % P
    for n in (1, 16, 36, 1000):
        x = np.array([rng.getrandbits(64) for _ in range(n)], np.uint64)
        assert emu.emu_gl_canon(emu.emu_acc_sum(ptr(x), n)) == sum(int(v) for v in x) % P


def test_dot_accumulator(emu):
    """DotAcc (exact 32 x 32 partial-product sums, one reduction) against
    python integers, with all-ones operands that force every carry."""
    import random
    rng = random.Random(5)
    cases = [[(2**64 - 1, 2**64 - 1)] * 128, [(2**64 - 1, P - 1)] * 65, [(0, 5)] * 3, []]
    for n in (1, 2, 16, 64, 128):
        cases.append([(rng.getrandbits(64), rng.getrandbits(64)) for _ in range(n)])
    for pairs in cases:
        e = np.array([a for a, _ in pairs] or [0], np.uint64)
        x = np.array([b for _, b in pairs] or [0], np.uint64)
        want = sum(a * b for a, b in pairs) % P
        assert emu.emu_dot(ptr(e), ptr(x), len(pairs)) == want


@pytest.mark.parametrize("fast", [0, 1])
def test_permutation(emu, oracle, fast):
    a, b, c, d = oracle.p2_constants()
    rng = random.Random(2 + fast)
    for _ in range(30):
        st = np.array([rng.getrandbits(64) % P for _ in range(16)], np.uint64)
        ref = oracle.p2_permute(st)
        s = st.copy()
        emu.emu_p2_permute(ptr(s), ptr(a), ptr(b), ptr(c), d, fast)
        assert (s == ref).all()
    # non-canonical inputs (values in [p, 2^64)) reduce to the same result
    st = np.array([P + i for i in range(16)], np.uint64)
    s = st.copy()
    emu.emu_p2_permute(ptr(s), ptr(a), ptr(b), ptr(c), d, fast)
    assert (s == oracle.p2_permute(np.arange(16, dtype=np.uint64))).all()


@pytest.mark.parametrize("big", [0xFFFFFFBFFFFFFFFF, 0xFFFFFFC000000000, 0xFFFFFFFF00000000])
def test_permutation_constant_bound(emu, oracle, big):
    """Linear-layer constants at the fast path's bound: just below 2^64 - 2^38
    the constants join the low sums whole (edge states make those sums as
    large as they get); at or above it the general path is chosen."""
    import random
    rng = random.Random(41)
    a, b, c, d = oracle.p2_constants()
    a2, b2, c2 = a.copy(), b.copy(), c.copy()
    a2[:] = big
    b2[:] = big
    c2[0] = big
    try:
        oracle.p2_set_constants(a2, b2, c2, d)
        for st in _edge_states(rng)[:30]:
            s = np.array(st, np.uint64)
            emu.emu_p2_permute(ptr(s), ptr(a2), ptr(b2), ptr(c2), d, 1)
            assert (s == oracle.p2_permute(np.array([v % P for v in st], np.uint64))).all(), (hex(big), st)
    finally:
        oracle.p2_set_constants(a, b, c, d)


def _edge_states(rng):
    """States that hit the ends of every lane form: all-ones words, values
    at and above p, halves of 0 and 2^32 - 1, powers of two, random."""
    edge = [0, 1, 2, P - 1, P, P + 1, 2**64 - 1, 2**64 - 2, 2**32 - 1, 2**32, 2**63, 2**63 - 1,
            0xFFFFFFFF00000000, 0x00000000FFFFFFFF, 0xFFFFFFFE00000002, 7, 2**31]
    states = [[v] * 16 for v in edge]
    for _ in range(40):
        states.append([rng.choice(edge) if rng.random() < 0.5 else rng.getrandbits(64) for _ in range(16)])
    return states


@pytest.mark.parametrize("fast", [0, 1])
def test_internal_round_edges(emu, oracle, fast):
    """The internal round's lane forms (halves sums, complements, 2^-k splits)
    against the oracle's round on edge states, including non-canonical input."""
    import random
    rng = random.Random(11 + fast)
    a, b, c, d = oracle.p2_constants()
    for st in _edge_states(rng):
        for rc in (0, 1, P - 1, int(c[5])):
            s = np.array(st, np.uint64)
            emu.emu_p2_internal_round(ptr(s), rc, d, fast)
            ref = np.array([v % P for v in st], np.uint64)
            ref[0] = pow((int(ref[0]) + rc) % P, 7, P)
            ref = oracle.p2_internal_linear(ref)
            assert (s == ref).all(), (st, rc)


def test_mds_light_edges(emu, oracle):
    import random
    rng = random.Random(13)
    for st in _edge_states(rng):
        s = np.array(st, np.uint64)
        emu.emu_p2_mds_light(ptr(s))
        assert (s == oracle.p2_mds_light(np.array([v % P for v in st], np.uint64))).all(), st


@pytest.mark.parametrize("lg,w", [(1, 1), (3, 1), (5, 3), (9, 16), (10, 1), (10, 16), (12, 5),
                                  (14, 32), (16, 8), (19, 1), (18, 16), (13, 128)])
def test_dft_passes(emu, oracle, lg, w):
    x = oracle.gen_uniform(lg * 100 + w, (1 << lg) * w).reshape(1 << lg, w)
    y = x.copy()
    assert emu.emu_dft(ptr(y), lg, w, 0, 256) == 0
    assert (y == oracle.dft_batch(x)).all()
    assert emu.emu_dft(ptr(y), lg, w, 1, 256) == 0
    assert (y == x).all()


# 512 threads per workgroup, the kernel's own count (one round per step).
@pytest.mark.parametrize("lg,w", [(13, 16), (18, 16), (10, 16), (12, 32), (9, 16), (14, 8), (19, 16)])
def test_dft_passes_kernel_threads(emu, oracle, lg, w):
    x = oracle.gen_uniform(lg * 10 + w, (1 << lg) * w).reshape(1 << lg, w)
    y = x.copy()
    assert emu.emu_dft(ptr(y), lg, w, 0, 512) == 0
    assert (y == oracle.dft_batch(x)).all()
    assert emu.emu_dft(ptr(y), lg, w, 1, 512) == 0
    assert (y == x).all()


@pytest.mark.parametrize("lg,w,lb", [(4, 1, 2), (10, 16, 2), (16, 1, 2), (9, 32, 3), (12, 16, 1),
                                     (16, 16, 2), (14, 16, 3), (11, 128, 1), (7, 1, 2), (2, 3, 4)])
def test_lde_passes(emu, oracle, lg, w, lb):
    x = oracle.gen_uniform(7, (1 << lg) * w).reshape(1 << lg, w)
    out = np.zeros(((1 << lg) << lb, w), np.uint64)
    assert emu.emu_lde(ptr(x), 1 << lg, w, lb, ptr(out), 256) == 0
    assert (out == oracle.lde_batch(x, lb)).all()


@pytest.mark.parametrize("lg,w,lb", [(16, 16, 2), (14, 16, 3), (17, 16, 2)])
def test_lde_passes_kernel_threads(emu, oracle, lg, w, lb):
    x = oracle.gen_uniform(8, (1 << lg) * w).reshape(1 << lg, w)
    out = np.zeros(((1 << lg) << lb, w), np.uint64)
    assert emu.emu_lde(ptr(x), 1 << lg, w, lb, ptr(out), 512) == 0
    assert (out == oracle.lde_batch(x, lb)).all()


@pytest.mark.parametrize("lg,w,lb,rows", [(10, 16, 2, 300), (13, 16, 2, 5000), (12, 4, 1, 1), (7, 1, 3, 100),
                                          (5, 16, 2, 17), (12, 16, 2, 3000), (13, 1, 1, 4097)])
def test_lde_passes_ragged_rows(emu, oracle, lg, w, lb, rows):
    """The LDE of a batch commit: only the first `rows` input rows exist (the
    buffer ends there, every read is bounds-checked), the rest are zero."""
    x = oracle.gen_uniform(9 + rows, rows * w).reshape(rows, w)
    full = np.zeros((1 << lg, w), np.uint64)
    full[:rows] = x
    out = np.zeros(((1 << lg) << lb, w), np.uint64)
    assert emu.emu_lde_rows(ptr(x), 1 << lg, rows, w, lb, ptr(out), 512) == 0
    assert (out == oracle.lde_batch(full, lb)).all()


@pytest.mark.parametrize("n_vars,k,E", [(31, 4, 2), (32, 4, 2), (32, 1, 1), (31, 31, 2), (20, 3, 2)])
def test_prefix_transpose_index_at_full_size(emu, n_vars, k, E):
    """The Prefix-order transpose's index map (output word t reads word
    ((j 2^lrows + i) E + c) with t = (i 2^k + j) E + c) in 64 bits, at the
    largest tables (2^33 words for 32 EF variables), against Python integers
    on the first, last and scattered words; the map is a permutation of the
    words (source words distinct and in range on a dense sample)."""
    lrows = n_vars - k
    total = E << n_vars
    ts = [0, 1, E, total - 1, total - E, total // 2, total // 3] + [(total * q) // 97 for q in range(97)]
    for t in ts:
        c, e = t % E, t // E
        j, i = e % (1 << k), e >> k
        assert emu.emu_prefix_source(t, lrows, k, E) == ((j << lrows) + i) * E + c
    dense = [emu.emu_prefix_source(t, lrows, k, E) for t in range(total - 4096, total)]
    assert len(set(dense)) == len(dense) and max(dense) < total


@pytest.mark.parametrize("lg,lb", [(8, 2), (10, 2), (12, 2), (11, 3), (13, 3), (16, 2)])
def test_lde_last_pass_fused_with_leaf_hash(emu, oracle, lg, lb):
    """The fused last NTT pass + leaf hash of the commitment (last_leaf.hpp),
    at the kernel's thread count, for last passes of 5 to 9 bits: the
    codeword and the leaf digests equal the oracle's LDE and layer 0."""
    w = 16
    x = oracle.gen_uniform(9 + lg, (1 << lg) * w).reshape(1 << lg, w)
    n = (1 << lg) << lb
    out = np.zeros((n, w), np.uint64)
    dig = np.zeros((n, 8), np.uint64)
    a, b, c, d = oracle.p2_constants()
    assert emu.emu_lde_leaf(ptr(x), 1 << lg, w, lb, ptr(out), ptr(dig), ptr(a), ptr(b), ptr(c), d, 1) == 0
    cw = oracle.lde_batch(x, lb)
    assert (out == cw).all()
    layers, _ = oracle.merkle_commit(cw)
    assert (dig == layers[0].reshape(n, 8)).all()
