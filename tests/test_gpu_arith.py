"""The device forms of the field arithmetic and of the Poseidon2 building
blocks, run on the GPU (tests/gpu_arith/arith.hip) on crafted operands that
reach their rare corrections (second wraps and borrows, products whose
reduction borrows, halves sums that wrap), against python integers and the
oracle. The host emulation of the device code runs the portable C forms;
these are the inline-assembly forms the kernels execute."""
import random

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = 0xFFFFFFFF00000001
M = (1 << 64) - 1


def _lib():
    from tests.gpu_arith import build as B

    return B.load()


def _p(a):
    from tests.emu.emu import ptr

    return ptr(a)


def _edge_values():
    v = {0, 1, 2, 3, P - 2, P - 1, P, P + 1, P + 2, M, M - 1, M - 2, 2**32 - 1, 2**32, 2**32 + 1,
         2**63, 2**63 - 1, P - 2**32, 2**64 - 2**32, 2**64 - 2**33, 0xFFFFFFFE00000002, 7, 2**31}
    v |= {1 << k for k in range(64)}
    v |= {M - (1 << k) for k in range(64)}
    return sorted(v)


def _mid_carry(a, b):
    """1 when X.hi + k = 2^32 for X = a1 b0 + a0 b1 mod 2^64 and k the carry
    of P.hi + X.lo, P = a0 b0 (32-bit halves a = a0 + a1 2^32)."""
    a0, a1, b0, b1 = a & 0xFFFFFFFF, a >> 32, b & 0xFFFFFFFF, b >> 32
    x = (a1 * b0 + a0 * b1) & M
    k = (((a0 * b0) >> 32) + (x & 0xFFFFFFFF)) >> 32
    return ((x >> 32) + k) >> 32


def test_binary_ops_on_edges_and_random(native):
    print("CASE gpu arith binary", flush=True)
    L = _lib()
    k = L.arith_ops()
    edge = _edge_values()
    pairs = [(a, b) for a in edge for b in edge]
    rng = random.Random(21)
    pairs += [(rng.getrandbits(64), rng.getrandbits(64)) for _ in range(20000)]
    # products that are a multiple of 2^96 plus a little (the reduction's borrow)
    pairs += [(1 << a, 1 << (96 - a)) for a in range(33, 64)]
    pairs += [((1 << a) + 1, 1 << (96 - a)) for a in range(33, 64)]
    # products and squares whose middle partial products sum to just below
    # 2^64 (X = a1 b0 + a0 b1 with X.hi = 2^32 - 1) and take a carry from
    # P.hi + X.lo (P = a0 b0): the product's 2^96 term is formed from carries
    mid = [((a1 << 32) | 0xFFFFFFFF, ((2**32 + 1 - a1) << 32) | 0xFFFFFFFF) for a1 in range(2, 2**32, 2**32 // 64)]
    sq = sorted({(((((2**64 - 2**32 + j) // (2 * a0)) & 0xFFFFFFFF) + 1) << 32) | a0
                 for a0 in range(2**32 - 256, 2**32) for j in range(0, 2**32, 2**28)})
    sq = [s for s in sq if _mid_carry(s, s)]
    assert sum(_mid_carry(x, y) for x, y in mid) == len(mid) and len(sq) >= 64
    pairs += mid + [(s, s) for s in sq[:256]]
    a = np.array([x for x, _ in pairs], np.uint64)
    b = np.array([y for _, y in pairs], np.uint64)
    out = np.zeros(len(pairs) * k, np.uint64)
    assert L.arith_binary(_p(a), _p(b), _p(out), len(pairs)) == 0
    out = out.reshape(len(pairs), k)
    i24 = pow(1 << 24, P - 2, P)
    for n, (x, y) in enumerate(pairs):
        want = [(x + y) % P, (x - y) % P, x * y % P, x * x % P, (x << 24) % P, (x << 48) % P, x * i24 % P,
                ((x >> 29) + ((y >> 29) << 32)) % P, ((x >> 29) + ((y >> 29) << 32)) % P, x * y % P, x * x % P,
                7 * x % P, 8 * x * y % P, (x * x + y * y) % P, x * y % P, y * y % P]
        got = [int(v) for v in out[n]]
        assert got == want, (hex(x), hex(y), got, want)


def _states(rng, n_random):
    edge = [0, 1, 2, P - 1, P, P + 1, M, M - 1, 2**32 - 1, 2**32, 2**63, 2**63 - 1,
            0xFFFFFFFF00000000, 0x00000000FFFFFFFF, 0xFFFFFFFE00000002, 7, 2**31]
    states = [[v] * 16 for v in edge]
    for _ in range(n_random):
        states.append([rng.choice(edge) if rng.random() < 0.5 else rng.getrandbits(64) for _ in range(16)])
    return np.array(states, np.uint64)


def _run_states(st, mode, rc, consts):
    init, final, internal, diag15 = consts
    ext = np.concatenate([np.asarray(init, np.uint64), np.asarray(final, np.uint64)])
    s = np.ascontiguousarray(st.copy())
    assert _lib().arith_states(_p(s), s.shape[0], mode, rc, _p(ext), _p(np.ascontiguousarray(internal, np.uint64)),
                               diag15) == 0
    return s


def _canon(st):
    return np.array([[int(v) % P for v in row] for row in st], np.uint64)


def test_mds_and_internal_round_edges(native, oracle):
    print("CASE gpu arith p2 layers", flush=True)
    rng = random.Random(22)
    st = _states(rng, 200)
    consts = oracle.p2_constants()
    got = _run_states(st, 0, 0, consts)
    for row, g in zip(_canon(st), got):
        assert (g == oracle.p2_mds_light(row)).all()
    for rc in (0, 1, P - 1, int(consts[2][5])):
        got = _run_states(st, 1, rc, consts)
        for row, g in zip(_canon(st), got):
            ref = row.copy()
            ref[0] = pow((int(ref[0]) + rc) % P, 7, P)
            assert (g == oracle.p2_internal_linear(ref)).all(), (row, rc)


@pytest.mark.parametrize("mode", [2, 3])
def test_permutation_one_lane_and_one_row(native, oracle, mode):
    """p2_permute (one state per lane) and p2_permute_x16 (one state per
    16-lane row) on edge and random states."""
    print("CASE gpu arith permutation mode", mode, flush=True)
    rng = random.Random(23 + mode)
    st = _states(rng, 300)
    got = _run_states(st, mode, 0, oracle.p2_constants())
    for row, g in zip(_canon(st), got):
        assert (g == oracle.p2_permute(row)).all()


def test_permutation_general_diagonal(native, oracle):
    """A diag15 other than 2^-32: the general-multiply lane form (one state
    per lane) and the diagonal table (one state per row) against the oracle
    with the same constants."""
    print("CASE gpu arith permutation diag15", flush=True)
    a, b, c, d = oracle.p2_constants()
    rng = random.Random(29)
    st = _states(rng, 100)
    try:
        oracle.p2_set_constants(a, b, c, 12345)
        for mode in (3, 4):
            got = _run_states(st, mode, 0, (a, b, c, 12345))
            for row, g in zip(_canon(st), got):
                assert (g == oracle.p2_permute(row)).all(), mode
    finally:
        oracle.p2_set_constants(a, b, c, d)
