"""Pins of the oracle permutation.

The permutation is checked against (a) the addition-chain restatement of
poseidon2_merkle.cu in oracle/pyref.py, (b) a composition written here from
the Poseidon2 paper's definitions (eprint 2023/323: M_E = circ(2 M4, M4, M4,
M4), M_I = 1 1^T + diag(V), x^7, R_F = 8 split 4 + 4, R_P = 22) with explicit
matrix products over python integers, and (c) the sponge / truncation rules
of PaddingFreeSponge and TruncatedPermutation. The round constants are pinned
by the rand 0.10 SmallRng derivation (Xoshiro256++ / SplitMix64 vectors in
test_oracle_field.py) and by an independent python derivation; their
equality with p3's own values is not pinned by any reference fixture.
"""
import random

import numpy as np

from oracle import pyref

P = 0xFFFFFFFF00000001
M4 = [[2, 3, 1, 1], [1, 2, 3, 1], [1, 1, 2, 3], [3, 1, 1, 2]]


def _inv(x):
    return pow(x, P - 2, P)


def _V(diag15):
    i2, i8, i16, i32 = _inv(2), _inv(8), _inv(16), _inv(32)
    return [P - 2, 1, 2, i2, 3, 4, P - i2, P - 3, P - 4, i8, i16, i32, P - i8, P - i16, P - i32, diag15]


def _ME():
    m = [[0] * 16 for _ in range(16)]
    for bi in range(4):
        for bj in range(4):
            f = 2 if bi == bj else 1
            for r in range(4):
                for c in range(4):
                    m[4 * bi + r][4 * bj + c] = f * M4[r][c]
    return m


def _matvec(m, v):
    return [sum(m[i][j] * v[j] for j in range(16)) % P for i in range(16)]


def _paper_permute(state, consts):
    init, final, internal, diag15 = consts
    ME = _ME()
    V = _V(diag15)
    MI = [[(1 + (V[i] if i == j else 0)) % P for j in range(16)] for i in range(16)]
    st = _matvec(ME, [int(v) for v in state])
    for r in range(4):
        st = _matvec(ME, [pow((st[i] + init[16 * r + i]) % P, 7, P) for i in range(16)])
    for r in range(22):
        st[0] = pow((st[0] + internal[r]) % P, 7, P)
        st = _matvec(MI, st)
    for r in range(4):
        st = _matvec(ME, [pow((st[i] + final[16 * r + i]) % P, 7, P) for i in range(16)])
    return st


def test_constants_derivation(oracle):
    a, b, c, d = oracle.p2_constants()
    init, final, internal, diag15 = pyref.derive_constants()
    assert [int(x) for x in a] == init and [int(x) for x in b] == final
    assert [int(x) for x in c] == internal and d == diag15
    assert d == 0xFFFFFFFE00000002  # 2^-32, poseidon2_merkle.cu:34
    allc = init + final + internal
    assert all(x < P for x in allc) and len(set(allc)) == len(allc)


def test_mds_light_is_paper_external_matrix(oracle):
    rng = random.Random(1)
    ME = _ME()
    for _ in range(20):
        v = [rng.randrange(P) for _ in range(16)]
        assert [int(x) for x in oracle.p2_mds_light(v)] == _matvec(ME, v)


def test_internal_layer_is_one_plus_diag(oracle):
    rng = random.Random(2)
    V = _V(0xFFFFFFFE00000002)
    for _ in range(20):
        v = [rng.randrange(P) for _ in range(16)]
        s = sum(v) % P
        assert [int(x) for x in oracle.p2_internal_linear(v)] == [(s + V[i] * v[i]) % P for i in range(16)]


def test_permutation_three_formulations_agree(oracle):
    consts = pyref.derive_constants()
    perm = pyref.Poseidon2(consts)
    rng = random.Random(5)
    states = [[0] * 16, list(range(16)), [P - 1] * 16] + [[rng.randrange(P) for _ in range(16)] for _ in range(5)]
    for st in states:
        a = [int(x) for x in oracle.p2_permute(st)]
        assert a == perm.permute(st)
        assert a == _paper_permute(st, consts)


def test_sponge_rules(oracle):
    perm = pyref.Poseidon2()
    # empty input: no permutation, zero digest
    assert (oracle.leaf_hash([]) == 0).all()
    row = [int(v) for v in oracle.gen_uniform(3, 20)]
    # exactly one chunk: one permutation of [row, 0^8]
    assert [int(x) for x in oracle.leaf_hash(row[:8])] == perm.permute(row[:8] + [0] * 8)[:8]
    # partial second chunk overwrites only state[0..len]
    s = perm.permute(row[:8] + [0] * 8)
    s[:3] = row[8:11]
    assert [int(x) for x in oracle.leaf_hash(row[:11])] == perm.permute(s)[:8]
    # one element
    assert [int(x) for x in oracle.leaf_hash(row[:1])] == perm.permute([row[0]] + [0] * 15)[:8]


def test_compress_rule(oracle):
    perm = pyref.Poseidon2()
    l = [int(v) for v in oracle.gen_uniform(1, 8)]
    r = [int(v) for v in oracle.gen_uniform(2, 8)]
    assert [int(x) for x in oracle.compress(l, r)] == perm.permute(l + r)[:8]
