"""GPU parity of every entry point against the oracle on seeded inputs.

Bit-exact comparisons (integer work). Each case prints its name first so a
failing device run names the case it was in."""
import ctypes

import numpy as np
import pytest

from zkie_amd import pcs
from zkie_amd._native import DeviceBuffer, check, p

pytestmark = pytest.mark.gpu

P = 0xFFFFFFFF00000001


def _case(*a):
    print("CASE", *a, flush=True)


def test_default_constants_match_oracle(native, oracle):
    _case("constants")
    g = native.p2_default_constants()
    o = oracle.p2_constants()
    for x, y in zip(g[:3], o[:3]):
        assert (x == y).all()
    assert g[3] == o[3]


@pytest.mark.parametrize("lg,w", [(1, 1), (4, 3), (9, 16), (10, 1), (13, 16), (16, 5), (19, 16),
                                  (20, 1), (14, 128), (12, 32), (18, 24)])
def test_dft_and_inverse(native, oracle, lg, w):
    _case("dft", lg, w)
    x = oracle.gen_uniform(lg * 7 + w, (1 << lg) * w).reshape(1 << lg, w)
    dft = pcs.HipDft()
    y = dft.dft_batch(x)
    assert (y == oracle.dft_batch(x)).all()
    assert (dft.idft_batch(y) == x).all()


@pytest.mark.parametrize("lg,w", [(5, 1), (18, 16), (11, 3)])
def test_reference_ntt_entry(native, oracle, lg, w):
    _case("zkie_ntt_forward_goldilocks", lg, w)
    x = oracle.gen_uniform(3, (1 << lg) * w).reshape(1 << lg, w)
    d = DeviceBuffer.from_array(x)
    tmp = DeviceBuffer(x.size)
    check(native.load().zkie_ntt_forward_goldilocks(d.addr, tmp.addr, lg, w, None), "ntt")
    assert (d.download().reshape(x.shape) == oracle.dft_batch(x)).all()


@pytest.mark.parametrize("h,w,lb,shift", [(16, 1, 2, 1), (1024, 16, 2, 1), (1 << 16, 1, 2, 1),
                                          (4096, 32, 3, 1), (256, 16, 2, 7), (2048, 128, 1, 1),
                                          (1, 4, 3, 1), (8, 2, 0, 1)])
def test_lde(native, oracle, h, w, lb, shift):
    _case("lde", h, w, lb, shift)
    x = oracle.gen_uniform(h + w, h * w).reshape(h, w)
    y = pcs.HipDft().lde_batch(x, lb, shift)
    assert (y == oracle.lde_batch(x, lb, shift)).all()


@pytest.mark.parametrize("h,w", [(1, 1), (1, 16), (2, 8), (3, 5), (7, 16), (100, 3), (513, 16),
                                 (1000, 32), (4096, 128), (1 << 14, 16), (1 << 12, 1), (300, 0),
                                 (64, 9)])
def test_merkle_commit(native, oracle, h, w):
    _case("merkle_commit", h, w)
    m = oracle.gen_uniform(h * 3 + w, h * w).reshape(h, w)
    root, tree = pcs.HipMerkleTreeMmcs().commit(m) if w else _commit_empty(h)
    layers, oroot = oracle.merkle_commit(m)
    got = tree.layers()
    assert len(got) == len(layers)
    for a, b in zip(got, layers):
        assert (a == b).all()
    assert (root == oroot).all()


def _commit_empty(h):
    # width-0 rows hash to the zero digest (no permutation)
    d = DeviceBuffer(1)
    tree = pcs.HipMerkleTreeMmcs().commit_device(d, h, 0)
    return tree.root, tree


@pytest.mark.parametrize("h,w", [(1000, 16), (37, 8), (64, 1)])
def test_reference_p2_entries(native, oracle, h, w):
    """The merkle_cuda.rs:226-280 schedule over the reference-compatible entry
    points (batch + scalar leaves, memset, batch + scalar compressions)."""
    _case("p2 entries", h, w)
    L = native.load()
    m = oracle.gen_uniform(11, h * w).reshape(h, w)
    lens = native.merkle_layout(h)
    d_mat = DeviceBuffer.from_array(m)
    layers = [DeviceBuffer(n * 8) for n in lens]
    check(L.zkie_memset(layers[0].addr, 0, lens[0] * 64), "memset")
    check(L.zkie_p2_leaf_batch(d_mat.addr, layers[0].addr, h, w), "leaf_batch")
    check(L.zkie_p2_leaf_scalar(d_mat.addr, layers[0].addr, h // 8 * 8, h, w), "leaf_scalar")
    for i in range(len(lens) - 1):
        raw = lens[i] // 2
        check(L.zkie_memset(layers[i + 1].addr, 0, lens[i + 1] * 64), "memset")
        check(L.zkie_p2_compress_batch(layers[i].addr, layers[i + 1].addr, raw, 2), "compress_batch")
        check(L.zkie_p2_compress_scalar(layers[i].addr, layers[i + 1].addr, raw // 8 * 8, raw, 2),
              "compress_scalar")
    check(L.zkie_device_synchronize(), "sync")
    ol, _ = oracle.merkle_commit(m)
    for d, o in zip(layers, ol):
        assert (d.download().reshape(-1, 8) == o).all()


@pytest.mark.parametrize("parents,step", [(24, 1), (1003, 1), (40000, 1), (1000, 2), (1 << 15, 2),
                                          ((1 << 15) + 13, 2)])
def test_compress_entries_one_and_two_children(native, oracle, parents, step):
    """zkie_p2_compress_batch/_scalar with one child per parent (the child in
    words 0..7, zeros after, poseidon2_merkle.cu:214-221) and with two, on
    both sides of the size where a level switches from one permutation per
    lane to one per 16-lane row."""
    _case("compress entries", parents, step)
    L = native.load()
    prev = oracle.gen_uniform(parents + step, parents * step * 8).reshape(parents * step, 8)
    d_prev = DeviceBuffer.from_array(prev)
    d_next = DeviceBuffer(parents * 8)
    end = parents // 8 * 8
    check(L.zkie_p2_compress_batch(d_prev.addr, d_next.addr, parents, step), "compress_batch")
    check(L.zkie_p2_compress_scalar(d_prev.addr, d_next.addr, end, parents, step), "compress_scalar")
    check(L.zkie_device_synchronize(), "sync")
    got = d_next.download().reshape(parents, 8)
    st = np.zeros(16, np.uint64)
    for r in range(parents):
        st[:] = 0
        st[: 8 * step] = prev[step * r: step * r + step].reshape(-1)
        assert (got[r] == oracle.p2_permute(st)[:8] % np.uint64(P)).all(), r


def test_openings(native, oracle):
    _case("openings")
    h, w = 1000, 16
    m = oracle.gen_uniform(5, h * w).reshape(h, w)
    mmcs = pcs.HipMerkleTreeMmcs()
    root, tree = mmcs.commit(m)
    layers, _ = oracle.merkle_commit(m)
    idx = [0, 1, 2, 999, 500, 501, 37, 37, 998]
    rows, sib = mmcs.open_batches(idx, tree)
    for k, i in enumerate(idx):
        assert (rows[k] == m[i]).all()
        assert (sib[k] == oracle.merkle_open(layers, h, i)).all()
        assert oracle.merkle_verify(root, h, i, rows[k], sib[k])
    prow, pruned = mmcs.open_multi_batch(idx, tree)
    assert (prow == m[idx]).all()
    assert (pruned == oracle.merkle_open_pruned(layers, h, idx)).all()
    # single-leaf tree: no siblings
    r1, t1 = mmcs.commit(m[:1])
    rr, ss = mmcs.open_batch(0, t1)
    assert ss.shape == (0, 8) and (rr == m[0]).all()


def test_open_rejects_out_of_range(native, oracle):
    _case("open out of range")
    m = oracle.gen_uniform(5, 64).reshape(16, 4)
    mmcs = pcs.HipMerkleTreeMmcs()
    _, tree = mmcs.commit(m)
    with pytest.raises(Exception):
        mmcs.open_batches([16], tree)


@pytest.mark.parametrize("k,ext", [(1, False), (2, False), (3, False), (4, False), (6, False), (8, False),
                                   (1, True), (2, True), (3, True), (4, True), (7, True), (0, False),
                                   (0, True)])
def test_fold_rows(native, oracle, k, ext):
    _case("fold", k, ext)
    h = 777
    width = (2 if ext else 1) << k
    m = oracle.gen_uniform(k + 31, h * width).reshape(h, width)
    r = oracle.gen_uniform(k + 77, 2 * k).reshape(k, 2) if k else np.zeros((0, 2), np.uint64)
    got = pcs.fold_rows(m, k, r, ext)
    assert (got == oracle.fold_rows(m, k, r, ext)).all()


def test_generic_diag15_path(native, oracle):
    """Constants with diag15 != 2^-32 select the general multiply; the default
    constants are restored afterwards on both sides."""
    _case("diag15 generic")
    a, b, c, d = oracle.p2_constants()
    try:
        oracle.p2_set_constants(a, b, c, 12345)
        mmcs = pcs.HipMerkleTreeMmcs((a, b, c, 12345))
        m = oracle.gen_uniform(9, 40 * 16).reshape(40, 16)
        root, _ = mmcs.commit(m)
        _, oroot = oracle.merkle_commit(m)
        assert (root == oroot).all()
    finally:
        oracle.p2_set_constants(a, b, c, d)
        pcs.HipMerkleTreeMmcs((a, b, c, d))
    m = oracle.gen_uniform(9, 40 * 16).reshape(40, 16)
    root, _ = pcs.HipMerkleTreeMmcs().commit(m)
    assert (root == oracle.merkle_commit(m)[1]).all()


def test_large_round_constants_path(native, oracle):
    """Linear-layer constants at or above 2^64 - 2^38 (with the default
    diag15) select the general path, whose constants join as two halves;
    the default constants are restored afterwards on both sides."""
    _case("large round constants")
    a, b, c, d = oracle.p2_constants()
    a2, b2, c2 = a.copy(), b.copy(), c.copy()
    a2[5] = 0xFFFFFFFF00000000          # p - 1, in an initial round
    b2[20] = 0xFFFFFFC000000000         # 2^64 - 2^38, in a terminal round
    c2[0] = 0xFFFFFFFF00000000          # the first internal round's constant
    try:
        oracle.p2_set_constants(a2, b2, c2, d)
        mmcs = pcs.HipMerkleTreeMmcs((a2, b2, c2, d))
        m = oracle.gen_uniform(10, 40 * 16).reshape(40, 16)
        root, _ = mmcs.commit(m)
        _, oroot = oracle.merkle_commit(m)
        assert (root == oroot).all()
    finally:
        oracle.p2_set_constants(a, b, c, d)
        pcs.HipMerkleTreeMmcs((a, b, c, d))
    m = oracle.gen_uniform(10, 40 * 16).reshape(40, 16)
    root, _ = pcs.HipMerkleTreeMmcs().commit(m)
    assert (root == oracle.merkle_commit(m)[1]).all()


def test_profile_counters(native, oracle):
    _case("profile")
    native.profile_enable(True)
    try:
        native.profile_reset()
        m = oracle.gen_uniform(1, 4096 * 16).reshape(4096, 16)
        pcs.HipMerkleTreeMmcs().commit(m)
        n, ms = native.profile_query("p2_leaf")
        assert n == 1 and ms > 0
        assert "p2_leaf" in native.profile_names()
    finally:
        native.profile_enable(False)


@pytest.mark.parametrize("h,w,lb,shift", [(1 << 8, 16, 2, 1), (1 << 10, 16, 2, 1), (1 << 12, 16, 2, 1),
                                          (1 << 11, 16, 3, 1), (1 << 13, 16, 3, 1), (1 << 16, 16, 2, 1),
                                          (1 << 17, 16, 2, 1), (1 << 14, 16, 3, 7), (1 << 12, 8, 2, 1),
                                          (1 << 10, 32, 2, 1), (64, 16, 1, 1), (1 << 12, 1, 2, 1)])
def test_lde_commit(native, oracle, h, w, lb, shift):
    """zkie_lde_commit: codeword, every digest layer and the root equal the
    oracle's LDE and commitment; 16-wide shapes of 10 to 19 rows' bits take
    the fused last pass + leaf hash (last passes of 5 to 9 bits), the others
    the separate leaf kernel."""
    _case("lde_commit", h, w, lb, shift)
    x = oracle.gen_uniform(h * 5 + w + lb, h * w).reshape(h, w)
    tree = pcs.HipMerkleTreeMmcs().lde_commit_device(DeviceBuffer.from_array(x), h, w, lb, shift=shift)
    cw = oracle.lde_batch(x, lb, shift)
    assert (tree.d_mat.download().reshape(cw.shape) == cw).all()
    layers, root = oracle.merkle_commit(cw)
    got = tree.layers()
    assert len(got) == len(layers)
    for a, b in zip(got, layers):
        assert (a == b).all()
    assert (tree.root == root).all()


def test_lde_at_the_largest_transform(native, oracle):
    """zkie_lde_batch at the library's largest transform: 2^30 coefficients of
    one column, blowup 4, a codeword of 2^32 rows (32 GiB; the reference caps
    its GPU DFT at 2^18 rows, dft_cuda.rs:96). Sampled rows equal direct
    evaluation at w_{2^32}^t (Horner over the 2^30 coefficients), and the
    inverse DFT of the whole codeword returns the zero-padded input."""
    _case("lde 2^30 -> 2^32 rows")
    h, lb = 1 << 30, 2
    n = h << lb
    x = native.gen_inputs(77, h, 0)
    d_in = DeviceBuffer.from_array(x)
    d_cw = DeviceBuffer(n)
    check(native.load().zkie_lde_batch(d_in.addr, h, 1, lb, 1, d_cw.addr, None), "zkie_lde_batch")
    del d_in
    g = oracle.two_adic_generator(32)
    col = x.reshape(h, 1)
    rng = np.random.default_rng(32)
    for t in [0, 1, n // 4, n // 2, n - 1] + [int(v) for v in rng.integers(0, n, 3)]:
        assert int(d_cw.download(1, t)[0]) == oracle.poly_eval(col, 0, pow(g, t, P)), t
    check(native.load().zkie_idft_batch(d_cw.addr, 32, 1, None), "zkie_idft_batch")
    back = d_cw.download()
    assert (back[:h] == x).all()
    assert not back[h:].any()
