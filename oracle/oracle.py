"""ctypes wrapper of the CPU oracle (oracle/libzkie_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package zkie_amd.
Arrays are numpy uint64, canonical Goldilocks values.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libzkie_oracle.so")
P = 0xFFFFFFFF00000001

_u64p = ctypes.POINTER(ctypes.c_uint64)
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc + OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u64, u32, i32 = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
        sig = {
            "or_add": (u64, [u64, u64]),
            "or_sub": (u64, [u64, u64]),
            "or_mul": (u64, [u64, u64]),
            "or_pow": (u64, [u64, u64]),
            "or_inv": (u64, [u64]),
            "or_ef_mul": (None, [_u64p, _u64p, _u64p]),
            "or_two_adic_generator": (u64, [u32]),
            "or_dft_batch": (None, [_u64p, u32, u64]),
            "or_idft_batch": (None, [_u64p, u32, u64]),
            "or_dft_naive": (None, [_u64p, _u64p, u32, u64]),
            "or_poly_eval": (u64, [_u64p, u64, u64, u64, u64]),
            "or_checksum": (u64, [_u64p, u64, u64]),
            "or_lde_batch": (None, [_u64p, u64, u64, u32, u64, _u64p]),
            "or_p2_derive_constants": (None, [_u64p, _u64p, _u64p, _u64p]),
            "or_p2_set_constants": (None, [_u64p, _u64p, _u64p, u64]),
            "or_p2_permute": (None, [_u64p]),
            "or_p2_mds_light": (None, [_u64p]),
            "or_p2_internal_linear": (None, [_u64p]),
            "or_leaf_hash": (None, [_u64p, u64, _u64p]),
            "or_compress": (None, [_u64p, _u64p, _u64p]),
            "or_xoshiro_seed_u64": (None, [_u64p, u64]),
            "or_xoshiro_from_state": (None, [_u64p, _u64p]),
            "or_xoshiro_next": (u64, [_u64p]),
            "or_splitmix64_next": (u64, [_u64p]),
            "or_padded_len": (u64, [u64, u64]),
            "or_merkle_num_layers": (u32, [u64]),
            "or_merkle_layer_lens": (None, [u64, _u64p]),
            "or_merkle_build_layers": (None, [_u64p, u64, _u64p, i32]),
            "or_merkle_compress_layer": (u64, [_u64p, u64, _u64p, i32]),
            "or_merkle_leaf_digests": (None, [_u64p, u64, u64, _u64p]),
            "or_merkle_commit": (None, [_u64p, u64, u64, _u64p, _u64p]),
            "or_merkle_open": (None, [_u64p, u64, u64, _u64p]),
            "or_merkle_open_pruned": (u64, [_u64p, u64, _u64p, u64, _u64p, u64]),
            "or_merkle_verify": (i32, [_u64p, u64, u64, _u64p, u64, _u64p]),
            "or_fold_rows": (None, [_u64p, u64, u32, i32, _u64p, _u64p]),
            "or_mle_eval_base": (u64, [_u64p, u32, _u64p]),
            "or_mle_eval": (None, [_u64p, u32, ctypes.c_int, _u64p, _u64p]),
            "or_eq_table": (None, [_u64p, u32, _u64p]),
            "or_constraint_weights": (None, [_u64p, u32, _u64p, u32, _u64p, u32, _u64p]),
            "or_sumcheck_prove": (None, [_u64p, ctypes.c_int, _u64p, u32, u32, _u64p, _u64p, _u64p,
                                         _u64p]),
            "or_xorshift_next": (u64, [_u64p]),
            "or_xorshift_init": (None, [_u64p, u64]),
            "or_gen_uniform": (None, [u64, u64, _u64p]),
            "or_gen_i16": (None, [u64, u64, _u64p]),
            "or_gen_i8": (None, [u64, u64, _u64p]),
            "or_gen_gauss_i16": (None, [u64, u64, u64, u64, u32, _u64p]),
            "or_set_threads": (None, [i32]),
            "or_get_threads": (i32, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.uint64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_u64p)


def u64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


# ---- field -----------------------------------------------------------------
def add(a, b): return lib().or_add(a, b)
def sub(a, b): return lib().or_sub(a, b)
def mul(a, b): return lib().or_mul(a, b)
def pow_(a, e): return lib().or_pow(a, e)
def inv(a): return lib().or_inv(a)
def two_adic_generator(k): return lib().or_two_adic_generator(k)


def ef_mul(a, b):
    a, b, o = u64(a), u64(b), np.zeros(2, np.uint64)
    lib().or_ef_mul(_p(a), _p(b), _p(o))
    return (int(o[0]), int(o[1]))


# ---- DFT -------------------------------------------------------------------
def dft_batch(mat: np.ndarray) -> np.ndarray:
    """mat: (h, w) uint64, h a power of two. Returns a new array."""
    m = u64(mat).copy()
    h, w = m.shape
    lg = h.bit_length() - 1
    assert 1 << lg == h
    lib().or_dft_batch(_p(m), lg, w)
    return m


def idft_batch(mat: np.ndarray) -> np.ndarray:
    m = u64(mat).copy()
    h, w = m.shape
    lg = h.bit_length() - 1
    lib().or_idft_batch(_p(m), lg, w)
    return m


def dft_naive(mat: np.ndarray) -> np.ndarray:
    m = u64(mat)
    h, w = m.shape
    out = np.zeros_like(m)
    lib().or_dft_naive(_p(m), _p(out), h.bit_length() - 1, w)
    return out


def poly_eval(mat: np.ndarray, c: int, x: int) -> int:
    """Column c of the (h, w) coefficient matrix evaluated at x."""
    m = u64(mat)
    h, w = m.shape
    return lib().or_poly_eval(_p(m), h, w, c, x)


CHECKSUM_Z = 0x1BADB002DEADBEEF


def checksum(v: np.ndarray, z: int = CHECKSUM_Z) -> int:
    """sum_i v[i] z^i mod p over the flattened array."""
    a = u64(v).reshape(-1)
    return lib().or_checksum(_p(a), a.size, z)


def lde_batch(mat: np.ndarray, log_blowup: int, shift: int = 1) -> np.ndarray:
    m = u64(mat)
    h, w = m.shape
    out = np.zeros((h << log_blowup, w), np.uint64)
    lib().or_lde_batch(_p(m), h, w, log_blowup, shift, _p(out))
    return out


def stack_tables(tables, log_width: int) -> np.ndarray:
    """The witness of Whir::commit_batch (crates/zkie-core/src/pcs/whir.rs:
    476-525): same-size tables of 2^arity entries, table-major (entry j of
    table i at i 2^arity + j), zero-padded to 2^total_vars entries with
    total_vars = ceil(log2(count 2^arity)), as rows of 2^log_width. The order
    is the one the reference hands to its external initial-round layout
    (p3-whir adapter.rs:106-113, MyLayout::new_witness): parity unpinned."""
    flat = [u64(t).reshape(-1) for t in tables]
    if not flat:
        raise ValueError("batch must not be empty")
    size = flat[0].size
    if size & (size - 1) or any(t.size != size for t in flat):
        raise ValueError("all tables must hold the same power-of-two count")
    total_vars = (len(flat) * size - 1).bit_length()
    if total_vars < log_width:
        raise ValueError("the stacked witness fills no row")
    out = np.zeros(1 << total_vars, np.uint64)
    out[:len(flat) * size] = np.concatenate(flat)
    return out.reshape(-1, 1 << log_width)


def commit_batch(tables, log_width: int, log_blowup: int):
    """Stack, encode (zero-padded DFT, writer.rs:73-85) and commit: returns
    (stacked witness rows, codeword, layers, root)."""
    stack = stack_tables(tables, log_width)
    cw = lde_batch(stack, log_blowup)
    layers, root = merkle_commit(cw)
    return stack, cw, layers, root


# ---- Poseidon2 ---------------------------------------------------------------
def p2_constants():
    a, b, c, d = (np.zeros(64, np.uint64), np.zeros(64, np.uint64),
                  np.zeros(22, np.uint64), np.zeros(1, np.uint64))
    lib().or_p2_derive_constants(_p(a), _p(b), _p(c), _p(d))
    return a, b, c, int(d[0])


def p2_set_constants(rc_init, rc_final, rc_internal, diag15):
    a, b, c = u64(rc_init), u64(rc_final), u64(rc_internal)
    lib().or_p2_set_constants(_p(a), _p(b), _p(c), diag15)


def p2_permute(state) -> np.ndarray:
    s = u64(state).copy()
    assert s.shape == (16,)
    lib().or_p2_permute(_p(s))
    return s


def p2_mds_light(state) -> np.ndarray:
    s = u64(state).copy()
    lib().or_p2_mds_light(_p(s))
    return s


def p2_internal_linear(state) -> np.ndarray:
    s = u64(state).copy()
    lib().or_p2_internal_linear(_p(s))
    return s


def leaf_hash(row) -> np.ndarray:
    r = u64(row)
    o = np.zeros(8, np.uint64)
    lib().or_leaf_hash(_p(r) if r.size else ctypes.cast(0, _u64p), r.size, _p(o))
    return o


def compress(left, right) -> np.ndarray:
    l, r, o = u64(left), u64(right), np.zeros(8, np.uint64)
    lib().or_compress(_p(l), _p(r), _p(o))
    return o


# ---- rand --------------------------------------------------------------------
class Xoshiro256pp:
    def __init__(self, seed: int | None = None, state=None):
        self._s = np.zeros(4, np.uint64)
        if state is not None:
            st = u64(state)
            lib().or_xoshiro_from_state(_p(self._s), _p(st))
        else:
            lib().or_xoshiro_seed_u64(_p(self._s), seed)

    def next_u64(self) -> int:
        return lib().or_xoshiro_next(_p(self._s))


def splitmix64(seed: int, n: int):
    st = np.array([seed], np.uint64)
    return [lib().or_splitmix64_next(_p(st)) for _ in range(n)]


# ---- Merkle ------------------------------------------------------------------
def padded_len(raw: int, n: int = 2) -> int:
    return lib().or_padded_len(raw, n)


def layer_lens(h: int):
    nl = lib().or_merkle_num_layers(h)
    lens = np.zeros(nl, np.uint64)
    lib().or_merkle_layer_lens(h, _p(lens))
    return [int(x) for x in lens]


class LayerList(list):
    """Digest layers as (len, 8) views of one flat array (kept in .flat)."""

    flat: np.ndarray


def split_layers(flat: np.ndarray, h: int) -> LayerList:
    out, off = LayerList(), 0
    for ln in layer_lens(h):
        out.append(flat[off:off + 8 * ln].reshape(ln, 8))
        off += 8 * ln
    out.flat = flat
    return out


def merkle_commit(mat: np.ndarray):
    """Returns (layers list of (len, 8) arrays, root (8,))."""
    m = u64(mat)
    h, w = m.shape
    total = sum(layer_lens(h))
    flat = np.zeros(total * 8, np.uint64)
    root = np.zeros(8, np.uint64)
    lib().or_merkle_commit(_p(m), h, w, _p(flat), _p(root))
    return split_layers(flat, h), root


def leaf_digests(mat: np.ndarray) -> np.ndarray:
    m = u64(mat)
    h, w = m.shape
    d = np.zeros((h, 8), np.uint64)
    lib().or_merkle_leaf_digests(_p(m), h, w, _p(d))
    return d


def build_layers(layer0: np.ndarray, compressor: int = 0):
    d = u64(layer0)
    h = d.shape[0]
    total = sum(layer_lens(h))
    flat = np.zeros(total * 8, np.uint64)
    lib().or_merkle_build_layers(_p(d), h, _p(flat), compressor)
    return split_layers(flat, h)


def compress_layer(prev: np.ndarray, compressor: int = 0) -> np.ndarray:
    pv = u64(prev)
    n = pv.shape[0]
    out = np.zeros((max(padded_len(n // 2), 1), 8), np.uint64)
    k = lib().or_merkle_compress_layer(_p(pv), n, _p(out), compressor)
    return out[:k]


def _flat_layers(layers):
    if isinstance(layers, LayerList):
        return layers.flat
    return np.ascontiguousarray(np.concatenate([np.asarray(l, np.uint64).reshape(-1) for l in layers]))


def merkle_open(layers, h: int, index: int) -> np.ndarray:
    flat = _flat_layers(layers)
    nl = len(layer_lens(h))
    sib = np.zeros((max(nl - 1, 0), 8), np.uint64)
    lib().or_merkle_open(_p(flat), h, index, _p(sib) if sib.size else ctypes.cast(0, _u64p))
    return sib


def merkle_open_pruned(layers, h: int, indices) -> np.ndarray:
    flat = _flat_layers(layers)
    idx = u64(indices)
    cap = max(1, len(idx) * len(layer_lens(h)))
    out = np.zeros((cap, 8), np.uint64)
    k = lib().or_merkle_open_pruned(_p(flat), h, _p(idx) if idx.size else ctypes.cast(0, _u64p),
                                    len(idx), _p(out), cap)
    assert k <= cap
    return out[:k]


def merkle_verify(root, h: int, index: int, row, siblings) -> bool:
    r, rw = u64(root), u64(row)
    sib = u64(siblings).reshape(-1)
    return bool(lib().or_merkle_verify(_p(r), h, index, _p(rw), rw.size,
                                       _p(sib) if sib.size else ctypes.cast(0, _u64p)))


# ---- fold --------------------------------------------------------------------
def fold_rows(mat: np.ndarray, k: int, r, is_ext: bool) -> np.ndarray:
    """mat: (h, 2^k) base or (h, 2^(k+1)) flattened EF. r: k EF pairs. Returns (h, 2)."""
    m = u64(mat)
    h = m.shape[0]
    rr = u64(r).reshape(-1)
    assert rr.size == 2 * k
    out = np.zeros((h, 2), np.uint64)
    lib().or_fold_rows(_p(m), h, k, 1 if is_ext else 0, _p(rr), _p(out))
    return out


def mle_eval_base(values, point) -> int:
    v, pt = u64(values), u64(point)
    return lib().or_mle_eval_base(_p(v), pt.size, _p(pt))


def mle_eval(values, point, is_ext: bool) -> np.ndarray:
    """mle::eval (mle.rs:8-22) of 2^t base or flattened-EF values at t EF coordinates."""
    v, pt = u64(values).reshape(-1), u64(point).reshape(-1)
    t = pt.size // 2
    assert v.size == (2 if is_ext else 1) << t
    out = np.zeros(2, np.uint64)
    lib().or_mle_eval(_p(v), t, 1 if is_ext else 0, _p(pt), _p(out))
    return out


def eq_table(point) -> np.ndarray:
    """eq(point, x) for x < 2^t, bit 0 first (mle.rs:44-56): (2^t, 2) EF."""
    pt = u64(point).reshape(-1)
    t = pt.size // 2
    out = np.zeros((1 << t, 2), np.uint64)
    lib().or_eq_table(_p(pt) if pt.size else _p(out), t, _p(out))
    return out


def constraint_weights(eq_points, sel_points, gamma, n: int) -> np.ndarray:
    """Batched constraint weights of a WHIR round: (2^n, 2) EF,
    sum_j gamma^j eq(p_j, x) + sum_k gamma^(m+k) z_k^x."""
    eqp = u64(eq_points).reshape(len(eq_points), n, 2) if len(eq_points) else np.zeros((0, n, 2), np.uint64)
    sel = u64(sel_points).reshape(-1, 2) if len(sel_points) else np.zeros((0, 2), np.uint64)
    g = u64(gamma).reshape(2)
    out = np.zeros((1 << n, 2), np.uint64)
    dummy = np.zeros(2, np.uint64)
    lib().or_constraint_weights(_p(np.ascontiguousarray(eqp)) if eqp.size else _p(dummy), eqp.shape[0],
                                _p(np.ascontiguousarray(sel)) if sel.size else _p(dummy), sel.shape[0],
                                _p(g), n, _p(out))
    return out


def sumcheck_prove(f, f_is_ext: bool, h, r):
    """`len(r)` rounds of common/sumcheck.rs:33-89 over sum_x f(x) h(x) with EF
    tables and challenges. f: 2^t base or flattened EF, h: flattened EF, r:
    (rounds, 2). Returns (polys (rounds, 3, 2) as c0, c1, c2, f_out, h_out),
    the folded tables as (2^(t - rounds), 2)."""
    fv, hv = u64(f).reshape(-1), u64(h).reshape(-1)
    rr = u64(r).reshape(-1)
    rounds = rr.size // 2
    t = (hv.size // 2).bit_length() - 1
    assert hv.size == 2 << t and fv.size == (2 if f_is_ext else 1) << t and rounds <= t
    polys = np.zeros((max(rounds, 1), 3, 2), np.uint64)
    fo = np.zeros((1 << (t - rounds), 2), np.uint64)
    ho = np.zeros_like(fo)
    lib().or_sumcheck_prove(_p(fv), 1 if f_is_ext else 0, _p(hv), t, rounds, _p(rr) if rr.size else _p(polys),
                            _p(polys), _p(fo), _p(ho))
    return polys[:rounds], fo, ho


def whir_encode(poly, num_vars: int, is_ext: bool, log_width: int, log_inv_rate: int,
                prefix: bool) -> np.ndarray:
    """commit_extension's encoding (p3-whir committer/writer.rs:21-86): the
    table as 2^(n-k) rows x 2^k entries, rows as stored (Suffix) or
    transposed so that entry (i, j) is poly[j 2^(n-k) + i] (Prefix,
    writer.rs:43-71), zero-padded by 2^log_inv_rate and transformed per base
    column (dft_algebra_batch is the base DFT of each component)."""
    E = 2 if is_ext else 1
    v = u64(poly).reshape(1 << num_vars, E)
    rows, cols = 1 << (num_vars - log_width), 1 << log_width
    m = v.reshape(cols, rows, E).transpose(1, 0, 2) if prefix else v.reshape(rows, cols, E)
    return lde_batch(np.ascontiguousarray(m).reshape(rows, cols * E), log_inv_rate)


# ---- prover-data cache stream -------------------------------------------------
def prover_data_bytes(mat, layers) -> bytes:
    """Whir::serialize_batch_prover_data_into (crates/zkie-core/src/pcs/whir.rs:542-560)
    of a tree over one matrix, then MerkleTree::write_digest_layers
    (vendor/p3-merkle-tree/src/merkle_tree.rs:223-243). Little-endian u64s:
    leaf-matrix count, width, value count, the values; layer count, layer
    lengths, arities (2 for the binary tree: merkle_tree.rs:146-158 with N = 2),
    the digests."""
    m = u64(mat)
    h, w = m.shape
    lay = [np.asarray(l, np.uint64).reshape(-1, 8) for l in layers]
    frame = [len(lay)] + [l.shape[0] for l in lay] + [2] * (len(lay) - 1)
    parts = [np.array([1, w, h * w], "<u8").tobytes(), m.astype("<u8").tobytes(),
             np.array(frame, "<u8").tobytes()]
    parts += [l.astype("<u8").tobytes() for l in lay]
    return b"".join(parts)


def parse_prover_data(buf: bytes):
    """Whir::restore_batch_prover_data_from (whir.rs:572-602) and
    MerkleTree::read_digest_layers (merkle_tree.rs:247-276): returns
    (matrices as (h, w) arrays, digest layers as (len, 8) arrays, arities).
    Raises ValueError on a stream that ends early or has bytes left over."""
    pos = 0

    def take(n_u64: int) -> np.ndarray:
        nonlocal pos
        end = pos + 8 * n_u64
        if end > len(buf):
            raise ValueError("prover-data stream ends early")
        a = np.frombuffer(buf, "<u8", n_u64, pos).astype(np.uint64)
        pos = end
        return a

    mats = []
    for _ in range(int(take(1)[0])):
        w, n = (int(x) for x in take(2))
        mats.append(take(n).reshape(-1, w) if w else take(n))
    nl = int(take(1)[0])
    lens = [int(x) for x in take(nl)]
    arities = [int(x) for x in take(max(nl - 1, 0))]
    layers = [take(8 * ln).reshape(ln, 8) for ln in lens]
    if pos != len(buf):
        raise ValueError("bytes left after the digest layers")
    return mats, layers, arities


# ---- inputs ------------------------------------------------------------------
def xorshift(seed: int, n: int):
    st = np.zeros(1, np.uint64)
    lib().or_xorshift_init(_p(st), seed)
    return [lib().or_xorshift_next(_p(st)) for _ in range(n)]


def gen_uniform(seed: int, n: int) -> np.ndarray:
    o = np.zeros(n, np.uint64)
    lib().or_gen_uniform(seed, n, _p(o))
    return o


def gen_i16(seed: int, n: int) -> np.ndarray:
    o = np.zeros(n, np.uint64)
    lib().or_gen_i16(seed, n, _p(o))
    return o


def gen_i8(seed: int, n: int) -> np.ndarray:
    o = np.zeros(n, np.uint64)
    lib().or_gen_i8(seed, n, _p(o))
    return o


def gen_gauss_i16(seed: int, n: int, std_num: int = 1, std_den: int = 50, frac_bits: int = 12) -> np.ndarray:
    o = np.zeros(n, np.uint64)
    lib().or_gen_gauss_i16(seed, n, std_num, std_den, frac_bits, _p(o))
    return o


def set_threads(n: int):
    lib().or_set_threads(n)


def get_threads() -> int:
    return lib().or_get_threads()
