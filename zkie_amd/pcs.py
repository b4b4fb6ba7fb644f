"""Python view of the per-stage dispatch seam, over the HIP C ABI.

Mirrors the engines of the reference's WHIR wrapper:
  * HipDft            <- CudaDft (crates/zkie-core/src/pcs/dft_cuda.rs:124-222),
                         TwoAdicSubgroupDft::dft_batch on row-major matrices;
  * HipMerkleTreeMmcs <- CudaMerkleTreeMmcs (merkle_cuda.rs:133-393),
                         Mmcs::{commit, open_batch, open_multi_batch};
  * HipMerkleTree     <- the MerkleTree prover data (p3-merkle-tree
                         merkle_tree.rs:32-70), kept device-resident;
  * fold_rows         <- the WHIR row fold (p3-whir prover/mod.rs:257-290);
    fold_rows_at      <- its queried-row form (prover/mod.rs:265-290);
  * mle_eval          <- the OOD answer sumcheck_prover.eval (prover/mod.rs:226-236);
  * whir_encode       <- commit_extension's encoding (committer/writer.rs:21-86);
  * serialize_batch_prover_data_into / restore_batch_prover_data_from
                      <- the prover-data part of the batch cache
                         (crates/zkie-core/src/pcs/whir.rs:542-602).
Unlike the reference there is no CPU fallback: every failure raises.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N
from ._native import DeviceBuffer, check


def _as_matrix(mat) -> np.ndarray:
    m = np.ascontiguousarray(np.asarray(mat, dtype=np.uint64))
    if m.ndim == 1:
        m = m.reshape(-1, 1)
    return m


class HipDft:
    """TwoAdicSubgroupDft<Goldilocks> on the GPU (dft_cuda.rs:161-222)."""

    def dft_batch(self, mat) -> np.ndarray:
        m = _as_matrix(mat)
        h, w = m.shape
        if h <= 1:
            return m.copy()
        lg = h.bit_length() - 1
        if 1 << lg != h:
            raise ValueError("height must be a power of two")
        d = DeviceBuffer.from_array(m)
        check(N.load().zkie_dft_batch(d.addr, lg, w, None), "zkie_dft_batch")
        return d.download().reshape(h, w)

    def idft_batch(self, mat) -> np.ndarray:
        m = _as_matrix(mat)
        h, w = m.shape
        lg = h.bit_length() - 1
        d = DeviceBuffer.from_array(m)
        check(N.load().zkie_idft_batch(d.addr, lg, w, None), "zkie_idft_batch")
        return d.download().reshape(h, w)

    def lde_batch(self, mat, log_blowup: int, shift: int = 1) -> np.ndarray:
        m = _as_matrix(mat)
        h, w = m.shape
        d_in = DeviceBuffer.from_array(m)
        d_out = DeviceBuffer((h << log_blowup) * w)
        check(N.load().zkie_lde_batch(d_in.addr, h, w, log_blowup, shift, d_out.addr, None),
              "zkie_lde_batch")
        return d_out.download().reshape(h << log_blowup, w)


def lde_device(d_in: DeviceBuffer, h: int, w: int, log_blowup: int, d_out: DeviceBuffer,
               shift: int = 1, stream=None):
    check(N.load().zkie_lde_batch(d_in.addr, h, w, log_blowup, shift, d_out.addr, stream),
          "zkie_lde_batch")


class HipMerkleTree:
    """Prover data of one commitment: the matrix and every digest layer in HBM."""

    def __init__(self, d_mat: DeviceBuffer, h: int, w: int, d_layers: DeviceBuffer, root):
        self.d_mat, self.h, self.w = d_mat, h, w
        self.d_layers = d_layers
        self.layer_lens = N.merkle_layout(h)
        self.root = np.asarray(root, np.uint64)

    def num_layers(self) -> int:
        return len(self.layer_lens)

    def layers(self):
        flat = self.d_layers.download()
        out, off = [], 0
        for ln in self.layer_lens:
            out.append(flat[off:off + 8 * ln].reshape(ln, 8))
            off += 8 * ln
        return out

    def matrix(self) -> np.ndarray:
        return self.d_mat.download(self.h * self.w).reshape(self.h, self.w)


class HipMerkleTreeMmcs:
    """Mmcs<Goldilocks> on the GPU: Poseidon2Goldilocks<16>,
    PaddingFreeSponge<Perm,16,8,8>, TruncatedPermutation<Perm,2,8,16>, cap 0."""

    def __init__(self, constants=None):
        if constants is not None:
            a, b, c, d = constants
            a, b, c = (np.ascontiguousarray(x, np.uint64) for x in (a, b, c))
            check(N.load().zkie_p2_upload_constants(N.p(a), N.p(b), N.p(c), d),
                  "zkie_p2_upload_constants")

    def commit_device(self, d_mat: DeviceBuffer, h: int, w: int, stream=None) -> HipMerkleTree:
        lens = N.merkle_layout(h)
        d_layers = DeviceBuffer(sum(lens) * 8)
        root = np.zeros(8, np.uint64)
        check(N.load().zkie_merkle_commit(d_mat.addr, h, w, d_layers.addr, N.p(root), stream),
              "zkie_merkle_commit")
        return HipMerkleTree(d_mat, h, w, d_layers, root)

    def lde_commit_device(self, d_in: DeviceBuffer, h: int, w: int, log_blowup: int,
                          d_codeword: DeviceBuffer | None = None, shift: int = 1,
                          stream=None) -> HipMerkleTree:
        """Encode then commit (writer.rs:73-85) in one call: the LDE of the
        h x w coefficient rows into d_codeword and the tree of its rows."""
        n = h << log_blowup
        if d_codeword is None:
            d_codeword = DeviceBuffer(n * w)
        lens = N.merkle_layout(n)
        d_layers = DeviceBuffer(sum(lens) * 8)
        root = np.zeros(8, np.uint64)
        check(N.load().zkie_lde_commit(d_in.addr, h, w, log_blowup, shift, d_codeword.addr, d_layers.addr,
                                        N.p(root), stream), "zkie_lde_commit")
        return HipMerkleTree(d_codeword, n, w, d_layers, root)

    def commit_batch_device(self, tables, arity: int, log_width: int, log_blowup: int,
                            d_stack: DeviceBuffer | None = None,
                            stream=None) -> tuple[HipMerkleTree, DeviceBuffer]:
        """Whir::commit_batch (whir.rs:476-525) on device tables of 2^arity
        entries each: stacked table-major into d_stack (2^total_vars entries,
        total_vars = ceil(log2(len(tables) 2^arity))), viewed as rows of
        2^log_width, encoded and committed. Returns the tree of the codeword
        and the stack."""
        count = len(tables)
        if count == 0:
            raise ValueError("batch must not be empty")
        total_vars = ((count << arity) - 1).bit_length()
        if total_vars < log_width:
            raise ValueError(f"{count} tables of 2^{arity} entries fill no row of 2^{log_width}")
        if d_stack is None:
            d_stack = DeviceBuffer(1 << total_vars)
        n = 1 << (total_vars - log_width + log_blowup)
        d_codeword = DeviceBuffer(n << log_width)
        d_layers = DeviceBuffer(sum(N.merkle_layout(n)) * 8)
        ptrs = np.array([t.addr for t in tables], np.uint64)
        root = np.zeros(8, np.uint64)
        check(N.load().zkie_commit_batch(N.p(ptrs), count, arity, log_width, log_blowup, d_stack.addr,
                                         d_codeword.addr, d_layers.addr, N.p(root), stream),
              "zkie_commit_batch")
        return HipMerkleTree(d_codeword, n, 1 << log_width, d_layers, root), d_stack

    def commit(self, mat) -> tuple[np.ndarray, HipMerkleTree]:
        m = _as_matrix(mat)
        h, w = m.shape
        tree = self.commit_device(DeviceBuffer.from_array(m), h, w)
        return tree.root, tree

    def open_batch(self, index: int, tree: HipMerkleTree):
        rows, sib = self.open_batches([index], tree)
        return rows[0], sib[0]

    def open_batches(self, indices, tree: HipMerkleTree, stream=None):
        idx = np.ascontiguousarray(indices, np.uint64)
        n = idx.size
        levels = tree.num_layers() - 1
        rows = np.zeros((n, tree.w), np.uint64)
        sib = np.zeros((n, max(levels, 0), 8), np.uint64)
        check(N.load().zkie_merkle_open_batch(
            tree.d_mat.addr, tree.h, tree.w, tree.d_layers.addr, N.p(idx), n,
            N.p(rows), N.p(sib) if sib.size else ctypes.cast(0, N._u64p), stream),
            "zkie_merkle_open_batch")
        return rows, sib

    def open_multi_batch(self, indices, tree: HipMerkleTree):
        idx = np.ascontiguousarray(indices, np.uint64)
        n = idx.size
        rows = np.zeros((n, tree.w), np.uint64)
        cap = max(1, n * tree.num_layers())
        out = np.zeros((cap, 8), np.uint64)
        count = ctypes.c_uint64()
        check(N.load().zkie_merkle_open_pruned(
            tree.d_mat.addr, tree.h, tree.w, tree.d_layers.addr, N.p(idx), n, N.p(rows),
            N.p(out), cap, ctypes.byref(count), None), "zkie_merkle_open_pruned")
        return rows, out[: count.value]


def serialize_batch_prover_data_into(tree: HipMerkleTree, writer, stream=None) -> int:
    """Whir::serialize_batch_prover_data_into (crates/zkie-core/src/pcs/whir.rs:542-560):
    write the committed matrix and its digest layers to the binary stream
    `writer` (anything with .write), straight from HBM. Returns the byte count."""
    n = [0]

    def sink(view):
        writer.write(view)
        n[0] += len(view)

    N.prover_data_write(tree.d_mat.addr, tree.h, tree.w, tree.d_layers.addr, sink, stream)
    return n[0]


def restore_batch_prover_data_from(reader, h: int, w: int, stream=None) -> HipMerkleTree:
    """Whir::restore_batch_prover_data_from (whir.rs:572-602): read a stream
    written for an h x w matrix (the table shape the caller already knows) into
    new device buffers. Framing of another shape raises ZkieError; a stream
    that ends early raises EOFError."""

    def source(view):
        got = 0
        while got < len(view):
            k = reader.readinto(view[got:])
            if not k:
                raise EOFError("prover-data stream ended early")
            got += k

    d_mat = DeviceBuffer(h * w)
    d_layers = DeviceBuffer(sum(N.merkle_layout(h)) * 8)
    root = N.prover_data_read(source, h, w, d_mat.addr, d_layers.addr, stream)
    return HipMerkleTree(d_mat, h, w, d_layers, root)


def fold_rows_device(d_mat: DeviceBuffer, h: int, k: int, r, is_ext: bool, d_out: DeviceBuffer,
                     stream=None):
    rr = np.ascontiguousarray(np.asarray(r, np.uint64).reshape(-1))
    assert rr.size == 2 * k
    check(N.load().zkie_fold_rows(d_mat.addr, h, k, 1 if is_ext else 0, N.p(rr), d_out.addr, stream),
          "zkie_fold_rows")


def fold_rows(mat, k: int, r, is_ext: bool) -> np.ndarray:
    m = np.ascontiguousarray(np.asarray(mat, np.uint64))
    h = m.shape[0]
    d = DeviceBuffer.from_array(m)
    out = DeviceBuffer(2 * h)
    fold_rows_device(d, h, k, r, is_ext, out)
    return out.download().reshape(h, 2)


def fold_rows_at(d_mat: DeviceBuffer, h: int, k: int, is_ext: bool, indices, r, stream=None) -> np.ndarray:
    """Fold of the rows `indices` of a device matrix only (n x 2 EF, host)."""
    idx = np.ascontiguousarray(np.asarray(indices, np.uint64).reshape(-1))
    rr = np.ascontiguousarray(np.asarray(r, np.uint64).reshape(-1))
    assert rr.size == 2 * k
    out = np.zeros(2 * idx.size, np.uint64)
    check(N.load().zkie_fold_rows_at(d_mat.addr, h, k, 1 if is_ext else 0, N.p(idx), idx.size, N.p(rr),
                                     N.p(out), stream), "zkie_fold_rows_at")
    return out.reshape(-1, 2)


def sumcheck_round(d_f: DeviceBuffer, f_is_ext: bool, d_h: DeviceBuffer, num_vars: int,
                   stream=None) -> np.ndarray:
    """The current round polynomial of the sumcheck of sum_x f(x) h(x)
    (common/sumcheck.rs:47-68): c0, c1, c2 as a (3, 2) EF array."""
    poly = np.zeros((3, 2), np.uint64)
    check(N.load().zkie_sumcheck_round(d_f.addr, 1 if f_is_ext else 0, d_h.addr, num_vars, N.p(poly), stream),
          "zkie_sumcheck_round")
    return poly


def eq_table(point, stream=None) -> DeviceBuffer:
    """eq(point, x) for every x < 2^n (EF, bit 0 first; mle.rs:44-56) as a
    device table: the weight table of one evaluation constraint."""
    pt = np.ascontiguousarray(np.asarray(point, np.uint64).reshape(-1))
    n = pt.size // 2
    out = DeviceBuffer(2 << n)
    check(N.load().zkie_eq_table(N.p(pt) if pt.size else N.p(np.zeros(2, np.uint64)), n, out.addr, stream),
          "zkie_eq_table")
    return out


def constraint_weights(eq_points, sel_points, gamma, num_vars: int, d_w: DeviceBuffer | None = None,
                       accumulate: bool = False, stream=None) -> DeviceBuffer:
    """The batched constraint of a WHIR round (p3-whir prover/mod.rs:228-314) as
    weights over the round table: d_w[x] (+)= sum_j gamma^j eq(p_j, x) +
    sum_k gamma^(m+k) z_k^x. eq_points: (m, num_vars, 2) EF; sel_points: (q, 2)."""
    m = len(eq_points)
    eqp = np.ascontiguousarray(np.asarray(eq_points, np.uint64).reshape(-1))
    sel = np.ascontiguousarray(np.asarray(sel_points, np.uint64).reshape(-1))
    g = np.ascontiguousarray(np.asarray(gamma, np.uint64).reshape(2))
    assert eqp.size == 2 * m * num_vars, "eq_points: (m, num_vars, 2) EF coordinates"
    q = sel.size // 2
    if d_w is None:
        d_w = DeviceBuffer(2 << num_vars)
    dummy = np.zeros(2, np.uint64)
    check(N.load().zkie_constraint_weights(N.p(eqp) if eqp.size else N.p(dummy), m,
                                           N.p(sel) if sel.size else N.p(dummy), q, N.p(g), num_vars,
                                           1 if accumulate else 0, d_w.addr, stream), "zkie_constraint_weights")
    return d_w


def sumcheck_fold(d_f: DeviceBuffer, f_is_ext: bool, d_h: DeviceBuffer, num_vars: int, r,
                  stream=None, next_poly: bool = False):
    """Both tables bound at variable 0 to the EF challenge r
    (common/sumcheck.rs:81-89); returns the two folded EF tables, and with
    next_poly also the next round's polynomial formed in the same pass."""
    rr = np.ascontiguousarray(np.asarray(r, np.uint64).reshape(-1))
    assert rr.size == 2
    half = 1 << (num_vars - 1)
    f_out, h_out = DeviceBuffer(2 * half), DeviceBuffer(2 * half)
    poly = np.zeros((3, 2), np.uint64)
    check(N.load().zkie_sumcheck_fold(d_f.addr, 1 if f_is_ext else 0, d_h.addr, num_vars, N.p(rr),
                                      f_out.addr, h_out.addr,
                                      N.p(poly) if next_poly else ctypes.cast(0, N._u64p), stream),
          "zkie_sumcheck_fold")
    return (f_out, h_out, poly) if next_poly else (f_out, h_out)


def sumcheck_prove(d_f: DeviceBuffer, f_is_ext: bool, d_h: DeviceBuffer, num_vars: int, r,
                   stream=None) -> tuple[np.ndarray, DeviceBuffer, DeviceBuffer]:
    """len(r) rounds of sumcheck::prove (common/sumcheck.rs:33-79) with the
    challenges given up front: (polys (rounds, 3, 2), f_out, h_out)."""
    rr = np.ascontiguousarray(np.asarray(r, np.uint64).reshape(-1))
    rounds = rr.size // 2
    polys = np.zeros((max(rounds, 1), 3, 2), np.uint64)
    n_out = 1 << (num_vars - rounds)
    f_out, h_out = DeviceBuffer(2 * n_out), DeviceBuffer(2 * n_out)
    check(N.load().zkie_sumcheck_prove(d_f.addr, 1 if f_is_ext else 0, d_h.addr, num_vars, rounds,
                                       N.p(rr) if rr.size else N.p(polys), N.p(polys), f_out.addr,
                                       h_out.addr, stream), "zkie_sumcheck_prove")
    return polys[:rounds], f_out, h_out


def mle_eval(d_vals: DeviceBuffer, num_vars: int, is_ext: bool, r, stream=None) -> np.ndarray:
    """sum_j eq(r, j) v[j] over a device table of 2^num_vars entries (EF, host)."""
    rr = np.ascontiguousarray(np.asarray(r, np.uint64).reshape(-1))
    assert rr.size == 2 * num_vars
    out = np.zeros(2, np.uint64)
    check(N.load().zkie_mle_eval(d_vals.addr, num_vars, 1 if is_ext else 0, N.p(rr), N.p(out), stream),
          "zkie_mle_eval")
    return out


def whir_encode(d_poly: DeviceBuffer, num_vars: int, is_ext: bool, log_width: int, log_inv_rate: int,
                prefix: bool, d_out: DeviceBuffer, stream=None):
    """commit_extension's codeword of a device table into d_out (row-major)."""
    check(N.load().zkie_whir_encode(d_poly.addr, num_vars, 1 if is_ext else 0, log_width, log_inv_rate,
                                    1 if prefix else 0, d_out.addr, stream), "zkie_whir_encode")
