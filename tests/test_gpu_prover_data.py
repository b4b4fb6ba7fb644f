"""GPU parity of the prover-data cache stream: the bytes streamed out of HBM
equal the oracle's serialisation of the oracle's tree over the same matrix,
byte for byte, and reading them back restores a tree that opens exactly like
the one committed. Framing errors, short streams and failing callbacks are
host-side errors (nothing malformed reaches a kernel)."""
import hashlib
import io

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _commit(native, oracle, h, w, seed):
    from zkie_amd import pcs
    from zkie_amd._native import DeviceBuffer

    mat = oracle.gen_uniform(seed, h * w).reshape(h, w)
    tree = pcs.HipMerkleTreeMmcs().commit_device(DeviceBuffer.from_array(mat), h, w)
    return mat, tree


@pytest.mark.parametrize("h,w", [(1, 1), (3, 2), (8, 8), (1000, 7), (4101, 16), (257, 33)])
def test_stream_matches_oracle_bytes(native, oracle, h, w):
    from zkie_amd import pcs

    print(f"CASE prover_data h={h} w={w}", flush=True)
    mat, tree = _commit(native, oracle, h, w, 40 + h + w)
    out = io.BytesIO()
    n = pcs.serialize_batch_prover_data_into(tree, out)
    layers, _ = oracle.merkle_commit(mat)
    want = oracle.prover_data_bytes(mat, layers)
    assert n == len(want) == native.prover_data_size(h, w)
    assert out.getvalue() == want


def test_stream_in_several_staged_pieces(native, oracle):
    """A 2^18 x 16 tree: 32 MiB of matrix and 32 MiB of digest layers, each
    more than one 16 MiB staging piece."""
    from zkie_amd import pcs

    h, w = 1 << 18, 16
    print(f"CASE prover_data pieces h={h} w={w}", flush=True)
    mat, tree = _commit(native, oracle, h, w, 5)
    pieces, digest = [], hashlib.sha256()

    def sink(view):
        pieces.append(len(view))
        digest.update(view)

    native.prover_data_write(tree.d_mat.addr, h, w, tree.d_layers.addr, sink)
    assert max(pieces) == 16 << 20 and len(pieces) >= 6
    layers, _ = oracle.merkle_commit(mat)
    assert digest.digest() == hashlib.sha256(oracle.prover_data_bytes(mat, layers)).digest()


@pytest.mark.parametrize("h,w", [(3, 2), (1000, 7), (1 << 18, 16)])
def test_restore_round_trip_opens_identically(native, oracle, h, w):
    from zkie_amd import pcs

    print(f"CASE prover_data restore h={h} w={w}", flush=True)
    mat, tree = _commit(native, oracle, h, w, 77 + w)
    buf = io.BytesIO()
    pcs.serialize_batch_prover_data_into(tree, buf)
    buf.seek(0)
    back = pcs.restore_batch_prover_data_from(buf, h, w)
    assert (back.root == tree.root).all()
    assert (back.matrix() == mat).all()
    assert (back.d_layers.download() == tree.d_layers.download()).all()
    mmcs = pcs.HipMerkleTreeMmcs()
    idx = np.array(sorted({0, h - 1, h // 2, h // 3}), np.uint64)
    r0, s0 = mmcs.open_batches(idx, tree)
    r1, s1 = mmcs.open_batches(idx, back)
    assert (r0 == r1).all() and (s0 == s1).all()
    assert (mmcs.open_multi_batch(idx, back)[1] == mmcs.open_multi_batch(idx, tree)[1]).all()


def test_restore_rejects_other_shapes_and_short_streams(native, oracle):
    from zkie_amd import pcs
    from zkie_amd._native import ZkieError

    print("CASE prover_data errors", flush=True)
    h, w = 100, 4
    mat, tree = _commit(native, oracle, h, w, 9)
    buf = io.BytesIO()
    pcs.serialize_batch_prover_data_into(tree, buf)
    data = buf.getvalue()
    for hh, ww in ((100, 5), (99, 4), (128, 4)):
        with pytest.raises(ZkieError):
            pcs.restore_batch_prover_data_from(io.BytesIO(data), hh, ww)
    with pytest.raises(EOFError):
        pcs.restore_batch_prover_data_from(io.BytesIO(data[:-8]), h, w)
    # a layer length that disagrees with the geometry of a 100-row tree
    off = 8 * (3 + h * w) + 8
    bad = data[:off] + (129).to_bytes(8, "little") + data[off + 8:]
    with pytest.raises(ZkieError):
        pcs.restore_batch_prover_data_from(io.BytesIO(bad), h, w)
    # an arity other than 2
    nl = len(oracle.layer_lens(h))
    off = 8 * (3 + h * w) + 8 * (1 + nl)
    bad = data[:off] + (4).to_bytes(8, "little") + data[off + 8:]
    with pytest.raises(ZkieError):
        pcs.restore_batch_prover_data_from(io.BytesIO(bad), h, w)


def test_write_callback_error_propagates(native, oracle):
    from zkie_amd import pcs

    print("CASE prover_data sink error", flush=True)
    _, tree = _commit(native, oracle, 64, 8, 3)

    class Full(io.RawIOBase):
        def write(self, b):
            raise OSError("no space left")

    with pytest.raises(OSError):
        pcs.serialize_batch_prover_data_into(tree, Full())
    # the library is still usable afterwards
    assert pcs.serialize_batch_prover_data_into(tree, io.BytesIO()) == native.prover_data_size(64, 8)
