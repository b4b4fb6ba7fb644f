"""Pins of the oracle's Whir::commit_batch restatement (stack_tables,
commit_batch). The table-major stacking order is the layout the reference
hands to its external initial-round committer, so the order itself is
parity unpinned; these tests pin that the stack is encoded as that layout
says, through what the encoding fixes:
- one table: the batch commit is the single-table commit of that table;
- linearity over the tables: the stack's codeword is the sum of the
  codewords of stacks holding one table each, the others zero;
- placement: a table at slot i (rows from i R on, R rows per table)
  multiplies the coefficient polynomial of every column by X^(i R), so
  codeword row t is w_n^(t i R) times that of the same table at slot 0;
- the zero padding: a stack of 3 tables equals one of 4 whose last is zero.
A plausible slip (tables in reverse order, column-major stacking, padding
in front) fails the placement or the padding check."""
import numpy as np
import pytest

P = 0xFFFFFFFF00000001


def _tables(oracle, count, arity, seed):
    return [oracle.gen_uniform(seed + 17 * i, 1 << arity) for i in range(count)]


def test_single_table_is_single_commit(oracle):
    t = _tables(oracle, 1, 8, 3)
    stack, cw, layers, root = oracle.commit_batch(t, 2, 2)
    m = t[0].reshape(-1, 4)
    assert (stack == m).all()
    assert (cw == oracle.lde_batch(m, 2)).all()
    _, root1 = oracle.merkle_commit(oracle.lde_batch(m, 2))
    assert (root == root1).all()


@pytest.mark.parametrize("count,arity,k,lb", [(3, 6, 2, 1), (4, 5, 3, 2), (5, 3, 1, 1), (2, 7, 4, 2)])
def test_linearity_and_placement(oracle, count, arity, k, lb):
    ts = _tables(oracle, count, arity, count + arity)
    stack, cw, _, _ = oracle.commit_batch(ts, k, lb)
    zero = np.zeros(1 << arity, np.uint64)
    n = cw.shape[0]
    w_n = oracle.two_adic_generator(n.bit_length() - 1)
    R = (1 << arity) >> k if arity >= k else None
    acc = np.zeros_like(cw)
    for i in range(count):
        alone = [ts[j] if j == i else zero for j in range(count)]
        _, cw_i, _, _ = oracle.commit_batch(alone, k, lb)
        acc = (acc.astype(object) + cw_i.astype(object)) % P
        if R is None:
            continue
        # the same table in slot 0 of an otherwise zero stack
        first = [ts[i]] + [zero] * (count - 1)
        _, cw_0, _, _ = oracle.commit_batch(first, k, lb)
        for t in range(0, n, max(1, n // 16)):
            f = pow(w_n, t * i * R, P)
            assert all(int(cw_i[t, c]) == int(cw_0[t, c]) * f % P for c in range(cw.shape[1])), (i, t)
    assert (acc.astype(np.uint64) == cw).all()


def test_padding_is_a_zero_table(oracle):
    ts = _tables(oracle, 3, 6, 9)
    s3, cw3, _, r3 = oracle.commit_batch(ts, 2, 2)
    s4, cw4, _, r4 = oracle.commit_batch(ts + [np.zeros(64, np.uint64)], 2, 2)
    assert s3.shape == s4.shape == (64, 4)
    assert (s3 == s4).all() and (cw3 == cw4).all() and (r3 == r4).all()
    assert (s3.reshape(-1)[192:] == 0).all()


def test_rejects_bad_batches(oracle):
    with pytest.raises(ValueError):
        oracle.stack_tables([], 2)
    with pytest.raises(ValueError):
        oracle.stack_tables([np.zeros(8, np.uint64), np.zeros(4, np.uint64)], 1)
    with pytest.raises(ValueError):
        oracle.stack_tables([np.zeros(2, np.uint64)], 3)
