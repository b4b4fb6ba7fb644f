"""STIR query indices (p3-whir src/pcs/utils.rs:70-119): min(q, H) distinct
uniform indices in [0, H), drawn until that many distinct ones exist, then
sorted ascending. The seeded generator stands in for the challenger, so the
checks are the function's contract: count, range, order, the cap at the
domain size, and how many draws it consumes (later rounds draw from the same
generator)."""
import numpy as np
import pytest

from zkie_amd import configs as C


def _stream(seed: int, n: int):
    g = C.XorShift64(seed)
    return [g.next_u64() for _ in range(n)]


@pytest.mark.parametrize("count,height", [(64, 1 << 19), (128, 1 << 13), (128, 1 << 9), (12, 16), (5, 8)])
def test_distinct_sorted_in_range(count, height):
    idx = C.query_indices(count, height, C.XorShift64(C.SEED_QUERIES))
    assert idx.dtype == np.uint64
    assert len(idx) == min(count, height)
    assert (np.diff(idx.astype(np.int64)) > 0).all()
    assert int(idx.max()) < height


@pytest.mark.parametrize("count,height", [(128, 1 << 9), (12, 16), (40, 64)])
def test_first_distinct_draws_and_consumption(count, height):
    """The indices are the first min(count, height) distinct draws, and the
    generator stops right after the draw that completed them."""
    g = C.XorShift64(7)
    idx = C.query_indices(count, height, g)
    raw = _stream(7, 4096)
    seen, used = [], 0
    for v in raw:
        used += 1
        if v % height not in seen:
            seen.append(v % height)
        if len(seen) == min(count, height):
            break
    assert [int(i) for i in idx] == sorted(seen)
    assert g.next_u64() == raw[used]
    # with this many draws into a small domain, repeats were rejected
    if height <= 64:
        assert used > len(seen)


def test_count_at_least_height_opens_every_row():
    for height in (1, 2, 16, 64):
        idx = C.query_indices(height + 3, height, C.XorShift64(3))
        assert [int(i) for i in idx] == list(range(height))


def test_height_must_be_a_power_of_two():
    with pytest.raises(AssertionError):
        C.query_indices(4, 24, C.XorShift64(1))
