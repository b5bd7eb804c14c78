"""Host-built decode work list (paged_ops.decode_work_list): every (row,
split) once, longest first, alternate dispatch passes reversed, then the rows
that need the split reduction. The small-batch path (plain Python) must give
the numpy path's list exactly."""
import numpy as np
import pytest

from minitorch_amd import paged_ops


def test_known_answer():
    # rows 0..4 of lengths 5, 9, 9, 1, 7 (ties by row), 2 rows per pass
    # (compute_units 4 // heads 2): LPT = 1, 2, 4, 0, 3 -> passes [1, 2], [4, 0]
    # reversed -> [0, 4], [3]
    work, items, merges = paged_ops.decode_work_list([5, 9, 9, 1, 7], 2, 1024, 4)
    assert items == 5 and merges == 0
    assert work.tolist() == [1, 0, 2, 0, 0, 0, 4, 0, 3, 0]


def test_split_rows_and_merge_list():
    # split 64: a 150-token row has splits of 64, 64, 22; merge rows follow
    work, items, merges = paged_ops.decode_work_list([150, 10], 1, 64, 1 << 20)
    assert items == 4 and merges == 1
    pairs = work[:2 * items].reshape(-1, 2).tolist()
    assert pairs == [[0, 0], [0, 1], [0, 2], [1, 0]]
    assert work[2 * items:].tolist() == [0]


@pytest.mark.parametrize('seed', range(20))
def test_small_path_equals_numpy_path(seed):
    rng = np.random.default_rng(seed)
    b = int(rng.integers(1, 33))
    heads = int(rng.choice([1, 12, 16, 25]))
    cu = int(rng.choice([8, 64, 256]))
    lengths = rng.integers(1, 1025, b).tolist()
    fast = paged_ops.decode_work_list(lengths, heads, 1024, cu)
    ref = paged_ops._numpy_work_list(lengths, heads, 1024, cu)
    assert fast[1:] == ref[1:]
    assert np.array_equal(fast[0], ref[0]) and fast[0].dtype == ref[0].dtype
