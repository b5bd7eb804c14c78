"""Host writer of the fragment-tiled operand layout (model.fragment_tiled),
which the decode projection kernel reads for its weights. Known answers: the
first lanes of the first 1 KB block, the zero padding rows, and the block
order; the GPU tests check that a tiled operand gives the row-major result bit
for bit."""
import numpy as np
import pytest

from minitorch_amd.model import fragment_tiled


def test_known_answer_first_block():
    a = np.arange(16 * 64, dtype=np.float32).reshape(16, 64)   # value = 64 r + c
    t = fragment_tiled(a)
    assert t.shape == (16 * 64,)
    # lane 0 of block (0, 0): row 0, columns 0..7; lane 1: row 1, columns 0..7
    assert t[:8].tolist() == list(range(8))
    assert t[8:16].tolist() == [64 + c for c in range(8)]
    # lane 16 (g = 1, c = 0): row 0, columns 8..15
    assert t[16 * 8:16 * 8 + 8].tolist() == list(range(8, 16))
    # block (0, 1) starts at element 512 with row 0, columns 32..39
    assert t[512:520].tolist() == list(range(32, 40))


def test_padding_rows_and_block_order():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((37, 96)).astype(np.float32)
    t = fragment_tiled(a)
    assert t.size == 48 * 96                              # rows padded to 48
    blocks = t.reshape(3, 3, 4, 16, 8)                    # [row tile, column tile, g, c, e]
    assert np.all(blocks[2, :, :, 5:, :] == 0)            # rows 37..47 are zeros
    for r, c in [(0, 0), (15, 31), (16, 32), (36, 95), (20, 47)]:
        assert blocks[r // 16, c // 32, (c % 32) // 8, r % 16, c % 8] == a[r, c]


def test_rejects_width_not_multiple_of_32():
    with pytest.raises(ValueError):
        fragment_tiled(np.zeros((16, 48), np.float32))
