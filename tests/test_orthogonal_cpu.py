"""Orthogonal draws (run.py:223-238) in the oracle, pinned by exact properties a wrong row, offset, cycle or
index rule breaks: a cycle of d draws at one frame position is an orthogonal set (A A^T = d I), a chunked
call continues the same frame, two ranks' shares of one cycle are orthogonal to each other (the shared
frame, run.py:228-231), frame positions use independent offsets, and entries are +-1."""
import numpy as np
import pytest

from oracle.orthogonal import OrthogonalDrawsOracle, orthogonal_directions


def test_one_cycle_is_orthogonal():
    for d in (8, 64, 512):
        A = OrthogonalDrawsOracle(seed=0)('s', d, 0, d, 1, 1, d).reshape(d, d)
        assert set(np.unique(A)) <= {-1.0, 1.0}
        assert np.array_equal(A @ A.T, d * np.eye(d))


def test_second_cycle_uses_its_own_pattern():
    d = 16
    A = OrthogonalDrawsOracle(seed=1)('s', 2 * d, 0, 2 * d, 1, 1, d).reshape(2 * d, d)
    assert np.array_equal(A[:d] @ A[:d].T, d * np.eye(d))
    assert np.array_equal(A[d:] @ A[d:].T, d * np.eye(d))
    # same Hadamard rows in both cycles (offset + index mod d), different cycle patterns: columns flip
    flips = (A[:d] * A[d:])  # row-wise product of draw i and draw i + d: pattern ratio times sign ratio
    assert not np.all(np.abs(flips.sum(1)) == d), 'cycle patterns must differ'


def test_chunks_continue_the_frame():
    d = 32
    od = OrthogonalDrawsOracle(seed=2)
    a = od('s', d, 0, d // 2, 1, 1, d).reshape(d // 2, d)
    b = od('s', d, 1, d // 2, 1, 1, d).reshape(d // 2, d)
    A = np.concatenate([a, b])
    assert np.array_equal(A @ A.T, d * np.eye(d))


def test_ranks_share_the_frame():
    d = 64
    parts = [OrthogonalDrawsOracle(seed=3, rank=r, world=2)('s', d // 2, 0, d // 2, 1, 1, d).reshape(d // 2, d)
             for r in (0, 1)]
    A = np.concatenate(parts)
    assert np.array_equal(A @ A.T, d * np.eye(d))


def test_frame_positions_are_independent():
    d = 16
    A = OrthogonalDrawsOracle(seed=4)('s', d, 0, d, 2, 3, d)   # [d, 2, 3, d]
    for bb in range(2):
        for tt in range(3):
            X = A[:, bb, tt, :]
            assert np.array_equal(X @ X.T, d * np.eye(d))
    # six positions, offsets drawn independently: their first draws are not all the same row (seed 4)
    first = {A[0, bb, tt].tobytes() for bb in range(2) for tt in range(3)}
    assert len(first) > 1


def test_non_power_of_two_rejected():
    with pytest.raises(ValueError, match='power-of-two'):
        OrthogonalDrawsOracle()('s', 4, 0, 4, 1, 1, 48)


def test_weight_space_directions_shapes():
    shapes = {'w1': (64, 16), 'w2': (16, 32)}
    dirs = orthogonal_directions(shapes, 8, seed=0)
    assert dirs['w1'][0].shape == (8, 64) and dirs['w1'][1].shape == (8, 16)
    assert dirs['w2'][0].shape == (8, 16) and dirs['w2'][1].shape == (8, 32)
    a = dirs['w1'][0]
    assert np.array_equal(a @ a.T, 64 * np.eye(8))  # 8 draws of one cycle of 64
