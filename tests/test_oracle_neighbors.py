"""Pins of the oracle's neighbour lists (swarp/core/neighbors.py:76-97) against an
independent library routine (scipy's KD-tree ball query) and the reference's own
neighbour tests (tests/unit/test_neighbors.py:213-264)."""

import numpy as np
import pytest
from scipy.spatial import cKDTree

from oracle.oracle import Oracle


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("E,A,r", [(20, 16, 0.3), (8, 64, 0.5), (50, 4, 0.2)])
def test_sets_match_kdtree(dtype, E, A, r):
    rng = np.random.default_rng(E + A)
    pos = ((rng.random((E, A, 2)) * 2 - 1) * 1.5).astype(dtype)
    idx, cnt, tru = Oracle(dtype).neighbors(pos, r, A)
    for e in range(E):
        tree = cKDTree(pos[e].astype(np.float64))
        for a in range(A):
            want = set(tree.query_ball_point(pos[e, a].astype(np.float64), r)) - {a}
            got = idx[e, a, :cnt[e, a]]
            assert set(got.tolist()) == want
            assert list(got) == sorted(got)  # ascending index order (list order)
            assert tru[e, a] == len(want)


def test_overflow_cap_and_true_count():
    pos = np.zeros((1, 5, 2))
    pos[0, :, 0] = np.linspace(0.0, 0.04, 5)
    idx, cnt, tru = Oracle().neighbors(pos, 0.5, 2)
    np.testing.assert_array_equal(cnt, np.full((1, 5), 2))
    np.testing.assert_array_equal(tru, np.full((1, 5), 4))
    for a in range(5):
        want = [b for b in range(5) if b != a][:2]
        assert idx[0, a, :2].tolist() == want
    _, cnt8, tru8 = Oracle().neighbors(pos, 0.5, 8)
    assert (tru8 <= cnt8).all()


def test_membership_is_sqrt_le_radius_in_float32():
    r = np.float32(0.125)
    xs = np.array([r, np.nextafter(r, np.float32(1)), np.nextafter(r, np.float32(0))], np.float32)
    pos = np.zeros((3, 2, 2), np.float32)
    pos[:, 1, 0] = xs
    _, cnt, _ = Oracle(np.float32).neighbors(pos, float(r), 2)
    np.testing.assert_array_equal(cnt[:, 0], [1, 0, 1])


def test_no_cross_env_leaks():
    rng = np.random.default_rng(7)
    single = (rng.random((1, 16, 2)) * 2 - 1) * 0.3
    pos = np.repeat(single, 8, axis=0)
    idx, cnt, _ = Oracle().neighbors(pos, 0.4, 32)
    for e in range(1, 8):
        np.testing.assert_array_equal(idx[e], idx[0])
    assert idx.max() < 16
