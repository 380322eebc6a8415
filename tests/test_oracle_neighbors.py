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


# ------------------------------------------------------------------ uniform-grid order
# Pins of the oracle's uniform-grid lists (swarp/core/neighbors.py:149-254) against the
# reference's own uniform-grid tests (tests/unit/test_neighbors.py:83-199): the same sets
# and counts as brute force when no list is truncated, pinned frames included, points
# outside a pinned rectangle included; and, for the order itself, a hand-placed layout
# whose traversal is written out below.


def _sets(idx, cnt):
    E, A, _ = idx.shape
    return [[set(idx[e, a, :cnt[e, a]].tolist()) for a in range(A)] for e in range(E)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("E,A", [(1, 8), (4, 32), (2, 128), (2, 600)])
@pytest.mark.parametrize("r", [0.15, 0.5])
@pytest.mark.parametrize("pinned", [False, True])
def test_grid_sets_match_brute(dtype, E, A, r, pinned):
    rng = np.random.default_rng(42)
    pos = ((rng.random((E, A, 2)) * 2 - 1) * 2.0).astype(dtype)
    O = Oracle(dtype)
    bins = max(4, min(128, int(np.ceil(np.sqrt(A)))))
    frame = (-2.0, -2.0, max(r, 4.0 / bins)) if pinned else None
    ui, uc, ut, _ = O.neighbors_grid(pos, r, 128, bins, frame)
    bi, bc, bt = O.neighbors(pos, r, 128)
    assert not (bt > 128).any()
    assert np.array_equal(uc, bc) and np.array_equal(ut, bt)
    assert _sets(ui, uc) == _sets(bi, bc)


def test_grid_points_outside_pinned_rectangle():
    rng = np.random.default_rng(11)
    pos = ((rng.random((3, 64, 2)) * 2 - 1) * 3.0).astype(np.float32)
    O = Oracle(np.float32)
    ui, uc, ut, _ = O.neighbors_grid(pos, 0.3, 128, 8, (-1.0, -1.0, max(0.3, 2.0 / 8)))
    bi, bc, bt = O.neighbors(pos, 0.3, 128)
    assert np.array_equal(uc, bc) and np.array_equal(ut, bt)
    assert _sets(ui, uc) == _sets(bi, bc)


def test_grid_adaptive_frame_is_min_corner_and_cell_floor():
    pos = np.array([[[0.5, -1.0], [2.5, 3.0], [1.0, 0.0]]], dtype=np.float32)
    O = Oracle(np.float32)
    _, _, _, fr = O.neighbors_grid(pos, 0.1, 4, 4)
    # origin = min corner; extent = max(2.0, 4.0) = 4.0; cell = max(0.1, 4.0 / 4)
    assert fr.tolist() == [0.5, -1.0, 1.0]
    _, _, _, fr = O.neighbors_grid(pos, 1.5, 4, 4)
    assert fr[2] == np.float32(1.5)  # the radius is a floor on the cell size


def test_grid_traversal_order_and_cap():
    """Agent 0 at the centre of cell (1, 1) of a 3 x 3 grid of unit cells; its in-radius
    neighbours sit in known cells.  The list visits the 3x3 block row by row (dy = -1, 0,
    +1 outer; dx = -1, 0, +1 inner) and a cell's agents by ascending index; the cap keeps
    the first K of that order."""
    P = {0: (1.5, 1.5),
         1: (2.2, 2.2),   # cell (2, 2): slot 8
         2: (0.8, 1.5),   # cell (0, 1): slot 3
         3: (1.5, 0.9),   # cell (1, 0): slot 1
         4: (1.4, 1.6),   # cell (1, 1): slot 4
         5: (2.1, 1.5),   # cell (2, 1): slot 5
         6: (1.2, 1.2),   # cell (1, 1): slot 4 (after 4)
         7: (0.95, 0.95)}  # cell (0, 0): slot 0
    pos = np.array([[P[a] for a in range(8)]], dtype=np.float64)
    O = Oracle(np.float64)
    frame = (0.0, 0.0, 1.0)
    idx, cnt, tru, _ = O.neighbors_grid(pos, 1.0, 8, 3, frame)
    assert cnt[0, 0] == 7 and tru[0, 0] == 7
    assert idx[0, 0, :7].tolist() == [7, 3, 2, 4, 6, 5, 1]
    bidx, _, _ = O.neighbors(pos, 1.0, 8)
    assert bidx[0, 0, :7].tolist() == [1, 2, 3, 4, 5, 6, 7]
    idx, cnt, tru, _ = O.neighbors_grid(pos, 1.0, 3, 3, frame)
    assert cnt[0, 0] == 3 and tru[0, 0] == 7 and idx[0, 0].tolist() == [7, 3, 2]


def test_grid_cell_clamps_into_the_edge_cells():
    """(p - o) / cs truncated, then clamped into [0, bins): a point left of the origin
    lands in cell 0, one far right in the last cell, and the distance test still decides
    membership."""
    pos = np.array([[[-0.5, 0.5], [0.4, 0.5], [9.0, 0.5], [2.6, 0.5]]], dtype=np.float64)
    O = Oracle(np.float64)
    # radius 1: 0 and 1 are neighbours (cells 0 and 0), 2 and 3 too (cells 2 and 2)
    idx, cnt, _, _ = O.neighbors_grid(pos, 1.0, 4, 3, (0.0, 0.0, 1.0))
    assert idx[0, 0, :cnt[0, 0]].tolist() == [1]
    assert cnt[0, 2] == 0  # |9.0 - 2.6| > 1 although both clamp into cell 2
    assert cnt[0, 3] == 0 and cnt[0, 1] == 1
