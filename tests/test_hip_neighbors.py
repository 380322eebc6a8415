"""Neighbour lists, overflow flag and COO radius graph on the HIP device: bit-exact
against the oracle's restatement of _brute_force (swarp/core/neighbors.py:76-97) and
the reference's own neighbour tests (tests/unit/test_neighbors.py:213-305)."""

import numpy as np
import pytest
import torch

from oracle.oracle import Oracle
from swarp_amd import NeighborGrid

pytestmark = pytest.mark.gpu


def _hip_lists(pos_np, radius, K, dtype=torch.float32):
    E, A = pos_np.shape[:2]
    g = NeighborGrid(E, A, radius=radius, max_neighbors=K, device="cuda:0", dtype=dtype)
    g.build(torch.tensor(pos_np, dtype=dtype, device="cuda"))
    return g, (g.neighbor_idx.cpu().numpy(), g.neighbor_count.cpu().numpy(),
               g.neighbor_true_count.cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("E,A,radius,K", [(64, 4, 0.125, 4), (500, 16, 0.3, 16), (40, 32, 0.5, 8),
                                          (30, 64, 0.3, 16), (7, 5, 0.2, 2), (3, 1, 0.5, 4),
                                          (33, 12, 0.4, 7), (9, 24, 0.35, 12)])
def test_lists_bitexact(dtype, E, A, radius, K):
    rng = np.random.default_rng(E * 131 + A)
    npdt = np.float32 if dtype == torch.float32 else np.float64
    pos = (rng.random((E, A, 2)) * 2 - 1).astype(npdt) * 1.5
    _, (idx, cnt, tru) = _hip_lists(pos, radius, K, dtype)
    oi, oc, ot = Oracle(npdt).neighbors(pos, radius, K)
    np.testing.assert_array_equal(cnt, oc)
    np.testing.assert_array_equal(tru, ot)
    for e in range(E):
        for a in range(A):
            np.testing.assert_array_equal(idx[e, a, :cnt[e, a]], oi[e, a, :oc[e, a]])
    mask = np.arange(K)[None, None, :] >= cnt[..., None]
    assert (idx[mask] == 0).all()


def test_boundary_pairs_exact():
    """Pairs placed exactly at and one ulp around the radius: the membership decision
    must equal sqrt(d2) <= r computed in float32."""
    r = np.float32(0.125)
    xs = np.array([r, np.nextafter(r, np.float32(1)), np.nextafter(r, np.float32(0)),
                   np.float32(0.1), np.float32(0.0883883476)], dtype=np.float32)
    pos = np.zeros((len(xs), 2, 2), dtype=np.float32)
    pos[:, 1, 0] = xs
    pos[-1, 1, 1] = np.float32(0.0883883476)
    _, (idx, cnt, tru) = _hip_lists(pos, float(r), 4)
    d = np.sqrt((pos[:, 1, 0] - pos[:, 0, 0]) ** 2 + (pos[:, 1, 1] - pos[:, 0, 1]) ** 2,
                dtype=np.float32)
    np.testing.assert_array_equal(cnt[:, 0], (d <= r).astype(np.int32))


def test_overflow_flag():
    pos = np.zeros((1, 5, 2), dtype=np.float32)
    pos[0, :, 0] = np.linspace(0.0, 0.04, 5)
    g, (idx, cnt, tru) = _hip_lists(pos, 0.5, 2)
    np.testing.assert_array_equal(tru, np.full((1, 5), 4))
    np.testing.assert_array_equal(cnt, np.full((1, 5), 2))
    assert g.overflow_view().all()
    g2, _ = _hip_lists(pos, 0.5, 8)
    assert not g2.overflow_view().any()


def test_no_cross_env_leaks():
    rng = np.random.default_rng(7)
    single = ((rng.random((1, 16, 2)) * 2 - 1) * 0.3).astype(np.float32)
    pos = np.repeat(single, 8, axis=0)
    _, (idx, cnt, _) = _hip_lists(pos, 0.4, 32)
    for e in range(1, 8):
        np.testing.assert_array_equal(idx[e], idx[0])
        np.testing.assert_array_equal(cnt[e], cnt[0])
    assert idx.min() >= 0 and idx.max() < 16


def test_edge_index_order_and_set():
    rng = np.random.default_rng(5)
    E, A = 3, 16
    pos = ((rng.random((E, A, 2)) * 2 - 1) * 0.4).astype(np.float32)
    g, (idx, cnt, _) = _hip_lists(pos, 0.3, 32)
    edges = g.edge_index().cpu().numpy()
    exp = [(e * A + idx[e, a, k], e * A + a) for e in range(E) for a in range(A) for k in range(cnt[e, a])]
    assert edges.dtype == np.int64
    assert [tuple(x) for x in edges.T.tolist()] == exp  # (e, a, slot) order, reference layout


def test_edge_index_empty():
    pos = np.array([[[0.0, 0.0], [5.0, 5.0]]], dtype=np.float32)
    g, _ = _hip_lists(pos, 0.3, 4)
    assert g.edge_index().shape == (2, 0)
