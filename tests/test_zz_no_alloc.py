"""``swarp_edge_index_noalloc`` (the allocation-free COO radius graph) against the existing
entry point ``swarp_edge_index`` (through ``NeighborGrid.edge_index``), both called
through the C ABI: identical edges in identical order, on two calls in a row with the
second one smaller (the file-scope scratch keeps the first call's partial sums), a
capacity below the edge count (edges past it dropped, the true count still reported),
the size limit rejected before any launch, and the call replayed from a captured HIP
graph."""

import ctypes

import numpy as np
import pytest
import torch

from swarp_amd import NeighborGrid, _lib

pytestmark = pytest.mark.gpu

LIMIT = 65536 * 256  # n_envs * n_agents the scratch array covers


def _lists(E, A, r, K, spread, seed):
    rng = np.random.default_rng(seed)
    pos = rng.uniform(-spread, spread, size=(E, A, 2)).astype(np.float32)
    g = NeighborGrid(E, A, radius=r, max_neighbors=K, device="cuda:0", dtype=torch.float32)
    g.build(torch.tensor(pos, device="cuda"))
    return g


def _noalloc(g, E, A, K, capacity):
    out = torch.full((2, max(capacity, 1)), -7, dtype=torch.int64, device="cuda")
    n = torch.full((1,), -1, dtype=torch.int64, device="cuda")
    lib = _lib.load()
    rc = lib.swarp_edge_index_noalloc(E, A, K, g.neighbor_idx.data_ptr(),
                                      g.neighbor_count.data_ptr(), capacity, out.data_ptr(),
                                      n.data_ptr(), _lib.stream_of(out.device))
    _lib.check(rc)
    return out, n


@pytest.mark.parametrize("shapes", [((4000, 64, 0.3, 16, 3.0), (700, 64, 0.3, 16, 3.0)),
                                    ((3000, 16, 0.5, 16, 1.0), (5, 16, 0.5, 16, 1.0))])
def test_two_calls_match_existing_entry_point(shapes):
    for k, (E, A, r, K, spread) in enumerate(shapes):
        g = _lists(E, A, r, K, spread, seed=10 + k)
        ref = g.edge_index()  # swarp_edge_index with torch's prefix sums
        cap = E * A * K
        out, n = _noalloc(g, E, A, K, cap)
        m = ref.shape[1]
        assert int(n.item()) == m
        assert m > 0
        assert torch.equal(out[:, :m], ref), f"call {k}: edges differ"
        assert (out[:, m:] == -7).all(), f"call {k}: wrote past the edge count"


def test_capacity_truncates_and_reports_the_count():
    E, A, K = 500, 32, 8
    g = _lists(E, A, 0.4, K, 1.0, seed=3)
    ref = g.edge_index()
    m = ref.shape[1]
    cap = m // 3
    out, n = _noalloc(g, E, A, K, cap)
    assert int(n.item()) == m
    assert torch.equal(out[:, :cap], ref[:, :cap])


def test_rejects_sizes_beyond_the_limit():
    g = _lists(2, 4, 0.3, 4, 1.0, seed=1)
    lib = _lib.load()
    n = torch.zeros(1, dtype=torch.int64, device="cuda")
    out = torch.zeros(2, 8, dtype=torch.int64, device="cuda")
    E = LIMIT // 64 + 1
    rc = lib.swarp_edge_index_noalloc(E, 64, 4, g.neighbor_idx.data_ptr(),
                                      g.neighbor_count.data_ptr(), 8, out.data_ptr(),
                                      n.data_ptr(), _lib.stream_of(out.device))
    assert rc != 0
    assert b"allocation-free limit" in lib.swarp_last_error()


_FIRST_CALL_IN_CAPTURE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np, torch
from swarp_amd import NeighborGrid, _lib
E, A, K = 300, 64, 16
g = NeighborGrid(E, A, radius=0.3, max_neighbors=K, device="cuda:0", dtype=torch.float32)
rng = np.random.default_rng(21)
g.build(torch.tensor(rng.uniform(-3, 3, size=(E, A, 2)), dtype=torch.float32, device="cuda"))
ref = g.edge_index()
cap = E * A * K
out = torch.full((2, cap), -7, dtype=torch.int64, device="cuda")
n = torch.zeros(1, dtype=torch.int64, device="cuda")
lib = _lib.load()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # the process's first call of the entry point
    _lib.check(lib.swarp_edge_index_noalloc(E, A, K, g.neighbor_idx.data_ptr(),
                                            g.neighbor_count.data_ptr(), cap, out.data_ptr(),
                                            n.data_ptr(), _lib.stream_of(out.device)))
for _ in range(2):
    out.fill_(-7)
    graph.replay()
    torch.cuda.synchronize()
    m = ref.shape[1]
    assert int(n.item()) == m and torch.equal(out[:, :m], ref)
print("ok", m)
"""


def test_first_call_inside_graph_capture():
    """The scratch array's address is looked up on the first call on a device; a first
    call made while torch captures a graph (global capture mode) must work too.  Run in a
    fresh process, so that this call is the process's first."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr


def test_replays_from_a_captured_graph():
    E, A, K = 1000, 64, 16
    g = _lists(E, A, 0.3, K, 3.0, seed=5)
    cap = E * A * K
    out = torch.full((2, cap), -7, dtype=torch.int64, device="cuda")
    n = torch.zeros(1, dtype=torch.int64, device="cuda")
    lib = _lib.load()
    pos = torch.empty(E, A, 2, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _lib.check(lib.swarp_edge_index_noalloc(E, A, K, g.neighbor_idx.data_ptr(),
                                                g.neighbor_count.data_ptr(), cap, out.data_ptr(),
                                                n.data_ptr(), _lib.stream_of(out.device)))
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.swarp_edge_index_noalloc(E, A, K, g.neighbor_idx.data_ptr(),
                                                g.neighbor_count.data_ptr(), cap, out.data_ptr(),
                                                n.data_ptr(), _lib.stream_of(out.device)))
    rng = np.random.default_rng(9)
    for k in range(3):
        pos.copy_(torch.tensor(rng.uniform(-3, 3, size=(E, A, 2)), dtype=torch.float32))
        g.build(pos)
        ref = g.edge_index()
        out.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        m = ref.shape[1]
        assert int(n.item()) == m, k
        assert torch.equal(out[:, :m], ref), f"replay {k}"
