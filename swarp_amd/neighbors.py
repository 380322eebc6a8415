"""Padded radius-neighbour lists, overflow flag and COO radius graph.

Counterpart of ``NeighborGrid`` (``swarp/core/neighbors.py:334-733``):
``build`` / ``query_into`` fill ``neighbor_idx [E,A,K]``, ``neighbor_count [E,A]`` and
``neighbor_true_count [E,A]`` on the HIP device in the order of the resolved method --
``"brute"`` (ascending agent index, ``:76-97``) or ``"uniform_grid"`` (the 3x3 cell block
row by row, ascending index within a cell, ``:149-254, 622-687``), ``"auto"`` picking the
grid above 512 agents as the reference does (``:388-389``).  The grid frame is pinned by
``bounds`` or reduced over the batch on every build.  ``overflow_view`` and
``edge_index`` keep the reference's semantics (including the one host sync
``edge_index`` needs for the edge count).  Entries of ``neighbor_idx`` past the count are
zero.  The hash-grid method (``"grid"``, Warp's ``HashGrid``, whose query order is
Warp's) is not built.
"""

from __future__ import annotations

import ctypes
import math
import warnings

import torch

from . import _lib


def resolve_method(method: str, n_agents: int) -> str:
    """NeighborGrid's choice of list order (``swarp/core/neighbors.py:387-389``)."""
    if method == "auto":
        return "uniform_grid" if n_agents > 512 else "brute"
    return method


def grid_bins(n_agents: int, uniform_bins: int | None) -> int:
    """Cells per axis of the uniform grid (``swarp/core/neighbors.py:390-393``)."""
    return uniform_bins or max(4, min(128, int(math.ceil(math.sqrt(n_agents)))))


def pinned_frame(bounds, radius: float, bins: int) -> tuple[float, float, float]:
    """The frame a world rectangle pins, in float64 as the reference computes it
    (``NeighborGrid._fill_static_grid``, ``swarp/core/neighbors.py:476-490``):
    origin (x_min, y_min), cell size max(radius, extent / bins)."""
    x_min, x_max, y_min, y_max = bounds
    extent = max(x_max - x_min, y_max - y_min)
    return float(x_min), float(y_min), float(max(radius, extent / bins))


def fill_list_order(d, method: str, n_agents: int, uniform_bins: int | None, bounds,
                    radius: float) -> None:
    """The descriptor's list-order fields for a resolved method."""
    if method == "uniform_grid":
        bins = grid_bins(n_agents, uniform_bins)
        d.neighbor_method = _lib.LISTS_GRID
        d.grid_bins = bins
        if bounds is not None:
            ox, oy, cs = pinned_frame(bounds, radius, bins)
            d.grid_pinned = 1
            d.grid_origin[0], d.grid_origin[1] = ox, oy
            d.grid_cell = cs
    else:
        d.neighbor_method = _lib.LISTS_BRUTE


def wide_slots(n_agents: int) -> int:
    """Agent slots of an env's workgroup (``wide_geom``): 64-agent granules spread over at
    most 1024 threads, 1, 2 or 4 agents per thread."""
    ap = -(-n_agents // 64) * 64
    apt = -(-ap // 1024)
    apt = 4 if apt == 3 else apt
    return -(-(-(-ap // apt)) // 64) * 64 * apt


def _check_bins(bins: int, n_agents: int) -> None:
    """The cell table (bins^2 + 1 offsets) and the env's float32 agent staging (44 B per
    agent slot) share one workgroup's 160 KiB of LDS (``wide_lds_bytes``); float64 and box
    worlds stage more, which the library checks at the call."""
    if wide_slots(n_agents) * 44 + (bins * bins + 1) * 4 + 64 > 163840:
        raise NotImplementedError(
            f"uniform_bins={bins}: {bins * bins} cells per env with {n_agents} agents exceed "
            "the 160 KiB of LDS of the workgroup that holds an env")


def check_list_method(method: str, n_agents: int, uniform_bins: int | None,
                      stepping: bool = False) -> str:
    """Validates a NeighborGrid / WorldConfig method for this build; returns the resolved
    method.  ``stepping``: the lists also order the step's contact sums, so the cell
    limit of the wide-env kernels applies now rather than at the first build."""
    if method not in ("auto", "grid", "brute", "uniform_grid"):
        raise ValueError('method must be "auto", "grid", "brute", or "uniform_grid"')
    if method == "grid":
        raise NotImplementedError(
            'method="grid" (Warp\'s HashGrid, whose query order is Warp\'s own) is not built; '
            'use "brute" or "uniform_grid"')
    if uniform_bins is not None and uniform_bins < 1:
        raise ValueError("uniform_bins must be >= 1")
    if n_agents > _lib.WIDE_MAX_AGENTS:
        raise NotImplementedError(
            f"this build lists at most {_lib.WIDE_MAX_AGENTS} agents per env (one workgroup "
            "per env)")
    m = resolve_method(method, n_agents)
    if m == "uniform_grid":
        bins = grid_bins(n_agents, uniform_bins)
        if stepping:
            _check_bins(bins, n_agents)
        if bins * bins > 16 * max(1, n_agents):
            warnings.warn(
                f"uniform_bins={bins} gives {bins * bins} cells per env for {n_agents} agents; "
                "the default heuristic (~sqrt(n_agents)) keeps occupancy near one agent per "
                "cell.", RuntimeWarning, stacklevel=3)
    return m


class NeighborGrid:
    def __init__(
        self,
        n_envs: int,
        n_agents: int,
        radius: float,
        max_neighbors: int = 32,
        device: str = "cuda:0",
        dtype=torch.float32,
        grid_dim: int = 128,
        method: str = "auto",
        uniform_bins: int | None = None,
        bounds: tuple[float, float, float, float] | None = None,
    ) -> None:
        if radius <= 0.0:
            raise ValueError("radius must be positive")
        if max_neighbors < 1:
            raise ValueError("max_neighbors must be >= 1")
        method = check_list_method(method, n_agents, uniform_bins)
        from .stepper import resolve_dtype

        self.n_envs = n_envs
        self.n_agents = n_agents
        self.radius = radius
        self.max_neighbors = max_neighbors
        self.device = str(device)
        self.dtype = resolve_dtype(dtype)
        self.method = method
        self.grid_dim = grid_dim
        self.uniform_bins = grid_bins(n_agents, uniform_bins)
        self._bounds = bounds
        z = {"device": self.device, "dtype": torch.int32}
        self.neighbor_idx = torch.zeros(n_envs, n_agents, max_neighbors, **z)
        self.neighbor_count = torch.zeros(n_envs, n_agents, **z)
        self.neighbor_true_count = torch.zeros(n_envs, n_agents, **z)
        # edge_index's running sums of the counts: [0, c0, c0 + c1, ...] (the leading
        # zero is written once, so [:-1] are the exclusive offsets and [-1] the edge count)
        self._csum = torch.zeros(n_envs * n_agents + 1, device=self.device, dtype=torch.int64)
        self.build_count = 0
        self.built_version = -1
        # the batch-reduced grid frame (origin x, y, cell size) of the last build
        self._frame = torch.zeros(3, device=self.device, dtype=self.dtype)
        self._descs = {m: self._make_desc(m) for m in ("brute", "uniform_grid")}

    def _make_desc(self, method: str):
        d = _lib.SwarpDesc()
        d.abi_version = _lib.ABI_VERSION
        d.dtype = _lib.F64 if self.dtype == torch.float64 else _lib.F32
        d.n_envs = self.n_envs
        d.n_agents = self.n_agents
        d.act_dim = 2
        d.substeps = 1
        d.max_neighbors = self.max_neighbors
        d.collisions = 1
        d.neighbor_radius = float(self.radius)
        d.dt = 1.0
        fill_list_order(d, method, self.n_agents, self.uniform_bins, self._bounds, self.radius)
        if method == "uniform_grid" and not d.grid_pinned:
            d.grid_frame = self._frame.data_ptr()
        return d

    def build(self, pos: torch.Tensor, reset_mask=None) -> None:
        """Refresh the internal lists from positions ``[n_envs, n_agents, 2]``."""
        self.query_into(pos, self.neighbor_idx, self.neighbor_count)

    def build_brute_force(self, pos: torch.Tensor) -> None:
        """Force the index-ordered lists into the internal buffers."""
        self._query(pos, self.neighbor_idx, self.neighbor_count, "brute")

    def build_uniform(self, pos: torch.Tensor) -> None:
        """Force the uniform-grid lists into the internal buffers."""
        self._query(pos, self.neighbor_idx, self.neighbor_count, "uniform_grid")

    def build_grid(self, pos: torch.Tensor) -> None:
        raise NotImplementedError("the hash-grid lists (Warp's HashGrid order) are not built")

    def grid_frame(self) -> torch.Tensor:
        """The batch-reduced frame of the last uniform-grid build: origin x, origin y,
        cell size (a pinned frame is not written here)."""
        return self._frame

    def query_into(self, pos: torch.Tensor, neighbor_idx: torch.Tensor,
                   neighbor_count: torch.Tensor, reset_mask=None) -> None:
        """Write padded lists into caller-owned int32 buffers (true count into the grid's)."""
        self._query(pos, neighbor_idx, neighbor_count, self.method)

    def _query(self, pos, neighbor_idx, neighbor_count, method: str) -> None:
        if method == "uniform_grid":
            _check_bins(self.uniform_bins, self.n_agents)
        if pos.shape != (self.n_envs, self.n_agents, 2):
            raise ValueError(
                f"pos must be [{self.n_envs}, {self.n_agents}, 2]; got {tuple(pos.shape)}"
            )
        if pos.dtype != self.dtype:
            raise TypeError(f"pos dtype {pos.dtype} does not match the grid's {self.dtype}")
        if not pos.is_cuda:
            raise RuntimeError("swarp_amd builds neighbour lists on the HIP device only")
        for t in (neighbor_idx, neighbor_count):
            if t.dtype != torch.int32 or not t.is_contiguous():
                raise TypeError("neighbour buffers must be contiguous int32")
        EA = self.n_envs * self.n_agents
        for t, n, name in ((neighbor_idx, EA * self.max_neighbors, "neighbor_idx"),
                           (neighbor_count, EA, "neighbor_count")):
            if t.numel() != n:  # the reach the list kernels write
                raise ValueError(f"{name}: {t.numel()} elements {tuple(t.shape)}, the build writes {n}")
        pos = pos.contiguous()
        lib = _lib.load()
        stream = _lib.stream_of(pos.device)
        _lib.check(lib.swarp_neighbors(
            ctypes.byref(self._descs[method]), pos.data_ptr(), neighbor_idx.data_ptr(),
            neighbor_count.data_ptr(), self.neighbor_true_count.data_ptr(), stream,
        ))
        self.build_count += 1

    def torch_views(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.neighbor_idx, self.neighbor_count

    def true_count_view(self) -> torch.Tensor:
        return self.neighbor_true_count

    def overflow_view(self) -> torch.Tensor:
        """bool ``[n_envs, n_agents]``: true count above ``max_neighbors`` (list truncated)."""
        return self.neighbor_true_count > self.neighbor_count

    def edge_index(self) -> torch.Tensor:
        """COO ``[2, n_edges]`` int64 (sender, receiver), global ids ``e * A + a``, in
        (env, agent, slot) order.  Reads the edge count back to the host (one sync)."""
        cnt = self.neighbor_count.reshape(-1)
        if cnt.numel() == 0:
            return torch.empty(2, 0, device=self.device, dtype=torch.int64)
        torch.cumsum(cnt, 0, dtype=torch.int64, out=self._csum[1:])
        n_edges = int(self._csum[-1].item())
        out = torch.empty(2, n_edges, device=self.device, dtype=torch.int64)
        if n_edges == 0:
            return out
        offsets = self._csum[:-1]
        lib = _lib.load()
        stream = _lib.stream_of(out.device)
        _lib.check(lib.swarp_edge_index(
            self.n_envs, self.n_agents, self.max_neighbors, self.neighbor_idx.data_ptr(),
            self.neighbor_count.data_ptr(), offsets.data_ptr(), n_edges, out.data_ptr(), stream,
        ))
        return out
