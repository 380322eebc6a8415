"""Padded radius-neighbour lists, overflow flag and COO radius graph.

Counterpart of ``NeighborGrid`` (``swarp/core/neighbors.py:334-733``) for the brute
method, which the reference itself selects for <= 512 agents per env
(``:388-389``): ``build`` / ``query_into`` fill ``neighbor_idx [E,A,K]``,
``neighbor_count [E,A]`` and ``neighbor_true_count [E,A]`` on the HIP device;
``overflow_view`` and ``edge_index`` keep the reference's semantics (including the
one host sync ``edge_index`` needs for the edge count).  Entries of ``neighbor_idx``
past the count are zero.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


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
        if method not in ("auto", "grid", "brute", "uniform_grid"):
            raise ValueError('method must be "auto", "grid", "brute", or "uniform_grid"')
        if method in ("grid", "uniform_grid"):
            raise NotImplementedError(f"method={method!r}: only the brute-force lists are built")
        if max_neighbors < 1:
            raise ValueError("max_neighbors must be >= 1")
        if n_agents > 64:
            raise NotImplementedError("this build lists at most 64 agents per env")
        from .stepper import resolve_dtype

        self.n_envs = n_envs
        self.n_agents = n_agents
        self.radius = radius
        self.max_neighbors = max_neighbors
        self.device = str(device)
        self.dtype = resolve_dtype(dtype)
        self.method = "brute"
        self.grid_dim = grid_dim
        self.uniform_bins = uniform_bins
        self._bounds = bounds
        z = {"device": self.device, "dtype": torch.int32}
        self.neighbor_idx = torch.zeros(n_envs, n_agents, max_neighbors, **z)
        self.neighbor_count = torch.zeros(n_envs, n_agents, **z)
        self.neighbor_true_count = torch.zeros(n_envs, n_agents, **z)
        self.build_count = 0
        self.built_version = -1
        d = _lib.SwarpDesc()
        d.abi_version = _lib.ABI_VERSION
        d.dtype = _lib.F64 if self.dtype == torch.float64 else _lib.F32
        d.n_envs = n_envs
        d.n_agents = n_agents
        d.act_dim = 2
        d.substeps = 1
        d.max_neighbors = max_neighbors
        d.collisions = 1
        d.neighbor_radius = float(radius)
        d.dt = 1.0
        self._desc = d

    def build(self, pos: torch.Tensor, reset_mask=None) -> None:
        """Refresh the internal lists from positions ``[n_envs, n_agents, 2]``."""
        self.query_into(pos, self.neighbor_idx, self.neighbor_count)

    def build_brute_force(self, pos: torch.Tensor) -> None:
        self.query_into(pos, self.neighbor_idx, self.neighbor_count)

    def query_into(self, pos: torch.Tensor, neighbor_idx: torch.Tensor,
                   neighbor_count: torch.Tensor, reset_mask=None) -> None:
        """Write padded lists into caller-owned int32 buffers (true count into the grid's)."""
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
        pos = pos.contiguous()
        lib = _lib.load()
        stream = _lib.stream_of(pos.device)
        _lib.check(lib.swarp_neighbors(
            ctypes.byref(self._desc), pos.data_ptr(), neighbor_idx.data_ptr(),
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
        cnt = self.neighbor_count.reshape(-1).to(torch.int64)
        incl = torch.cumsum(cnt, 0)
        n_edges = int(incl[-1].item()) if cnt.numel() else 0
        out = torch.empty(2, n_edges, device=self.device, dtype=torch.int64)
        if n_edges == 0:
            return out
        offsets = (incl - cnt).contiguous()
        lib = _lib.load()
        stream = _lib.stream_of(out.device)
        _lib.check(lib.swarp_edge_index(
            self.n_envs, self.n_agents, self.max_neighbors, self.neighbor_idx.data_ptr(),
            self.neighbor_count.data_ptr(), offsets.data_ptr(), n_edges, out.data_ptr(), stream,
        ))
        return out
