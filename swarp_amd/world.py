"""``World``: the torch-facing container of one batched world -- state tensors, the
stepper, goals, obstacles, the neighbour lists (``swarp/core/world.py:35-491``).

The step is the HIP rollout kernel behind ``warp_step`` (differentiable when something
requires grad); there is no persistent CUDA-graph runtime (``enable_persistent``), so
every no-grad step takes the functional path with the stepper's two recycled output
slots.  Neighbour lists, the overflow flag and the COO graph come from the stepper's
``NeighborGrid`` built on the current (post-step) positions.
"""

from __future__ import annotations

import torch

from .autograd import TorchState, warp_step
from .config import AgentConfig, Obstacles, WorldConfig, action_dim
from .stepper import Stepper

_DTYPES = (torch.float32, torch.float64)


class World:
    """One batched multi-agent world: ``[n_envs, n_agents]`` on one device.

    Scenarios build it in ``make_world`` and write ``state`` / ``goals`` / obstacles in
    ``reset_world``; ``step`` advances it by one env step.
    """

    def __init__(
        self,
        agent_configs: list[AgentConfig],
        world_config: WorldConfig | None = None,
        n_envs: int = 1,
        device: str = "cuda:0",
        dt: float = 0.1,
        substeps: int = 1,
        dtype: torch.dtype = torch.float32,
    ) -> None:
        if n_envs < 1:
            raise ValueError(f"n_envs must be >= 1, got {n_envs}")
        if dtype not in _DTYPES:
            supported = ", ".join(str(k) for k in _DTYPES)
            raise TypeError(f"unsupported dtype {dtype!r} for World; supported: {supported}")
        self.n_envs = n_envs
        self.n_agents = len(agent_configs)
        self.device = str(device)
        self.dtype = dtype
        self.agent_configs = agent_configs
        # env-level action width: the widest model of the fleet
        self.act_dim = max(action_dim(c.model) for c in agent_configs)
        self.config = world_config
        self.stepper = Stepper(agent_configs, dt=dt, substeps=substeps, device=device,
                               dtype=dtype, world=world_config)
        self.state: TorchState = self.zero_state()
        self.action: torch.Tensor | None = None   # last applied action (set by Environment)
        self.goals: torch.Tensor | None = None    # [n_envs, n_agents, 2]
        self.obstacles: Obstacles | None = None
        self.obstacle_pos: torch.Tensor | None = None
        self.obstacle_radius: torch.Tensor | None = None
        self.obstacle_shape: torch.Tensor | None = None
        self.obstacle_angle: torch.Tensor | None = None
        self.obstacle_half_extents: torch.Tensor | None = None
        self.obstacle_kind: torch.Tensor | None = None
        self.generator: torch.Generator | None = None  # installed by Environment
        self.agent_radius = torch.tensor([c.radius for c in agent_configs], device=device,
                                         dtype=dtype)
        self.agent_shape = torch.tensor([int(c.shape) for c in agent_configs], device=device,
                                        dtype=torch.int32)
        self.agent_half_extents = torch.tensor([c.half_extents for c in agent_configs],
                                               device=device, dtype=dtype)
        # positions the neighbour lists were built on (None: stale)
        self._lists_of: torch.Tensor | None = None

    # ------------------------------------------------------------------ state

    def zero_state(self) -> TorchState:
        e, a = self.n_envs, self.n_agents

        def z(*shape):
            return torch.zeros(*shape, device=self.device, dtype=self.dtype)

        # every field materialised once (identity attitude), so a step never has to
        # allocate the defaults of the fields a 2-D fleet passes through
        att = z(e, a, 4)
        att[..., 3] = 1.0
        return TorchState(pos=z(e, a, 2), theta=z(e, a), vel=z(e, a, 2), speed=z(e, a),
                          ang_vel=z(e, a), z=z(e, a), vz=z(e, a), attitude=att,
                          body_rates=z(e, a, 3))

    def step(self, actions: torch.Tensor) -> None:
        """Advance the world one step (differentiable when grads are enabled)."""
        self.state = warp_step(self.stepper, self.state, actions)
        self._lists_of = None

    def write_state(
        self,
        mask: torch.Tensor | None = None,
        *,
        pos: torch.Tensor | None = None,
        theta: torch.Tensor | None = None,
        vel: torch.Tensor | None = None,
        speed: torch.Tensor | None = None,
        ang_vel: torch.Tensor | None = None,
    ) -> None:
        """Write state fields in place, optionally only into the envs of ``mask``
        (bool ``[n_envs]``); values broadcast against the destination
        (``swarp/core/world.py:216-255``)."""
        for name, value in (("pos", pos), ("theta", theta), ("vel", vel), ("speed", speed),
                            ("ang_vel", ang_vel)):
            if value is None:
                continue
            dst = getattr(self.state, name).data
            if mask is None:
                if torch.is_tensor(value):
                    dst.copy_(value.expand_as(dst))
                else:  # a number: a fill, not a copy from a host tensor (no sync)
                    dst.fill_(value)
            else:
                m = mask.view(-1, *([1] * (dst.dim() - 1)))
                dst.copy_(torch.where(m, value, dst))
        if pos is not None:
            self.mark_pos_dirty()

    def reset_state(self) -> None:
        """Reset the state to zeros (fresh tensors)."""
        self.state = self.zero_state()
        self.mark_pos_dirty()

    # ------------------------------------------------------------- randomness

    def sample_uniform(self, shape: tuple[int, ...], low: float, high: float) -> torch.Tensor:
        u = torch.rand(shape, generator=self.generator, device=self.device, dtype=self.dtype)
        return u * (high - low) + low

    # -------------------------------------------------------------- obstacles

    def set_obstacles(self, obstacles: Obstacles) -> None:
        """Install an obstacle set and keep the resolved spec
        (``swarp/core/world.py:333-357``)."""
        obs = obstacles.resolve(self.device, self.dtype)
        self.obstacles = obs
        self.obstacle_pos = obs.pos
        self.obstacle_radius = obs.radius
        self.obstacle_shape = obs.shape
        self.obstacle_angle = obs.angle
        self.obstacle_half_extents = obs.half_extents
        self.obstacle_kind = obs.kind
        self.stepper.set_obstacles(obs)

    # -------------------------------------------------------------- neighbours

    def build_neighbors(self) -> None:
        """Build the padded neighbour lists on the current (post-step) positions
        (``swarp/core/world.py:393-446``); a repeat call on unchanged positions is free."""
        if not self.stepper.collisions:
            raise RuntimeError("neighbor lists require WorldConfig.collisions=True")
        pos = self.state.pos
        if self._lists_of is pos:
            return
        self.stepper.grid(self.n_envs).build(pos.detach())
        self._lists_of = pos

    def neighbors(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``(neighbor_idx [n_envs, n_agents, K] int32, neighbor_count [n_envs, n_agents]
        int32)`` on the current state; overwritten by the next build."""
        self.build_neighbors()
        return self.stepper.grid(self.n_envs).torch_views()

    def lists_built_on(self, pos: torch.Tensor) -> None:
        """Record that the grid's lists were just built on ``pos`` by another launch
        (the scenario's fused pass builds them with its observations)."""
        self._lists_of = pos

    def mark_pos_dirty(self) -> None:
        """Invalidate the lists after positions were written out of band."""
        self._lists_of = None

    def neighbor_overflow(self) -> torch.Tensor:
        """Bool ``[n_envs, n_agents]``: in-radius count above ``max_neighbors`` on the
        last build (``swarp/core/world.py:476-480``)."""
        return self.stepper.grid(self.n_envs).overflow_view()

    def edge_index(self, rebuild: bool = True) -> torch.Tensor:
        """COO ``[2, n_edges]`` radius graph of the current state (one host sync)."""
        if rebuild:
            self.build_neighbors()
        return self.stepper.grid(self.n_envs).edge_index()
