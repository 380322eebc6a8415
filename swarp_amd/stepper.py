"""Host side of the step: per-agent parameters, world constants, obstacles, and the
descriptor handed to the HIP library.

Counterpart of ``Stepper`` (``swarp/core/stepper.py:66-239, 295-432, 581-710``): the
same constructor, validation and error types, the same derived constants
(``sub_dt = dt / substeps``, the contact reach check, soft-wall / clamp flags), and
``set_obstacles`` with the same defaults.  The substep pipeline itself lives in one
HIP launch per rollout (``swarp_amd/csrc``), so there are no per-substep buffers
here; the no-grad path keeps the reference's two-slot ping-pong outputs.
"""

from __future__ import annotations

import ctypes
from typing import NamedTuple

import torch

from . import _lib
from .config import (
    AgentConfig,
    AgentShape,
    ControlMode,
    DynamicsModel,
    NUM_PARAMS,
    P_MAX_SPEED,
    P_RADIUS,
    P_SHAPE,
    Integrator,
    ObstacleKind,
    Obstacles,
    WorldConfig,
    action_dim,
)
from .neighbors import NeighborGrid, check_list_method, fill_list_order


class AgentParams(NamedTuple):
    """Device-resident per-agent parameters (``swarp/dynamics/base.py:334-349``)."""

    floats: torch.Tensor     # [n_agents, NUM_PARAMS]
    model_tag: torch.Tensor  # [n_agents] int32
    ctrl_mode: torch.Tensor  # [n_agents] int32


def build_agent_params(configs: list[AgentConfig], device, dtype) -> AgentParams:
    """Pack AgentConfig rows into device tensors (``swarp/dynamics/base.py:352-366``)."""
    rows = torch.tensor([c.to_row() for c in configs], dtype=torch.float64).to(dtype)
    tags = torch.tensor([int(c.model) for c in configs], dtype=torch.int32)
    modes = torch.tensor([int(c.ctrl_mode) for c in configs], dtype=torch.int32)
    return AgentParams(rows.to(device).contiguous(), tags.to(device), modes.to(device))


_DTYPES = {
    torch.float32: torch.float32,
    torch.float64: torch.float64,
    "float32": torch.float32,
    "float64": torch.float64,
    "fp32": torch.float32,
    "fp64": torch.float64,
}


def resolve_dtype(dtype) -> torch.dtype:
    """torch dtype of a Stepper precision given as a torch dtype or its name."""
    if isinstance(dtype, str):
        dtype = dtype.replace("torch.", "")
    try:
        return _DTYPES[dtype]
    except (KeyError, TypeError):
        raise TypeError(f"unsupported dtype {dtype!r}; use torch.float32 or torch.float64") from None


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class Stepper:
    """Owns per-agent parameters, interaction config and obstacles of one world.

    ``dtype`` is a torch dtype (``torch.float32`` / ``torch.float64``) or its name; the
    reference takes the matching Warp dtype.  Unlike the reference, a bare Stepper
    refuses model features this build does not implement instead of running them.
    """

    def __init__(
        self,
        configs: list[AgentConfig],
        dt: float = 0.1,
        substeps: int = 1,
        device: str = "cuda:0",
        dtype=torch.float32,
        world: WorldConfig | None = None,
    ) -> None:
        world = world if world is not None else WorldConfig(collisions=False)
        if substeps < 1:
            raise ValueError("substeps must be >= 1")
        if len(configs) < 1:
            raise ValueError("a Stepper needs at least one AgentConfig")
        self.configs = configs
        self.n_agents = len(configs)
        self.dt = dt
        self.substeps = substeps
        self.sub_dt = dt / substeps
        self.device = str(device)
        self.dtype = resolve_dtype(dtype)
        self.torch_dtype = self.dtype
        self.world = world
        self._check_supported()
        self.params = build_agent_params(configs, self.device, self.dtype)
        #: per-env parameter override [n_envs, n_agents, NUM_PARAMS] (None: shared rows)
        self.params_per_env: torch.Tensor | None = None
        self.act_dim = max(action_dim(c.model) for c in configs)
        self.has_drone = any(c.model == DynamicsModel.DRONE for c in configs)
        #: a box agent selects the box-aware contact pass and the footprint clamp
        #: (swarp/core/stepper.py:211-215)
        self.has_boxes = any(c.shape == AgentShape.BOX for c in configs)
        self.holo_velocity_only = all(
            c.model == DynamicsModel.HOLONOMIC and c.ctrl_mode == ControlMode.VELOCITY
            for c in configs
        )
        #: route eligible fleets to the specialised kernels (set False to force the
        #: generic ones; both give bit-identical results)
        self.use_specialised = True
        #: grad rollouts on the specialised kernels keep a tape of the substep
        #: intermediates, grad rollouts with movable bodies one of the body pass, so that
        #: the backward does not recompute them (set False to recompute; both give
        #: bit-identical results)
        self.use_tape = True
        #: route fleets whose features a compiled profile covers (2-D fleets with
        #: obstacles and walls under Euler, drone fleets, holonomic fleets pushing movable
        #: bodies) to the kernel instances compiled without the absent paths (set False
        #: for the general instances; both give bit-identical results)
        self.use_profiles = True

        self.collisions = world.collisions
        self.max_agent_radius = max(c.radius for c in configs)
        self.neighbor_radius = 0.0
        if self.collisions:
            reach = 2.0 * self.max_agent_radius + world.collision_margin
            self.neighbor_radius = world.neighbor_radius or reach
            if self.neighbor_radius < reach:
                raise ValueError(
                    f"neighbor_radius={self.neighbor_radius} is smaller than the collision "
                    f"reach {reach} (= 2 * max radius + margin); collisions would be missed."
                )
        self._soft_walls = world.bounds is not None and world.bounds_mode == "soft"
        self._clamp = world.bounds is not None and world.bounds_mode == "clamp"
        if world.bounds is not None:
            x_min, x_max, y_min, y_max = world.bounds
            self._bounds = (x_min, y_min, x_max, y_max)
        else:
            self._bounds = (0.0, 0.0, 0.0, 0.0)

        self.n_obstacles = 0
        self.n_body_roots = 0
        self._obstacle_types = 0  # bit set of the obstacle shape types present
        self.obstacles: Obstacles | None = None
        self._obs: dict[str, torch.Tensor] = {}
        self.any_movable = False
        #: movable bodies: the per-env obstacle state [n_envs, 12 N] entering the next
        #: rollout (advanced by every rollout) and the last rollout's [T, n_envs, 12 N]
        self.ob_state: torch.Tensor | None = None
        self.ob_trajectory: torch.Tensor | None = None
        self._descs: dict[tuple[int, int], _lib.SwarpDesc] = {}
        self._tape_sizes: dict[tuple[int, int], int] = {}
        self._grids: dict[int, NeighborGrid] = {}
        self._out_states: dict[int, list] = {}
        self._out_idx: dict[int, int] = {}
        self.mutation_version = 0

    # ------------------------------------------------------------------ checks

    def _check_supported(self) -> None:
        w = self.world
        #: the resolved neighbour-list order ("brute" or "uniform_grid")
        self.list_method = check_list_method(w.neighbor_method, self.n_agents, w.uniform_bins,
                                             stepping=True)
        # envs over 64 agents, or grid-ordered lists, step on the wide-env kernels
        self.wide = self.n_agents > 64 or self.list_method == "uniform_grid"
        if self.wide:
            if self.list_method == "uniform_grid" and w.collisions and w.bounds is None:
                raise NotImplementedError(
                    "stepping with uniform-grid lists needs WorldConfig.bounds: the adaptive "
                    "grid frame is a reduction over every env at every substep")
        drone = any(c.model == DynamicsModel.DRONE for c in self.configs)
        if w.wheel_contacts and (drone or w.integrator.value != "euler"):
            # swarp/core/stepper.py:852-857
            raise ValueError(
                "WorldConfig.wheel_contacts runs on the slim Euler 2D path only (no drone "
                "agents, untaped, Integrator.EULER)")

    # ------------------------------------------------------- per-env parameters

    def set_agent_params_per_env(self, floats) -> None:
        """Install a per-env parameter table ``[n_envs, n_agents, NUM_PARAMS]`` (domain
        randomization; columns in ``AgentConfig.to_row()`` order, see
        ``per_env_float_template``).  Counterpart of
        ``swarp/core/stepper.py:493-575``: the shape is checked, the ``P_SHAPE`` column
        must equal the configs' (a footprint is structural), and with collisions the
        largest per-env radius must fit the neighbour radius; those two host reads run
        only on a first install or a reallocation.  Refreshing an installed table with a
        device tensor of the same shape and dtype is an in-place copy with no host read
        (the per-reset re-randomization path), trusted against the bound checked then."""
        is_torch = torch.is_tensor(floats)
        shape = tuple(floats.shape)
        if len(shape) != 3 or shape[1:] != (self.n_agents, NUM_PARAMS):
            raise ValueError(
                f"per-env params must have shape [n_envs, n_agents={self.n_agents}, "
                f"NUM_PARAMS={NUM_PARAMS}]; got {shape}")
        cur = self.params_per_env
        if (is_torch and cur is not None and tuple(cur.shape) == shape
                and floats.dtype == self.dtype and floats.device == cur.device):
            cur.copy_(floats)
            return
        t = torch.as_tensor(floats, dtype=torch.float64).to("cpu")
        shared = torch.tensor([float(c.shape) for c in self.configs], dtype=torch.float64)
        if not torch.equal(t[..., P_SHAPE], shared.expand(shape[0], -1)):
            raise ValueError("per-env params must not change the P_SHAPE column: an agent's "
                             "AgentShape is structural and fixed by its AgentConfig.")
        if self.collisions:
            max_r = float(t[..., P_RADIUS].max())
            reach = 2.0 * max_r + self.world.collision_margin
            if self.neighbor_radius < reach:
                raise ValueError(
                    f"per-env radius up to {max_r} needs neighbor_radius >= {reach} "
                    f"(= 2 * max per-env radius + margin), but neighbor_radius="
                    f"{self.neighbor_radius}; set WorldConfig.neighbor_radius accordingly.")
        self.params_per_env = t.to(device=self.device, dtype=self.dtype).contiguous()
        self._pe_skin_speed = float(t[..., P_MAX_SPEED].max())
        self._descs.clear()
        self._tape_sizes.clear()
        # a new table is a new device address: descriptors and captured graphs that baked
        # the old one must be rebuilt
        self.mutation_version += 1

    # --------------------------------------------------------------- obstacles

    def set_obstacles(self, obstacles: Obstacles) -> None:
        """Install the obstacle set (``swarp/core/stepper.py:295-432``); absent fields
        take their documented defaults.  With MOVABLE obstacles the per-env obstacle state
        ``ob_state`` ``[n_envs, 12 N]`` is seeded from the shapes' installed poses
        (``_body_seed``, ``swarp/core/stepper.py:434-476``) and advanced by every rollout."""
        obs = obstacles.resolve(self.device, self.dtype)
        n_envs, n = obs.n_envs, obs.n_obstacles
        z = {"device": self.device, "dtype": self.dtype}
        zi = {"device": self.device, "dtype": torch.int32}
        self._obs = {
            "pos": obs.pos,
            "radius": obs.radius,
            "type": obs.shape if obs.shape is not None else torch.zeros(n, **zi),
            "angle": obs.angle if obs.angle is not None else torch.zeros(n_envs, n, **z),
            "half": obs.half_extents if obs.half_extents is not None else torch.zeros(n, 2, **z),
            "vel": obs.vel if obs.vel is not None else torch.zeros(n_envs, n, 2, **z),
            "ang_vel": obs.ang_vel if obs.ang_vel is not None else torch.zeros(n_envs, n, **z),
            "kind": obs.kind if obs.kind is not None else torch.zeros(n, **zi),
            "body": obs.body if obs.body is not None else torch.arange(n, **zi),
            "mass": obs.mass if obs.mass is not None else torch.ones(n, **z),
            "inertia": obs.inertia if obs.inertia is not None else torch.ones(n, **z),
            "off": obs.body_offset if obs.body_offset is not None else torch.zeros(n, 2, **z),
        }
        body = self._obs["body"]
        if n > 0 and bool(((body < 0) | (body >= n)).any()):
            raise ValueError(f"obstacle body indices must lie in [0, {n})")
        movable = obs.any_movable
        if movable and self.has_boxes:
            raise NotImplementedError("movable bodies with box agents are not implemented")
        if movable and self.n_agents > 1024:
            raise NotImplementedError(
                "movable bodies step at most 1024 agents per env (one thread per agent in the "
                "env's workgroup)")
        self.obstacles = obstacles
        self.n_obstacles = n
        self._obs_envs = n_envs
        self.any_movable = movable
        # shape types present (bit t: type t), for the kernel instance without box / segment
        # terms when every obstacle is a circle
        self._obstacle_types = sum(1 << int(t) for t in torch.unique(self._obs["type"].cpu())) if n else 0
        # movable bodies (roots: body[o] = o and kind[o] = 1), the records of a body tape
        if n:
            b, k = body.cpu(), self._obs["kind"].cpu()
            self.n_body_roots = int(((b == torch.arange(n, dtype=b.dtype)) & (k == 1)).sum())
        else:
            self.n_body_roots = 0
        self.ob_state = self._body_seed() if movable else None
        self.ob_trajectory = None
        self._descs.clear()
        self._tape_sizes.clear()
        self.mutation_version += 1

    def _body_seed(self) -> torch.Tensor:
        """Obstacle state [n_envs, 12 N]: per shape its installed pose and velocity, then
        per index the state of the body rooted there, derived from the root shape: origin
        = root pos - R(root angle) @ root offset; heading, velocity and spin the root's."""
        o = self._obs
        pos, ang, vel, om = (o["pos"].double(), o["angle"].double(), o["vel"].double(),
                             o["ang_vel"].double())
        n_envs, n = pos.shape[0], pos.shape[1]
        root = o["body"].long()
        off = o["off"].double()[root]                       # [N, 2] offset of each root
        ra = ang[:, root]                                   # [E, N]
        ca, sa = torch.cos(ra), torch.sin(ra)
        wx = ca * off[:, 0] - sa * off[:, 1]
        wy = sa * off[:, 0] + ca * off[:, 1]
        shapes = torch.cat([pos, ang.unsqueeze(-1), vel, om.unsqueeze(-1)], -1)  # [E, N, 6]
        bodies = torch.stack([pos[:, root, 0] - wx, pos[:, root, 1] - wy, ra,
                              vel[:, root, 0], vel[:, root, 1], om[:, root]], -1)
        return torch.cat([shapes.reshape(n_envs, 6 * n), bodies.reshape(n_envs, 6 * n)],
                         -1).to(self.dtype).contiguous()

    @property
    def _needs_forces(self) -> bool:
        return self.collisions or self._soft_walls or self.n_obstacles > 0

    # --------------------------------------------------------------- descriptor

    def desc(self, n_envs: int, act_dim: int) -> _lib.SwarpDesc:
        """The (cached) C descriptor of this world for a batch of ``n_envs``."""
        key = (n_envs, act_dim)
        d = self._descs.get(key)
        if d is not None:
            return d
        if self.n_obstacles > 0 and self._obs_envs != n_envs:
            raise ValueError(
                f"obstacles were installed for {self._obs_envs} envs, stepping {n_envs}"
            )
        d = _lib.SwarpDesc()
        d.abi_version = _lib.ABI_VERSION
        d.dtype = _lib.F64 if self.dtype == torch.float64 else _lib.F32
        d.n_envs = n_envs
        d.n_agents = self.n_agents
        d.act_dim = act_dim
        d.substeps = self.substeps
        d.max_neighbors = self.world.max_neighbors if self.collisions else 0
        d.n_obstacles = self.n_obstacles
        d.collisions = int(self.collisions)
        d.soft_walls = int(self._soft_walls)
        # a world holding box agents clamps every agent's footprint (kernels.py:74-99)
        d.clamp_bounds = (2 if self.has_boxes else 1) if self._clamp else 0
        d.has_drone = int(self.has_drone)
        d.has_boxes = int(self.has_boxes)
        d.wheel_contacts = int(self.world.wheel_contacts)
        d.lat_grip = float(self.world.wheel_lateral_friction * self.world.gravity)
        d.turn_cap = float(self.world.wheel_turn_torque)
        d.holo_velocity_only = int(self.use_specialised and self.holo_velocity_only
                                   and self.n_obstacles == 0 and not self._clamp
                                   and not self.has_boxes and not self.world.wheel_contacts)
        d.dt = float(self.dt)
        d.k = float(self.world.collision_k)
        d.c = float(self.world.collision_c)
        d.margin = float(self.world.collision_margin)
        d.max_overlap = float(self.world.contact_max_overlap)
        d.neighbor_radius = float(self.neighbor_radius)
        bx0, by0, bx1, by1 = self._bounds
        d.bounds_min[0], d.bounds_min[1] = bx0, by0
        d.bounds_max[0], d.bounds_max[1] = bx1, by1
        if self.params_per_env is not None:
            if self.params_per_env.shape[0] != n_envs:
                raise ValueError(
                    f"per-env params were installed for {self.params_per_env.shape[0]} envs, "
                    f"stepping {n_envs}")
            d.params = self.params_per_env.data_ptr()
            d.params_per_env = 1
            # the body pass reads the shared rows (swarp/core/stepper.py:961-964)
            d.body_params = self.params.floats.data_ptr()
        else:
            d.params = self.params.floats.data_ptr()
        d.model_tag = self.params.model_tag.data_ptr()
        d.ctrl_mode = self.params.ctrl_mode.data_ptr()
        if self.n_obstacles > 0:
            o = self._obs
            d.obs_pos = o["pos"].data_ptr()
            d.obs_radius = o["radius"].data_ptr()
            d.obs_angle = o["angle"].data_ptr()
            d.obs_half = o["half"].data_ptr()
            d.obs_vel = o["vel"].data_ptr()
            d.obs_ang_vel = o["ang_vel"].data_ptr()
            d.obs_type = o["type"].data_ptr()
            d.obs_kind = o["kind"].data_ptr()
            d.obs_body = o["body"].data_ptr()
            d.obs_mass = o["mass"].data_ptr()
            d.obs_inertia = o["inertia"].data_ptr()
            d.obs_body_off = o["off"].data_ptr()
        d.obstacle_types = self._obstacle_types
        d.lin_damping = float(self.world.obstacle_linear_damping)
        d.ang_damping = float(self.world.obstacle_angular_damping)
        d.integrator = _lib.RK4 if self.world.integrator == Integrator.RK4 else _lib.EULER
        d.skin_speed = self._skin_speed()
        fill_list_order(d, self.list_method, self.n_agents, self.world.uniform_bins,
                        self.world.bounds, float(self.neighbor_radius))
        if self.use_profiles:  # 0 (unset) selects the general instances
            d.fleet_models = sum(1 << m for m in {int(c.model) for c in self.configs})
            d.fleet_modes = sum(1 << m for m in {int(c.ctrl_mode) for c in self.configs})
        self._descs[key] = d
        return d

    def _skin_speed(self) -> float:
        """The fleet's top speed (largest max_speed of the rows in use): sizes the
        neighbour search's per-step skin (speed only; the lists are exact regardless)."""
        if self.params_per_env is not None:
            return self._pe_skin_speed  # recorded at install (no device read here)
        return float(max(c.max_speed for c in self.configs))

    # --------------------------------------------------------------- neighbours

    def tape_bytes(self, n_envs: int, act_dim: int, T: int) -> int:
        """Size of the rollout tape of a T-step grad rollout (0: no tape is kept)."""
        if not self.use_tape:
            return 0
        d = self.desc(n_envs, act_dim)
        key = (ctypes.addressof(d), T)  # a descriptor lives until the world changes
        n = self._tape_sizes.get(key)
        if n is None:
            c = ctypes.c_uint64(0)
            _lib.check(_lib.load().swarp_tape_bytes(ctypes.byref(d), T, ctypes.byref(c)))
            n = self._tape_sizes[key] = int(c.value)
        return n

    def ob_tape_bytes(self, n_envs: int, act_dim: int, T: int) -> int:
        """Size of the body tape of a T-step grad rollout of a world with movable bodies,
        holding every movable body (0: no tape is kept)."""
        if not self.use_tape or not self.any_movable or self.n_body_roots < 1 or self.wide:
            return 0  # (the wide kernels keep no body tape)
        d = self.desc(n_envs, act_dim)
        key = (ctypes.addressof(d), T, "ob")
        n = self._tape_sizes.get(key)
        if n is None:
            c = ctypes.c_uint64(0)
            _lib.check(_lib.load().swarp_ob_tape_bytes(ctypes.byref(d), T, self.n_body_roots,
                                                       ctypes.byref(c)))
            n = self._tape_sizes[key] = int(c.value)
        return n

    def grid(self, n_envs: int) -> NeighborGrid:
        g = self._grids.get(n_envs)
        if g is None:
            g = NeighborGrid(
                n_envs,
                self.n_agents,
                radius=self.neighbor_radius if self.collisions else 2.0 * self.max_agent_radius
                + self.world.collision_margin,
                max_neighbors=self.world.max_neighbors,
                device=self.device,
                dtype=self.dtype,
                grid_dim=self.world.grid_dim,
                method=self.world.neighbor_method,
                uniform_bins=self.world.uniform_bins,
                bounds=self.world.bounds,
            )
            self._grids[n_envs] = g
        return g

    # --------------------------------------------------------------- allocation

    def alloc_state(self, n_envs: int, requires_grad: bool = False):
        from .autograd import TorchState

        z = {"device": self.device, "dtype": self.dtype}
        att = torch.zeros(n_envs, self.n_agents, 4, **z)
        att[..., 3] = 1.0
        st = TorchState(
            pos=torch.zeros(n_envs, self.n_agents, 2, **z),
            theta=torch.zeros(n_envs, self.n_agents, **z),
            vel=torch.zeros(n_envs, self.n_agents, 2, **z),
            speed=torch.zeros(n_envs, self.n_agents, **z),
            ang_vel=torch.zeros(n_envs, self.n_agents, **z),
            z=torch.zeros(n_envs, self.n_agents, **z),
            vz=torch.zeros(n_envs, self.n_agents, **z),
            attitude=att,
            body_rates=torch.zeros(n_envs, self.n_agents, 3, **z),
        )
        if requires_grad:
            st = type(st)(*(t.requires_grad_(True) for t in st))
        return st

    def output_state(self, n_envs: int):
        """Ping-pong output slot of the no-grad path (``swarp/core/stepper.py:688-710``):
        valid until this batch size is stepped twice more."""
        states = self._out_states.get(n_envs)
        if states is None:
            states = [self.alloc_state(n_envs), self.alloc_state(n_envs)]
            self._out_states[n_envs] = states
            self._out_idx[n_envs] = 0
        i = self._out_idx[n_envs]
        self._out_idx[n_envs] = 1 - i
        return states[i]

    def launch_substeps(self, state_in, actions: torch.Tensor, state_out) -> None:
        """Advance one env step from ``state_in`` into ``state_out`` (no autograd)."""
        from .autograd import _launch_fwd

        _launch_fwd(self, state_in, actions.unsqueeze(0), None, state_out)


_FIELD_NAMES = ("pos", "theta", "vel", "speed", "ang_vel", "z", "vz", "attitude", "body_rates")
_FIELD_WIDTH = (2, 1, 2, 1, 1, 1, 1, 4, 3)


def check_extent(t, n: int, name: str, dtype=None) -> None:
    """Host-side extent check of a tensor handed to the library: contiguous, of `dtype`,
    with exactly `n` elements -- the reach the kernels index it with.  Raises before any
    launch instead of letting a kernel read or write past the tensor."""
    if t is None:
        return
    if not t.is_contiguous():
        raise ValueError(f"{name}: the library takes contiguous tensors")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, the launch needs {dtype}")
    if t.numel() != n:
        raise ValueError(f"{name}: {t.numel()} elements {tuple(t.shape)}, the launch indexes {n}")


def state_struct(fields, n: int | None = None, dtype=None, what: str = "state") -> _lib.SwarpState:
    """SwarpState of up to nine tensors (None = NULL).  With `n` (the lead dimensions times
    n_envs * n_agents), each field is checked to hold exactly n * its width elements."""
    s = _lib.SwarpState()
    for k, (name, t) in enumerate(zip(_FIELD_NAMES, fields)):
        if n is not None:
            check_extent(t, n * _FIELD_WIDTH[k], f"{what}.{name}", dtype)
        setattr(s, name, _ptr(t))
    return s


def byref(x):
    return ctypes.byref(x)
