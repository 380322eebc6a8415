"""Agent, world and obstacle configuration: the reference's public config surface.

These dataclasses keep the reference's field names, defaults, validation and error
types so a caller's configuration code carries over unchanged:

* ``AgentConfig`` / ``DynamicsModel`` / ``ControlMode`` / ``AgentShape`` /
  ``Integrator`` / ``PARAM_FIELDS`` / ``action_bounds`` follow
  ``swarp/dynamics/base.py:12-331`` (the parameter-row layout is an interface the
  kernels index by column, so its order is kept exactly).
* ``WorldConfig`` follows ``swarp/core/config.py:181-322`` (``override_with`` keeps
  the "non-default fields only" rule of ``:277-302``).
* ``Obstacles`` follows ``swarp/core/config.py:39-178``.
* ``drone_config`` follows ``swarp/dynamics/drone.py:24-53``.

What the MI355X build does not run is rejected loudly rather than silently
approximated, with ``NotImplementedError`` when a ``Stepper`` is built with it (or the
bodies installed): movable bodies together with box agents or wheel contacts; more than
4096 agents per env (1024 with movable bodies); the hash-grid list order; and stepping with grid-ordered lists
without world bounds.  Configurations whose per-env staging exceeds a workgroup's LDS
fail at the library call with a message that says so.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field, fields, replace
from enum import Enum, IntEnum

import torch


class DynamicsModel(IntEnum):
    """Model tag read by the integrate kernels (``swarp/dynamics/base.py:12-19``)."""

    HOLONOMIC = 0
    DIFF_DRIVE = 1
    KINEMATIC_BICYCLE = 2
    DRONE = 3


MODEL_ACTION_DIM = {
    "HOLONOMIC": 2,
    "DIFF_DRIVE": 2,
    "KINEMATIC_BICYCLE": 2,
    "DRONE": 4,
}


class ControlMode(IntEnum):
    """Meaning of the action slots (``swarp/dynamics/base.py:57-78``)."""

    VELOCITY = 0
    ACCELERATION = 1
    SERVO = 2


class AgentShape(IntEnum):
    """Agent footprint tag (``swarp/dynamics/base.py:81-94``)."""

    DISC = 0
    BOX = 1


class Integrator(Enum):
    """Time integrator (``swarp/dynamics/base.py:97-101``)."""

    EULER = "euler"
    RK4 = "rk4"


def _coerce(enum_cls, val, argname: str):
    """Member of ``enum_cls`` from a member, a name (case/dash-insensitive) or a value."""
    if isinstance(val, enum_cls):
        return val
    if isinstance(val, str):
        key = val.strip().upper().replace("-", "_")
        if key in enum_cls.__members__:
            return enum_cls[key]
        valid = ", ".join(m.name.lower() for m in enum_cls)
        raise ValueError(
            f"unknown {argname} {val!r}; valid names are {valid} (or a {enum_cls.__name__} member)"
        )
    return enum_cls(val)


def action_dim(model) -> int:
    """Action arity of a dynamics model."""
    return MODEL_ACTION_DIM[_coerce(DynamicsModel, model, "model").name]


#: Column layout of the ``[n_agents, NUM_PARAMS]`` parameter table. The kernels read
#: columns by these indices, so the order is an interface: it is the reference's
#: (``swarp/dynamics/base.py:114-145``).
PARAM_FIELDS: tuple[str, ...] = (
    "radius",
    "mass",
    "max_speed",
    "max_accel",
    "max_ang_vel",
    "max_ang_accel",
    "l_f",
    "l_r",
    "max_steer",
    "thrust_max",
    "arm_length",
    "inertia_xx",
    "inertia_yy",
    "inertia_zz",
    "torque_coeff",
    "gravity",
    "min_speed",
    "shape",
    "half_x",
    "half_y",
    "cmd_gain_v",
    "cmd_gain_w",
)
NUM_PARAMS = len(PARAM_FIELDS)
_COL = {name: i for i, name in enumerate(PARAM_FIELDS)}
P_RADIUS = _COL["radius"]
P_MASS = _COL["mass"]
P_MAX_SPEED = _COL["max_speed"]
P_MAX_ACCEL = _COL["max_accel"]
P_MAX_ANG_VEL = _COL["max_ang_vel"]
P_MAX_ANG_ACCEL = _COL["max_ang_accel"]
P_LF = _COL["l_f"]
P_LR = _COL["l_r"]
P_MAX_STEER = _COL["max_steer"]
P_THRUST_MAX = _COL["thrust_max"]
P_ARM = _COL["arm_length"]
P_IXX = _COL["inertia_xx"]
P_IYY = _COL["inertia_yy"]
P_IZZ = _COL["inertia_zz"]
P_KAPPA = _COL["torque_coeff"]
P_GRAVITY = _COL["gravity"]
P_MIN_SPEED = _COL["min_speed"]
P_SHAPE = _COL["shape"]
P_HALF_X = _COL["half_x"]
P_HALF_Y = _COL["half_y"]
P_CMD_GAIN_V = _COL["cmd_gain_v"]
P_CMD_GAIN_W = _COL["cmd_gain_w"]


@dataclass
class AgentConfig:
    """Static per-agent definition (``swarp/dynamics/base.py:172-286``)."""

    model: DynamicsModel | str | int = DynamicsModel.HOLONOMIC
    ctrl_mode: ControlMode | str | int = ControlMode.VELOCITY
    radius: float | None = None
    mass: float = 1.0
    max_speed: float = 1.0
    max_accel: float = 1.0
    max_ang_vel: float = math.pi
    max_ang_accel: float = 2.0 * math.pi
    l_f: float = 0.1
    l_r: float = 0.1
    max_steer: float = math.pi / 4
    min_speed: float | None = None
    thrust_max: float = 10.0
    arm_length: float = 0.15
    inertia_xx: float = 0.01
    inertia_yy: float = 0.01
    inertia_zz: float = 0.02
    torque_coeff: float = 0.02
    gravity: float = 9.81
    shape: AgentShape | str | int = AgentShape.DISC
    half_extents: tuple[float, float] = (0.0, 0.0)
    cmd_gain_v: float = 1.0
    cmd_gain_w: float = 1.0

    def __post_init__(self) -> None:
        self.model = _coerce(DynamicsModel, self.model, "model")
        self.ctrl_mode = _coerce(ControlMode, self.ctrl_mode, "ctrl_mode")
        self.shape = _coerce(AgentShape, self.shape, "shape")
        self.half_extents = tuple(float(h) for h in self.half_extents)
        if len(self.half_extents) != 2:
            raise ValueError("AgentConfig.half_extents must be a pair (hx, hy).")
        if self.shape == AgentShape.BOX:
            hx, hy = self.half_extents
            if hx <= 0.0 or hy <= 0.0:
                raise ValueError("A box agent needs positive half_extents (hx, hy).")
            if self.model == DynamicsModel.DRONE:
                raise ValueError("A drone cannot be a box agent; its footprint is a disc.")
            circ = math.hypot(hx, hy)
            if self.radius is not None and not math.isclose(
                self.radius, circ, rel_tol=1e-9, abs_tol=1e-12
            ):
                raise ValueError(
                    f"A box agent's radius is derived from its half_extents (the "
                    f"circumscribed radius {circ}); got radius={self.radius}. "
                    "Leave radius unset (None)."
                )
            self.radius = circ
        else:
            if self.half_extents != (0.0, 0.0):
                raise ValueError(
                    "AgentConfig.half_extents is only meaningful for shape=AgentShape.BOX; "
                    "a disc's footprint is its radius."
                )
            if self.radius is None:
                self.radius = 0.05
        if self.l_f + self.l_r <= 0.0:
            raise ValueError("Bicycle wheelbase l_f + l_r must be positive.")
        for name in (
            "radius", "mass", "max_speed", "max_accel", "max_ang_vel", "max_ang_accel",
            "cmd_gain_v", "cmd_gain_w",
        ):
            if getattr(self, name) <= 0.0:
                raise ValueError(f"AgentConfig.{name} must be positive.")
        if self.ctrl_mode == ControlMode.SERVO and self.model != DynamicsModel.DIFF_DRIVE:
            raise ValueError(
                f"ControlMode.SERVO is a diff-drive mode; got model {self.model.name}."
            )
        if self.min_speed is not None and not -self.max_speed <= self.min_speed <= self.max_speed:
            raise ValueError("AgentConfig.min_speed must lie in [-max_speed, max_speed].")
        if self.model == DynamicsModel.DRONE:
            for name in ("thrust_max", "arm_length", "inertia_xx", "inertia_yy", "inertia_zz"):
                if getattr(self, name) <= 0.0:
                    raise ValueError(f"AgentConfig.{name} must be positive for a drone.")

    @property
    def half_x(self) -> float:
        return self.half_extents[0]

    @property
    def half_y(self) -> float:
        return self.half_extents[1]

    def to_row(self) -> list[float]:
        """This agent as one parameter row in ``PARAM_FIELDS`` order."""
        row = {name: getattr(self, name) for name in PARAM_FIELDS}
        if row["min_speed"] is None:
            row["min_speed"] = -self.max_speed
        return [float(row[name]) for name in PARAM_FIELDS]


def per_env_float_template(configs: list[AgentConfig], n_envs: int):
    """A ``[n_envs, n_agents, NUM_PARAMS]`` float64 array pre-filled from ``configs``
    (``swarp/dynamics/base.py:369-377``): every env starts as a copy of the shared rows;
    edit columns (e.g. ``[..., P_MASS]``) to randomize, then hand the result to
    ``Stepper.set_agent_params_per_env``."""
    import numpy as np

    rows = np.array([c.to_row() for c in configs], dtype=np.float64)
    return np.broadcast_to(rows, (n_envs, *rows.shape)).copy()


#: Per-slot action limits each model clamps against (``swarp/dynamics/base.py:294-331``).
_ACTION_LIMITS = {
    ("HOLONOMIC", "VELOCITY"): ((None, "max_speed"), (None, "max_speed")),
    ("HOLONOMIC", "ACCELERATION"): ((None, "max_accel"), (None, "max_accel")),
    ("DIFF_DRIVE", "VELOCITY"): ((None, "max_speed"), (None, "max_ang_vel")),
    ("DIFF_DRIVE", "ACCELERATION"): ((None, "max_accel"), (None, "max_ang_accel")),
    ("DIFF_DRIVE", "SERVO"): ((None, "max_speed"), (None, "max_ang_vel")),
    ("KINEMATIC_BICYCLE", "VELOCITY"): ((None, "max_accel"), (None, "max_steer")),
    ("KINEMATIC_BICYCLE", "ACCELERATION"): ((None, "max_accel"), (None, "max_steer")),
    ("DRONE", "VELOCITY"): ((0.0, "thrust_max"),) * 4,
    ("DRONE", "ACCELERATION"): ((0.0, "thrust_max"),) * 4,
}


def action_bounds(cfg: AgentConfig) -> tuple[list[float], list[float]]:
    """``(low, high)`` per action slot, the physical limits the integrator clamps to."""
    key = (DynamicsModel(cfg.model).name, ControlMode(cfg.ctrl_mode).name)
    slots = _ACTION_LIMITS[key]
    high = [getattr(cfg, f) for _, f in slots]
    low = [-h if lo is None else lo for (lo, _), h in zip(slots, high)]
    return low, high


def drone_config(
    *,
    mass: float = 1.0,
    radius: float = 0.15,
    thrust_max: float = 10.0,
    arm_length: float = 0.15,
    inertia_xx: float = 0.01,
    inertia_yy: float = 0.01,
    inertia_zz: float = 0.02,
    torque_coeff: float = 0.02,
    gravity: float = 9.81,
) -> AgentConfig:
    """A "+" quadrotor ``AgentConfig`` (``swarp/dynamics/drone.py:24-53``)."""
    return AgentConfig(
        model=DynamicsModel.DRONE,
        ctrl_mode=ControlMode.ACCELERATION,
        radius=radius,
        mass=mass,
        thrust_max=thrust_max,
        arm_length=arm_length,
        inertia_xx=inertia_xx,
        inertia_yy=inertia_yy,
        inertia_zz=inertia_zz,
        torque_coeff=torque_coeff,
        gravity=gravity,
    )


class ObstacleShape(IntEnum):
    """Obstacle geometry tag (``swarp/core/config.py:13-22``)."""

    CIRCLE = 0
    BOX = 1
    SEGMENT = 2


class ObstacleKind(IntEnum):
    """Whether an obstacle can be pushed (``swarp/core/config.py:25-36``)."""

    IMMOVABLE = 0
    MOVABLE = 1


@dataclass
class Obstacles:
    """One batched obstacle set (``swarp/core/config.py:39-178``).

    ``pos [E, N, 2]`` and ``radius [N]`` are required; every optional field ``None``
    means its documented default (circle, angle 0, half-extents 0, velocity 0,
    immovable, mass/inertia 1, each shape its own body, offset 0).
    """

    pos: torch.Tensor
    radius: torch.Tensor
    shape: torch.Tensor | None = None
    angle: torch.Tensor | None = None
    half_extents: torch.Tensor | None = None
    vel: torch.Tensor | None = None
    ang_vel: torch.Tensor | None = None
    kind: torch.Tensor | None = None
    mass: torch.Tensor | None = None
    inertia: torch.Tensor | None = None
    body: torch.Tensor | None = None
    body_offset: torch.Tensor | None = None
    _resolved_for: tuple | None = field(default=None, init=False, repr=False, compare=False)
    _any_movable: bool | None = field(default=None, init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        if self.pos.dim() != 3 or self.pos.shape[-1] != 2:
            raise ValueError(f"obstacle pos must be [n_envs, n_obstacles, 2]; got {self.pos.shape}")
        n = self.pos.shape[1]
        if self.radius.dim() != 1 or self.radius.shape[0] != n:
            raise ValueError(
                f"obstacle radius must be [n_obstacles={n}]; got {tuple(self.radius.shape)}"
            )
        if self.angle is not None and self.angle.dim() not in (1, 2):
            raise ValueError(
                "obstacle angle must be [n_obstacles] or [n_envs, n_obstacles]; got "
                f"{tuple(self.angle.shape)}"
            )

    @property
    def n_envs(self) -> int:
        return self.pos.shape[0]

    @property
    def n_obstacles(self) -> int:
        return self.pos.shape[1]

    @property
    def any_movable(self) -> bool:
        if self._any_movable is None:
            self._any_movable = self.kind is not None and bool((self.kind != 0).any().item())
        return self._any_movable

    def resolve(self, device, dtype: torch.dtype) -> "Obstacles":
        """This set detached, cast, contiguous and on ``device``; ``angle`` per-env."""
        key = (str(device), dtype)
        if self._resolved_for == key:
            return self

        def f(t):
            return None if t is None else t.detach().to(device=device, dtype=dtype).contiguous()

        def i(t):
            return None if t is None else t.detach().to(device=device, dtype=torch.int32).contiguous()

        angle = f(self.angle)
        if angle is not None and angle.dim() == 1:
            angle = angle.unsqueeze(0).expand(self.n_envs, -1).contiguous()
        out = Obstacles(
            pos=f(self.pos),
            radius=f(self.radius),
            shape=i(self.shape),
            angle=angle,
            half_extents=f(self.half_extents),
            vel=f(self.vel),
            ang_vel=f(self.ang_vel),
            kind=i(self.kind),
            mass=f(self.mass),
            inertia=f(self.inertia),
            body=i(self.body),
            body_offset=f(self.body_offset),
        )
        out._resolved_for = key
        out._any_movable = self._any_movable
        return out


@dataclass
class WorldConfig:
    """Interaction and boundary settings shared by all envs (``swarp/core/config.py:181-322``)."""

    collisions: bool = True
    collision_k: float = 100.0
    collision_c: float = 1.0
    collision_margin: float = 0.02
    obstacle_linear_damping: float = 10.0
    obstacle_angular_damping: float = 10.0
    obstacle_friction: float = 0.0
    gravity: float = 9.81
    wheel_contacts: bool = False
    wheel_lateral_friction: float = 0.2
    wheel_turn_torque: float = 0.0
    obstacle_friction_speed: float = 0.005
    obstacle_friction_grid: int = 6
    contact_max_overlap: float = 0.0
    bounds: tuple[float, float, float, float] | None = None
    bounds_mode: str = "soft"
    neighbor_radius: float | None = None
    max_neighbors: int = 32
    neighbor_method: str = "auto"
    grid_dim: int = 128
    uniform_bins: int | None = None
    integrator: Integrator = Integrator.EULER
    neighbor_reuse: bool = True

    def override_with(self, other: "WorldConfig | None") -> "WorldConfig":
        """This config with ``other``'s non-default fields applied on top."""
        if other is None:
            return self
        default = WorldConfig()
        changed = {
            f.name: getattr(other, f.name)
            for f in fields(self)
            if getattr(other, f.name) != getattr(default, f.name)
        }
        return replace(self, **changed) if changed else self

    def __post_init__(self) -> None:
        if self.bounds_mode not in ("soft", "clamp"):
            raise ValueError('bounds_mode must be "soft" or "clamp"')
        if self.bounds is not None:
            x_min, x_max, y_min, y_max = self.bounds
            if x_min >= x_max or y_min >= y_max:
                raise ValueError("bounds must satisfy x_min < x_max and y_min < y_max")
        if self.collision_k < 0.0 or self.collision_c < 0.0 or self.collision_margin < 0.0:
            raise ValueError("collision constants must be non-negative")
        if self.obstacle_friction < 0.0 or self.obstacle_friction_speed <= 0.0:
            raise ValueError("obstacle_friction must be >= 0 and obstacle_friction_speed > 0")
        if self.wheel_lateral_friction < 0.0 or self.wheel_turn_torque < 0.0:
            raise ValueError("wheel_lateral_friction and wheel_turn_torque must be >= 0")
        if self.obstacle_friction_grid < 1:
            raise ValueError("obstacle_friction_grid must be >= 1")
        if self.obstacle_linear_damping < 0.0 or self.obstacle_angular_damping < 0.0:
            raise ValueError("obstacle damping must be non-negative")
        if self.contact_max_overlap < 0.0:
            raise ValueError("contact_max_overlap must be non-negative (0 disables)")
        if self.neighbor_method not in ("auto", "grid", "brute", "uniform_grid"):
            raise ValueError('neighbor_method must be "auto", "grid", "brute", or "uniform_grid"')
