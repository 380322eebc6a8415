"""Shared builders: one world description -> the HIP Stepper and the oracle's inputs.

A case is (agent configs, WorldConfig, dt, substeps, obstacles).  ``oracle_inputs``
derives the oracle's configuration from the same description with the reference's
rules (neighbour radius = max(user, reach), sub_dt = dt / substeps, soft walls vs clamp).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, WorldConfig

FIELDS = ("pos", "theta", "vel", "speed", "ang_vel", "z", "vz", "attitude", "body_rates")


def oracle_cfg(configs, world: WorldConfig, dt, substeps, n_envs, act_dim, n_threads=1):
    collisions = world.collisions
    max_r = max(c.radius for c in configs)
    reach = 2.0 * max_r + world.collision_margin
    nbr = (world.neighbor_radius or reach) if collisions else 0.0
    b = world.bounds
    # list order: NeighborGrid's method choice (swarp/core/neighbors.py:387-393) and the
    # frame a world rectangle pins (:476-490), in float64
    method = world.neighbor_method
    if method == "auto":
        method = "uniform_grid" if len(configs) > 512 else "brute"
    grid = {}
    if method == "uniform_grid" and b is not None:
        bins = world.uniform_bins or max(4, min(128, int(math.ceil(math.sqrt(len(configs))))))
        extent = max(b[1] - b[0], b[3] - b[2])
        grid = dict(grid_bins=bins, grid_ox=b[0], grid_oy=b[2], grid_cell=max(nbr, extent / bins))
    return dict(
        **grid,
        n_envs=n_envs,
        n_agents=len(configs),
        act_dim=act_dim,
        substeps=substeps,
        max_neighbors=world.max_neighbors,
        collisions=int(collisions),
        soft_walls=int(b is not None and world.bounds_mode == "soft"),
        # 2: the footprint clamp a world holding box agents uses (kernels.py:74-99)
        clamp_bounds=(0 if b is None or world.bounds_mode != "clamp" else
                      2 if any(int(c.shape) == 1 for c in configs) else 1),
        n_threads=n_threads,
        dt=dt,
        k=world.collision_k,
        c=world.collision_c,
        margin=world.collision_margin,
        max_overlap=world.contact_max_overlap,
        neighbor_radius=nbr,
        bmin_x=b[0] if b else 0.0,
        bmax_x=b[1] if b else 0.0,
        bmin_y=b[2] if b else 0.0,
        bmax_y=b[3] if b else 0.0,
        lin_damping=world.obstacle_linear_damping,
        ang_damping=world.obstacle_angular_damping,
        rk4=int(world.integrator.value == "rk4"),
        wheel=int(world.wheel_contacts),
        lat_grip=world.wheel_lateral_friction * world.gravity,
        turn_cap=world.wheel_turn_torque,
    )


def params_of(configs):
    rows = np.array([c.to_row() for c in configs], dtype=np.float64)
    tags = np.array([int(c.model) for c in configs], dtype=np.int32)
    modes = np.array([int(c.ctrl_mode) for c in configs], dtype=np.int32)
    return rows, tags, modes


def obstacles_np(obs: dict | None, n_envs: int):
    """Obstacle dict with every field filled (numpy, float64)."""
    if obs is None:
        return None
    pos = np.asarray(obs["pos"], dtype=np.float64)
    n = pos.shape[1]
    out = {
        "pos": pos,
        "radius": np.asarray(obs["radius"], dtype=np.float64),
        "type": np.asarray(obs.get("type", np.zeros(n)), dtype=np.int32),
        "half": np.asarray(obs.get("half", np.zeros((n, 2))), dtype=np.float64),
        "vel": np.asarray(obs.get("vel", np.zeros((n_envs, n, 2))), dtype=np.float64),
        "ang_vel": np.asarray(obs.get("ang_vel", np.zeros((n_envs, n))), dtype=np.float64),
    }
    ang = np.asarray(obs.get("angle", np.zeros(n)), dtype=np.float64)
    if ang.ndim == 1:
        ang = np.broadcast_to(ang, (n_envs, n)).copy()
    out["angle"] = ang
    if obs.get("kind") is not None:
        out["kind"] = np.asarray(obs["kind"], dtype=np.int32)
        out["body"] = np.asarray(obs.get("body", np.arange(n)), dtype=np.int32)
        out["mass"] = np.asarray(obs.get("mass", np.ones(n)), dtype=np.float64)
        out["inertia"] = np.asarray(obs.get("inertia", np.ones(n)), dtype=np.float64)
        out["body_off"] = np.asarray(obs.get("body_off", np.zeros((n, 2))), dtype=np.float64)
    return out


def body_seed_np(ob: dict) -> np.ndarray:
    """Initial obstacle state [E, 12 N] of a filled obstacle dict: each shape's installed
    pose and velocity, then per index the body state of its root, derived as
    Stepper._body_seed does (swarp/core/stepper.py:434-476): origin = root pos - R(root
    angle) root offset, heading / velocity / spin = the root's."""
    pos, ang, vel, om = ob["pos"], ob["angle"], ob["vel"], ob["ang_vel"]
    E, n = pos.shape[:2]
    out = np.zeros((E, 12 * n))
    sh = out[:, :6 * n].reshape(E, n, 6)
    sh[..., 0:2] = pos
    sh[..., 2] = ang
    sh[..., 3:5] = vel
    sh[..., 5] = om
    body = ob.get("body", np.arange(n))
    off = ob.get("body_off", np.zeros((n, 2)))
    bd = out[:, 6 * n:].reshape(E, n, 6)
    for o in range(n):
        r = int(body[o])
        ca, sa = np.cos(ang[:, r]), np.sin(ang[:, r])
        wx = ca * off[r, 0] - sa * off[r, 1]
        wy = sa * off[r, 0] + ca * off[r, 1]
        bd[:, o, 0] = pos[:, r, 0] - wx
        bd[:, o, 1] = pos[:, r, 1] - wy
        bd[:, o, 2] = ang[:, r]
        bd[:, o, 3:5] = vel[:, r]
        bd[:, o, 5] = om[:, r]
    return out


def holo(n, radius=0.1, mode=ControlMode.VELOCITY, big=100.0):
    return [
        AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=mode, radius=radius,
                    max_speed=big, max_accel=big)
        for _ in range(n)
    ]


def nav_world(n_agents, agent_radius=0.05, world_size=1.0, **kw):
    """NavigationScenario.make_world's WorldConfig (swarp/scenarios/navigation.py:127-141)."""
    margin = 0.5 * agent_radius
    reach = 2.0 * agent_radius + margin
    return WorldConfig(
        collisions=True,
        collision_k=100.0,
        collision_c=1.0,
        collision_margin=margin,
        bounds=(-world_size, world_size, -world_size, world_size),
        bounds_mode="soft",
        neighbor_radius=max(kw.pop("neighbor_radius", None) or 0.0, reach),
        max_neighbors=min(32, max(4, n_agents)),
        **kw,
    )


def nav_agents(n_agents, agent_radius=0.05, max_speed=1.0, model=DynamicsModel.HOLONOMIC,
               mode=ControlMode.VELOCITY):
    """NavigationScenario._agent_configs (swarp/scenarios/navigation.py:107-125)."""
    return [
        AgentConfig(model=model, ctrl_mode=mode, radius=agent_radius, max_speed=max_speed,
                    max_accel=2.0 * max_speed)
        for _ in range(n_agents)
    ]


def nav_inputs(n_envs, n_agents, T, extent=1.0, seed=0, dtype=torch.float32):
    """Config-1/2 synthetic inputs: fixed draw order pos, goals, actions from a CPU
    generator; zero velocity / heading."""
    g = torch.Generator("cpu").manual_seed(seed)
    pos = (torch.rand(n_envs, n_agents, 2, generator=g, dtype=torch.float64) * 2 - 1) * extent
    goals = (torch.rand(n_envs, n_agents, 2, generator=g, dtype=torch.float64) * 2 - 1) * extent
    acts = torch.rand(T, n_envs, n_agents, 2, generator=g, dtype=torch.float64) * 2 - 1
    return pos.to(dtype), goals.to(dtype), acts.to(dtype)


def state_dict_np(pos, **fields):
    """Numpy state dict with zeros for missing 2-D fields."""
    pos = np.asarray(pos)
    E, A = pos.shape[:2]
    d = {"pos": pos}
    for name in ("theta", "speed", "ang_vel"):
        d[name] = np.asarray(fields.get(name, np.zeros((E, A))))
    d["vel"] = np.asarray(fields.get("vel", np.zeros((E, A, 2))))
    for name in ("z", "vz", "attitude", "body_rates"):
        if name in fields:
            d[name] = np.asarray(fields[name])
    return d


def rel_err(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = max(np.abs(b).max(), 1e-30)
    return float(np.abs(a - b).max() / den)


def deg(x):
    return x * math.pi / 180.0
