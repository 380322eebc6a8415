"""Feature-profile kernel instances vs the general instances.

The generic, drone and body kernels are compiled once with every optional path (RK4,
saturated contacts, obstacles, walls, clamp, control modes, every dynamics model) and,
for float32, once per profile with only the paths of a common kind of world: 2-D fleets
with obstacles and walls under Euler, drone fleets, holonomic fleets pushing movable
bodies.  The host picks a profile instance when the descriptor's features fit it
(Stepper.use_profiles, on by default).  A profile instance folds the absent paths away at
compile time and changes no operation of the paths it keeps, so its results must be
BIT-IDENTICAL to the general instance's -- states and gradients alike.  (The parity tests
compare the default, profile-routed path with the oracle.)
"""

import numpy as np
import pytest
import torch

from cases import nav_agents
from hip_helpers import hip_run, make_stepper, state_to16, to_torch_state
from oracle.oracle import pack_state
from swarp_amd import rollout
from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, Integrator, WorldConfig

pytestmark = pytest.mark.gpu


def _both(cfgs, world, dt, S, s0, acts, w, obs=None):
    out = []
    for prof in (True, False):
        st = make_stepper(cfgs, world, dt, S, torch.float32, obs=obs, n_envs=s0.shape[0])
        st.use_profiles = prof
        d = st.desc(s0.shape[0], acts.shape[-1])
        assert (d.fleet_models != 0) == prof
        out.append(hip_run(st, s0, acts, w, np.float32))
    return out


def _same(name, a, b):
    for lab, x, y in zip(("states", "d/d state0", "d/d actions"), a, b):
        assert np.array_equal(x, y), f"{name}: {lab} differ between the profile and general instances"


def test_profile_2d_fleet_obstacles_walls():
    """Diff-drive + bicycle agents, circle / box / segment obstacles, soft walls, Euler."""
    E, A, T, S = 96, 32, 8, 4
    rng = np.random.default_rng(31)
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(A // 2)] + [
        AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, radius=0.05) for _ in range(A // 2)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0), max_neighbors=32)
    n = 8
    obs = {"pos": rng.uniform(-1, 1, size=(E, n, 2)),
           "radius": np.r_[rng.uniform(0.05, 0.2, 4), np.zeros(2), np.full(2, 0.05)],
           "type": np.r_[np.zeros(4), np.ones(2), np.full(2, 2)].astype(np.int32),
           "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
           "half": np.r_[np.zeros((4, 2)), rng.uniform(0.05, 0.3, size=(2, 2)),
                         np.c_[rng.uniform(0.1, 0.4, 2), np.zeros(2)]]}
    s0 = pack_state({"pos": rng.uniform(-1, 1, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16)) * 0.1
    w[..., 7:] = 0.0
    a, b = _both(cfgs, world, 0.05, S, s0, acts, w, obs=obs)
    _same("2d", a, b)


def test_profile_2d_fleet_single_model():
    """A diff-drive-only fleet (the profile pins the model tag) without obstacles."""
    E, A, T, S = 64, 16, 6, 2
    rng = np.random.default_rng(32)
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-0.6, 0.6, -0.6, 0.6), max_neighbors=8)
    s0 = pack_state({"pos": rng.uniform(-0.6, 0.6, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16))
    w[..., 7:] = 0.0
    a, b = _both(cfgs, world, 0.05, S, s0, acts, w)
    _same("diff-only", a, b)


@pytest.mark.parametrize("walls,mode", [(False, ControlMode.VELOCITY),
                                        (True, ControlMode.ACCELERATION)])
def test_profile_drones(walls, mode):
    """Quadrotor fleets, with and without soft walls (a drone reads its rotor thrusts the
    same way in every control mode, so the drone profile takes any mode)."""
    E, A, T, S = 64, 8, 12, 2
    rng = np.random.default_rng(33)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0, ctrl_mode=mode)
            for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.6, 0.6, -0.6, 0.6) if walls else None)
    ax = rng.normal(size=(E, A, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(E, A, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)), "z": np.ones((E, A)),
                     "attitude": q}).astype(np.float32)
    acts = (rng.uniform(0, 1, size=(T, E, A, 4)) * 10.0).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16)) * 0.01
    a, b = _both(cfgs, world, 0.02, S, s0, acts, w)
    _same("drones", a, b)


def test_profile_general_features_fall_back():
    """A fleet no profile covers (servo control, RK4) runs the general instances either way."""
    E, A, T, S = 32, 8, 5, 2
    rng = np.random.default_rng(34)
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.SERVO, radius=0.05)
            for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-0.5, 0.5, -0.5, 0.5), max_neighbors=8,
                        integrator=Integrator.RK4)
    s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16))
    w[..., 7:] = 0.0
    a, b = _both(cfgs, world, 0.05, S, s0, acts, w)
    _same("servo-rk4", a, b)


def _body_run(prof, E, A, seed):
    rng = np.random.default_rng(seed)
    d, r, m = 0.2, 0.1, 1.0
    offs = [[0, 0], [d, 0], [-d, 0], [0, d], [0, -d]]
    inertia = sum(0.5 * (m / 5) * r * r + (m / 5) * (o[0] ** 2 + o[1] ** 2) for o in offs)
    obs = {"pos": np.broadcast_to(np.asarray(offs, np.float64), (E, 5, 2)).copy(),
           "radius": np.full(5, r), "kind": np.ones(5, np.int32), "body": np.zeros(5, np.int32),
           "body_off": np.asarray(offs, np.float64), "mass": np.full(5, m),
           "inertia": np.full(5, inertia)}
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0), max_neighbors=16, neighbor_radius=0.3)
    st = make_stepper(nav_agents(A), world, 0.05, 4, torch.float32, obs=obs, n_envs=E)
    st.use_profiles = prof
    pos = rng.uniform(-0.8, 0.8, size=(E, A, 2))
    acts = rng.uniform(-1, 1, size=(6, E, A, 2))
    acts[..., : A // 2, :] = -pos[None, :, : A // 2] / np.linalg.norm(
        pos[None, :, : A // 2], axis=-1, keepdims=True)
    ob0 = st.ob_state.detach().clone().requires_grad_(True)
    st.ob_state = ob0
    s0 = to_torch_state(pack_state({"pos": pos}).astype(np.float32), torch.float32, True, 5)
    a = torch.tensor(acts, dtype=torch.float32, device="cuda", requires_grad=True)
    final, traj = rollout(st, s0, a)
    wob = torch.tensor(rng.normal(size=tuple(st.ob_trajectory.shape)), dtype=torch.float32,
                       device="cuda")
    loss = (wob * st.ob_trajectory).sum() + sum((x.pos * (t + 1)).sum() for t, x in enumerate(traj))
    loss.backward()
    return (np.stack([state_to16(x) for x in traj]), st.ob_trajectory.detach().cpu().numpy(),
            s0.pos.grad.cpu().numpy(), ob0.grad.cpu().numpy(), a.grad.cpu().numpy())


def test_profile_bodies():
    """Holonomic agents pushing a movable cross inside soft walls (config 5's kind)."""
    E, A = 12, 64
    a, b = _body_run(True, E, A, 35), _body_run(False, E, A, 35)
    for lab, x, y in zip(("states", "obstacle states", "d/d pos0", "d/d ob0", "d/d actions"), a, b):
        assert np.array_equal(x, y), f"bodies: {lab} differ between the profile and general instances"
