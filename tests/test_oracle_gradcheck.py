"""Pins of the oracle's hand-written adjoint against central finite differences (fp64).

For a random cotangent on every step output, the oracle's d(loss)/d(state0) and
d(loss)/d(actions) must equal the finite-difference derivative of the oracle's own
forward, coordinate by coordinate.  The cases mirror the reference's gradcheck suite
(tests/unit/test_gradients.py:50-171, test_collisions.py:151-178, test_drone.py:206-234,
test_geometry.py:250-274) plus truncated neighbour lists, moving obstacles, the
saturated-overlap contact law and the position clamp.
"""

import numpy as np
import pytest

from cases import holo, obstacles_np, oracle_cfg, params_of
from oracle.oracle import Oracle, pack_state
from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, ObstacleShape, WorldConfig

O = Oracle(np.float64)
BIG = 100.0


def _fd_check(configs, world, dt, substeps, s0, acts, obs=None, fields=None, eps=1e-6, tol=2e-7,
              seed=0):
    E = s0.shape[0]
    cfg = oracle_cfg(configs, world, dt, substeps, E, acts.shape[-1])
    p, t, m = params_of(configs)
    ob = obstacles_np(obs, E)
    rng = np.random.default_rng(seed)
    T = acts.shape[0]
    w_traj = rng.normal(size=(T,) + s0.shape)
    # only fields the models actually integrate carry weight; all 16 are differentiated
    def loss(s0_, acts_):
        tr = O.rollout(cfg, p, t, m, ob, s0_, acts_)
        return float((w_traj * tr).sum())

    tr = O.rollout(cfg, p, t, m, ob, s0, acts)
    g0, ga = O.rollout_adj(cfg, p, t, m, ob, s0, acts, tr, w_traj, None)
    idx0 = list(np.ndindex(*s0.shape)) if fields is None else [
        i for i in np.ndindex(*s0.shape) if i[-1] in fields]
    for i in idx0:
        a, b = s0.copy(), s0.copy()
        a[i] += eps
        b[i] -= eps
        fd = (loss(a, acts) - loss(b, acts)) / (2 * eps)
        assert abs(fd - g0[i]) <= tol * max(1.0, abs(fd)), f"state0{i}: fd {fd} vs adj {g0[i]}"
    for i in np.ndindex(*acts.shape):
        a, b = acts.copy(), acts.copy()
        a[i] += eps
        b[i] -= eps
        fd = (loss(s0, a) - loss(s0, b)) / (2 * eps)
        assert abs(fd - ga[i]) <= tol * max(1.0, abs(fd)), f"actions{i}: fd {fd} vs adj {ga[i]}"


def _rand_state(E, A, seed, scale=0.5):
    rng = np.random.default_rng(seed)
    s = pack_state({
        "pos": rng.normal(size=(E, A, 2)) * scale,
        "theta": rng.normal(size=(E, A)) * scale,
        "vel": rng.normal(size=(E, A, 2)) * scale,
        "speed": rng.normal(size=(E, A)) * scale,
        "ang_vel": rng.normal(size=(E, A)) * scale,
    })
    return s


MODEL_CASES = [
    ("holonomic-vel", DynamicsModel.HOLONOMIC, ControlMode.VELOCITY),
    ("holonomic-acc", DynamicsModel.HOLONOMIC, ControlMode.ACCELERATION),
    ("diffdrive-vel", DynamicsModel.DIFF_DRIVE, ControlMode.VELOCITY),
    ("diffdrive-acc", DynamicsModel.DIFF_DRIVE, ControlMode.ACCELERATION),
    ("bicycle", DynamicsModel.KINEMATIC_BICYCLE, ControlMode.ACCELERATION),
]


def _cfgs(model, mode, n=2):
    return [AgentConfig(model=model, ctrl_mode=mode, max_speed=BIG, max_accel=BIG, max_ang_vel=BIG,
                        max_ang_accel=BIG, max_steer=1.0, l_f=0.16, l_r=0.14) for _ in range(n)]


@pytest.mark.parametrize("name,model,mode", MODEL_CASES, ids=[c[0] for c in MODEL_CASES])
def test_single_step(name, model, mode):
    rng = np.random.default_rng(1)
    _fd_check(_cfgs(model, mode), WorldConfig(collisions=False), 0.1, 1, _rand_state(2, 2, 1),
              0.3 * rng.normal(size=(1, 2, 2, 2)))


def test_substeps_diffdrive():
    rng = np.random.default_rng(2)
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=BIG, max_ang_vel=BIG)]
    _fd_check(cfgs, WorldConfig(collisions=False), 0.1, 4, _rand_state(1, 1, 2),
              0.3 * rng.normal(size=(1, 1, 1, 2)))


def test_multistep_rollout_mixed():
    rng = np.random.default_rng(3)
    cfgs = [
        AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, max_speed=BIG, max_accel=BIG,
                    max_steer=1.0, l_f=0.16, l_r=0.14),
        AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=BIG, max_ang_vel=BIG),
    ]
    _fd_check(cfgs, WorldConfig(collisions=False), 0.1, 1, _rand_state(1, 2, 3),
              0.3 * rng.normal(size=(5, 1, 2, 2)))


def test_collisions_walls_substeps():
    world = WorldConfig(collision_k=10.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-1.0, 1.0, -1.0, 1.0), bounds_mode="soft")
    s0 = pack_state({"pos": [[[0.0, 0.0], [0.18, 0.02]]], "vel": [[[0.1, 0.0], [-0.1, 0.05]]]})
    rng = np.random.default_rng(0)
    _fd_check(holo(2, mode=ControlMode.ACCELERATION), world, 0.1, 2, s0,
              0.1 * rng.normal(size=(1, 1, 2, 2)))


def test_collisions_wall_contact_and_tanh_saturation():
    world = WorldConfig(collision_k=30.0, collision_c=0.7, collision_margin=0.02,
                        contact_max_overlap=0.05, bounds=(-0.3, 0.3, -0.3, 0.3), bounds_mode="soft")
    s0 = pack_state({"pos": [[[0.21, 0.0], [0.05, 0.03], [0.02, -0.12]]],
                     "vel": [[[0.2, 0.1], [-0.1, 0.05], [0.0, -0.3]]]})
    rng = np.random.default_rng(9)
    _fd_check(holo(3, radius=0.08, mode=ControlMode.ACCELERATION), world, 0.05, 3, s0,
              0.2 * rng.normal(size=(2, 1, 3, 2)))


def test_truncated_lists_asymmetric():
    # 5 agents within radius of each other, K = 2: lists are truncated and asymmetric
    world = WorldConfig(collision_k=20.0, collision_c=0.5, collision_margin=0.05, max_neighbors=2,
                        neighbor_radius=0.5)
    rng = np.random.default_rng(11)
    pos = np.stack([np.linspace(0.0, 0.2, 5), 0.03 * rng.normal(size=5)], -1)[None]
    s0 = pack_state({"pos": pos, "vel": 0.1 * rng.normal(size=(1, 5, 2))})
    _fd_check(holo(5, radius=0.06, mode=ControlMode.ACCELERATION), world, 0.05, 2, s0,
              0.2 * rng.normal(size=(2, 1, 5, 2)))


def test_box_and_segment_obstacles():
    # tests/unit/test_geometry.py:250-274 (exterior contact, away from the corner kink)
    world = WorldConfig(collision_k=10.0, collision_c=1.0, collision_margin=0.02)
    obs = {"pos": [[[0.22, 0.0], [0.0, -0.2]]], "radius": [0.0, 0.05],
           "type": [int(ObstacleShape.BOX), int(ObstacleShape.SEGMENT)], "angle": [0.0, 0.0],
           "half": [[0.1, 0.1], [0.2, 0.0]]}
    s0 = pack_state({"pos": [[[0.05, -0.05]]]})
    rng = np.random.default_rng(0)
    _fd_check(holo(1, 0.1), world, 0.1, 2, s0, 0.05 * rng.normal(size=(1, 1, 1, 2)), obs=obs)


def test_moving_rotated_obstacles():
    world = WorldConfig(collision_k=15.0, collision_c=0.8, collision_margin=0.02)
    obs = {"pos": [[[0.2, 0.05], [-0.1, -0.22], [0.0, 0.25]]], "radius": [0.0, 0.04, 0.1],
           "type": [1, 2, 0], "angle": [[0.4, -0.7, 0.0]], "half": [[0.08, 0.05], [0.15, 0.0], [0.0, 0.0]],
           "vel": [[[0.1, -0.05], [0.0, 0.2], [-0.1, 0.0]]], "ang_vel": [[0.5, -1.0, 0.3]]}
    s0 = pack_state({"pos": [[[0.06, 0.03], [-0.08, -0.12], [0.02, 0.13]]],
                     "vel": [[[0.1, 0.0], [0.0, -0.1], [0.05, 0.05]]]})
    rng = np.random.default_rng(5)
    _fd_check(holo(3, 0.06, mode=ControlMode.ACCELERATION), world, 0.1, 2, s0,
              0.1 * rng.normal(size=(2, 1, 3, 2)), obs=obs)


def test_drone():
    # tests/unit/test_drone.py:206-234
    cfg = AgentConfig(model=DynamicsModel.DRONE, thrust_max=20.0)
    rng = np.random.default_rng(7)
    q = np.array([0.05, -0.03, 0.02, 1.0])
    q /= np.linalg.norm(q)
    s0 = pack_state({"pos": [[[0.0, 0.0]]], "vel": 0.05 * rng.normal(size=(1, 1, 2)),
                     "z": [[1.0]], "vz": [[0.1]], "attitude": q.reshape(1, 1, 4),
                     "body_rates": 0.02 * rng.normal(size=(1, 1, 3))})
    hover = 9.81 / 4.0
    _fd_check([cfg], WorldConfig(collisions=False), 0.02, 1, s0,
              hover + 0.1 * rng.normal(size=(3, 1, 1, 4)))


def test_drones_with_contacts():
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=20.0) for _ in range(2)]
    world = WorldConfig(collision_k=20.0, collision_c=0.5, collision_margin=0.02)
    rng = np.random.default_rng(8)
    s0 = pack_state({"pos": [[[0.0, 0.0], [0.15, 0.05]]], "vel": 0.05 * rng.normal(size=(1, 2, 2)),
                     "z": [[1.0, 1.1]], "attitude": np.tile([0.0, 0.0, 0.0, 1.0], (1, 2, 1)),
                     "body_rates": 0.02 * rng.normal(size=(1, 2, 3))})
    _fd_check(cfgs, world, 0.02, 2, s0, 9.81 / 4 + 0.1 * rng.normal(size=(2, 1, 2, 4)))


def test_clamp_bounds_interior():
    world = WorldConfig(collisions=False, bounds=(-0.5, 0.5, -0.5, 0.5), bounds_mode="clamp")
    rng = np.random.default_rng(12)
    s0 = pack_state({"pos": [[[0.44, 0.0], [0.0, -0.1]]]})
    # first agent is pushed into the clamp (zero position gradient), the second is free
    _fd_check(holo(2, 0.05), world, 0.1, 1, s0, np.array([[[[1.0, 0.1], [0.2, -0.3]]]]) +
              0.01 * rng.normal(size=(1, 1, 2, 2)))


def test_nav_c1_shape():
    """Config 1 shape (holonomic, soft contacts + walls) at a reduced size."""
    from cases import nav_agents, nav_world

    E, A, T = 2, 4, 3
    rng = np.random.default_rng(0)
    pos = rng.uniform(-0.15, 0.15, size=(E, A, 2))  # crowded -> contacts
    s0 = pack_state({"pos": pos})
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    _fd_check(nav_agents(A), nav_world(A), 0.05, 1, s0, acts, fields=(0, 1, 3, 4))
