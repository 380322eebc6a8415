"""Pins of the CPU oracle against closed-form answers.

Each case restates a known-answer test of the reference suite (file:line cited) and
checks the oracle, in float64, against the hand-computed value: no oracle formula is
re-typed here, only the physics answer.  These pin the contact law, the obstacle
geometry, the walls, the clamp, the integrators and the BPTT chain rule.
"""

import math

import numpy as np
import pytest

from cases import holo, obstacles_np, oracle_cfg, params_of, state_dict_np
from oracle.oracle import Oracle, pack_state, unpack_state
from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, ObstacleShape, WorldConfig

O64 = Oracle(np.float64)


def step(configs, world, dt, state, actions, substeps=1, obs=None, T_actions=None):
    E = np.asarray(state["pos"]).shape[0]
    acts = np.asarray(actions, dtype=np.float64)
    if acts.ndim == 3:
        acts = acts[None]
    cfg = oracle_cfg(configs, world, dt, substeps, E, acts.shape[-1])
    p, t, m = params_of(configs)
    out = O64.rollout(cfg, p, t, m, obstacles_np(obs, E), pack_state(state), acts)
    return unpack_state(out[-1]), out


def test_two_agent_spring_analytic():
    # tests/unit/test_collisions.py:23-37: overlap 0.07, |F| = 7, v = F*dt
    world = WorldConfig(collision_k=100.0, collision_c=0.0, collision_margin=0.02)
    st = state_dict_np([[[0.0, 0.0], [0.15, 0.0]]])
    out, _ = step(holo(2), world, 0.1, st, np.zeros((1, 2, 2)))
    np.testing.assert_allclose(out["pos"][0, 0], [-0.07, 0.0], atol=1e-12)
    np.testing.assert_allclose(out["pos"][0, 1], [0.22, 0.0], atol=1e-12)
    np.testing.assert_allclose(out["vel"][0, 0], [-0.7, 0.0], atol=1e-12)


def test_two_agent_spring_damper_analytic():
    # tests/unit/test_collisions.py:40-63: coefficient (k*0.07 + c) / (1 + c*dt/m) = 7.5
    world = WorldConfig(collision_k=100.0, collision_c=2.0, collision_margin=0.02)
    st = state_dict_np([[[0.0, 0.0], [0.15, 0.0]]], vel=[[[0.5, 0.0], [-0.5, 0.0]]])
    out, _ = step(holo(2, mode=ControlMode.ACCELERATION), world, 0.1, st, np.zeros((1, 2, 2)))
    np.testing.assert_allclose(out["vel"][0, 0], [-0.25, 0.0], atol=1e-12)
    np.testing.assert_allclose(out["pos"][0, 0], [-0.025, 0.0], atol=1e-12)
    np.testing.assert_allclose(out["vel"][0, 1], [0.25, 0.0], atol=1e-12)


def test_momentum_symmetry():
    # tests/unit/test_collisions.py:66-89: equal agents, centre of mass is conserved
    world = WorldConfig(collision_k=50.0, collision_c=0.5, collision_margin=0.05)
    rng = np.random.default_rng(0)
    pos0 = rng.random((1, 4, 2)) * 0.2
    st = state_dict_np(pos0)
    _, traj = step(holo(4, mode=ControlMode.ACCELERATION), world, 0.05, st,
                   np.zeros((20, 1, 4, 2)), substeps=2)
    fin = unpack_state(traj[-1])
    np.testing.assert_allclose(fin["pos"].mean(axis=1), pos0.mean(axis=1), atol=1e-10, rtol=0)
    assert np.linalg.norm(fin["pos"][0, 0] - fin["pos"][0, 1]) > np.linalg.norm(pos0[0, 0] - pos0[0, 1])


def test_obstacle_repulsion_analytic():
    # tests/unit/test_collisions.py:92-108: dist 0.2, min_dist 0.27, overlap 0.07
    world = WorldConfig(collision_k=100.0, collision_c=0.0, collision_margin=0.02)
    obs = {"pos": [[[0.3, 0.0]]], "radius": [0.15]}
    out, _ = step(holo(1), world, 0.1, state_dict_np([[[0.1, 0.0]]]), np.zeros((1, 1, 2)), obs=obs)
    np.testing.assert_allclose(out["pos"][0, 0], [0.1 - 0.07, 0.0], atol=1e-12)


def test_soft_wall_analytic():
    # tests/unit/test_collisions.py:111-126: overlap 0.02 against x = 1 -> F = (-2, 0)
    world = WorldConfig(collision_k=100.0, collision_c=0.0, collision_margin=0.02,
                        bounds=(-1.0, 1.0, -1.0, 1.0), bounds_mode="soft")
    out, _ = step(holo(1, radius=0.05), world, 0.1, state_dict_np([[[0.95, 0.0]]]), np.zeros((1, 1, 2)))
    np.testing.assert_allclose(out["pos"][0, 0], [0.95 - 0.02, 0.0], atol=1e-12)


def test_clamp_bounds():
    # tests/unit/test_collisions.py:129-138
    world = WorldConfig(bounds=(-1.0, 1.0, -1.0, 1.0), bounds_mode="clamp")
    out, _ = step(holo(1, radius=0.05), world, 0.1, state_dict_np([[[0.98, 0.0]]]),
                  [[[5.0, 0.0]]])
    np.testing.assert_allclose(out["pos"][0, 0], [1.0 - 0.05, 0.0], atol=1e-12)


# ---------------------------------------------------- obstacle geometry (test_geometry.py)

K, DT = 100.0, 0.1


def _geom_step(shape, center, p, radius=0.0, angle=0.0, half=(0.0, 0.0), agent_radius=0.1):
    world = WorldConfig(collision_k=K, collision_c=0.0, collision_margin=0.02)
    obs = {"pos": [[center]], "radius": [radius], "type": [int(shape)], "angle": [angle],
           "half": [half]}
    out, _ = step(holo(1, agent_radius), world, DT, state_dict_np([[p]]), np.zeros((1, 1, 2)), obs=obs)
    return out["pos"][0, 0]


def _box_expect(p, center, angle, half, reach):
    # independent signed-distance field of a box (tests/unit/test_geometry.py:77-101)
    ca, sa = math.cos(angle), math.sin(angle)
    d = np.asarray(p) - np.asarray(center)
    lx, ly = ca * d[0] + sa * d[1], -sa * d[0] + ca * d[1]
    q = np.array([abs(lx), abs(ly)]) - np.asarray(half)
    cl = np.clip([lx, ly], [-half[0], -half[1]], [half[0], half[1]])
    o = np.array([lx, ly]) - cl
    od = math.hypot(*o)
    if od > 1e-5:
        s, nl = od, o / od
    elif q[0] > q[1]:
        s, nl = q[0], np.array([1.0 if lx >= 0 else -1.0, 0.0])
    else:
        s, nl = q[1], np.array([0.0, 1.0 if ly >= 0 else -1.0])
    n = np.array([ca * nl[0] - sa * nl[1], sa * nl[0] + ca * nl[1]])
    return np.asarray(p) + n * (K * (reach - s)) * DT * DT


def test_box_face_analytic():
    got = _geom_step(ObstacleShape.BOX, [0.3, 0.0], [0.1, 0.0], half=(0.1, 0.2))
    np.testing.assert_allclose(got, [0.08, 0.0], atol=1e-12)


def test_box_corner_analytic():
    p = [0.16, 0.16]
    got = _geom_step(ObstacleShape.BOX, [0.0, 0.0], p, half=(0.1, 0.1))
    np.testing.assert_allclose(got, _box_expect(p, [0.0, 0.0], 0.0, (0.1, 0.1), 0.12), atol=1e-12)


def test_box_rotated_analytic():
    p, ang = [0.18, 0.02], math.pi / 4
    got = _geom_step(ObstacleShape.BOX, [0.0, 0.0], p, angle=ang, half=(0.1, 0.1))
    np.testing.assert_allclose(got, _box_expect(p, [0.0, 0.0], ang, (0.1, 0.1), 0.12), atol=1e-12)


def test_box_interior_pushout():
    got = _geom_step(ObstacleShape.BOX, [0.0, 0.0], [0.03, 0.0], half=(0.1, 0.1))
    assert got[0] > 0.12 and abs(got[1]) < 1e-9


def test_segment_midspan_analytic():
    got = _geom_step(ObstacleShape.SEGMENT, [0.0, 0.0], [0.0, 0.1], radius=0.05, half=(0.2, 0.0),
                     agent_radius=0.05)
    np.testing.assert_allclose(got, [0.0, 0.12], atol=1e-12)


def test_segment_endpoint_analytic():
    p = np.array([0.3, 0.05])
    got = _geom_step(ObstacleShape.SEGMENT, [0.0, 0.0], p.tolist(), radius=0.05, half=(0.2, 0.0),
                     agent_radius=0.05)
    d = p - np.array([0.2, 0.0])
    dist = math.hypot(*d)
    np.testing.assert_allclose(got, p + (d / dist) * (K * (0.12 - dist)) * DT * DT, atol=1e-12)


def test_segment_degenerate_matches_circle():
    seg = _geom_step(ObstacleShape.SEGMENT, [0.3, 0.0], [0.1, 0.0], radius=0.15, half=(0.0, 0.0))
    circ = _geom_step(ObstacleShape.CIRCLE, [0.3, 0.0], [0.1, 0.0], radius=0.15)
    np.testing.assert_allclose(seg, circ, atol=1e-14)


def test_no_activation_outside_reach():
    got = _geom_step(ObstacleShape.BOX, [0.0, 0.0], [0.5, 0.5], half=(0.1, 0.1))
    np.testing.assert_allclose(got, [0.5, 0.5], atol=1e-14)


# ------------------------------------------------------- BPTT closed forms (test_gradients.py)

BIG = 100.0


def _rollout_grad(configs, dt, state, acts, loss_pos_index):
    E = np.asarray(state["pos"]).shape[0]
    world = WorldConfig(collisions=False)
    cfg = oracle_cfg(configs, world, dt, 1, E, acts.shape[-1])
    p, t, m = params_of(configs)
    s0 = pack_state(state)
    traj = O64.rollout(cfg, p, t, m, None, s0, acts)
    afin = np.zeros_like(s0)
    afin[loss_pos_index] = 1.0
    return O64.rollout_adj(cfg, p, t, m, None, s0, acts, traj, None, afin)


def test_bptt_analytic_holonomic():
    # tests/unit/test_gradients.py:174-187: d x_T / d a_t = dt for every t
    T, dt = 6, 0.1
    cfgs = [AgentConfig(model=DynamicsModel.HOLONOMIC, max_speed=BIG)]
    rng = np.random.default_rng(4)
    st = state_dict_np(rng.normal(size=(1, 1, 2)) * 0.5, vel=rng.normal(size=(1, 1, 2)) * 0.5)
    acts = 0.2 * rng.normal(size=(T, 1, 1, 2))
    _, g = _rollout_grad(cfgs, dt, st, acts, (0, 0, 0))
    expected = np.zeros_like(g)
    expected[:, 0, 0, 0] = dt
    np.testing.assert_allclose(g, expected, atol=1e-15)


def test_bptt_analytic_holonomic_accel():
    # tests/unit/test_gradients.py:190-209: d x_2 / d a_0x = 2 dt^2
    dt = 0.1
    cfgs = [AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=ControlMode.ACCELERATION,
                        max_speed=BIG, max_accel=BIG)]
    rng = np.random.default_rng(5)
    st = state_dict_np(rng.normal(size=(1, 1, 2)) * 0.5, vel=rng.normal(size=(1, 1, 2)) * 0.5)
    acts = 0.2 * rng.normal(size=(2, 1, 1, 2))
    _, g = _rollout_grad(cfgs, dt, st, acts, (0, 0, 0))
    assert abs(g[0, 0, 0, 0] - 2 * dt * dt) < 1e-15


def test_grads_finite_zero_when_clamped():
    # tests/unit/test_gradients.py:212-221: saturated diff-drive command -> zero grad
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=1.0, max_ang_vel=1.0)]
    rng = np.random.default_rng(6)
    st = state_dict_np(rng.normal(size=(1, 1, 2)) * 0.5, theta=rng.normal(size=(1, 1)))
    acts = np.full((1, 1, 1, 2), 50.0)
    E = 1
    world = WorldConfig(collisions=False)
    cfg = oracle_cfg(cfgs, world, 0.1, 1, E, 2)
    p, t, m = params_of(cfgs)
    s0 = pack_state(st)
    traj = O64.rollout(cfg, p, t, m, None, s0, acts)
    afin = np.zeros_like(s0)
    afin[..., 0:2] = 1.0
    _, g = O64.rollout_adj(cfg, p, t, m, None, s0, acts, traj, None, afin)
    assert np.isfinite(g).all() and np.abs(g).sum() == 0.0


# ------------------------------------------------------------- drone (test_drone.py)

PRM = dict(mass=1.0, arm=0.15, ixx=0.01, iyy=0.01, izz=0.02, kappa=0.02, gravity=9.81,
           thrust_max=20.0)


def _drone():
    return AgentConfig(model=DynamicsModel.DRONE, mass=PRM["mass"], arm_length=PRM["arm"],
                       inertia_xx=PRM["ixx"], inertia_yy=PRM["iyy"], inertia_zz=PRM["izz"],
                       torque_coeff=PRM["kappa"], gravity=PRM["gravity"],
                       thrust_max=PRM["thrust_max"])


def _drone_rollout(init, thrusts, dt):
    st = state_dict_np(init["p"].reshape(1, 1, 2), vel=init["v"].reshape(1, 1, 2),
                       z=np.array([[init["z"]]]), vz=np.array([[init["vz"]]]),
                       attitude=init["q"].reshape(1, 1, 4), body_rates=init["br"].reshape(1, 1, 3))
    world = WorldConfig(collisions=False)
    cfg = oracle_cfg([_drone()], world, dt, 1, 1, 4)
    p, t, m = params_of([_drone()])
    traj = O64.rollout(cfg, p, t, m, None, pack_state(st), thrusts.reshape(-1, 1, 1, 4))
    return unpack_state(traj[-1])


def _rest():
    return {"p": np.array([0.3, -0.2]), "z": 1.0, "v": np.zeros(2), "vz": 0.0,
            "q": np.array([0.0, 0.0, 0.0, 1.0]), "br": np.zeros(3)}


def test_drone_hover_equilibrium():
    hover = PRM["mass"] * PRM["gravity"] / 4.0
    last = _drone_rollout(_rest(), np.tile(np.full(4, hover), (50, 1)), 0.02)
    np.testing.assert_allclose(last["pos"][0, 0], [0.3, -0.2], atol=1e-10)
    np.testing.assert_allclose(last["z"][0, 0], 1.0, atol=1e-10)
    np.testing.assert_allclose(last["attitude"][0, 0], [0, 0, 0, 1], atol=1e-10)
    np.testing.assert_allclose(last["body_rates"][0, 0], [0, 0, 0], atol=1e-12)


def test_drone_vertical_climb_analytic():
    # semi-implicit Euler: z_T = z0 + az dt^2 T (T+1) / 2, vz_T = az dt T
    dt, T = 0.02, 40
    f = PRM["mass"] * PRM["gravity"] / 4.0 + 0.5
    last = _drone_rollout(_rest(), np.tile(np.full(4, f), (T, 1)), dt)
    az = 4.0 * f / PRM["mass"] - PRM["gravity"]
    np.testing.assert_allclose(last["z"][0, 0], 1.0 + az * dt * dt * T * (T + 1) / 2.0, atol=1e-9)
    np.testing.assert_allclose(last["vz"][0, 0], az * dt * T, atol=1e-10)
    np.testing.assert_allclose(last["attitude"][0, 0], [0, 0, 0, 1], atol=1e-12)


def _quat_mul(a, b):
    ax, ay, az, aw = a
    bx, by, bz, bw = b
    return np.array([aw * bx + ax * bw + ay * bz - az * by,
                     aw * by - ax * bz + ay * bw + az * bx,
                     aw * bz + ax * by - ay * bx + az * bw,
                     aw * bw - ax * bx - ay * by - az * bz])


def _drone_numpy(init, thrusts, dt):
    """Independent numpy 6-DOF recurrence: rotation by R(q) v = q v q*, body-frame
    Euler equation, q' = 0.5 q (x) (w, 0), semi-implicit Euler (rates first)."""
    p, z, v, vz = init["p"].copy(), init["z"], init["v"].copy(), init["vz"]
    q, w = init["q"].copy(), init["br"].copy()
    I = np.array([PRM["ixx"], PRM["iyy"], PRM["izz"]])
    for a in thrusts:
        f = np.clip(a, 0.0, PRM["thrust_max"])
        fw = _quat_mul(_quat_mul(q, np.array([0.0, 0.0, f.sum(), 0.0])), q * [-1, -1, -1, 1])[:3]
        acc = fw / PRM["mass"] - np.array([0.0, 0.0, PRM["gravity"]])
        tau = np.array([PRM["arm"] * (f[1] - f[3]), PRM["arm"] * (f[2] - f[0]),
                        PRM["kappa"] * (f[0] - f[1] + f[2] - f[3])])
        w = w + (tau - np.cross(w, I * w)) / I * dt
        vz = vz + acc[2] * dt
        v = v + acc[:2] * dt
        q = q + 0.5 * _quat_mul(q, np.array([w[0], w[1], w[2], 0.0])) * dt
        q = q / np.linalg.norm(q)
        p = p + v * dt
        z = z + vz * dt
    return p, z, v, vz, q, w


def test_drone_matches_independent_numpy():
    rng = np.random.default_rng(0)
    dt, T = 0.01, 60
    hover = PRM["mass"] * PRM["gravity"] / 4.0
    thrusts = hover + 0.4 * rng.standard_normal((T, 4))
    init = {"p": np.array([0.0, 0.0]), "z": 0.5, "v": np.array([0.1, -0.05]), "vz": 0.2,
            "q": np.array([0.0, 0.0, 0.0, 1.0]), "br": np.array([0.05, -0.03, 0.1])}
    last = _drone_rollout(init, thrusts, dt)
    p, z, v, vz, q, w = _drone_numpy(init, thrusts, dt)
    np.testing.assert_allclose(last["pos"][0, 0], p, atol=1e-9)
    np.testing.assert_allclose(last["z"][0, 0], z, atol=1e-9)
    np.testing.assert_allclose(last["vel"][0, 0], v, atol=1e-9)
    np.testing.assert_allclose(last["vz"][0, 0], vz, atol=1e-9)
    np.testing.assert_allclose(last["attitude"][0, 0], q, atol=1e-9)
    np.testing.assert_allclose(last["body_rates"][0, 0], w, atol=1e-9)


def test_drone_yaw_torque():
    dt, T = 0.01, 30
    hover = PRM["mass"] * PRM["gravity"] / 4.0
    th = np.tile(np.array([hover + 0.5, hover - 0.5, hover + 0.5, hover - 0.5]), (T, 1))
    last = _drone_rollout(_rest(), th, dt)
    np.testing.assert_allclose(last["z"][0, 0], 1.0, atol=1e-9)
    assert last["body_rates"][0, 0, 2] > 1e-3 and abs(last["attitude"][0, 0, 2]) > 1e-3


# ----------------------------------------------- diff-drive / bicycle kinematics closed forms

def test_diffdrive_velocity_closed_form():
    # velocity mode: theta += w dt, p += s (cos th, sin th) dt with the OLD heading
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=BIG, max_ang_vel=BIG)]
    world = WorldConfig(collisions=False)
    st = state_dict_np([[[0.2, -0.1]]], theta=[[0.3]])
    out, _ = step(cfgs, world, 0.1, st, [[[0.7, 0.4]]])
    np.testing.assert_allclose(out["pos"][0, 0], [0.2 + 0.07 * math.cos(0.3), -0.1 + 0.07 * math.sin(0.3)], atol=1e-15)
    np.testing.assert_allclose(out["theta"][0, 0], 0.3 + 0.04, atol=1e-15)


def test_bicycle_closed_form():
    # slip angle beta = atan(tan(delta) l_r / (l_f + l_r)); omega = s / L cos(beta) tan(delta)
    cfgs = [AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, max_speed=BIG, max_accel=BIG,
                        max_steer=1.0, l_f=0.16, l_r=0.14)]
    world = WorldConfig(collisions=False)
    st = state_dict_np([[[0.0, 0.0]]], theta=[[0.2]], speed=[[0.5]])
    out, _ = step(cfgs, world, 0.1, st, [[[1.0, 0.3]]])
    s = 0.5 + 1.0 * 0.1
    beta = math.atan(math.tan(0.3) * 0.14 / 0.3)
    om = s / 0.3 * math.cos(beta) * math.tan(0.3)
    np.testing.assert_allclose(out["speed"][0, 0], s, atol=1e-15)
    np.testing.assert_allclose(out["pos"][0, 0], [s * math.cos(0.2 + beta) * 0.1, s * math.sin(0.2 + beta) * 0.1], atol=1e-15)
    np.testing.assert_allclose(out["theta"][0, 0], 0.2 + om * 0.1, atol=1e-15)
