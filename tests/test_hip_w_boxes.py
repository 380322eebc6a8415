"""Box agents on the HIP path vs the CPU oracle (collision_forces_box_kernel and the
footprint clamp, swarp/core/collisions.py:999-1059, swarp/dynamics/kernels.py:79-99).

Bars:
* float64, every case at full length: states at 1e-10 and gradients at 1e-8 relative
  (max-norm) -- the pin of the box adjoint;
* float32 states at 1e-5 relative over the full rollout (box geometry runs through
  cos / sin, whose device and host results differ by an ulp);
* float32 gradients: at least as accurate as the float32 oracle's.  Both are measured
  against the float64 oracle run on the same (float32-rounded) inputs, and the HIP
  error may be at most twice the oracle's (floor 1e-5).  A fixed float32-vs-float32
  tolerance does not fit box contacts: a point sunk just inside a box's surface (the
  exterior distance |o| barely above its floor, o the short difference of two nearly
  equal coordinates) has a normal o / |o| whose derivative scales with 1 / |o|, so
  one-ulp differences of cos / sin become relative gradient differences of 1e-4 to a
  few 1e-3 between any two float32 evaluations of the same formula (both sit equally
  far from the float64 result).
The HIP reverse pass differentiates the box contacts with forward-mode tangents per lane
(gathering each pair's cotangents), the oracle with seeded one-tangent duals per pair
(scattering to both agents): the comparison checks two assemblies of the same
Jacobians.
"""

import numpy as np
import pytest
import torch

from hip_helpers import hip_run, make_stepper, oracle_run, rel
from oracle.oracle import pack_state
from swarp_amd.config import AgentConfig, AgentShape, ControlMode, DynamicsModel, Integrator, WorldConfig
from test_hip_parity import _cotangent

pytestmark = pytest.mark.gpu


def _box(hx, hy, model, **kw):
    return AgentConfig(model=model, shape=AgentShape.BOX, half_extents=(hx, hy), radius=None,
                       max_speed=2.0, max_accel=4.0, **kw)


def _fleet(A):
    q = A // 3
    cfgs = [AgentConfig(radius=0.05, max_speed=2.0, max_accel=4.0,
                        ctrl_mode=ControlMode.ACCELERATION) for _ in range(q)]
    cfgs += [_box(0.07, 0.04, DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION)
             for _ in range(q)]
    cfgs += [_box(0.06, 0.035, DynamicsModel.KINEMATIC_BICYCLE, l_f=0.05, l_r=0.05,
                  max_steer=0.6) for _ in range(A - 2 * q)]
    return cfgs


def _state(E, A, rng, extent, dtype):
    return pack_state({
        "pos": rng.uniform(-extent, extent, size=(E, A, 2)),
        "theta": rng.uniform(-np.pi, np.pi, size=(E, A)),
        "vel": rng.normal(size=(E, A, 2)) * 0.2,
        "speed": rng.normal(size=(E, A)) * 0.2,
        "ang_vel": rng.normal(size=(E, A)) * 0.5,
    }).astype(dtype)


def _obstacles(E, rng):
    n = 6
    return {"pos": rng.uniform(-0.5, 0.5, size=(E, n, 2)),
            "radius": np.r_[rng.uniform(0.04, 0.1, 2), np.zeros(2), np.full(2, 0.03)],
            "type": np.r_[np.zeros(2), np.ones(2), np.full(2, 2)].astype(np.int32),
            "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
            "half": np.r_[np.zeros((2, 2)), rng.uniform(0.04, 0.12, size=(2, 2)),
                          np.c_[rng.uniform(0.05, 0.15, 2), np.zeros(2)]]}


def _run(cfgs, world, S, s0, acts, w, dtype, obs=None, E=None):
    td = torch.float32 if dtype == np.float32 else torch.float64
    st = make_stepper(cfgs, world, 0.05, S, td, obs=obs, n_envs=E)
    assert st.has_boxes
    hip = hip_run(st, s0, acts, w, dtype)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, dtype, obs=obs)
    return hip, orc


def _check_box(name, cfgs, world, S, s0, acts, w, obs=None, E=None):
    hip, orc = _run(cfgs, world, S, s0.astype(np.float64), acts.astype(np.float64), w,
                    np.float64, obs=obs, E=E)
    hs, hg0, hga = hip
    os_, og0, oga = orc
    print(f"\n{name} f64: states rel {rel(hs[..., :7], os_[..., :7]):.3e}, d/d actions rel "
          f"{rel(hga, oga):.3e}, d/d state0 rel {rel(hg0[..., :7], og0[..., :7]):.3e}")
    assert rel(hs[..., :7], os_[..., :7]) <= 1e-10, f"{name} f64 states"
    assert rel(hga, oga) <= 1e-8, f"{name} f64 d/d actions {rel(hga, oga):.3e}"
    assert rel(hg0[..., :7], og0[..., :7]) <= 1e-8, f"{name} f64 d/d state0"
    s32, a32 = s0.astype(np.float32), acts.astype(np.float32)
    _, truth = _run(cfgs, world, S, s32.astype(np.float64), a32.astype(np.float64), w,
                    np.float64, obs=obs, E=E)
    hip, orc = _run(cfgs, world, S, s32, a32, w, np.float32, obs=obs, E=E)
    print(f"{name} f32: states rel {rel(hip[0][..., :7], orc[0][..., :7]):.3e}")
    assert rel(hip[0][..., :7], orc[0][..., :7]) <= 1e-5, f"{name} f32 states"
    for k, what in ((2, "d/d actions"), (1, "d/d state0")):
        h, o, t = (x[k][..., :7] if k == 1 else x[k] for x in (hip, orc, truth))
        e_hip, e_orc = rel(h, t), rel(o, t)
        print(f"{name} f32 {what}: HIP vs f32 oracle {rel(h, o):.3e}; vs f64: HIP {e_hip:.3e}, "
              f"f32 oracle {e_orc:.3e}")
        assert e_hip <= max(2.0 * e_orc, 1e-5), (
            f"{name} f32 {what}: error vs f64 {e_hip:.3e}, the f32 oracle's {e_orc:.3e}")


def test_box_fleet_with_obstacles_and_walls():
    """Discs, diff-drive boxes and bicycle boxes in crowded envs with circle, box and
    capsule obstacles inside soft walls, four substeps (12 agents: padded lanes)."""
    E, A, T, S = 48, 12, 8, 4
    rng = np.random.default_rng(31)
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.6, 0.6, -0.6, 0.6), max_neighbors=8,
                        contact_max_overlap=0.05)
    s0 = _state(E, A, rng, 0.45, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 3, scale=0.1)
    _check_box("box fleet", _fleet(A), world, S, s0, acts, w, obs=_obstacles(E, rng), E=E)


@pytest.mark.parametrize("integ", [Integrator.EULER, Integrator.RK4], ids=["euler", "rk4"])
def test_box_footprint_clamp(integ):
    """Box and disc agents against the footprint clamp."""
    E, A, T, S = 40, 8, 8, 2
    rng = np.random.default_rng(32)
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.3, 0.3, -0.3, 0.3), bounds_mode="clamp", max_neighbors=7,
                        integrator=integ)
    s0 = _state(E, A, rng, 0.25, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 4, scale=0.1)
    _check_box(f"box clamp {integ.name}", _fleet(A), world, S, s0, acts, w)


def test_sixty_four_box_agents():
    """A full wave per env (64 agents, 64-bit list masks), all boxes."""
    E, A, T, S = 6, 64, 4, 2
    rng = np.random.default_rng(34)
    cfgs = [_box(0.05, 0.03, DynamicsModel.DIFF_DRIVE) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.7, 0.7, -0.7, 0.7), max_neighbors=12)
    s0 = _state(E, A, rng, 0.6, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 6, scale=0.1)
    _check_box("64 boxes", cfgs, world, S, s0, acts, w)



def test_wide_env_box_fleet():
    """80 agents per env (the wide-env kernels: one workgroup per env): discs, diff-drive
    boxes and bicycle boxes among circle, box and capsule obstacles inside soft walls."""
    E, A, T, S = 5, 80, 5, 2
    rng = np.random.default_rng(36)
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.9, 0.9, -0.9, 0.9), max_neighbors=10)
    s0 = _state(E, A, rng, 0.8, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 7, scale=0.1)
    obs = _obstacles(E, rng)
    obs["pos"] = obs["pos"] * 1.6
    _check_box("wide boxes A=80", _fleet(A), world, S, s0, acts, w, obs=obs, E=E)



def test_box_fleet_1024_agents_per_env():
    """1024 agents per env, a third of them discs: the box world's staging (headings, spins,
    footprints) takes the workgroup beyond 64 KiB of LDS."""
    E, A, T, S = 1, 1024, 3, 2
    rng = np.random.default_rng(39)
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-2.5, 2.5, -2.5, 2.5), max_neighbors=8)
    s0 = _state(E, A, rng, 2.4, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 9, scale=0.1)
    _check_box("wide boxes A=1024", _fleet(A), world, S, s0, acts, w)

def test_grid_ordered_box_fleet():
    """Box agents with uniform-grid lists (pinned frame), capped at 4 neighbours so the
    grid's traversal order decides which contacts act; footprint clamp."""
    E, A, T, S = 6, 36, 5, 2
    rng = np.random.default_rng(37)
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.5, 0.5, -0.5, 0.5), bounds_mode="clamp", max_neighbors=4,
                        neighbor_method="uniform_grid", uniform_bins=6)
    s0 = _state(E, A, rng, 0.45, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 8, scale=0.1)
    st = make_stepper(_fleet(A), world, 0.05, S, torch.float64)
    assert st.wide and st.list_method == "uniform_grid"
    _check_box("grid boxes A=36", _fleet(A), world, S, s0, acts, w)

def test_wheel_contacts_forward_and_no_reverse():
    """WorldConfig.wheel_contacts: contact torques (pair torques at the manifold point or
    the disc's nearest point, obstacle and wall torques) and wheel_contact's rework of the
    diff-drive step, forward only (collisions.py:1128-1403, kernels.py:1328-1478): states
    within 1e-10 of the fp64 oracle, 1e-5 of the fp32 one; a differentiated rollout raises
    as the reference's taped path does (swarp/core/stepper.py:852-857)."""
    from hip_helpers import state_to16, to_torch_state
    from oracle.oracle import Oracle
    from cases import obstacles_np, oracle_cfg, params_of
    from swarp_amd import rollout

    E, A, T, S = 40, 9, 8, 2
    rng = np.random.default_rng(35)
    cfgs = ([AgentConfig(radius=0.05, max_speed=2.0, max_accel=4.0) for _ in range(3)]
            + [_box(0.07, 0.04, DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION)
               for _ in range(6)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.5, 0.5, -0.5, 0.5), max_neighbors=8, wheel_contacts=True,
                        wheel_lateral_friction=0.3, wheel_turn_torque=0.02)
    obs = _obstacles(E, rng)
    s0 = _state(E, A, rng, 0.4, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    for dt_np, td, tol in ((np.float64, torch.float64, 1e-10), (np.float32, torch.float32, 1e-5)):
        st = make_stepper(cfgs, world, 0.05, S, td, obs=obs, n_envs=E)
        state = to_torch_state(s0.astype(dt_np), td, False, 5)
        a = torch.tensor(acts.astype(dt_np), dtype=td, device="cuda")
        with torch.no_grad():
            _, traj = rollout(st, state, a)
        hs = np.stack([state_to16(x) for x in traj])
        cfg = oracle_cfg(cfgs, world, 0.05, S, E, 2)
        p, t, m = params_of(cfgs)
        os_ = Oracle(dt_np).rollout(cfg, p, t, m, obstacles_np(obs, E), s0.astype(dt_np),
                                    acts.astype(dt_np))
        assert np.isfinite(hs).all()
        assert rel(hs[..., :7], os_[..., :7]) <= tol, f"{np.dtype(dt_np).name} states"
    # the wheel rework changes the trajectory (the parity above is not vacuous)
    plain = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.5, 0.5, -0.5, 0.5), max_neighbors=8)
    cfg = oracle_cfg(cfgs, plain, 0.05, S, E, 2)
    ref = Oracle(np.float64).rollout(cfg, p, t, m, obstacles_np(obs, E), s0, acts)
    assert rel(ref[..., :7], os_[..., :7].astype(np.float64)) > 1e-3
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    state = to_torch_state(s0.astype(np.float32), torch.float32, True, 5)
    with pytest.raises(ValueError, match="wheel_contacts"):
        rollout(st, state, torch.zeros(T, E, A, 2, device="cuda", requires_grad=True))



def test_wheel_contacts_wide_env():
    """Wheel contacts (forward only) in envs of 72 agents on the wide-env kernels: states
    within 1e-10 of the fp64 oracle and 1e-5 of the fp32 one."""
    from hip_helpers import state_to16, to_torch_state
    from oracle.oracle import Oracle
    from cases import obstacles_np, oracle_cfg, params_of
    from swarp_amd import rollout

    E, A, T, S = 4, 72, 5, 2
    rng = np.random.default_rng(38)
    cfgs = ([AgentConfig(radius=0.05, max_speed=2.0, max_accel=4.0) for _ in range(24)]
            + [_box(0.07, 0.04, DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION)
               for _ in range(48)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.8, 0.8, -0.8, 0.8), max_neighbors=8, wheel_contacts=True,
                        wheel_lateral_friction=0.3, wheel_turn_torque=0.02)
    obs = _obstacles(E, rng)
    s0 = _state(E, A, rng, 0.7, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    for dt_np, td, tol in ((np.float64, torch.float64, 1e-10), (np.float32, torch.float32, 1e-5)):
        st = make_stepper(cfgs, world, 0.05, S, td, obs=obs, n_envs=E)
        assert st.wide
        state = to_torch_state(s0.astype(dt_np), td, False, 5)
        with torch.no_grad():
            _, traj = rollout(st, state, torch.tensor(acts.astype(dt_np), dtype=td, device="cuda"))
        hs = np.stack([state_to16(x) for x in traj])
        cfg = oracle_cfg(cfgs, world, 0.05, S, E, 2)
        p, t, m = params_of(cfgs)
        os_ = Oracle(dt_np).rollout(cfg, p, t, m, obstacles_np(obs, E), s0.astype(dt_np),
                                    acts.astype(dt_np))
        assert np.isfinite(hs).all()
        assert rel(hs[..., :7], os_[..., :7]) <= tol, f"{np.dtype(dt_np).name} states"

def test_wheel_contacts_disc_diff_drive():
    """Disc diff-drive agents (velocity and servo control) under wheel_contacts: no
    footprint inertia, so the reference's torque term would be 0 * inf = NaN
    (swarp/dynamics/kernels.py:1379-1386); here it is skipped when there is no excess
    torque, headings stay finite, and HIP equals the oracle (fp64 1e-10, fp32 1e-5)."""
    from hip_helpers import state_to16, to_torch_state
    from oracle.oracle import Oracle
    from cases import oracle_cfg, params_of
    from swarp_amd import rollout

    E, A, T, S = 32, 6, 8, 2
    rng = np.random.default_rng(41)
    cfgs = ([AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(3)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.SERVO,
                           radius=0.05, max_speed=1.5, max_accel=2.0) for _ in range(3)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.3, 0.3, -0.3, 0.3), max_neighbors=6, wheel_contacts=True,
                        wheel_lateral_friction=0.3, wheel_turn_torque=0.02)
    s0 = _state(E, A, rng, 0.25, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    for dt_np, td, tol in ((np.float64, torch.float64, 1e-10), (np.float32, torch.float32, 1e-5)):
        st = make_stepper(cfgs, world, 0.05, S, td)
        state = to_torch_state(s0.astype(dt_np), td, False, 5)
        with torch.no_grad():
            _, traj = rollout(st, state, torch.tensor(acts.astype(dt_np), dtype=td, device="cuda"))
        hs = np.stack([state_to16(x) for x in traj])
        cfg = oracle_cfg(cfgs, world, 0.05, S, E, 2)
        p, t, m = params_of(cfgs)
        os_ = Oracle(dt_np).rollout(cfg, p, t, m, None, s0.astype(dt_np), acts.astype(dt_np))
        assert np.isfinite(hs).all() and np.isfinite(os_).all()
        assert rel(hs[..., :7], os_[..., :7]) <= tol, f"{np.dtype(dt_np).name} states"


def test_per_env_parameter_tables():
    """Stepper.set_agent_params_per_env (swarp/core/stepper.py:493-575; the *_per_env
    kernels): masses, radii, speed and turn limits randomized per env.  Each env of the HIP
    rollout equals an independent oracle rollout with that env's rows (states and
    gradients, fp64 1e-10 / 1e-8), with box and disc agents, obstacles and walls."""
    from swarp_amd import per_env_float_template
    from swarp_amd.config import P_MASS, P_MAX_ANG_VEL, P_MAX_SPEED, P_RADIUS

    E, A, T, S = 12, 6, 5, 2
    rng = np.random.default_rng(36)
    cfgs = ([AgentConfig(radius=0.05, max_speed=2.0, max_accel=4.0) for _ in range(3)]
            + [_box(0.07, 0.04, DynamicsModel.DIFF_DRIVE) for _ in range(3)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-0.4, 0.4, -0.4, 0.4), max_neighbors=6, neighbor_radius=0.3)
    obs = _obstacles(E, rng)
    tab = per_env_float_template(cfgs, E)
    tab[..., P_MASS] *= rng.uniform(0.5, 2.0, size=(E, A))
    tab[:, :3, P_RADIUS] *= rng.uniform(0.7, 1.3, size=(E, 3))
    tab[..., P_MAX_SPEED] *= rng.uniform(0.5, 1.5, size=(E, A))
    tab[..., P_MAX_ANG_VEL] *= rng.uniform(0.5, 1.5, size=(E, A))
    s0 = _state(E, A, rng, 0.3, np.float64)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cotangent(T, E, A, 7, scale=0.1)
    st = make_stepper(cfgs, world, 0.05, S, torch.float64, obs=obs, n_envs=E)
    st.set_agent_params_per_env(tab)
    hs, hg0, hga = hip_run(st, s0, acts, w, np.float64)
    from cases import obstacles_np, oracle_cfg
    from oracle.oracle import Oracle

    O = Oracle(np.float64)
    cfg = oracle_cfg(cfgs, world, 0.05, S, 1, 2)
    tags = np.array([int(c.model) for c in cfgs], dtype=np.int32)
    modes = np.array([int(c.ctrl_mode) for c in cfgs], dtype=np.int32)
    for e in range(E):
        # env e's obstacles: the per-env arrays (poses, angles) sliced, the shared kept
        ob_e = {k: (np.asarray(v)[e:e + 1] if k in ("pos", "angle") else v)
                for k, v in obs.items()}
        obn = obstacles_np(ob_e, 1)
        tr = O.rollout(cfg, tab[e], tags, modes, obn, s0[e:e + 1], acts[:, e:e + 1])
        g0, ga = O.rollout_adj(cfg, tab[e], tags, modes, obn, s0[e:e + 1], acts[:, e:e + 1], tr,
                               w[:, e:e + 1], None)
        assert rel(hs[:, e:e + 1, :, :7], tr[..., :7]) <= 1e-10, f"env {e} states"
        assert rel(hga[:, e:e + 1], ga) <= 1e-8, f"env {e} d/d actions"
        assert rel(hg0[e:e + 1, :, :7], g0[..., :7]) <= 1e-8, f"env {e} d/d state0"


def test_servo_control_mode():
    """ControlMode.SERVO (servo_command, swarp/dynamics/kernels.py:165-191, applied before
    Euler or RK4): diff-drive servo agents (discs and boxes) with contacts and walls,
    states and gradients against the oracle (fp64 1e-10 / 1e-8, fp32 states 1e-5)."""
    from swarp_amd.config import ControlMode as CM

    E, A, T, S = 24, 6, 6, 2
    rng = np.random.default_rng(37)
    cfgs = ([AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=CM.SERVO, radius=0.05,
                         max_speed=1.5, max_accel=2.0, cmd_gain_v=0.8, cmd_gain_w=1.2)
             for _ in range(3)]
            + [_box(0.07, 0.04, DynamicsModel.DIFF_DRIVE, ctrl_mode=CM.SERVO) for _ in range(3)])
    for integ in (Integrator.EULER, Integrator.RK4):
        world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                            bounds=(-0.35, 0.35, -0.35, 0.35), max_neighbors=6, integrator=integ)
        s0 = _state(E, A, rng, 0.3, np.float64)
        acts = rng.uniform(-2, 2, size=(T, E, A, 2))
        w = _cotangent(T, E, A, 8, scale=0.1)
        hip, orc = _run(cfgs, world, S, s0, acts, w, np.float64)
        assert rel(hip[0][..., :7], orc[0][..., :7]) <= 1e-10, integ
        assert rel(hip[2], orc[2]) <= 1e-8 and rel(hip[1][..., :7], orc[1][..., :7]) <= 1e-8, integ
        hip, orc = _run(cfgs, world, S, s0.astype(np.float32), acts.astype(np.float32), w,
                        np.float32)
        assert rel(hip[0][..., :7], orc[0][..., :7]) <= 1e-5, integ
