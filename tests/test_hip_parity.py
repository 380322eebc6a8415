"""HIP path vs the CPU oracle on identical seeded inputs (the parity tests proper).

Bars (written per test):
* float32 states are compared BIT-EXACT with the float32 oracle: both keep the
  reference's op order with no FMA contraction and correctly rounded divide / sqrt, and
  the transcendental functions (diff-drive, bicycle, box / segment obstacles) come from
  one portable evaluation (include/swarp_pmath.h) on host and device;
* gradients are compared at 1e-5 relative (max-norm) against the float32 oracle, and at
  the reference's own cross-precision bar (rtol 1e-3, tests/unit/test_gradients.py:257)
  against the float64 oracle;
* where a float32 rollout is long enough for its own rounding to show against float64
  (config 3 and config 4 workloads), the HIP float32 gradient's error against the float64
  oracle (same float32-rounded inputs) is also held to the float32 oracle's own error
  against it, within 1 %: the HIP path loses no accuracy that a float32 evaluation of the
  same formulas in the oracle's order does not.
Measured errors are printed (run with -s to see them).
"""

import numpy as np
import pytest
import torch

from cases import nav_agents, nav_inputs, nav_world
from hip_helpers import check_grad, hip_run, make_stepper, oracle_run, rel
from oracle.oracle import pack_state
from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, ObstacleShape, WorldConfig

pytestmark = pytest.mark.gpu


def _nav_case(E, A, T, S, extent, seed=0, dtype=np.float32):
    pos, goals, acts = nav_inputs(E, A, T, extent=extent, seed=seed, dtype=torch.float64)
    s0 = pack_state({"pos": pos.numpy()}, dtype=np.float64).astype(dtype)
    acts = acts.numpy().astype(dtype)
    # loss = sum ||p_T - g||^2  ->  adjoint 2 (p_T - g) on the final position only;
    # plus a random cotangent on every trajectory state so every adjoint path is used
    return s0, acts, goals.numpy()


def _cotangent(T, E, A, seed, nf=5, scale=1.0):
    rng = np.random.default_rng(seed)
    w = rng.normal(size=(T, E, A, 16)) * scale
    if nf == 5:
        w[..., 7:] = 0.0
    return w


def _check(name, hip, orc, state_exact, g_tol=1e-5, nf=5, o64=None):
    hs, hg0, hga = hip
    os_, og0, oga = orc
    cols = slice(0, 7) if nf == 5 else slice(0, 16)
    print(f"\n{name}: states rel {rel(hs[..., cols], os_[..., cols]):.3e}, d/d actions rel "
          f"{rel(hga, oga):.3e}, d/d state0 rel {rel(hg0[..., cols], og0[..., cols]):.3e}")
    if o64 is not None:
        _, g064, ga64 = o64
        for lab, h, o, t in (("d/d actions", hga, oga, ga64),
                             ("d/d state0", hg0[..., cols], og0[..., cols], g064[..., cols])):
            eh, eo = rel(h, t), rel(o, t)
            print(f"{name}: {lab} vs float64 oracle: HIP {eh:.3e}, float32 oracle {eo:.3e}")
            assert eh <= 1.01 * eo + 1e-7, (
                f"{name}: {lab} HIP error vs float64 {eh:.3e} exceeds the float32 oracle's {eo:.3e}")
    if state_exact:
        assert np.array_equal(hs[..., cols], os_[..., cols]), (
            f"{name}: states not bit-exact, max rel {rel(hs[..., cols], os_[..., cols]):.3e}")
    else:
        assert rel(hs[..., cols], os_[..., cols]) <= 1e-5, f"{name}: states rel {rel(hs[..., cols], os_[..., cols]):.3e}"
    check_grad(f"{name}: d/d actions", hga, oga, tol=g_tol)
    check_grad(f"{name}: d/d state0", hg0[..., cols], og0[..., cols], tol=g_tol)


def test_config1_navigation_bitexact():
    """Config 1: 64 envs x 4 holonomic agents, dt 0.05, 1 substep, 10 steps."""
    E, A, T = 64, 4, 10
    s0, acts, goals = _nav_case(E, A, T, 1, extent=1.0)
    w = _cotangent(T, E, A, 1)
    cfgs, world = nav_agents(A), nav_world(A, world_size=1.0)
    st = make_stepper(cfgs, world, 0.05, 1, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, 1, s0, acts, w, np.float32)
    _check("c1", hip, orc, state_exact=True)
    o64 = oracle_run(cfgs, world, 0.05, 1, s0.astype(np.float64), acts.astype(np.float64), w, np.float64)
    np.testing.assert_allclose(hip[2], o64[2], rtol=1e-3, atol=1e-4)


def test_config2_shape_reduced():
    """Config 2 shape: 16 agents in a 4x4 arena, 4 substeps, 32 steps (1000 envs)."""
    E, A, T, S = 1000, 16, 32, 4
    s0, acts, _ = _nav_case(E, A, T, S, extent=2.0, seed=3)
    w = _cotangent(T, E, A, 2)
    cfgs, world = nav_agents(A), nav_world(A, world_size=2.0)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    _check("c2-reduced", hip, orc, state_exact=True)


def test_crowded_contacts_truncated_lists():
    """Dense envs with truncated lists (K < A - 1), velocity damping, walls, 3 substeps."""
    E, A, T, S = 128, 12, 6, 3
    rng = np.random.default_rng(5)
    s0 = pack_state({"pos": rng.uniform(-0.3, 0.3, size=(E, A, 2)),
                     "vel": 0.3 * rng.normal(size=(E, A, 2))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    cfgs = nav_agents(A, agent_radius=0.08, mode=ControlMode.ACCELERATION)
    world = WorldConfig(collision_k=50.0, collision_c=2.0, collision_margin=0.03, max_neighbors=4,
                        neighbor_radius=0.3, bounds=(-0.4, 0.4, -0.4, 0.4))
    w = _cotangent(T, E, A, 3)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    _check("crowded", hip, orc, state_exact=True)


def test_mixed_fleet_obstacles():
    """Config 3 workload (1024 of its 4096 envs): 16 diff-drive + 16 bicycle agents,
    headings U[-pi, pi], 8 obstacles per env (4 circles, 2 boxes, 2 segments), soft walls,
    4 substeps, 20 steps.  States bit-exact; gradients 1e-5 of the float32 oracle and no
    less accurate than it against the float64 oracle."""
    E, A, T, S = 1024, 32, 20, 4
    rng = np.random.default_rng(7)
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(A // 2)] + [
        AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, radius=0.05) for _ in range(A // 2)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-2.0, 2.0, -2.0, 2.0), max_neighbors=32)
    n = 8
    obs = {"pos": rng.uniform(-2, 2, size=(E, n, 2)),
           "radius": np.r_[rng.uniform(0.05, 0.2, 4), np.zeros(2), np.full(2, 0.05)],
           "type": np.r_[np.zeros(4), np.ones(2), np.full(2, 2)].astype(np.int32),
           "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
           "half": np.r_[np.zeros((4, 2)), rng.uniform(0.05, 0.3, size=(2, 2)),
                         np.c_[rng.uniform(0.1, 0.4, 2), np.zeros(2)]]}
    s0 = pack_state({"pos": rng.uniform(-2, 2, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cotangent(T, E, A, 4, scale=0.1)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32, obs=obs)
    o64 = oracle_run(cfgs, world, 0.05, S, s0.astype(np.float64), acts.astype(np.float64), w,
                     np.float64, obs=obs)
    _check("mixed", hip, orc, state_exact=True, o64=o64)


def test_drones_config4_workload():
    """Config 4 workload (1024 of its 8192 envs): 8 quadrotors per env, rotor thrusts
    U[0, 1] x thrust_max (10), attitude axis uniform on the sphere with angle U[0, 0.1],
    planar contacts r = 0.1, dt 0.02, 1 substep, 64-step horizon.  States bit-exact;
    gradients 1e-5 of the float32 oracle and no less accurate than it against float64."""
    E, A, T, S = 1024, 8, 64, 1
    rng = np.random.default_rng(9)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    ax = rng.normal(size=(E, A, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(E, A, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    s0 = pack_state({"pos": rng.uniform(-1, 1, size=(E, A, 2)) * np.sqrt(A) * 0.25,
                     "z": np.ones((E, A)), "attitude": q}).astype(np.float32)
    acts = (rng.uniform(0, 1, size=(T, E, A, 4)) * 10.0).astype(np.float32)
    w = _cotangent(T, E, A, 5, nf=9, scale=0.01)
    st = make_stepper(cfgs, world, 0.02, S, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.02, S, s0, acts, w, np.float32)
    o64 = oracle_run(cfgs, world, 0.02, S, s0.astype(np.float64), acts.astype(np.float64), w,
                     np.float64)
    _check("drones-c4", hip, orc, state_exact=True, nf=9, o64=o64)


def test_drones_substeps_bitexact():
    """Quadrotors with 2 substeps and contacts in a tighter spawn (more contacts per step)."""
    E, A, T, S = 64, 8, 16, 2
    rng = np.random.default_rng(9)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    ax = rng.normal(size=(E, A, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(E, A, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)), "z": np.ones((E, A)),
                     "attitude": q}).astype(np.float32)
    acts = (rng.uniform(0, 1, size=(T, E, A, 4)) * 10.0).astype(np.float32)
    w = _cotangent(T, E, A, 5, nf=9, scale=0.01)
    st = make_stepper(cfgs, world, 0.02, S, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.02, S, s0, acts, w, np.float32)
    _check("drones-S2", hip, orc, state_exact=True, nf=9)


def test_float64_matches_float64_oracle():
    E, A, T, S = 32, 8, 8, 2
    s0, acts, _ = _nav_case(E, A, T, S, extent=0.4, seed=11, dtype=np.float64)
    cfgs, world = nav_agents(A), nav_world(A, world_size=0.5)
    w = _cotangent(T, E, A, 6)
    st = make_stepper(cfgs, world, 0.05, S, torch.float64)
    hip = hip_run(st, s0, acts, w, np.float64)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float64)
    _check("f64", hip, orc, state_exact=True, g_tol=1e-12)


def test_specialised_matches_generic_kernels():
    """The holonomic-velocity kernels and the generic kernels: identical forward bits,
    gradients equal to rounding (the adjoint sums in a different order)."""
    E, A, T, S = 400, 16, 12, 4
    s0, acts, _ = _nav_case(E, A, T, S, extent=0.6, seed=21)
    cfgs, world = nav_agents(A), nav_world(A, world_size=0.7)
    w = _cotangent(T, E, A, 7)
    lean = make_stepper(cfgs, world, 0.05, S, torch.float32)
    gen = make_stepper(cfgs, world, 0.05, S, torch.float32)
    gen.use_specialised = False
    a = hip_run(lean, s0, acts, w, np.float32)
    b = hip_run(gen, s0, acts, w, np.float32)
    assert np.array_equal(a[0][..., :7], b[0][..., :7])
    assert rel(a[2], b[2]) <= 1e-6 and rel(a[1][..., :7], b[1][..., :7]) <= 1e-6


def test_partial_last_wave():
    """n_envs that leave the last wave partly empty: a wave holds 64 / PA envs, so an env
    count that is not a multiple of that leaves env slots of the last wave past n_envs."""
    for A, E in ((4, 45), (16, 37), (16, 3), (64, 3)):
        T, S = 5, 2
        rng = np.random.default_rng(100 + A + E)
        s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2))}).astype(np.float32)
        acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
        cfgs = nav_agents(A)
        world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                            bounds=(-0.6, 0.6, -0.6, 0.6), max_neighbors=min(32, max(4, A)))
        w = _cotangent(T, E, A, 9)
        st = make_stepper(cfgs, world, 0.05, S, torch.float32)
        hip = hip_run(st, s0, acts, w, np.float32)
        orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
        _check(f"partial A={A} E={E}", hip, orc, state_exact=True)


def test_padded_agent_slots():
    """n_agents not a power of two (pad lanes in every env slot): 5, 12 and 20 agents."""
    for A, K in ((5, 4), (12, 12), (20, 8)):
        E, T, S = 96, 6, 2
        rng = np.random.default_rng(A)
        s0 = pack_state({"pos": rng.uniform(-0.4, 0.4, size=(E, A, 2))}).astype(np.float32)
        acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
        cfgs = nav_agents(A)
        world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                            bounds=(-0.5, 0.5, -0.5, 0.5), max_neighbors=K, neighbor_radius=0.2)
        w = _cotangent(T, E, A, A)
        for spec in (True, False):
            st = make_stepper(cfgs, world, 0.05, S, torch.float32)
            st.use_specialised = spec
            hip = hip_run(st, s0, acts, w, np.float32)
            orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
            _check(f"pad A={A} spec={spec}", hip, orc, state_exact=True)


def test_listed_neighbours_beyond_contact_reach():
    """Lists wider than any contact (neighbour radius 0.35) in dense envs with per-agent
    radii from 0.02 to 0.12 and truncated lists: the forward visits only the listed
    neighbours within the env's contact bound (the largest radius of the env sets it), so
    this case has listed pairs on both sides of every agent's reach, and agents whose
    largest-radius neighbour decides the bound.  States bit-exact with the oracle,
    gradients 1e-5, generic kernels in velocity and acceleration mode."""
    E, A, T, S = 160, 12, 8, 3
    rng = np.random.default_rng(11)
    radii = np.linspace(0.02, 0.12, A)[rng.permutation(A)]
    for mode in (ControlMode.VELOCITY, ControlMode.ACCELERATION):
        cfgs = [AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=mode, radius=float(r),
                            max_speed=1.0, max_accel=2.0) for r in radii]
        world = WorldConfig(collision_k=80.0, collision_c=1.5, collision_margin=0.03,
                            max_neighbors=5, neighbor_radius=0.35, bounds=(-0.6, 0.6, -0.6, 0.6))
        s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)),
                         "vel": 0.2 * rng.normal(size=(E, A, 2))}).astype(np.float32)
        acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
        w = _cotangent(T, E, A, 13)
        st = make_stepper(cfgs, world, 0.05, S, torch.float32)
        st.use_specialised = False
        hip = hip_run(st, s0, acts, w, np.float32)
        orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
        _check(f"wide lists {mode.name}", hip, orc, state_exact=True)


@pytest.mark.parametrize("E,A", [(13, 5), (40, 16), (9, 64)])
def test_obstacle_worlds_across_env_widths(E, A):
    """2-D fleets among static obstacles at every env width the two-wave forward serves
    (pad lanes and a partial last workgroup at A = 5, four envs per wave at A = 16, one
    at A = 64): diff-drive, bicycle and holonomic agents, circles, boxes and segments,
    soft walls.  States bit-exact with the float32 oracle, gradients 1e-5."""
    T, S = 6, 3
    rng = np.random.default_rng(E * 7 + A)
    models = (DynamicsModel.DIFF_DRIVE, DynamicsModel.KINEMATIC_BICYCLE, DynamicsModel.HOLONOMIC)
    cfgs = [AgentConfig(model=models[a % 3], radius=0.05) for a in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0), max_neighbors=min(16, A))
    n = 6
    obs = {"pos": rng.uniform(-1, 1, size=(E, n, 2)),
           "radius": np.r_[rng.uniform(0.05, 0.2, 2), np.zeros(2), np.full(2, 0.05)],
           "type": np.r_[np.zeros(2), np.ones(2), np.full(2, 2)].astype(np.int32),
           "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
           "half": np.r_[np.zeros((2, 2)), rng.uniform(0.05, 0.3, size=(2, 2)),
                         np.c_[rng.uniform(0.1, 0.4, 2), np.zeros(2)]]}
    s0 = pack_state({"pos": rng.uniform(-1, 1, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cotangent(T, E, A, 5, scale=0.1)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32, obs=obs)
    _check(f"obstacles E={E} A={A}", hip, orc, state_exact=True)


@pytest.mark.parametrize("n", [3, 7, 40])
def test_obstacle_counts_across_forward_layouts(n):
    """Obstacle counts from a few to more than a wave's agents: 3, 7 (an odd count) and 40
    obstacles per env, circles, boxes and segments in turn, soft walls, 12 agents of the
    three 2-D models.  States bit-exact with the float32 oracle, gradients 1e-5."""
    E, A, T, S = 9, 12, 5, 2
    rng = np.random.default_rng(100 + n)
    models = (DynamicsModel.DIFF_DRIVE, DynamicsModel.KINEMATIC_BICYCLE, DynamicsModel.HOLONOMIC)
    cfgs = [AgentConfig(model=models[a % 3], radius=0.05) for a in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0), max_neighbors=8)
    kind = np.arange(n) % 3
    half = np.zeros((n, 2))
    half[kind == 1] = rng.uniform(0.05, 0.3, size=(int((kind == 1).sum()), 2))
    half[kind == 2, 0] = rng.uniform(0.1, 0.4, size=int((kind == 2).sum()))
    obs = {"pos": rng.uniform(-1, 1, size=(E, n, 2)),
           "radius": np.where(kind == 0, rng.uniform(0.05, 0.2, n), np.where(kind == 2, 0.05, 0.0)),
           "type": kind.astype(np.int32),
           "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
           "half": half}
    s0 = pack_state({"pos": rng.uniform(-1, 1, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cotangent(T, E, A, 6, scale=0.1)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32, obs=obs)
    _check(f"obstacles n={n}", hip, orc, state_exact=True)
