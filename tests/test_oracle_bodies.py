"""Pins of the oracle's movable-body pass (obstacle_dynamics_kernel, disc variant,
swarp/core/bodies.py:367-568) and of its hand-written adjoint.

The reference never tapes the body pass, so no reference gradient exists for it: the
adjoint is pinned by central finite differences of the oracle's own forward (fp64).  The
forward is pinned by closed forms (one substep of one contact, computed here from the
contact law's formula), by Newton's third law (with zero drag the agents' and bodies'
momentum is conserved exactly up to rounding), by rigidity of compound bodies, and by the
behaviours the reference's own tests check (tests/unit/test_obstacle_kinds.py:74-215):
a head-on push moves a circle along the push without deflecting or spinning it, an
off-centre push spins a compound body, drag bounds a pushed body, scenery stops it.
"""

import numpy as np
import pytest

from cases import body_seed_np, holo, obstacles_np, oracle_cfg, params_of
from oracle.oracle import Oracle, pack_state
from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, WorldConfig

O = Oracle(np.float64)
MOVABLE = 1


def _world(**kw):
    base = dict(collisions=True, collision_k=1000.0, collision_c=20.0, collision_margin=0.01,
                bounds=(-2.0, 2.0, -2.0, 2.0))
    base.update(kw)
    return WorldConfig(**base)


def _agents(n, mode=ControlMode.VELOCITY, radius=0.05, big=False):
    v = 100.0 if big else 1.0
    return [AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=mode, radius=radius,
                        max_speed=v, max_accel=v) for _ in range(n)]


def _circles(E, centers, radius, kind, body=None, off=None, mass=None, inertia=None, vel=None):
    n = len(centers)
    pos = np.broadcast_to(np.asarray(centers, dtype=np.float64), (E, n, 2)).copy()
    d = {"pos": pos, "radius": np.full(n, radius) if np.isscalar(radius) else np.asarray(radius),
         "kind": np.asarray(kind, dtype=np.int32)}
    if body is not None:
        d["body"] = np.asarray(body, dtype=np.int32)
    if off is not None:
        d["body_off"] = np.asarray(off, dtype=np.float64)
    if mass is not None:
        d["mass"] = np.asarray(mass, dtype=np.float64)
    if inertia is not None:
        d["inertia"] = np.asarray(inertia, dtype=np.float64)
    if vel is not None:
        d["vel"] = np.broadcast_to(np.asarray(vel, dtype=np.float64), (E, n, 2)).copy()
    return obstacles_np(d, E)


def _cross(E, center, d=0.2, r=0.1, mass=1.0):
    """Config 5's body: 5 circles in a rigid cross, the centre circle as the root."""
    offs = np.array([[0, 0], [d, 0], [-d, 0], [0, d], [0, -d]], dtype=np.float64)
    inertia = sum(0.5 * (mass / 5) * r * r + (mass / 5) * (o @ o) for o in offs)
    return _circles(E, np.asarray(center) + offs, r, [MOVABLE] * 5, body=[0] * 5, off=offs,
                    mass=[mass] * 5, inertia=[inertia] * 5)


def _run(cfgs, world, dt, S, s0, acts, ob):
    E = s0.shape[0]
    cfg = oracle_cfg(cfgs, world, dt, S, E, acts.shape[-1])
    p, t, m = params_of(cfgs)
    return O.rollout_ob(cfg, p, t, m, ob, s0, body_seed_np(ob), acts)


def _pair_force(d, rv, md, k, c, dd):
    """The contact law's formula (swarp/core/collisions.py:108-143), written directly."""
    dist = max(np.sqrt(d @ d), 1e-5)
    ov = md - dist
    if ov <= 0:
        return np.zeros(2)
    n = d / dist
    return max((k * ov - c * (rv @ n)) / dd, 0.0) * n


def test_one_contact_one_substep_closed_form():
    """Agent at the origin moving +x into a circle body 0.15 away: the body's new velocity
    is (v + R/m sub_dt)(1 - lin_damping sub_dt) with R the negated agent-side force."""
    world = _world(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    cfgs = _agents(1, radius=0.1)
    ob = _circles(1, [[0.15, 0.0]], 0.1, [MOVABLE], mass=[2.0], inertia=[0.3])
    s0 = pack_state({"pos": [[[0.0, 0.0]]], "vel": [[[0.3, 0.0]]]})
    acts = np.array([[[[0.3, 0.0]]]])
    dt = 0.01
    _, obo = _run(cfgs, world, dt, 1, s0, acts, ob)
    dd = 1.0 + 1.0 * dt / 1.0
    f_agent = _pair_force(np.array([-0.15, 0.0]), np.array([0.3, 0.0]), 0.22, 100.0, 1.0, dd)
    R = -f_agent
    decay = 1.0 - 10.0 * dt
    v = (R / 2.0 * dt) * decay
    body = obo[0, 0, 6:12]
    assert body[3] == pytest.approx(v[0], rel=1e-14) and body[4] == 0.0
    assert body[0] == pytest.approx(0.15 + v[0] * dt, rel=1e-14)
    assert body[2] == 0.0 and body[5] == 0.0, "a head-on push on a circle spun it"
    shape = obo[0, 0, 0:6]
    np.testing.assert_array_equal(shape[[0, 1, 3, 4]], body[[0, 1, 3, 4]])


def test_newton_third_law_conserves_momentum():
    """With zero drag and zero commands (acceleration mode) every contact impulse appears
    once on each side: total momentum of agents and bodies is conserved."""
    world = _world(collision_k=200.0, collision_c=2.0, bounds=None, obstacle_linear_damping=0.0)
    cfgs = _agents(3, mode=ControlMode.ACCELERATION, radius=0.08, big=True)
    ob = _cross(1, [0.0, 0.0], mass=1.5)
    s0 = pack_state({"pos": [[[-0.38, 0.02], [0.1, 0.35], [0.31, -0.05]]],
                     "vel": [[[0.8, 0.0], [0.0, -0.6], [-0.5, 0.1]]]})
    acts = np.zeros((20, 1, 3, 2))
    st, obo = _run(cfgs, world, 0.05, 4, s0, acts, ob)
    p0 = s0[0, :, 3:5].sum(0) * 1.0
    p1 = st[-1, 0, :, 3:5].sum(0) * 1.0 + 1.5 * obo[-1, 0, 30 + 3:30 + 5]
    assert np.abs(obo[-1, 0, 30 + 3:30 + 5]).max() > 1e-2, "the body was never pushed"
    np.testing.assert_allclose(p1, p0, rtol=0, atol=1e-12)


def test_compound_body_stays_rigid_and_spins_off_centre():
    """(tests/unit/test_obstacle_kinds.py:172-203) every shape stays at body + R(angle)
    offset with the body's angle; an off-centre push rotates the body."""
    world = _world()
    cfgs = _agents(1)
    ob = _cross(1, [0.0, 0.0], mass=1.0)
    s0 = pack_state({"pos": [[[-0.45, 0.12]]]})
    acts = np.broadcast_to(np.array([1.0, 0.0]), (60, 1, 1, 2)).copy()
    _, obo = _run(cfgs, world, 0.05, 4, s0, acts, ob)
    last = obo[-1, 0]
    body = last[30:36]
    offs = ob["body_off"]
    ca, sa = np.cos(body[2]), np.sin(body[2])
    for s in range(5):
        want = body[:2] + np.array([ca * offs[s, 0] - sa * offs[s, 1],
                                    sa * offs[s, 0] + ca * offs[s, 1]])
        np.testing.assert_allclose(last[6 * s:6 * s + 2], want, rtol=0, atol=1e-12)
        assert last[6 * s + 2] == body[2] and last[6 * s + 5] == body[5]
    assert body[0] > 0.02, "compound body was not pushed"
    assert abs(body[2]) > 1e-4, "off-centre push did not rotate the body"


def test_head_on_push_and_drag_and_scenery():
    """(tests/unit/test_obstacle_kinds.py:87-170) a circle pushed head-on moves along the
    push and does not spin; more drag, slower body; immovable scenery stops it."""
    cfgs = _agents(1)
    s0 = pack_state({"pos": [[[-0.4, 0.0]]]})
    acts = np.broadcast_to(np.array([1.0, 0.0]), (80, 1, 1, 2)).copy()
    vmax = {}
    for damp in (2.0, 40.0):
        ob = _circles(1, [[0.0, 0.0], [1.2, 0.0]], 0.1, [MOVABLE, 0], mass=[1.0, 1.0],
                      inertia=[0.01, 1.0])
        _, obo = _run(cfgs, _world(obstacle_linear_damping=damp), 0.05, 4, s0, acts, ob)
        assert np.all(obo[:, 0, 1] == 0.0) and np.all(obo[:, 0, 2] == 0.0), "deflected or spun"
        np.testing.assert_array_equal(obo[:, 0, 6:8], np.broadcast_to([1.2, 0.0], (80, 2)))
        assert 0.0 < obo[-1, 0, 0] < 1.2, "movable circle passed through the scenery"
        vmax[damp] = obo[:, 0, 3].max()
    assert vmax[40.0] < vmax[2.0]


def test_clamp_bounds_keeps_the_body_inside():
    """bounds_mode "clamp": the whole body stays inside and a clamped axis loses its
    velocity (swarp/core/bodies.py:514-537)."""
    world = _world(bounds=(-0.5, 0.5, -2.0, 2.0), bounds_mode="clamp")
    cfgs = _agents(1)
    ob = _cross(1, [0.1, 0.0])
    s0 = pack_state({"pos": [[[-0.3, 0.0]]]})
    acts = np.broadcast_to(np.array([1.0, 0.0]), (60, 1, 1, 2)).copy()
    _, obo = _run(cfgs, world, 0.05, 4, s0, acts, ob)
    ext = np.sqrt(0.2 * 0.2 + 0.0 * 0.0) + 0.1
    x = obo[:, 0, 30]
    assert x.max() <= 0.5 - ext + 1e-12
    hit = np.nonzero(x == 0.5 - ext)[0]
    assert hit.size > 0, "the body never reached the bound"
    assert np.all(obo[hit, 0, 33] == 0.0)


def test_determinism():
    world = _world()
    cfgs = _agents(3)
    rng = np.random.default_rng(4)
    s0 = pack_state({"pos": rng.uniform(-0.6, 0.6, size=(4, 3, 2))})
    acts = rng.uniform(-1, 1, size=(12, 4, 3, 2))
    ob = _cross(4, [0.0, 0.0])
    a = _run(cfgs, world, 0.05, 4, s0, acts, ob)
    b = _run(cfgs, world, 0.05, 4, s0, acts, ob)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def _fd_bodies(cfgs, world, dt, S, s0, acts, ob, eps=1e-6, tol=2e-7, seed=0):
    E = s0.shape[0]
    cfg = oracle_cfg(cfgs, world, dt, S, E, acts.shape[-1])
    p, t, m = params_of(cfgs)
    ob0 = body_seed_np(ob)
    rng = np.random.default_rng(seed)
    T = acts.shape[0]
    w_st = rng.normal(size=(T,) + s0.shape)
    w_st[..., 5:] = 0.0
    w_ob = rng.normal(size=(T,) + ob0.shape)

    def loss(s0_, ob0_, acts_):
        st, obo = O.rollout_ob(cfg, p, t, m, ob, s0_, ob0_, acts_)
        return float((w_st * st).sum() + (w_ob * obo).sum())

    st, obo = O.rollout_ob(cfg, p, t, m, ob, s0, ob0, acts)
    g0, gob0, ga = O.rollout_adj_ob(cfg, p, t, m, ob, s0, ob0, acts, st, obo, w_st, None, w_ob,
                                    None)

    def check(name, x, g, fn):
        for i in np.ndindex(*x.shape):
            a, b = x.copy(), x.copy()
            a[i] += eps
            b[i] -= eps
            fd = (fn(a) - fn(b)) / (2 * eps)
            assert abs(fd - g[i]) <= tol * max(1.0, abs(fd)), f"{name}{i}: fd {fd} vs adj {g[i]}"

    check("actions", acts, ga, lambda a: loss(s0, ob0, a))
    sub = [i for i in np.ndindex(*s0.shape) if i[-1] in (0, 1, 3, 4)]
    for i in sub:
        a, b = s0.copy(), s0.copy()
        a[i] += eps
        b[i] -= eps
        fd = (loss(a, ob0, acts) - loss(b, ob0, acts)) / (2 * eps)
        assert abs(fd - g0[i]) <= tol * max(1.0, abs(fd)), f"state0{i}: fd {fd} vs adj {g0[i]}"
    check("ob0", ob0, gob0, lambda b: loss(s0, b, acts))
    return st, obo


def test_body_adjoint_matches_finite_differences():
    """Agents pushing a 3-circle compound body into a second (single-circle) body and
    a static circle: every adjoint path of the body pass (reactions and their levers,
    body-body contacts with a movable and a static circle, drag, re-installed shapes)."""
    world = _world(collision_k=60.0, collision_c=0.8, collision_margin=0.02, bounds=None,
                   obstacle_linear_damping=3.0, obstacle_angular_damping=2.0)
    cfgs = _agents(3, mode=ControlMode.ACCELERATION, radius=0.07, big=True)
    offs = [[0.0, 0.0], [0.16, 0.0], [0.0, 0.16], [0.0, 0.0], [0.0, 0.0]]
    centers = [[0.0, 0.0], [0.16, 0.0], [0.0, 0.16], [0.33, 0.05], [-0.05, 0.35]]
    ob = _circles(1, centers, [0.08, 0.08, 0.08, 0.09, 0.08], [MOVABLE, MOVABLE, MOVABLE,
                                                              MOVABLE, 0],
                  body=[0, 0, 0, 3, 4], off=offs, mass=[0.7, 0.7, 0.7, 0.5, 1.0],
                  inertia=[0.05, 0.05, 0.05, 0.02, 1.0],
                  vel=[[0.05, -0.02]] * 3 + [[-0.1, 0.0], [0.0, 0.0]])
    s0 = pack_state({"pos": [[[-0.13, 0.03], [0.12, -0.13], [0.2, 0.2]]],
                     "vel": [[[0.4, 0.05], [-0.1, 0.3], [-0.2, -0.2]]]})
    rng = np.random.default_rng(7)
    acts = 0.5 * rng.normal(size=(3, 1, 3, 2))
    st, obo = _fd_bodies(cfgs, world, 0.05, 2, s0, acts, ob)
    assert np.abs(obo[-1, 0, 30 + 5]) > 1e-4, "the compound body never turned"


def test_body_pass_reads_its_own_parameter_rows():
    """With per-env agent rows the reference's body pass still reads the shared table
    (swarp/core/stepper.py:961-964): the body's reaction uses that table's radius and mass,
    while the agent's own force (and so its step) uses the agent's row."""
    world = _world(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    cfgs = _agents(1, radius=0.1)
    ob = _circles(1, [[0.15, 0.0]], 0.1, [MOVABLE], mass=[2.0], inertia=[0.3])
    s0 = pack_state({"pos": [[[0.0, 0.0]]], "vel": [[[0.3, 0.0]]]})
    acts = np.array([[[[0.3, 0.0]]]])
    dt = 0.01
    cfg = oracle_cfg(cfgs, world, dt, 1, 1, 2)
    p, t, m = params_of(cfgs)
    shared = p.copy()
    shared[0, 0], shared[0, 1] = 0.12, 3.0  # the body pass's radius and mass
    ob_b = dict(ob, body_params=shared)
    st_a, obo_a = O.rollout_ob(cfg, p, t, m, ob, s0, body_seed_np(ob), acts)
    st_b, obo_b = O.rollout_ob(cfg, p, t, m, ob_b, s0, body_seed_np(ob), acts)
    np.testing.assert_array_equal(st_a, st_b)  # the agent side reads its own row
    dd = 1.0 + 1.0 * dt / 3.0
    R = -_pair_force(np.array([-0.15, 0.0]), np.array([0.3, 0.0]), 0.24, 100.0, 1.0, dd)
    v = (R / 2.0 * dt) * (1.0 - 10.0 * dt)
    assert obo_b[0, 0, 6 + 3] == pytest.approx(v[0], rel=1e-14)
    assert obo_b[0, 0, 6 + 3] != obo_a[0, 0, 6 + 3]
    # the same table as the agents' rows changes nothing
    _, obo_c = O.rollout_ob(cfg, p, t, m, dict(ob, body_params=p), s0, body_seed_np(ob), acts)
    np.testing.assert_array_equal(obo_c, obo_a)


def test_drone_fleet_pushes_a_body():
    """Drones take part in the body pass by their planar position and velocity (the disc
    variant reads pos / vel only, swarp/core/bodies.py:384-393): a drone flying into a
    circle body pushes it, and the body's adjoint matches finite differences."""
    world = _world(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0)]
    ob = _circles(1, [[0.17, 0.0]], 0.1, [MOVABLE], mass=[2.0], inertia=[0.3])
    s0 = pack_state({"pos": [[[0.0, 0.0]]], "vel": [[[0.5, 0.05]]], "z": [[1.0]]})
    acts = np.full((6, 1, 1, 4), 2.5)
    st, obo = _run(cfgs, world, 0.02, 2, s0, acts, ob)
    assert obo[-1, 0, 6 + 3] > 1e-3, "the drone never pushed the body"
    cfg = oracle_cfg(cfgs, world, 0.02, 2, 1, 4)
    p, t, m = params_of(cfgs)
    b0 = body_seed_np(ob)
    rng = np.random.default_rng(3)
    w_st = rng.normal(size=st.shape)
    w_ob = rng.normal(size=obo.shape)
    _, _, ga = O.rollout_adj_ob(cfg, p, t, m, ob, s0, b0, acts, st, obo, w_st, None, w_ob, None)

    def loss(a):
        s, o = O.rollout_ob(cfg, p, t, m, ob, s0, b0, a)
        return float((w_st * s).sum() + (w_ob * o).sum())

    h = 1e-6
    for idx in [(0, 0, 0, 0), (2, 0, 0, 1), (4, 0, 0, 3), (5, 0, 0, 2)]:
        ap, am = acts.copy(), acts.copy()
        ap[idx] += h
        am[idx] -= h
        fd = (loss(ap) - loss(am)) / (2 * h)
        assert ga[idx] == pytest.approx(fd, rel=2e-6, abs=1e-9)


def _shapes(E, centers, radius, types, half, kind, body, off, mass, inertia, angle=None):
    """Obstacles of any shape type (0 circle, 1 box, 2 segment) with body fields."""
    n = len(centers)
    d = {"pos": np.broadcast_to(np.asarray(centers, dtype=np.float64), (E, n, 2)).copy(),
         "radius": np.asarray(radius, dtype=np.float64), "type": np.asarray(types, np.int32),
         "half": np.asarray(half, dtype=np.float64), "kind": np.asarray(kind, np.int32),
         "body": np.asarray(body, np.int32), "body_off": np.asarray(off, dtype=np.float64),
         "mass": np.asarray(mass, dtype=np.float64),
         "inertia": np.asarray(inertia, dtype=np.float64)}
    if angle is not None:
        d["angle"] = np.broadcast_to(np.asarray(angle, dtype=np.float64), (E, n)).copy()
    return obstacles_np(d, E)


def test_box_body_off_centre_push_closed_form():
    """One substep of a disc agent pressing on a box body's face off its centre line
    (swarp/core/bodies.py:80-127): the force on the body is minus box_force, the lever
    runs from the body origin to the agent's centre (r = p - c), so the body spins."""
    world = _world(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    cfgs = _agents(1, radius=0.1)
    ob = _shapes(1, [[0.2, 0.0]], [0.0], [1], [[0.1, 0.05]], [MOVABLE], [0], [[0.0, 0.0]],
                 [2.0], [0.3])
    s0 = pack_state({"pos": [[[0.0, 0.03]]], "vel": [[[0.3, 0.0]]]})
    acts = np.array([[[[0.3, 0.0]]]])
    dt = 0.01
    _, obo = _run(cfgs, world, dt, 1, s0, acts, ob)
    dd = 1.0 + 1.0 * dt / 1.0
    # face x = -0.1 of the box: normal (-1, 0), overlap = reach - 0.1 = 0.02, vn = -0.3
    coef = (100.0 * 0.02 - 1.0 * (-0.3)) / dd
    R = np.array([coef, 0.0])                      # minus the agent's force coef * (-1, 0)
    lever = np.array([0.0 - 0.2, 0.03 - 0.0])      # r = p - c, the root's offset is 0
    tau = lever[0] * R[1] - lever[1] * R[0]
    decay, adecay = 1.0 - 10.0 * dt, 1.0 - 10.0 * dt
    body = obo[0, 0, 6:12]
    assert body[3] == pytest.approx(R[0] / 2.0 * dt * decay, rel=1e-13) and body[4] == 0.0
    assert body[5] == pytest.approx(tau / 0.3 * dt * adecay, rel=1e-13) and body[5] < 0.0
    assert body[2] == pytest.approx(body[5] * dt, rel=1e-13)


def test_segment_body_and_box_scenery():
    """A capsule body pushed along its axis into static box scenery: the agent's push
    moves it, and the box stops it.  The reference's body-body term takes a round body as
    a disc of its radius at its centre against a box (swarp/core/bodies.py:238-242), so
    the capsule's centre, not its end, is what the box holds back."""
    world = _world(collision_k=200.0, collision_c=2.0, collision_margin=0.01, bounds=None)
    cfgs = _agents(1, radius=0.06)
    s0 = pack_state({"pos": [[[-0.35, 0.0]]]})
    acts = np.broadcast_to(np.array([1.0, 0.0]), (60, 1, 1, 2)).copy()
    x = {}
    for box_x in (0.7, 5.0):
        ob = _shapes(1, [[0.0, 0.0], [box_x, 0.0]], [0.05, 0.0], [2, 1],
                     [[0.2, 0.0], [0.05, 0.4]], [MOVABLE, 0], [0, 1], [[0.0, 0.0], [0.0, 0.0]],
                     [1.0, 1.0], [0.05, 1.0])
        _, obo = _run(cfgs, world, 0.05, 4, s0, acts, ob)
        x[box_x] = obo[:, 0, 0]
        np.testing.assert_array_equal(obo[:, 0, 6:12], np.broadcast_to(obo[0, 0, 6:12], (60, 6)))
    assert x[5.0][-1] > 2.0, "the capsule was not pushed"
    assert x[0.7].max() < 0.7 and x[0.7][-1] < 0.6, "the box did not stop the capsule"


def test_box_and_segment_body_adjoint_matches_finite_differences():
    """Every adjoint path of box and segment shapes in the body pass: agent reactions on a
    box + capsule compound body (lever p - c on the box, the closest core point on the
    capsule), the body-body terms box vs circle, box vs capsule, capsule vs box, circle vs
    box, and the agents' own forces from the moving box and capsule shapes."""
    world = _world(collision_k=60.0, collision_c=0.8, collision_margin=0.02, bounds=None,
                   obstacle_linear_damping=3.0, obstacle_angular_damping=2.0)
    cfgs = _agents(3, mode=ControlMode.ACCELERATION, radius=0.07, big=True)
    th = 0.3
    off1 = np.array([0.05, 0.21])
    c1 = np.array([np.cos(th) * off1[0] - np.sin(th) * off1[1],
                   np.sin(th) * off1[0] + np.cos(th) * off1[1]])
    centers = [[0.0, 0.0], list(c1), [c1[0] + 0.01, c1[1] + 0.1], [0.0, -0.2], [0.2, -0.1]]
    ob = _shapes(1, centers, [0.0, 0.04, 0.0, 0.08, 0.06], [1, 2, 1, 0, 0],
                 [[0.12, 0.07], [0.15, 0.0], [0.06, 0.05], [0.0, 0.0], [0.0, 0.0]],
                 [MOVABLE, MOVABLE, MOVABLE, 0, MOVABLE], [0, 0, 2, 3, 4],
                 [[0.0, 0.0], list(off1), [0.0, 0.0], [0.0, 0.0], [0.0, 0.0]],
                 [0.8, 0.8, 0.5, 1.0, 0.4], [0.04, 0.04, 0.02, 1.0, 0.01],
                 angle=[th, th, -0.4, 0.0, 0.0])
    s0 = pack_state({"pos": [[[-0.24, 0.05], [-0.1, 0.36], [0.2, -0.26]]],
                     "vel": [[[0.5, 0.0], [0.1, -0.4], [0.0, 0.3]]]})
    acts = np.random.default_rng(8).normal(size=(5, 1, 3, 2)) * 0.5
    st, obo = _fd_bodies(cfgs, world, 0.05, 2, s0, acts, ob, tol=5e-7, seed=3)
    assert np.abs(obo[-1, 0, 6 * 5 + 5]).max() > 1e-4, "the compound body never turned"
