"""Pins of the oracle's box-agent restatement (oriented-rectangle footprints).

Forward: closed forms the geometry fixes (face overlap of two boxes, a box corner at a
small gap from a face, a box against a circle / box / capsule obstacle, the support
extent of a rotated box against a soft wall, the footprint clamp of a rotated box) and
the pair law's action = reaction, bit for bit, that the reference's lower-index-as-A rule
guarantees (swarp/core/collisions.py:489-541).  Reverse: the oracle's dual-number
Jacobians against central finite differences of its own forward in fp64, across the
regimes of obb_contact (overlap, vertex distance), every shape pairing, obstacles,
walls and the footprint clamp.  Geometry follows swarp/core/collisions.py:266-688 and
swarp/dynamics/kernels.py:79-99; the reference's own tests of it are
tests/unit/test_box_agents.py (not runnable here: they need warp-lang).
"""

import math

import numpy as np
import pytest

from cases import obstacles_np, oracle_cfg, params_of
from oracle.oracle import Oracle, pack_state
from swarp_amd.config import AgentConfig, AgentShape, ControlMode, DynamicsModel, WorldConfig
from test_oracle_gradcheck import _fd_check

O = Oracle(np.float64)
K = 100.0
M = 0.025


def _box(hx, hy, model=DynamicsModel.HOLONOMIC, **kw):
    return AgentConfig(model=model, shape=AgentShape.BOX, half_extents=(hx, hy), radius=None, **kw)


def _disc(r, model=DynamicsModel.HOLONOMIC, **kw):
    return AgentConfig(model=model, radius=r, **kw)


def _forces(configs, world, state, obs=None, dtype=np.float64):
    o = Oracle(dtype)
    E = state.shape[0]
    cfg = oracle_cfg(configs, world, 0.05, 1, E, 2)
    p, t, m = params_of(configs)
    return o.forces(cfg, p, t, m, obstacles_np(obs, E), state.astype(dtype))


def _world(**kw):
    base = dict(collision_k=K, collision_c=0.0, collision_margin=M, max_neighbors=8)
    base.update(kw)
    return WorldConfig(**base)


def test_face_overlap_of_two_boxes():
    """Aligned boxes overlapping by 0.05 along x: the least-overlap axis is A's x face,
    the normal points from B to A, overlap = margin + 0.05 (collisions.py:400-447)."""
    cfgs = [_box(0.2, 0.1), _box(0.2, 0.1)]
    s = pack_state({"pos": [[[0.0, 0.0], [0.35, 0.02]]]})
    F = _forces(cfgs, _world(), s)
    want = K * (M + 0.05)
    assert F[0, 0, 0] == pytest.approx(-want, rel=1e-12) and F[0, 0, 1] == 0.0
    assert np.array_equal(F[0, 1], -F[0, 0])


def test_face_overlap_damper_reads_the_contact_point():
    """The damper of the face overlap above reads the material-point velocities at the
    contact point: on A's right face (x = 0.2), midway along the overlap of the two
    boxes' extents across it (y in [-0.08, 0.1] -> 0.01).  A spins at wa, B moves and
    spins; the closing speed along n = (-1, 0) follows from v + w x (x - c)."""
    cfgs = [_box(0.2, 0.1), _box(0.2, 0.1)]
    c, wa, wb, vb = 2.0, 3.0, -1.5, np.array([0.4, 0.7])
    s = pack_state({"pos": [[[0.0, 0.0], [0.35, 0.02]]], "vel": [[[0.0, 0.0], vb]],
                    "ang_vel": [[wa, wb]]})
    F = _forces(cfgs, _world(collision_c=c), s)
    x = np.array([0.2, 0.01])
    ra, rb = x - np.array([0.0, 0.0]), x - np.array([0.35, 0.02])
    vpa = np.array([-wa * ra[1], wa * ra[0]])
    vpb = vb + np.array([-wb * rb[1], wb * rb[0]])
    vn = float((vpa - vpb) @ np.array([-1.0, 0.0]))
    coef = (K * (M + 0.05) - c * vn) / (1.0 + c * 0.05 / 1.0)
    assert F[0, 0, 0] == pytest.approx(-coef, rel=1e-12)


def test_disc_box_damper_reads_the_box_surface():
    """A disc over a spinning box's top face: the closing velocity is taken against the
    box's surface point under the disc, v_b + w_b x (q - c_b) with q = (0.15, 0.1)."""
    cfgs = [_disc(0.05), _box(0.2, 0.1)]
    c, vd, vb, wb = 1.0, np.array([0.2, -0.3]), np.array([0.1, 0.25]), 2.0
    s = pack_state({"pos": [[[0.15, 0.16], [0.0, 0.0]]], "vel": [[vd, vb]], "ang_vel": [[0.0, wb]]})
    F = _forces(cfgs, _world(collision_c=c), s)
    q = np.array([0.15, 0.1])
    vs = vb + np.array([-wb * q[1], wb * q[0]])
    vn = float((vd - vs) @ np.array([0.0, 1.0]))
    coef = (K * (0.05 + M - 0.06) - c * vn) / (1.0 + c * 0.05 / 1.0)
    assert F[0, 0, 1] == pytest.approx(coef, rel=1e-12) and F[0, 0, 0] == 0.0
    assert np.array_equal(F[0, 1], -F[0, 0])


def test_corner_at_a_small_gap():
    """A box turned 45 degrees points a corner at an aligned box's face from 0.01 away
    (inside the margin): SAT reports a positive gap, the vertex pass finds the exact
    distance, and the force is k (margin - 0.01) along the face normal (:384-398)."""
    h = 0.1
    c = h * math.sqrt(2.0)
    cfgs = [_box(h, h), _box(0.2, 0.2)]
    s = pack_state({"pos": [[[0.0, 0.0], [c + 0.01 + 0.2, 0.0]]], "theta": [[math.pi / 4, 0.0]]})
    F = _forces(cfgs, _world(), s)
    assert F[0, 0, 0] == pytest.approx(-K * (M - 0.01), rel=1e-9)
    assert abs(F[0, 0, 1]) < 1e-9
    assert np.array_equal(F[0, 1], -F[0, 0])


def test_disc_against_a_box_agent():
    """A disc centre 0.06 from a box's long face: box_force with the disc as the point on
    the disc, its negation on the box (:515-527)."""
    cfgs = [_disc(0.05), _box(0.2, 0.1)]
    s = pack_state({"pos": [[[0.0, 0.16], [0.0, 0.0]]]})
    F = _forces(cfgs, _world(), s)
    want = K * (0.05 + M - 0.06)
    assert F[0, 0, 1] == pytest.approx(want, rel=1e-12) and F[0, 0, 0] == 0.0
    assert np.array_equal(F[0, 1], -F[0, 0])


@pytest.mark.parametrize("seed", range(4))
def test_pair_forces_cancel_exactly(seed):
    """Both threads of a pair evaluate one contact with the lower index as box A (or the
    disc as the point): with equal masses the two forces are exact negatives, in both
    precisions, whatever the poses (:489-541)."""
    rng = np.random.default_rng(seed)
    for a_box, b_box in ((True, True), (True, False), (False, True)):
        cfgs = [_box(0.15, 0.08) if a_box else _disc(0.07),
                _box(0.12, 0.1) if b_box else _disc(0.06)]
        pos = rng.uniform(-0.12, 0.12, size=(8, 2, 2))
        s = pack_state({"pos": pos, "theta": rng.uniform(-np.pi, np.pi, size=(8, 2)),
                        "vel": rng.normal(size=(8, 2, 2)), "ang_vel": rng.normal(size=(8, 2))})
        for dt in (np.float64, np.float32):
            F = _forces(cfgs, _world(collision_c=2.0), s, dtype=dt)
            assert np.array_equal(F[:, 1], -F[:, 0])
            assert np.count_nonzero(F) > 0


def test_box_agent_against_obstacles():
    """A box agent (0.2 x 0.1 half extents, heading 0) against one obstacle of each kind:
    a circle whose centre is 0.1 above its top face, a box overlapping its right face by
    0.02, a capsule whose core is 0.06 below its bottom face (:543-626)."""
    cfgs = [_box(0.2, 0.1)]
    w = _world(collisions=False)
    s = pack_state({"pos": [[[0.0, 0.0]]]})
    circle = {"pos": [[[0.0, 0.2]]], "radius": [0.1], "type": [0]}
    F = _forces(cfgs, w, s, circle)
    assert F[0, 0, 0] == 0.0 and F[0, 0, 1] == pytest.approx(-K * (0.1 + M - 0.1), rel=1e-12)
    box = {"pos": [[[0.38, 0.0]]], "radius": [0.0], "type": [1], "half": [[0.2, 0.3]]}
    F = _forces(cfgs, w, s, box)
    assert F[0, 0, 0] == pytest.approx(-K * (M + 0.02), rel=1e-12) and F[0, 0, 1] == 0.0
    seg = {"pos": [[[0.05, -0.16]]], "radius": [0.05], "type": [2], "half": [[0.3, 0.0]]}
    F = _forces(cfgs, w, s, seg)
    assert abs(F[0, 0, 0]) < 1e-12
    assert F[0, 0, 1] == pytest.approx(K * (0.05 + M - 0.06), rel=1e-9)


def test_rotated_box_against_a_soft_wall():
    """The wall sees the support extent ex = hx |cos| + hy |sin| (:641-688)."""
    cfgs = [_box(0.2, 0.1)]
    w = _world(collisions=False, bounds=(-1.0, 1.0, -1.0, 1.0))
    th = 0.7
    s = pack_state({"pos": [[[-0.8, 0.0]]], "theta": [[th]]})
    F = _forces(cfgs, w, s)
    ex = 0.2 * abs(math.cos(th)) + 0.1 * abs(math.sin(th))
    assert F[0, 0, 0] == pytest.approx(K * (ex + M - 0.2), rel=1e-12) and F[0, 0, 1] == 0.0
    # damped and spinning: the wall's damper reads the velocity of the vertex touching it
    c, v, w_ = 1.5, np.array([-0.3, 0.2]), 2.5
    s = pack_state({"pos": [[[-0.8, 0.0]]], "theta": [[th]], "vel": [[v]], "ang_vel": [[w_]]})
    F = _forces(cfgs, _world(collisions=False, collision_c=c, bounds=(-1.0, 1.0, -1.0, 1.0)), s)
    e0 = 0.2 * np.array([math.cos(th), math.sin(th)])
    e1 = 0.1 * np.array([-math.sin(th), math.cos(th)])
    verts = [e0 + e1, -e0 + e1, -e0 - e1, e0 - e1]
    r = min(verts, key=lambda q: q[0])  # the vertex reaching furthest toward -x
    vn = v[0] - w_ * r[1]
    coef = (K * (-r[0] + M - 0.2) - c * vn) / (1.0 + c * 0.05)
    assert F[0, 0, 0] == pytest.approx(coef, rel=1e-12)


def test_footprint_clamp():
    """A box turned to 1.2 rad driven into the right wall stops with its support extent
    against it (kernels.py:79-99); a disc in the same world keeps the radius inset."""
    cfgs = [_box(0.2, 0.1, max_speed=10.0), _disc(0.05, max_speed=10.0)]
    w = WorldConfig(collisions=False, bounds=(-0.5, 0.5, -0.5, 0.5), bounds_mode="clamp")
    cfg = oracle_cfg(cfgs, w, 0.1, 1, 1, 2)
    assert cfg["clamp_bounds"] == 2
    p, t, m = params_of(cfgs)
    s0 = pack_state({"pos": [[[0.3, 0.0], [0.4, 0.2]]], "theta": [[1.2, 0.0]]})
    tr = O.rollout(cfg, p, t, m, None, s0, np.array([[[[2.0, 0.0], [2.0, 0.0]]]]))
    ex = 0.2 * abs(math.cos(1.2)) + 0.1 * abs(math.sin(1.2))
    assert tr[0, 0, 0, 0] == 0.5 - ex
    assert tr[0, 0, 1, 0] == 0.5 - 0.05


def test_disc_past_a_box_corner():
    """A disc beyond a box's corner: the normal is the corner-to-centre diagonal and the
    depth uses the corner distance (the exterior SDF of box_force)."""
    cfgs = [_disc(0.08), _box(0.2, 0.1)]
    s = pack_state({"pos": [[[0.24, 0.14], [0.0, 0.0]]]})
    F = _forces(cfgs, _world(), s)
    d = 0.04 * math.sqrt(2.0)
    mag = K * (0.08 + M - d)
    assert F[0, 0] == pytest.approx([mag / math.sqrt(2.0)] * 2, rel=1e-9)
    assert np.array_equal(F[0, 1], -F[0, 0])


@pytest.mark.parametrize("phi", [0.3, 0.9, 1.4])
def test_capsule_end_cap_is_round(phi):
    """A box corner 0.04 from a capsule core's end, at angle phi: the end cap is a circle,
    so the push is radial with the same depth at every phi (obb_contact with the
    degenerate box (half_len, 0))."""
    seg = {"pos": [[[0.0, 0.0]]], "radius": [0.05], "type": [2], "half": [[0.25, 0.0]]}
    end = np.array([0.25, 0.0])
    u = np.array([math.cos(phi), math.sin(phi)])
    # an aligned 0.06-square whose lower-left corner sits at end + 0.04 u
    centre = end + 0.04 * u + 0.06
    F = _forces([_box(0.06, 0.06)], _world(collisions=False), pack_state({"pos": [[centre]]}), seg)
    assert F[0, 0] == pytest.approx(K * (0.05 + M - 0.04) * u, rel=1e-9, abs=1e-12)


def test_plus_crossing_is_detected():
    """Two thin boxes crossing in a '+': no corner of either lies inside the other, so
    only the separating-axis test sees the overlap; the push is along a face normal."""
    cfgs = [_box(0.25, 0.015), _box(0.25, 0.015)]
    s = pack_state({"pos": [[[0.0, 0.0], [0.02, 0.01]]], "theta": [[0.0, math.pi / 2]]})
    F = _forces(cfgs, _world(), s)
    assert np.linalg.norm(F[0, 0]) > 1.0
    assert np.array_equal(F[0, 1], -F[0, 0])
    assert min(abs(F[0, 0, 0]), abs(F[0, 0, 1])) < 1e-9


def test_rotation_and_translation_invariance():
    """Rotating and shifting a whole mixed scene (agents, obstacles, velocities) rotates
    every force with it."""
    cfgs = [_box(0.18, 0.09), _box(0.12, 0.07), _box(0.09, 0.09), _disc(0.07)]
    pos = np.array([[0.0, 0.0], [0.24, 0.1], [0.03, 0.19], [-0.22, -0.05]])
    th = np.array([0.25, -0.35, 1.0, 0.0])
    vel = np.array([[0.2, -0.1], [-0.3, 0.05], [0.1, 0.2], [0.4, 0.0]])
    om = np.array([0.6, -1.1, 1.8, 0.0])
    obs = {"pos": np.array([[[0.18, -0.19], [-0.28, 0.18], [0.4, 0.28]]]),
           "radius": [0.0, 0.03, 0.09], "type": [1, 2, 0],
           "half": [[0.14, 0.05], [0.18, 0.0], [0.0, 0.0]], "angle": np.array([[0.2, -0.5, 0.0]]),
           "vel": np.array([[[0.1, 0.0], [0.0, -0.2], [0.0, 0.1]]]),
           "ang_vel": np.array([[0.3, -0.4, 1.0]])}
    w = _world(collision_c=1.0, bounds=(-0.6, 0.6, -0.6, 0.6), collision_margin=0.02)
    w_free = _world(collision_c=1.0, collision_margin=0.02)
    s = pack_state({"pos": pos[None], "theta": th[None], "vel": vel[None], "ang_vel": om[None]})
    f0 = _forces(cfgs, w_free, s, obs)[0]
    assert (np.linalg.norm(f0, axis=-1) > 1e-3).sum() >= 3
    a, shift = 0.8, np.array([0.25, -0.4])
    r = np.array([[math.cos(a), -math.sin(a)], [math.sin(a), math.cos(a)]])
    obs1 = dict(obs, pos=obs["pos"] @ r.T + shift, angle=obs["angle"] + a, vel=obs["vel"] @ r.T)
    s1 = pack_state({"pos": (pos @ r.T + shift)[None], "theta": (th + a)[None],
                     "vel": (vel @ r.T)[None], "ang_vel": om[None]})
    f1 = _forces(cfgs, w_free, s1, obs1)[0]
    np.testing.assert_allclose(f1, f0 @ r.T, atol=1e-9, rtol=0)
    assert np.count_nonzero(_forces(cfgs, w, s, obs)) > 0


# ------------------------------------------------------------------ finite differences

def _rs(E, A, seed, spread, ang=True):
    rng = np.random.default_rng(seed)
    return pack_state({
        "pos": rng.uniform(-spread, spread, size=(E, A, 2)),
        "theta": rng.uniform(-np.pi, np.pi, size=(E, A)) if ang else np.zeros((E, A)),
        "vel": rng.normal(size=(E, A, 2)) * 0.3,
        "speed": rng.normal(size=(E, A)) * 0.3,
        "ang_vel": rng.normal(size=(E, A)) * 0.5,
    }), rng


def _dd(n, **kw):
    return [_box(0.12, 0.07, model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION,
                 max_speed=5.0, max_accel=5.0, max_ang_vel=8.0, max_ang_accel=8.0, **kw)
            for _ in range(n)]


def test_fd_box_pairs_overlapping():
    """Crowded diff-drive boxes: SAT overlap contacts, damped, two substeps."""
    s0, rng = _rs(2, 3, 1, 0.1)
    acts = rng.uniform(-1, 1, size=(2, 2, 3, 2))
    _fd_check(_dd(3), _world(collision_c=1.5), 0.05, 2, s0, acts, fields=(0, 1, 2, 3, 4, 5, 6))


def test_fd_box_pairs_within_margin():
    """Boxes a few millimetres apart: the vertex-distance regime of obb_contact."""
    cfgs = _dd(2)
    rng = np.random.default_rng(5)
    # B turned 45 degrees, its leftmost corner 6 mm from A's right face (A at heading 0)
    c, sn = math.cos(math.pi / 4), math.sin(math.pi / 4)
    corner = (-0.12 * c + 0.07 * sn, -0.12 * sn - 0.07 * c)  # -e0 + e1
    b = (0.12 + 0.006 - corner[0], 0.02 - corner[1])
    s0 = pack_state({"pos": [[[0.0, 0.0], list(b)]],
                     "theta": [[0.0, math.pi / 4]], "vel": rng.normal(size=(1, 2, 2)) * 0.1,
                     "speed": [[0.1, -0.1]], "ang_vel": [[0.2, -0.4]]})
    acts = rng.uniform(-0.5, 0.5, size=(2, 1, 2, 2))
    _fd_check(cfgs, _world(collision_margin=0.04, collision_c=1.0), 0.05, 2, s0, acts,
              fields=(0, 1, 2, 3, 4, 5, 6))


def test_fd_mixed_discs_and_boxes():
    """Discs (holonomic), diff-drive boxes and a bicycle box in one crowded env."""
    cfgs = [_disc(0.06, max_speed=5.0, max_accel=5.0, ctrl_mode=ControlMode.ACCELERATION),
            _disc(0.05, max_speed=5.0)] + _dd(2) + [
        _box(0.1, 0.05, model=DynamicsModel.KINEMATIC_BICYCLE, max_speed=5.0, max_accel=5.0,
             max_steer=1.0, l_f=0.16, l_r=0.14)]
    s0, rng = _rs(2, 5, 3, 0.15)
    acts = rng.uniform(-1, 1, size=(2, 2, 5, 2))
    _fd_check(cfgs, _world(collision_c=1.0, contact_max_overlap=0.05), 0.05, 2, s0, acts,
              fields=(0, 1, 2, 3, 4, 5, 6))


def test_fd_box_agents_obstacles_and_walls():
    """Boxes against a circle, a rotated box and a capsule, inside soft walls."""
    cfgs = _dd(3)
    obs = {"pos": [[[0.15, 0.0], [-0.2, 0.1], [0.0, -0.25]], [[0.1, 0.1], [-0.15, -0.1], [0.2, -0.2]]],
           "radius": [0.08, 0.0, 0.03], "type": [0, 1, 2],
           "angle": [0.0, 0.4, -0.3], "half": [[0.0, 0.0], [0.1, 0.06], [0.2, 0.0]],
           "vel": [[[0.0, 0.0], [0.1, -0.2], [0.0, 0.0]]] * 2, "ang_vel": [[0.0, 0.5, -0.3]] * 2}
    s0, rng = _rs(2, 3, 7, 0.22)
    acts = rng.uniform(-1, 1, size=(2, 2, 3, 2))
    w = _world(collision_c=1.0, bounds=(-0.32, 0.32, -0.32, 0.32))
    _fd_check(cfgs, w, 0.05, 2, s0, acts, obs=obs, fields=(0, 1, 2, 3, 4, 5, 6))


def test_fd_footprint_clamp():
    """Diff-drive boxes driven into the clamp: the position gradient stops and the heading
    picks up the footprint's dependence on it."""
    cfgs = [_box(0.15, 0.05, model=DynamicsModel.DIFF_DRIVE, max_speed=5.0, max_ang_vel=5.0)
            for _ in range(2)]
    w = WorldConfig(collisions=False, bounds=(-0.4, 0.4, -0.4, 0.4), bounds_mode="clamp")
    s0 = pack_state({"pos": [[[0.2, 0.0], [-0.1, -0.3]]], "theta": [[0.3, -1.9]]})
    acts = np.array([[[[3.0, 0.7], [2.5, -0.4]]], [[[3.0, 0.5], [2.5, 0.3]]]])
    _fd_check(cfgs, w, 0.1, 2, s0, acts, fields=(0, 1, 2, 3, 4, 5, 6))
    # the clamp is active in this case (otherwise the test would not pin it)
    cfg = oracle_cfg(cfgs, w, 0.1, 2, 1, 2)
    p, t, m = params_of(cfgs)
    tr = O.rollout(cfg, p, t, m, None, s0, acts)
    th = tr[-1, 0, 0, 2]
    ex = 0.15 * abs(math.cos(th)) + 0.05 * abs(math.sin(th))
    assert tr[-1, 0, 0, 0] == pytest.approx(0.4 - ex, abs=1e-15)


# ------------------------------------------------------------------ wheel contacts

def _wheel_step(cfgs, world, s0, acts, dt=0.1, obs=None):
    cfg = oracle_cfg(cfgs, world, dt, 1, s0.shape[0], 2)
    p, t, m = params_of(cfgs)
    return O.rollout(cfg, p, t, m, obstacles_np(obs, s0.shape[0]), s0, acts)


def test_wheel_contacts_grip_and_turn():
    """wheel_contact (swarp/dynamics/kernels.py:1328-1387) on a diff-drive box at heading 0
    under a circle obstacle pressing down on the right end of its top face: the force is
    (0, -f) with f = k * depth, applied at the circle's point nearest the box (0.15, 0.09),
    so the torque about the centre is -0.15 f.  Sideways the box moves only by what
    exceeds the grip mu g m; the heading turns by (|tau| - turn_cap)+ dt / I with
    I = m (hx^2 + hy^2) / 3."""
    cfgs = [_box(0.2, 0.1, model=DynamicsModel.DIFF_DRIVE)]
    circle = {"pos": [[[0.15, 0.19]]], "radius": [0.1], "type": [0]}
    s0 = pack_state({"pos": [[[0.0, 0.0]]]})
    acts = np.zeros((1, 1, 1, 2))
    dt = 0.1
    f = K * (0.1 + M - 0.09)
    for mu, cap in ((0.2, 0.0), (10.0, 0.0), (0.2, 0.2)):
        w = _world(collisions=False, wheel_contacts=True, wheel_lateral_friction=mu,
                   wheel_turn_torque=cap)
        tr = _wheel_step(cfgs, w, s0, acts, dt, circle)[0, 0, 0]
        grip = mu * 9.81
        vy = -max(f - grip, 0.0) * dt   # the slip beyond the grip (mass 1)
        assert tr[4] == pytest.approx(vy, abs=1e-12) and tr[1] == pytest.approx(vy * dt, abs=1e-13)
        tau, inertia = -0.15 * f, (0.2 ** 2 + 0.1 ** 2) / 3.0
        excess = -max(abs(tau) - cap, 0.0)
        assert tr[2] == pytest.approx(excess * dt / inertia * dt, rel=1e-12, abs=1e-15)
    # without wheel contacts the same push moves it sideways by the whole force, no turn
    tr = _wheel_step(cfgs, _world(collisions=False), s0, acts, dt, circle)[0, 0, 0]
    assert tr[4] == pytest.approx(-f * dt, rel=1e-12) and tr[2] == 0.0


def test_wheel_contacts_symmetric_push_has_no_torque():
    """Two aligned boxes face to face on one axis: the manifold point lies on the centre
    line, so the contact torque and the heading change are zero."""
    cfgs = [_box(0.2, 0.1, model=DynamicsModel.DIFF_DRIVE) for _ in range(2)]
    w = _world(wheel_contacts=True)
    s0 = pack_state({"pos": [[[0.0, 0.0], [0.38, 0.0]]]})
    tr = _wheel_step(cfgs, w, s0, np.zeros((1, 1, 2, 2)))[0, 0]
    assert tr[0, 2] == 0.0 and tr[1, 2] == 0.0 and tr[0, 0] < 0.0 < tr[1, 0]


def test_wheel_contacts_have_no_reverse_mode():
    cfgs = [_box(0.2, 0.1, model=DynamicsModel.DIFF_DRIVE)]
    w = _world(collisions=False, wheel_contacts=True)
    cfg = oracle_cfg(cfgs, w, 0.1, 1, 1, 2)
    p, t, m = params_of(cfgs)
    s0 = pack_state({"pos": [[[0.0, 0.0]]]})
    acts = np.zeros((1, 1, 1, 2))
    tr = O.rollout(cfg, p, t, m, None, s0, acts)
    with pytest.raises(RuntimeError):
        O.rollout_adj(cfg, p, t, m, None, s0, acts, tr, np.ones_like(tr), None)


# ------------------------------------------------------------------ ControlMode.SERVO

def _servo(n=2, **kw):
    from swarp_amd.config import ControlMode as CM
    return [AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=CM.SERVO, max_speed=1.5,
                        max_accel=2.0, max_ang_vel=3.0, max_ang_accel=4.0, cmd_gain_v=0.8,
                        cmd_gain_w=1.2, **kw) for _ in range(n)]


def test_servo_closed_form():
    """servo_command (swarp/dynamics/kernels.py:165-191): speed and turn rate move toward
    the gained, clamped command by at most max_accel dt / max_ang_accel dt, then the
    VELOCITY branch runs on the result."""
    cfgs = _servo(1)
    w = WorldConfig(collisions=False)
    dt = 0.1
    s0 = pack_state({"pos": [[[0.0, 0.0]]], "speed": [[0.3]], "ang_vel": [[-0.2]]})
    tr = _wheel_step(cfgs, w, s0, np.array([[[[5.0, 0.5]]]]), dt)[0, 0, 0]
    s = 0.3 + min(max(1.5 * 0.8 - 0.3, -0.2), 0.2)        # clamped command 1.5, step <= 0.2
    om = -0.2 + min(max(0.5 * 1.2 + 0.2, -0.4), 0.4)      # step <= 0.4
    assert tr[5] == pytest.approx(s, rel=1e-14) and tr[6] == pytest.approx(om, rel=1e-14)
    assert tr[2] == pytest.approx(om * dt, rel=1e-14)
    assert tr[0] == pytest.approx(s * dt, rel=1e-14)


def test_fd_servo():
    """Finite differences through the servo conversion (saturated and unsaturated steps),
    with contacts, walls and substeps."""
    cfgs = _servo(3)
    s0, rng = _rs(2, 3, 9, 0.15)
    acts = rng.uniform(-2, 2, size=(3, 2, 3, 2))
    _fd_check(cfgs, _world(collision_c=1.0, bounds=(-0.3, 0.3, -0.3, 0.3)), 0.05, 2, s0, acts,
              fields=(0, 1, 2, 3, 4, 5, 6))


def test_wheel_contacts_disc_diff_drive_stays_finite():
    """A disc diff-drive agent has no footprint inertia (half extents 0).  Under
    wheel_contacts the reference evaluates excess * (dt / inertia), which is 0 * inf = NaN
    whenever the contact torque stays below turn_cap (swarp/dynamics/kernels.py:1379-1386);
    the restatement skips the term when there is no excess, so headings stay finite and
    equal the plain step's heading update."""
    E, A, T, S = 6, 4, 5, 2
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(A)]
    world = _world(bounds=(-0.4, 0.4, -0.4, 0.4), max_neighbors=4, wheel_contacts=True,
                   wheel_lateral_friction=0.3, wheel_turn_torque=0.02)
    rng = np.random.default_rng(3)
    s0 = pack_state({"pos": rng.uniform(-0.12, 0.12, size=(E, A, 2)),
                     "theta": rng.uniform(-3, 3, size=(E, A))})
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    cfg = oracle_cfg(cfgs, world, 0.05, S, E, 2)
    p, t, m = params_of(cfgs)
    st = Oracle(np.float64).rollout(cfg, p, t, m, None, s0, acts)
    assert np.isfinite(st).all()
    # discs feel no contact torque, so the heading advances by the commanded turn rate
    # exactly as without wheel contacts
    plain = oracle_cfg(cfgs, _world(bounds=(-0.4, 0.4, -0.4, 0.4), max_neighbors=4), 0.05, S,
                       E, 2)
    ref = Oracle(np.float64).rollout(plain, p, t, m, None, s0, acts)
    np.testing.assert_array_equal(st[..., 2], ref[..., 2])
