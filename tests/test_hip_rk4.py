"""RK4 (``WorldConfig(integrator=Integrator.RK4)``) on the GPU: the HIP step against the
CPU oracle's RK4 (swarp/dynamics/kernels.py:416-793) on identical seeded inputs, and fp64
gradcheck through the boundary (tests/unit/test_gradients.py:77-108).

Bars as in the Euler parity tests: float32 states bit-exact with the float32 oracle (the
diff-drive and bicycle models' cos / sin / tan / atan come from the portable evaluation
both sides share, include/swarp_pmath.h); gradients at 1e-5 relative of the float32
oracle's (measured errors are printed; run with -s).
"""

import numpy as np
import pytest
import torch

from hip_helpers import hip_run, make_stepper, oracle_run, rel
from oracle.oracle import pack_state
from swarp_amd import (AgentConfig, ControlMode, DynamicsModel, Integrator, Stepper, TorchState,
                       WorldConfig, rollout, warp_step)

pytestmark = pytest.mark.gpu
BIG = 100.0
D = torch.float64


def _world(**kw):
    kw.setdefault("collision_k", 100.0)
    kw.setdefault("collision_c", 1.0)
    kw.setdefault("collision_margin", 0.02)
    return WorldConfig(integrator=Integrator.RK4, **kw)


def _check(name, hip, orc, exact, g_tol=1e-5, cols=slice(0, 7)):
    hs, hg0, hga = hip
    os_, og0, oga = orc
    print(f"\n{name}: states rel {rel(hs[..., cols], os_[..., cols]):.3e}, d/d actions rel "
          f"{rel(hga, oga):.3e}, d/d state0 rel {rel(hg0[..., cols], og0[..., cols]):.3e}")
    if exact:
        assert np.array_equal(hs[..., cols], os_[..., cols]), (
            f"{name}: states not bit-exact, max rel {rel(hs[..., cols], os_[..., cols]):.3e}")
    else:
        assert rel(hs[..., cols], os_[..., cols]) <= 1e-5, f"{name}: states rel {rel(hs[..., cols], os_[..., cols]):.3e}"
    assert rel(hga, oga) <= g_tol, f"{name}: d/d actions rel {rel(hga, oga):.3e}"
    assert rel(hg0[..., cols], og0[..., cols]) <= g_tol, f"{name}: d/d state0 rel {rel(hg0[..., cols], og0[..., cols]):.3e}"


def _cot(T, E, A, seed, n=7, scale=0.1):
    w = np.random.default_rng(seed).normal(size=(T, E, A, 16)) * scale
    w[..., n:] = 0.0
    return w


def _run(cfgs, world, dt, S, s0, acts, w, np_dtype):
    st = make_stepper(cfgs, world, dt, S, torch.float32 if np_dtype == np.float32 else D)
    return hip_run(st, s0, acts, w, np_dtype), oracle_run(cfgs, world, dt, S, s0, acts, w, np_dtype)


@pytest.mark.parametrize("mode", [ControlMode.VELOCITY, ControlMode.ACCELERATION], ids=["vel", "acc"])
def test_holonomic_rk4_bitexact(mode):
    """Holonomic fleet with contacts and soft walls, 4 substeps: bit-exact states.  In
    velocity mode this also checks that RK4 leaves the specialised Euler kernels alone."""
    E, A, T, S = 64, 16, 10, 4
    rng = np.random.default_rng(31)
    cfgs = [AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=mode, radius=0.05, max_speed=1.0,
                        max_accel=2.0) for _ in range(A)]
    world = _world(bounds=(-0.6, 0.6, -0.6, 0.6), max_neighbors=16)
    s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)),
                     "vel": rng.normal(size=(E, A, 2)) * 0.3}).astype(np.float32)
    acts = rng.uniform(-1.5, 1.5, size=(T, E, A, 2)).astype(np.float32)
    hip, orc = _run(cfgs, world, 0.05, S, s0, acts, _cot(T, E, A, 1), np.float32)
    _check(f"holonomic-{mode.name}", hip, orc, exact=True)


def test_holonomic_rk4_clamp_bounds_bitexact():
    E, A, T, S = 32, 8, 8, 2
    rng = np.random.default_rng(32)
    cfgs = [AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=ControlMode.ACCELERATION,
                        radius=0.05, max_speed=1.0, max_accel=3.0) for _ in range(A)]
    world = _world(bounds=(-0.3, 0.3, -0.3, 0.3), bounds_mode="clamp", max_neighbors=8)
    s0 = pack_state({"pos": rng.uniform(-0.25, 0.25, size=(E, A, 2))}).astype(np.float32)
    acts = rng.uniform(-3, 3, size=(T, E, A, 2)).astype(np.float32)
    hip, orc = _run(cfgs, world, 0.05, S, s0, acts, _cot(T, E, A, 2), np.float32)
    _check("holonomic-clamp", hip, orc, exact=True)


def test_diffdrive_bicycle_rk4():
    """Diff-drive (both modes) and bicycle agents mixed, contacts and soft walls."""
    E, A, T, S = 64, 12, 10, 2
    rng = np.random.default_rng(33)
    cfgs = ([AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.VELOCITY, radius=0.05)
             for _ in range(4)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION,
                           radius=0.05) for _ in range(4)]
            + [AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, radius=0.05, min_speed=0.0)
               for _ in range(4)])
    world = _world(bounds=(-0.6, 0.6, -0.6, 0.6), max_neighbors=12)
    s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A)),
                     "speed": rng.uniform(0, 0.5, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    hip, orc = _run(cfgs, world, 0.05, S, s0, acts, _cot(T, E, A, 3), np.float32)
    _check("diffdrive-bicycle", hip, orc, exact=True)


def test_drones_rk4_bitexact():
    E, A, T, S = 64, 8, 12, 2
    rng = np.random.default_rng(34)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0) for _ in range(A)]
    world = _world()
    ax = rng.normal(size=(E, A, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(E, A, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    s0 = pack_state({"pos": rng.uniform(-0.5, 0.5, size=(E, A, 2)), "z": np.ones((E, A)),
                     "attitude": q, "body_rates": rng.normal(size=(E, A, 3)) * 0.2}).astype(np.float32)
    acts = (rng.uniform(0, 1, size=(T, E, A, 4)) * 5.0).astype(np.float32)
    hip, orc = _run(cfgs, world, 0.02, S, s0, acts, _cot(T, E, A, 4, n=16, scale=0.01), np.float32)
    _check("drones", hip, orc, exact=True, cols=slice(0, 16))


def test_float64_rk4_matches_float64_oracle():
    E, A, T, S = 16, 8, 6, 2
    rng = np.random.default_rng(35)
    cfgs = ([AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=ControlMode.ACCELERATION,
                         radius=0.05) for _ in range(4)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(2)]
            + [AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, radius=0.05) for _ in range(2)])
    world = _world(bounds=(-0.5, 0.5, -0.5, 0.5), max_neighbors=8)
    s0 = pack_state({"pos": rng.uniform(-0.4, 0.4, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))})
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    (hs, hg0, hga), (os_, og0, oga) = _run(cfgs, world, 0.05, S, s0, acts, _cot(T, E, A, 5), np.float64)
    assert rel(hs[..., :7], os_[..., :7]) <= 1e-13
    assert np.array_equal(hs[:, :, :4, :7], os_[:, :, :4, :7])  # the holonomic agents' states
    assert rel(hga, oga) <= 1e-11 and rel(hg0[..., :7], og0[..., :7]) <= 1e-11


def test_rk4_differs_from_euler():
    """The integrator switch reaches the kernels: RK4 and Euler disagree on a curved path."""
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=5.0, max_ang_vel=5.0)]
    s = TorchState(torch.zeros(1, 1, 2, device="cuda"), torch.zeros(1, 1, device="cuda"),
                   torch.zeros(1, 1, 2, device="cuda"), torch.zeros(1, 1, device="cuda"),
                   torch.zeros(1, 1, device="cuda"))
    a = torch.tensor([[[1.3, 0.9]]], device="cuda")
    outs = []
    for integ in (Integrator.EULER, Integrator.RK4):
        st = Stepper(cfgs, dt=0.5, device="cuda:0", world=WorldConfig(collisions=False, integrator=integ))
        outs.append(warp_step(st, s, a).pos)
    assert not torch.equal(outs[0], outs[1])


# -------------------------------------------------- fp64 gradcheck (test_gradients.py:77-108)

MODEL_CASES = [
    ("holonomic-vel", DynamicsModel.HOLONOMIC, ControlMode.VELOCITY),
    ("holonomic-acc", DynamicsModel.HOLONOMIC, ControlMode.ACCELERATION),
    ("diffdrive-vel", DynamicsModel.DIFF_DRIVE, ControlMode.VELOCITY),
    ("diffdrive-acc", DynamicsModel.DIFF_DRIVE, ControlMode.ACCELERATION),
    ("bicycle", DynamicsModel.KINEMATIC_BICYCLE, ControlMode.ACCELERATION),
]


def _state(E, A, seed):
    g = torch.Generator().manual_seed(seed)

    def t(*shape):
        return (torch.randn(*shape, generator=g, dtype=D) * 0.5).cuda().requires_grad_(True)

    return (t(E, A, 2), t(E, A), t(E, A, 2), t(E, A), t(E, A))


def _fn(stepper):
    def fn(pos, theta, vel, speed, ang_vel, act):
        return tuple(warp_step(stepper, TorchState(pos, theta, vel, speed, ang_vel), act))[:5]
    return fn


@pytest.mark.parametrize("name,model,mode", MODEL_CASES, ids=[c[0] for c in MODEL_CASES])
def test_gradcheck_single_step_rk4(name, model, mode):
    cfgs = [AgentConfig(model=model, ctrl_mode=mode, max_speed=BIG, max_accel=BIG, max_ang_vel=BIG,
                        max_ang_accel=BIG, max_steer=1.0, l_f=0.16, l_r=0.14) for _ in range(2)]
    st = Stepper(cfgs, dt=0.1, device="cuda:0", dtype=D,
                 world=WorldConfig(collisions=False, integrator=Integrator.RK4))
    s = _state(2, 2, 1)
    a = (0.3 * torch.randn(2, 2, 2, dtype=D)).cuda().requires_grad_(True)
    assert torch.autograd.gradcheck(_fn(st), (*s, a), eps=1e-6, atol=1e-5)


def test_gradcheck_rk4_rollout_with_contacts():
    """Multi-step rollout with contacts, soft walls and substeps on the RK4 path."""
    cfgs = [AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=ControlMode.ACCELERATION,
                        radius=0.1, max_speed=BIG, max_accel=BIG),
            AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION,
                        radius=0.1, max_speed=BIG, max_accel=BIG, max_ang_vel=BIG, max_ang_accel=BIG)]
    world = WorldConfig(collision_k=10.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-1.0, 1.0, -1.0, 1.0), bounds_mode="soft", integrator=Integrator.RK4)
    st = Stepper(cfgs, dt=0.1, substeps=2, device="cuda:0", dtype=D, world=world)
    z = torch.zeros(1, 2, dtype=D, device="cuda")
    s = TorchState(torch.tensor([[[0.0, 0.0], [0.18, 0.02]]], dtype=D, device="cuda"), z.clone(),
                   torch.tensor([[[0.1, 0.0], [-0.1, 0.05]]], dtype=D, device="cuda"),
                   z.clone() + 0.1, z.clone())
    s = tuple(t.requires_grad_(True) for t in tuple(s)[:5])
    acts = (0.1 * torch.randn(3, 1, 2, 2, dtype=D, generator=torch.Generator().manual_seed(0))).cuda()

    def fn(pos, theta, vel, speed, ang_vel, a):
        final, _ = rollout(st, TorchState(pos, theta, vel, speed, ang_vel), a)
        return final.pos, final.theta, final.vel

    assert torch.autograd.gradcheck(fn, (*s, acts.requires_grad_(True)), eps=1e-6, atol=1e-5)


def test_gradcheck_drone_rk4():
    cfg = AgentConfig(model=DynamicsModel.DRONE, thrust_max=20.0)
    st = Stepper([cfg], dt=0.02, device="cuda:0", dtype=D,
                 world=WorldConfig(collisions=False, integrator=Integrator.RK4))
    g = torch.Generator().manual_seed(0)
    c = lambda x: x.cuda().requires_grad_(True)  # noqa: E731
    q = torch.tensor([[[0.05, -0.03, 0.02, 1.0]]], dtype=D)
    args = (
        c(torch.zeros(1, 1, 2, dtype=D)), c(torch.zeros(1, 1, dtype=D)),
        c(0.05 * torch.randn(1, 1, 2, dtype=D, generator=g)), c(torch.zeros(1, 1, dtype=D)),
        c(torch.zeros(1, 1, dtype=D)), c(torch.ones(1, 1, dtype=D)), c(torch.zeros(1, 1, dtype=D)),
        c(q / q.norm()), c(0.3 * torch.randn(1, 1, 3, dtype=D, generator=g)),
        c(9.81 / 4 + 0.3 * torch.randn(1, 1, 4, dtype=D, generator=g)),
    )

    def fn(*a):
        return tuple(warp_step(st, TorchState(*a[:9]), a[9]))

    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-5)
