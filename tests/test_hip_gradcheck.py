"""torch.autograd.gradcheck (float64) through the HIP boundary on the GPU.

The cases are the reference's own gradcheck cases (tests/unit/test_gradients.py:50-171,
tests/unit/test_collisions.py:151-178, tests/unit/test_drone.py:206-234,
tests/unit/test_geometry.py:250-274) with eps=1e-6, atol=1e-5 as there.
"""

import numpy as np
import pytest
import torch

from cases import holo
from swarp_amd import (AgentConfig, ControlMode, DynamicsModel, Obstacles, ObstacleShape, Stepper,
                       TorchState, WorldConfig, rollout, warp_step)

pytestmark = pytest.mark.gpu
BIG = 100.0
D = torch.float64


def _state(E, A, seed, requires_grad=True):
    g = torch.Generator().manual_seed(seed)

    def t(*shape):
        return (torch.randn(*shape, generator=g, dtype=D) * 0.5).cuda().requires_grad_(requires_grad)

    return (t(E, A, 2), t(E, A), t(E, A, 2), t(E, A), t(E, A))


def _fn(stepper):
    def fn(pos, theta, vel, speed, ang_vel, act):
        return tuple(warp_step(stepper, TorchState(pos, theta, vel, speed, ang_vel), act))[:5]
    return fn


MODEL_CASES = [
    ("holonomic-vel", DynamicsModel.HOLONOMIC, ControlMode.VELOCITY),
    ("holonomic-acc", DynamicsModel.HOLONOMIC, ControlMode.ACCELERATION),
    ("diffdrive-vel", DynamicsModel.DIFF_DRIVE, ControlMode.VELOCITY),
    ("diffdrive-acc", DynamicsModel.DIFF_DRIVE, ControlMode.ACCELERATION),
    ("bicycle", DynamicsModel.KINEMATIC_BICYCLE, ControlMode.ACCELERATION),
]


@pytest.mark.parametrize("name,model,mode", MODEL_CASES, ids=[c[0] for c in MODEL_CASES])
def test_gradcheck_single_step(name, model, mode):
    cfgs = [AgentConfig(model=model, ctrl_mode=mode, max_speed=BIG, max_accel=BIG, max_ang_vel=BIG,
                        max_ang_accel=BIG, max_steer=1.0, l_f=0.16, l_r=0.14) for _ in range(2)]
    st = Stepper(cfgs, dt=0.1, device="cuda:0", dtype=D)
    s = _state(2, 2, 1)
    a = (0.3 * torch.randn(2, 2, 2, dtype=D)).cuda().requires_grad_(True)
    assert torch.autograd.gradcheck(_fn(st), (*s, a), eps=1e-6, atol=1e-5)


def test_gradcheck_substeps():
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=BIG, max_ang_vel=BIG)]
    st = Stepper(cfgs, dt=0.1, substeps=4, device="cuda:0", dtype=D)
    s = _state(1, 1, 2)
    a = (0.3 * torch.randn(1, 1, 2, dtype=D)).cuda().requires_grad_(True)
    assert torch.autograd.gradcheck(_fn(st), (*s, a), eps=1e-6, atol=1e-5)


def test_gradcheck_multistep_rollout():
    cfgs = [AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, max_speed=BIG, max_accel=BIG,
                        max_steer=1.0, l_f=0.16, l_r=0.14),
            AgentConfig(model=DynamicsModel.DIFF_DRIVE, max_speed=BIG, max_ang_vel=BIG)]
    st = Stepper(cfgs, dt=0.1, device="cuda:0", dtype=D)
    s = _state(1, 2, 3)
    acts = (0.3 * torch.randn(5, 1, 2, 2, dtype=D)).cuda().requires_grad_(True)

    def fn(pos, theta, vel, speed, ang_vel, a):
        final, _ = rollout(st, TorchState(pos, theta, vel, speed, ang_vel), a)
        return final.pos, final.theta

    assert torch.autograd.gradcheck(fn, (*s, acts), eps=1e-6, atol=1e-5)


def test_gradcheck_with_collisions():
    world = WorldConfig(collision_k=10.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-1.0, 1.0, -1.0, 1.0), bounds_mode="soft")
    st = Stepper(holo(2, mode=ControlMode.ACCELERATION), dt=0.1, substeps=2, device="cuda:0",
                 dtype=D, world=world)
    z = torch.zeros(1, 2, dtype=D, device="cuda")
    s = TorchState(torch.tensor([[[0.0, 0.0], [0.18, 0.02]]], dtype=D, device="cuda"), z.clone(),
                   torch.tensor([[[0.1, 0.0], [-0.1, 0.05]]], dtype=D, device="cuda"), z.clone(),
                   z.clone())
    s = tuple(t.requires_grad_(True) for t in tuple(s)[:5])
    a = (0.1 * torch.randn(1, 2, 2, dtype=D, generator=torch.Generator().manual_seed(0))).cuda()
    assert torch.autograd.gradcheck(_fn(st), (*s, a.requires_grad_(True)), eps=1e-6, atol=1e-5)


def test_gradcheck_box_and_segment():
    world = WorldConfig(collision_k=10.0, collision_c=1.0, collision_margin=0.02)
    st = Stepper(holo(1, 0.1), dt=0.1, substeps=2, device="cuda:0", dtype=D, world=world)
    st.set_obstacles(Obstacles(
        pos=torch.tensor([[[0.22, 0.0], [0.0, -0.2]]], dtype=D),
        radius=torch.tensor([0.0, 0.05], dtype=D),
        shape=torch.tensor([int(ObstacleShape.BOX), int(ObstacleShape.SEGMENT)], dtype=torch.int32),
        angle=torch.tensor([0.0, 0.0], dtype=D),
        half_extents=torch.tensor([[0.1, 0.1], [0.2, 0.0]], dtype=D),
    ))
    z = torch.zeros(1, 1, dtype=D, device="cuda")
    s = TorchState(torch.tensor([[[0.05, -0.05]]], dtype=D, device="cuda"), z.clone(),
                   torch.zeros(1, 1, 2, dtype=D, device="cuda"), z.clone(), z.clone())
    s = tuple(t.requires_grad_(True) for t in tuple(s)[:5])
    a = (0.05 * torch.randn(1, 1, 2, dtype=D, generator=torch.Generator().manual_seed(0))).cuda()
    assert torch.autograd.gradcheck(_fn(st), (*s, a.requires_grad_(True)), eps=1e-6, atol=1e-5)


def test_gradcheck_drone():
    cfg = AgentConfig(model=DynamicsModel.DRONE, thrust_max=20.0)
    st = Stepper([cfg], dt=0.02, device="cuda:0", dtype=D)
    hover = 9.81 / 4.0
    g = torch.Generator().manual_seed(0)
    c = lambda x: x.cuda().requires_grad_(True)  # noqa: E731
    args = (
        c(torch.zeros(1, 1, 2, dtype=D)), c(torch.zeros(1, 1, dtype=D)),
        c(0.05 * torch.randn(1, 1, 2, dtype=D, generator=g)), c(torch.zeros(1, 1, dtype=D)),
        c(torch.zeros(1, 1, dtype=D)), c(torch.ones(1, 1, dtype=D)), c(torch.zeros(1, 1, dtype=D)),
        c(torch.tensor([[[0.0, 0.0, 0.0, 1.0]]], dtype=D)),
        c(0.02 * torch.randn(1, 1, 3, dtype=D, generator=g)),
        c(hover + 0.1 * torch.randn(1, 1, 4, dtype=D, generator=g)),
    )

    def fn(pos, theta, vel, speed, ang_vel, z, vz, att, br, act):
        return tuple(warp_step(st, TorchState(pos, theta, vel, speed, ang_vel, z, vz, att, br), act))

    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-5)


def test_gradcheck_config4_small():
    """Config 4's fp64 gradcheck run: 4 envs x 3 drones x 5 steps, planar contacts."""
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1) for _ in range(3)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    st = Stepper(cfgs, dt=0.02, device="cuda:0", dtype=D, world=world)
    rng = np.random.default_rng(0)
    ax = rng.normal(size=(4, 3, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(4, 3, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    pos = rng.uniform(-0.15, 0.15, size=(4, 3, 2))
    c = lambda x: torch.tensor(x, dtype=D).cuda().requires_grad_(True)  # noqa: E731
    s = (c(pos), c(np.zeros((4, 3))), c(np.zeros((4, 3, 2))), c(np.zeros((4, 3))),
         c(np.zeros((4, 3))), c(np.ones((4, 3))), c(np.zeros((4, 3))), c(q), c(np.zeros((4, 3, 3))))
    acts = c(rng.uniform(0.2, 0.8, size=(5, 4, 3, 4)) * 10.0)

    def fn(*args):
        final, _ = rollout(st, TorchState(*args[:9]), args[9])
        return final.pos, final.z, final.attitude

    assert torch.autograd.gradcheck(fn, (*s, acts), eps=1e-6, atol=1e-5)
