"""The ``swarp_amd::step`` custom op (``swarp_amd.compile``), the torch.compile-safe
step: same results as ``warp_step``, fp64 gradcheck through its autograd rule, and a
compiled rollout that matches eager (swarp/interop/compile.py; the reference's
tests/interop/test_compile.py).  ``torch.compile`` runs with the ``aot_eager`` backend:
it traces the op through its fake implementation and AOTAutograd, then runs the HIP
kernels themselves (no generated kernels)."""

import pytest
import torch

from swarp_amd import AgentConfig, ControlMode, DynamicsModel, Stepper, TorchState, warp_step
from swarp_amd.compile import compiled_warp_step

pytestmark = pytest.mark.gpu
BIG = 100.0
D = torch.float64


def _stepper(substeps=1, model=DynamicsModel.DIFF_DRIVE):
    cfgs = [AgentConfig(model=model, ctrl_mode=ControlMode.ACCELERATION, max_speed=BIG,
                        max_accel=BIG, max_ang_vel=BIG, max_ang_accel=BIG) for _ in range(2)]
    return Stepper(cfgs, dt=0.1, substeps=substeps, device="cuda:0", dtype=D)


def _state(n_envs=2, n_agents=2, requires_grad=False):
    g = torch.Generator().manual_seed(0)

    def t(*s):
        return (0.4 * torch.randn(*s, generator=g, dtype=D)).cuda().requires_grad_(requires_grad)

    return TorchState(t(n_envs, n_agents, 2), t(n_envs, n_agents), t(n_envs, n_agents, 2),
                      t(n_envs, n_agents), t(n_envs, n_agents))


def test_compiled_matches_eager_forward():
    stepper = _stepper()
    state = _state()
    actions = (0.3 * torch.randn(2, 2, 2, dtype=D)).cuda()
    with torch.no_grad():
        a = warp_step(stepper, state, actions)
        b = compiled_warp_step(stepper, state, actions)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
        assert x.data_ptr() != y.data_ptr()


def test_compiled_step_gradcheck():
    stepper = _stepper(substeps=2)
    state = _state(requires_grad=True)
    actions = (0.3 * torch.randn(2, 2, 2, dtype=D)).cuda().requires_grad_(True)

    def fn(pos, theta, vel, speed, ang_vel, act):
        return tuple(compiled_warp_step(stepper, TorchState(pos, theta, vel, speed, ang_vel), act))[:5]

    assert torch.autograd.gradcheck(fn, (*tuple(state)[:5], actions), eps=1e-6, atol=1e-5)


def test_compiled_gradients_equal_warp_step():
    stepper = _stepper(substeps=2, model=DynamicsModel.KINEMATIC_BICYCLE)
    s1, s2 = _state(requires_grad=True), _state(requires_grad=True)
    a1 = (0.3 * torch.randn(2, 2, 2, dtype=D)).cuda().requires_grad_(True)
    a2 = a1.detach().clone().requires_grad_(True)
    out1 = warp_step(stepper, s1, a1)
    out2 = compiled_warp_step(stepper, s2, a2)
    (out1.pos.square().sum() + out1.theta.sum()).backward()
    (out2.pos.square().sum() + out2.theta.sum()).backward()
    assert torch.equal(a1.grad, a2.grad)
    for x, y in zip(tuple(s1)[:5], tuple(s2)[:5]):
        assert torch.equal(x.grad, y.grad)


def test_torch_compile_runs_and_matches():
    stepper = _stepper()
    state = _state()
    actions = (0.2 * torch.randn(2, 2, 2, dtype=D)).cuda()

    def rollout(state, actions):
        s = state
        total = torch.zeros((), dtype=D, device="cuda")
        for _ in range(3):
            s = compiled_warp_step(stepper, s, actions)
            total = total + s.pos.square().sum()
        return total

    eager = rollout(state, actions)
    compiled = torch.compile(rollout, backend="aot_eager")(state, actions)
    assert torch.isfinite(compiled)
    torch.testing.assert_close(compiled, eager, rtol=0, atol=0)
