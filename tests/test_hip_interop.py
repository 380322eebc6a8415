"""Hot-loop contracts of the no-grad path (the reference's tests/interop/
test_no_host_copies.py:44-140, test_persistent.py:91-120 and the autograd contract of
swarp/interop/autograd.py:277-296):

* no device-to-host transfer while an environment steps or resets (host-transfer entry
  points patched to raise, and torch's sync debug mode set to error);
* no allocation at steady state: ``warp_step`` without grad and ``Environment.step``
  (eager and graph) request no memory from the caching allocator;
* a rollout under a caller-created stream equals the default-stream rollout, eager and
  graph;
* a second ``backward`` over a retained graph gives the same gradient as the first.
"""

import contextlib
from unittest import mock

import pytest
import torch

from swarp_amd import Environment, NavigationScenario, TorchState, rollout, warp_step

pytestmark = pytest.mark.gpu


def make_env(use_graph=False, n_envs=32, auto_reset=True):
    sc = NavigationScenario(n_agents=8, n_obstacles=2)
    return Environment(sc, n_envs=n_envs, device="cuda:0", dt=0.05, substeps=2, seed=0,
                       use_graph=use_graph, auto_reset=auto_reset, max_steps=7)


def _raise(*args, **kwargs):
    raise AssertionError("device->host transfer on the hot path")


@contextlib.contextmanager
def forbid_host_transfers():
    with (mock.patch.object(torch.Tensor, "cpu", _raise),
          mock.patch.object(torch.Tensor, "item", _raise),
          mock.patch.object(torch.Tensor, "numpy", _raise),
          mock.patch.object(torch.Tensor, "tolist", _raise),
          mock.patch.object(torch.Tensor, "__bool__", _raise)):
        yield


@contextlib.contextmanager
def sync_is_an_error():
    torch.cuda.set_sync_debug_mode("error")
    try:
        yield
    finally:
        torch.cuda.set_sync_debug_mode(0)


@pytest.mark.parametrize("use_graph", [False, True], ids=["eager", "graph"])
def test_hot_loop_has_no_host_transfer_or_sync(use_graph):
    env = make_env(use_graph)
    env.reset(seed=0)
    actions = torch.zeros(32, 8, 2, device="cuda:0")
    with torch.no_grad():
        for _ in range(3):  # warm-up outside the guard (captures, first launches)
            env.step(actions)
        with forbid_host_transfers(), sync_is_an_error():
            for _ in range(20):
                obs, rew, term, trunc, info = env.step(actions)
            env.reset_at(torch.ones(32, dtype=torch.bool, device="cuda:0"))
            env.reset(seed=1)
    assert obs.is_cuda and env.graph_mode is use_graph


def _allocations():
    return torch.cuda.memory_stats()["allocation.all.allocated"]


def test_warp_step_without_grad_allocates_nothing():
    env = make_env(auto_reset=False)
    env.reset(seed=0)
    w = env.world
    a = torch.rand(32, 8, 2, device="cuda:0") * 2 - 1
    with torch.no_grad():
        s = w.state
        for _ in range(3):
            s = warp_step(w.stepper, s, a)
        torch.cuda.synchronize()
        n0 = _allocations()
        for _ in range(20):
            s = warp_step(w.stepper, s, a)
        torch.cuda.synchronize()
        assert _allocations() == n0


@pytest.mark.parametrize("use_graph", [False, True], ids=["eager", "graph"])
def test_environment_step_allocates_nothing(use_graph):
    env = make_env(use_graph, auto_reset=False)
    env.reset(seed=0)
    a = torch.rand(32, 8, 2, device="cuda:0") * 2 - 1
    with torch.no_grad():
        for _ in range(4):
            env.step(a)
        torch.cuda.synchronize()
        n0 = _allocations()
        for _ in range(20):
            env.step(a)
        torch.cuda.synchronize()
        assert _allocations() == n0


def _run(env, steps, seed):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    out = []
    env.reset(seed=seed)
    with torch.no_grad():
        for _ in range(steps):
            a = torch.rand(env.n_envs, env.n_agents, 2, device="cuda:0", generator=g) * 2 - 1
            o, r, d, _, _ = env.step(a)
            out.append((o.clone(), r.clone(), d.clone()))
    return out


@pytest.mark.parametrize("use_graph", [False, True], ids=["eager", "graph"])
def test_matches_under_a_user_created_stream(use_graph):
    ref = _run(make_env(use_graph), 12, 4)
    env = make_env(use_graph)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        got = _run(env, 12, 4)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for (og, rg, dg), (oe, re_, de) in zip(got, ref):
        assert torch.equal(og, oe) and torch.equal(rg, re_) and torch.equal(dg, de)


def test_repeated_backward_with_retain_graph():
    env = make_env(auto_reset=False)
    env.reset(seed=0)
    w = env.world
    s0 = TorchState(w.state.pos.clone().requires_grad_(True), *w.state[1:])
    acts = (torch.rand(6, 32, 8, 2, device="cuda:0") * 2 - 1).requires_grad_(True)
    final, traj = rollout(w.stepper, s0, acts)
    loss = (final.pos ** 2).sum() + sum(x.vel.sum() for x in traj)
    loss.backward(retain_graph=True)
    g1, p1 = acts.grad.clone(), s0.pos.grad.clone()
    loss.backward()
    assert torch.equal(acts.grad, 2 * g1) and torch.equal(s0.pos.grad, 2 * p1)
