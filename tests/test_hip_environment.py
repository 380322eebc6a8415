"""``make("navigation")`` / ``Environment.step`` / ``World`` on the GPU: the drop-in
surface that calls the step (swarp/__init__.py:95-121, swarp/core/environment.py:567-685,
swarp/core/world.py:163-491).

* the physics of ``env.step`` is the HIP step: bit-exact with the float32 oracle from
  the same (reset) state;
* observations, rewards, termination and info follow the navigation scenario's
  definitions (swarp/scenarios/navigation.py:671-839), recomputed here with numpy from
  the oracle's own neighbour lists;
* BPTT through ``env.step`` (dynamics adjoint + torch autograd of the reward) equals the
  same loss written on ``rollout`` (rel 1e-5);
* radius graph = COO of the step's lists; masked and automatic resets, seeding.
"""

import numpy as np
import pytest
import torch

from cases import oracle_cfg, params_of
from hip_helpers import state_to16
from oracle.oracle import Oracle
from swarp_amd import TorchState, make, rollout

pytestmark = pytest.mark.gpu

E, A, DT = 64, 4, 0.05


def _env(**kw):
    kw.setdefault("n_agents", A)
    return make("navigation", E, dt=DT, seed=0, **kw)


def _oracle_step(env, s16, acts):
    w = env.world
    cfg = oracle_cfg(w.agent_configs, w.stepper.world, DT, 1, E, 2)
    p, t, m = params_of(w.agent_configs)
    O = Oracle(np.float32)
    return O.rollout(cfg, p, t, m, None, s16.astype(np.float32), acts[None])[0]


def test_reset_and_step_match_oracle_and_scenario_definitions():
    env = _env()
    obs0 = env.reset()
    assert obs0.shape == (E, A, env.obs_dim) and env.obs_dim == 9 + 5 * 2
    w = env.world
    s16 = state_to16(w.state).astype(np.float32)
    # spawns keep the scenario's minimum separation (3 r) and stay inside the walls
    p0 = s16[..., 0:2]
    d = np.linalg.norm(p0[:, :, None] - p0[:, None], axis=-1) + np.eye(A)[None] * 9
    assert d.min() >= 3 * 0.05 - 1e-6 and np.abs(p0).max() <= 1.0 - 2 * 0.05 + 1e-6
    goals = w.goals.cpu().numpy()
    dist0 = np.linalg.norm(p0 - goals, axis=-1)

    rng = np.random.default_rng(1)
    acts = rng.uniform(-1, 1, size=(E, A, 2)).astype(np.float32)
    obs, rew, term, trunc, info = env.step(torch.tensor(acts, device="cuda"))
    ref = _oracle_step(env, s16, acts)
    got = state_to16(w.state).astype(np.float32)
    assert np.array_equal(got[..., :7], ref[..., :7]), "env.step physics differs from the oracle"

    # observations: pos, vel, cos/sin theta, ang_vel, goal - pos, then 2 neighbour slots
    o = obs.cpu().numpy()
    pos, vel, th = ref[..., 0:2], ref[..., 3:5], ref[..., 2]
    assert np.array_equal(o[..., 0:2], pos) and np.array_equal(o[..., 2:4], vel)
    np.testing.assert_allclose(o[..., 4], np.cos(th), rtol=0, atol=2e-7)
    np.testing.assert_allclose(o[..., 5], np.sin(th), rtol=0, atol=2e-7)
    assert np.array_equal(o[..., 7:9], goals - pos)
    idx, cnt, _ = Oracle(np.float32).neighbors(pos, w.stepper.neighbor_radius, w.stepper.world.max_neighbors)
    k = 2
    valid = np.arange(idx.shape[-1])[None, None] < cnt[..., None]
    npos = np.take_along_axis(pos, idx.reshape(E, -1)[..., None].repeat(2, -1), 1).reshape(E, A, -1, 2)
    nvel = np.take_along_axis(vel, idx.reshape(E, -1)[..., None].repeat(2, -1), 1).reshape(E, A, -1, 2)
    rel_p = (npos - pos[:, :, None]) * valid[..., None]
    rel_v = (nvel - vel[:, :, None]) * valid[..., None]
    np.testing.assert_array_equal(o[..., 9:9 + 2 * k], rel_p[:, :, :k].reshape(E, A, -1))
    np.testing.assert_array_equal(o[..., 9 + 2 * k:9 + 4 * k], rel_v[:, :, :k].reshape(E, A, -1))
    np.testing.assert_array_equal(o[..., 9 + 4 * k:], valid[:, :, :k].astype(np.float32))

    # reward = -1 per touching listed neighbour + shaping (dist_prev - dist) + 5 if all on goal
    dist = np.linalg.norm(pos - goals, axis=-1)
    touching = ((np.linalg.norm(npos - pos[:, :, None], axis=-1) < 0.1) & valid).sum(-1)
    on = dist < 0.05
    want = -1.0 * touching + (dist0 - dist) + 5.0 * on.all(-1)[:, None]
    np.testing.assert_allclose(rew.cpu().numpy(), want, rtol=0, atol=2e-6)
    assert np.array_equal(term.cpu().numpy(), on.all(-1))
    assert not trunc.any()
    assert set(info) == {"dist_to_goal", "on_goal", "collisions", "neighbor_overflow"}
    assert env.step_count.tolist() == [1] * E


def test_bptt_through_env_step_equals_rollout():
    """d(sum of shaping rewards over 3 steps)/d(actions) through env.step equals the same
    loss (-sum of goal distances, the baseline being detached) through rollout."""
    T = 3
    env = _env()
    env.reset()
    w = env.world
    s0 = TorchState(*(None if t is None else t.clone() for t in w.state))
    goals = w.goals.clone()
    rng = np.random.default_rng(2)
    acts = torch.tensor(rng.uniform(-1, 1, size=(T, E, A, 2)), dtype=torch.float32, device="cuda")
    a1 = acts.clone().requires_grad_(True)
    loss = 0.0
    for t in range(T):
        _, rew, _, _, _ = env.step(a1[t])
        loss = loss + rew.sum()
    loss.backward()

    a2 = acts.clone().requires_grad_(True)
    _, traj = rollout(w.stepper, s0, a2)
    loss2 = -sum((st.pos - goals).norm(dim=-1).sum() for st in traj)
    loss2.backward()
    g1, g2 = a1.grad.double().cpu().numpy(), a2.grad.double().cpu().numpy()
    assert np.abs(g1 - g2).max() <= 1e-5 * np.abs(g2).max()


def test_radius_graph_is_the_lists_as_coo():
    env = _env(n_agents=16, world_size=0.4)
    env.reset()
    env.step(torch.zeros(E, 16, 2, device="cuda"))
    ei = env.radius_graph().cpu().numpy()
    idx, cnt = (t.cpu().numpy() for t in env.world.neighbors())
    want = [(e * 16 + idx[e, a, s], e * 16 + a) for e in range(E) for a in range(16) for s in range(cnt[e, a])]
    assert ei.shape[1] == len(want) > 0
    assert [tuple(c) for c in ei.T.tolist()] == want
    ov = env.world.neighbor_overflow()
    assert ov.dtype == torch.bool and ov.shape == (E, 16)


def test_reset_at_and_auto_reset():
    env = _env(max_steps=2, auto_reset=True)
    env.reset()
    z = torch.zeros(E, A, 2, device="cuda")
    env.step(z)
    before = env.world.state.pos.clone()
    obs, _, _, trunc, _ = env.step(z)
    assert trunc.all() and env.step_count.tolist() == [0] * E
    now = env.world.state.pos
    assert not torch.equal(now, before)  # every env restarted
    assert torch.equal(obs[..., 0:2], now)

    env2 = _env()
    env2.reset()
    p = env2.world.state.pos.clone()
    mask = torch.arange(E, device="cuda") % 2 == 0
    env2.reset_at(mask)
    q = env2.world.state.pos
    assert torch.equal(q[~mask], p[~mask]) and not torch.equal(q[mask], p[mask])


def test_seed_determinism():
    a, b, c = _env(), _env(), _env()
    a.reset()
    b.reset()
    c.reset(seed=7)
    assert torch.equal(a.world.state.pos, b.world.state.pos)
    assert torch.equal(a.world.goals, b.world.goals)
    assert not torch.equal(a.world.state.pos, c.world.state.pos)
