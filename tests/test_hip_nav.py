"""The navigation scenario's fused no-grad pass on the GPU (``swarp_nav_obs``): one launch
for the lists, observations, reward inputs, reward and done.

* against the CPU oracle (``oracle/nav.py``, a restatement of
  swarp/scenarios/navigation_kernels.py:41-243) on the same seeded states: lists, counts,
  overflow, touching, goal distance, shaping, baseline, flags, reward and done EXACT;
  observation rows exact except the cos / sin slots (device vs host libm, 1 ulp);
* step, reset and auto-reset passes, padded agent slots (A = 5), every env-slot width
  (A = 4 .. 64), shared reward, list caps, the staged and the direct row-store paths;
* through ``Environment``: the fused path equals the torch path (the reference's own
  oracle for its fused kernels) step by step, with auto-reset and time limits.
"""

import numpy as np
import pytest
import torch

from oracle.nav import nav_pass
from swarp_amd import WorldConfig, make

pytestmark = pytest.mark.gpu
TDT = {np.float32: torch.float32, np.float64: torch.float64}


def _env(E, A, dtype=torch.float32, **kw):
    kw.setdefault("world_size", max(1.0, A ** 0.5 / 4))
    return make("navigation", E, n_agents=A, dt=0.05, seed=0, dtype=dtype, **kw)


def _random_state(env, seed, spread):
    w = env.world
    g = torch.Generator(device="cpu").manual_seed(seed)
    E, A = w.n_envs, w.n_agents
    r = lambda *s: (torch.rand(*s, generator=g, dtype=torch.float64) * 2 - 1)  # noqa: E731
    w.write_state(pos=(r(E, A, 2) * spread).to(w.dtype).cuda(), vel=r(E, A, 2).to(w.dtype).cuda(),
                  theta=(r(E, A) * 3.2).to(w.dtype).cuda(), ang_vel=r(E, A).to(w.dtype).cuda())
    w.goals.copy_((r(E, A, 2) * spread).to(w.dtype).cuda())


def _np(t):
    return t.detach().cpu().numpy()


def _oracle_pass(env, prev, reset_mask, advance_prev, full_pass, out=None):
    w, sc = env.world, env.scenario
    s = w.state
    npdt = np.float32 if w.dtype == torch.float32 else np.float64
    return nav_pass(_np(s.pos), _np(s.vel), _np(s.theta), _np(s.ang_vel), _np(w.goals),
                    _np(w.agent_radius).astype(npdt), float(w.stepper.neighbor_radius),
                    w.stepper.world.max_neighbors, sc._k_obs, prev, reset_mask, advance_prev,
                    full_pass, sc.pos_shaping_factor, sc.goal_tolerance, sc.collision_penalty,
                    sc.final_reward, sc.shared_reward, out)


def _compare(env, o, trig_tol):
    sc, grid = env.scenario, env.world.stepper.grid(env.n_envs)
    fb = sc._fb
    assert np.array_equal(_np(grid.neighbor_count), o["cnt"])
    assert np.array_equal(_np(grid.neighbor_true_count), o["true"])
    K = o["idx"].shape[-1]
    valid = np.arange(K)[None, None] < o["cnt"][..., None]
    assert np.array_equal(np.where(valid, _np(grid.neighbor_idx), 0), np.where(valid, o["idx"], 0))
    got = _np(fb["obs"])
    cols = [c for c in range(got.shape[-1]) if c not in (4, 5)]
    assert np.array_equal(got[..., cols], o["obs"][..., cols])
    np.testing.assert_allclose(got[..., 4:6], o["obs"][..., 4:6], rtol=0, atol=trig_tol)
    for k, ok in (("touch", "touching"), ("dist", "dist"), ("shaping", "shaping"),
                  ("ongoal", "on_goal"), ("overflow", "overflow"), ("reward", "reward"),
                  ("done", "done")):
        assert np.array_equal(_np(fb[k]), o[ok]), k


# (n_envs, n_agents, observed neighbours, shared reward, list cap K or the default)
CASES = [(64, 4, 2, False, None), (37, 5, 2, True, None), (48, 16, 8, False, None),
         (40, 16, 3, True, 3), (20, 32, 4, True, None), (6, 64, 2, False, 8)]


@pytest.mark.parametrize("E,A,k_obs,shared,K", CASES,
                         ids=[f"E{c[0]}xA{c[1]}k{c[2]}K{c[4]}" for c in CASES])
def test_fused_pass_matches_oracle_fp32(E, A, k_obs, shared, K):
    wc = None if K is None else WorldConfig(max_neighbors=K)
    env = _env(E, A, neighbor_obs=k_obs, shared_reward=shared, goal_tolerance=0.3, world_config=wc)
    env.reset()
    _random_state(env, seed=E + A, spread=0.3)   # crowded: touching, capped lists
    sc = env.scenario
    sc.set_fused_active(True)
    prev = _np(sc._prev_dist).copy()
    sc.launch_fused(advance_prev=1, full_pass=1)
    torch.cuda.synchronize()
    o = _oracle_pass(env, prev, None, 1, 1)
    _compare(env, o, trig_tol=2.5e-7)
    assert np.array_equal(_np(sc._prev_dist), prev)
    assert o["touching"].any()
    assert o["overflow"].any() == (K is not None)
    # an obs-only auto-reset pass over a moved state: only the masked envs change
    mask = torch.arange(E, device="cuda") % 3 == 0
    _random_state(env, seed=E + A + 1, spread=0.5)
    sc.launch_fused(advance_prev=0, full_pass=0, reset_mask=mask)
    o = _oracle_pass(env, prev, _np(mask), 0, 0, out=o)
    _compare(env, o, trig_tol=2.5e-7)
    assert np.array_equal(_np(sc._prev_dist), prev)
    # a standalone reset pass (full, reward recomputed)
    sc.launch_fused(advance_prev=0, full_pass=1, reset_mask=mask)
    o = _oracle_pass(env, prev, _np(mask), 0, 1, out=o)
    _compare(env, o, trig_tol=2.5e-7)


def test_fused_pass_matches_oracle_fp64_direct_rows():
    """fp64 with 32 observed neighbours: rows too wide to stage in LDS go out directly."""
    E, A = 5, 64
    env = _env(E, A, dtype=torch.float64, neighbor_obs=32, neighbor_radius=0.6)
    env.reset()
    _random_state(env, seed=3, spread=1.0)
    sc = env.scenario
    sc.set_fused_active(True)
    prev = _np(sc._prev_dist).copy()
    sc.launch_fused(advance_prev=1, full_pass=1)
    torch.cuda.synchronize()
    o = _oracle_pass(env, prev, None, 1, 1)
    assert o["cnt"].max() > 8
    _compare(env, o, trig_tol=4e-16)


@pytest.mark.parametrize("shape", ["disc", "box"])
@pytest.mark.parametrize("auto_reset", [False, True])
def test_environment_fused_equals_torch_path(auto_reset, shape):
    """The fused pass and the torch path give the same episode, with disc agents and with
    box agents (agent_shape="box": the box contact pass steps the world and the
    circumscribed radius is the scenario's agent radius, navigation.py:61-79)."""
    E, A, T = 64, 16, 12
    kw = dict(max_steps=5, auto_reset=auto_reset, goal_tolerance=0.2, agent_shape=shape)
    ef, et = _env(E, A, fused=True, **kw), _env(E, A, fused=False, **kw)
    of, ot = ef.reset(), et.reset()
    assert ef.scenario._fresh == "fused" and et.scenario._fresh == "torch"
    torch.testing.assert_close(of, ot, rtol=0, atol=1e-6)
    g = torch.Generator(device="cuda").manual_seed(1)
    for t in range(T):
        a = torch.rand(E, A, 2, device="cuda", generator=g) * 2 - 1
        with torch.no_grad():
            rf = ef.step(a)
            rt = et.step(a)
        assert torch.equal(ef.world.state.pos, et.world.state.pos), t
        torch.testing.assert_close(rf[0], rt[0], rtol=0, atol=1e-6)      # obs
        torch.testing.assert_close(rf[1], rt[1], rtol=0, atol=2e-6)      # reward
        assert torch.equal(rf[2], rt[2]) and torch.equal(rf[3], rt[3])   # terminated, truncated
        for k in rt[4]:
            v1, v2 = rf[4][k], rt[4][k]
            if v2.dtype == torch.bool:
                assert torch.equal(v1, v2), k
            else:
                torch.testing.assert_close(v1, v2, rtol=0, atol=1e-6)
    assert ef.scenario._fresh == "fused"
    assert ef.world.stepper.has_boxes == (shape == "box")


def test_grad_step_takes_the_torch_path():
    env = _env(16, 4, fused=True)
    env.reset()
    a = torch.zeros(16, 4, 2, device="cuda", requires_grad=True)
    _, rew, _, _, _ = env.step(a)
    assert env.scenario._fresh == "torch" and rew.requires_grad
    rew.sum().backward()
    assert a.grad is not None
    with torch.no_grad():
        env.step(torch.zeros(16, 4, 2, device="cuda"))
    assert env.scenario._fresh == "fused"


def test_fused_pass_uses_static_radius_under_per_env_tables():
    """With radii randomized per env (Stepper.set_agent_params_per_env) the touching count
    still uses the scenario's static radius, as the reference's navigation kernels receive
    it (swarp/scenarios/navigation.py:556-557) and as the torch path computes it: fused ==
    torch path == oracle/nav.py with the static radius."""
    from swarp_amd import per_env_float_template
    from swarp_amd.config import P_RADIUS

    E, A = 48, 16
    ef = _env(E, A, fused=True, neighbor_radius=0.4)
    et = _env(E, A, fused=False, neighbor_radius=0.4)
    rng = np.random.default_rng(12)
    table = per_env_float_template(ef.world.agent_configs, E)
    table[..., P_RADIUS] = rng.uniform(0.02, 0.15, size=(E, A))
    for env in (ef, et):
        env.world.stepper.set_agent_params_per_env(table)
    ef.reset()
    et.reset()
    g = torch.Generator(device="cuda").manual_seed(2)
    for t in range(4):
        a = torch.rand(E, A, 2, device="cuda", generator=g) * 2 - 1
        with torch.no_grad():
            rf = ef.step(a)
            rt = et.step(a)
        assert torch.equal(ef.world.state.pos, et.world.state.pos), t
        assert torch.equal(rf[4]["collisions"], rt[4]["collisions"]), t
        torch.testing.assert_close(rf[1], rt[1], rtol=0, atol=2e-6)
        s = ef.world.state
        o = nav_pass(_np(s.pos), _np(s.vel), _np(s.theta), _np(s.ang_vel), _np(ef.world.goals),
                     _np(ef.world.agent_radius), float(ef.world.stepper.neighbor_radius),
                     ef.world.stepper.world.max_neighbors, ef.scenario._k_obs,
                     np.zeros((E, A), np.float32), None, 0, 1, ef.scenario.pos_shaping_factor,
                     ef.scenario.goal_tolerance, ef.scenario.collision_penalty,
                     ef.scenario.final_reward, ef.scenario.shared_reward)
        assert np.array_equal(_np(rf[4]["collisions"]), o["touching"]), t
    assert rf[4]["collisions"].sum() > 0  # contacts happened (the check is not vacuous)
