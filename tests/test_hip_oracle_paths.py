"""Paths around the step checked against the CPU oracle rather than against another HIP
path:

* the whole-step HIP graph (``Environment(use_graph=True)``): every replayed step's state
  bit-exact with the oracle's step from the oracle's previous state, and its
  observations / reward / done against ``oracle/nav.py`` (the restatement of
  swarp/scenarios/navigation_kernels.py:41-243) on the oracle's states;
* the ``swarp_amd::step`` custom op (swarp/interop/compile.py:92-171) under
  ``torch.compile`` (aot_eager): a compiled T-step rollout's states bit-exact and its
  gradients within 1e-5 of the oracle's;
* the COO radius graph (swarp/core/neighbors.py:716-733) against the COO built from the
  ORACLE's lists, at config 5's shape (64 agents, r 0.3, K 16) and with truncated lists;
* ``rollout(..., ring=)`` / ``warp_step(..., slot=)`` (swarp/interop/autograd.py:172-226):
  results and gradients equal to the allocating path and to the oracle, ring reuse;
* coincident agents (the distance floor sqrt(1e-10) the reference keeps for coincident
  points, swarp/core/collisions.py:48): forward bit-exact, gradients finite and within
  1e-5 of the oracle, on the specialised and on the generic kernels;
* tanh-saturated contacts (``contact_max_overlap > 0``, swarp/core/collisions.py:87-105)
  on the specialised holonomic kernels.
"""

import numpy as np
import pytest
import torch

from cases import nav_agents, nav_world, oracle_cfg, params_of
from hip_helpers import hip_run, make_stepper, oracle_run, rel, state_to16
from oracle.nav import nav_pass
from oracle.oracle import Oracle, pack_state
from swarp_amd import (AgentConfig, DynamicsModel, GradRing, NeighborGrid, Stepper, TorchState,
                       WorldConfig, make, rollout, warp_step)
from swarp_amd.compile import compiled_warp_step

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------ graph runtime


def test_graph_env_steps_match_oracle():
    E, A, T, DT = 48, 16, 12, 0.05
    env = make("navigation", E, n_agents=A, dt=DT, seed=0, use_graph=True, auto_reset=False,
               max_steps=1000, world_size=1.0)
    assert env.graph_mode
    env.reset()
    w, sc = env.world, env.scenario
    s = state_to16(w.state).astype(np.float32)
    goals = _np(w.goals)
    prev = _np(sc._prev_dist).copy()
    cfg = oracle_cfg(w.agent_configs, w.stepper.world, DT, 1, E, 2)
    p, t_, m = params_of(w.agent_configs)
    O = Oracle(np.float32)
    radius = _np(w.agent_radius).astype(np.float32)
    g = torch.Generator(device="cpu").manual_seed(3)
    for t in range(T):
        a = (torch.rand(E, A, 2, generator=g) * 2 - 1).float()
        with torch.no_grad():
            obs, rew, term, trunc, info = env.step(a.cuda())
        s = O.rollout(cfg, p, t_, m, None, s, a.numpy()[None])[0].astype(np.float32)
        got = state_to16(w.state).astype(np.float32)
        assert np.array_equal(got[..., :7], s[..., :7]), f"graph step {t}: state differs"
        o = nav_pass(s[..., 0:2].copy(), s[..., 3:5].copy(), s[..., 2].copy(), s[..., 6].copy(),
                     goals, radius, float(w.stepper.neighbor_radius),
                     w.stepper.world.max_neighbors, sc._k_obs, prev, None, 1, 1,
                     sc.pos_shaping_factor, sc.goal_tolerance, sc.collision_penalty,
                     sc.final_reward, sc.shared_reward)
        ob = _np(obs)
        cols = [c for c in range(ob.shape[-1]) if c not in (4, 5)]
        assert np.array_equal(ob[..., cols], o["obs"][..., cols]), f"graph step {t}: obs differ"
        np.testing.assert_allclose(ob[..., 4:6], o["obs"][..., 4:6], rtol=0, atol=2e-7)
        assert np.array_equal(_np(rew), o["reward"]), f"graph step {t}: reward differs"
        assert np.array_equal(_np(term), o["done"].astype(bool))
        assert np.array_equal(_np(info["collisions"]), o["touching"])
        assert np.array_equal(_np(info["neighbor_overflow"]), o["overflow"].astype(bool))
    assert env._graph.captures == 2


# ------------------------------------------------------------------ compiled op


def test_compiled_rollout_matches_oracle():
    E, A, T, S, DT = 32, 8, 6, 2, 0.05
    cfgs, world = nav_agents(A), nav_world(A, world_size=0.5)
    st = make_stepper(cfgs, world, DT, S, torch.float32)
    rng = np.random.default_rng(41)
    s0 = pack_state({"pos": rng.uniform(-0.45, 0.45, size=(E, A, 2))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    wt = rng.normal(size=(E, A, 2)).astype(np.float32)

    pos0 = torch.tensor(s0[..., 0:2], device="cuda", requires_grad=True)
    z = torch.zeros(E, A, device="cuda")
    a = torch.tensor(acts, device="cuda", requires_grad=True)
    w = torch.tensor(wt, device="cuda")

    def run(pos0, a):
        s = TorchState(pos0, z, torch.zeros(E, A, 2, device="cuda"), z, z)
        outs = []
        for t in range(T):
            s = compiled_warp_step(st, s, a[t])
            outs.append(s.pos)
        return torch.stack(outs), (w * s.pos).sum()

    traj, loss = torch.compile(run, backend="aot_eager")(pos0, a)
    loss.backward()
    orc = Oracle(np.float32)
    cfg = oracle_cfg(cfgs, st.world, DT, S, E, 2)
    p, t_, m = params_of(cfgs)
    states = orc.rollout(cfg, p, t_, m, None, s0, acts)
    assert np.array_equal(_np(traj), states[..., 0:2]), "compiled rollout differs from the oracle"
    afin = np.zeros_like(s0)
    afin[..., 0:2] = wt
    g0, ga = orc.rollout_adj(cfg, p, t_, m, None, s0, acts, states, None, afin)
    assert rel(_np(a.grad), ga) <= 1e-5, rel(_np(a.grad), ga)
    assert rel(_np(pos0.grad), g0[..., 0:2]) <= 1e-5


# ------------------------------------------------------------------ COO radius graph


def _coo_from_lists(idx, cnt):
    E, A = cnt.shape
    snd, rcv = [], []
    for e in range(E):
        for a in range(A):
            for k in range(cnt[e, a]):
                snd.append(e * A + idx[e, a, k])
                rcv.append(e * A + a)
    return np.array([snd, rcv], dtype=np.int64).reshape(2, -1)


@pytest.mark.parametrize("E,A,r,K,spread", [(64, 64, 0.3, 16, 3.0), (24, 64, 0.3, 4, 0.6),
                                            (100, 16, 0.125, 16, 2.0), (9, 5, 0.5, 2, 0.3)])
def test_edge_index_matches_oracle_coo(E, A, r, K, spread):
    rng = np.random.default_rng(E + A + K)
    pos = rng.uniform(-spread, spread, size=(E, A, 2)).astype(np.float32)
    g = NeighborGrid(E, A, radius=r, max_neighbors=K, device="cuda:0", dtype=torch.float32)
    g.build(torch.tensor(pos, device="cuda"))
    got = _np(g.edge_index())
    oi, oc, ot = Oracle(np.float32).neighbors(pos, r, K)
    want = _coo_from_lists(oi, oc)
    assert got.dtype == np.int64 and got.shape == want.shape
    assert np.array_equal(got, want)
    assert np.array_equal(_np(g.overflow_view()), ot > oc)


# ------------------------------------------------------------------ GradRing / slot


def _ring_case(E=40, A=8, T=5, S=2):
    cfgs, world = nav_agents(A), nav_world(A, world_size=0.5)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    rng = np.random.default_rng(17)
    pos = rng.uniform(-0.45, 0.45, size=(E, A, 2)).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    wt = rng.normal(size=(T, E, A, 2)).astype(np.float32)
    return cfgs, st, pos, acts, wt


def _leaf(x):
    return torch.tensor(x, device="cuda", requires_grad=True)


def _state(pos):
    E, A = pos.shape[:2]
    z = torch.zeros(E, A, device="cuda")
    return TorchState(pos, z, torch.zeros(E, A, 2, device="cuda"), z, z)


def _loss(traj, wt):
    w = torch.tensor(wt, device="cuda")
    return sum((w[t] * s.pos).sum() + s.speed.sum() for t, s in enumerate(traj))


def test_rollout_with_ring_matches_fresh_and_oracle():
    cfgs, st, pos, acts, wt = _ring_case()
    T, E, A = acts.shape[:3]
    ring = GradRing(st, E, 2, capacity=T + 2)
    res = []
    for use_ring in (False, True, True):  # the ring twice: reuse overwrites it
        p0, a = _leaf(pos), _leaf(acts)
        final, traj = rollout(st, _state(p0), a, ring=ring if use_ring else None)
        states = np.stack([_np(s.pos) for s in traj])
        _loss(traj, wt).backward()
        res.append((states, _np(a.grad), _np(p0.grad)))
        if use_ring:
            assert traj[-1].pos.data_ptr() == ring.bufs[0][T - 1].data_ptr()
    for k in (1, 2):
        for x, y in zip(res[0], res[k]):
            assert np.array_equal(x, y)
    orc = Oracle(np.float32)
    cfg = oracle_cfg(cfgs, st.world, 0.05, 2, E, 2)
    p, t_, m = params_of(cfgs)
    s0 = pack_state({"pos": pos}).astype(np.float32)
    ost = orc.rollout(cfg, p, t_, m, None, s0, acts)
    assert np.array_equal(res[1][0], ost[..., 0:2])
    w16 = np.zeros((T, E, A, 16))
    w16[..., 0:2] = wt
    w16[..., 5] = 1.0  # d(sum speed)
    g0, ga = orc.rollout_adj(cfg, p, t_, m, None, s0, acts, ost, w16, None)
    assert rel(res[1][1], ga) <= 1e-5 and rel(res[1][2], g0[..., 0:2]) <= 1e-5


def test_warp_step_with_slots_matches_fresh():
    cfgs, st, pos, acts, wt = _ring_case()
    T, E, A = acts.shape[:3]
    ring = GradRing(st, E, 2, capacity=T)
    out = []
    for use_slot in (False, True):
        ring.reset()
        p0, a = _leaf(pos), _leaf(acts)
        s = _state(p0)
        traj = []
        for t in range(T):
            s = warp_step(st, s, a[t], slot=ring.acquire() if use_slot else None)
            traj.append(s)
        if use_slot:
            assert traj[0].pos.data_ptr() == ring.bufs[0][0].data_ptr()
            with pytest.raises(RuntimeError):
                ring.acquire()
        _loss(traj, wt).backward()
        out.append((np.stack([_np(x.pos) for x in traj]), _np(a.grad), _np(p0.grad)))
    for x, y in zip(out[0], out[1]):
        assert np.array_equal(x, y)


# ------------------------------------------------------------------ coincident agents


@pytest.mark.parametrize("model", [DynamicsModel.HOLONOMIC, DynamicsModel.DIFF_DRIVE])
def test_coincident_agents_finite_and_match_oracle(model):
    E, A, T, S = 16, 4, 4, 2
    cfgs = [AgentConfig(model=model, radius=0.05) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0))
    rng = np.random.default_rng(23)
    pos = rng.uniform(-0.5, 0.5, size=(E, A, 2))
    pos[:, 1] = pos[:, 0]  # agents 0 and 1 coincide exactly
    pos[::2, 3] = pos[::2, 2]
    s0 = pack_state({"pos": pos}).astype(np.float32)
    acts = np.zeros((T, E, A, 2), np.float32)
    acts[1:] = rng.uniform(-1, 1, size=(T - 1, E, A, 2))
    w = np.random.default_rng(5).normal(size=(T, E, A, 16))
    w[..., 7:] = 0.0
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    # every model keeps a rollout tape here: the holonomic fleet's specialised kernels
    # their contact records, the generic kernels each substep's forces and lists
    assert st.tape_bytes(E, 2, T) > 0
    hs, hg0, hga = hip_run(st, s0, acts, w, np.float32)
    os_, og0, oga = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    assert np.isfinite(hga).all() and np.isfinite(hg0).all()
    exact = model == DynamicsModel.HOLONOMIC
    if exact:
        assert np.array_equal(hs[..., :7], os_[..., :7])
    else:
        assert rel(hs[..., :7], os_[..., :7]) <= 1e-5
    assert rel(hga, oga) <= 1e-5, rel(hga, oga)
    assert rel(hg0[..., :7], og0[..., :7]) <= 1e-5


# ------------------------------------------------------------------ tanh saturation


def test_saturated_contacts_on_specialised_kernels():
    E, A, T, S = 200, 16, 10, 4
    cfgs = nav_agents(A)
    world = nav_world(A, world_size=0.6, contact_max_overlap=0.01)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    assert st.tape_bytes(E, 2, T) > 0  # the specialised holonomic kernels run
    rng = np.random.default_rng(61)
    s0 = pack_state({"pos": rng.uniform(-0.55, 0.55, size=(E, A, 2))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = np.random.default_rng(6).normal(size=(T, E, A, 16))
    w[..., 7:] = 0.0
    hs, hg0, hga = hip_run(st, s0, acts, w, np.float32)
    os_, og0, oga = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    assert rel(hs[..., :7], os_[..., :7]) <= 1e-5
    assert rel(hga, oga) <= 1e-5, rel(hga, oga)
    assert rel(hg0[..., :7], og0[..., :7]) <= 1e-5
    o64 = oracle_run(cfgs, world, 0.05, S, s0.astype(np.float64), acts.astype(np.float64), w,
                     np.float64)
    assert rel(hga, o64[2]) <= 1.01 * rel(oga, o64[2]) + 1e-7
