"""Movable compound bodies on the HIP path (swarp/core/bodies.py:367-568) vs the CPU
oracle, and this build's body adjoint vs finite differences.  (The file name sorts after
the other GPU parity files, so a full GPU run exercises the generic and drone kernels
before these.)

Bars: the body pass computes with +, -, *, /, sqrt and a portable sin / cos evaluated
identically on host and device, so float32 agent states AND obstacle states are compared
BIT-EXACT with the float32 oracle; gradients within 1e-5 relative (max-norm) of the
oracle's.  The reference has no gradient through bodies (it skips the body pass on taped
steps, swarp/core/stepper.py:952), so the adjoint is also checked by fp64 gradcheck.
"""

import numpy as np
import pytest
import torch

from cases import body_seed_np, nav_agents, obstacles_np, oracle_cfg, params_of
from hip_helpers import check_grad, make_stepper, rel, state_to16, to_torch_state
from oracle.oracle import Oracle, pack_state
from swarp_amd import rollout
from swarp_amd.config import AgentConfig, Integrator, WorldConfig

pytestmark = pytest.mark.gpu
MOVABLE = 1
TDT = {np.float32: torch.float32, np.float64: torch.float64}


def cross_obs(E, center, d=0.2, r=0.1, mass=1.0, extra=()):
    """Config 5's body (5 circles in a rigid cross, centre circle as root) plus `extra`
    circles given as (centre, radius, movable)."""
    offs = [[0, 0], [d, 0], [-d, 0], [0, d], [0, -d]]
    inertia = sum(0.5 * (mass / 5) * r * r + (mass / 5) * (o[0] ** 2 + o[1] ** 2) for o in offs)
    centers = [[center[0] + o[0], center[1] + o[1]] for o in offs]
    radius, kind, body = [r] * 5, [MOVABLE] * 5, [0] * 5
    m, inert = [mass] * 5, [inertia] * 5
    for i, (c, rr, mov) in enumerate(extra):
        centers.append(list(c))
        radius.append(rr)
        kind.append(MOVABLE if mov else 0)
        body.append(5 + i)
        offs.append([0.0, 0.0])
        m.append(0.5)
        inert.append(0.5 * 0.5 * rr * rr)
    pos = np.broadcast_to(np.asarray(centers, dtype=np.float64), (E, len(centers), 2)).copy()
    return {"pos": pos, "radius": np.asarray(radius), "kind": np.asarray(kind, np.int32),
            "body": np.asarray(body, np.int32), "body_off": np.asarray(offs, np.float64),
            "mass": np.asarray(m), "inertia": np.asarray(inert)}


def hip_body_run(st, s0, acts, td, seed=0):
    """HIP rollout + backward of a random linear loss on the agent trajectory and the
    obstacle-state trajectory: (states, ob, g_state0, g_ob0, g_act), and the loss weights."""
    E, A = s0.shape[:2]
    T = acts.shape[0]
    ob0 = st.ob_state.detach().clone().requires_grad_(True)
    st.ob_state = ob0
    rng = np.random.default_rng(seed)
    w_st = rng.normal(size=(T, E, A, 16))
    w_st[..., 5:] = 0.0
    w_ob = rng.normal(size=(T,) + tuple(ob0.shape))
    s0t = to_torch_state(s0, td, True, 5)
    a = torch.tensor(acts, dtype=td, device="cuda", requires_grad=True)
    final, traj = rollout(st, s0t, a)
    obtr = st.ob_trajectory
    loss = (torch.tensor(w_ob, dtype=td, device="cuda") * obtr).sum()
    wt = torch.tensor(w_st, dtype=td, device="cuda")
    for t in range(T):
        loss = loss + (wt[t, ..., 0:2] * traj[t].pos).sum() + (wt[t, ..., 2] * traj[t].theta).sum() \
            + (wt[t, ..., 3:5] * traj[t].vel).sum()
    loss.backward()
    hip = (np.stack([state_to16(x) for x in traj]), obtr.detach().double().cpu().numpy(),
           s0t.pos.grad.double().cpu().numpy(), ob0.grad.double().cpu().numpy(),
           a.grad.double().cpu().numpy())
    return hip, ob0, w_st, w_ob


def run_pair(cfgs, world, dt, S, s0, acts, obs, np_dtype, seed=0):
    """HIP and oracle rollouts + backward of a random linear loss on the agent trajectory
    and the obstacle-state trajectory; returns both (states, ob, g_state0, g_ob0, g_act)."""
    E = s0.shape[0]
    td = TDT[np_dtype]
    st = make_stepper(cfgs, world, dt, S, td, obs=obs, n_envs=E)
    hip, ob0, w_st, w_ob = hip_body_run(st, s0, acts, td, seed)
    O = Oracle(np_dtype)
    cfg = oracle_cfg(cfgs, world, dt, S, E, acts.shape[-1], n_threads=8)
    p, t_, m = params_of(cfgs)
    ob = obstacles_np(obs, E)
    ob0n = ob0.detach().cpu().numpy().astype(np_dtype)
    s0n, actn = s0.astype(np_dtype), acts.astype(np_dtype)
    ost, oob = O.rollout_ob(cfg, p, t_, m, ob, s0n, ob0n, actn)
    g0, gob0, ga = O.rollout_adj_ob(cfg, p, t_, m, ob, s0n, ob0n, actn, ost, oob, w_st, None,
                                    w_ob, None)
    orc = (ost.astype(np.float64), oob.astype(np.float64), g0[..., 0:2].astype(np.float64),
           gob0.astype(np.float64), ga.astype(np.float64))
    return hip, orc


def check(name, hip, orc, exact=True, g_tol=1e-5):
    hs, hob, hg0, hgob, hga = hip
    os_, oob, og0, ogob, oga = orc
    if exact:
        assert np.array_equal(hs[..., :7], os_[..., :7]), (
            f"{name}: agent states not bit-exact (rel {rel(hs[..., :7], os_[..., :7]):.2e})")
        assert np.array_equal(hob, oob), f"{name}: obstacle states not bit-exact (rel {rel(hob, oob):.2e})"
    else:
        assert rel(hs[..., :7], os_[..., :7]) <= 1e-12 and rel(hob, oob) <= 1e-12, name
    check_grad(f"{name}: d/d actions", hga, oga, tol=g_tol)
    check_grad(f"{name}: d/d pos0", hg0, og0, tol=g_tol)
    check_grad(f"{name}: d/d ob0", hgob, ogob, tol=g_tol)


def _world(bounds=1.5, mode="soft", **kw):
    base = dict(collisions=True, collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                bounds=None if bounds is None else (-bounds, bounds, -bounds, bounds),
                bounds_mode=mode, max_neighbors=16, neighbor_radius=0.3)
    base.update(kw)
    return WorldConfig(**base)


def _pushers(E, A, seed, spread=0.6):
    rng = np.random.default_rng(seed)
    pos = rng.uniform(-spread, spread, size=(E, A, 2))
    acts = rng.uniform(-1, 1, size=(8, E, A, 2))
    # half the agents drive towards the body at the origin
    acts[..., : A // 2, :] = -pos[None, :, : A // 2, :] / np.linalg.norm(pos[None, :, : A // 2, :],
                                                                         axis=-1, keepdims=True)
    return pack_state({"pos": pos}), acts


def test_bodies_match_oracle_multi_env_waves():
    """12 agents per env (4 envs per wave, last wave partial): a cross body, a second
    movable circle and a static circle; soft walls."""
    E, A = 37, 12
    s0, acts = _pushers(E, A, 1)
    obs = cross_obs(E, (0.0, 0.0), extra=(((0.55, 0.1), 0.12, True), ((-0.5, -0.45), 0.1, False)))
    hip, orc = run_pair(nav_agents(A), _world(), 0.05, 4, s0, acts, obs, np.float32)
    check("multi-env", hip, orc)
    assert np.abs(orc[1][-1, :, 6 * 7 + 5]).max() > 1e-3, "the cross never turned"


def test_bodies_match_oracle_config5_shape():
    """Config 5's shape at reduced E: 64 agents per env (one env per wave), radius-0.3
    lists capped at K=16."""
    E, A = 6, 64
    s0, acts = _pushers(E, A, 2, spread=1.2)
    obs = cross_obs(E, (0.0, 0.0))
    hip, orc = run_pair(nav_agents(A), _world(bounds=3.0), 0.05, 4, s0, acts, obs, np.float32)
    check("config5", hip, orc)


def _coo(idx, cnt):
    """COO [2, n] (row 0 sender e*A + idx, row 1 receiver e*A + a, (e, a, slot) order) of
    padded lists, as NeighborGrid.edge_index (swarp/core/neighbors.py:716-733)."""
    E, A = cnt.shape
    snd, rcv = [], []
    for e in range(E):
        for a in range(A):
            for k in range(cnt[e, a]):
                snd.append(e * A + idx[e, a, k])
                rcv.append(e * A + a)
    return np.array([snd, rcv], dtype=np.int64).reshape(2, -1)


def test_bodies_config5_spec_against_oracle():
    """Config 5 at its specification, on 64 of its 16000 envs: 64 agents per env with
    positions U[-3, 3]^2 and actions U[-1, 1]^2 around the cross (5 circles r 0.1, mass 1,
    inertia from the geometry) in soft walls at +-3, 16 steps of 4 substeps, lists of
    radius 0.3 capped at K = 16, loss = squared distance of the body to a goal U[-2, 2]^2.
    Agent and body states bit-exact; every step's lists, counts, overflow flags and COO
    radius graph equal to the oracle's; gradients to the actions, the initial positions
    and the initial obstacle state within 1e-5 (max-norm and element-wise)."""
    E, A, T, S = 64, 64, 16, 4
    rng = np.random.default_rng(55)
    pos = rng.uniform(-3.0, 3.0, size=(E, A, 2))
    acts = rng.uniform(-1.0, 1.0, size=(T, E, A, 2)).astype(np.float32)
    goals = rng.uniform(-2.0, 2.0, size=(E, 2)).astype(np.float32)
    s0 = pack_state({"pos": pos}).astype(np.float32)
    cfgs = [AgentConfig(radius=0.05, max_speed=1.0, max_accel=2.0) for _ in range(A)]
    world = _world(bounds=3.0)
    obs = cross_obs(E, (0.0, 0.0))
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    ob0 = st.ob_state.detach().clone().requires_grad_(True)
    st.ob_state = ob0
    s0t = to_torch_state(s0, torch.float32, True, 5)
    a = torch.tensor(acts, device="cuda", requires_grad=True)
    final, traj = rollout(st, s0t, a)
    body = st.ob_trajectory[-1][:, 30:32]  # the body rooted at shape 0: its position
    loss = ((body - torch.tensor(goals, device="cuda")) ** 2).sum()
    loss.backward()
    hs = np.stack([state_to16(x) for x in traj])
    hob = st.ob_trajectory.detach().double().cpu().numpy()
    grid = st.grid(E)
    h_lists = []
    for x in traj:
        grid.build(x.pos.detach())
        idx, cnt = grid.neighbor_idx.cpu().numpy(), grid.neighbor_count.cpu().numpy()
        h_lists.append((idx, cnt, grid.overflow_view().cpu().numpy(),
                        grid.edge_index().cpu().numpy()))

    O = Oracle(np.float32)
    cfg = oracle_cfg(cfgs, world, 0.05, S, E, 2, n_threads=8)
    p, t_, m = params_of(cfgs)
    ob = obstacles_np(obs, E)
    ob0n = ob0.detach().cpu().numpy()
    ost, oob = O.rollout_ob(cfg, p, t_, m, ob, s0, ob0n, acts)
    w_ob = np.zeros(oob.shape)
    w_ob[-1, :, 30:32] = 2.0 * (oob[-1, :, 30:32].astype(np.float64) - goals)
    g0, gob0, ga = O.rollout_adj_ob(cfg, p, t_, m, ob, s0, ob0n, acts, ost, oob, None, None,
                                    w_ob, None)

    assert np.array_equal(hs[..., :7], ost[..., :7].astype(np.float64)), (
        f"agent states not bit-exact (rel {rel(hs[..., :7], ost[..., :7]):.2e})")
    assert np.array_equal(hob, oob.astype(np.float64)), "body states not bit-exact"
    n_over = n_edges = 0
    for k, (idx, cnt, over, coo) in enumerate(h_lists):
        oi, oc, ot = O.neighbors(ost[k, ..., 0:2], 0.3, 16)
        assert np.array_equal(cnt, oc), f"step {k}: counts differ"
        for e in range(E):
            for i in range(A):
                assert np.array_equal(idx[e, i, :cnt[e, i]], oi[e, i, :oc[e, i]]), f"step {k}: lists differ"
        assert np.array_equal(over, ot > oc), f"step {k}: overflow flags differ"
        assert np.array_equal(coo, _coo(oi, oc)), f"step {k}: COO differs"
        n_over += int(over.sum())
        n_edges += coo.shape[1]
    print(f"\nconfig5 spec: {n_edges} edges and {n_over} overflowing lists over {T} steps")
    assert n_edges > 0
    check_grad("config5 spec d/d actions", a.grad.double().cpu().numpy(), ga)
    check_grad("config5 spec d/d pos0", s0t.pos.grad.double().cpu().numpy(), g0[..., 0:2])
    check_grad("config5 spec d/d ob0", ob0.grad.double().cpu().numpy(), gob0)
    assert np.abs(ga).max() > 0, "no gradient reached the actions"



def _ring_extra(n, radius=1.0, r=0.07):
    """n circles on a ring around the cross, every third one static."""
    ang = np.linspace(0.0, 2 * np.pi, n, endpoint=False)
    return tuple(((radius * np.cos(a), radius * np.sin(a)), r, k % 3 != 2)
                 for k, a in enumerate(ang))


@pytest.mark.parametrize("A,n_extra", [(64, 35), (16, 19), (16, 59), (16, 75), (64, 195)])
def test_bodies_beyond_sixteen_obstacles(A, n_extra):
    """More than 16 obstacles per env (each env's obstacle state staged in LDS sized by the
    obstacle count): the cross body and a ring of movable and static circles, one env per
    wave at 64 agents and four per wave at 16.  64 shapes is the most the instances that
    keep the shape sets as wave masks take; 80 runs the instances that test the shapes
    one by one; 200 needs a backward workgroup of more than 64 KiB of LDS."""
    E = 6 if A == 64 else 9
    s0, acts = _pushers(E, A, 3, spread=1.2)
    obs = cross_obs(E, (0.0, 0.0), extra=_ring_extra(n_extra))
    hip, orc = run_pair(nav_agents(A), _world(bounds=2.0), 0.05, 4, s0, acts, obs, np.float32)
    check(f"{5 + n_extra} obstacles", hip, orc)
    assert np.abs(orc[1][-1] - orc[1][0]).max() > 1e-3, "no body moved"


@pytest.mark.parametrize("A,n_extra,roots,np_dtype", [
    (64, 0, None, np.float32),   # config 5's body
    (16, 19, None, np.float32),  # several movable bodies, four envs per wave
    (16, 19, 2, np.float32),     # a tape of the first two bodies: the others evaluated
    (8, 6, None, np.float64),
])
def test_body_tape_matches_recompute(A, n_extra, roots, np_dtype):
    """The backward reading each substep's body pass from the forward's body tape against
    the backward evaluating it again: the same values reach the same arithmetic in the
    same order, so states and every gradient are equal bit for bit.  With `roots` the
    tape holds only the first bodies in root order and the backward evaluates the rest."""
    E, S = 7, 4
    s0, acts = _pushers(E, A, 11, spread=1.0)
    obs = cross_obs(E, (0.0, 0.0), extra=_ring_extra(n_extra, radius=0.6) if n_extra else ())
    td = TDT[np_dtype]
    runs = []
    for tape in (True, False):
        st = make_stepper(nav_agents(A), _world(), 0.05, S, td, obs=obs, n_envs=E)
        st.use_tape = tape
        if tape and roots is not None:
            assert st.n_body_roots > roots
            st.n_body_roots = roots
        assert (st.ob_tape_bytes(E, 2, acts.shape[0]) > 0) == tape
        runs.append(hip_body_run(st, s0, acts, td, seed=3)[0])
    names = ("agent states", "obstacle states", "d/d pos0", "d/d ob0", "d/d actions")
    for name, x, y in zip(names, runs[0], runs[1]):
        assert np.array_equal(x, y), f"{name} differ between the taped and recomputed backward"
    assert np.abs(runs[0][4]).max() > 0 and np.abs(runs[0][1][-1] - runs[0][1][0]).max() > 1e-4


@pytest.mark.parametrize("A,E,method,np_dtype", [
    (128, 4, "brute", np.float32),
    (512, 2, "brute", np.float32),
    (100, 3, "uniform_grid", np.float32),
    (72, 2, "brute", np.float64),
])
def test_bodies_wide_envs_match_oracle(A, E, method, np_dtype):
    """Movable bodies in envs of more than 64 agents, and with grid-ordered lists: the wide
    kernels (one workgroup of ceil(A / 64) waves per env, the body pass's sums over the
    env's waves in agent order).  Agent and obstacle states bit-exact with the oracle,
    gradients within the bars."""
    s0, acts = _pushers(E, A, 17, spread=1.4)
    obs = cross_obs(E, (0.0, 0.0), extra=_ring_extra(4, radius=0.7))
    world = _world(bounds=2.0, neighbor_method=method)
    hip, orc = run_pair(nav_agents(A), world, 0.05, 4, s0, acts, obs, np_dtype)
    check(f"{A} agents per env, {method} lists", hip, orc, exact=True,
          g_tol=1e-5 if np_dtype == np.float32 else 1e-12)
    assert np.abs(orc[1][-1] - orc[1][0]).max() > 1e-3, "no body moved"


def test_bodies_few_agents_many_obstacles():
    """4 agents per env with 13 obstacles: at 16 env slots per wave the backward's obstacle
    staging would exceed 64 KiB of LDS, so the body kernels run wider env slots (pad lanes)."""
    E, A = 10, 4
    s0, acts = _pushers(E, A, 5)
    obs = cross_obs(E, (0.0, 0.0), extra=_ring_extra(8, radius=0.5))
    hip, orc = run_pair(nav_agents(A), _world(), 0.05, 4, s0, acts, obs, np.float32)
    check("4 agents, 13 obstacles", hip, orc)
    assert np.abs(orc[1][-1] - orc[1][0]).max() > 1e-3, "no body moved"


def test_bodies_obstacle_count_beyond_lds_is_rejected():
    """An obstacle count whose backward staging exceeds the 160 KiB of LDS of a workgroup
    even at one env per wave (float64, 250 obstacles) is refused by the host -- when a
    gradient is required, before the forward runs, so the stepper's obstacle state is not
    advanced; a no-grad rollout of the same world still runs."""
    E, A = 3, 4
    s0, acts = _pushers(E, A, 4)
    obs = cross_obs(E, (0.0, 0.0), extra=_ring_extra(245, radius=1.5, r=0.01))
    with pytest.raises(RuntimeError, match="LDS"):
        run_pair(nav_agents(A), _world(), 0.05, 4, s0, acts, obs, np.float64)
    st = make_stepper(nav_agents(A), _world(), 0.05, 4, torch.float64, obs=obs, n_envs=E)
    before = st.ob_state.detach().clone()
    s0t = to_torch_state(s0, torch.float64, True, 5)
    a = torch.tensor(acts, dtype=torch.float64, device="cuda", requires_grad=True)
    with pytest.raises(RuntimeError, match="LDS"):
        rollout(st, s0t, a)
    assert torch.equal(st.ob_state.detach(), before) and st.ob_trajectory is None
    with torch.no_grad():
        rollout(st, s0t, a)
    assert st.ob_trajectory is not None and st.ob_trajectory.shape[0] == acts.shape[0]


def test_bodies_wide_env_many_obstacles():
    """1024 agents per env with 40 obstacles: the wide body backward's staging (agents,
    five obstacle states) needs more than 64 KiB of LDS."""
    E, A = 1, 1024
    s0, acts = _pushers(E, A, 5, spread=1.4)
    obs = cross_obs(E, (0.0, 0.0), extra=_ring_extra(35, radius=0.9, r=0.04))
    hip, orc = run_pair(nav_agents(A), _world(bounds=2.0), 0.05, 4, s0, acts, obs, np.float32)
    check("1024 agents, 40 obstacles", hip, orc, exact=True)

def test_bodies_clamp_bounds():
    E, A = 8, 8
    s0, acts = _pushers(E, A, 3, spread=0.4)
    acts[...] = np.array([1.0, 0.0])
    obs = cross_obs(E, (0.15, 0.0))
    hip, orc = run_pair(nav_agents(A), _world(bounds=0.55, mode="clamp"), 0.05, 4, s0, acts, obs,
                        np.float32)
    check("clamp", hip, orc)


def test_bodies_float64_matches_float64_oracle():
    E, A = 5, 6
    s0, acts = _pushers(E, A, 4, spread=0.4)
    obs = cross_obs(E, (0.0, 0.0), extra=(((0.4, 0.0), 0.1, True),))
    hip, orc = run_pair(nav_agents(A), _world(), 0.05, 2, s0, acts, obs, np.float64)
    check("f64", hip, orc, exact=True, g_tol=1e-12)


def test_bodies_with_rk4_agents():
    """Integrator.RK4 inside the body kernels' substeps: bit-exact agent and body states."""
    E, A = 16, 8
    s0, acts = _pushers(E, A, 5, spread=0.5)
    obs = cross_obs(E, (0.0, 0.0), extra=(((0.45, 0.1), 0.1, True),))
    hip, orc = run_pair(nav_agents(A), _world(integrator=Integrator.RK4), 0.05, 4, s0, acts, obs,
                        np.float32)
    check("rk4", hip, orc)


def test_body_gradcheck_fp64():
    """torch.autograd.gradcheck through rollout with a movable body: d(final body state,
    final agent positions)/d(actions, initial obstacle state)."""
    E, A, T = 2, 3, 3
    cfgs = nav_agents(A, max_speed=100.0)
    world = _world(collision_k=40.0, collision_c=0.5, bounds=None)
    obs = cross_obs(E, (0.0, 0.0), d=0.15, r=0.08, extra=(((0.33, 0.05), 0.09, True),))
    st = make_stepper(cfgs, world, 0.05, 2, torch.float64, obs=obs, n_envs=E)
    base_ob = st.ob_state.detach().clone()
    pos = torch.tensor([[[-0.2, 0.03], [0.1, -0.19], [0.05, 0.24]],
                        [[-0.21, -0.02], [0.12, 0.2], [0.42, 0.1]]], dtype=torch.float64,
                       device="cuda")
    z = torch.zeros(E, A, dtype=torch.float64, device="cuda")
    acts0 = torch.tensor(np.random.default_rng(5).normal(size=(T, E, A, 2)) * 0.5,
                         dtype=torch.float64, device="cuda")

    def f(acts, ob0):
        st.ob_state = ob0
        from swarp_amd import TorchState
        s = TorchState(pos, z, torch.zeros(E, A, 2, dtype=torch.float64, device="cuda"), z, z)
        final, _ = rollout(st, s, acts)
        return final.pos, st.ob_state

    assert torch.autograd.gradcheck(f, (acts0.clone().requires_grad_(True),
                                        base_ob.clone().requires_grad_(True)),
                                    eps=1e-6, atol=1e-5, rtol=1e-4)


def test_grad_and_nograd_forward_agree_and_state_advances():
    E, A = 4, 8
    s0, acts = _pushers(E, A, 6, spread=0.5)
    obs = cross_obs(E, (0.0, 0.0))
    st = make_stepper(nav_agents(A), _world(), 0.05, 4, torch.float32, obs=obs, n_envs=E)
    ob0 = st.ob_state.clone()
    a = torch.tensor(acts, dtype=torch.float32, device="cuda")
    with torch.no_grad():
        f1, _ = rollout(st, to_torch_state(s0, torch.float32, False, 5), a)
    ob1 = st.ob_state.clone()
    st.ob_state = ob0.clone()
    f2, _ = rollout(st, to_torch_state(s0, torch.float32, True, 5), a.clone().requires_grad_(True))
    assert torch.equal(f1.pos, f2.pos.detach()) and torch.equal(ob1, st.ob_state.detach())
    assert not torch.equal(ob1, ob0), "the obstacle state did not advance"


def _run_fields(cfgs, world, dt, S, s0, acts, obs, np_dtype, seed=0, per_env=None):
    """run_pair for any fleet: every stepped field (nine with drones) enters the loss and
    the comparison; `per_env` ([E, A, 22]) installs per-env agent rows, and the oracle then
    runs each env on its own rows with the shared table as the body pass's rows."""
    from hip_helpers import FIELDS
    from oracle.oracle import OFFSET, WIDTH
    E, A = s0.shape[:2]
    T = acts.shape[0]
    td = TDT[np_dtype]
    nf = 9 if any(int(c.model) == 3 for c in cfgs) else 5
    st = make_stepper(cfgs, world, dt, S, td, obs=obs, n_envs=E)
    if per_env is not None:
        st.set_agent_params_per_env(torch.tensor(per_env, dtype=td))
    ob0 = st.ob_state.detach().clone().requires_grad_(True)
    st.ob_state = ob0
    rng = np.random.default_rng(seed)
    w_st = rng.normal(size=(T, E, A, 16))
    if nf == 5:
        w_st[..., 7:] = 0.0
    w_ob = rng.normal(size=(T,) + tuple(ob0.shape))
    s0t = to_torch_state(s0, td, True, nf)
    a = torch.tensor(acts, dtype=td, device="cuda", requires_grad=True)
    final, traj = rollout(st, s0t, a)
    obtr = st.ob_trajectory
    loss = (torch.tensor(w_ob, dtype=td, device="cuda") * obtr).sum()
    wt = torch.tensor(w_st, dtype=td, device="cuda")
    for t in range(T):
        for k, (name, w, o) in enumerate(zip(FIELDS, WIDTH, OFFSET)):
            if k >= nf:
                continue
            ww = wt[t, ..., o:o + w]
            loss = loss + ((ww[..., 0] if w == 1 else ww) * getattr(traj[t], name)).sum()
    loss.backward()
    g0 = np.zeros((E, A, 16))
    for k, (name, w, o) in enumerate(zip(FIELDS, WIDTH, OFFSET)):
        if k < nf and getattr(s0t, name).grad is not None:
            g0[..., o:o + w] = getattr(s0t, name).grad.double().cpu().numpy().reshape(E, A, w)
    hip = (np.stack([state_to16(x) for x in traj]), obtr.detach().double().cpu().numpy(), g0,
           ob0.grad.double().cpu().numpy(), a.grad.double().cpu().numpy())
    O = Oracle(np_dtype)
    p, t_, m = params_of(cfgs)
    ob = obstacles_np(obs, E)
    ob0n = ob0.detach().cpu().numpy().astype(np_dtype)
    s0n, actn = s0.astype(np_dtype), acts.astype(np_dtype)
    if per_env is None:
        groups = [(slice(0, E), p, ob)]
    else:
        groups = []
        for e in range(E):
            obe = {k: (v[e:e + 1] if k in ("pos", "angle", "vel", "ang_vel") else v)
                   for k, v in ob.items()}
            obe["body_params"] = p
            groups.append((slice(e, e + 1), per_env[e], obe))
    ost = np.zeros((T, E, A, 16))
    oob = np.zeros((T,) + tuple(ob0.shape))
    og0, ogob, oga = np.zeros((E, A, 16)), np.zeros(tuple(ob0.shape)), np.zeros(acts.shape)
    for sl, pe, obe in groups:
        n = sl.stop - sl.start
        cfg = oracle_cfg(cfgs, world, dt, S, n, acts.shape[-1], n_threads=8)
        s_, o_ = O.rollout_ob(cfg, pe, t_, m, obe, s0n[sl], ob0n[sl], actn[:, sl])
        g0_, gob_, ga_ = O.rollout_adj_ob(cfg, pe, t_, m, obe, s0n[sl], ob0n[sl], actn[:, sl],
                                          s_, o_, w_st[:, sl], None, w_ob[:, sl], None)
        ost[:, sl], oob[:, sl], og0[sl], ogob[sl], oga[:, sl] = s_, o_, g0_, gob_, ga_
    cols = slice(0, 16) if nf == 9 else slice(0, 7)
    return hip, (ost, oob, og0, ogob, oga), cols


def _check_fields(name, hip, orc, cols, exact=True, g_tol=1e-5):
    hs, hob, hg0, hgob, hga = hip
    os_, oob, og0, ogob, oga = orc
    print(f"\n{name}: states rel {rel(hs[..., cols], os_[..., cols]):.2e}, ob rel {rel(hob, oob):.2e}, "
          f"d/d actions {rel(hga, oga):.2e}, d/d state0 {rel(hg0[..., cols], og0[..., cols]):.2e}, "
          f"d/d ob0 {rel(hgob, ogob):.2e}")
    if exact:
        assert np.array_equal(hs[..., cols], os_[..., cols]), (
            f"{name}: agent states not bit-exact (rel {rel(hs[..., cols], os_[..., cols]):.2e})")
        assert np.array_equal(hob, oob), f"{name}: obstacle states not bit-exact (rel {rel(hob, oob):.2e})"
    else:
        assert rel(hs[..., cols], os_[..., cols]) <= 1e-12 and rel(hob, oob) <= 1e-12, name
    assert rel(hga, oga) <= g_tol, f"{name}: d/d actions rel {rel(hga, oga):.3e}"
    assert rel(hg0[..., cols], og0[..., cols]) <= g_tol, f"{name}: d/d state0 rel {rel(hg0, og0):.3e}"
    assert rel(hgob, ogob) <= g_tol, f"{name}: d/d ob0 rel {rel(hgob, ogob):.3e}"


@pytest.mark.parametrize("np_dtype", [np.float32, np.float64])
def test_bodies_with_drones(np_dtype):
    """A drone fleet (config 4's quadrotors) flying into the cross body and a second
    movable circle: every one of the nine state fields and the obstacle states bit-exact,
    gradients 1e-5 (fp32) / 1e-12 (fp64) of the oracle."""
    from swarp_amd.config import AgentConfig, DynamicsModel
    E, A, T = 24, 8, 10
    rng = np.random.default_rng(11)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0) for _ in range(A)]
    pos = rng.uniform(-0.7, 0.7, size=(E, A, 2))
    vel = -0.6 * pos / np.linalg.norm(pos, axis=-1, keepdims=True)
    ax = rng.normal(size=(E, A, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(E, A, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    s0 = pack_state({"pos": pos, "vel": vel, "z": np.ones((E, A)), "attitude": q})
    acts = rng.uniform(0, 1, size=(T, E, A, 4)) * 10.0
    obs = cross_obs(E, (0.0, 0.0), extra=(((0.5, 0.2), 0.12, True),))
    hip, orc, cols = _run_fields(cfgs, _world(), 0.02, 2, s0, acts, obs, np_dtype, seed=3)
    _check_fields("drones", hip, orc, cols, exact=True, g_tol=1e-5 if np_dtype == np.float32 else 1e-12)
    assert np.abs(orc[1][-1, :, 6 * 5 + 3:6 * 5 + 5]).max() > 1e-3, "the drones never pushed the cross"


def test_bodies_with_per_env_parameter_rows():
    """Per-env agent rows (Stepper.set_agent_params_per_env) with a movable body: the
    agents step on their env's rows and the body pass reads the shared table, as the
    reference's launch_obstacle_dynamics does (swarp/core/stepper.py:961-964).  Each env
    equals an independent oracle rollout with its rows; the body states would differ if
    the body pass read the per-env rows."""
    from swarp_amd import per_env_float_template
    E, A = 12, 8
    s0, acts = _pushers(E, A, 12, spread=0.5)
    cfgs = nav_agents(A)
    rows = np.array(per_env_float_template(cfgs, E), dtype=np.float64)
    rng = np.random.default_rng(13)
    rows[..., 0] = rng.uniform(0.04, 0.08, size=(E, A))   # radius
    rows[..., 1] = rng.uniform(0.5, 2.0, size=(E, A))     # mass
    obs = cross_obs(E, (0.0, 0.0))
    hip, orc, cols = _run_fields(cfgs, _world(), 0.05, 4, s0, acts, obs, np.float32, seed=4,
                                 per_env=rows)
    _check_fields("per-env", hip, orc, cols)
    # the same rollout with the body pass on the per-env rows moves the body differently
    O = Oracle(np.float32)
    ob = obstacles_np(obs, E)
    e = 0
    obe = {k: (v[e:e + 1] if k in ("pos", "angle", "vel", "ang_vel") else v) for k, v in ob.items()}
    p, t_, m = params_of(cfgs)
    cfg = oracle_cfg(cfgs, _world(), 0.05, 4, 1, 2, n_threads=1)
    _, o_own = O.rollout_ob(cfg, rows[e].astype(np.float32), t_, m, obe,
                            s0[e:e + 1].astype(np.float32), body_seed_np(obe).astype(np.float32),
                            acts[:, e:e + 1].astype(np.float32))
    assert not np.array_equal(o_own, orc[1][:, e:e + 1]), "the test cannot tell the tables apart"


def shaped_obs(E, th=0.3):
    """A box + capsule compound body (box root at the origin, capsule offset in the body
    frame), a movable box body near the capsule, a static circle under the box and a
    movable circle by its side: every shape-type pairing of the body pass."""
    off1 = np.array([0.05, 0.21])
    c1 = [np.cos(th) * off1[0] - np.sin(th) * off1[1], np.sin(th) * off1[0] + np.cos(th) * off1[1]]
    centers = [[0.0, 0.0], c1, [c1[0] + 0.01, c1[1] + 0.1], [0.0, -0.2], [0.2, -0.1]]
    pos = np.broadcast_to(np.asarray(centers), (E, 5, 2)).copy()
    return {"pos": pos, "radius": np.array([0.0, 0.04, 0.0, 0.08, 0.06]),
            "type": np.array([1, 2, 1, 0, 0], np.int32),
            "half": np.array([[0.12, 0.07], [0.15, 0.0], [0.06, 0.05], [0.0, 0.0], [0.0, 0.0]]),
            "angle": np.broadcast_to(np.array([th, th, -0.4, 0.0, 0.0]), (E, 5)).copy(),
            "kind": np.array([MOVABLE, MOVABLE, MOVABLE, 0, MOVABLE], np.int32),
            "body": np.array([0, 0, 2, 3, 4], np.int32),
            "body_off": np.array([[0.0, 0.0], list(off1), [0.0, 0.0], [0.0, 0.0], [0.0, 0.0]]),
            "mass": np.array([0.8, 0.8, 0.5, 1.0, 0.4]),
            "inertia": np.array([0.04, 0.04, 0.02, 1.0, 0.01])}


@pytest.mark.parametrize("np_dtype", [np.float32, np.float64])
def test_box_and_segment_bodies_match_oracle(np_dtype):
    """Box and capsule shapes on movable bodies (the reference's body pass for every shape
    type, swarp/core/bodies.py:80-253): agent reactions with the lever to the agent's
    centre on a box and the closest core point on a capsule, the body-body terms box vs
    circle, box vs capsule, capsule vs box, circle vs box, and the agents' forces from
    moving boxes and capsules.  Agent and obstacle states bit-exact; gradients 1e-5 (fp32)
    / 1e-12 (fp64) of the oracle."""
    E, A = 20, 6
    rng = np.random.default_rng(21)
    ang = rng.uniform(0, 2 * np.pi, size=(E, A))
    rad = rng.uniform(0.3, 0.45, size=(E, A))
    pos = np.stack([rad * np.cos(ang), rad * np.sin(ang)], -1)
    s0 = pack_state({"pos": pos})
    acts = np.broadcast_to(-pos / np.linalg.norm(pos, axis=-1, keepdims=True), (8, E, A, 2)).copy()
    acts += rng.uniform(-0.3, 0.3, size=acts.shape)
    obs = shaped_obs(E)
    hip, orc, cols = _run_fields(nav_agents(A, agent_radius=0.06), _world(bounds=None), 0.05, 2,
                                 s0, acts, obs, np_dtype, seed=5)
    _check_fields("shapes", hip, orc, cols, exact=True,
                  g_tol=1e-5 if np_dtype == np.float32 else 1e-12)
    assert np.abs(orc[1][-1, :, 6 * 5 + 5]).max() > 1e-4, "the compound body never turned"


def test_bodies_heterogeneous_radii_wide_lists():
    """Per-agent radii from 0.02 to 0.1 under radius-0.3 lists (K = 6, truncated): the
    agent-pair pass visits only listed neighbours within the env's contact bound, set by
    its largest radius.  Agent and body states bit-exact, gradients 1e-5."""
    E, A = 24, 16
    s0, acts = _pushers(E, A, 5, spread=0.7)
    rng = np.random.default_rng(6)
    radii = np.linspace(0.02, 0.1, A)[rng.permutation(A)]
    cfgs = [AgentConfig(radius=float(r), max_speed=1.0, max_accel=2.0) for r in radii]
    obs = cross_obs(E, (0.0, 0.0))
    hip, orc = run_pair(cfgs, _world(max_neighbors=6), 0.05, 4, s0, acts, obs, np.float32)
    check("hetero radii", hip, orc)
