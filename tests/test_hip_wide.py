"""Envs of more than 64 agents, and the uniform-grid list order, on the HIP path (the
wide-env kernels: one workgroup per env) vs the CPU oracle.

Bars: neighbour lists, counts, true counts and batch-reduced grid frames BIT-EXACT;
float32 states BIT-EXACT (the same op order and portable transcendentals as the oracle);
gradients within 1e-5 relative (max-norm) of the float32 oracle -- the backward gathers
both sides of each pair where the oracle scatters them, a different summation order --
and float64 states and gradients within 1e-12.
"""

import numpy as np
import pytest
import torch

from cases import obstacles_np  # noqa: F401  (make_stepper converts obstacle dicts)
from hip_helpers import hip_run, make_stepper, oracle_run, rel
from oracle.oracle import Oracle, pack_state
from swarp_amd import NeighborGrid
from swarp_amd.config import AgentConfig, ControlMode, DynamicsModel, Integrator, WorldConfig

pytestmark = pytest.mark.gpu


def _bins(A):
    return max(4, min(128, int(np.ceil(np.sqrt(A)))))


def _lists(g, pos):
    g.build(torch.tensor(pos, device="cuda:0"))
    torch.cuda.synchronize()
    return (g.neighbor_idx.cpu().numpy(), g.neighbor_count.cpu().numpy(),
            g.neighbor_true_count.cpu().numpy())


@pytest.mark.parametrize("A,K,r", [(100, 16, 0.3), (256, 8, 0.5), (1024, 32, 0.15),
                                   (1500, 16, 0.1), (3000, 12, 0.08)])
def test_wide_brute_lists_bitexact(A, K, r):
    E = 5
    rng = np.random.default_rng(A)
    pos = ((rng.random((E, A, 2)) * 2 - 1) * 2.0).astype(np.float32)
    g = NeighborGrid(E, A, radius=r, max_neighbors=K, device="cuda:0", method="brute")
    idx, cnt, tru = _lists(g, pos)
    oi, oc, ot = Oracle(np.float32).neighbors(pos, r, K)
    print(f"\nbrute A={A}: mean true count {ot.mean():.2f}, capped {(ot > K).mean():.3f}")
    assert np.array_equal(cnt, oc) and np.array_equal(tru, ot) and np.array_equal(idx, oi)


@pytest.mark.parametrize("A,pinned,extent,K", [(600, False, 2.2, 16), (600, True, 2.2, 16),
                                               (40, False, 2.2, 16), (1000, True, 2.2, 16),
                                               (600, True, 1.0, 6), (2500, True, 2.2, 8),
                                               (1200, False, 1.0, 6)])
def test_grid_lists_bitexact(A, pinned, extent, K):
    """extent 1.0 with K = 6: most lists are capped, so the order decides the members."""
    E, r = 3, 0.15
    rng = np.random.default_rng(A + pinned)
    pos = ((rng.random((E, A, 2)) * 2 - 1) * extent).astype(np.float32)  # 2.2: some beyond +-2
    bounds = (-2.0, 2.0, -2.0, 2.0) if pinned else None
    g = NeighborGrid(E, A, radius=r, max_neighbors=K, device="cuda:0", method="uniform_grid",
                     bounds=bounds)
    idx, cnt, tru = _lists(g, pos)
    bins = _bins(A)
    frame = (-2.0, -2.0, max(r, 4.0 / bins)) if pinned else None
    oi, oc, ot, ofr = Oracle(np.float32).neighbors_grid(pos, r, K, bins, frame)
    print(f"\ngrid A={A} pinned={pinned}: frame {ofr}, capped {(ot > K).mean():.3f}")
    if not pinned:
        assert np.array_equal(g.grid_frame().cpu().numpy(), ofr)
    assert np.array_equal(cnt, oc) and np.array_equal(tru, ot) and np.array_equal(idx, oi)
    if A >= 600:  # dense enough that lists span several cells: the orders differ
        bi, _, _ = Oracle(np.float32).neighbors(pos, r, K)
        assert not np.array_equal(idx, bi)


def test_grid_lists_float64():
    E, A, K, r = 2, 300, 24, 0.2
    rng = np.random.default_rng(5)
    pos = (rng.random((E, A, 2)) * 2 - 1) * 2.0
    g = NeighborGrid(E, A, radius=r, max_neighbors=K, device="cuda:0", dtype=torch.float64,
                     method="uniform_grid")
    idx, cnt, tru = _lists(g, pos)
    oi, oc, ot, ofr = Oracle(np.float64).neighbors_grid(pos, r, K, _bins(A))
    assert np.array_equal(g.grid_frame().cpu().numpy(), ofr)
    assert np.array_equal(cnt, oc) and np.array_equal(tru, ot) and np.array_equal(idx, oi)


def _cot(T, E, A, seed, nf=5, scale=1.0):
    w = np.random.default_rng(seed).normal(size=(T, E, A, 16)) * scale
    if nf == 5:
        w[..., 7:] = 0.0
    return w


def _check(name, hip, orc, g_tol=1e-5, cols=slice(0, 7), exact=True):
    hs, hg0, hga = hip
    os_, og0, oga = orc
    es, ea, e0 = rel(hs[..., cols], os_[..., cols]), rel(hga, oga), rel(hg0[..., cols], og0[..., cols])
    print(f"\n{name}: states rel {es:.3e}, d/d actions rel {ea:.3e}, d/d state0 rel {e0:.3e}")
    if exact:
        assert np.array_equal(hs[..., cols], os_[..., cols]), f"{name}: states not bit-exact"
    else:
        assert es <= g_tol, name
    assert ea <= g_tol and e0 <= g_tol, name


def _obstacles(E, rng):
    n = 4
    return {"pos": rng.uniform(-1.2, 1.2, size=(E, n, 2)),
            "radius": np.array([0.15, 0.1, 0.0, 0.03]),
            "type": np.array([0, 0, 1, 2], dtype=np.int32),
            "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
            "half": np.array([[0.0, 0.0], [0.0, 0.0], [0.2, 0.1], [0.25, 0.0]])}


def test_wide_step_mixed_fleet_brute():
    """100 agents per env (holonomic, diff-drive, bicycle), obstacles of every shape, soft
    walls, capped lists in index order, 2 substeps, 5 steps."""
    E, A, T, S = 6, 100, 5, 2
    rng = np.random.default_rng(21)
    cfgs = ([AgentConfig(radius=0.04) for _ in range(40)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.04) for _ in range(30)]
            + [AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, radius=0.04) for _ in range(30)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02,
                        bounds=(-1.5, 1.5, -1.5, 1.5), max_neighbors=12, neighbor_radius=0.25)
    obs = _obstacles(E, rng)
    s0 = pack_state({"pos": rng.uniform(-1.4, 1.4, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cot(T, E, A, 22)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    assert st.wide and st.list_method == "brute"
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32, obs=obs)
    _check("wide brute A=100", hip, orc)


def test_wide_step_grid_pinned_600():
    """600 agents per env: "auto" picks the uniform grid (the reference's rule above 512),
    the world bounds pin its frame; spawned in [-1, 1]^2 with K = 4, most lists are
    capped, so the grid's order decides which neighbours act."""
    E, A, T, S = 3, 600, 3, 2
    rng = np.random.default_rng(23)
    cfgs = ([AgentConfig(radius=0.03) for _ in range(300)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.03) for _ in range(300)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.015,
                        bounds=(-1.5, 1.5, -1.5, 1.5), max_neighbors=4, neighbor_radius=0.12)
    s0 = pack_state({"pos": rng.uniform(-1.0, 1.0, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cot(T, E, A, 24)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    assert st.wide and st.list_method == "uniform_grid"
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    _check("wide grid A=600", hip, orc)



def test_wide_step_grid_100_bins():
    """uniform_bins = 100 (10000 cells per env): the cell table and 600 agents' staging take
    the workgroup beyond 64 KiB of LDS.  Lists bit-exact, states bit-exact with the oracle
    stepping in the same grid order."""
    E, A, T, S = 2, 600, 3, 2
    rng = np.random.default_rng(25)
    cfgs = ([AgentConfig(radius=0.03) for _ in range(300)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.03) for _ in range(300)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.015,
                        bounds=(-1.5, 1.5, -1.5, 1.5), max_neighbors=4, neighbor_radius=0.12,
                        neighbor_method="uniform_grid", uniform_bins=100)
    pos = rng.uniform(-1.0, 1.0, size=(E, A, 2))
    g = NeighborGrid(E, A, radius=0.05, max_neighbors=6, device="cuda:0", method="uniform_grid",
                     uniform_bins=100)
    gi, gc, gt = _lists(g, pos.astype(np.float32))
    oi, oc, ot, _ = Oracle(np.float32).neighbors_grid(pos.astype(np.float32), 0.05, 6, 100)
    assert np.array_equal(gc, oc) and np.array_equal(gt, ot) and np.array_equal(gi, oi)
    s0 = pack_state({"pos": pos, "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cot(T, E, A, 26)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    assert st.wide and st.list_method == "uniform_grid"
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    _check("grid A=600 bins=100", hip, orc)


@pytest.mark.parametrize("A,method,np_dtype", [(1500, "brute", np.float32),
                                               (3000, "uniform_grid", np.float32),
                                               (1100, "uniform_grid", np.float64)])
def test_wide_step_beyond_1024_agents(A, method, np_dtype):
    """Envs of more than 1024 agents: 2 or 4 agents per thread of the env's workgroup
    (1100 and 1500: 2 per thread; 3000: 4).  A mixed fleet among obstacles inside soft
    walls, lists capped at K = 6; states bit-exact with the oracle, gradients within the
    bars."""
    E, T, S = 1, 3, 2
    rng = np.random.default_rng(A)
    h = A // 2
    cfgs = ([AgentConfig(radius=0.02) for _ in range(h)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.02) for _ in range(A - h)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.01,
                        bounds=(-1.6, 1.6, -1.6, 1.6), max_neighbors=6, neighbor_radius=0.08,
                        neighbor_method=method)
    s0 = pack_state({"pos": rng.uniform(-1.5, 1.5, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np_dtype)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np_dtype)
    w = _cot(T, E, A, A + 1)
    obs = _obstacles(E, rng)
    td = torch.float32 if np_dtype == np.float32 else torch.float64
    st = make_stepper(cfgs, world, 0.05, S, td, obs=obs, n_envs=E)
    assert st.wide
    hip = hip_run(st, s0, acts, w, np_dtype)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np_dtype, obs=obs)
    f32 = np_dtype == np.float32
    _check(f"wide A={A} {method}", hip, orc, g_tol=1e-5 if f32 else 1e-12, exact=f32)

def test_grid_step_small_env():
    """A 32-agent env with uniform_grid lists asked for explicitly (the wide kernels serve
    every grid-ordered world)."""
    E, A, T, S = 16, 32, 6, 2
    rng = np.random.default_rng(25)
    cfgs = [AgentConfig(radius=0.05) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-0.6, 0.6, -0.6, 0.6), max_neighbors=4,
                        neighbor_method="uniform_grid")
    s0 = pack_state({"pos": rng.uniform(-0.6, 0.6, size=(E, A, 2))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cot(T, E, A, 26)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    assert st.wide
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    _check("grid A=32", hip, orc)


def test_wide_step_drones():
    E, A, T, S = 4, 72, 6, 1
    rng = np.random.default_rng(27)
    cfgs = [AgentConfig(model=DynamicsModel.DRONE, radius=0.1, thrust_max=10.0) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.02)
    ax = rng.normal(size=(E, A, 3))
    ax /= np.linalg.norm(ax, axis=-1, keepdims=True)
    ang = rng.uniform(0, 0.1, size=(E, A, 1))
    q = np.concatenate([ax * np.sin(ang / 2), np.cos(ang / 2)], -1)
    s0 = pack_state({"pos": rng.uniform(-1.5, 1.5, size=(E, A, 2)), "z": np.ones((E, A)),
                     "attitude": q}).astype(np.float32)
    acts = (rng.uniform(0, 1, size=(T, E, A, 4)) * 10.0).astype(np.float32)
    w = _cot(T, E, A, 28, nf=9, scale=0.01)
    st = make_stepper(cfgs, world, 0.02, S, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.02, S, s0, acts, w, np.float32)
    _check("wide drones A=72", hip, orc, cols=slice(0, 16))


def test_wide_step_rk4_control_modes():
    """RK4 with holonomic ACCELERATION and diff-drive SERVO agents, walls, 80 agents."""
    E, A, T, S = 4, 80, 4, 2
    rng = np.random.default_rng(29)
    cfgs = ([AgentConfig(ctrl_mode=ControlMode.ACCELERATION, radius=0.05) for _ in range(40)]
            + [AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.SERVO,
                           radius=0.05) for _ in range(40)])
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0), max_neighbors=10,
                        integrator=Integrator.RK4)
    s0 = pack_state({"pos": rng.uniform(-1.0, 1.0, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = _cot(T, E, A, 30)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32)
    hip = hip_run(st, s0, acts, w, np.float32)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float32)
    _check("wide rk4 A=80", hip, orc)


def test_wide_step_float64():
    E, A, T, S = 2, 70, 4, 2
    rng = np.random.default_rng(31)
    cfgs = [AgentConfig(radius=0.05) for _ in range(A)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-0.8, 0.8, -0.8, 0.8), max_neighbors=6)
    s0 = pack_state({"pos": rng.uniform(-0.8, 0.8, size=(E, A, 2))})
    acts = rng.uniform(-1, 1, size=(T, E, A, 2))
    w = _cot(T, E, A, 32)
    st = make_stepper(cfgs, world, 0.05, S, torch.float64)
    hip = hip_run(st, s0, acts, w, np.float64)
    orc = oracle_run(cfgs, world, 0.05, S, s0, acts, w, np.float64)
    _check("wide f64 A=70", hip, orc, g_tol=1e-12, exact=False)
