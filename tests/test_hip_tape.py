"""Rollout tape on the GPU: the backward that reads the substep intermediates from the
forward's tape against the backward that recomputes them.

Bar: BIT-IDENTICAL.  The reverse pass runs the same arithmetic in the same order on the
same values either way (positions of substeps 1..S-1 are re-derived with the forward's own
update), so forward states and both gradients must be equal bit for bit.  The tape path is
also the default one, so every specialised-kernel parity test against the oracle runs
through it.
"""

import dataclasses

import numpy as np
import pytest
import torch

from cases import nav_agents, nav_world
from hip_helpers import hip_run, make_stepper
from oracle.oracle import pack_state
from swarp_amd.config import WorldConfig

pytestmark = pytest.mark.gpu


def _case(E, A, T, extent, seed, dtype=np.float32):
    rng = np.random.default_rng(seed)
    s0 = pack_state({"pos": rng.uniform(-extent, extent, size=(E, A, 2)),
                     "vel": rng.uniform(-0.3, 0.3, size=(E, A, 2))}).astype(dtype)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(dtype)
    w = rng.normal(size=(T, E, A, 16))
    w[..., 7:] = 0.0
    return s0, acts, w


def _pair(cfgs, world, S, dtype=torch.float32):
    on = make_stepper(cfgs, world, 0.05, S, dtype)
    off = make_stepper(cfgs, world, 0.05, S, dtype)
    off.use_tape = False
    return on, off


CASES = [
    # (E, A, T, S, extent, world kwargs) -- contacts + soft walls unless stated
    (400, 16, 12, 4, 0.6, dict(world_size=0.7)),          # config-2 shape, dense
    (37, 16, 6, 3, 0.5, dict(world_size=0.55)),           # partial last wave, S = 3
    (45, 4, 5, 1, 0.4, dict(world_size=0.45)),            # S = 1: no velocity entries
    (20, 12, 7, 2, 0.15, dict(world_size=0.3, max_neighbors=3)),  # truncated lists
    (9, 32, 4, 4, 0.4, dict(world_size=0.45)),            # 8-byte mask words
    (3, 64, 4, 2, 0.5, dict(world_size=0.55)),            # 16-byte mask words
]


@pytest.mark.parametrize("E,A,T,S,extent,kw", CASES)
def test_tape_matches_recompute(E, A, T, S, extent, kw):
    kw = dict(kw)
    ws = kw.pop("world_size")
    mk = kw.pop("max_neighbors", None)
    world = nav_world(A, world_size=ws)
    if mk is not None:
        world = dataclasses.replace(world, max_neighbors=mk)
    cfgs = nav_agents(A)
    on, off = _pair(cfgs, world, S)
    assert on.tape_bytes(E, 2, T) > 0 and off.tape_bytes(E, 2, T) == 0
    s0, acts, w = _case(E, A, T, extent, seed=E + A + S)
    a = hip_run(on, s0, acts, w, np.float32)
    b = hip_run(off, s0, acts, w, np.float32)
    assert np.array_equal(a[0][..., :7], b[0][..., :7]), "forward states differ"
    assert np.array_equal(a[2], b[2]), "d/d actions differ"
    assert np.array_equal(a[1][..., :7], b[1][..., :7]), "d/d state0 differ"


def test_tape_walls_only_and_contacts_only():
    E, A, T, S = 30, 8, 6, 4
    s0, acts, w = _case(E, A, T, 0.5, seed=5)
    walls = WorldConfig(collisions=False, bounds=(-0.5, 0.5, -0.5, 0.5), bounds_mode="soft")
    contacts = WorldConfig(collisions=True, collision_margin=0.025, max_neighbors=8)
    for world in (walls, contacts):
        on, off = _pair(nav_agents(A), world, S)
        assert on.tape_bytes(E, 2, T) > 0
        a = hip_run(on, s0, acts, w, np.float32)
        b = hip_run(off, s0, acts, w, np.float32)
        for x, y in zip(a, b):
            assert np.array_equal(x[..., :7], y[..., :7])


def test_tape_float64():
    E, A, T, S = 32, 8, 6, 4
    s0, acts, w = _case(E, A, T, 0.3, seed=8, dtype=np.float64)
    on, off = _pair(nav_agents(A), nav_world(A, world_size=0.35), S, torch.float64)
    a = hip_run(on, s0, acts, w, np.float64)
    b = hip_run(off, s0, acts, w, np.float64)
    for x, y in zip(a, b):
        assert np.array_equal(x[..., :7], y[..., :7])


def test_no_tape_beyond_four_substeps():
    """Five substeps keep no tape; the rollout recomputes and still runs."""
    E, A, T, S = 10, 8, 3, 5
    s0, acts, w = _case(E, A, T, 0.4, seed=3)
    st = make_stepper(nav_agents(A), nav_world(A, world_size=0.45), 0.05, S, torch.float32)
    assert st.tape_bytes(E, 2, T) == 0
    states, g0, ga = hip_run(st, s0, acts, w, np.float32)
    assert np.isfinite(ga).all() and np.isfinite(g0).all()


def _obstacle_world(E, A, n, seed):
    """A mixed 2-D fleet (diff-drive + bicycle) among n static obstacles of every shape."""
    from swarp_amd.config import AgentConfig, DynamicsModel
    rng = np.random.default_rng(seed)
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, radius=0.05) for _ in range(A // 2)] + [
        AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE, radius=0.05)
        for _ in range(A - A // 2)]
    world = WorldConfig(collision_k=100.0, collision_c=1.0, collision_margin=0.025,
                        bounds=(-1.0, 1.0, -1.0, 1.0), max_neighbors=32)
    ty = np.arange(n) % 3
    obs = {"pos": rng.uniform(-1, 1, size=(E, n, 2)),
           "radius": np.where(ty == 0, rng.uniform(0.05, 0.2, n), np.where(ty == 2, 0.05, 0.0)),
           "type": ty.astype(np.int32),
           "angle": rng.uniform(-np.pi, np.pi, size=(E, n)),
           "half": np.where((ty == 1)[:, None], rng.uniform(0.05, 0.3, size=(n, 2)),
                            np.where((ty == 2)[:, None],
                                     np.c_[rng.uniform(0.1, 0.4, n), np.zeros(n)], 0.0))}
    s0 = pack_state({"pos": rng.uniform(-1, 1, size=(E, A, 2)),
                     "theta": rng.uniform(-np.pi, np.pi, size=(E, A))}).astype(np.float32)
    return cfgs, world, obs, s0, rng


@pytest.mark.parametrize("E,A,T,S,n", [
    (300, 32, 8, 4, 8),     # config-3 shape: two envs per workgroup
    (41, 8, 6, 3, 12),      # eight envs per workgroup, partial last one, S = 3
    (17, 64, 5, 2, 30),     # one env per workgroup, many obstacles
    (23, 4, 4, 1, 16),      # sixteen envs per workgroup at the table's limit, S = 1
    (9, 40, 4, 2, 40),      # more than 32 obstacles: sums only, no contact masks
])
def test_obstacle_sum_tape_matches_recompute(E, A, T, S, n):
    """Static obstacles: the forward keeps each substep's total force, neighbour lists and
    obstacle contacts, and the backward reads them instead of evaluating the forces and
    scanning again, and reverses only the obstacles in contact -- the same values."""
    cfgs, world, obs, s0, rng = _obstacle_world(E, A, n, seed=E + n)
    on = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    off = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    off.use_tape = False
    al = lambda x: x + (-x % 256)  # noqa: E731
    n_ = T * S * E * A
    mw = 1 if n <= 8 else (2 if n <= 16 else (4 if n <= 32 else 0))  # contact-mask word
    nw = 8 if A > 32 else 4  # neighbour-mask word (64-lane envs: 64-bit masks)
    assert on.tape_bytes(E, 2, T) == al(al(al(2 * 4 * n_) + mw * n_) + nw * n_)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16)) * 0.1
    w[..., 7:] = 0.0
    a = hip_run(on, s0, acts, w, np.float32)
    b = hip_run(off, s0, acts, w, np.float32)
    assert np.array_equal(a[0][..., :7], b[0][..., :7]), "forward states differ"
    assert np.array_equal(a[2], b[2]), "d/d actions differ"
    assert np.array_equal(a[1][..., :7], b[1][..., :7]), "d/d state0 differ"


def test_obstacle_tape_without_agent_collisions():
    """Obstacles and walls but no agent-agent contacts: the forward keeps no neighbour
    lists, and the taped backward must build none either -- the untaped values."""
    E, A, T, S, n = 37, 16, 5, 3, 8
    cfgs, _, obs, s0, rng = _obstacle_world(E, A, n, seed=5)
    world = WorldConfig(collisions=False, collision_k=100.0, collision_c=1.0,
                        collision_margin=0.025, bounds=(-1.0, 1.0, -1.0, 1.0),
                        bounds_mode="soft")
    on = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    off = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    off.use_tape = False
    assert on.tape_bytes(E, 2, T) > 0
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16)) * 0.1
    w[..., 7:] = 0.0
    a = hip_run(on, s0, acts, w, np.float32)
    b = hip_run(off, s0, acts, w, np.float32)
    assert np.array_equal(a[0][..., :7], b[0][..., :7]), "forward states differ"
    assert np.array_equal(a[2], b[2]), "d/d actions differ"
    assert np.array_equal(a[1][..., :7], b[1][..., :7]), "d/d state0 differ"


def test_no_obstacle_tape_beyond_the_pose_table():
    """Seventeen obstacles at four agents per env overflow the two-wave forward's
    per-launch obstacle table (16 envs x 17 > 256 entries): the one-wave forward runs and
    keeps the generic tape (forces and lists, no contact masks) -- the untaped values."""
    E, A, T, S, n = 20, 4, 3, 2, 17
    cfgs, world, obs, s0, rng = _obstacle_world(E, A, n, seed=1)
    st = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    off = make_stepper(cfgs, world, 0.05, S, torch.float32, obs=obs, n_envs=E)
    off.use_tape = False
    al = lambda x: x + (-x % 256)  # noqa: E731
    n_ = T * S * E * A
    assert st.tape_bytes(E, 2, T) == al(al(2 * 4 * n_) + 4 * n_)
    acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
    w = rng.normal(size=(T, E, A, 16)) * 0.1
    w[..., 7:] = 0.0
    a = hip_run(st, s0, acts, w, np.float32)
    b = hip_run(off, s0, acts, w, np.float32)
    assert np.isfinite(a[2]).all() and np.isfinite(a[1]).all()
    assert np.array_equal(a[0][..., :7], b[0][..., :7]), "forward states differ"
    assert np.array_equal(a[2], b[2]), "d/d actions differ"
    assert np.array_equal(a[1][..., :7], b[1][..., :7]), "d/d state0 differ"
