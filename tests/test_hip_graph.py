"""The whole-step HIP graph (``Environment(use_graph=...)``, ``swarp_amd.persistent``):
every replay equals the eager fused step -- state, observations, reward, termination,
time limit and info, bit for bit -- across ping-pong flips, auto-resets, standalone
resets, a differentiated step in between (the state is adopted back into the graph's
buffers) and a recapture after the baked pointers move.  Eager work and host syncs run
between the replays, and each replay is checked on its own.
"""

import pytest
import torch

from swarp_amd import make

pytestmark = pytest.mark.gpu


def _pair(E, A, **kw):
    kw.setdefault("world_size", max(1.0, A ** 0.5 / 4))
    g = make("navigation", E, n_agents=A, dt=0.05, seed=0, use_graph=True, **kw)
    e = make("navigation", E, n_agents=A, dt=0.05, seed=0, use_graph=False, **kw)
    assert g.graph_mode and not e.graph_mode
    return g, e


def _same(rg, re_, where):
    for k, (x, y) in enumerate(zip(rg[:4], re_[:4])):
        assert torch.equal(x, y), f"{where}: output {k} differs"
    for key in re_[4]:
        assert torch.equal(rg[4][key], re_[4][key]), f"{where}: info[{key}] differs"


def _acts(E, A, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.rand(E, A, 2, device="cuda", generator=g) * 2 - 1


@pytest.mark.parametrize("auto_reset", [False, True])
def test_graph_replays_equal_eager_steps(auto_reset):
    E, A, T = 96, 16, 24
    ge, ee = _pair(E, A, max_steps=7, auto_reset=auto_reset, goal_tolerance=0.15)
    assert torch.equal(ge.reset(), ee.reset())
    for t in range(T):
        a = _acts(E, A, t)
        with torch.no_grad():
            rg = ge.step(a)
            re_ = ee.step(a)
        torch.cuda.synchronize()
        assert torch.equal(ge.world.state.pos, ee.world.state.pos), t
        assert torch.equal(ge.world.state.vel, ee.world.state.vel), t
        _same(rg, re_, f"step {t}")
        assert torch.equal(ge.step_count, ee.step_count)
        _ = float(rg[1].sum())  # eager work + a host sync between replays
    assert ge._graph.captures == 2  # one graph per ping-pong parity, never recaptured


def test_graph_with_resets_and_a_differentiated_step():
    E, A = 64, 8
    ge, ee = _pair(E, A, max_steps=50)
    ge.reset()
    ee.reset()
    for t in range(5):
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")
    # a differentiated step takes the functional path on both envs
    a1 = _acts(E, A, 100).requires_grad_(True)
    a2 = a1.detach().clone().requires_grad_(True)
    rg, re_ = ge.step(a1), ee.step(a2)
    rg[1].sum().backward()
    re_[1].sum().backward()
    assert torch.equal(a1.grad, a2.grad)
    assert torch.equal(ge.world.state.pos, ee.world.state.pos)
    # back on the graph: the functional step's state is adopted into its buffers
    for t in range(5, 9):
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")
    mask = torch.arange(E, device="cuda") % 4 == 1
    assert torch.equal(ge.reset_at(mask), ee.reset_at(mask))
    for t in range(9, 12):
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")
    assert torch.equal(ge.reset(seed=3), ee.reset(seed=3))
    for t in range(12, 15):
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")


def test_graph_recaptures_when_obstacles_move_pointers():
    E, A = 32, 4
    ge, ee = _pair(E, A, n_obstacles=3)
    ge.reset()
    ee.reset()
    for t in range(4):
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")
    n0 = ge._graph.captures
    assert n0 == 2
    # reinstalling obstacles moves the descriptor: the next replay recaptures
    for env in (ge, ee):
        env.world.set_obstacles(env.world.obstacles)
    for t in range(4, 8):
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")
    assert ge._graph.captures == n0 + 2


def test_graph_follows_a_reinstalled_per_env_table():
    """Re-randomizing per-env parameters with a host (numpy) table reallocates the device
    table: the next replay recaptures instead of replaying the freed address, and every
    step equals the eager environment's."""
    import numpy as np

    from swarp_amd import per_env_float_template
    from swarp_amd.config import P_MAX_SPEED, P_RADIUS

    E, A = 64, 8
    ge, ee = _pair(E, A, max_steps=100, neighbor_radius=0.2)
    rng = np.random.default_rng(4)
    ge.reset()
    ee.reset()
    for t in range(9):
        if t % 3 == 0:
            table = per_env_float_template(ge.world.agent_configs, E)
            table[..., P_RADIUS] = rng.uniform(0.03, 0.06, size=(E, A))
            table[..., P_MAX_SPEED] = rng.uniform(0.5, 1.5, size=(E, A))
            for env in (ge, ee):
                env.world.stepper.set_agent_params_per_env(table)
        with torch.no_grad():
            _same(ge.step(_acts(E, A, t)), ee.step(_acts(E, A, t)), f"step {t}")
        assert torch.equal(ge.world.state.pos, ee.world.state.pos), t
    assert ge._graph.captures >= 2 + 2 * 3 - 2  # recaptured after each reallocation
