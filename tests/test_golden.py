"""Config 1 against the committed fixture tests/golden/config1.npz (made by
tests/golden/make_golden.py from the CPU oracle)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from cases import nav_agents, nav_world, oracle_cfg, params_of
from oracle.oracle import Oracle, pack_state

G = np.load(Path(__file__).with_name("golden") / "config1.npz")
E, A, T = 64, 4, 10


def test_oracle_reproduces_fixture():
    cfgs, world = nav_agents(A), nav_world(A, world_size=1.0)
    for name, dt in (("f32", np.float32), ("f64", np.float64)):
        O = Oracle(dt)
        cfg = oracle_cfg(cfgs, world, 0.05, 1, E, 2)
        p, t, m = params_of(cfgs)
        s0 = pack_state({"pos": G["pos0"].astype(np.float64)}, dtype=dt)
        states = O.rollout(cfg, p, t, m, None, s0, G["actions"].astype(dt))
        np.testing.assert_array_equal(states[..., 0:2], G[f"{name}_pos"])
        np.testing.assert_array_equal(states[..., 3:5], G[f"{name}_vel"])
    # the fixture has contacts and walls in it (otherwise it would pin little)
    assert np.abs(G["f64_vel"]).max() > 1.0


@pytest.mark.gpu
def test_hip_matches_fixture():
    from swarp_amd import Stepper, TorchState, rollout

    cfgs, world = nav_agents(A), nav_world(A, world_size=1.0)
    st = Stepper(cfgs, dt=0.05, substeps=1, device="cuda:0", dtype=torch.float32, world=world)
    z = torch.zeros(E, A, device="cuda")
    pos = torch.tensor(G["pos0"], device="cuda").requires_grad_(True)
    acts = torch.tensor(G["actions"], device="cuda").requires_grad_(True)
    final, traj = rollout(st, TorchState(pos, z, torch.zeros(E, A, 2, device="cuda"), z, z), acts)
    ((final.pos - torch.tensor(G["goals"], device="cuda")) ** 2).sum().backward()
    hp = np.stack([s.pos.detach().cpu().numpy() for s in traj])
    np.testing.assert_array_equal(hp, G["f32_pos"])  # bit-exact
    ga, g0 = acts.grad.cpu().numpy(), pos.grad.cpu().numpy()
    assert np.abs(ga - G["f32_grad_actions"]).max() <= 1e-5 * np.abs(G["f32_grad_actions"]).max()
    assert np.abs(g0 - G["f32_grad_pos0"]).max() <= 1e-5 * np.abs(G["f32_grad_pos0"]).max()
    np.testing.assert_allclose(ga, G["f64_grad_actions"], rtol=1e-3, atol=1e-4)
