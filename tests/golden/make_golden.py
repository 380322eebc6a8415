"""Writes tests/golden/config1.npz: config 1 (64 envs x 4 holonomic agents, dt 0.05,
1 substep, 10-step BPTT, seed 0) computed by the float32 and float64 CPU oracle.

The reference (Python on warp-lang) cannot run here, so these vectors come from the
oracle; they freeze its config-1 answer so that a change to the oracle or to the HIP path
shows up against a committed file.  Regenerate with:  python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

from cases import nav_agents, nav_inputs, nav_world, oracle_cfg, params_of  # noqa: E402
from oracle.oracle import Oracle, pack_state  # noqa: E402

E, A, T, S, DT = 64, 4, 10, 1, 0.05


def main():
    pos, goals, acts = nav_inputs(E, A, T, extent=1.0, seed=0, dtype=torch.float32)
    cfgs, world = nav_agents(A), nav_world(A, world_size=1.0)
    out = {"pos0": pos.numpy(), "goals": goals.numpy(), "actions": acts.numpy()}
    for name, dt in (("f32", np.float32), ("f64", np.float64)):
        O = Oracle(dt)
        cfg = oracle_cfg(cfgs, world, DT, S, E, 2)
        p, t, m = params_of(cfgs)
        s0 = pack_state({"pos": pos.numpy().astype(np.float64)}, dtype=dt)
        a = acts.numpy().astype(dt)
        states = O.rollout(cfg, p, t, m, None, s0, a)
        afin = np.zeros_like(s0)
        afin[..., 0:2] = 2.0 * (states[-1][..., 0:2] - goals.numpy().astype(dt))
        g0, ga = O.rollout_adj(cfg, p, t, m, None, s0, a, states, None, afin)
        out[f"{name}_pos"] = states[..., 0:2]
        out[f"{name}_vel"] = states[..., 3:5]
        out[f"{name}_grad_actions"] = ga
        out[f"{name}_grad_pos0"] = g0[..., 0:2]
    np.savez_compressed(Path(__file__).with_name("config1.npz"), **out)


if __name__ == "__main__":
    main()
