"""Headline benchmark: fwd+bwd BPTT env-steps/s of the swarp physics step on one MI355X.

Workload: navigation, holonomic point agents, float32,
16000 envs x 16 agents, 4 fused substeps per step, 32-step BPTT; positions and goals
uniform in the 4x4 arena (walls at +-2), zero initial velocity, actions uniform in
[-1, 1]^2, loss = sum of squared goal distances at the final step.

One benchmark step = one BPTT iteration through the public API:
``rollout(stepper, state0, actions)`` (32 env steps, one HIP launch), the loss, and
``loss.backward()`` (one HIP launch).  ``value`` = n_envs * T * steps / elapsed, with
inputs already resident in HBM.  The per-kernel durations for the roofline come from
HIP events recorded around each launch on its own stream during the timed steps.

``cpu_baseline`` times the CPU oracle (oracle/swarp_oracle.c, OpenMP over envs) on a
bounded sample of the same workload on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fwd+bwd BPTT env-steps/s at 16k envs x 16 agents; % of HBM roofline"
HBM_PEAK = 8.0e12  # MI355X published HBM3E bandwidth, bytes/s

# Algorithmic bytes per env-step (2-D models: 7 state floats, act_dim 2, no obstacles):
# forward  = 4 A (2 S_f + a)   (in-state, actions, out-state)
# backward = 4 A (3 S_f + 2 a) (checkpoint, actions, adj_out, adj_in, adj_act)
S_F, ACT = 7, 2


def fwd_bytes(A):
    return 4 * A * (2 * S_F + ACT)


def bwd_bytes(A):
    return 4 * A * (3 * S_F + 2 * ACT)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--envs", type=int, default=16000)
    ap.add_argument("--agents", type=int, default=16)
    ap.add_argument("--horizon", type=int, default=32)
    ap.add_argument("--substeps", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target duration of the CPU-baseline sample (0 = skip)")
    ap.add_argument("--env-steps", type=int, default=100,
                    help="timed Environment.step calls of the no-grad navigation leg "
                         "(16000 x 16, graph on and off); 0 skips it")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="after the benchmark, run 3 plain device copies of this many MiB "
                         "(calibrates rocprof byte counters against a known traffic)")
    return ap.parse_args()


def make_problem(E, A, T, S, seed=0):
    import torch

    from swarp_amd import AgentConfig, Stepper, TorchState, WorldConfig

    ws, r = 2.0, 0.05
    margin = 0.5 * r
    cfgs = [AgentConfig(radius=r, max_speed=1.0, max_accel=2.0) for _ in range(A)]
    world = WorldConfig(collisions=True, collision_k=100.0, collision_c=1.0, collision_margin=margin,
                        bounds=(-ws, ws, -ws, ws), bounds_mode="soft",
                        neighbor_radius=2 * r + margin, max_neighbors=min(32, max(4, A)))
    stepper = Stepper(cfgs, dt=0.05, substeps=S, device="cuda:0", dtype=torch.float32, world=world)
    g = torch.Generator(device="cuda").manual_seed(seed)
    pos = (torch.rand(E, A, 2, generator=g, device="cuda") * 2 - 1) * ws
    goals = (torch.rand(E, A, 2, generator=g, device="cuda") * 2 - 1) * ws
    acts = torch.rand(T, E, A, 2, generator=g, device="cuda") * 2 - 1
    z = torch.zeros(E, A, device="cuda")
    state = TorchState(pos, z.clone(), torch.zeros(E, A, 2, device="cuda"), z.clone(), z.clone())
    return stepper, state, goals, acts, cfgs, world


def cpu_baseline(E_full, A, T, S, seconds, cfgs, world):
    """Oracle fwd+bwd on a bounded env sample, OpenMP over every host core."""
    import numpy as np

    from oracle.oracle import Oracle, cores, pack_state

    n = cores()
    O = Oracle(np.float32)
    rows = np.array([c.to_row() for c in cfgs], dtype=np.float32)
    tags = np.zeros(A, np.int32)
    modes = np.zeros(A, np.int32)
    b = world.bounds

    def run(E):
        rng = np.random.default_rng(0)
        s0 = pack_state({"pos": rng.uniform(-2, 2, size=(E, A, 2))}, dtype=np.float32)
        acts = rng.uniform(-1, 1, size=(T, E, A, 2)).astype(np.float32)
        goals = rng.uniform(-2, 2, size=(E, A, 2)).astype(np.float32)
        cfg = dict(n_envs=E, n_agents=A, act_dim=2, substeps=S, max_neighbors=world.max_neighbors,
                   collisions=1, soft_walls=1, clamp_bounds=0, n_threads=n, dt=0.05,
                   k=world.collision_k, c=world.collision_c, margin=world.collision_margin,
                   max_overlap=0.0, neighbor_radius=world.neighbor_radius,
                   bmin_x=b[0], bmax_x=b[1], bmin_y=b[2], bmax_y=b[3])
        t0 = time.perf_counter()
        states = O.rollout(cfg, rows, tags, modes, None, s0, acts)
        afin = np.zeros_like(s0)
        afin[..., 0:2] = 2 * (states[-1][..., 0:2] - goals)
        O.rollout_adj(cfg, rows, tags, modes, None, s0, acts, states, None, afin)
        return time.perf_counter() - t0

    probe = max(n * 8, 64)
    dt_probe = run(probe)
    E = int(min(E_full, max(probe, probe * seconds / max(dt_probe, 1e-6))))
    el = run(E) if E != probe else dt_probe
    reps, total = 1, el
    while total < seconds and reps < 50:
        total += run(E)
        reps += 1
    return {
        "value": E * T * reps / total,
        "unit": "env-steps/s",
        "cores": n,
        "kind": "port",
        "sample": f"{reps} x {E} of {E_full} envs x {A} agents, {S} substeps, {T}-step BPTT "
                  f"fwd+bwd, float32 C oracle, OpenMP over envs ({total:.1f} s)",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (every box here has one); --gpus {args.gpus} "
              "is not supported: the step shards over envs with no exchange, see DESIGN.md.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import swarp_amd.autograd as ag
    from swarp_amd import rollout

    E, A, T, S = args.envs, args.agents, args.horizon, args.substeps
    stepper, state, goals, acts, cfgs, world = make_problem(E, A, T, S)
    a = acts.clone().requires_grad_(True)
    s0 = type(state)(state.pos.clone().requires_grad_(True), *state[1:])

    def bptt_step():
        a.grad = None
        s0.pos.grad = None
        final, _ = rollout(stepper, s0, a)
        loss = ((final.pos - goals) ** 2).sum()
        loss.backward()

    for _ in range(args.warmup):
        bptt_step()
    torch.cuda.synchronize()
    ag.KERNEL_EVENTS = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        bptt_step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    events = ag.KERNEL_EVENTS
    ag.KERNEL_EVENTS = None
    dur = {"fwd": [], "bwd": []}
    for kind, e0, e1 in events:
        dur[kind].append(e0.elapsed_time(e1) * 1e-3)
    ms_per_step = el / args.steps * 1e3
    value = E * T * args.steps / el

    # forward-only (no graph) throughput of the same rollout
    with torch.no_grad():
        for _ in range(args.warmup):
            rollout(stepper, state, acts)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            rollout(stepper, state, acts)
        torch.cuda.synchronize()
        el_f = time.perf_counter() - t1
    fwd_only = E * T * args.steps / el_f

    # the library launches the specialised holonomic-velocity kernels when the desc allows
    fam = "k_holo" if stepper.desc(E, 2).holo_velocity_only else "k_rollout"
    pa = 1 << max(2, (A - 1).bit_length())
    kernels = {}
    for kind, per in (("fwd", fwd_bytes(A)), ("bwd", bwd_bytes(A))):
        d = sum(dur[kind]) / max(len(dur[kind]), 1)
        alg = per * E * T
        kernels[kind] = {
            "name": f"{fam}_{kind}<float, {pa}>",
            "avg_ms": d * 1e3,
            "alg_bytes_per_launch": alg,
            "achieved_GBps": alg / d / 1e9 if d > 0 else None,
            "frac": alg / d / HBM_PEAK if d > 0 else None,
        }
    dom = max(kernels, key=lambda k: kernels[k]["avg_ms"])
    kd = kernels[dom]
    traffic = None
    prof = ROOT / "profiles" / "traffic_c2.json"
    if prof.exists() and (E, A, T, S) == (16000, 16, 32, 4):
        # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
        # of this same workload, scaled by the copy-kernel calibration they record
        tr = json.loads(prof.read_text())
        k = tr["kernels"][dom]
        traffic = 1024 * (k["fetch_kib"] * tr["fetch_scale"] + k["write_kib"] * tr["write_scale"])
    fused_frac = (fwd_bytes(A) + bwd_bytes(A)) * E * T / (
        (kernels["fwd"]["avg_ms"] + kernels["bwd"]["avg_ms"]) * 1e-3) / HBM_PEAK

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"navigation holonomic, {E} envs x {A} agents, {S} substeps, "
                        f"{T}-step BPTT (BASELINE configs[1])",
            "n_envs": E, "n_agents": A, "substeps": S, "horizon": T, "dt": 0.05,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kd["name"],
            "achieved": kd["achieved_GBps"],
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": kd["frac"],
            "traffic": traffic,
        },
        "fwd_bwd_kernel_roofline_frac": fused_frac,
        "fwd_only_env_steps_per_s": fwd_only,
        "kernels": kernels,
    }
    if args.env_steps > 0:
        # the reference's own published benchmark: no-grad Environment.step of the
        # navigation scenario (step + lists + obs/reward), 1 substep, graph on and off
        from swarp_amd.throughput import bench_one

        rows = {}
        for g in (True, False):
            r = bench_one(16000, 16, steps=args.env_steps, use_graph=g)
            rows["graph" if g else "eager"] = {
                "env_steps_s": r["env_steps_s"], "ms_per_step": r["ms_per_step"],
                "reference_rtx3070_env_steps_s": r["reference_rtx3070_env_steps_s"],
            }
        out["env_step_nograd_16000x16"] = rows
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline(E, A, T, S, args.cpu_seconds, cfgs, world)
    if args.copy_mb > 0:
        n = args.copy_mb * (1 << 20) // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_calibration_bytes"] = {"read": 4 * n, "write": 4 * n}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
