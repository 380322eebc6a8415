"""Throughput of ``Environment.step`` on the navigation scenario, no grad: env-steps/s
and agent-steps/s over the reference's batch grid.

Counterpart of the reference's ``python -m swarp.benchmark.throughput``
(swarp/benchmark/throughput.py:1-145): the same scenario construction
(``NavigationScenario(n_agents, world_size=max(1, sqrt(n_agents) / 4))``), float32,
``dt=0.05``, ``substeps=1``, ``seed=0``, ``env.reset(seed=0)``, fresh uniform actions in
[-1, 1] drawn on the device inside the timed loop, 10 warm-up and 100 timed steps under
``torch.no_grad()``, graph on by default (``--no-graph`` for the eager table).  The
reference's published figures (RTX 3070 Laptop GPU, ``docs/benchmarks.md:27-59``) are
printed beside each row for comparison.

Run:  python -m swarp_amd.throughput [--steps 100] [--no-graph] [--json] [--rows 16000x16,...]
      python -m swarp_amd.throughput --launch-cost   # host cost of a graph replay vs eager
"""

from __future__ import annotations

import argparse
import ctypes
import json
import time

import torch

from .environment import Environment
from .scenarios import NavigationScenario

ENV_COUNTS = (1_000, 4_000, 8_000, 16_000)
AGENT_COUNTS = (4, 16, 64)

#: (n_envs, n_agents) -> (graph-off env-steps/s, graph-on env-steps/s) published for the
#: reference on an RTX 3070 Laptop GPU (docs/benchmarks.md:29-40, 48-59)
PUBLISHED = {
    (1000, 4): (3_398_312, 36_852_108), (1000, 16): (2_753_071, 16_372_076),
    (1000, 64): (2_803_282, 4_150_284), (4000, 4): (13_747_433, 82_862_931),
    (4000, 16): (11_334_742, 27_297_834), (4000, 64): (6_863_382, 6_475_123),
    (8000, 4): (21_737_790, 100_176_473), (8000, 16): (22_375_841, 30_806_414),
    (8000, 64): (7_541_604, 7_382_113), (16000, 4): (45_393_422, 145_785_598),
    (16000, 16): (33_916_430, 38_818_634), (16000, 64): (7_490_570, 8_227_839),
}


def bench_one(n_envs: int, n_agents: int, device: str = "cuda:0", steps: int = 100,
              warmup: int = 10, use_graph: bool = True) -> dict:
    """One row of the grid (swarp/benchmark/throughput.py:50-93)."""
    scenario = NavigationScenario(n_agents=n_agents, world_size=max(1.0, n_agents ** 0.5 / 4))
    env = Environment(scenario, n_envs=n_envs, device=device, dt=0.05, substeps=1, seed=0,
                      use_graph=use_graph)
    env.reset(seed=0)
    gen = torch.Generator(device=device).manual_seed(0)
    actions = torch.empty(n_envs, n_agents, 2, device=device)
    with torch.no_grad():
        for _ in range(warmup):
            actions.uniform_(-1.0, 1.0, generator=gen)
            env.step(actions)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            actions.uniform_(-1.0, 1.0, generator=gen)
            env.step(actions)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    eps = n_envs * steps / elapsed
    pub = PUBLISHED.get((n_envs, n_agents))
    return {
        "n_envs": n_envs, "n_agents": n_agents, "graph": bool(env.graph_mode),
        "ms_per_step": 1e3 * elapsed / steps, "env_steps_s": eps,
        "agent_steps_s": eps * n_agents,
        "reference_rtx3070_env_steps_s": None if pub is None else pub[1 if use_graph else 0],
    }


def launch_cost(device: str = "cuda:0", calls: int = 2000) -> dict:
    """Host time per call, in microseconds, of issuing a two-kernel step three ways: two
    eager launches, ``torch.cuda.CUDAGraph.replay()`` of the same two kernels captured in a
    graph, and ``hipGraphLaunch`` on that graph's executable called directly through
    ctypes.  The two kernels are tiny element-wise updates of a 16000 x 16 float buffer, so
    the figures are launch costs, not kernel times; "total" adds the drain of the queue."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphLaunch.restype = ctypes.c_int
    x = torch.zeros(16000 * 16, device=device)
    y = torch.zeros_like(x)
    stream = torch.cuda.Stream(device=device)

    def work():
        x.add_(1.0)
        y.mul_(0.5)

    def timed(fn):
        for _ in range(50):
            fn()
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize(device)
        t2 = time.perf_counter()
        return {"host_us": (t1 - t0) / calls * 1e6, "total_us": (t2 - t0) / calls * 1e6}

    with torch.cuda.stream(stream):
        work()
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            work()
        torch.cuda.synchronize(device)
        exe = ctypes.c_void_p(graph.raw_cuda_graph_exec())
        raw_stream = ctypes.c_void_p(stream.cuda_stream)

        def raw():
            rc = hip.hipGraphLaunch(exe, raw_stream)
            if rc:
                raise RuntimeError(f"hipGraphLaunch returned {rc}")

        return {"eager_two_launches": timed(work), "graph_replay": timed(graph.replay),
                "hipGraphLaunch": timed(raw)}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--device", default="cuda:0")
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--graph", action=argparse.BooleanOptionalAction, default=True)
    ap.add_argument("--json", action="store_true", help="one JSON line per row")
    ap.add_argument("--rows", default=None,
                    help="comma-separated EnvsxAgents rows to run (default: the whole grid)")
    ap.add_argument("--launch-cost", action="store_true",
                    help="print the host cost of a graph replay against two eager launches")
    args = ap.parse_args()
    if args.launch_cost:
        for name, r in launch_cost(args.device).items():
            print(f"{name:>20}: host {r['host_us']:6.1f} us/call, total {r['total_us']:6.1f} us/call",
                  flush=True)
        return
    rows = [(e, a) for e in ENV_COUNTS for a in AGENT_COUNTS]
    if args.rows:
        rows = [tuple(int(x) for x in r.split("x")) for r in args.rows.split(",")]
    print(f"device: {args.device} ({torch.cuda.get_device_name(args.device)}); "
          f"timed steps per config: {args.steps}; whole-step graph: "
          f"{'on' if args.graph else 'off'}", flush=True)
    head = (f"{'n_envs':>8} {'n_agents':>9} {'ms/step':>9} {'env-steps/s':>14} "
            f"{'agent-steps/s':>15} {'ref (3070)':>14} {'x ref':>7}")
    if not args.json:
        print(head)
        print("-" * len(head))
    for n_envs, n_agents in rows:
        r = bench_one(n_envs, n_agents, args.device, args.steps, use_graph=args.graph)
        if args.json:
            print(json.dumps(r), flush=True)
            continue
        ref = r["reference_rtx3070_env_steps_s"]
        cmp = (f"{ref:>14,} {r['env_steps_s'] / ref:>7.1f}" if ref else f"{'-':>14} {'-':>7}")
        print(f"{n_envs:>8} {n_agents:>9} {r['ms_per_step']:>9.3f} {r['env_steps_s']:>14,.0f} "
              f"{r['agent_steps_s']:>15,.0f} {cmp}", flush=True)


if __name__ == "__main__":
    main()
