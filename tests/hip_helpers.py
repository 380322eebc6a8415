"""Helpers of the GPU tests: run the HIP path through the public API and the oracle on
the same inputs, and return both as numpy arrays in the oracle's [.., 16] layout."""

from __future__ import annotations

import numpy as np
import torch

from cases import obstacles_np, oracle_cfg, params_of
from oracle.oracle import OFFSET, WIDTH, Oracle, pack_state
from swarp_amd import Obstacles, Stepper, TorchState, rollout

FIELDS = ("pos", "theta", "vel", "speed", "ang_vel", "z", "vz", "attitude", "body_rates")
TDT = {np.float32: torch.float32, np.float64: torch.float64}


def to_torch_state(s16: np.ndarray, dtype, requires_grad: bool, n_fields: int) -> TorchState:
    """[E,A,16] -> TorchState on cuda (first n_fields fields; the rest default)."""
    fields = []
    for k, (w, o) in enumerate(zip(WIDTH, OFFSET)):
        if k >= n_fields:
            fields.append(None)
            continue
        v = s16[..., o:o + w]
        if w == 1:
            v = v[..., 0]
        t = torch.tensor(np.ascontiguousarray(v), dtype=dtype, device="cuda")
        fields.append(t.requires_grad_(requires_grad))
    return TorchState(*fields)


def state_to16(st: TorchState) -> np.ndarray:
    parts = []
    pos = st.pos.detach()
    E, A = pos.shape[:2]
    for k, (name, w) in enumerate(zip(FIELDS, WIDTH)):
        t = getattr(st, name)
        if t is None:
            v = np.zeros((E, A, w))
            if name == "attitude":
                v[..., 3] = 1.0
        else:
            v = t.detach().double().cpu().numpy().reshape(E, A, w)
        parts.append(v)
    return np.concatenate(parts, -1)


def make_stepper(configs, world, dt, substeps, dtype, obs: dict | None = None, n_envs=None):
    st = Stepper(configs, dt=dt, substeps=substeps, device="cuda:0", dtype=dtype, world=world)
    if obs is not None:
        o = obstacles_np(obs, n_envs)
        body = {}
        if "kind" in o:  # movable compound bodies
            body = dict(kind=torch.tensor(o["kind"]), body=torch.tensor(o["body"]),
                        mass=torch.tensor(o["mass"]), inertia=torch.tensor(o["inertia"]),
                        body_offset=torch.tensor(o["body_off"]))
        st.set_obstacles(Obstacles(
            pos=torch.tensor(o["pos"]), radius=torch.tensor(o["radius"]),
            shape=torch.tensor(o["type"]), angle=torch.tensor(o["angle"]),
            half_extents=torch.tensor(o["half"]), vel=torch.tensor(o["vel"]),
            ang_vel=torch.tensor(o["ang_vel"]), **body,
        ))
    return st


def hip_run(stepper, s0_16, acts_np, w_traj, np_dtype):
    """Rollout + backward of loss = sum(w_traj * trajectory) on the HIP path.
    Returns (states [T,E,A,16], g_state0 [E,A,16] (stepped fields), g_actions)."""
    td = TDT[np_dtype]
    nf = 9 if stepper.has_drone else 5
    st = to_torch_state(s0_16, td, True, nf)
    acts = torch.tensor(np.ascontiguousarray(acts_np), dtype=td, device="cuda", requires_grad=True)
    final, traj = rollout(stepper, st, acts)
    loss = 0.0
    T = acts_np.shape[0]
    wt = torch.tensor(w_traj, dtype=td, device="cuda") if w_traj is not None else None
    for t in range(T):
        for k, (name, w, o) in enumerate(zip(FIELDS, WIDTH, OFFSET)):
            if k >= nf or wt is None:
                continue
            x = getattr(traj[t], name)
            ww = wt[t, ..., o:o + w]
            if w == 1:
                ww = ww[..., 0]
            loss = loss + (ww * x).sum()
    loss.backward()
    states = np.stack([state_to16(s) for s in traj])
    g0 = np.zeros_like(s0_16, dtype=np.float64)
    for k, (name, w, o) in enumerate(zip(FIELDS, WIDTH, OFFSET)):
        if k >= nf:
            continue
        g = getattr(st, name).grad
        if g is not None:
            g0[..., o:o + w] = g.double().cpu().numpy().reshape(g0.shape[:2] + (w,))
    return states, g0, acts.grad.double().cpu().numpy()


def oracle_run(configs, world, dt, substeps, s0_16, acts_np, w_traj, np_dtype, obs=None,
               n_threads=8):
    E = s0_16.shape[0]
    O = Oracle(np_dtype)
    cfg = oracle_cfg(configs, world, dt, substeps, E, acts_np.shape[-1], n_threads=n_threads)
    p, t, m = params_of(configs)
    ob = obstacles_np(obs, E)
    states = O.rollout(cfg, p, t, m, ob, s0_16, acts_np)
    g0, ga = O.rollout_adj(cfg, p, t, m, ob, s0_16, acts_np, states, w_traj, None)
    return states.astype(np.float64), g0.astype(np.float64), ga.astype(np.float64)


def rel(a, b):
    """Max-norm relative error: max |a - b| / max |b|."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


# Element-wise bar of the gradient parity tests: every element within ELEM_FACTOR times
# the max-norm tolerance of the reference value, relative to its magnitude plus an
# absolute floor of ELEM_FLOOR times the tensor's largest magnitude.  (An adjoint element
# that cancels to a small value carries the rounding of the terms it was summed from,
# and the summation order of the reverse pass is not the oracle's everywhere, so an
# element-wise bar needs the floor; fp32 runs measure up to 7e-5 with floor 1e-3, fp64
# runs 2e-13.)  With the fp32 tolerance 1e-5: each element within 1e-4 relative, or
# within 1e-7 of the largest element absolutely.
ELEM_FACTOR, ELEM_FLOOR = 10.0, 1e-3


def rel_elem(a, b, floor=ELEM_FLOOR):
    """Element-wise relative error with an absolute floor:
    max_i |a_i - b_i| / (|b_i| + floor * max |b|)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.abs(b) + floor * max(np.abs(b).max(), 1e-30)
    return float((np.abs(a - b) / den).max())


def check_grad(name, h, o, tol=1e-5, rtol=None, floor=ELEM_FLOOR):
    """Gradient parity: max-norm relative error <= tol and element-wise relative error
    (with the absolute floor) <= rtol (default ELEM_FACTOR * tol); both are printed."""
    rtol = ELEM_FACTOR * tol if rtol is None else rtol
    mn, el = rel(h, o), rel_elem(h, o, floor)
    print(f"{name}: max-norm rel {mn:.3e}, element-wise rel (floor {floor:g}) {el:.3e}")
    assert mn <= tol, f"{name}: max-norm rel {mn:.3e} > {tol:g}"
    assert el <= rtol, f"{name}: element-wise rel {el:.3e} > {rtol:g}"
