"""ctypes wrapper of the CPU restatement (oracle/swarp_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; never by the swarp_amd package.

States cross this wrapper as numpy arrays ``[..., 16]`` in TorchState field order:
pos(2) theta vel(2) speed ang_vel z vz attitude(4) body_rates(3).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libswarp_oracle.so"

FIELDS = ("pos", "theta", "vel", "speed", "ang_vel", "z", "vz", "attitude", "body_rates")
WIDTH = (2, 1, 2, 1, 1, 1, 1, 4, 3)
OFFSET = tuple(int(x) for x in np.cumsum((0,) + WIDTH[:-1]))


class OracleCfg(ctypes.Structure):
    _fields_ = [
        ("n_envs", ctypes.c_int), ("n_agents", ctypes.c_int), ("act_dim", ctypes.c_int),
        ("substeps", ctypes.c_int), ("max_neighbors", ctypes.c_int),
        ("collisions", ctypes.c_int), ("soft_walls", ctypes.c_int),
        ("clamp_bounds", ctypes.c_int), ("n_threads", ctypes.c_int),
        ("dt", ctypes.c_double), ("k", ctypes.c_double), ("c", ctypes.c_double),
        ("margin", ctypes.c_double), ("max_overlap", ctypes.c_double),
        ("neighbor_radius", ctypes.c_double),
        ("bmin_x", ctypes.c_double), ("bmin_y", ctypes.c_double),
        ("bmax_x", ctypes.c_double), ("bmax_y", ctypes.c_double),
        ("lin_damping", ctypes.c_double), ("ang_damping", ctypes.c_double),
        ("rk4", ctypes.c_int), ("wheel", ctypes.c_int),
        ("lat_grip", ctypes.c_double), ("turn_cap", ctypes.c_double),
        ("grid_bins", ctypes.c_int), ("grid_ox", ctypes.c_double), ("grid_oy", ctypes.c_double),
        ("grid_cell", ctypes.c_double),
    ]


class OracleObs(ctypes.Structure):
    _fields_ = [
        ("n_obstacles", ctypes.c_int),
        ("pos", ctypes.c_void_p), ("radius", ctypes.c_void_p), ("angle", ctypes.c_void_p),
        ("half", ctypes.c_void_p), ("vel", ctypes.c_void_p), ("ang_vel", ctypes.c_void_p),
        ("type", ctypes.c_void_p),
        ("kind", ctypes.c_void_p), ("body", ctypes.c_void_p),
        ("mass", ctypes.c_void_p), ("inertia", ctypes.c_void_p), ("body_off", ctypes.c_void_p),
        ("body_params", ctypes.c_void_p),
    ]


def build() -> Path:
    """Compile the restatement with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def pack_state(state: dict, dtype=np.float64) -> np.ndarray:
    """dict of field arrays ([E,A,w] or [E,A]) -> [E,A,16]; missing drone fields default."""
    pos = np.asarray(state["pos"])
    E, A = pos.shape[:2]
    out = np.zeros((E, A, 16), dtype=dtype)
    out[..., 12] = 1.0  # attitude w
    for name, w, o in zip(FIELDS, WIDTH, OFFSET):
        v = state.get(name)
        if v is None:
            continue
        v = np.asarray(v, dtype=dtype).reshape(E, A, w)
        out[..., o:o + w] = v
    return out


def unpack_state(arr: np.ndarray) -> dict:
    """[..., 16] -> dict of field arrays with TorchState shapes."""
    res = {}
    for name, w, o in zip(FIELDS, WIDTH, OFFSET):
        v = arr[..., o:o + w]
        res[name] = v[..., 0] if w == 1 else v
    return res


class Oracle:
    """One precision of the restatement.  ``cfg`` is a dict with the keys of OracleCfg."""

    def __init__(self, dtype=np.float64):
        self.dtype = np.dtype(dtype)
        self.suf = "f64" if self.dtype == np.float64 else "f32"

    def _fn(self, name):
        return getattr(lib(), f"oracle_{name}_{self.suf}")

    def _cfg(self, cfg: dict) -> OracleCfg:
        c = OracleCfg()
        for k, _ in OracleCfg._fields_:
            setattr(c, k, cfg.get(k, 0))
        if c.n_threads == 0:
            c.n_threads = 1
        return c

    def _obs(self, obs: dict | None, keep: list):
        o = OracleObs()
        if not obs:
            o.n_obstacles = 0
            return o
        arrs = {}
        for k in ("pos", "radius", "angle", "half", "vel", "ang_vel"):
            arrs[k] = np.ascontiguousarray(obs[k], dtype=self.dtype)
        arrs["type"] = np.ascontiguousarray(obs["type"], dtype=np.int32)
        if obs.get("kind") is not None:
            n = arrs["radius"].shape[0]
            arrs["kind"] = np.ascontiguousarray(obs["kind"], dtype=np.int32)
            body = obs.get("body")
            arrs["body"] = np.ascontiguousarray(np.arange(n) if body is None else body, dtype=np.int32)
            arrs["mass"] = np.ascontiguousarray(obs.get("mass", np.ones(n)), dtype=self.dtype)
            arrs["inertia"] = np.ascontiguousarray(obs.get("inertia", np.ones(n)), dtype=self.dtype)
            off = obs.get("body_off")
            arrs["body_off"] = np.ascontiguousarray(np.zeros((n, 2)) if off is None else off,
                                                    dtype=self.dtype)
        if obs.get("body_params") is not None:
            # [A, 22] rows the body pass reads (the shared table under per-env rows)
            arrs["body_params"] = np.ascontiguousarray(obs["body_params"], dtype=self.dtype)
        keep.append(arrs)
        o.n_obstacles = int(arrs["radius"].shape[0])
        for k, v in arrs.items():
            setattr(o, k, _p(v))
        return o

    def _prm(self, params, tags, modes, keep):
        p = np.ascontiguousarray(params, dtype=self.dtype)
        t = np.ascontiguousarray(tags, dtype=np.int32)
        m = np.ascontiguousarray(modes, dtype=np.int32)
        keep += [p, t, m]
        return p, t, m

    def rollout(self, cfg, params, tags, modes, obs, state0, actions):
        keep = []
        c = self._cfg(cfg)
        p, t, m = self._prm(params, tags, modes, keep)
        o = self._obs(obs, keep)
        s0 = np.ascontiguousarray(state0, dtype=self.dtype)
        act = np.ascontiguousarray(actions, dtype=self.dtype)
        T = act.shape[0]
        out = np.zeros((T,) + s0.shape, dtype=self.dtype)
        fn = self._fn("rollout")
        fn.restype = ctypes.c_int
        rc = fn(ctypes.byref(c), _p(p), _p(t), _p(m), ctypes.byref(o), ctypes.c_int(T), _p(s0),
                _p(act), _p(out))
        if rc != 0:
            raise RuntimeError("oracle_rollout failed")
        return out

    def rollout_adj(self, cfg, params, tags, modes, obs, state0, actions, states,
                    adj_states=None, adj_final=None):
        keep = []
        c = self._cfg(cfg)
        p, t, m = self._prm(params, tags, modes, keep)
        o = self._obs(obs, keep)
        s0 = np.ascontiguousarray(state0, dtype=self.dtype)
        act = np.ascontiguousarray(actions, dtype=self.dtype)
        st = np.ascontiguousarray(states, dtype=self.dtype)
        T = act.shape[0]
        ast = None if adj_states is None else np.ascontiguousarray(adj_states, dtype=self.dtype)
        afin = None if adj_final is None else np.ascontiguousarray(adj_final, dtype=self.dtype)
        a0 = np.zeros_like(s0)
        aact = np.zeros_like(act)
        fn = self._fn("rollout_adj")
        fn.restype = ctypes.c_int
        rc = fn(ctypes.byref(c), _p(p), _p(t), _p(m), ctypes.byref(o), ctypes.c_int(T), _p(s0),
                _p(act), _p(st), _p(ast), _p(afin), _p(a0), _p(aact))
        if rc != 0:
            raise RuntimeError("oracle_rollout_adj failed")
        return a0, aact

    def rollout_ob(self, cfg, params, tags, modes, obs, state0, ob0, actions):
        """Rollout with the obstacle state (``[E, 12 N]`` per step: shape pos, angle, vel,
        ang_vel, then the body state of each root) carried along; returns (states, ob)."""
        keep = []
        c = self._cfg(cfg)
        p, t, m = self._prm(params, tags, modes, keep)
        o = self._obs(obs, keep)
        s0 = np.ascontiguousarray(state0, dtype=self.dtype)
        b0 = None if ob0 is None else np.ascontiguousarray(ob0, dtype=self.dtype)
        act = np.ascontiguousarray(actions, dtype=self.dtype)
        T = act.shape[0]
        E = s0.shape[0]
        out = np.zeros((T,) + s0.shape, dtype=self.dtype)
        obo = np.zeros((T, E, 12 * o.n_obstacles), dtype=self.dtype)
        fn = self._fn("rollout_ob")
        fn.restype = ctypes.c_int
        rc = fn(ctypes.byref(c), _p(p), _p(t), _p(m), ctypes.byref(o), ctypes.c_int(T), _p(s0),
                _p(b0), _p(act), _p(out), _p(obo))
        if rc != 0:
            raise RuntimeError("oracle_rollout_ob failed")
        return out, obo

    def rollout_adj_ob(self, cfg, params, tags, modes, obs, state0, ob0, actions, states, ob_states,
                       adj_states=None, adj_final=None, adj_ob_states=None, adj_ob_final=None):
        keep = []
        c = self._cfg(cfg)
        p, t, m = self._prm(params, tags, modes, keep)
        o = self._obs(obs, keep)
        cast = lambda a: None if a is None else np.ascontiguousarray(a, dtype=self.dtype)  # noqa: E731
        s0, b0, act, st, obst = cast(state0), cast(ob0), cast(actions), cast(states), cast(ob_states)
        ast, afin, aob, aobf = cast(adj_states), cast(adj_final), cast(adj_ob_states), cast(adj_ob_final)
        T = act.shape[0]
        a0 = np.zeros_like(s0)
        aob0 = np.zeros((s0.shape[0], 12 * o.n_obstacles), dtype=self.dtype)
        aact = np.zeros_like(act)
        fn = self._fn("rollout_adj_ob")
        fn.restype = ctypes.c_int
        rc = fn(ctypes.byref(c), _p(p), _p(t), _p(m), ctypes.byref(o), ctypes.c_int(T), _p(s0),
                _p(b0), _p(act), _p(st), _p(obst), _p(ast), _p(afin), _p(aob), _p(aobf), _p(a0),
                _p(aob0), _p(aact))
        if rc != 0:
            raise RuntimeError("oracle_rollout_adj_ob failed")
        return a0, aob0, aact

    def neighbors(self, pos, radius, K):
        pos = np.ascontiguousarray(pos, dtype=self.dtype)
        E, A = pos.shape[:2]
        idx = np.zeros((E, A, K), dtype=np.int32)
        cnt = np.zeros((E, A), dtype=np.int32)
        tru = np.zeros((E, A), dtype=np.int32)
        fn = self._fn("neighbors")
        fn.restype = ctypes.c_int
        fn(ctypes.c_int(E), ctypes.c_int(A), ctypes.c_int(K), _p(pos), ctypes.c_double(radius),
           _p(idx), _p(cnt), _p(tru))
        return idx, cnt, tru

    def neighbors_grid(self, pos, radius, K, bins, frame=None):
        """Lists in the uniform grid's order; ``frame`` = (ox, oy, cell) pins the frame (as
        float64, rounded to the oracle's precision), None reduces it over the batch.
        Returns idx, cnt, tru and the frame used."""
        pos = np.ascontiguousarray(pos, dtype=self.dtype)
        E, A = pos.shape[:2]
        idx = np.zeros((E, A, K), dtype=np.int32)
        cnt = np.zeros((E, A), dtype=np.int32)
        tru = np.zeros((E, A), dtype=np.int32)
        fr = np.zeros(3, dtype=self.dtype)
        ox, oy, cs = frame if frame is not None else (0.0, 0.0, 0.0)
        fn = self._fn("neighbors_grid")
        fn.restype = ctypes.c_int
        rc = fn(ctypes.c_int(E), ctypes.c_int(A), ctypes.c_int(K), _p(pos),
                ctypes.c_double(radius), ctypes.c_int(bins), ctypes.c_int(frame is not None),
                ctypes.c_double(ox), ctypes.c_double(oy), ctypes.c_double(cs), _p(idx), _p(cnt),
                _p(tru), _p(fr))
        if rc != 0:
            raise RuntimeError("oracle_neighbors_grid failed")
        return idx, cnt, tru, fr

    def forces(self, cfg, params, tags, modes, obs, state):
        keep = []
        c = self._cfg(cfg)
        p, t, m = self._prm(params, tags, modes, keep)
        o = self._obs(obs, keep)
        s = np.ascontiguousarray(state, dtype=self.dtype)
        F = np.zeros(s.shape[:2] + (2,), dtype=self.dtype)
        fn = self._fn("forces")
        fn.restype = ctypes.c_int
        fn(ctypes.byref(c), _p(p), _p(t), _p(m), ctypes.byref(o), _p(s), _p(F))
        return F


def cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


PMATH = {"sin": 0, "cos": 1, "tan": 2, "atan": 3, "tanh": 4}


def pmath(name: str, x: np.ndarray) -> np.ndarray:
    """The portable transcendental ``name`` (include/swarp_pmath.h) over ``x`` (float32:
    evaluated in double and rounded once, as the kernels do; float64: as is)."""
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    L = lib()
    fn = L.oracle_pmath_f32 if x.dtype == np.float32 else L.oracle_pmath_f64
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long]
    fn.restype = None
    fn(PMATH[name], _p(x), _p(y), x.size)
    return y
