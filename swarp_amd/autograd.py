"""PyTorch autograd boundary of the step: ``TorchState``, ``warp_step``, ``rollout``,
``GradRing`` -- the drop-in surface of ``swarp/interop/autograd.py:29-369``.

The reference records every substep launch on a ``wp.Tape`` and replays Warp's
generated adjoints per step.  Here a rollout of T steps is one autograd node over two
HIP launches:

* forward: ``swarp_rollout_fwd`` runs all T steps, writing each step's output state
  (the trajectory, which doubles as the backward's checkpoints);
* backward: ``swarp_rollout_bwd`` walks the steps in reverse, recomputing each step's
  substeps from its checkpoint, and returns d(loss)/d(actions_seq) and d(loss)/d(state0).

``warp_step`` is the T = 1 case.  The per-step semantics are the reference's: grads flow
to the initial state and every action, every trajectory state can feed the loss, a
repeated backward (``retain_graph``) gives the same result, and returned grads are fresh
tensors.  Under ``torch.no_grad()`` (or when nothing requires grad) no graph is built
and ``warp_step`` writes into the stepper's two recycled output slots
(``swarp/core/stepper.py:688-710``).

For a fleet without drones the four drone fields (``z, vz, attitude, body_rates``) are
not stepped: every output state carries its own copies of the input's drone tensors,
whose values the reference copies unchanged (``swarp/dynamics/kernels.py:1856-1864``),
with their gradient passed through.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import NamedTuple

import torch

from . import _lib
from .stepper import Stepper, check_extent, state_struct

FIELDS = ("pos", "theta", "vel", "speed", "ang_vel", "z", "vz", "attitude", "body_rates")

#: Optional kernel timing sink: when a list, every rollout launch appends
#: (kind, start_event, end_event) recorded on the launch stream ("fwd" / "bwd").
KERNEL_EVENTS: list | None = None


#: timing events to record into instead of creating one per launch (a caller that times
#: kernels fills it with events already created on the device; creating an event on the
#: hot path costs host time that shows up in the timed loop)
EVENT_POOL: list | None = None


def _event(stream_tensor: torch.Tensor):
    pool = EVENT_POOL
    ev = pool.pop() if pool else torch.cuda.Event(enable_timing=True)
    ev.record(torch.cuda.current_stream(stream_tensor.device))
    return ev


_TAIL = ((2,), (), (2,), (), (), (), (), (4,), (3,))


class TorchState(NamedTuple):
    """Torch view of the world state (``swarp/interop/autograd.py:29-45``)."""

    pos: torch.Tensor  # [n_envs, n_agents, 2]
    theta: torch.Tensor  # [n_envs, n_agents]
    vel: torch.Tensor  # [n_envs, n_agents, 2]
    speed: torch.Tensor  # [n_envs, n_agents]
    ang_vel: torch.Tensor  # [n_envs, n_agents]
    z: torch.Tensor | None = None  # [n_envs, n_agents]
    vz: torch.Tensor | None = None  # [n_envs, n_agents]
    attitude: torch.Tensor | None = None  # [n_envs, n_agents, 4] (x, y, z, w)
    body_rates: torch.Tensor | None = None  # [n_envs, n_agents, 3]


def fill_state_defaults(state: TorchState) -> TorchState:
    """Materialise ``None`` drone fields as zeros / identity attitude
    (``swarp/interop/autograd.py:48-68``)."""
    if all(t is not None for t in state):
        return state
    ref = state.pos
    e, a = ref.shape[0], ref.shape[1]
    n = e * a
    # the missing fields are disjoint views of one allocation [z | vz | attitude |
    # body_rates], written by one library launch on a GPU (zeros and identity
    # quaternions), by torch elsewhere
    if ref.is_cuda and ref.dtype in (torch.float32, torch.float64):
        buf = torch.empty(9 * n, device=ref.device, dtype=ref.dtype)
        _lib.check(_lib.load().swarp_state_defaults(
            0 if ref.dtype == torch.float32 else 1, n, buf.data_ptr(), _stream(ref)))
    else:
        buf = torch.zeros(9 * n, device=ref.device, dtype=ref.dtype)
        buf[2 * n:6 * n].view(n, 4)[:, 3] = 1.0
    z = state.z if state.z is not None else buf[:n].view(e, a)
    vz = state.vz if state.vz is not None else buf[n:2 * n].view(e, a)
    att = state.attitude if state.attitude is not None else buf[2 * n:6 * n].view(e, a, 4)
    br = state.body_rates if state.body_rates is not None else buf[6 * n:].view(e, a, 3)
    return state._replace(z=z, vz=vz, attitude=att, body_rates=br)


def _nfields(stepper: Stepper) -> int:
    return 9 if stepper.has_drone else 5


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_of(t.device)


def _validate(stepper: Stepper, state: TorchState, actions_seq: torch.Tensor) -> tuple[int, int, int]:
    if actions_seq.dim() != 4:
        raise ValueError(
            f"actions must be [T, n_envs, n_agents, act_dim]; got {tuple(actions_seq.shape)}"
        )
    T, E, A, ad = actions_seq.shape
    if A != stepper.n_agents:
        raise ValueError(f"actions carry {A} agents, the stepper has {stepper.n_agents}")
    if ad < 1:
        raise ValueError("act_dim must be >= 1")
    if actions_seq.dtype != stepper.dtype:
        raise TypeError(f"actions dtype {actions_seq.dtype} does not match the stepper's {stepper.dtype}")
    if not actions_seq.is_cuda:
        raise RuntimeError(
            "swarp_amd steps on the HIP device only (no CPU fallback); got tensors on "
            f"{actions_seq.device}"
        )
    for name, t, tail in zip(FIELDS, state, _TAIL):
        if t is None:
            continue
        if tuple(t.shape) != (E, A, *tail):
            raise ValueError(f"state.{name} must be {[E, A, *tail]}; got {list(t.shape)}")
        if t.dtype != stepper.dtype:
            raise TypeError(f"state.{name} dtype {t.dtype} does not match the stepper's {stepper.dtype}")
        if t.device != actions_seq.device:
            raise ValueError(f"state.{name} is on {t.device}, actions on {actions_seq.device}")
    return T, E, ad


def _launch_fwd(stepper: Stepper, state0, actions_seq: torch.Tensor, traj, final,
                tape: torch.Tensor | None = None) -> None:
    """One forward launch; ``traj``/``final`` are field lists (``traj`` stacked [T-1,...]).
    ``tape`` (uint8, ``Stepper.tape_bytes`` long) also receives the rollout tape."""
    T, E, _, ad = actions_seq.shape
    nf = _nfields(stepper)
    lib = _lib.load()
    desc = stepper.desc(E, ad)
    EA, dt = E * stepper.n_agents, stepper.dtype
    check_extent(actions_seq, T * EA * ad, "actions", dt)
    s0 = state_struct(list(state0)[:nf], EA, dt, "state0")
    fin = state_struct(list(final)[:nf], EA, dt, "final")
    tr = state_struct(list(traj)[:nf], (T - 1) * EA, dt, "traj") if traj is not None and T > 1 else None
    if tape is not None:
        check_extent(tape, stepper.tape_bytes(E, ad, T), "tape", torch.uint8)
    if tape is None:
        _lib.check(lib.swarp_rollout_fwd(
            ctypes.byref(desc), T, ctypes.byref(s0), actions_seq.data_ptr(),
            ctypes.byref(tr) if tr is not None else None, ctypes.byref(fin), _stream(actions_seq),
        ))
        return
    _lib.check(lib.swarp_rollout_fwd_tape(
        ctypes.byref(desc), T, ctypes.byref(s0), actions_seq.data_ptr(),
        ctypes.byref(tr) if tr is not None else None, ctypes.byref(fin), tape.data_ptr(),
        tape.numel(), _stream(actions_seq),
    ))


def _empty_like_fields(stepper: Stepper, lead: tuple[int, ...], E: int, dev) -> list[torch.Tensor]:
    nf = _nfields(stepper)
    A = stepper.n_agents
    return [torch.empty(*lead, E, A, *_TAIL[k], device=dev, dtype=stepper.dtype) for k in range(nf)]


class _RolloutFn(torch.autograd.Function):
    """T steps as one autograd node; outputs = final state fields, then the stacked
    trajectory fields of steps 0..T-2."""

    @staticmethod
    def forward(ctx, stepper: Stepper, bufs, actions_seq: torch.Tensor, *state0: torch.Tensor):
        if stepper.world.wheel_contacts:  # swarp/core/stepper.py:852-857
            raise ValueError(
                "WorldConfig.wheel_contacts runs on the slim Euler 2D path only (no drone "
                "agents, untaped, Integrator.EULER)")
        ctx.set_materialize_grads(False)
        T, E = actions_seq.shape[0], actions_seq.shape[1]
        dev = actions_seq.device
        actions_seq = actions_seq.contiguous()
        state0 = tuple(t.contiguous() for t in state0)
        if bufs is None:
            final = _empty_like_fields(stepper, (), E, dev)
            traj = _empty_like_fields(stepper, (max(T - 1, 0),), E, dev)
        else:
            final, traj = bufs
        # the rollout tape lets the backward skip recomputing the substeps
        nb = stepper.tape_bytes(E, actions_seq.shape[3], T)
        tape = torch.empty(nb, device=dev, dtype=torch.uint8) if nb else None
        sink = KERNEL_EVENTS
        if sink is not None:
            e0 = _event(actions_seq)
        _launch_fwd(stepper, state0, actions_seq, traj, final, tape)
        if sink is not None:
            sink.append(("fwd", e0, _event(actions_seq)))
        ctx.stepper = stepper
        ctx.nf = len(state0)
        ctx.T = T
        ctx.tape = tape
        ctx.save_for_backward(actions_seq, *state0, *traj)
        return (*final, *traj)

    @staticmethod
    def backward(ctx, *grads):
        stepper: Stepper = ctx.stepper
        nf, T = ctx.nf, ctx.T
        saved = ctx.saved_tensors
        actions_seq = saved[0]
        state0 = saved[1:1 + nf]
        traj = saved[1 + nf:1 + 2 * nf]
        g_final = [None if g is None else g.contiguous() for g in grads[:nf]]
        g_traj = [None if g is None else g.contiguous() for g in grads[nf:2 * nf]]
        need = ctx.needs_input_grad
        adj_act = torch.empty_like(actions_seq)
        adj0 = [torch.empty_like(s) if need[3 + k] else None for k, s in enumerate(state0)]
        E, ad = actions_seq.shape[1], actions_seq.shape[3]
        lib = _lib.load()
        desc = stepper.desc(E, ad)
        EA, dt = E * stepper.n_agents, stepper.dtype
        check_extent(actions_seq, T * EA * ad, "actions", dt)
        check_extent(adj_act, T * EA * ad, "adj_actions", dt)
        s0 = state_struct(state0, EA, dt, "state0")
        tr = state_struct(traj, (T - 1) * EA, dt, "traj") if T > 1 else None
        gtr = (state_struct(g_traj, (T - 1) * EA, dt, "adj_traj")
               if T > 1 and any(g is not None for g in g_traj) else None)
        gfin = (state_struct(g_final, EA, dt, "adj_final")
                if any(g is not None for g in g_final) else None)
        a0 = state_struct(adj0, EA, dt, "adj_state0")
        sink = KERNEL_EVENTS
        if sink is not None:
            e0 = _event(actions_seq)
        tape = ctx.tape
        if tape is not None:
            check_extent(tape, stepper.tape_bytes(E, ad, T), "tape", torch.uint8)
        if tape is None:
            _lib.check(lib.swarp_rollout_bwd(
                ctypes.byref(desc), T, ctypes.byref(s0), actions_seq.data_ptr(),
                ctypes.byref(tr) if tr is not None else None,
                ctypes.byref(gtr) if gtr is not None else None,
                ctypes.byref(gfin) if gfin is not None else None,
                ctypes.byref(a0), adj_act.data_ptr(), _stream(actions_seq),
            ))
        else:
            _lib.check(lib.swarp_rollout_bwd_tape(
                ctypes.byref(desc), T, ctypes.byref(s0), actions_seq.data_ptr(),
                ctypes.byref(tr) if tr is not None else None,
                ctypes.byref(gtr) if gtr is not None else None,
                ctypes.byref(gfin) if gfin is not None else None,
                ctypes.byref(a0), adj_act.data_ptr(), tape.data_ptr(), tape.numel(),
                _stream(actions_seq),
            ))
        if sink is not None:
            sink.append(("bwd", e0, _event(actions_seq)))
        return (None, None, adj_act if need[2] else None, *adj0)


def _launch_fwd_ob(stepper: Stepper, state0, ob0: torch.Tensor, actions_seq: torch.Tensor,
                   traj, final, ob_traj: torch.Tensor, tape: torch.Tensor | None = None) -> None:
    """One forward launch of a world with movable bodies (five state fields, nine with
    drones); ``tape`` (uint8, ``Stepper.ob_tape_bytes`` long) also receives the body tape."""
    T, E, _, ad = actions_seq.shape
    nf = _nfields(stepper)
    lib = _lib.load()
    desc = stepper.desc(E, ad)
    EA, dt, NW = E * stepper.n_agents, stepper.dtype, 12 * stepper.n_obstacles
    check_extent(actions_seq, T * EA * ad, "actions", dt)
    check_extent(ob0, E * NW, "ob_state", dt)
    check_extent(ob_traj, T * E * NW, "ob_trajectory", dt)
    s0 = state_struct(list(state0)[:nf], EA, dt, "state0")
    fin = state_struct(list(final)[:nf], EA, dt, "final")
    tr = state_struct(list(traj)[:nf], (T - 1) * EA, dt, "traj") if traj is not None and T > 1 else None
    if tape is None:
        _lib.check(lib.swarp_rollout_fwd_ob(
            ctypes.byref(desc), T, ctypes.byref(s0), ob0.data_ptr(), actions_seq.data_ptr(),
            ctypes.byref(tr) if tr is not None else None, ctypes.byref(fin), ob_traj.data_ptr(),
            _stream(actions_seq),
        ))
        return
    check_extent(tape, stepper.ob_tape_bytes(E, ad, T), "ob_tape", torch.uint8)
    _lib.check(lib.swarp_rollout_fwd_ob_tape(
        ctypes.byref(desc), T, ctypes.byref(s0), ob0.data_ptr(), actions_seq.data_ptr(),
        ctypes.byref(tr) if tr is not None else None, ctypes.byref(fin), ob_traj.data_ptr(),
        tape.data_ptr(), tape.numel(), _stream(actions_seq),
    ))


class _RolloutObFn(torch.autograd.Function):
    """T steps of a world with movable bodies as one autograd node: inputs (actions,
    obstacle state, the five state fields, nine with drones); outputs the final state
    fields, the stacked trajectory fields of steps 0..T-2, and the obstacle states after
    every step ``[T, n_envs, 12 N]``."""

    @staticmethod
    def forward(ctx, stepper: Stepper, actions_seq: torch.Tensor, ob0: torch.Tensor,
                *state0: torch.Tensor):
        ctx.set_materialize_grads(False)
        T, E = actions_seq.shape[0], actions_seq.shape[1]
        dev = actions_seq.device
        actions_seq = actions_seq.contiguous()
        ob0 = ob0.contiguous()
        state0 = tuple(t.contiguous() for t in state0)
        final = _empty_like_fields(stepper, (), E, dev)
        traj = _empty_like_fields(stepper, (max(T - 1, 0),), E, dev)
        ob_traj = torch.empty((T,) + tuple(ob0.shape), device=dev, dtype=ob0.dtype)
        # the body tape lets the backward skip evaluating the body pass again
        nb = stepper.ob_tape_bytes(E, actions_seq.shape[3], T)
        tape = torch.empty(nb, device=dev, dtype=torch.uint8) if nb else None
        sink = KERNEL_EVENTS
        if sink is not None:
            e0 = _event(actions_seq)
        _launch_fwd_ob(stepper, state0, ob0, actions_seq, traj, final, ob_traj, tape)
        if sink is not None:
            sink.append(("fwd", e0, _event(actions_seq)))
        ctx.stepper = stepper
        ctx.tape = tape
        ctx.T = T
        ctx.nf = len(state0)
        ctx.save_for_backward(actions_seq, ob0, ob_traj, *state0, *traj)
        return (*final, *traj, ob_traj)

    @staticmethod
    def backward(ctx, *grads):
        stepper: Stepper = ctx.stepper
        T, nf = ctx.T, ctx.nf
        saved = ctx.saved_tensors
        actions_seq, ob0, ob_traj = saved[0], saved[1], saved[2]
        state0 = saved[3:3 + nf]
        traj = saved[3 + nf:3 + 2 * nf]
        g_final = [None if g is None else g.contiguous() for g in grads[:nf]]
        g_traj = [None if g is None else g.contiguous() for g in grads[nf:2 * nf]]
        g_ob = grads[2 * nf].contiguous() if grads[2 * nf] is not None else None
        need = ctx.needs_input_grad
        adj_act = torch.empty_like(actions_seq)
        adj_ob0 = torch.empty_like(ob0) if need[2] else None
        adj0 = [torch.empty_like(s) if need[3 + k] else None for k, s in enumerate(state0)]
        E, ad = actions_seq.shape[1], actions_seq.shape[3]
        lib = _lib.load()
        desc = stepper.desc(E, ad)
        EA, dt, NW = E * stepper.n_agents, stepper.dtype, 12 * stepper.n_obstacles
        check_extent(actions_seq, T * EA * ad, "actions", dt)
        check_extent(adj_act, T * EA * ad, "adj_actions", dt)
        check_extent(ob0, E * NW, "ob_state", dt)
        check_extent(ob_traj, T * E * NW, "ob_trajectory", dt)
        check_extent(g_ob, T * E * NW, "adj_ob_trajectory", dt)
        check_extent(adj_ob0, E * NW, "adj_ob_state", dt)
        s0 = state_struct(state0, EA, dt, "state0")
        tr = state_struct(traj, (T - 1) * EA, dt, "traj") if T > 1 else None
        gtr = (state_struct(g_traj, (T - 1) * EA, dt, "adj_traj")
               if T > 1 and any(g is not None for g in g_traj) else None)
        gfin = (state_struct(g_final, EA, dt, "adj_final")
                if any(g is not None for g in g_final) else None)
        a0 = state_struct(adj0, EA, dt, "adj_state0")
        sink = KERNEL_EVENTS
        if sink is not None:
            e0 = _event(actions_seq)
        args = (
            ctypes.byref(desc), T, ctypes.byref(s0), ob0.data_ptr(), actions_seq.data_ptr(),
            ctypes.byref(tr) if tr is not None else None, ob_traj.data_ptr(),
            ctypes.byref(gtr) if gtr is not None else None,
            ctypes.byref(gfin) if gfin is not None else None,
            g_ob.data_ptr() if g_ob is not None else None, ctypes.byref(a0),
            adj_ob0.data_ptr() if adj_ob0 is not None else None, adj_act.data_ptr(),
        )
        tape = ctx.tape
        if tape is None:
            _lib.check(lib.swarp_rollout_bwd_ob(*args, _stream(actions_seq)))
        else:
            check_extent(tape, stepper.ob_tape_bytes(E, ad, T), "ob_tape", torch.uint8)
            _lib.check(lib.swarp_rollout_bwd_ob_tape(*args, tape.data_ptr(), tape.numel(),
                                                     _stream(actions_seq)))
        if sink is not None:
            sink.append(("bwd", e0, _event(actions_seq)))
        return (None, adj_act if need[1] else None, adj_ob0, *adj0)


def _rollout_bodies(stepper: Stepper, state: TorchState, actions_seq: torch.Tensor,
                    given=(True,) * 9):
    """rollout / warp_step of a world with movable bodies: consumes ``stepper.ob_state``,
    leaves the obstacle state after the last step in it and every step's in
    ``stepper.ob_trajectory``."""
    T, E, _ = _validate(stepper, state, actions_seq)
    ob0 = stepper.ob_state
    if ob0 is None or tuple(ob0.shape) != (E, 12 * stepper.n_obstacles):
        raise ValueError(f"stepper.ob_state must be [{E}, {12 * stepper.n_obstacles}]")
    grad = torch.is_grad_enabled() and (
        ob0.requires_grad or actions_seq.requires_grad
        or any(t is not None and t.requires_grad for t in state))
    nf = _nfields(stepper)
    if grad:
        # a configuration the body backward refuses is refused before the forward runs,
        # so that stepper.ob_state / ob_trajectory are not advanced by a forward whose
        # backward could not follow
        _lib.check(_lib.load().swarp_rollout_bwd_ob_check(
            ctypes.byref(stepper.desc(E, actions_seq.shape[3]))))
        outs = _RolloutObFn.apply(stepper, actions_seq, ob0, *state[:nf])
        ob_traj = outs[2 * nf]
        outs = outs[:2 * nf]
    else:
        final = _empty_like_fields(stepper, (), E, actions_seq.device)
        traj = _empty_like_fields(stepper, (T - 1,), E, actions_seq.device)
        ob_traj = torch.empty((T,) + tuple(ob0.shape), device=ob0.device, dtype=ob0.dtype)
        _launch_fwd_ob(stepper, [t.contiguous() for t in state[:nf]], ob0.contiguous(),
                       actions_seq.contiguous(), traj, final, ob_traj)
        outs = (*final, *traj)
    stepper.ob_trajectory = ob_traj
    stepper.ob_state = ob_traj[T - 1]
    return _assemble(stepper, state, outs, T, given)


def _grad_mode(state: TorchState, actions: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and (
        actions.requires_grad or any(t is not None and t.requires_grad for t in state)
    )


class Trajectory(list):
    """The states after each step of a rollout: a ``list`` of :class:`TorchState` whose
    per-step states are built on first use.  A BPTT loop that only reads the final state
    never pays for the T - 1 per-step views (one unbind per field and a TorchState per
    step); any read, iteration or change of the list builds them all first, after which
    it behaves as a plain list.  ``len`` needs no build."""

    def __init__(self, n: int, build):
        super().__init__()
        self._n = n
        self._build = build

    def _fill(self) -> None:
        if self._build is not None:
            build, self._build = self._build, None
            list.extend(self, build())

    def __len__(self) -> int:
        return self._n if self._build is not None else list.__len__(self)

    def __bool__(self) -> bool:
        return len(self) > 0

    def __reduce_ex__(self, protocol):
        self._fill()
        return (list, (list(self),))


def _list_method(name):
    base = getattr(list, name)

    def method(self, *args, **kwargs):
        self._fill()
        return base(self, *args, **kwargs)

    method.__name__ = name
    return method


for _name in ("__getitem__", "__setitem__", "__delitem__", "__iter__", "__reversed__",
              "__contains__", "__eq__", "__ne__", "__lt__", "__le__", "__gt__", "__ge__",
              "__add__", "__iadd__", "__mul__", "__rmul__", "__imul__", "__repr__",
              "append", "extend", "insert", "pop", "remove", "index", "count",
              "clear", "copy", "sort", "reverse"):
    setattr(Trajectory, _name, _list_method(_name))
Trajectory.__hash__ = None


def _with_defaults(state: TorchState) -> tuple[TorchState, tuple[bool, ...]]:
    """fill_state_defaults, and which fields the caller provided."""
    given = tuple(t is not None for t in state)
    return fill_state_defaults(state), given


def _assemble(stepper: Stepper, state: TorchState, outs, T: int, given=(True,) * 9):
    """(final TorchState, trajectory) from the Function's outputs.  Every returned state
    owns its tensors, as the reference's per-step outputs do: for a 2-D fleet the four
    drone fields it does not step are passed through as copies of the input's (the
    defaults this call made are handed to the final state as they are)."""
    nf = _nfields(stepper)
    final_f = outs[:nf]
    traj_f = outs[nf:2 * nf]
    tail = tuple(state[nf:]) if nf == 5 else ()
    final_tail = tuple(t.clone() if given[nf + k] else t for k, t in enumerate(tail))
    final = TorchState(*final_f, *final_tail)
    # the per-step views are built later, possibly under another grad mode (a no_grad
    # logging read, inference mode): they are built under the modes of this call, so that
    # they carry the same autograd history as states built eagerly here would
    grad_on = torch.is_grad_enabled()
    inference_on = torch.is_inference_mode_enabled()

    def build():
        # one unbind per field (a single autograd node) instead of T - 1 selects per field;
        # the passed-through fields of the T - 1 states as one broadcast copy per field
        # (each state owns its own slice) instead of T - 1 copies
        with torch.inference_mode(inference_on), torch.set_grad_enabled(grad_on):
            per_step = [f.unbind(0) for f in traj_f] if T > 1 else []
            tails = ([x.unsqueeze(0).expand(T - 1, *x.shape).clone().unbind(0) for x in tail]
                     if T > 1 else [])
        steps = [TorchState(*(u[t] for u in per_step), *(v[t] for v in tails))
                 for t in range(T - 1)]
        steps.append(final)
        return steps

    return final, Trajectory(T, build)


@dataclass
class StepGradSlot:
    """One step's pre-allocated outputs inside a :class:`GradRing`."""

    ring: "GradRing"
    index: int

    @property
    def out(self) -> list[torch.Tensor]:
        return [b[self.index] for b in self.ring.bufs]


class GradRing:
    """Reusable output buffers for BPTT rollouts (``swarp/interop/autograd.py:184-226``).

    Holds ``capacity`` step outputs.  ``rollout(..., ring=ring)`` writes a T-step
    trajectory (T <= capacity) into it with no allocation; ``warp_step(..., slot=...)``
    writes one step into the slot ``acquire`` hands out.  Reusing the ring overwrites
    the previous rollout's outputs (the returned grads are always fresh tensors).
    """

    def __init__(self, stepper: Stepper, n_envs: int, act_dim: int, capacity: int) -> None:
        if capacity < 1:
            raise ValueError("GradRing capacity must be >= 1")
        self.stepper = stepper
        self.capacity = capacity
        self.n_envs = n_envs
        self.act_dim = act_dim
        self._idx = 0
        self.bufs = _empty_like_fields(stepper, (capacity,), n_envs, torch.device(stepper.device))
        self.slots = [StepGradSlot(self, i) for i in range(capacity)]

    def reset(self) -> None:
        self._idx = 0

    def acquire(self) -> StepGradSlot:
        if self._idx >= self.capacity:
            raise RuntimeError(
                f"GradRing capacity {self.capacity} exhausted; size it to the rollout length T"
            )
        slot = self.slots[self._idx]
        self._idx += 1
        return slot

    def rollout_buffers(self, T: int):
        if T > self.capacity:
            raise RuntimeError(
                f"GradRing capacity {self.capacity} exhausted; size it to the rollout length T"
            )
        self._idx = T
        final = [b[T - 1] for b in self.bufs]
        traj = [b[: T - 1] for b in self.bufs]
        return final, traj


def warp_step(
    stepper: Stepper,
    state: TorchState,
    actions: torch.Tensor,
    slot: StepGradSlot | None = None,
) -> TorchState:
    """Differentiable env step ``state, actions -> next state``
    (``swarp/interop/autograd.py:299-338``)."""
    state, given = _with_defaults(state)
    if actions.dim() != 3:
        raise ValueError(f"actions must be [n_envs, n_agents, act_dim]; got {tuple(actions.shape)}")
    seq = actions.unsqueeze(0)
    if stepper.any_movable:
        final, _ = _rollout_bodies(stepper, state, seq, given)
        return final
    _validate(stepper, state, seq)
    nf = _nfields(stepper)
    if _grad_mode(state, actions):
        bufs = None
        if slot is not None:
            bufs = (slot.out, [b[:0] for b in slot.ring.bufs])
        outs = _RolloutFn.apply(stepper, bufs, seq, *state[:nf])
        final, _ = _assemble(stepper, state, outs, 1, given)
        return final
    out = stepper.output_state(actions.shape[0])
    final = list(out[:nf])
    _launch_fwd(stepper, [t.contiguous() for t in state[:nf]], seq.contiguous(), None, final)
    tail = tuple(state[nf:]) if nf == 5 else ()
    return TorchState(*final, *tail)


def rollout(
    stepper: Stepper,
    state: TorchState,
    actions_seq: torch.Tensor,
    ring: GradRing | None = None,
) -> tuple[TorchState, list[TorchState]]:
    """Backprop-through-time rollout (``swarp/interop/autograd.py:341-369``).

    ``actions_seq [T, n_envs, n_agents, act_dim]``.  Returns ``(final_state,
    trajectory)`` with the state after each of the T steps (a :class:`Trajectory`, a
    list built on first use); gradients flow to ``state`` and ``actions_seq``.
    """
    state, given = _with_defaults(state)
    if stepper.any_movable:
        return _rollout_bodies(stepper, state, actions_seq, given)
    T, E, _ = _validate(stepper, state, actions_seq)
    if T < 1:
        raise ValueError("actions_seq must hold at least one step")
    nf = _nfields(stepper)
    bufs = None
    if ring is not None:
        ring.reset()
        bufs = ring.rollout_buffers(T)
    if _grad_mode(state, actions_seq):
        outs = _RolloutFn.apply(stepper, bufs, actions_seq, *state[:nf])
    else:
        if bufs is None:
            final = _empty_like_fields(stepper, (), E, actions_seq.device)
            traj = _empty_like_fields(stepper, (T - 1,), E, actions_seq.device)
        else:
            final, traj = bufs
        _launch_fwd(stepper, [t.contiguous() for t in state[:nf]], actions_seq.contiguous(), traj, final)
        outs = (*final, *traj)
    return _assemble(stepper, state, outs, T, given)
