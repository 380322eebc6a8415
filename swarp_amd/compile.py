"""``torch.compile``-compatible step: the HIP step registered as the functional custom op
``swarp_amd::step`` with a fake (meta) implementation and an autograd rule
(counterpart of ``swarp/interop/compile.py:1-186``).

``warp_step`` wraps a ``torch.autograd.Function`` around ctypes launches, which Dynamo
cannot trace (it graph-breaks there).  Routed through the custom op, a compiled policy /
environment loop sees the step as one opaque, differentiable operator.

The op is functional: the forward writes freshly allocated outputs (the four drone
fields of a 2-D fleet are copied through, never aliased) and mutates no input; the
backward is a second opaque op, ``swarp_amd::step_bwd``, which launches the step's
adjoint (``swarp_rollout_bwd``, T = 1) on the saved inputs, recomputing the substeps
inside the kernel, so nothing survives between the two calls.  Both ops have fake
implementations: AOTAutograd traces the backward graph with fake tensors, so the
autograd rule itself must not touch device memory.
Steppers cross the op boundary as integer handles from a weak registry: a handle does not
keep its stepper (and its device buffers) alive.  Worlds with movable bodies carry an
obstacle state the op's signature has no room for; they raise ``NotImplementedError``.
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from . import _lib
from .autograd import (TorchState, _empty_like_fields, _launch_fwd, _nfields, _stream,
                       fill_state_defaults, warp_step)
from .stepper import Stepper, check_extent, state_struct

_STEPPERS: "weakref.WeakValueDictionary[int, Stepper]" = weakref.WeakValueDictionary()
_HANDLES: dict[int, int] = {}  # id(stepper) -> handle
_NEXT_ID = 0


def register_stepper(stepper: Stepper) -> int:
    """A stable integer handle for ``stepper`` (held weakly; the caller keeps the stepper
    alive for as long as the compiled step is used)."""
    global _NEXT_ID
    handle = _HANDLES.get(id(stepper))
    if handle is not None:
        return handle
    handle = _NEXT_ID
    _NEXT_ID += 1
    _STEPPERS[handle] = stepper
    _HANDLES[id(stepper)] = handle
    weakref.finalize(stepper, _HANDLES.pop, id(stepper), None)
    return handle


def _stepper(handle: int) -> Stepper:
    try:
        return _STEPPERS[handle]
    except KeyError:
        raise RuntimeError(
            f"swarp_amd::step was called with handle {handle}, whose Stepper has been "
            "garbage-collected. Keep the Environment/World (or the Stepper itself) alive for "
            "as long as the compiled step is used.") from None


@torch.library.custom_op("swarp_amd::step", mutates_args=())
def _step_op(stepper_id: int, actions: torch.Tensor, pos: torch.Tensor, theta: torch.Tensor,
             vel: torch.Tensor, speed: torch.Tensor, ang_vel: torch.Tensor, z: torch.Tensor,
             vz: torch.Tensor, attitude: torch.Tensor,
             body_rates: torch.Tensor) -> list[torch.Tensor]:
    stepper = _stepper(stepper_id)
    if stepper.any_movable:
        raise NotImplementedError("the compiled step does not carry movable-body state")
    state = (pos, theta, vel, speed, ang_vel, z, vz, attitude, body_rates)
    nf = _nfields(stepper)
    seq = actions.unsqueeze(0).contiguous()
    final = _empty_like_fields(stepper, (), actions.shape[0], actions.device)
    _launch_fwd(stepper, [t.contiguous() for t in state[:nf]], seq, None, final)
    return [*final, *(t.clone() for t in state[nf:])]


@_step_op.register_fake
def _step_op_fake(stepper_id, actions, pos, theta, vel, speed, ang_vel, z, vz, attitude,
                  body_rates):
    # fresh contiguous outputs, like the real op (not the inputs' strides)
    return [torch.empty(t.shape, dtype=t.dtype, device=t.device)
            for t in (pos, theta, vel, speed, ang_vel, z, vz, attitude, body_rates)]


@torch.library.custom_op("swarp_amd::step_bwd", mutates_args=())
def _step_bwd_op(stepper_id: int, actions: torch.Tensor, pos: torch.Tensor, theta: torch.Tensor,
                 vel: torch.Tensor, speed: torch.Tensor, ang_vel: torch.Tensor, z: torch.Tensor,
                 vz: torch.Tensor, attitude: torch.Tensor, body_rates: torch.Tensor,
                 g_pos: torch.Tensor | None, g_theta: torch.Tensor | None,
                 g_vel: torch.Tensor | None, g_speed: torch.Tensor | None,
                 g_ang_vel: torch.Tensor | None, g_z: torch.Tensor | None,
                 g_vz: torch.Tensor | None, g_attitude: torch.Tensor | None,
                 g_body_rates: torch.Tensor | None) -> list[torch.Tensor]:
    """Adjoint of one step: [d actions, d pos, ..., d body_rates] (fresh tensors)."""
    stepper = _stepper(stepper_id)
    state = (pos, theta, vel, speed, ang_vel, z, vz, attitude, body_rates)
    grads = (g_pos, g_theta, g_vel, g_speed, g_ang_vel, g_z, g_vz, g_attitude, g_body_rates)
    nf = _nfields(stepper)
    E, ad = actions.shape[0], actions.shape[2]
    seq = actions.unsqueeze(0).contiguous()
    s0 = [t.contiguous() for t in state[:nf]]
    g_final = [None if g is None else g.contiguous() for g in grads[:nf]]
    adj0 = [torch.empty_like(t) for t in s0]
    adj_act = torch.empty_like(seq)
    lib = _lib.load()
    desc = stepper.desc(E, ad)
    EA, dt = E * stepper.n_agents, stepper.dtype
    check_extent(seq, EA * ad, "actions", dt)
    gfin = state_struct(g_final, EA, dt, "adj_final") if any(g is not None for g in g_final) else None
    st0, a0 = state_struct(s0, EA, dt, "state0"), state_struct(adj0, EA, dt, "adj_state0")
    _lib.check(lib.swarp_rollout_bwd(
        ctypes.byref(desc), 1, ctypes.byref(st0), seq.data_ptr(), None, None,
        ctypes.byref(gfin) if gfin is not None else None, ctypes.byref(a0), adj_act.data_ptr(),
        _stream(seq)))
    # the fields a 2-D fleet does not step pass through: so does their adjoint
    tail = [torch.zeros_like(state[k]) if grads[k] is None else grads[k].clone()
            for k in range(nf, 9)]
    return [adj_act[0], *adj0, *tail]


@_step_bwd_op.register_fake
def _step_bwd_op_fake(stepper_id, actions, pos, theta, vel, speed, ang_vel, z, vz, attitude,
                      body_rates, g_pos, g_theta, g_vel, g_speed, g_ang_vel, g_z, g_vz,
                      g_attitude, g_body_rates):
    return [torch.empty(t.shape, dtype=t.dtype, device=t.device)
            for t in (actions, pos, theta, vel, speed, ang_vel, z, vz, attitude, body_rates)]


def _setup_context(ctx, inputs, output):
    stepper_id, actions, *state = inputs
    ctx.stepper_id = stepper_id
    ctx.save_for_backward(actions, *state)


def _backward(ctx, *grad_outputs):
    grads = grad_outputs[0] if len(grad_outputs) == 1 else grad_outputs
    actions, *state = ctx.saved_tensors
    outs = torch.ops.swarp_amd.step_bwd(ctx.stepper_id, actions, *state, *grads)
    return (None, *outs)


_step_op.register_autograd(_backward, setup_context=_setup_context)


def compiled_warp_step(stepper: Stepper, state: TorchState, actions: torch.Tensor) -> TorchState:
    """``warp_step`` routed through the ``swarp_amd::step`` custom op (torch.compile-safe)."""
    state = fill_state_defaults(state)
    outs = torch.ops.swarp_amd.step(register_stepper(stepper), actions, *state)
    return TorchState(*outs)


__all__ = ["compiled_warp_step", "register_stepper", "warp_step"]
