"""Whole-step HIP graph of a ``World``: the step plus the scenario's post-step pass in
one graph replay (counterpart of the reference's persistent runtime,
``swarp/interop/persistent.py:72-390``, and ``World.enable_persistent``).

The world's state lives in two persistent buffer sets (ping-pong): graph ``g[k]`` steps
set ``k`` into set ``1 - k`` and runs the post-step hook on set ``1 - k``, so a replay
reads and writes only pointers fixed at capture time.  A step copies the caller's
actions into a persistent buffer, replays the graph of the current set and flips.  A
state the caller replaced (a differentiated step, ``reset_state``) is copied into the
current set before the next replay.  The graphs are captured lazily and recaptured when
a pointer they baked in moves (obstacles, buffers) -- the reference's recapture token.

Differentiated steps never come here: a graph replay records nothing for autograd.

Lifetime: bound-method hooks are held weakly, so an owner (an ``Environment``) and its
StepGraph form no reference cycle and the captured graphs die by reference counting when
the owner does.  A graph left to the cyclic collector could be destroyed in the middle of
another capture -- a collection can start at any Python allocation -- and destroying a
graph while a stream is capturing aborts the process.  For the same reason the collector
is paused while a capture is open.
"""

from __future__ import annotations

import ctypes
import gc
import inspect
import weakref
from typing import Callable

import torch

from . import _lib
from .autograd import FIELDS, TorchState
from .stepper import check_extent, state_struct

#: hook(state_out, stream, warm): launches the post-step work on ``state_out``; ``warm``
#: marks the eager warm-up launch before a capture, which must leave carried state alone
Hook = Callable[[TorchState, int, bool], None]


def _held(fn):
    """A zero-argument getter for ``fn``: weak for a bound method (no cycle through its
    owner), strong otherwise."""
    if fn is None:
        return lambda: None
    if inspect.ismethod(fn):
        return weakref.WeakMethod(fn)
    return lambda: fn


class StepGraph:
    """Ping-pong state buffers and the two captured whole-step graphs of one World."""

    def __init__(self, world, hook: Hook | None = None, token: Callable[[], tuple] | None = None):
        if world.stepper.has_drone or world.stepper.any_movable:
            raise NotImplementedError(
                "whole-step graphs cover 2-D fleets without movable bodies in this build")
        self.world = world
        self._hook = _held(hook)
        self._extra_token = _held(token)
        E, A = world.n_envs, world.n_agents
        self.bufs = [world.zero_state(), world.zero_state()]
        self.act = torch.zeros(E, A, world.act_dim, device=world.device, dtype=world.dtype)
        self.cur = 0
        self.graphs: list[torch.cuda.CUDAGraph | None] = [None, None]
        self.token: tuple | None = None
        self.captures = 0

    def _token(self) -> tuple:
        w = self.world
        d = w.stepper.desc(w.n_envs, w.act_dim)
        pe = w.stepper.params_per_env
        # every device address the captured kernels bake in: the descriptor, the shared
        # parameter rows and the per-env table (a re-randomization may reallocate it)
        base = (w.stepper.mutation_version, ctypes.addressof(d), w.stepper.params.floats.data_ptr(),
                pe.data_ptr() if pe is not None else 0)
        extra = self._extra_token()
        return base + (extra() if extra is not None else ())

    def adopt_state(self) -> None:
        """Make ``world.state`` the current persistent set (copying a replaced state in)."""
        w = self.world
        b = self.bufs[self.cur]
        s = w.state
        if s is b:
            return
        with torch.no_grad():
            for name in FIELDS[:5]:
                getattr(b, name).copy_(getattr(s, name).detach())
        w.state = b

    def _launch_step(self, src: TorchState, dst: TorchState, stream: int) -> None:
        w = self.world
        lib = _lib.load()
        desc = w.stepper.desc(w.n_envs, w.act_dim)
        EA, dt = w.n_envs * w.n_agents, w.stepper.dtype
        check_extent(self.act, EA * w.act_dim, "actions", dt)
        s_in = state_struct(list(src)[:5], EA, dt, "state")
        s_out = state_struct(list(dst)[:5], EA, dt, "next state")
        _lib.check(lib.swarp_rollout_fwd(ctypes.byref(desc), 1, ctypes.byref(s_in),
                                         self.act.data_ptr(), None, ctypes.byref(s_out),
                                         ctypes.c_void_p(stream)))

    def _capture(self, k: int) -> torch.cuda.CUDAGraph:
        src, dst = self.bufs[k], self.bufs[1 - k]
        # eager warm-up of the same launches (first-launch set-up stays out of the
        # capture); the hook's warm launch leaves carried state (the baseline) alone,
        # and the replay below overwrites everything it wrote
        hook = self._hook()
        stream = _lib.stream_of(self.act.device)
        self._launch_step(src, dst, stream)
        if hook is not None:
            hook(dst, stream, True)
        torch.cuda.current_stream(self.act.device).synchronize()
        g = torch.cuda.CUDAGraph()
        collecting = gc.isenabled()
        gc.disable()  # no collection (and no graph destructor) inside the capture
        try:
            with torch.cuda.graph(g):
                cap = _lib.stream_of(self.act.device)
                self._launch_step(src, dst, cap)
                if hook is not None:
                    hook(dst, cap, False)
        finally:
            if collecting:
                gc.enable()
        self.captures += 1
        return g

    def step(self, actions: torch.Tensor) -> None:
        """One whole step: actions in, graph replay, state flip."""
        tok = self._token()
        if tok != self.token:
            self.graphs = [None, None]
            self.token = tok
        self.adopt_state()
        self.act.copy_(actions)
        k = self.cur
        if self.graphs[k] is None:
            self.graphs[k] = self._capture(k)
        self.graphs[k].replay()
        self.cur = 1 - k
        w = self.world
        w.state = self.bufs[self.cur]
        w.lists_built_on(w.state.pos)
