"""``Environment`` and ``make``: the vectorised multi-agent environment over a Scenario
(``swarp/core/environment.py:17-749``, ``swarp/__init__.py:95-121``).

``step`` advances the world through the HIP step and returns the Gymnasium 5-tuple
``(obs, reward, terminated, truncated, info)``.  Three paths, chosen per step as the
reference chooses them (``swarp/core/environment.py:155-182, 395-421``):
* a differentiated step (grad mode on and something requires grad): the functional
  step with its hand-written adjoint, observations and rewards through torch autograd;
* an untaped step with ``fused``: the step, then the scenario's fused HIP pass;
* an untaped step with ``use_graph=True``: the step and the fused pass (which also
  advances the step counter) replayed as one HIP graph (``swarp_amd.persistent.StepGraph``).
  ``"auto"`` leaves the graph off: on MI355X a replay of the two-node graph costs more
  host time than the two eager launches it replaces (measured with the reference's
  throughput grid, ``swarp_amd.throughput``), unlike the many-launch step the reference
  captures on CUDA.
``auto_reset=True`` resets finished envs in place with a masked, host-sync-free reset,
run eagerly after the step (the reference folds it into its graph for scenarios whose
reset kernels are capturable; here the reset's sampler is torch on the world generator).
"""

from __future__ import annotations

import inspect
import warnings
from typing import Any

import torch

from .config import WorldConfig, action_bounds
from .persistent import StepGraph
from .scenarios import SCENARIOS, Scenario, make_scenario


class Environment:
    """Vectorised environment: all tensors stay on ``device``."""

    def __init__(
        self,
        scenario: Scenario,
        n_envs: int,
        device: str = "cuda:0",
        dt: float = 0.1,
        substeps: int = 1,
        dtype: torch.dtype = torch.float32,
        max_steps: int | None = None,
        seed: int = 0,
        auto_reset: bool = False,
        use_graph: bool | str = "auto",
        clone_outputs: bool = False,
        fused: bool | str = "auto",
        world_config: WorldConfig | None = None,
    ) -> None:
        if n_envs < 1:
            raise ValueError(f"n_envs must be >= 1, got {n_envs}")
        self.scenario = scenario
        self.n_envs = n_envs
        self.device = str(device)
        if self.device.startswith("cuda") and not torch.cuda.is_available():
            raise RuntimeError(
                f"device {self.device!r} requested but no HIP device is visible; pass "
                "device='cpu' to build and reset on the host (stepping needs the GPU)"
            )
        self.dtype = dtype
        self.max_steps = max_steps
        self.auto_reset = auto_reset
        self.clone_outputs = clone_outputs
        self.world = scenario.make_world(n_envs=n_envs, device=self.device, dt=dt,
                                         substeps=substeps, dtype=dtype,
                                         world_config=world_config)
        self.n_agents = self.world.n_agents
        # the scenario's fused no-grad obs/reward pass (environment.py:155)
        self._fused = scenario.fused_available if fused == "auto" else bool(fused)
        self._seed(seed)
        self._step_count = torch.zeros(n_envs, device=self.device, dtype=torch.int32)
        self._never_truncated = torch.zeros(n_envs, device=self.device, dtype=torch.bool)
        self._truncated_buf = torch.zeros(n_envs, device=self.device, dtype=torch.bool)
        self._episode_end_buf = torch.zeros(n_envs, device=self.device, dtype=torch.bool)
        # whole-step graph (environment.py:166-170); "auto" keeps it off: the eager step is
        # two launches, which replay no faster as a graph on this platform
        st = self.world.stepper
        coverable = (self._fused and self.device.startswith("cuda") and not st.has_drone
                     and not st.any_movable)
        want = False if use_graph == "auto" else bool(use_graph)
        if want and not coverable:
            warnings.warn("use_graph=True: this world cannot be captured (needs the fused "
                          "pass on a HIP device, 2-D agents, no movable bodies); stepping "
                          "eagerly", RuntimeWarning, stacklevel=2)
            want = False
        self._graph = StepGraph(self.world, hook=self._graph_hook,
                                token=self._graph_token) if want else None
        if self._fused and hasattr(scenario, "attach_counter"):
            # the fused step pass advances the step counter and writes the time limit
            scenario.attach_counter(self._step_count, self._truncated_buf, self.max_steps)

    # ------------------------------------------------------------------ seeding

    def seed(self, seed: int) -> None:
        """Reseed the world RNG without touching episode state."""
        self._seed(seed)

    def _seed(self, seed: int) -> None:
        self.world.generator = torch.Generator(device=self.device)
        self.world.generator.manual_seed(seed)

    # --------------------------------------------------------------- properties

    @property
    def step_count(self) -> torch.Tensor:
        """Steps since each env's last reset, ``[n_envs]`` int32 (live buffer)."""
        return self._step_count

    @property
    def graph_mode(self) -> bool:
        """Whether untaped steps replay the whole-step graph."""
        return self._graph is not None

    def _graph_hook(self, state_out, stream: int, warm: bool) -> None:
        """Post-physics work of a graph step: the fused pass, whose step variant also
        advances the shaping baseline, the step counter and the time limit
        (``step_count_kernel``); the warm-up launch before a capture does none of those."""
        import ctypes

        from . import _lib

        sc = self.scenario
        nav = sc.fused_nav(state_out, advance_prev=0 if warm else 1, full_pass=1, reset_mask=None)
        desc = self.world.stepper.desc(self.n_envs, self.world.act_dim)
        _lib.check(_lib.load().swarp_nav_obs(ctypes.byref(desc), ctypes.byref(nav),
                                             ctypes.c_void_p(stream)))

    def _graph_token(self) -> tuple:
        """Pointers the captured pass bakes in besides the step's (recapture on a move)."""
        sc, w = self.scenario, self.world
        fb = sc.ensure_fused()
        grid = w.stepper.grid(self.n_envs)
        return (w.goals.data_ptr(), sc._prev_dist.data_ptr(), fb["obs"].data_ptr(),
                grid.neighbor_idx.data_ptr(), sc._k_obs)

    @property
    def obs_dim(self) -> int:
        return self.scenario.obs_dim

    @property
    def act_dim(self) -> int:
        return self.world.act_dim

    @property
    def state_dim(self) -> int:
        return self.scenario.state_dim

    @property
    def n_roles(self) -> int:
        return self.scenario.n_roles

    @property
    def role_counts(self) -> tuple[int, ...]:
        return tuple(self.scenario.role_counts)

    @property
    def aux_dim(self) -> int:
        return self.scenario.aux_dim

    def critic_state(self) -> torch.Tensor | None:
        return self.scenario.critic_state()

    def agent_roles(self) -> torch.Tensor | None:
        return self.scenario.agent_roles()

    def aux_targets(self) -> torch.Tensor | None:
        return self.scenario.aux_targets()

    def comm_mask(self) -> torch.Tensor | None:
        return self.scenario.comm_mask()

    @property
    def action_bounds(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``(low, high)``, each ``[n_agents, act_dim]``: the box the dynamics clamp
        against; slots past an agent's model arity are ``[0, 0]``."""
        na, ad = self.n_agents, self.world.act_dim
        low = torch.zeros(na, ad, device=self.device, dtype=self.dtype)
        high = torch.zeros_like(low)
        for i, cfg in enumerate(self.world.agent_configs):
            lo, hi = action_bounds(cfg)
            low[i, : len(lo)] = torch.tensor(lo, device=self.device, dtype=self.dtype)
            high[i, : len(hi)] = torch.tensor(hi, device=self.device, dtype=self.dtype)
        return low, high

    # ------------------------------------------------------------ path choice

    def _taped_step(self, actions: torch.Tensor | None = None) -> bool:
        """Whether the coming step is differentiated: grad mode on and something
        requires grad (``swarp/core/environment.py:403-417``)."""
        if not torch.is_grad_enabled():
            return False
        if actions is not None and actions.requires_grad:
            return True
        return any(t is not None and t.requires_grad for t in self.world.state)

    def _set_fused_active(self, actions: torch.Tensor | None = None) -> None:
        """The fused pass serves untaped steps; a differentiated step takes torch."""
        self.scenario.set_fused_active(self._fused and not self._taped_step(actions))

    # ------------------------------------------------------------------ episodes

    def reset(self, seed: int | None = None) -> torch.Tensor:
        """Reset every env; returns observations ``[n_envs, n_agents, obs_dim]``."""
        if seed is not None:
            self._seed(seed)
        self.world.action = None
        self._set_fused_active()
        with torch.no_grad():
            self.world.reset_state()
            self.scenario.reset_world(None)
        self._step_count.zero_()
        return self.scenario.observations()

    def reset_at(self, env_mask: torch.Tensor) -> torch.Tensor:
        """Reset the envs where ``env_mask`` (bool ``[n_envs]``) is True."""
        self._set_fused_active()
        with torch.no_grad():
            self.scenario.reset_world(env_mask)
        self._step_count.masked_fill_(env_mask, 0)
        return self.scenario.observations()

    def step(
        self, actions: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, dict[str, Any]]:
        """Advance every env one step; ``actions [n_envs, n_agents, act_dim]``.

        Returns ``(obs, reward [n_envs, n_agents], terminated [n_envs] bool, truncated
        [n_envs] bool, info)``.  ``terminated`` is the scenario's own terminal condition,
        ``truncated`` the ``max_steps`` limit (a persistent buffer written in place)."""
        act_dim = self.world.act_dim
        if actions.shape != (self.n_envs, self.n_agents, act_dim):
            raise ValueError(
                f"actions must have shape {(self.n_envs, self.n_agents, act_dim)}, "
                f"got {tuple(actions.shape)}"
            )
        if actions.dtype != self.dtype:
            raise TypeError(f"actions dtype {actions.dtype} != env dtype {self.dtype}")
        self._set_fused_active(actions)
        self.world.action = actions
        sc = self.scenario
        counted = getattr(sc, "counts_steps", False)
        if self._graph is not None and sc.fused_active:
            # step + fused pass (incl. step counter / time limit): one replay
            self._graph.step(actions)
            sc._fresh = "fused"
        else:
            self.world.step(actions)
            sc.post_step()
            if not counted:
                self._step_count += 1
        reward = sc.rewards()
        terminated = sc.done()
        if self.max_steps is not None:
            truncated = (self._truncated_buf if counted else
                         torch.ge(self._step_count, self.max_steps, out=self._truncated_buf))
        else:
            truncated = self._never_truncated
        info = self.scenario.info()
        if self.auto_reset:
            end = torch.logical_or(terminated, truncated, out=self._episode_end_buf)
            with torch.no_grad():
                self.scenario.reset_world(end, obs_only=True)
            self._step_count.masked_fill_(end, 0)
        obs = self.scenario.observations()
        if self.clone_outputs:
            obs, reward = obs.clone(), reward.clone()
            terminated, truncated = terminated.clone(), truncated.clone()
            info = {k: v.clone() if torch.is_tensor(v) else v for k, v in info.items()}
        return obs, reward, terminated, truncated, info

    def radius_graph(self) -> torch.Tensor:
        """COO ``[2, n_edges]`` of the current radius graph, from the lists the step or
        reset already built (one host sync for the edge count)."""
        return self.world.edge_index(rebuild=False)


#: Keywords ``make`` forwards to ``Environment``; the rest go to the scenario.
_ENV_KWARGS = frozenset(inspect.signature(Environment.__init__).parameters) - {
    "self", "scenario", "n_envs"}


def make(name: str, n_envs: int, **kwargs) -> Environment:
    """Build an ``Environment`` for a registered scenario (``swarp/__init__.py:95-121``):
    keywords ``Environment`` accepts go to it, every other keyword to the scenario; an
    unknown scenario name raises ``ValueError``, a keyword neither takes ``TypeError``."""
    env_kwargs = {k: v for k, v in kwargs.items() if k in _ENV_KWARGS}
    scen_kwargs = {k: v for k, v in kwargs.items() if k not in _ENV_KWARGS}
    if name in SCENARIOS:
        params = inspect.signature(SCENARIOS[name].__init__).parameters
        bad = sorted(k for k in scen_kwargs if k not in params)
        if bad:
            raise TypeError(
                f"make({name!r}): unexpected keyword(s) {bad}; the scenario takes "
                f"{sorted(p for p in params if p != 'self')} and Environment takes "
                f"{sorted(_ENV_KWARGS)}"
            )
    scenario = make_scenario(name, **scen_kwargs)
    return Environment(scenario, n_envs=n_envs, **env_kwargs)
