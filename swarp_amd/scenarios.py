"""Scenarios that build a ``World`` for ``Environment``: the ``Scenario`` interface
(``swarp/scenarios/base.py:29-228``) and ``NavigationScenario``
(``swarp/scenarios/navigation.py:38-839``), the step's caller in every benchmark of the
reference.

Observations and rewards have two paths, as in the reference:
* torch ops on the step's outputs -- the reference's own differentiable path
  (``_refresh_step_cache`` / ``observations`` / ``rewards``,
  ``swarp/scenarios/navigation.py:671-839``), taken when the step is differentiated;
* the fused no-grad pass: one HIP launch (``swarp_nav_obs``) builds the lists and writes
  the observation, reward, done and info buffers in place -- the counterpart of the
  reference's fused Warp kernels (``swarp/scenarios/navigation.py:508-650``,
  ``navigation_kernels.py``).  ``Environment`` switches it on for untaped steps.
Resets draw spawns and goals with the stratified separated sampler the reference keeps
as its torch reference (``_sample_separated``, ``:222-272``) on the world's generator,
so they are reproducible per seed but are not the reference's Warp RNG stream.
"""

from __future__ import annotations

import math
from abc import ABC, abstractmethod
from typing import Any

import ctypes

import torch

from . import _lib
from .config import AgentConfig, AgentShape, ControlMode, DynamicsModel, Obstacles, WorldConfig
from .config import _coerce
from .world import World


class Scenario(ABC):
    """A task on top of a World: ``make_world``, ``reset_world``, ``observations``,
    ``rewards``, ``done``, ``info`` and the ``post_step`` hook."""

    world: World

    @property
    @abstractmethod
    def obs_dim(self) -> int:
        """Per-agent observation width."""

    @property
    def state_dim(self) -> int:
        return 0

    @property
    def n_roles(self) -> int:
        return 1

    @property
    def role_counts(self) -> tuple[int, ...]:
        return ()

    @property
    def aux_dim(self) -> int:
        return 0

    def critic_state(self) -> torch.Tensor | None:
        return None

    def agent_roles(self) -> torch.Tensor | None:
        return None

    def aux_targets(self) -> torch.Tensor | None:
        return None

    def comm_mask(self) -> torch.Tensor | None:
        return None

    @abstractmethod
    def make_world(self, n_envs: int, device: str, dt: float, substeps: int,
                   dtype: torch.dtype, world_config: WorldConfig | None = None) -> World:
        """Build the World; the scenario's own WorldConfig ends with
        ``.override_with(world_config)``."""

    @abstractmethod
    def reset_world(self, env_mask: torch.Tensor | None = None, *, obs_only: bool = False) -> None:
        """(Re)randomise every env (``env_mask=None``) or the ``True`` envs of a bool
        ``[n_envs]`` mask, without a host sync."""

    @abstractmethod
    def observations(self) -> torch.Tensor:
        """``[n_envs, n_agents, obs_dim]``."""

    def observation(self, agent_idx: int) -> torch.Tensor:
        return self.observations()[:, agent_idx]

    def agent_reward(self, agent_idx: int) -> torch.Tensor:
        w = self.world
        return torch.zeros(w.n_envs, device=w.device, dtype=w.dtype)

    def global_reward(self) -> torch.Tensor:
        w = self.world
        return torch.zeros(w.n_envs, device=w.device, dtype=w.dtype)

    def rewards(self) -> torch.Tensor:
        per_agent = torch.stack([self.agent_reward(i) for i in range(self.world.n_agents)], 1)
        return per_agent + self.global_reward().unsqueeze(1)

    def done(self) -> torch.Tensor:
        w = self.world
        return torch.zeros(w.n_envs, device=w.device, dtype=torch.bool)

    def info(self) -> dict[str, Any]:
        return {}

    def post_step(self) -> None:  # noqa: B027 (optional hook)
        """Called right after the physics step, before observations and rewards."""

    #: whether the scenario has a fused no-grad obs/reward pass
    #: (``swarp/scenarios/base.py`` ``fused_available``)
    fused_available: bool = False
    fused_active: bool = False

    def set_fused_active(self, on: bool) -> None:
        """Route the next passes through the fused kernels (``on``) or torch.  The fused
        pass lists at most 64 agents per env in index order; wider worlds (and grid-ordered
        lists) take the torch pass over the library's lists."""
        st = getattr(getattr(self, "world", None), "stepper", None)
        wide = bool(getattr(st, "wide", False))
        self.fused_active = bool(on) and self.fused_available and not wide


class NavigationScenario(Scenario):
    """Agents navigate to per-agent goals with soft collision avoidance
    (``swarp/scenarios/navigation.py:1-11``).

    Reward per agent: position shaping ``(prev_dist - dist) * pos_shaping_factor``
    (summed over the env's agents when ``shared_reward``), ``collision_penalty`` per
    touching listed neighbour, and ``final_reward`` to every agent of an env whose agents
    are all within ``goal_tolerance`` of their goals (which also ends the episode).
    Observation per agent (``9 + 5 * neighbor_obs``): pos, vel, cos/sin heading, angular
    velocity, goal - pos, then the first ``neighbor_obs`` listed neighbours' relative
    positions, relative velocities and validity flags.
    """

    def __init__(
        self,
        n_agents: int = 4,
        agent_radius: float = 0.05,
        model: DynamicsModel = DynamicsModel.HOLONOMIC,
        ctrl_mode: ControlMode = ControlMode.VELOCITY,
        max_speed: float = 1.0,
        world_size: float = 1.0,
        n_obstacles: int = 0,
        obstacle_radius: float = 0.1,
        neighbor_obs: int = 2,
        neighbor_radius: float | None = None,
        shared_reward: bool = False,
        pos_shaping_factor: float = 1.0,
        collision_penalty: float = -1.0,
        final_reward: float = 5.0,
        goal_tolerance: float | None = None,
        min_spawn_separation: float | None = None,
        neighbor_method: str = "auto",
        agent_shape: AgentShape | str = AgentShape.DISC,
        agent_half_extents: tuple[float, float] | None = None,
    ) -> None:
        # agent_shape="box": every agent a box of agent_half_extents (default
        # (agent_radius, agent_radius / 2)); its circumscribed radius then replaces
        # agent_radius everywhere the scenario reads it (navigation.py:61-79)
        shape = _coerce(AgentShape, agent_shape, "agent_shape")
        if shape == AgentShape.BOX:
            if agent_half_extents is None:
                agent_half_extents = (agent_radius, 0.5 * agent_radius)
            footprint = AgentConfig(shape=shape, half_extents=agent_half_extents)
        else:
            footprint = AgentConfig(radius=agent_radius,
                                    half_extents=agent_half_extents or (0.0, 0.0))
        self.agent_shape = footprint.shape
        self.agent_half_extents = footprint.half_extents
        self.n_agents = n_agents
        self.agent_radius = footprint.radius
        self.model = model
        self.ctrl_mode = ctrl_mode
        self.max_speed = max_speed
        self.world_size = world_size
        self.n_obstacles = n_obstacles
        self.obstacle_radius = obstacle_radius
        self.neighbor_obs = neighbor_obs
        self.neighbor_radius = neighbor_radius
        self.shared_reward = shared_reward
        self.pos_shaping_factor = pos_shaping_factor
        self.collision_penalty = collision_penalty
        self.final_reward = final_reward
        self.goal_tolerance = goal_tolerance if goal_tolerance is not None else self.agent_radius
        self.min_spawn_separation = (min_spawn_separation if min_spawn_separation is not None
                                     else 3.0 * self.agent_radius)
        self.neighbor_method = neighbor_method
        # provisional until make_world resolves max_neighbors (navigation.py:100-103)
        self._k_obs = min(self.neighbor_obs, min(32, max(4, self.n_agents)))
        self._cache: dict[str, torch.Tensor] | None = None
        self._prev_dist: torch.Tensor | None = None
        self._fb: dict[str, torch.Tensor] | None = None   # fused-pass buffers
        self._fresh = "torch"   # which path wrote the current obs / reward
        self._navs: dict[tuple, _lib.SwarpNav] = {}      # swarp_nav_t per pointer set
        # (step_count int32 [E], truncated bool [E] or None, max_steps): the episode
        # counter the fused step pass advances (attached by Environment)
        self._counter: tuple | None = None

    # ------------------------------------------------------------------ world

    def _agent_configs(self) -> list[AgentConfig]:
        return [
            AgentConfig(model=self.model, ctrl_mode=self.ctrl_mode,
                        radius=None if self.agent_shape == AgentShape.BOX else self.agent_radius,
                        max_speed=self.max_speed, max_accel=2.0 * self.max_speed,
                        shape=self.agent_shape, half_extents=self.agent_half_extents)
            for _ in range(self.n_agents)
        ]

    def make_world(self, n_envs, device, dt, substeps, dtype, world_config=None) -> World:
        """World constants of ``swarp/scenarios/navigation.py:127-141``: k = 100, c = 1,
        margin = r / 2, soft walls at +-world_size, neighbour radius = max(user, 2r +
        margin), K = min(32, max(4, n_agents))."""
        margin = 0.5 * self.agent_radius
        reach = 2.0 * self.agent_radius + margin
        cfg = WorldConfig(
            collisions=True,
            collision_k=100.0,
            collision_c=1.0,
            collision_margin=margin,
            bounds=(-self.world_size, self.world_size, -self.world_size, self.world_size),
            bounds_mode="soft",
            neighbor_radius=max(self.neighbor_radius or 0.0, reach),
            max_neighbors=min(32, max(4, self.n_agents)),
            neighbor_method=self.neighbor_method,
        ).override_with(world_config)
        self.world = World(self._agent_configs(), cfg, n_envs=n_envs, device=device, dt=dt,
                           substeps=substeps, dtype=dtype)
        self.world.goals = torch.zeros(n_envs, self.n_agents, 2, device=device, dtype=dtype)
        self._k_obs = min(self.neighbor_obs, cfg.max_neighbors)
        self._cache = None
        self._prev_dist = None
        self._fb = None
        self._fresh = "torch"
        self._navs = {}
        if self.n_obstacles > 0:
            tt = {"device": device, "dtype": dtype}
            self.world.set_obstacles(Obstacles(
                torch.zeros(n_envs, self.n_obstacles, 2, **tt),
                torch.full((self.n_obstacles,), self.obstacle_radius, **tt),
            ))
        return self.world

    @property
    def obs_dim(self) -> int:
        return 9 + 5 * self._k_obs

    _SPAWN_CELL_OVERSAMPLE = 8

    def _sample_separated(self, n_envs: int, n_points: int, min_dist: float) -> torch.Tensor:
        """Points at least ``min_dist`` apart by construction: each env takes
        ``n_points`` distinct cells of a g x g grid over the spawn square and jitters each
        point inside its cell's centred sub-square of side ``cell - min_dist``; plain
        uniform when no grid leaves jitter room (``navigation.py:222-272``)."""
        w = self.world
        lim = self.world_size - 2.0 * self.agent_radius
        shape = (n_envs, n_points, 2)
        if n_points == 1 or min_dist <= 0.0:
            return w.sample_uniform(shape, -lim, lim)
        side = 2.0 * lim
        g = math.ceil(math.sqrt(n_points * self._SPAWN_CELL_OVERSAMPLE))
        g = min(g, int(side // (2.0 * min_dist)))
        g = max(g, math.ceil(math.sqrt(n_points)))
        if side / g <= min_dist:
            return w.sample_uniform(shape, -lim, lim)
        s = side / g
        jitter = s - min_dist
        cell = w.sample_uniform((n_envs, g * g), 0.0, 1.0).argsort(dim=-1)[:, :n_points]
        col = (cell % g).to(w.dtype)
        row = torch.div(cell, g, rounding_mode="floor").to(w.dtype)
        centers = torch.stack([col, row], dim=-1) * s + (0.5 * s - lim)
        return centers + (w.sample_uniform(shape, 0.0, 1.0) - 0.5) * jitter

    def reset_world(self, env_mask: torch.Tensor | None = None, *, obs_only: bool = False) -> None:
        """Spawns, goals, headings U[-pi, pi] and zero velocities for the selected envs
        (``navigation.py:439-473``); obstacles uniform inside the walls."""
        w = self.world
        n = w.n_envs
        pos = self._sample_separated(n, self.n_agents, self.min_spawn_separation)
        goals = self._sample_separated(n, self.n_agents, self.min_spawn_separation)
        theta = w.sample_uniform((n, self.n_agents), -math.pi, math.pi)
        w.write_state(env_mask, pos=pos, theta=theta, vel=0.0, speed=0.0, ang_vel=0.0)
        if env_mask is None:
            w.goals.copy_(goals)
        else:
            w.goals.copy_(torch.where(env_mask.view(-1, 1, 1), goals, w.goals))
        if self.n_obstacles > 0:
            lim = self.world_size - self.obstacle_radius
            opos = w.sample_uniform((n, self.n_obstacles, 2), -lim, lim)
            # in place: the stepper reads this very tensor (static circles, nothing to seed)
            if env_mask is None:
                w.obstacle_pos.copy_(opos)
            else:
                w.obstacle_pos.copy_(torch.where(env_mask.view(-1, 1, 1), opos, w.obstacle_pos))
        # a full reset rebases every env's shaping baseline
        mask = env_mask if env_mask is not None else torch.ones(n, dtype=torch.bool,
                                                                device=w.device)
        if self.fused_active:
            # an auto-reset pass leaves the returned reward / done alone (full_pass 0)
            self.launch_fused(advance_prev=0, full_pass=0 if obs_only else 1, reset_mask=mask)
        else:
            self._refresh(reset_mask=mask)

    # ------------------------------------------------------------ obs / rewards

    def post_step(self) -> None:
        if self.fused_active:
            self.launch_fused(advance_prev=1, full_pass=1)
        else:
            self._refresh()

    # ------------------------------------------------------ fused pass (HIP)

    fused_available = True

    def ensure_fused(self) -> dict[str, torch.Tensor]:
        """The fused pass's persistent buffers (``fused_spec``,
        ``swarp/scenarios/navigation.py:508-522``), allocated once per world."""
        w = self.world
        if self._fb is None:
            e, a = w.n_envs, w.n_agents
            f = {"device": w.device, "dtype": w.dtype}
            u8 = {"device": w.device, "dtype": torch.uint8}
            self._fb = {
                "obs": torch.zeros(e, a, self.obs_dim, **f),
                "touch": torch.zeros(e, a, **f), "dist": torch.zeros(e, a, **f),
                "shaping": torch.zeros(e, a, **f), "reward": torch.zeros(e, a, **f),
                "ongoal": torch.zeros(e, a, **u8), "overflow": torch.zeros(e, a, **u8),
                "done": torch.zeros(e, **u8), "resetmask": torch.zeros(e, **u8),
            }
        if self._prev_dist is None:
            self._prev_dist = torch.zeros(w.n_envs, w.n_agents, device=w.device, dtype=w.dtype)
        return self._fb

    def attach_counter(self, step_count: torch.Tensor, truncated: torch.Tensor | None,
                       max_steps: int | None) -> None:
        """Let the fused step pass advance ``step_count`` and write ``truncated``
        (``step_count >= max_steps``) in the same launch."""
        self._counter = (step_count, truncated, max_steps)
        self._navs = {}

    @property
    def counts_steps(self) -> bool:
        """Whether a fused step pass advances the attached episode counter."""
        return self.fused_active and self._counter is not None

    def fused_nav(self, state, advance_prev: int, full_pass: int, reset_mask) -> _lib.SwarpNav:
        """The ``swarp_nav_t`` of one pass over ``state`` (pointers only; no launch).
        Cached per pointer set: a step alternates between two output buffers."""
        key = (state.pos.data_ptr(), state.vel.data_ptr(), state.theta.data_ptr(),
               state.ang_vel.data_ptr(), int(advance_prev), int(full_pass),
               None if reset_mask is None else reset_mask.data_ptr())
        nav = self._navs.get(key)
        if nav is None:
            nav = self._make_nav(state, advance_prev, full_pass, reset_mask)
            if len(self._navs) > 16:
                self._navs.clear()
            self._navs[key] = nav
        return nav

    def _make_nav(self, state, advance_prev: int, full_pass: int, reset_mask) -> _lib.SwarpNav:
        w = self.world
        fb = self.ensure_fused()
        grid = w.stepper.grid(w.n_envs)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        nav = _lib.SwarpNav()
        nav.pos, nav.vel = p(state.pos), p(state.vel)
        nav.theta, nav.ang_vel = p(state.theta), p(state.ang_vel)
        nav.goals = p(w.goals)
        # the touching test uses the static radius, as the torch path and the
        # reference's navigation kernels do (navigation.py:556-557)
        nav.radius = p(w.agent_radius)
        nav.reset_mask = None if reset_mask is None else p(reset_mask)
        nav.prev_dist = p(self._prev_dist)
        nav.nbr_idx, nav.nbr_cnt = p(grid.neighbor_idx), p(grid.neighbor_count)
        nav.nbr_true = p(grid.neighbor_true_count)
        nav.obs, nav.touching, nav.dist = p(fb["obs"]), p(fb["touch"]), p(fb["dist"])
        nav.shaping, nav.reward = p(fb["shaping"]), p(fb["reward"])
        nav.on_goal, nav.overflow, nav.done = p(fb["ongoal"]), p(fb["overflow"]), p(fb["done"])
        nav.k_obs = self._k_obs
        nav.advance_prev, nav.full_pass = int(advance_prev), int(full_pass)
        nav.shared_reward = int(self.shared_reward)
        nav.pos_shaping_factor = float(self.pos_shaping_factor)
        nav.goal_tolerance = float(self.goal_tolerance)
        nav.collision_penalty = float(self.collision_penalty)
        nav.final_reward = float(self.final_reward)
        if self._counter is not None and advance_prev and full_pass:
            sc, tr, ms = self._counter
            nav.step_count = p(sc)
            nav.truncated = None if (tr is None or ms is None) else p(tr)
            nav.max_steps = 0 if ms is None else int(ms)
        return nav

    def launch_fused(self, advance_prev: int, full_pass: int,
                     reset_mask: torch.Tensor | None = None) -> None:
        """One fused pass on the current state: lists, observations, shaping and flags,
        and (``full_pass``) reward and done (``launch_fused``,
        ``swarp/scenarios/navigation.py:524-537``)."""
        w = self.world
        fb = self.ensure_fused()
        rm = None
        if reset_mask is not None:
            rm = fb["resetmask"]
            rm.copy_(reset_mask)
        st = w.state
        for t in (st.pos, st.vel, st.theta, st.ang_vel):
            if not t.is_contiguous():
                raise ValueError("world state fields must be contiguous")
        nav = self.fused_nav(st, advance_prev, full_pass, rm)
        desc = w.stepper.desc(w.n_envs, w.act_dim)
        lib = _lib.load()
        _lib.check(lib.swarp_nav_obs(ctypes.byref(desc), ctypes.byref(nav),
                                     ctypes.c_void_p(_lib.stream_of(st.pos.device))))
        w.lists_built_on(st.pos)
        self._fresh = "fused"

    def _refresh(self, reset_mask: torch.Tensor | None = None) -> None:
        """Neighbour features, goal distances and reward terms of the current state
        (``navigation.py:671-761``).  ``reset_mask`` marks envs just reset: their shaping
        baseline restarts at the spawn distance and their shaping term is zero."""
        w = self.world
        pos, vel = w.state.pos, w.state.vel
        idx, cnt = w.neighbors()
        k_all = idx.shape[-1]
        k = min(self.neighbor_obs, k_all)
        idx_long = idx.long()
        valid = torch.arange(k_all, device=w.device).view(1, 1, -1) < cnt.long().unsqueeze(-1)
        flat = idx_long.reshape(w.n_envs, -1)
        npos = torch.gather(pos, 1, flat.unsqueeze(-1).expand(-1, -1, 2))
        npos = npos.view(w.n_envs, w.n_agents, k_all, 2)
        rel_pos_all = npos - pos.unsqueeze(2)
        # touching listed pairs (|d| < r_i + r_j) per agent: a count, not differentiated
        ndist = rel_pos_all.norm(dim=-1)
        r = w.agent_radius
        touching = ((ndist < r.view(1, -1, 1) + r[idx_long]) & valid).sum(dim=-1).to(w.dtype)
        rel_pos = rel_pos_all[:, :, :k] * valid[:, :, :k].unsqueeze(-1)
        flat_k = idx_long[:, :, :k].reshape(w.n_envs, -1)
        nvel = torch.gather(vel, 1, flat_k.unsqueeze(-1).expand(-1, -1, 2))
        nvel = nvel.view(w.n_envs, w.n_agents, k, 2)
        rel_vel = (nvel - vel.unsqueeze(2)) * valid[:, :, :k].unsqueeze(-1)
        dist = (pos - w.goals).norm(dim=-1)
        if self._prev_dist is None:
            self._prev_dist = dist.detach().clone()
        shaping = (self._prev_dist - dist) * self.pos_shaping_factor
        # the baseline is one persistent buffer shared with the fused pass
        if reset_mask is None:
            self._prev_dist.copy_(dist.detach())
        else:
            m = reset_mask.unsqueeze(-1)
            shaping = torch.where(m, torch.zeros_like(shaping), shaping)
            self._prev_dist.copy_(torch.where(m, dist.detach(), self._prev_dist))
        self._cache = {
            "rel_pos": rel_pos,
            "rel_vel": rel_vel,
            "valid": valid,
            "touching": touching,
            "dist_to_goal": dist,
            "on_goal": dist < self.goal_tolerance,
            "pos_shaping": shaping,
            "neighbor_overflow": w.neighbor_overflow(),
        }
        self._fresh = "torch"

    def observations(self) -> torch.Tensor:
        if self._fresh == "fused":
            return self._fb["obs"]
        w = self.world
        s = w.state
        c = self._cache
        feats = [s.pos, s.vel, torch.cos(s.theta).unsqueeze(-1), torch.sin(s.theta).unsqueeze(-1),
                 s.ang_vel.unsqueeze(-1), w.goals - s.pos]
        k = min(self.neighbor_obs, c["rel_pos"].shape[2])
        if k > 0:
            e, a = w.n_envs, w.n_agents
            feats += [c["rel_pos"][:, :, :k].reshape(e, a, -1),
                      c["rel_vel"][:, :, :k].reshape(e, a, -1),
                      c["valid"][:, :, :k].to(w.dtype)]
        return torch.cat(feats, dim=-1)

    def rewards(self) -> torch.Tensor:
        if self._fresh == "fused":
            return self._fb["reward"]
        c = self._cache
        rew = self.collision_penalty * c["touching"]
        if self.shared_reward:
            rew = rew + c["pos_shaping"].sum(dim=-1, keepdim=True)
        else:
            rew = rew + c["pos_shaping"]
        final = self.final_reward * c["on_goal"].all(dim=-1).to(self.world.dtype)
        return rew + final.unsqueeze(-1)

    def _terms(self) -> dict[str, torch.Tensor]:
        """touching / pos_shaping / on_goal of whichever path ran last."""
        if self._fresh == "fused":
            fb = self._fb
            return {"touching": fb["touch"], "pos_shaping": fb["shaping"],
                    "on_goal": fb["ongoal"].view(torch.bool)}
        return self._cache

    def agent_reward(self, agent_idx: int) -> torch.Tensor:
        c = self._terms()
        rew = self.collision_penalty * c["touching"][:, agent_idx]
        if not self.shared_reward:
            rew = rew + c["pos_shaping"][:, agent_idx]
        return rew

    def global_reward(self) -> torch.Tensor:
        c = self._terms()
        rew = self.final_reward * c["on_goal"].all(dim=-1).to(self.world.dtype)
        if self.shared_reward:
            rew = rew + c["pos_shaping"].sum(dim=-1)
        return rew

    def done(self) -> torch.Tensor:
        if self._fresh == "fused":
            return self._fb["done"].view(torch.bool)
        return self._cache["on_goal"].all(dim=-1)

    def info(self) -> dict[str, Any]:
        if self._fresh == "fused":
            fb = self._fb
            return {"dist_to_goal": fb["dist"], "on_goal": fb["ongoal"].view(torch.bool),
                    "collisions": fb["touch"], "neighbor_overflow": fb["overflow"].view(torch.bool)}
        c = self._cache
        return {"dist_to_goal": c["dist_to_goal"], "on_goal": c["on_goal"],
                "collisions": c["touching"], "neighbor_overflow": c["neighbor_overflow"]}


#: Registered scenarios of this build (``swarp/scenarios/__init__.py`` registers twelve;
#: the physics step's caller in every benchmark is navigation).
SCENARIOS: dict[str, type[Scenario]] = {"navigation": NavigationScenario}


def make_scenario(name: str, **kwargs) -> Scenario:
    try:
        cls = SCENARIOS[name]
    except KeyError:
        raise ValueError(f"unknown scenario {name!r}; valid names: {sorted(SCENARIOS)}") from None
    return cls(**kwargs)
