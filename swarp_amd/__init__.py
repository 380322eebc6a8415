"""swarp_amd -- swarp's differentiable physics step, native to AMD MI355X (gfx950).

The step (neighbour search, soft contacts, integration of holonomic / diff-drive /
bicycle / quadrotor agents) and its adjoint run as hand-written HIP kernels in
``libswarp_hip.so`` behind a C ABI (``include/swarp_hip.h``); this package is the
PyTorch-facing host side with the reference's API (``Stepper``, ``TorchState``,
``warp_step``, ``rollout``, ``GradRing``, ``NeighborGrid``, the config classes, and the
``World`` / ``Environment`` / ``make("navigation", ...)`` surface that calls the step).
"""

from .autograd import GradRing, StepGradSlot, TorchState, fill_state_defaults, rollout, warp_step
from .config import (
    MODEL_ACTION_DIM,
    NUM_PARAMS,
    PARAM_FIELDS,
    AgentConfig,
    AgentShape,
    ControlMode,
    DynamicsModel,
    Integrator,
    ObstacleKind,
    Obstacles,
    ObstacleShape,
    WorldConfig,
    action_bounds,
    action_dim,
    drone_config,
    per_env_float_template,
)
from .environment import Environment, make
from .neighbors import NeighborGrid
from .scenarios import SCENARIOS, NavigationScenario, Scenario, make_scenario
from .stepper import AgentParams, Stepper, build_agent_params
from .world import World

__all__ = [
    "AgentConfig", "AgentParams", "AgentShape", "ControlMode", "DynamicsModel", "Environment",
    "GradRing", "Integrator", "MODEL_ACTION_DIM", "NUM_PARAMS", "NavigationScenario",
    "NeighborGrid", "ObstacleKind", "per_env_float_template", "ObstacleShape", "Obstacles", "PARAM_FIELDS", "SCENARIOS",
    "Scenario", "StepGradSlot", "Stepper", "TorchState", "World", "WorldConfig",
    "action_bounds", "action_dim", "build_agent_params", "drone_config", "fill_state_defaults",
    "make", "make_scenario", "rollout", "warp_step",
]
