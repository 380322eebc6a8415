"""swarp_amd -- swarp's differentiable physics step, native to AMD MI355X (gfx950).

The step (neighbour search, soft contacts, integration of holonomic / diff-drive /
bicycle / quadrotor agents) and its adjoint run as hand-written HIP kernels in
``libswarp_hip.so`` behind a C ABI (``include/swarp_hip.h``); this package is the
PyTorch-facing host side with the reference's API (``Stepper``, ``TorchState``,
``warp_step``, ``rollout``, ``GradRing``, ``NeighborGrid`` and the config classes).
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
)
from .neighbors import NeighborGrid
from .stepper import AgentParams, Stepper, build_agent_params

__all__ = [
    "AgentConfig", "AgentParams", "AgentShape", "ControlMode", "DynamicsModel", "GradRing",
    "Integrator", "MODEL_ACTION_DIM", "NUM_PARAMS", "NeighborGrid", "ObstacleKind",
    "ObstacleShape", "Obstacles", "PARAM_FIELDS", "StepGradSlot", "Stepper", "TorchState",
    "WorldConfig", "action_bounds", "action_dim", "build_agent_params", "drone_config",
    "fill_state_defaults", "rollout", "warp_step",
]
