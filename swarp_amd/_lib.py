"""ctypes binding of libswarp_hip.so (the C ABI declared in include/swarp_hip.h).

The library is built in-tree (``python -m swarp_amd.build``) and loaded from this
package directory.  There is no fallback: if the library is missing or was built
for another ABI, every step raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

ABI_VERSION = 16
F32, F64 = 0, 1
EULER, RK4 = 0, 1
LISTS_BRUTE, LISTS_GRID = 0, 1
WIDE_MAX_AGENTS = 4096

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("SWARP_HIP_LIB", _PKG / "libswarp_hip.so"))


class SwarpDesc(ctypes.Structure):
    """Mirror of ``swarp_desc_t``."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("n_envs", ctypes.c_int32),
        ("n_agents", ctypes.c_int32),
        ("act_dim", ctypes.c_int32),
        ("substeps", ctypes.c_int32),
        ("max_neighbors", ctypes.c_int32),
        ("n_obstacles", ctypes.c_int32),
        ("collisions", ctypes.c_int32),
        ("soft_walls", ctypes.c_int32),
        ("clamp_bounds", ctypes.c_int32),
        ("has_drone", ctypes.c_int32),
        ("holo_velocity_only", ctypes.c_int32),
        ("dt", ctypes.c_double),
        ("k", ctypes.c_double),
        ("c", ctypes.c_double),
        ("margin", ctypes.c_double),
        ("max_overlap", ctypes.c_double),
        ("neighbor_radius", ctypes.c_double),
        ("bounds_min", ctypes.c_double * 2),
        ("bounds_max", ctypes.c_double * 2),
        ("params", ctypes.c_void_p),
        ("model_tag", ctypes.c_void_p),
        ("ctrl_mode", ctypes.c_void_p),
        ("obs_pos", ctypes.c_void_p),
        ("obs_radius", ctypes.c_void_p),
        ("obs_angle", ctypes.c_void_p),
        ("obs_half", ctypes.c_void_p),
        ("obs_vel", ctypes.c_void_p),
        ("obs_ang_vel", ctypes.c_void_p),
        ("obs_type", ctypes.c_void_p),
        ("obs_kind", ctypes.c_void_p),
        ("obs_body", ctypes.c_void_p),
        ("obs_mass", ctypes.c_void_p),
        ("obs_inertia", ctypes.c_void_p),
        ("obs_body_off", ctypes.c_void_p),
        ("lin_damping", ctypes.c_double),
        ("ang_damping", ctypes.c_double),
        ("integrator", ctypes.c_int32),
        ("has_boxes", ctypes.c_int32),
        ("wheel_contacts", ctypes.c_int32),
        ("lat_grip", ctypes.c_double),
        ("turn_cap", ctypes.c_double),
        ("params_per_env", ctypes.c_int32),
        ("skin_speed", ctypes.c_double),
        ("fleet_models", ctypes.c_int32),
        ("fleet_modes", ctypes.c_int32),
        ("neighbor_method", ctypes.c_int32),
        ("grid_bins", ctypes.c_int32),
        ("grid_pinned", ctypes.c_int32),
        ("grid_origin", ctypes.c_double * 2),
        ("grid_cell", ctypes.c_double),
        ("grid_frame", ctypes.c_void_p),
        ("body_params", ctypes.c_void_p),
        ("obstacle_types", ctypes.c_int32),
    ]


class SwarpState(ctypes.Structure):
    """Mirror of ``swarp_state_t`` (nine nullable field pointers)."""

    _fields_ = [
        (name, ctypes.c_void_p)
        for name in ("pos", "theta", "vel", "speed", "ang_vel", "z", "vz", "attitude", "body_rates")
    ]


class SwarpNav(ctypes.Structure):
    """Mirror of ``swarp_nav_t`` (the navigation pass's buffers and constants)."""

    _fields_ = [
        ("pos", ctypes.c_void_p), ("vel", ctypes.c_void_p), ("theta", ctypes.c_void_p),
        ("ang_vel", ctypes.c_void_p), ("goals", ctypes.c_void_p),
        ("reset_mask", ctypes.c_void_p), ("prev_dist", ctypes.c_void_p),
        ("nbr_idx", ctypes.c_void_p), ("nbr_cnt", ctypes.c_void_p), ("nbr_true", ctypes.c_void_p),
        ("obs", ctypes.c_void_p), ("touching", ctypes.c_void_p), ("dist", ctypes.c_void_p),
        ("shaping", ctypes.c_void_p), ("on_goal", ctypes.c_void_p),
        ("overflow", ctypes.c_void_p), ("reward", ctypes.c_void_p), ("done", ctypes.c_void_p),
        ("k_obs", ctypes.c_int32), ("advance_prev", ctypes.c_int32),
        ("full_pass", ctypes.c_int32), ("shared_reward", ctypes.c_int32),
        ("pos_shaping_factor", ctypes.c_double), ("goal_tolerance", ctypes.c_double),
        ("collision_penalty", ctypes.c_double), ("final_reward", ctypes.c_double),
        ("step_count", ctypes.c_void_p), ("truncated", ctypes.c_void_p),
        ("max_steps", ctypes.c_int32),
        ("radius", ctypes.c_void_p),
    ]


#: Exported entry points and their ctypes signatures.
SIGNATURES = {
    "swarp_abi_version": ([], ctypes.c_int),
    "swarp_last_error": ([], ctypes.c_char_p),
    "swarp_rollout_fwd": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState), ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_rollout_bwd": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState),
         ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_tape_bytes": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)],
        ctypes.c_int,
    ),
    "swarp_rollout_fwd_tape": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.c_uint64,
         ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_rollout_bwd_tape": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState),
         ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
         ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_rollout_fwd_ob": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_rollout_bwd_ob": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.POINTER(SwarpState),
         ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_rollout_bwd_ob_check": ([ctypes.POINTER(SwarpDesc)], ctypes.c_int),
    "swarp_ob_tape_bytes": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)],
        ctypes.c_int,
    ),
    "swarp_rollout_fwd_ob_tape": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.POINTER(SwarpState), ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_rollout_bwd_ob_tape": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_int32, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.POINTER(SwarpState),
         ctypes.POINTER(SwarpState), ctypes.c_void_p, ctypes.POINTER(SwarpState), ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_neighbors": (
        [ctypes.POINTER(SwarpDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_nav_obs": (
        [ctypes.POINTER(SwarpDesc), ctypes.POINTER(SwarpNav), ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_edge_index": (
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_edge_index_noalloc": (
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "swarp_state_defaults": (
        [ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p],
        ctypes.c_int,
    ),
}

_lib = None


class SwarpLibraryError(RuntimeError):
    """The HIP library is missing, stale, or rejected a call."""


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise SwarpLibraryError(
            f"{LIB_PATH} is missing: build it with `python -m swarp_amd.build` "
            "(hipcc, gfx950). swarp_amd has no CPU fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    ver = lib.swarp_abi_version()
    if ver != ABI_VERSION:
        raise SwarpLibraryError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}: rebuild it")
    _lib = lib
    return lib


def stream_of(device: torch.device) -> int:
    """Raw handle of torch's current stream on ``device`` (the stream every launch of
    this package goes to; inside a graph capture it is the capture stream)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def check(rc: int) -> None:
    """Raise the library's own message when a call returned non-zero."""
    if rc != 0:
        msg = load().swarp_last_error().decode(errors="replace")
        raise SwarpLibraryError(f"libswarp_hip: {msg}")
