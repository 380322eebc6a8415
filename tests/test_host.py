"""Host-side tests (no GPU): the C-ABI library loads and exports every function the header
declares, the ctypes struct layouts equal the C header's, and the host logic keeps the
reference's validation and error types."""

import ctypes
import math
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from swarp_amd import (AgentConfig, ControlMode, DynamicsModel, GradRing, Integrator, Obstacles,
                       Stepper, TorchState, WorldConfig, action_bounds, action_dim, drone_config,
                       rollout, warp_step)
from swarp_amd import _lib
from swarp_amd.config import PARAM_FIELDS, AgentShape

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "swarp_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(swarp_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = _declared_functions()
    assert names == sorted(_lib.SIGNATURES), names
    for n in names:
        assert hasattr(lib, n), n
    assert lib.swarp_abi_version() == _lib.ABI_VERSION
    assert lib.swarp_last_error() == b""


def test_state_defaults_rejects_bad_arguments_without_gpu():
    """swarp_state_defaults checks its arguments on the host; n = 0 launches nothing."""
    lib = _lib.load()
    assert lib.swarp_state_defaults(2, 4, None, None) != 0
    assert b"dtype" in lib.swarp_last_error()
    assert lib.swarp_state_defaults(0, -1, None, None) != 0
    assert lib.swarp_state_defaults(0, 4, None, None) != 0
    assert b"buf" in lib.swarp_last_error()
    assert lib.swarp_state_defaults(0, 4, 8, None) != 0  # misaligned: rejected before launch
    assert b"aligned" in lib.swarp_last_error()
    assert lib.swarp_state_defaults(1, 0, None, None) == 0
    assert lib.swarp_last_error() == b""


def test_struct_layout_matches_header(tmp_path):
    prog = tmp_path / "layout.c"
    desc_fields = [f for f, _ in _lib.SwarpDesc._fields_]
    state_fields = [f for f, _ in _lib.SwarpState._fields_]
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){",
             'printf("%zu\\n", sizeof(swarp_desc_t));', 'printf("%zu\\n", sizeof(swarp_state_t));']
    lines += [f'printf("%zu\\n", offsetof(swarp_desc_t, {f}));' for f in desc_fields]
    lines += [f'printf("%zu\\n", offsetof(swarp_state_t, {f}));' for f in state_fields]
    lines.append("return 0;}")
    prog.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", str(prog), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(_lib.SwarpDesc), ctypes.sizeof(_lib.SwarpState)]
    want += [getattr(_lib.SwarpDesc, f).offset for f in desc_fields]
    want += [getattr(_lib.SwarpState, f).offset for f in state_fields]
    assert got == want


def test_library_rejects_bad_descriptor_without_gpu():
    """Argument checks run on the host before any launch and report through the error
    channel (no device call is made for a rejected descriptor)."""
    lib = _lib.load()
    d = _lib.SwarpDesc()
    d.abi_version = 999
    s = _lib.SwarpState()
    rc = lib.swarp_rollout_fwd(ctypes.byref(d), 1, ctypes.byref(s), None, None, ctypes.byref(s), None)
    assert rc != 0 and b"abi_version" in lib.swarp_last_error()
    d.abi_version = _lib.ABI_VERSION
    d.dtype = 0
    d.n_envs, d.n_agents, d.act_dim, d.substeps = 1, 4097, 2, 1
    rc = lib.swarp_rollout_fwd(ctypes.byref(d), 1, ctypes.byref(s), None, None, ctypes.byref(s), None)
    assert rc != 0 and b"n_agents" in lib.swarp_last_error()
    # per-env agent rows with moving bodies need the shared table for the body pass
    from swarp_amd import per_env_float_template
    cfgs = [AgentConfig(radius=0.05)]
    st = Stepper(cfgs, device="cpu", world=WorldConfig(neighbor_radius=0.3))
    st.set_obstacles(Obstacles(pos=torch.zeros(1, 1, 2), radius=torch.ones(1),
                               kind=torch.ones(1, dtype=torch.int32)))
    st.set_agent_params_per_env(per_env_float_template(cfgs, 1))
    d = st.desc(1, 2)
    d.body_params = None
    rc = lib.swarp_rollout_fwd_ob(ctypes.byref(d), 1, ctypes.byref(s), None, None, None,
                                  ctypes.byref(s), None, None)
    assert rc != 0
    rc = lib.swarp_rollout_fwd_ob(ctypes.byref(d), 1, ctypes.byref(s), 1, 1, None,
                                  ctypes.byref(s), 1, None)
    assert rc != 0 and b"body_params" in lib.swarp_last_error()


def test_tape_size_without_gpu():
    """Rollout tape size (a host computation): one record per step and lane of every
    workgroup (64 / PA envs each, PA = agents padded to a power of two) -- 4 mask words
    (4 B up to 16 agents, 8 B up to 32, 16 B up to 64; the wall bits ride in the agent's
    own bits), 3 velocity pairs, padded to 16 B -- then the last step's velocities, each
    region 256-byte aligned.
    No tape where the backward recomputes (generic kernels, more than 4 substeps, nothing
    to record)."""
    from cases import nav_agents, nav_world

    def al(x):
        return (x + 255) // 256 * 256

    def stepper(A, S, dtype=torch.float32, **kw):
        return Stepper(nav_agents(A), dt=0.05, substeps=S, device="cpu", dtype=dtype,
                       world=nav_world(A, **kw))

    E, T = 1000, 32
    for A, PA, S, dtype, rec, pair in ((16, 16, 4, torch.float32, 48, 8),    # 16 + 24 -> 48
                                       (8, 8, 1, torch.float32, 48, 8),
                                       (20, 32, 4, torch.float64, 80, 16),   # 32 + 48 -> 80
                                       (40, 64, 2, torch.float32, 96, 8),    # 64 + 24 -> 96
                                       (64, 64, 3, torch.float64, 112, 16)):  # 64 + 48 -> 112
        lanes = -(-E // (64 // PA)) * 64
        assert stepper(A, S, dtype).tape_bytes(E, 2, T) == al(T * lanes * rec) + al(lanes * pair), (A, S)
    # contacts without walls keep the same records; 10 envs of 8 agents fill 2 workgroups
    st = Stepper(nav_agents(8), dt=0.05, substeps=2, device="cpu", dtype=torch.float32,
                 world=WorldConfig(collisions=True, collision_margin=0.025))
    assert st.tape_bytes(10, 2, 3) == al(3 * 128 * 48) + al(128 * 8)
    assert stepper(16, 5).tape_bytes(E, 2, T) == 0
    st = stepper(16, 4)
    st.use_tape = False
    assert st.tape_bytes(E, 2, T) == 0
    dd = Stepper(nav_agents(4, model=DynamicsModel.DIFF_DRIVE), dt=0.05, device="cpu",
                 world=nav_world(4))
    # the generic kernels' tape: per substep and agent the force pair and the 4-byte
    # neighbour mask, each part rounded up to 256 bytes
    n_ = T * dd.substeps * E * 4
    assert dd.tape_bytes(E, 2, T) == al(al(8 * n_) + 4 * n_)
    free = Stepper(nav_agents(4), dt=0.05, device="cpu", world=WorldConfig(collisions=False))
    assert free.tape_bytes(E, 2, T) == 0
    lib = _lib.load()
    n = ctypes.c_uint64(7)
    assert lib.swarp_tape_bytes(ctypes.byref(st.desc(E, 2)), 0, ctypes.byref(n)) != 0


# ------------------------------------------------------------------ config surface

def test_param_fields_layout():
    # column order of swarp/dynamics/base.py:114-145
    assert PARAM_FIELDS == (
        "radius", "mass", "max_speed", "max_accel", "max_ang_vel", "max_ang_accel", "l_f", "l_r",
        "max_steer", "thrust_max", "arm_length", "inertia_xx", "inertia_yy", "inertia_zz",
        "torque_coeff", "gravity", "min_speed", "shape", "half_x", "half_y", "cmd_gain_v",
        "cmd_gain_w")
    row = AgentConfig(max_speed=2.0).to_row()
    assert row[PARAM_FIELDS.index("min_speed")] == -2.0
    assert row[0] == 0.05 and len(row) == 22


def test_agent_config_validation_and_coercion():
    assert AgentConfig(model="diff-drive").model == DynamicsModel.DIFF_DRIVE
    assert AgentConfig(model="drone").model == DynamicsModel.DRONE
    with pytest.raises(ValueError, match="unknown model"):
        AgentConfig(model="tank")
    with pytest.raises(ValueError, match="SERVO"):
        AgentConfig(model=DynamicsModel.HOLONOMIC, ctrl_mode=ControlMode.SERVO)
    with pytest.raises(ValueError, match="positive"):
        AgentConfig(mass=0.0)
    box = AgentConfig(shape=AgentShape.BOX, half_extents=(0.3, 0.4))
    assert math.isclose(box.radius, 0.5)
    assert action_dim("drone") == 4 and action_dim(DynamicsModel.HOLONOMIC) == 2
    lo, hi = action_bounds(AgentConfig(model="diff_drive", max_speed=2.0, max_ang_vel=1.5))
    assert lo == [-2.0, -1.5] and hi == [2.0, 1.5]
    assert drone_config().radius == 0.15


def test_world_config_validation_and_override():
    with pytest.raises(ValueError):
        WorldConfig(bounds_mode="sticky")
    with pytest.raises(ValueError):
        WorldConfig(bounds=(1.0, -1.0, 0.0, 1.0))
    with pytest.raises(ValueError):
        WorldConfig(collision_k=-1.0)
    base = WorldConfig(collision_k=100.0, bounds=(-2.0, 2.0, -2.0, 2.0), max_neighbors=16)
    merged = base.override_with(WorldConfig(collision_c=3.0))
    assert merged.collision_c == 3.0 and merged.bounds == (-2.0, 2.0, -2.0, 2.0)
    assert base.override_with(None) is base


def test_stepper_reach_check_and_unsupported_features():
    cfgs = [AgentConfig(radius=0.2) for _ in range(2)]
    with pytest.raises(ValueError, match="neighbor_radius"):
        Stepper(cfgs, device="cpu", world=WorldConfig(neighbor_radius=0.1))
    with pytest.raises(ValueError, match="substeps"):
        Stepper(cfgs, substeps=0, device="cpu")
    rk = Stepper(cfgs, device="cpu", world=WorldConfig(integrator=Integrator.RK4))
    assert rk.desc(2, 2).integrator == 1 and Stepper(cfgs, device="cpu").desc(2, 2).integrator == 0
    # box agents: the box-aware pass and, under bounds_mode="clamp", the footprint clamp
    bx = Stepper([AgentConfig(shape="box", half_extents=(0.1, 0.1)), AgentConfig(radius=0.05)],
                 device="cpu", world=WorldConfig(bounds=(-1, 1, -1, 1), bounds_mode="clamp"))
    d = bx.desc(2, 2)
    assert bx.has_boxes and d.has_boxes == 1 and d.clamp_bounds == 2 and d.holo_velocity_only == 0
    assert Stepper(cfgs, device="cpu", world=WorldConfig(bounds=(-1, 1, -1, 1),
                                                         bounds_mode="clamp")).desc(2, 2).clamp_bounds == 1
    # wheel contacts: Euler 2-D fleets only (swarp/core/stepper.py:852-857)
    wd = Stepper(cfgs, device="cpu", world=WorldConfig(wheel_contacts=True, wheel_turn_torque=0.1,
                                                       wheel_lateral_friction=0.5)).desc(2, 2)
    assert wd.wheel_contacts == 1 and wd.holo_velocity_only == 0
    assert math.isclose(wd.lat_grip, 0.5 * 9.81) and math.isclose(wd.turn_cap, 0.1)
    with pytest.raises(ValueError, match="wheel_contacts"):
        Stepper(cfgs, device="cpu", world=WorldConfig(wheel_contacts=True, integrator=Integrator.RK4))
    with pytest.raises(ValueError, match="wheel_contacts"):
        Stepper([AgentConfig(model=DynamicsModel.DRONE)], device="cpu",
                world=WorldConfig(wheel_contacts=True))
    st = Stepper(cfgs, dt=0.1, substeps=4, device="cpu", world=WorldConfig())
    assert math.isclose(st.sub_dt, 0.025)
    assert math.isclose(st.neighbor_radius, 2 * 0.2 + 0.02)
    assert st.holo_velocity_only and not st.has_drone
    # a movable body seeds the per-env obstacle state (swarp/core/stepper.py:434-476):
    # shapes at their installed poses, the body origin = root pos - R(root angle) @ offset
    E = 2
    pos = torch.tensor([[[1.0, 2.0], [1.0, 2.5]], [[0.0, 0.0], [0.0, 0.5]]])
    ang = torch.tensor([[0.5, 0.5], [0.0, 0.0]])
    vel = torch.tensor([[[0.1, 0.2], [0.3, 0.4]], [[0.0, 0.0], [0.0, 0.0]]])
    st.set_obstacles(Obstacles(pos=pos, radius=torch.tensor([0.1, 0.1]), angle=ang, vel=vel,
                               kind=torch.tensor([1, 1], dtype=torch.int32),
                               body=torch.tensor([0, 0], dtype=torch.int32),
                               body_offset=torch.tensor([[0.2, -0.1], [0.2, 0.4]])))
    assert st.any_movable and st.ob_state.shape == (E, 24)
    ob = st.ob_state.double().reshape(E, 2, 2, 6)  # [env, shapes | bodies, index, 6]
    assert torch.allclose(ob[:, 0, :, 0:2], pos.double()) and torch.allclose(ob[:, 0, :, 3:5], vel.double())
    c, s_ = math.cos(0.5), math.sin(0.5)
    origin = (1.0 - (c * 0.2 - s_ * -0.1), 2.0 - (s_ * 0.2 + c * -0.1))
    for idx in (0, 1):  # every index carries the state of its body (rooted at 0)
        assert torch.allclose(ob[0, 1, idx, 0:3], torch.tensor([*origin, 0.5], dtype=torch.float64))
        assert torch.allclose(ob[0, 1, idx, 3:5], torch.tensor([0.1, 0.2], dtype=torch.float64))
    # box and segment shapes move with their bodies too (the body pass of any shape)
    st.set_obstacles(Obstacles(pos=torch.zeros(1, 1, 2), radius=torch.ones(1),
                               shape=torch.ones(1, dtype=torch.int32),
                               kind=torch.ones(1, dtype=torch.int32)))
    assert st.any_movable
    # the descriptor names the shape types present (bit t: type t), which picks the body
    # kernel instance: circles only run the one compiled without box / segment terms
    assert st.desc(1, 2).obstacle_types == 0b10
    st.set_obstacles(Obstacles(pos=torch.zeros(1, 2, 2), radius=torch.ones(2),
                               shape=torch.tensor([0, 2], dtype=torch.int32),
                               kind=torch.ones(2, dtype=torch.int32)))
    assert st.desc(1, 2).obstacle_types == 0b101
    # drone fleets push bodies by their planar state (the body kernels' DRONE instances)
    dr = Stepper([drone_config()], device="cpu")
    dr.set_obstacles(Obstacles(pos=torch.zeros(1, 1, 2), radius=torch.ones(1),
                               kind=torch.ones(1, dtype=torch.int32)))
    assert dr.any_movable and dr.ob_state.shape == (1, 12)


def test_desc_fleet_models_and_modes():
    """The descriptor's fleet bit sets describe the configs (they select the kernel
    instance: a profile compiled without the absent models and modes); use_profiles=False
    leaves them 0, the general instances."""
    cfgs = [AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.SERVO),
            AgentConfig(model=DynamicsModel.KINEMATIC_BICYCLE),
            AgentConfig(model=DynamicsModel.DIFF_DRIVE, ctrl_mode=ControlMode.ACCELERATION)]
    d = Stepper(cfgs, device="cpu").desc(3, 2)
    assert d.fleet_models == (1 << 1) | (1 << 2) and d.fleet_modes == 0b111
    d = Stepper([drone_config()], device="cpu").desc(3, 4)
    assert d.fleet_models == 1 << 3 and d.fleet_modes == 1 << int(drone_config().ctrl_mode)
    st = Stepper([AgentConfig()], device="cpu")
    st.use_profiles = False
    d = st.desc(1, 2)
    assert d.fleet_models == 0 and d.fleet_modes == 0


def test_list_method_resolution_and_grid_frame():
    """NeighborGrid's method choice (swarp/core/neighbors.py:387-393) and the frame a world
    rectangle pins (:476-490), as the reference's tests pin them
    (tests/unit/test_neighbors.py:139-163, 201-209, 348-365)."""
    from swarp_amd import NeighborGrid

    assert NeighborGrid(4, 600, radius=0.1, method="auto", device="cpu").method == "uniform_grid"
    assert NeighborGrid(4, 512, radius=0.1, method="auto", device="cpu").method == "brute"
    kw = dict(device="cpu", method="uniform_grid")
    adaptive = NeighborGrid(4, 600, radius=0.2, **kw)._descs["uniform_grid"]
    assert adaptive.neighbor_method == _lib.LISTS_GRID and adaptive.grid_pinned == 0
    assert adaptive.grid_bins == 25 and adaptive.grid_frame
    # bounds is (x_min, x_max, y_min, y_max): origin = the min corner, cell = the larger
    # side / bins (4.0 / 25 beats the 0.1 radius), the radius a floor on the cell
    pinned = NeighborGrid(4, 600, radius=0.1, bounds=(-1.0, 1.0, -2.0, 2.0), **kw)._descs["uniform_grid"]
    assert pinned.grid_pinned == 1 and list(pinned.grid_origin) == [-1.0, -2.0]
    assert pinned.grid_cell == pytest.approx(4.0 / 25)
    coarse = NeighborGrid(4, 600, radius=0.5, bounds=(-1.0, 1.0, -2.0, 2.0), **kw)._descs["uniform_grid"]
    assert coarse.grid_cell == pytest.approx(0.5)
    assert NeighborGrid(4, 8, radius=0.2, device="cpu", method="brute")._descs["brute"].neighbor_method == 0
    with pytest.warns(RuntimeWarning, match="cells per env"):
        NeighborGrid(2, 8, radius=0.5, device="cpu", method="uniform_grid", uniform_bins=128)
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        NeighborGrid(2, 8, radius=0.5, device="cpu", method="uniform_grid")
    with pytest.raises(ValueError, match="uniform_bins"):
        NeighborGrid(2, 8, radius=0.5, device="cpu", method="uniform_grid", uniform_bins=0)
    with pytest.raises(NotImplementedError, match="HashGrid"):
        NeighborGrid(2, 8, radius=0.5, device="cpu", method="grid")
    with pytest.raises(NotImplementedError, match="4096"):
        NeighborGrid(2, 4097, radius=0.5, device="cpu")
    NeighborGrid(2, 3000, radius=0.5, device="cpu")  # 4 agents per thread
    with pytest.raises(NotImplementedError, match="1024 agents"):
        big_bodies = Stepper([AgentConfig(radius=0.01) for _ in range(1100)], device="cpu",
                             world=WorldConfig(bounds=(-5.0, 5.0, -5.0, 5.0)))
        big_bodies.set_obstacles(Obstacles(pos=torch.zeros(1, 1, 2), radius=torch.ones(1),
                                           kind=torch.ones(1, dtype=torch.int32)))
    # stepping: more than 64 agents or grid lists take the wide-env kernels
    big = Stepper([AgentConfig(radius=0.02) for _ in range(600)], device="cpu",
                  world=WorldConfig(bounds=(-2.0, 2.0, -2.0, 2.0)))
    d = big.desc(2, 2)
    assert big.wide and d.neighbor_method == _lib.LISTS_GRID and d.grid_pinned == 1
    assert list(d.grid_origin) == [-2.0, -2.0] and d.grid_cell == pytest.approx(max(big.neighbor_radius, 4.0 / 25))
    assert Stepper([AgentConfig() for _ in range(100)], device="cpu").desc(2, 2).neighbor_method == 0
    with pytest.raises(NotImplementedError, match="bounds"):
        Stepper([AgentConfig(radius=0.02) for _ in range(600)], device="cpu", world=WorldConfig())
    # box worlds too (box agents, wheel contacts): the wide kernels' box pass
    wb = Stepper([AgentConfig(shape="box", half_extents=(0.02, 0.02)) for _ in range(70)], device="cpu")
    assert wb.wide and wb.desc(2, 2).has_boxes == 1


def test_step_refuses_cpu_tensors():
    """No CPU fallback: stepping host tensors raises instead of computing."""
    st = Stepper([AgentConfig()], device="cpu", world=WorldConfig(collisions=False))
    z = torch.zeros(1, 1)
    s = TorchState(torch.zeros(1, 1, 2), z, torch.zeros(1, 1, 2), z, z)
    with pytest.raises(RuntimeError, match="HIP device"):
        warp_step(st, s, torch.zeros(1, 1, 2))
    with pytest.raises(ValueError, match="act_dim"):
        rollout(st, s, torch.zeros(3, 1, 1))
    with pytest.raises(TypeError):
        warp_step(st, s, torch.zeros(1, 1, 2, dtype=torch.float64))


def test_grad_ring_overrun():
    st = Stepper([AgentConfig()], device="cpu", world=WorldConfig(collisions=False))
    ring = GradRing(st, n_envs=2, act_dim=2, capacity=2)
    ring.acquire()
    ring.acquire()
    with pytest.raises(RuntimeError, match="capacity"):
        ring.acquire()
    ring.reset()
    ring.acquire()
    with pytest.raises(RuntimeError, match="capacity"):
        ring.rollout_buffers(3)


# ------------------------------------------------------------------ make / Environment

def test_make_routes_keywords_and_rejects_unknown_ones():
    """``make`` (swarp/__init__.py:95-121): Environment keywords go to Environment, the
    rest to the scenario; an unknown scenario raises ValueError, a stray keyword
    TypeError naming both signatures."""
    from swarp_amd import NavigationScenario, make

    env = make("navigation", 8, device="cpu", dt=0.05, substeps=2, n_agents=5, world_size=2.0)
    assert isinstance(env.scenario, NavigationScenario)
    assert env.scenario.n_agents == 5 and env.n_agents == 5
    assert env.world.stepper.sub_dt == pytest.approx(0.025)
    assert env.obs_dim == 9 + 5 * 2 and env.act_dim == 2
    # navigation's world constants (swarp/scenarios/navigation.py:127-141)
    st = env.world.stepper
    assert st.world.bounds == (-2.0, 2.0, -2.0, 2.0) and st.world.max_neighbors == 5
    assert st.neighbor_radius == pytest.approx(0.125)
    lo, hi = env.action_bounds
    assert lo.shape == (5, 2) and float(hi.max()) == 1.0
    with pytest.raises(ValueError, match="valid names"):
        make("flocking", 2, device="cpu")
    with pytest.raises(TypeError, match="n_agent"):
        make("navigation", 2, device="cpu", n_agent=3)
    with pytest.raises(ValueError):
        make("navigation", 0, device="cpu")
    # box agents: the circumscribed radius replaces agent_radius (navigation.py:61-79)
    benv = make("navigation", 2, device="cpu", agent_shape="box", agent_radius=0.04)
    assert benv.world.stepper.has_boxes
    assert math.isclose(benv.scenario.agent_radius, math.hypot(0.04, 0.02))
    # a world_config override reaches the engine (WorldConfig.override_with)
    env = make("navigation", 2, device="cpu", world_config=WorldConfig(max_neighbors=2))
    assert env.world.stepper.world.max_neighbors == 2 and env.obs_dim == 9 + 5 * 2


def test_environment_validates_actions_before_any_launch():
    from swarp_amd import make

    env = make("navigation", 3, device="cpu", n_agents=2)
    with pytest.raises(ValueError, match="actions must have shape"):
        env.step(torch.zeros(3, 2, 3))
    with pytest.raises(TypeError, match="dtype"):
        env.step(torch.zeros(3, 2, 2, dtype=torch.float64))


def test_compile_registry_does_not_keep_the_stepper_alive():
    """The custom op's handle registry holds steppers weakly (swarp/interop/compile.py:45-90;
    the reference's tests/interop/test_compile.py:91-113)."""
    import gc
    import weakref

    from swarp_amd import compile as compile_mod

    st = Stepper([AgentConfig() for _ in range(2)], device="cpu")
    handle = compile_mod.register_stepper(st)
    assert compile_mod.register_stepper(st) == handle
    ref = weakref.ref(st)
    del st
    gc.collect()
    assert ref() is None and handle not in compile_mod._STEPPERS
    with pytest.raises(RuntimeError, match="garbage-collected"):
        compile_mod._stepper(handle)
    assert hasattr(torch.ops.swarp_amd, "step")


def test_step_graph_forms_no_cycle_with_its_owner():
    """A StepGraph holds its owner's bound-method hooks weakly: the owner (and the graphs
    it captured) die by reference counting, never inside the cyclic collector, which may
    run in the middle of another capture."""
    import gc
    import weakref

    from swarp_amd import make
    from swarp_amd.persistent import StepGraph

    env = make("navigation", 3, device="cpu", n_agents=2)
    env._graph = StepGraph(env.world, hook=env._graph_hook, token=env._graph_token)
    ref, gref = weakref.ref(env), weakref.ref(env._graph)
    gc.disable()
    try:
        del env
        assert ref() is None and gref() is None
    finally:
        gc.enable()


def test_per_env_params_validation():
    """Stepper.set_agent_params_per_env checks (swarp/core/stepper.py:493-575)."""
    from swarp_amd import per_env_float_template
    from swarp_amd.config import P_MASS, P_RADIUS, P_SHAPE

    cfgs = [AgentConfig(radius=0.05), AgentConfig(radius=0.05)]
    st = Stepper(cfgs, device="cpu", world=WorldConfig(neighbor_radius=0.3))
    tab = per_env_float_template(cfgs, 3)
    assert tab.shape == (3, 2, len(PARAM_FIELDS))
    tab[..., P_MASS] = [[1.0, 2.0], [0.5, 1.5], [3.0, 1.0]]
    st.set_agent_params_per_env(tab)
    d = st.desc(3, 2)
    assert d.params_per_env == 1 and d.params == st.params_per_env.data_ptr()
    # the body pass reads the shared rows (swarp/core/stepper.py:961-964)
    assert d.body_params == st.params.floats.data_ptr()
    with pytest.raises(ValueError, match="installed for 3 envs"):
        st.desc(4, 2)
    with pytest.raises(ValueError, match="shape"):
        st.set_agent_params_per_env(tab[:, :1])
    bad = tab.copy()
    bad[0, 0, P_SHAPE] = 1.0
    with pytest.raises(ValueError, match="P_SHAPE"):
        st.set_agent_params_per_env(bad)
    big = tab.copy()
    big[..., P_RADIUS] = 0.2
    with pytest.raises(ValueError, match="neighbor_radius"):
        st.set_agent_params_per_env(big)
    # a same-shape device tensor refreshes in place (no reallocation)
    ptr = st.params_per_env.data_ptr()
    st.set_agent_params_per_env(torch.as_tensor(tab, dtype=torch.float32))
    assert st.params_per_env.data_ptr() == ptr


def test_extent_checks_before_launch():
    """Every tensor handed to the library is checked, on the host, to hold exactly the
    elements the kernels index (contiguous, of the stepper's dtype) -- before any launch."""
    from swarp_amd.stepper import check_extent, state_struct

    t = torch.zeros(4, 3, 2)
    check_extent(t, 24, "x", torch.float32)
    with pytest.raises(ValueError, match="indexes 25"):
        check_extent(t, 25, "x", torch.float32)
    with pytest.raises(TypeError, match="dtype"):
        check_extent(t, 24, "x", torch.float64)
    with pytest.raises(ValueError, match="contiguous"):
        check_extent(t.transpose(0, 1), 24, "x")
    E, A = 4, 3
    ok = [torch.zeros(E, A, 2), torch.zeros(E, A), torch.zeros(E, A, 2), torch.zeros(E, A),
          torch.zeros(E, A)]
    state_struct(ok, E * A, torch.float32, "s")
    bad = list(ok)
    bad[2] = torch.zeros(E, A)  # vel missing its pair
    with pytest.raises(ValueError, match="s.vel"):
        state_struct(bad, E * A, torch.float32, "s")
    state_struct([None] * 5, E * A, torch.float32, "s")  # NULL fields are not read


def test_trajectory_is_a_list_built_on_first_use():
    """rollout's trajectory: a list whose per-step states are built on first use (a loop
    that reads only the final state never builds them); len needs no build."""
    from swarp_amd.autograd import Trajectory

    built = []

    def build():
        built.append(1)
        return ["s0", "s1", "s2"]

    t = Trajectory(3, build)
    assert isinstance(t, list) and len(t) == 3 and bool(t) and not built
    assert t[-1] == "s2" and built == [1]
    assert list(t) == ["s0", "s1", "s2"] and t == ["s0", "s1", "s2"] and "s1" in t
    assert [x for x in reversed(t)] == ["s2", "s1", "s0"] and t[1:] == ["s1", "s2"]
    t.append("s3")
    assert len(t) == 4 and t.index("s3") == 3 and built == [1]
    e = Trajectory(0, list)
    assert len(e) == 0 and not e and list(e) == []


def test_trajectory_built_under_no_grad_keeps_the_rollout_grad_mode():
    """A trajectory first read under no_grad (or inference mode) must still give the
    gradients an eager build would: the per-step views are built under the grad mode of
    the rollout call, not of the first read."""
    from swarp_amd.autograd import _assemble

    class St:
        has_drone = False

    T, E, A = 4, 3, 2
    torch.manual_seed(0)
    src = [torch.randn(T, E, A, 2, requires_grad=True), torch.randn(T, E, A, requires_grad=True),
           torch.randn(T, E, A, 2, requires_grad=True), torch.randn(T, E, A, requires_grad=True),
           torch.randn(T, E, A, requires_grad=True)]
    tail = [torch.zeros(E, A, requires_grad=True), torch.zeros(E, A, requires_grad=True),
            torch.zeros(E, A, 4, requires_grad=True), torch.zeros(E, A, 3, requires_grad=True)]

    def run(read_first):
        outs = [f[T - 1] * 2.0 for f in src] + [f[:T - 1] * 2.0 for f in src]
        state = [None] * 5 + tail
        final, traj = _assemble(St(), state, outs, T)
        if read_first is not None:
            with read_first():
                _ = traj[0].pos.sum().item()
        loss = sum((s.pos ** 2).sum() + s.theta.sum() + s.vel.sum() + s.speed.sum()
                   + s.ang_vel.sum() + s.z.sum() for s in traj[:T - 1])
        grads = torch.autograd.grad(loss, src + tail[:1])
        return [g.clone() for g in grads]

    eager = run(None)
    for mode in (torch.no_grad, torch.inference_mode):
        lazy = run(mode)
        assert all(torch.equal(a, b) for a, b in zip(eager, lazy)), mode
    assert eager[0].abs().sum() > 0 and eager[-1].abs().sum() > 0
