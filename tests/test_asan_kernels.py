"""The HIP kernels and the library's host code, built for the CPU under AddressSanitizer
and UndefinedBehaviorSanitizer (tests/asan: the kernels run on a host emulation of the
HIP device model; one host thread per work-item, barriers and wave collectives by
exchange).  Every kernel family but the DPP-specialised ones runs through the C entry
points on host buffers of exactly the extents the ABI documents, in the order of the run
whose GPU memory fault is on record (movable bodies, then the float32 drone rollout
with every adjoint field, then the others).  A planted mistake -- an actions buffer one
element short -- must be reported, so the harness is shown to see an out-of-bounds read.
"""

import importlib.util
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def driver():
    spec = importlib.util.spec_from_file_location("asan_build", HERE / "asan" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build()


def _run(exe, *args):
    return subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=900,
                          cwd="/tmp")


def test_kernels_clean_under_sanitizers(driver):
    r = _run(driver)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert "0 case(s) failed" in r.stdout
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr


def test_planted_short_buffer_is_reported(driver):
    r = _run(driver, "--plant-short-actions")
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr and "load_act" in r.stderr
