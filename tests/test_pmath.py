"""The portable transcendental functions (include/swarp_pmath.h) that the HIP kernels and
the CPU oracle share, pinned against numpy's float64 libm.

float32 (what the float32 step computes: a double evaluation rounded once): within one
ulp of the correctly rounded value everywhere sampled, and equal to it on all but a tiny
fraction of inputs (a double result within 2^-29 ulp of a float32 rounding boundary);
float64: within 4 ulps, or within 2^-80 (1 + |x|) absolute next to the zeros of sin and
cos (the reduction's pi/2 has two parts).  Special values: odd symmetry with signed zeros, NaN in NaN
out, atan(+-inf) = +-pi/2, tanh saturating to +-1.
"""

import numpy as np
import pytest

from oracle.oracle import pmath

REF = {"sin": np.sin, "cos": np.cos, "tan": np.tan, "atan": np.arctan, "tanh": np.tanh}


def _inputs(name, rng):
    if name in ("sin", "cos"):
        parts = [rng.uniform(-7, 7, 200000), rng.uniform(-1e4, 1e4, 50000),
                 rng.uniform(-1e-4, 1e-4, 20000), np.arange(-64, 65) * (np.pi / 4)]
    elif name == "tan":
        parts = [rng.uniform(-1.4, 1.4, 200000), rng.uniform(-1e-4, 1e-4, 20000),
                 rng.uniform(-np.pi / 4, np.pi / 4, 50000)]
    elif name == "atan":
        parts = [rng.uniform(-4, 4, 200000), rng.uniform(-1e5, 1e5, 50000),
                 rng.uniform(-1e-4, 1e-4, 20000), np.array([0.125, 0.375, 0.625, 0.875, 1.0])]
    else:
        parts = [rng.uniform(-4, 4, 200000), rng.uniform(-30, 30, 50000),
                 rng.uniform(-1e-4, 1e-4, 20000), rng.uniform(0.24, 0.26, 20000)]
    return np.concatenate(parts)


@pytest.mark.parametrize("name", list(REF))
def test_float32_correctly_rounded(name):
    x64 = _inputs(name, np.random.default_rng(hash(name) % 2**32)).astype(np.float32).astype(np.float64)
    got = pmath(name, x64.astype(np.float32)).astype(np.float64)
    ref = REF[name](x64)
    ref32 = ref.astype(np.float32)
    ulp = np.spacing(np.abs(ref32)).astype(np.float64)
    err = np.abs(got - ref) / np.maximum(ulp, 1e-45)
    assert err.max() <= 1.0, f"{name}: {err.max():.3f} ulp"
    assert np.mean(got != ref32.astype(np.float64)) <= 1e-4


@pytest.mark.parametrize("name", list(REF))
def test_float64_few_ulps(name):
    x = _inputs(name, np.random.default_rng(7 + len(name)))
    got = pmath(name, x)
    ref = REF[name](x)
    bound = np.maximum(4.0 * np.spacing(np.abs(ref)), 2.0 ** -80 * (1.0 + np.abs(x)))
    err = np.abs(got - ref) / bound
    assert err.max() <= 1.0, f"{name}: {err.max():.2f} of the bound"


def test_special_values():
    for dt in (np.float32, np.float64):
        z = np.array([0.0, -0.0], dt)
        for name in ("sin", "tan", "atan", "tanh"):
            y = pmath(name, z)
            assert np.array_equal(np.signbit(y), [False, True]) and (y == 0).all(), name
        assert (pmath("cos", z) == 1).all()
        nan = np.array([np.nan], dt)
        for name in REF:
            assert np.isnan(pmath(name, nan)).all(), name
        inf = np.array([np.inf, -np.inf], dt)
        np.testing.assert_array_equal(pmath("atan", inf), np.array([np.pi / 2, -np.pi / 2], dt))
        big = np.array([25.0, -25.0, 1e30, -1e30], dt)
        np.testing.assert_array_equal(pmath("tanh", big), np.array([1, -1, 1, -1], dt))
    # odd / even symmetry holds exactly
    x = np.random.default_rng(3).uniform(-5, 5, 1000)
    for name in ("sin", "tan", "atan", "tanh"):
        np.testing.assert_array_equal(pmath(name, -x), -pmath(name, x))
    np.testing.assert_array_equal(pmath("cos", -x), pmath("cos", x))
