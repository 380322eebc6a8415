"""CPU restatement of the navigation scenario's per-step observation / reward pass.

TEST INFRASTRUCTURE ONLY: the parity checker of the fused HIP pass (``swarp_nav_obs``);
nothing in the product imports it.

Restates, in numpy at the arrays' own precision and in the reference's operation order:
  * the radius lists of the current positions (``_brute_force``,
    swarp/core/neighbors.py:76-97) -- through the C oracle's ``neighbors``;
  * ``nav_obs_kernel`` with ``_obs_row`` and ``_shaping_and_flags``
    (swarp/scenarios/navigation_kernels.py:41-208);
  * ``nav_reward_kernel`` (swarp/scenarios/navigation_kernels.py:211-243): the env's
    shaping summed sequentially in agent order.

Cosine and sine go through numpy's libm, so those two observation slots agree with a
device to within an ulp, not bit for bit; every other value is +, -, *, sqrt and compares.
"""

from __future__ import annotations

import numpy as np

from .oracle import Oracle


def nav_pass(pos, vel, theta, ang_vel, goals, radius, nbr_radius, K, k_obs, prev,
             reset_mask=None, advance_prev=1, full_pass=1, shaping_factor=1.0, goal_tol=0.05,
             coll_pen=-1.0, final_rew=5.0, shared=False, out=None):
    """One pass over ``[E, A]`` agents.  ``prev`` (the shaping baseline) is updated in
    place.  ``out`` (a dict of the previous pass's outputs, or None) receives the results;
    an obs-only pass (``full_pass=0``) only rewrites the envs of ``reset_mask``, as the
    reference's early return does.  Returns ``out``."""
    dt = pos.dtype
    E, A = pos.shape[:2]
    f = lambda x: np.asarray(x, dtype=dt)  # noqa: E731
    W = 9 + 5 * k_obs
    if out is None:
        out = {
            "idx": np.zeros((E, A, K), np.int32), "cnt": np.zeros((E, A), np.int32),
            "true": np.zeros((E, A), np.int32), "obs": np.zeros((E, A, W), dt),
            "touching": np.zeros((E, A), dt), "dist": np.zeros((E, A), dt),
            "shaping": np.zeros((E, A), dt), "on_goal": np.zeros((E, A), np.uint8),
            "overflow": np.zeros((E, A), np.uint8), "reward": np.zeros((E, A), dt),
            "done": np.zeros(E, np.uint8),
        }
    rm = np.zeros(E, bool) if reset_mask is None else np.asarray(reset_mask, bool)
    work = np.ones(E, bool) if full_pass else rm
    idx, cnt, tru = Oracle(dt.type).neighbors(pos, nbr_radius, K)
    out["idx"][work], out["cnt"][work], out["true"][work] = idx[work], cnt[work], tru[work]
    sf, gt, cp, fr = f(shaping_factor), f(goal_tol), f(coll_pen), f(final_rew)
    one, zero = f(1.0), f(0.0)
    shaping_all = np.zeros((E, A), dt)
    og_all = np.zeros((E, A), bool)
    touch_all = np.zeros((E, A), dt)
    for e in range(E):
        if not work[e]:
            continue
        for a in range(A):
            p, v = pos[e, a], vel[e, a]
            g = goals[e, a]
            grel = g - p
            dd = p - g
            d = np.sqrt(dd[0] * dd[0] + dd[1] * dd[1])
            n = cnt[e, a]
            touch = zero
            for j in range(n):
                b = idx[e, a, j]
                r = pos[e, b] - p
                if np.sqrt(r[0] * r[0] + r[1] * r[1]) < radius[a] + radius[b]:
                    touch = touch + one
            row = out["obs"][e, a]
            row[0], row[1], row[2], row[3] = p[0], p[1], v[0], v[1]
            row[4], row[5] = np.cos(theta[e, a]), np.sin(theta[e, a])
            row[6], row[7], row[8] = ang_vel[e, a], grel[0], grel[1]
            for j in range(k_obs):
                if j < n:
                    b = idx[e, a, j]
                    rp, rv, val = pos[e, b] - p, vel[e, b] - v, one
                else:
                    rp, rv, val = np.zeros(2, dt), np.zeros(2, dt), zero
                row[9 + 2 * j], row[10 + 2 * j] = rp
                row[9 + 2 * k_obs + 2 * j], row[10 + 2 * k_obs + 2 * j] = rv
                row[9 + 4 * k_obs + j] = val
            ps = (prev[e, a] - d) * sf
            if rm[e]:
                prev[e, a] = d
                shp = zero
            else:
                if advance_prev:
                    prev[e, a] = d
                shp = ps
            og = bool(d < gt)
            shaping_all[e, a], og_all[e, a], touch_all[e, a] = shp, og, touch
            if full_pass:
                out["shaping"][e, a] = shp
                out["touching"][e, a] = touch
                out["dist"][e, a] = d
                out["on_goal"][e, a] = og
                out["overflow"][e, a] = tru[e, a] > n
    if full_pass:
        for e in range(E):
            s = zero
            for a in range(A):
                s = s + shaping_all[e, a]
            all_og = bool(og_all[e].all())
            for a in range(A):
                r = cp * touch_all[e, a]
                r = r + (s if shared else shaping_all[e, a])
                out["reward"][e, a] = r + (fr if all_og else zero)
            out["done"][e] = all_og
    return out
