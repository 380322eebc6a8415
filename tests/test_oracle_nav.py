"""Pins of the navigation-pass oracle (``oracle/nav.py``) against hand-computed answers
of the reference's definitions (swarp/scenarios/navigation_kernels.py:41-243,
swarp/scenarios/navigation.py:671-839)."""

import numpy as np

from oracle.nav import nav_pass

F = np.float64


def _scene():
    # env 0: agents 0 and 1 overlap (0.08 apart, radii 0.05 + 0.05), agent 2 far away;
    # env 1: agent 1 sits on its goal, the others do not
    pos = np.array([[[0.0, 0.0], [0.08, 0.0], [1.0, 1.0]],
                    [[0.5, 0.5], [-0.5, -0.5], [0.5, -0.5]]], F)
    vel = np.array([[[0.1, 0.0], [0.0, 0.2], [0.0, 0.0]],
                    [[0.0, 0.0], [0.0, 0.0], [0.3, 0.3]]], F)
    theta = np.array([[0.0, np.pi / 2, 1.0], [0.0, 0.0, 0.0]], F)
    ang_vel = np.array([[0.0, 0.5, 0.0], [0.0, 0.0, -1.0]], F)
    goals = np.array([[[0.3, 0.4], [0.08, 0.0], [1.0, 1.0]],
                      [[0.5, 0.5], [-0.5, -0.49], [0.0, -0.5]]], F)
    radius = np.full(3, 0.05, F)
    return pos, vel, theta, ang_vel, goals, radius


def test_observation_rows_and_lists():
    pos, vel, theta, ang_vel, goals, radius = _scene()
    prev = np.zeros((2, 3), F)
    o = nav_pass(pos, vel, theta, ang_vel, goals, radius, nbr_radius=0.125, K=2, k_obs=2,
                 prev=prev, reset_mask=np.ones(2, bool), advance_prev=0, full_pass=1)
    # lists: 0 <-> 1 only (0.08 <= 0.125), no neighbours in env 1
    assert o["cnt"].tolist() == [[1, 1, 0], [0, 0, 0]]
    assert o["idx"][0, 0, 0] == 1 and o["idx"][0, 1, 0] == 0
    row = o["obs"][0, 0]
    want = [0.0, 0.0, 0.1, 0.0, 1.0, 0.0, 0.0, 0.3, 0.4,     # own features, goal - pos
            0.08, 0.0, 0.0, 0.0,                             # rel pos of slots 0, 1
            -0.1, 0.2, 0.0, 0.0,                             # rel vel of slots 0, 1
            1.0, 0.0]                                        # validity
    np.testing.assert_allclose(row, want, rtol=0, atol=1e-15)
    np.testing.assert_allclose(o["obs"][0, 1, 4:6], [np.cos(np.pi / 2), 1.0], atol=1e-15)
    assert o["obs"].shape == (2, 3, 9 + 5 * 2)
    # a reset pass: baseline = spawn distance, shaping 0, touching counted
    np.testing.assert_allclose(prev[0], [0.5, 0.0, 0.0], atol=1e-15)
    assert o["touching"].tolist() == [[1.0, 1.0, 0.0], [0.0, 0.0, 0.0]]
    assert (o["shaping"] == 0).all()
    # env 0: -1 per touching neighbour; agent 1 and 2 are on their goals, agent 0 is not
    assert o["reward"].tolist()[0] == [-1.0, -1.0, 0.0]
    assert o["on_goal"].tolist() == [[0, 1, 1], [1, 1, 0]] and o["done"].tolist() == [0, 0]


def test_shaping_final_reward_and_shared_sum():
    pos, vel, theta, ang_vel, goals, radius = _scene()
    prev = np.array([[0.9, 0.1, 0.0], [0.2, 0.3, 0.6]], F)
    o = nav_pass(pos, vel, theta, ang_vel, goals, radius, 0.125, 2, 2, prev, None, 1, 1,
                 shaping_factor=2.0, goal_tol=0.6, final_rew=5.0, shared=True)
    d = np.array([[0.5, 0.0, 0.0], [0.0, 0.01, 0.5]])
    np.testing.assert_allclose(o["dist"], d, atol=1e-15)
    shp = (np.array([[0.9, 0.1, 0.0], [0.2, 0.3, 0.6]]) - d) * 2.0
    np.testing.assert_allclose(o["shaping"], shp, atol=1e-15)
    np.testing.assert_allclose(prev, d, atol=1e-15)             # the baseline advanced
    # goal_tol 0.6 puts every agent on its goal: +5 each, done; shared sum of shaping
    assert o["done"].tolist() == [1, 1]
    want = -1.0 * o["touching"] + shp.sum(-1, keepdims=True) + 5.0
    np.testing.assert_allclose(o["reward"], want, atol=1e-14)


def test_obs_only_pass_rewrites_only_the_reset_envs():
    pos, vel, theta, ang_vel, goals, radius = _scene()
    prev = np.zeros((2, 3), F)
    o = nav_pass(pos, vel, theta, ang_vel, goals, radius, 0.125, 2, 2, prev, None, 1, 1)
    snap = {k: v.copy() for k, v in o.items()}
    prev_before = prev.copy()
    pos2 = pos + 0.01
    o = nav_pass(pos2, vel, theta, ang_vel, goals, radius, 0.125, 2, 2, prev,
                 np.array([False, True]), 0, 0, out=o)
    for k in ("reward", "done", "touching", "dist", "shaping", "on_goal", "overflow"):
        assert np.array_equal(o[k], snap[k]), k                 # reward inputs untouched
    assert np.array_equal(o["obs"][0], snap["obs"][0])          # env 0 not rewritten
    np.testing.assert_allclose(o["obs"][1, :, 0:2], pos2[1], atol=0)
    assert np.array_equal(prev[0], prev_before[0])
    np.testing.assert_allclose(prev[1], np.linalg.norm(pos2[1] - goals[1], axis=-1), atol=1e-15)


def test_overflow_flag_and_list_cap():
    pos = np.zeros((1, 5, 2), F)
    pos[0, :, 0] = [0.0, 0.01, 0.02, 0.03, 0.04]
    o = nav_pass(pos, np.zeros_like(pos), np.zeros((1, 5), F), np.zeros((1, 5), F),
                 np.zeros_like(pos), np.full(5, 0.05, F), 0.125, 2, 2, np.zeros((1, 5), F))
    assert o["true"].tolist() == [[4] * 5] and o["cnt"].tolist() == [[2] * 5]
    assert o["overflow"].all()
    assert o["idx"][0, 0].tolist() == [1, 2] and o["idx"][0, 4].tolist() == [0, 1]
    # touching counts only the capped list
    assert o["touching"].tolist() == [[2.0] * 5]
