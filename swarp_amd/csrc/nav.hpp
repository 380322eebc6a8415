// nav.hpp -- the navigation scenario's per-step observation / reward pass, fused into one
// launch: radius-neighbour lists of the post-step positions, the observation rows, the
// touching count, goal distance, position shaping (with its carried baseline), the
// on-goal / overflow flags, the per-agent reward and the per-env done flag.
//
// Counterpart of the reference's no-grad fast path: NeighborGrid build + nav_obs_kernel +
// nav_reward_kernel (swarp/scenarios/navigation_kernels.py:41-243, launched by
// NavigationScenario._launch_obs / _launch_reward, swarp/scenarios/navigation.py:539-650).
// Same formulas, same per-agent order of the reward's shaping sum.
//
// Layout: one lane per (env, agent) as in the step kernels -- an env is PA consecutive
// lanes of a wave64, so the env's lists and its reward reduction stay inside the wave
// (positions and per-agent terms in LDS, no global atomics).  Observation rows are
// assembled in LDS and leave as contiguous, coalesced stores when they fit.
// Instantiated by k_nav.hip.
#pragma once
#include "common.hpp"

namespace swarp {

template <typename T> struct NavArgs {
    const T *pos, *vel, *th, *om, *goal, *params;
    const T *radius;       // [A] static radii of the touching test (NULL: params column)
    const uint8_t *rmask;  // [E] just-reset envs (NULL: none)
    T *prev, *obs, *touch, *dist, *shaping, *reward;
    int32_t *idx, *cnt, *tru;
    uint8_t *ongoal, *overflow, *done;
    int32_t *step_count;   // [E] (NULL: not counted here)
    uint8_t *truncated;    // [E] (NULL: not written)
    T shaping_factor, goal_tol, coll_pen, final_rew;
    int k_obs, W, advance_prev, full_pass, shared, stage, max_steps;
};

// Copy `n` elements of type X from LDS to global memory with the wave's 64 lanes, in
// 16-byte pieces when both ends and the length allow it.
template <typename X>
__device__ __forceinline__ void wave_copy(X *dst, const X *src, int n, int lane)
{
    const size_t bytes = (size_t)n * sizeof(X);
    if (((uintptr_t)dst & 15) == 0 && ((uintptr_t)src & 15) == 0 && (bytes & 15) == 0) {
        uint4 *d = reinterpret_cast<uint4 *>(dst);
        const uint4 *q = reinterpret_cast<const uint4 *>(src);
        const int n4 = (int)(bytes >> 4);
        for (int k = lane; k < n4; k += 64) d[k] = q[k];
    } else {
        for (int k = lane; k < n; k += 64) dst[k] = src[k];
    }
}

template <typename T, int PA>
__global__ __launch_bounds__(64) void k_nav(const Cst<T> C, const NavArgs<T> g)
{
    typedef typename MaskT<PA>::type M;
    __shared__ T lx[64], ly[64], lvx[64], lvy[64], lra[64], lsh[64];
    __shared__ int log_[64];
    extern __shared__ __align__(16) unsigned char nav_dyn[];
    // staged output rows: observation rows [64][W], then list rows [64][K]
    T *row_lds = reinterpret_cast<T *>(nav_dyn);
    int32_t *idx_lds = reinterpret_cast<int32_t *>(nav_dyn + (size_t)64 * g.W * sizeof(T));

    const int lane = threadIdx.x, agent = lane % PA, base = lane - agent;
    const int env = blockIdx.x * (64 / PA) + lane / PA;
    const bool real = agent < C.A;
    const bool active = real && env < C.E;
    const size_t i = active ? (size_t)env * C.A + agent : 0;
    const bool reset_hit = active && g.rmask != nullptr && g.rmask[env] != 0;
    // an obs-only pass (auto-reset) recomputes only the envs it resets: the others'
    // positions are unchanged since the step pass that already wrote every output
    const bool work = active && (g.full_pass != 0 || reset_hit);

    const T qnan = __builtin_nan("");
    T px = qnan, py = qnan, vx = T(0), vy = T(0);
    if (active) {
        px = g.pos[2 * i];
        py = g.pos[2 * i + 1];
        vx = g.vel[2 * i];
        vy = g.vel[2 * i + 1];
    }
    // the static radius: the scenario's per-agent radius (the reference's navigation
    // kernels take it even under per-env randomization), else column P_RADIUS
    const T ra = g.radius ? g.radius[real ? agent : 0]
                          : g.params[((C.per_env ? (size_t)(env < C.E ? env : 0) * C.A : 0) +
                                      (real ? agent : 0)) * 22];
    lx[lane] = px;
    ly[lane] = py;
    lvx[lane] = vx;
    lvy[lane] = vy;
    lra[lane] = ra;
    __syncthreads();

    // radius lists of the current positions (the NeighborGrid build the reference runs
    // before nav_obs_kernel): ascending index order, first K, uncapped count
    M cd;
    const M incl = scan_all<T, PA>(lx, ly, base, C.A, agent, px, py, C.t_nbr, C.t_nbr, cd);
    const M m = cap_list(incl, C.K);
    const int n = m_popc(m);
    if (g.stage || work) {
        int32_t *irow = g.stage ? idx_lds + (size_t)lane * C.K : g.idx + i * C.K;
        M mm = m;
        for (int k = 0; k < C.K; ++k) {
            int v = 0;
            if (k < n) {
                v = m_ctz(mm);
                mm &= mm - 1;
            }
            irow[k] = v;
        }
    }
    if (work) {
        g.cnt[i] = n;
        if (g.tru) g.tru[i] = m_popc(incl);
    }

    // touching listed neighbours: |p_b - p| < r_a + r_b (navigation_kernels.py:175-180)
    T touch = T(0);
    {
        M mm = m;
        while (mm) {
            const int b = m_ctz(mm);
            mm &= mm - 1;
            const T dx = lx[base + b] - px, dy = ly[base + b] - py;
            const T nd = m_sqrt(dx * dx + dy * dy);
            if (nd < ra + lra[base + b]) touch += T(1);
        }
    }

    // own features, goal distance (navigation_kernels.py:165-170)
    T gx = T(0), gy = T(0), th = T(0), om = T(0);
    if (active) {
        gx = g.goal[2 * i];
        gy = g.goal[2 * i + 1];
        th = g.th[i];
        om = g.om[i];
    }
    const T grx = gx - px, gry = gy - py;
    const T ddx = px - gx, ddy = py - gy;
    const T d = m_sqrt(ddx * ddx + ddy * ddy);

    // observation row (_obs_row, :41-89)
    const int W = g.W, KO = g.k_obs;
    {
        T *dst = g.stage ? row_lds + (size_t)lane * W : g.obs + i * W;
        const bool put = g.stage || work;
        if (put) {
            dst[0] = px;
            dst[1] = py;
            dst[2] = vx;
            dst[3] = vy;
            dst[4] = m_cos(th);
            dst[5] = m_sin(th);
            dst[6] = om;
            dst[7] = grx;
            dst[8] = gry;
            M mm = m;
            for (int j = 0; j < KO; ++j) {
                T rpx = T(0), rpy = T(0), rvx = T(0), rvy = T(0), valid = T(0);
                if (j < n) {
                    const int b = m_ctz(mm);
                    mm &= mm - 1;
                    rpx = lx[base + b] - px;
                    rpy = ly[base + b] - py;
                    rvx = lvx[base + b] - vx;
                    rvy = lvy[base + b] - vy;
                    valid = T(1);
                }
                dst[9 + 2 * j] = rpx;
                dst[9 + 2 * j + 1] = rpy;
                dst[9 + 2 * KO + 2 * j] = rvx;
                dst[9 + 2 * KO + 2 * j + 1] = rvy;
                dst[9 + 4 * KO + j] = valid;
            }
        }
    }

    // shaping baseline and reward inputs (_shaping_and_flags, :92-139)
    T shp = T(0);
    bool og = false;
    if (work) {
        const T prev = g.prev[i];
        const T ps = (prev - d) * g.shaping_factor;
        if (reset_hit) {
            g.prev[i] = d;
            shp = T(0);
        } else {
            if (g.advance_prev) g.prev[i] = d;
            shp = ps;
        }
        og = d < g.goal_tol;
        if (g.full_pass) {
            g.shaping[i] = shp;
            g.touch[i] = touch;
            g.dist[i] = d;
            g.ongoal[i] = og ? 1 : 0;
            g.overflow[i] = m_popc(incl) > n ? 1 : 0;
        }
    }

    if (g.stage) {
        // an env's rows are A consecutive rows both in LDS (lanes e*PA .. e*PA+A-1) and in
        // memory, so each env leaves as one contiguous block; with no pad slots (A == PA)
        // and every env written, the whole wave's rows are one block
        __syncthreads();
        const int env0 = blockIdx.x * (64 / PA);
        const int n_env = min(64 / PA, C.E - env0);
        if (g.full_pass != 0 && PA == C.A) {
            const size_t first = (size_t)env0 * C.A;
            wave_copy(g.obs + first * W, row_lds, n_env * C.A * W, lane);
            wave_copy(g.idx + first * C.K, idx_lds, n_env * C.A * C.K, lane);
        } else {
            for (int e = 0; e < n_env; ++e) {
                if (g.full_pass == 0 && !(g.rmask != nullptr && g.rmask[env0 + e] != 0)) continue;
                const size_t first = (size_t)(env0 + e) * C.A;
                wave_copy(g.obs + first * W, row_lds + (size_t)e * PA * W, C.A * W, lane);
                wave_copy(g.idx + first * C.K, idx_lds + (size_t)e * PA * C.K, C.A * C.K, lane);
            }
        }
    }

    // reward and done (nav_reward_kernel, :211-243), full passes only: sequential
    // per-agent sum of the env's shaping, all-on-goal flag
    if (g.full_pass) {
        lsh[lane] = shp;
        log_[lane] = og ? 1 : 0;
        __syncthreads();
        if (active) {
            T sum = T(0);
            int all_og = 1;
            for (int a = 0; a < C.A; ++a) {
                sum += lsh[base + a];
                all_og &= log_[base + a];
            }
            T r = g.coll_pen * touch;
            r += g.shared ? sum : shp;
            const T fin = all_og ? g.final_rew : T(0);
            g.reward[i] = r + fin;
            if (agent == 0) {
                g.done[env] = all_og ? 1 : 0;
                // the env's step counter and time limit (a step pass)
                if (g.step_count != nullptr && g.advance_prev) {
                    const int sc = g.step_count[env] + 1;
                    g.step_count[env] = sc;
                    if (g.truncated) g.truncated[env] = (g.max_steps > 0 && sc >= g.max_steps) ? 1 : 0;
                }
            }
        }
    }
}

template <typename T>
void launch_nav(int PA, const Cst<T> &C, const NavArgs<T> &g, unsigned dyn, hipStream_t st)
{
    const dim3 grid((C.E + (64 / PA) - 1) / (64 / PA));
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_nav<T, 4>), grid, dim3(64), dyn, st, C, g); break;
    case 8: hipLaunchKernelGGL((k_nav<T, 8>), grid, dim3(64), dyn, st, C, g); break;
    case 16: hipLaunchKernelGGL((k_nav<T, 16>), grid, dim3(64), dyn, st, C, g); break;
    case 32: hipLaunchKernelGGL((k_nav<T, 32>), grid, dim3(64), dyn, st, C, g); break;
    default: hipLaunchKernelGGL((k_nav<T, 64>), grid, dim3(64), dyn, st, C, g); break;
    }
}

}  // namespace swarp
