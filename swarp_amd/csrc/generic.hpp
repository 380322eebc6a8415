// generic.hpp -- the generic rollout kernels (every fleet the specialised holonomic kernels
// do not cover: diff-drive, bicycle, drones, obstacles, clamps, box agents, RK4) and their
// launchers.  Instantiated per (dtype, DRONE, BOXES) by the k_generic*.hip units.
//
// k_rollout_fwd and k_rollout_bwd run one wave per workgroup, so their lanes exchange
// values through LDS behind wave_lds_sync (a wavefront-scope fence) instead of a
// workgroup barrier, whose fence would also wait for every outstanding global load and
// store.
// k_rollout_fwd_split runs two waves per workgroup and synchronises them with barriers.
#pragma once
#include "common.hpp"

namespace swarp {

// ------------------------------------------------------------------ forward rollout

// BOXES: the box-aware contact pass is compiled in (a world holding box agents); the
// disc-only instances keep the register budget of the disc contact law.
template <typename T, int PA, bool DRONE, bool BOXES, unsigned F>
__global__ __launch_bounds__(64) void k_rollout_fwd(const Cst<T> Cin, const Args<T> g)
{
    typedef typename MaskT<PA>::type M;
    const Cst<T> C = fold_cst<F>(Cin);
    __shared__ T sl[7 * 64];  // px py vx vy th (s) w of the current substep
    __shared__ T lr[64];      // agent radius per lane
    __shared__ T lbx[3 * 64]; // footprint per lane: shape, hx, hy (box worlds)
    __shared__ T lcs[2 * 64]; // cos, sin of each lane's heading this substep (box worlds)
    __shared__ T ocs_lds[2 * OCS_MAX];
    Lane<T, PA> L;
    lane_init<T, PA>(C, g, L);
    fold_prm<F>(L.pr);
    lr[L.lane] = L.pr.radius;
    lbx[L.lane] = L.pr.shape;
    lbx[64 + L.lane] = L.pr.hx;
    lbx[128 + L.lane] = L.pr.hy;
    const T *ocs = ob_trig_table<T, PA>(C, g, L, ocs_lds);
    St<T> st;
    load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
    if (!L.real) st.px = st.py = __builtin_nan("");
    const size_t EA = (size_t)C.E * C.A;
    // each step's action is loaded one step ahead and taken into registers before the
    // step's state stores: memory operations complete in order, so a load issued after
    // the stores would also wait for them
    T a[4];
    load_act(g.act, L.idx, C.ad, a);
    for (int t = 0; t < g.nsteps; ++t) {
        // no progress_priority: this kernel's main user, the quadrotor fleet, runs one wave
        // per SIMD, and the priority switches cost it 3 % there
        T an[4] = {a[0], a[1], a[2], a[3]};
        if (t + 1 < g.nsteps) load_act(g.act, (size_t)(t + 1) * EA + L.idx, C.ad, an);
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            T Fx = T(0), Fy = T(0), Tq = T(0);
            if (C.needs_forces) {
                if (C.collisions) {
                    wave_lds_sync();
                    sl[F_PX * 64 + L.lane] = st.px;
                    sl[F_PY * 64 + L.lane] = st.py;
                    sl[F_VX * 64 + L.lane] = st.vx;
                    sl[F_VY * 64 + L.lane] = st.vy;
                    if (BOXES) {
                        sl[F_TH * 64 + L.lane] = st.th;
                        sl[F_W * 64 + L.lane] = st.w;
                    }
                }
                if (BOXES) {
                    if (!C.collisions) wave_lds_sync();
                    lcs[L.lane] = m_cos(st.th);
                    lcs[64 + L.lane] = m_sin(st.th);
                }
                if (C.collisions || BOXES) wave_lds_sync();
                const M incl =
                    forces<T, PA, BOXES>(C, g, L, sl, lr, st, s, s == 0 || !ok, cand, Fx, Fy, ocs,
                                         lbx, lcs, nullptr, nullptr, nullptr, nullptr,
                                         BOXES && C.wheel ? &Tq : nullptr);
                if (!BOXES && g.fsum && L.active) {
                    const size_t k = ((size_t)t * C.S + s) * EA + L.idx;
                    g.fsum[2 * k] = Fx;
                    g.fsum[2 * k + 1] = Fy;
                    if (C.collisions) ((M *)g.nmask)[k] = incl;
                }
            }
            St<T> nx;
            if (BOXES && C.wheel) {
                // the unclamped step, wheel_contact, then the clamp (integrate2d_wheel_kernel,
                // swarp/dynamics/kernels.py:1389-1478)
                Cst<T> C0 = C;
                C0.clamp = 0;
                integrate<T, DRONE>(C0, L.pr, st, a, Fx, Fy, nx);
                wheel_contact(C, L.pr, st, Fx, Fy, Tq, nx);
                if (C.clamp) clamp_position(C, L.pr, nx.th, nx.px, nx.py);
            } else {
                integrate<T, DRONE>(C, L.pr, st, a, Fx, Fy, nx);
            }
            if (C.use_skin) {
                D += (m_abs(nx.px - st.px) + m_abs(nx.py - st.py)) * T(1.0001);
                ok = env_all<PA>(!L.real || D <= C.half_margin, L.base);
            }
            st = nx;
        }
        asm volatile("" ::"v"(an[0]), "v"(an[1]), "v"(an[2]), "v"(an[3]));
        if (L.active) {
            if (t + 1 < g.nsteps)
                store_state<T, DRONE>(g.traj.f, (size_t)t * EA + L.idx, st);
            else
                store_state<T, DRONE>(g.fin.f, L.idx, st);
        }
        for (int k = 0; k < 4; ++k) a[k] = an[k];
    }
}


// Forward rollout of 2-D fleets among static obstacles (feature profile F with FT_OBST,
// no box agents, no drones), two waves per workgroup holding the same envs: wave 0 (the
// agent wave) publishes each substep's state, scans, sums the listed pairs' forces and the
// walls', integrates and stores; wave 1 (the obstacle wave) sums each agent's obstacle
// forces in index order from the published state.  The force is fx + (so + w): the pair
// sum plus the static sum, obstacles then walls, the reference's order
// (swarp/core/collisions.py:852-880, 781-815), so the bits are k_rollout_fwd's.  The
// obstacle pass is about half of such a step; on its own wave it overlaps the agent wave's
// work and doubles the resident waves of a launch that is latency-bound with two.
constexpr int SPLIT_TAIL_MAX = 2;  // obstacles the two-wave forward's agent wave may take
// How many of N obstacles (the last ones) the agent wave takes.
__device__ __forceinline__ int split_tail(int N)
{
    return N / 4 < SPLIT_TAIL_MAX ? N / 4 : SPLIT_TAIL_MAX;
}

template <typename T, int PA, unsigned F>
__global__ __launch_bounds__(128, 4) void k_rollout_fwd_split(const Cst<T> Cin, const Args<T> g)
{
    typedef typename MaskT<PA>::type M;
    const Cst<T> C = fold_cst<F>(Cin);
    __shared__ T sl[7 * 64];  // px py vx vy of the current substep (F_* rows)
    __shared__ T lr[64];      // agent radius per lane
    __shared__ T lso[2 * 64]; // the obstacle wave's sums: x row, y row
    __shared__ uint32_t lom[2 * 64];  // obstacles in contact: obstacle wave's, agent wave's
    __shared__ T ocs_lds[2 * OCS_MAX];
    // the env slots' obstacle poses and bounds (the launcher runs this kernel only when
    // the per-launch obstacle tables fit)
    __shared__ T opos_lds[OPOSE_W * OCS_MAX];
    const bool agent_wave = threadIdx.x < 64;
    Lane<T, PA> L;
    lane_init<T, PA>(C, g, L, (int)(threadIdx.x & 63));
    fold_prm<F>(L.pr);
    if (agent_wave) lr[L.lane] = L.pr.radius;
    const T *opos = ob_pose_table<T, PA>(C, g, L, opos_lds);
    const T *ocs = ob_trig_table<T, PA>(C, g, L, ocs_lds);
    const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
    // the last NT obstacles go to the agent wave, which adds their forces to the obstacle
    // wave's sum in index order (the same sum): it balances the two waves' work
    const int NT = split_tail(C.N);
    St<T> st;
    load_state<T, false>(g.s0.f, L.idx, 0, st);
    if (!L.real) st.px = st.py = __builtin_nan("");
    const size_t EA = (size_t)C.E * C.A;
    T a[4] = {T(0), T(0), T(0), T(0)};  // the step's action, loaded one step ahead
    if (agent_wave) load_act(g.act, L.idx, C.ad, a);
    for (int t = 0; t < g.nsteps; ++t) {
        progress_priority(t, g.nsteps);
        T an[4] = {a[0], a[1], a[2], a[3]};
        if (agent_wave && t + 1 < g.nsteps) load_act(g.act, (size_t)(t + 1) * EA + L.idx, C.ad, an);
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            __syncthreads();  // the previous substep's readers are done with sl / lso
            if (agent_wave) {
                sl[F_PX * 64 + L.lane] = st.px;
                sl[F_PY * 64 + L.lane] = st.py;
                sl[F_VX * 64 + L.lane] = st.vx;
                sl[F_VY * 64 + L.lane] = st.vy;
            }
            __syncthreads();
            if (!agent_wave) {
                const T px = sl[F_PX * 64 + L.lane], py = sl[F_PY * 64 + L.lane];
                const T vx = sl[F_VX * 64 + L.lane], vy = sl[F_VY * 64 + L.lane];
                T sx = T(0), sy = T(0);
                uint32_t om = 0u;  // obstacles in contact (kept for at most 32)
                for (int o = 0; o < C.N - NT; ++o) {
                    T gx, gy;
                    if (obstacle_force<T, Dv<T>, true>(C, g.obs, eN, o, px, py, vx, vy,
                                                       L.pr.radius, L.ddv, gx, gy, ocs, opos))
                        om |= 1u << (o & 31);
                    sx += gx;
                    sy += gy;
                }
                lso[L.lane] = sx;
                lso[64 + L.lane] = sy;
                lom[L.lane] = om;
            }
            T fx = T(0), fy = T(0), wx = T(0), wy = T(0);
            T tfx[SPLIT_TAIL_MAX], tfy[SPLIT_TAIL_MAX];  // the tail obstacles' forces
            M incl = 0;
            if (agent_wave) {
                uint32_t omt = 0u;
#pragma unroll
                for (int k = 0; k < SPLIT_TAIL_MAX; ++k) {
                    tfx[k] = tfy[k] = T(0);
                    if (k < NT &&
                        obstacle_force<T, Dv<T>, true>(C, g.obs, eN, C.N - NT + k, st.px, st.py,
                                                       st.vx, st.vy, L.pr.radius, L.ddv, tfx[k],
                                                       tfy[k], ocs, opos))
                        omt |= 1u << ((C.N - NT + k) & 31);
                }
                lom[64 + L.lane] = omt;
                if (C.collisions) {
                    const T *lx = sl + F_PX * 64, *ly = sl + F_PY * 64;
                    const T *lvx = sl + F_VX * 64, *lvy = sl + F_VY * 64;
                    if (s == 0 || !ok) {
                        M cd;
                        incl = scan_all<T, PA>(lx, ly, L.base, C.A, L.agent, st.px, st.py, C.t_nbr,
                                               C.t_skin, cd);
                        if (s == 0) cand = cd;
                    } else {
                        incl = scan_cand<T, PA>(lx, ly, L.base, st.px, st.py, C.t_nbr, cand);
                    }
                    if (g.nmask && L.active)
                        ((M *)g.nmask)[((size_t)t * C.S + s) * EA + L.idx] = incl;
                    M m = cap_list(incl, C.K);
                    const T ra = L.pr.radius;
                    while (m) {
                        const int b = m_ctz(m);
                        m &= m - 1;
                        const int j = L.base + b;
                        T gx, gy;
                        pair_force(C, st.px - lx[j], st.py - ly[j], st.vx - lvx[j], st.vy - lvy[j],
                                   ra + lr[j] + C.margin, L.ddv, gx, gy);
                        fx += gx;
                        fy += gy;
                    }
                }
                if (C.soft_walls) {
                    unsigned wb;
                    wall_force_axes(C, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, wx, wy, wb);
                }
            }
            __syncthreads();  // the obstacle sums are in lso, the contact masks in lom
            if (!agent_wave && g.omask && L.active)
                omask_put(g.omask, C.N, ((size_t)t * C.S + s) * EA + L.idx,
                          lom[L.lane] | lom[64 + L.lane]);
            if (agent_wave) {
                T sx = lso[L.lane], sy = lso[64 + L.lane];
#pragma unroll
                for (int k = 0; k < SPLIT_TAIL_MAX; ++k)
                    if (k < NT) {
                        sx += tfx[k];
                        sy += tfy[k];
                    }
                if (C.soft_walls) {
                    sx += wx;
                    sy += wy;
                }
                const T Fx = fx + sx, Fy = fy + sy;
                if (g.fsum && L.active) {
                    T *const o2 = g.fsum + 2 * (((size_t)t * C.S + s) * EA + L.idx);
                    o2[0] = Fx;
                    o2[1] = Fy;
                }
                St<T> nx;
                integrate<T, false>(C, L.pr, st, a, Fx, Fy, nx);
                if (C.use_skin) {
                    D += (m_abs(nx.px - st.px) + m_abs(nx.py - st.py)) * T(1.0001);
                    ok = env_all<PA>(!L.real || D <= C.half_margin, L.base);
                }
                st = nx;
            }
        }
        asm volatile("" ::"v"(an[0]), "v"(an[1]), "v"(an[2]), "v"(an[3]));
        if (agent_wave && L.active) {
            if (t + 1 < g.nsteps)
                store_state<T, false>(g.traj.f, (size_t)t * EA + L.idx, st);
            else
                store_state<T, false>(g.fin.f, L.idx, st);
        }
        for (int k = 0; k < 4; ++k) a[k] = an[k];
    }
}

// Reverse pass of one substep's box contacts, as one wave-wide work list.  Lane a's items
// are its force-exerting box pairs (ascending neighbour), then for a box agent its
// force-exerting obstacles (ascending index) and walls -- or, when an obstacle past the
// 64th exerts a force, one item for all its static contacts.  The wave evaluates the
// items one per lane, 64 at a time (the owner of item q found by binary search over the
// item offsets), and each lane adds its own items' results in item order.  A per-lane
// loop would run one dual evaluation for the whole wave per list position, obstacle and
// wall that any lane needs.
// `sl`: the substep's slot (force rows holding force adjoint / damping denominator),
// `lcs`: its heading cos / sin rows, `lmask_s` its list masks; this lane's force-exerting
// box pairs `imask`, obstacles `om` and flags `wf` (1 walls, 2 a later obstacle).
template <typename T, int PA>
__device__ __forceinline__ void box_rounds(const Cst<T> &C, const Args<T> &g,
                                           const Lane<T, PA> &L, const T *sl, const T *lr,
                                           const T *ldd, const T *lbx, const T *lcs,
                                           const typename MaskT<PA>::type *lmask_s,
                                           const T *ocs_base, typename MaskT<PA>::type imask,
                                           uint64_t om, unsigned wf, T gFx, T gFy, St<T> &gi)
{
    typedef typename MaskT<PA>::type M;
    __shared__ int pre[64];
    __shared__ M imk[64];
    __shared__ uint64_t iom[64];
    __shared__ unsigned char iwf[64];
    __shared__ T gfr[2 * 64];
    __shared__ T res[6 * 64];
    const int lane = L.lane;
    if (wf & 2u) om = 0;  // one item for every static contact
    const int n = m_popc(imask) + __builtin_popcountll(om) + ((wf & 3u) ? 1 : 0);
    int x = n;  // inclusive prefix sum of the item counts over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    const int start = x - n;
    const int total = __shfl(x, 63, 64);
    if (total == 0) return;
    pre[lane] = start;
    imk[lane] = imask;
    iom[lane] = om;
    iwf[lane] = (unsigned char)wf;
    gfr[lane] = gFx;
    gfr[64 + lane] = gFy;
    wave_lds_sync();
    for (int r = 0; r < total; r += 64) {
        const int q = r + lane;
        if (q < total) {
            int lo = 0, hi = 63;  // the last lane whose first item is <= q owns it
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (pre[mid] <= q) lo = mid;
                else hi = mid - 1;
            }
            const int a = lo, ag = a % PA, base = a - ag;
            int k = q - pre[a];
            St<T> ins;
            slot_get<T, false>(sl, a, ins);
            const Foot<T> fa = {lbx[a], lr[a], lbx[64 + a], lbx[128 + a]};
            const int env = blockIdx.x * (64 / PA) + a / PA;
            const size_t eN = (size_t)(env < C.E ? env : 0) * C.N;
            const T *ocs_a = ocs_base ? ocs_base + 2 * (a / PA) * C.N : nullptr;
            M mk = imk[a];
            uint64_t mo = iom[a];
            const int np = m_popc(mk), no = __builtin_popcountll(mo);
            int kind, b = 0, o = 0, j = base;
            T wx, wy, dd;
            if (k < np) {
                kind = BI_PAIR;
                for (; k > 0; --k) mk &= mk - 1;
                b = m_ctz(mk);
                j = base + b;
                const bool own = in_list(lmask_s[a], b, C.K);
                const bool rev = in_list(lmask_s[j], ag, C.K);
                wx = (own ? sl[F_FX * 64 + a] : T(0)) - (rev ? sl[F_FX * 64 + j] : T(0));
                wy = (own ? sl[F_FY * 64 + a] : T(0)) - (rev ? sl[F_FY * 64 + j] : T(0));
                dd = T(1);
            } else {
                k -= np;
                if (k < no) {
                    kind = BI_OBST;
                    for (; k > 0; --k) mo &= mo - 1;
                    o = __builtin_ctzll(mo);
                } else {
                    kind = (iwf[a] & 2u) ? BI_FULL : BI_WALL;
                }
                wx = gfr[a];
                wy = gfr[64 + a];
                dd = ldd[a];
            }
            const Foot<T> fb = {lbx[j], lr[j], lbx[64 + j], lbx[128 + j]};
            const T ob[6] = {sl[F_PX * 64 + j], sl[F_PY * 64 + j], sl[F_TH * 64 + j],
                             sl[F_VX * 64 + j], sl[F_VY * 64 + j], sl[F_W * 64 + j]};
            St<T> acc;
            st_zero(acc);
            box_item_adj(C, g.obs, eN, ocs_a, kind, ag, fa, ins, b, fb, ob, lcs[j], lcs[64 + j], o,
                         dd, wx, wy, acc);
            res[lane] = acc.px;
            res[64 + lane] = acc.py;
            res[128 + lane] = acc.th;
            res[192 + lane] = acc.vx;
            res[256 + lane] = acc.vy;
            res[320 + lane] = acc.w;
        }
        wave_lds_sync();
        const int q0 = start > r ? start : r, q1 = min(start + n, r + 64);
        for (int c = q0 - r; c < q1 - r; ++c) {
            gi.px += res[c];
            gi.py += res[64 + c];
            gi.th += res[128 + c];
            gi.vx += res[192 + c];
            gi.vy += res[256 + c];
            gi.w += res[320 + c];
        }
        wave_lds_sync();
    }
}

template <typename T, int PA, bool DRONE, bool BOXES, unsigned F>
__global__ __launch_bounds__(64) void k_rollout_bwd(const Cst<T> Cin, const Args<T> g)
{
    const Cst<T> C = fold_cst<F>(Cin);
    typedef typename MaskT<PA>::type M;
    constexpr int NF = DRONE ? NF_DRONE : NF_2D;
    extern __shared__ __align__(16) unsigned char smem[];
    T *lr = (T *)smem;          // radius per lane
    T *ldd = lr + 64;           // damping denominator per lane
    T *slots = ldd + 64;        // S slots of NF fields
    M *lmask = (M *)(slots + (size_t)C.S * NF * 64);  // S inclusion masks per lane
    // worlds without box agents, with the obstacle-contact tape: S contact masks per lane
    uint32_t *lomk = (uint32_t *)(lmask + (size_t)C.S * 64);
    // box worlds, per substep: the masks of force-exerting box pairs, the cos / sin of
    // every lane's heading, a box agent's force-exerting obstacles (first 64) and flags
    // (1: a wall exerts a force, 2: a later obstacle does)
    M *lact = lmask + (size_t)C.S * 64;
    T *lcsb = (T *)(lact + (size_t)C.S * 64);
    uint64_t *lom = (uint64_t *)(lcsb + (size_t)C.S * 128);
    unsigned char *lwf = (unsigned char *)(lom + (size_t)C.S * 64);
    __shared__ T ocs_lds[2 * OCS_MAX];
    __shared__ T lbx[3 * 64];  // footprint per lane: shape, hx, hy (box worlds)
    Lane<T, PA> L;
    lane_init<T, PA>(C, g, L);
    fold_prm<F>(L.pr);
    lr[L.lane] = L.pr.radius;
    lbx[L.lane] = L.pr.shape;
    lbx[64 + L.lane] = L.pr.hx;
    lbx[128 + L.lane] = L.pr.hy;
    ldd[L.lane] = L.dd;
    const T *ocs = ob_trig_table<T, PA>(C, g, L, ocs_lds);
    const size_t EA = (size_t)C.E * C.A;
    St<T> gs;  // adjoint of the current step's output
    st_zero(gs);
    // the trajectory and trajectory-adjoint field pointers the step loop reads, in vector
    // registers (see vgpr_ptr)
    const SWARP_GLOBAL T *trf[9], *atf[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        trf[k] = vgpr_ptr(g.traj.f[k]);
        atf[k] = vgpr_ptr(g.atraj.f[k]);
    }
    for (int t = g.nsteps - 1; t >= 0; --t) {
        progress_priority(g.nsteps - 1 - t, g.nsteps);
        if (t == g.nsteps - 1)
            add_adj<T, DRONE>(g.afin.f, L.idx, gs);
        else
            add_adj<T, DRONE>(atf, (size_t)t * EA + L.idx, gs);
        St<T> st;
        if (t == 0)
            load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
        else
            load_state<T, DRONE>(trf, L.idx, (size_t)(t - 1) * EA, st);
        T a[4];
        load_act(g.act, (size_t)t * EA + L.idx, C.ad, a);
        if (!L.real) st.px = st.py = __builtin_nan("");

        // ---- recompute the substep chain of this step into LDS
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            T *sl = slots + (size_t)s * NF * 64;
            wave_lds_sync();
            slot_put<T, DRONE>(sl, L.lane, st);
            if (BOXES) {
                lcsb[s * 128 + L.lane] = m_cos(st.th);
                lcsb[s * 128 + 64 + L.lane] = m_sin(st.th);
            }
            wave_lds_sync();
            T Fx = T(0), Fy = T(0);
            M incl = 0;
            if (C.needs_forces) {
                M am = 0;
                uint64_t om = 0;
                bool wl = false, far = false;
                const T *fsum =
                    !BOXES && g.fsum ? g.fsum + 2 * (((size_t)t * C.S + s) * EA + L.idx) : nullptr;
                if (!BOXES && g.omask)
                    lomk[s * 64 + L.lane] =
                        L.active ? omask_get(g.omask, C.N, ((size_t)t * C.S + s) * EA + L.idx) : 0u;
                if (!BOXES && fsum && g.nmask) {
                    // the forward's force and lists (the same bits): no force pass at all
                    Fx = fsum[0];
                    Fy = fsum[1];
                    incl = L.active && C.collisions
                               ? ((const M *)g.nmask)[((size_t)t * C.S + s) * EA + L.idx]
                               : M(0);
                } else {
                    incl = forces<T, PA, BOXES>(C, g, L, sl, lr, st, s, s == 0 || !ok, cand, Fx,
                                                Fy, ocs, lbx, lcsb + s * 128, &am, &om, &wl, &far,
                                                nullptr, fsum);
                }
                if (BOXES) {
                    lact[s * 64 + L.lane] = am;
                    lom[s * 64 + L.lane] = om;
                    lwf[s * 64 + L.lane] = (wl ? 1 : 0) | (far ? 2 : 0);
                }
            }
            sl[F_FX * 64 + L.lane] = Fx;
            sl[F_FY * 64 + L.lane] = Fy;
            lmask[s * 64 + L.lane] = incl;
            // the reverse pass reads each substep's input and force; the last substep's
            // output is the step's checkpoint and is not needed here
            if (s + 1 < C.S) {
                St<T> nx;
                integrate<T, DRONE>(C, L.pr, st, a, Fx, Fy, nx);
                if (C.use_skin) {
                    D += (m_abs(nx.px - st.px) + m_abs(nx.py - st.py)) * T(1.0001);
                    ok = env_all<PA>(!L.real || D <= C.half_margin, L.base);
                }
                st = nx;
            }
        }

        // ---- reverse pass
        T ga[4] = {T(0), T(0), T(0), T(0)};
        for (int s = C.S - 1; s >= 0; --s) {
            T *sl = slots + (size_t)s * NF * 64;
            wave_lds_sync();
            St<T> in;
            slot_get<T, DRONE>(sl, L.lane, in);
            const T Fx = sl[F_FX * 64 + L.lane], Fy = sl[F_FY * 64 + L.lane];
            St<T> gi;
            T gFx, gFy;
            integrate_adj<T, DRONE>(C, L.pr, in, a, Fx, Fy, gs, gi, ga, gFx, gFy);
            if (C.needs_forces) {
                // the slot now carries the force adjoint divided by the damping denominator
                const T wFx = gFx * L.inv_dd, wFy = gFy * L.inv_dd;
                wave_lds_sync();
                sl[F_FX * 64 + L.lane] = wFx;
                sl[F_FY * 64 + L.lane] = wFy;
                wave_lds_sync();
                M imask = 0;  // force-exerting box pairs, reversed in box_rounds
                if (C.collisions) {
                    const T *lx = sl + F_PX * 64, *ly = sl + F_PY * 64;
                    const T *lvx = sl + F_VX * 64, *lvy = sl + F_VY * 64;
                    const T *lgx = sl + F_FX * 64, *lgy = sl + F_FY * 64;
                    const M mine = lmask[s * 64 + L.lane];
                    M m = mine;
                    while (m) {
                        const int b = m_ctz(m);
                        m &= m - 1;
                        const int j = L.base + b;
                        const bool own = in_list(mine, b, C.K);
                        const bool rev = in_list(lmask[s * 64 + j], L.agent, C.K);
                        if (!own && !rev) continue;
                        if (BOXES && (L.pr.shape > T(0.5) || lbx[j] > T(0.5))) {
                            // one contact seen from both sides: it exerts a force, or
                            // every derivative of it is zero
                            const bool on = own ? ((lact[s * 64 + L.lane] >> b) & M(1)) != 0
                                                : ((lact[s * 64 + j] >> L.agent) & M(1)) != 0;
                            if (on) imask |= M(1) << b;
                            continue;
                        }
                        const T wx = (own ? wFx : T(0)) - (rev ? lgx[j] : T(0));
                        const T wy = (own ? wFy : T(0)) - (rev ? lgy[j] : T(0));
                        pair_adj_combined(C, in.px - lx[j], in.py - ly[j], in.vx - lvx[j],
                                          in.vy - lvy[j], L.pr.radius + lr[j] + C.margin, wx, wy,
                                          gi.px, gi.py, gi.vx, gi.vy);
                    }
                }
                if (BOXES) {
                    const bool bx = L.pr.shape > T(0.5);
                    box_rounds<T, PA>(C, g, L, sl, lr, ldd, lbx, lcsb + s * 128, lmask + s * 64,
                                      ocs ? ocs_lds : nullptr, imask,
                                      bx ? lom[s * 64 + L.lane] : 0ull,
                                      bx ? lwf[s * 64 + L.lane] : 0, gFx, gFy, gi);
                }
                if (BOXES && L.pr.shape > T(0.5)) {
                    // a box agent's static contacts were reversed in box_rounds
                } else {
                    if (C.N > 0) {
                        const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
                        if (!BOXES && g.omask) {
                            // the obstacles in contact at this substep, in index order
                            uint32_t m = lomk[s * 64 + L.lane];
                            while (m) {
                                const int o = __builtin_ctz(m);
                                m &= m - 1;
                                obstacle_force_adj(C, g.obs, eN, o, in.px, in.py, in.vx, in.vy,
                                                   L.pr.radius, L.dd, gFx, gFy, gi, ocs);
                            }
                        } else {
                            for (int o = 0; o < C.N; ++o)
                                obstacle_force_adj(C, g.obs, eN, o, in.px, in.py, in.vx, in.vy,
                                                   L.pr.radius, L.dd, gFx, gFy, gi, ocs);
                        }
                    }
                    if (C.soft_walls)
                        wall_force_adj(C, in.px, in.py, in.vx, in.vy, L.pr.radius, L.dd, gFx,
                                       gFy, gi);
                }
            }
            gs = gi;
        }
        if (L.active) {
            T *pa = g.aact + ((size_t)t * EA + L.idx) * C.ad;
            for (int k = 0; k < C.ad; ++k) pa[k] = k < 4 ? ga[k] : T(0);
        }
    }
    if (L.active) store_adj<T, DRONE>(g.a0.f, L.idx, gs);
}

// ---------------------------------------------------------------------- launchers

#define SWARP_DISPATCH_PA(PA_, KERNEL, ...)                                        \
    switch (PA_) {                                                                 \
    case 4: hipLaunchKernelGGL((KERNEL<T, 4, __VA_ARGS__>), grid4, dim3(64), shm, st, C, a); break; \
    case 8: hipLaunchKernelGGL((KERNEL<T, 8, __VA_ARGS__>), grid8, dim3(64), shm, st, C, a); break; \
    case 16: hipLaunchKernelGGL((KERNEL<T, 16, __VA_ARGS__>), grid16, dim3(64), shm, st, C, a); break; \
    case 32: hipLaunchKernelGGL((KERNEL<T, 32, __VA_ARGS__>), grid32, dim3(64), shm, st, C, a); break; \
    default: hipLaunchKernelGGL((KERNEL<T, 64, __VA_ARGS__>), grid64, dim3(64), shm, st, C, a); break; \
    }

// The profile besides FT_ALL each (DRONE, BOXES) family compiles for float32 (0: none).
template <typename T, bool DRONE, bool BOXES> constexpr unsigned family_profile()
{
    return sizeof(T) != 4 || BOXES ? 0u : (DRONE ? FT_PROF_DRONE : FT_PROF_2D);
}

// feat: the FT_* paths the world uses; the family's profile runs when it covers them.
template <typename T, bool DRONE, bool BOXES>
void launch_fwd(int PA, const Cst<T> &C, const Args<T> &a, unsigned feat, hipStream_t st)
{
    const size_t shm = 0;
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    constexpr unsigned P = family_profile<T, DRONE, BOXES>();
    if (!DRONE && !BOXES && P != 0u && (feat & ~P) == 0u && (feat & FT_OBST) && C.N > 0 &&
        (64 / PA) * C.N <= OCS_MAX) {
        // static obstacles (whose per-launch tables fit): the obstacle pass on a wave of its own
        constexpr unsigned PS = P ? P : FT_ALL;
        switch (PA) {
        case 4: hipLaunchKernelGGL((k_rollout_fwd_split<T, 4, PS>), grid4, dim3(128), 0, st, C, a); break;
        case 8: hipLaunchKernelGGL((k_rollout_fwd_split<T, 8, PS>), grid8, dim3(128), 0, st, C, a); break;
        case 16: hipLaunchKernelGGL((k_rollout_fwd_split<T, 16, PS>), grid16, dim3(128), 0, st, C, a); break;
        case 32: hipLaunchKernelGGL((k_rollout_fwd_split<T, 32, PS>), grid32, dim3(128), 0, st, C, a); break;
        default: hipLaunchKernelGGL((k_rollout_fwd_split<T, 64, PS>), grid64, dim3(128), 0, st, C, a); break;
        }
        return;
    }
    if (P != 0u && (feat & ~P) == 0u) {
        SWARP_DISPATCH_PA(PA, k_rollout_fwd, DRONE, BOXES, P ? P : FT_ALL)
    } else {
        SWARP_DISPATCH_PA(PA, k_rollout_fwd, DRONE, BOXES, FT_ALL)
    }
}

template <typename T, bool DRONE, bool BOXES>
void launch_bwd(int PA, const Cst<T> &C, const Args<T> &a, unsigned feat, size_t shm,
                hipStream_t st)
{
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    constexpr unsigned P = family_profile<T, DRONE, BOXES>();
    if (P != 0u && (feat & ~P) == 0u) {
        SWARP_DISPATCH_PA(PA, k_rollout_bwd, DRONE, BOXES, P ? P : FT_ALL)
    } else {
        SWARP_DISPATCH_PA(PA, k_rollout_bwd, DRONE, BOXES, FT_ALL)
    }
}

#undef SWARP_DISPATCH_PA

}  // namespace swarp
