// swarp_hip.hip -- gfx950 kernels and C ABI of the swarp physics step (include/swarp_hip.h).
//
// Execution model
//   * One lane per (env, agent).  An env occupies PA consecutive lanes of a wave64
//     (PA = next power of two >= n_agents, <= 64), so an env never spans waves and
//     every exchange between its agents stays inside one wave: positions, velocities,
//     neighbour masks and force adjoints go through a small LDS staging area.
//   * Workgroup = one wave (64 lanes), so the workgroup barrier costs nothing and
//     envs are spread over the whole chip at wave granularity.
//   * One launch runs a whole T-step rollout: the state stays in registers between
//     steps; HBM sees the actions in and each step's output state (the checkpoint).
//   * The backward launch walks t = T-1..0, reloads each step's input checkpoint,
//     recomputes that step's substeps into LDS, then runs the reverse pass.  The force
//     adjoint of a pair is gathered by both agents from the same recomputed pair, in
//     ascending neighbour order: deterministic, no atomics.
//   * Neighbour membership uses the exact threshold test d2 <= t_nbr, where t_nbr is
//     the largest value whose correctly rounded square root is <= the radius, which
//     is bit-identical to the reference's sqrt(d2) <= radius (neighbors.py:91).
//     Within a step, substeps after the first scan only a skin list built at substep 0;
//     a per-env displacement bound proves the skin list complete, and an env whose
//     agents moved too far rescans all pairs.  Both give the same lists.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "physics.hpp"
#include "boxes.hpp"
#include "swarp_hip.h"

namespace swarp {

template <int PA> struct MaskT { typedef uint32_t type; };
template <> struct MaskT<64> { typedef uint64_t type; };

__device__ __forceinline__ int m_ctz(uint32_t m) { return __builtin_ctz(m); }
__device__ __forceinline__ int m_ctz(uint64_t m) { return __builtin_ctzll(m); }
__device__ __forceinline__ int m_popc(uint32_t m) { return __builtin_popcount(m); }
__device__ __forceinline__ int m_popc(uint64_t m) { return __builtin_popcountll(m); }

// Field pointers of one state; strides (in scalars) 2,1,2,1,1,1,1,4,3.
template <typename T> struct Fields {
    T *f[9];
};
template <typename T> struct CFields {
    const T *f[9];
};

template <typename T> struct Args {
    const T *params;
    const int32_t *tag, *mode;
    Obs<T> obs;
    CFields<T> s0;       // rollout input state
    const T *act;        // [T,E,A,ad]
    Fields<T> traj;      // outputs of steps 0..T-2 (stride E*A per step)
    Fields<T> fin;       // output of step T-1
    CFields<T> atraj;    // adjoints arriving at traj (nullable per field)
    CFields<T> afin;     // adjoint arriving at fin (nullable per field)
    Fields<T> a0;        // adjoint of s0 (nullable per field)
    T *aact;             // adjoint of actions
    int nsteps;
};

__device__ __forceinline__ int fstride(int k)
{
    // pos theta vel speed ang_vel z vz attitude body_rates
    return k == 0 || k == 2 ? 2 : (k == 7 ? 4 : (k == 8 ? 3 : 1));
}

template <typename T, bool DRONE>
__device__ __forceinline__ void load_state(const T *const *f, size_t i, size_t off, St<T> &s)
{
    // `off` = element offset of the state in the trajectory (step * E * A)
    const size_t j = i + off;
    s.px = f[0][2 * j]; s.py = f[0][2 * j + 1];
    s.th = f[1][j];
    s.vx = f[2][2 * j]; s.vy = f[2][2 * j + 1];
    s.s = f[3][j];
    s.w = f[4][j];
    if (DRONE) {
        s.z = f[5][j]; s.vz = f[6][j];
        s.qx = f[7][4 * j]; s.qy = f[7][4 * j + 1]; s.qz = f[7][4 * j + 2]; s.qw = f[7][4 * j + 3];
        s.bx = f[8][3 * j]; s.by = f[8][3 * j + 1]; s.bz = f[8][3 * j + 2];
    } else {
        s.z = s.vz = s.qx = s.qy = s.qz = s.bx = s.by = s.bz = T(0);
        s.qw = T(1);
    }
}

template <typename T, bool DRONE>
__device__ __forceinline__ void store_state(T *const *f, size_t j, const St<T> &s)
{
    f[0][2 * j] = s.px; f[0][2 * j + 1] = s.py;
    f[1][j] = s.th;
    f[2][2 * j] = s.vx; f[2][2 * j + 1] = s.vy;
    f[3][j] = s.s;
    f[4][j] = s.w;
    if (DRONE) {
        f[5][j] = s.z; f[6][j] = s.vz;
        f[7][4 * j] = s.qx; f[7][4 * j + 1] = s.qy; f[7][4 * j + 2] = s.qz; f[7][4 * j + 3] = s.qw;
        f[8][3 * j] = s.bx; f[8][3 * j + 1] = s.by; f[8][3 * j + 2] = s.bz;
    }
}

// Adds a nullable adjoint state (fields may be NULL) at element j.
template <typename T, bool DRONE>
__device__ __forceinline__ void add_adj(const T *const *f, size_t j, St<T> &g)
{
    if (f[0]) { g.px += f[0][2 * j]; g.py += f[0][2 * j + 1]; }
    if (f[1]) g.th += f[1][j];
    if (f[2]) { g.vx += f[2][2 * j]; g.vy += f[2][2 * j + 1]; }
    if (f[3]) g.s += f[3][j];
    if (f[4]) g.w += f[4][j];
    if (DRONE) {
        if (f[5]) g.z += f[5][j];
        if (f[6]) g.vz += f[6][j];
        if (f[7]) { g.qx += f[7][4 * j]; g.qy += f[7][4 * j + 1]; g.qz += f[7][4 * j + 2]; g.qw += f[7][4 * j + 3]; }
        if (f[8]) { g.bx += f[8][3 * j]; g.by += f[8][3 * j + 1]; g.bz += f[8][3 * j + 2]; }
    }
}

template <typename T, bool DRONE>
__device__ __forceinline__ void store_adj(T *const *f, size_t j, const St<T> &g)
{
    if (f[0]) { f[0][2 * j] = g.px; f[0][2 * j + 1] = g.py; }
    if (f[1]) f[1][j] = g.th;
    if (f[2]) { f[2][2 * j] = g.vx; f[2][2 * j + 1] = g.vy; }
    if (f[3]) f[3][j] = g.s;
    if (f[4]) f[4][j] = g.w;
    if (DRONE) {
        if (f[5]) f[5][j] = g.z;
        if (f[6]) f[6][j] = g.vz;
        if (f[7]) { f[7][4 * j] = g.qx; f[7][4 * j + 1] = g.qy; f[7][4 * j + 2] = g.qz; f[7][4 * j + 3] = g.qw; }
        if (f[8]) { f[8][3 * j] = g.bx; f[8][3 * j + 1] = g.by; f[8][3 * j + 2] = g.bz; }
    }
}

template <typename T>
__device__ __forceinline__ void load_prm(const Args<T> &g, size_t row, int a, Prm<T> &p)
{
    const T *r = g.params + row * 22;
    p.radius = r[0]; p.mass = r[1]; p.max_speed = r[2]; p.max_accel = r[3];
    p.max_ang_vel = r[4]; p.max_ang_accel = r[5]; p.l_f = r[6]; p.l_r = r[7];
    p.max_steer = r[8]; p.thrust_max = r[9]; p.arm = r[10]; p.ixx = r[11];
    p.iyy = r[12]; p.izz = r[13]; p.kappa = r[14]; p.gravity = r[15]; p.min_speed = r[16];
    p.shape = r[17]; p.hx = r[18]; p.hy = r[19];
    p.gain_v = r[20]; p.gain_w = r[21];
    p.tag = g.tag[a];
    p.mode = g.mode[a];
}

template <typename T>
__device__ __forceinline__ void load_act(const T *act, size_t j, int ad, T (&a)[4])
{
    const T *p = act + j * ad;
    a[0] = p[0];
    a[1] = ad > 1 ? p[1] : T(0);
    a[2] = ad > 2 ? p[2] : T(0);
    a[3] = ad > 3 ? p[3] : T(0);
}

// LDS staging of one substep.  Fields: 0 px, 1 py, 2 vx, 3 vy, 4 th, 5 s, 6 w, 7 Fx, 8 Fy,
// then (drone) 9 z, 10 vz, 11..14 q, 15..17 br.  Each field is 64 consecutive scalars.
constexpr int F_PX = 0, F_PY = 1, F_VX = 2, F_VY = 3, F_TH = 4, F_S = 5, F_W = 6, F_FX = 7,
              F_FY = 8, NF_2D = 9, NF_DRONE = 18;

// Neighbour lists of one agent as a bitmask over the env's agents, ascending bit =
// ascending list order (neighbors.py:90-96).  Full scan over every pair of the env.
template <typename T, int PA>
__device__ __forceinline__ typename MaskT<PA>::type scan_all(const T *lx, const T *ly, int base,
                                                             int A, int me, T px, T py, T t_nbr,
                                                             T t_skin,
                                                             typename MaskT<PA>::type &cand)
{
    typedef typename MaskT<PA>::type M;
    M incl = 0, cd = 0;
    (void)A;  // pad slots (b >= A) hold NaN positions and never pass the test
#pragma unroll
    for (int b = 0; b < PA; ++b) {
        T dx = lx[base + b] - px, dy = ly[base + b] - py;
        T d2 = dx * dx + dy * dy;
        incl |= d2 <= t_nbr ? (M(1) << b) : M(0);
        cd |= d2 <= t_skin ? (M(1) << b) : M(0);
    }
    const M self = ~(M(1) << me);
    cand = cd & self;
    return incl & self;
}

// Same membership, evaluated only on the skin candidates.
template <typename T, int PA>
__device__ __forceinline__ typename MaskT<PA>::type scan_cand(const T *lx, const T *ly, int base,
                                                              T px, T py, T t_nbr,
                                                              typename MaskT<PA>::type cand)
{
    typedef typename MaskT<PA>::type M;
    M incl = 0;
    while (cand) {
        const int b = m_ctz(cand);
        cand &= cand - 1;
        T dx = lx[base + b] - px, dy = ly[base + b] - py;
        T d2 = dx * dx + dy * dy;
        incl |= d2 <= t_nbr ? (M(1) << b) : M(0);
    }
    return incl;
}

// First K members of an inclusion mask (the padded list of length K).
template <typename M> __device__ __forceinline__ M cap_list(M incl, int K)
{
    if (m_popc(incl) <= K) return incl;
    M rest = incl;
    for (int i = 0; i < K; ++i) rest &= rest - 1;
    return incl ^ rest;
}

// Per-lane context shared by the forward and backward kernels.
template <typename T, int PA> struct Lane {
    int lane, agent, base, env;
    bool real;     // agent < A (lane holds a real agent slot of its env)
    bool active;   // real and env < E
    size_t idx;    // env * A + agent (clamped to a valid element for inactive lanes)
    Prm<T> pr;
    T dd;          // implicit damping denominator 1 + c*sub_dt/m (collisions.py:845)
    T inv_dd;      // 1 / dd (adjoint arithmetic only)
    Dv<T> ddv;     // dd as a prepared divisor (exact fp32 division by dd)
};

template <typename T, int PA>
__device__ __forceinline__ void lane_init(const Cst<T> &C, const Args<T> &g, Lane<T, PA> &L)
{
    constexpr int EPW = 64 / PA;
    L.lane = threadIdx.x;
    L.agent = L.lane % PA;
    L.base = L.lane - L.agent;
    L.env = blockIdx.x * EPW + L.lane / PA;
    L.real = L.agent < C.A;
    L.active = L.real && L.env < C.E;
    const int ag = L.real ? L.agent : 0;
    const int ev = L.env < C.E ? L.env : 0;
    L.idx = (size_t)ev * C.A + ag;
    // per-env parameter tables (Stepper.set_agent_params_per_env) index [env, agent]
    load_prm(g, C.per_env ? (size_t)ev * C.A + ag : (size_t)ag, ag, L.pr);
    L.dd = T(1) + C.c * C.sub_dt / L.pr.mass;
    L.inv_dd = T(1) / L.dd;
    L.ddv = divisor(L.dd, true);
}

// Whether every real agent of this lane's env stayed within the skin budget.
template <int PA> __device__ __forceinline__ bool env_all(bool ok, int base)
{
    const uint64_t bal = __ballot(ok);
    const uint64_t full = PA == 64 ? ~0ull : ((1ull << PA) - 1ull);
    return ((bal >> base) & full) == full;
}

// Contact + static forces of one substep, reading the env's positions/velocities from
// the LDS slot `sl`.  Returns the uncapped inclusion mask (for the true count).
// Obstacle angles as (cos, sin) per env slot of the wave, filled once per launch when
// 64/PA envs x N obstacles fit (OCS_MAX pairs); NULL table otherwise.
constexpr int OCS_MAX = 256;

template <typename T, int PA>
__device__ __forceinline__ const T *ob_trig_table(const Cst<T> &C, const Args<T> &g,
                                                  const Lane<T, PA> &L, T *ocs)
{
    if (C.N <= 0 || (64 / PA) * C.N > OCS_MAX) return nullptr;
    const int ew = L.lane / PA;
    const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
    for (int q = L.agent; q < C.N; q += PA) {
        const T ang = g.obs.ang[eN + q];
        ocs[2 * (ew * C.N + q)] = m_cos(ang);
        ocs[2 * (ew * C.N + q) + 1] = m_sin(ang);
    }
    __syncthreads();
    return ocs + 2 * ew * C.N;
}

// Box worlds (BOXES; false compiles the box paths out): `lbx` holds per lane the
// footprint (shape, hx, hy rows of 64), `lcs` the cos and sin of every lane's heading
// (rows of 64), and the slot `sl` also carries the headings and spins (F_TH, F_W rows).
// `act` (nullable) receives the mask of listed neighbours whose box contact exerts a
// force; for a box agent `om` / `wall` / `beyond` which of its first 64 obstacles, its
// walls, and any later obstacle do: the contacts without force have zero derivatives.
template <typename T, int PA, bool BOXES>
__device__ __forceinline__ typename MaskT<PA>::type forces(
    const Cst<T> &C, const Args<T> &g, const Lane<T, PA> &L, const T *sl, const T *lr,
    const St<T> &st, int s, bool full, typename MaskT<PA>::type &cand, T &Fx, T &Fy,
    const T *ocs = nullptr, const T *lbx = nullptr, const T *lcs = nullptr,
    typename MaskT<PA>::type *act = nullptr, uint64_t *om = nullptr, bool *wall = nullptr,
    bool *beyond = nullptr, T *tq = nullptr)
{
    const bool box_me = BOXES && L.pr.shape > T(0.5);
    T me[6] = {st.px, st.py, st.th, st.vx, st.vy, st.w};
    T cme = T(1), sme = T(0);
    if (BOXES) {
        cme = lcs[L.lane];
        sme = lcs[64 + L.lane];
    }
    typename MaskT<PA>::type am = 0;
    const bool wheel = BOXES && tq != nullptr;  // contact torques (wheel contacts)
    T tau = T(0);
    typedef typename MaskT<PA>::type M;
    const T *lx = sl + F_PX * 64, *ly = sl + F_PY * 64, *lvx = sl + F_VX * 64, *lvy = sl + F_VY * 64;
    M incl = 0;
    T fx = T(0), fy = T(0);
    if (C.collisions) {
        if (full) {
            M cd;
            incl = scan_all<T, PA>(lx, ly, L.base, C.A, L.agent, st.px, st.py, C.t_nbr, C.t_skin, cd);
            if (s == 0) cand = cd;
        } else {
            incl = scan_cand<T, PA>(lx, ly, L.base, st.px, st.py, C.t_nbr, cand);
        }
        M m = cap_list(incl, C.K);
        const T ra = L.pr.radius;
        const Foot<T> fa = {L.pr.shape, ra, L.pr.hx, L.pr.hy};
        const T *lth = sl + F_TH * 64, *lw = sl + F_W * 64;
        while (m) {
            const int b = m_ctz(m);
            m &= m - 1;
            const int j = L.base + b;
            T gx, gy;
            if (BOXES && (box_me || lbx[j] > T(0.5))) {
                // a pair with a box (collision_forces_box_kernel, collisions.py:1044-1052)
                const Foot<T> fb = {lbx[j], lr[j], lbx[64 + j], lbx[128 + j]};
                const T ob[6] = {lx[j], ly[j], lth[j], lvx[j], lvy[j], lw[j]};
                agent_pair_force_box<T, T>(C, L.agent, b, fa, me, cme, sme, fb, ob, lcs[j],
                                           lcs[64 + j], L.dd, gx, gy);
                if (gx != T(0) || gy != T(0)) am |= typename MaskT<PA>::type(1) << b;
                if (wheel)
                    tau += pair_torque(C, L.agent, b, fa, me, cme, sme, fb, ob, lcs[j], lcs[64 + j],
                                       gx, gy);
            } else {
                pair_force(C, st.px - lx[j], st.py - ly[j], st.vx - lvx[j], st.vy - lvy[j],
                           ra + lr[j] + C.margin, L.dd, gx, gy);
            }
            fx += gx;
            fy += gy;
        }
    }
    T sx = T(0), sy = T(0);
    if (box_me) {
        // a box agent's obstacles and walls (_static_forces_shaped, collisions.py:950-996)
        const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
        box_static_forces<T, T>(C, g.obs, eN, ocs, L.pr.hx, L.pr.hy, me, cme, sme, L.dd, sx, sy,
                                om, wall, beyond);
        if (wheel)
            tau = tau + box_static_torque(C, g.obs, eN, ocs, L.pr.hx, L.pr.hy, me, cme, sme, L.dd);
    } else if (C.N > 0) {
        const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
        for (int o = 0; o < C.N; ++o) {
            T gx, gy;
            obstacle_force(C, g.obs, eN, o, st.px, st.py, st.vx, st.vy, L.pr.radius, L.dd, gx, gy,
                           ocs);
            sx += gx;
            sy += gy;
        }
    }
    if (C.soft_walls && !box_me) {
        T gx, gy;
        unsigned wb;
        wall_force_axes(C, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx, gy, wb);
        sx += gx;
        sy += gy;
    }
    Fx = fx + sx;
    Fy = fy + sy;
    if (act) *act = am;
    if (wheel) *tq = tau;
    return incl;
}

// ------------------------------------------------------------------ forward rollout

// BOXES: the box-aware contact pass is compiled in (a world holding box agents); the
// disc-only instances keep the register budget of the disc contact law.
template <typename T, int PA, bool DRONE, bool BOXES>
__global__ __launch_bounds__(64) void k_rollout_fwd(const Cst<T> C, const Args<T> g)
{
    typedef typename MaskT<PA>::type M;
    __shared__ T sl[7 * 64];  // px py vx vy th (s) w of the current substep
    __shared__ T lr[64];      // agent radius per lane
    __shared__ T lbx[3 * 64]; // footprint per lane: shape, hx, hy (box worlds)
    __shared__ T lcs[2 * 64]; // cos, sin of each lane's heading this substep (box worlds)
    __shared__ T ocs_lds[2 * OCS_MAX];
    Lane<T, PA> L;
    lane_init<T, PA>(C, g, L);
    lr[L.lane] = L.pr.radius;
    lbx[L.lane] = L.pr.shape;
    lbx[64 + L.lane] = L.pr.hx;
    lbx[128 + L.lane] = L.pr.hy;
    const T *ocs = ob_trig_table<T, PA>(C, g, L, ocs_lds);
    St<T> st;
    load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
    if (!L.real) st.px = st.py = __builtin_nan("");
    const size_t EA = (size_t)C.E * C.A;
    for (int t = 0; t < g.nsteps; ++t) {
        T a[4];
        load_act(g.act, (size_t)t * EA + L.idx, C.ad, a);
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            T Fx = T(0), Fy = T(0), Tq = T(0);
            if (C.needs_forces) {
                if (C.collisions) {
                    __syncthreads();
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
                    if (!C.collisions) __syncthreads();
                    lcs[L.lane] = m_cos(st.th);
                    lcs[64 + L.lane] = m_sin(st.th);
                }
                if (C.collisions || BOXES) __syncthreads();
                forces<T, PA, BOXES>(C, g, L, sl, lr, st, s, s == 0 || !ok, cand, Fx, Fy, ocs, lbx,
                                     lcs, nullptr, nullptr, nullptr, nullptr,
                                     BOXES && C.wheel ? &Tq : nullptr);
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
        if (L.active) {
            if (t + 1 < g.nsteps)
                store_state<T, DRONE>(g.traj.f, (size_t)t * EA + L.idx, st);
            else
                store_state<T, DRONE>(g.fin.f, L.idx, st);
        }
    }
}

// ----------------------------------------------------------------- backward rollout

template <typename T, bool DRONE>
__device__ __forceinline__ void slot_put(T *sl, int lane, const St<T> &s)
{
    sl[F_PX * 64 + lane] = s.px; sl[F_PY * 64 + lane] = s.py;
    sl[F_VX * 64 + lane] = s.vx; sl[F_VY * 64 + lane] = s.vy;
    sl[F_TH * 64 + lane] = s.th; sl[F_S * 64 + lane] = s.s; sl[F_W * 64 + lane] = s.w;
    if (DRONE) {
        sl[9 * 64 + lane] = s.z; sl[10 * 64 + lane] = s.vz;
        sl[11 * 64 + lane] = s.qx; sl[12 * 64 + lane] = s.qy;
        sl[13 * 64 + lane] = s.qz; sl[14 * 64 + lane] = s.qw;
        sl[15 * 64 + lane] = s.bx; sl[16 * 64 + lane] = s.by; sl[17 * 64 + lane] = s.bz;
    }
}

template <typename T, bool DRONE>
__device__ __forceinline__ void slot_get(const T *sl, int lane, St<T> &s)
{
    s.px = sl[F_PX * 64 + lane]; s.py = sl[F_PY * 64 + lane];
    s.vx = sl[F_VX * 64 + lane]; s.vy = sl[F_VY * 64 + lane];
    s.th = sl[F_TH * 64 + lane]; s.s = sl[F_S * 64 + lane]; s.w = sl[F_W * 64 + lane];
    if (DRONE) {
        s.z = sl[9 * 64 + lane]; s.vz = sl[10 * 64 + lane];
        s.qx = sl[11 * 64 + lane]; s.qy = sl[12 * 64 + lane];
        s.qz = sl[13 * 64 + lane]; s.qw = sl[14 * 64 + lane];
        s.bx = sl[15 * 64 + lane]; s.by = sl[16 * 64 + lane]; s.bz = sl[17 * 64 + lane];
    } else {
        s.z = s.vz = s.qx = s.qy = s.qz = s.bx = s.by = s.bz = T(0);
        s.qw = T(1);
    }
}

// Whether agent `me` is among the first K members of inclusion mask `incl`.
template <typename M> __device__ __forceinline__ bool in_list(M incl, int me, int K)
{
    return ((incl >> me) & M(1)) && m_popc(incl & ((M(1) << me) - M(1))) < K;
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
    __syncthreads();
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
        __syncthreads();
        const int q0 = start > r ? start : r, q1 = min(start + n, r + 64);
        for (int c = q0 - r; c < q1 - r; ++c) {
            gi.px += res[c];
            gi.py += res[64 + c];
            gi.th += res[128 + c];
            gi.vx += res[192 + c];
            gi.vy += res[256 + c];
            gi.w += res[320 + c];
        }
        __syncthreads();
    }
}

template <typename T, int PA, bool DRONE, bool BOXES>
__global__ __launch_bounds__(64) void k_rollout_bwd(const Cst<T> C, const Args<T> g)
{
    typedef typename MaskT<PA>::type M;
    constexpr int NF = DRONE ? NF_DRONE : NF_2D;
    extern __shared__ __align__(16) unsigned char smem[];
    T *lr = (T *)smem;          // radius per lane
    T *ldd = lr + 64;           // damping denominator per lane
    T *slots = ldd + 64;        // S slots of NF fields
    M *lmask = (M *)(slots + (size_t)C.S * NF * 64);  // S inclusion masks per lane
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
    lr[L.lane] = L.pr.radius;
    lbx[L.lane] = L.pr.shape;
    lbx[64 + L.lane] = L.pr.hx;
    lbx[128 + L.lane] = L.pr.hy;
    ldd[L.lane] = L.dd;
    const T *ocs = ob_trig_table<T, PA>(C, g, L, ocs_lds);
    const size_t EA = (size_t)C.E * C.A;
    St<T> gs;  // adjoint of the current step's output
    st_zero(gs);
    for (int t = g.nsteps - 1; t >= 0; --t) {
        if (t == g.nsteps - 1)
            add_adj<T, DRONE>(g.afin.f, L.idx, gs);
        else
            add_adj<T, DRONE>(g.atraj.f, (size_t)t * EA + L.idx, gs);
        St<T> st;
        if (t == 0)
            load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
        else
            load_state<T, DRONE>(g.traj.f, L.idx, (size_t)(t - 1) * EA, st);
        if (!L.real) st.px = st.py = __builtin_nan("");
        T a[4];
        load_act(g.act, (size_t)t * EA + L.idx, C.ad, a);

        // ---- recompute the substep chain of this step into LDS
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            T *sl = slots + (size_t)s * NF * 64;
            __syncthreads();
            slot_put<T, DRONE>(sl, L.lane, st);
            if (BOXES) {
                lcsb[s * 128 + L.lane] = m_cos(st.th);
                lcsb[s * 128 + 64 + L.lane] = m_sin(st.th);
            }
            __syncthreads();
            T Fx = T(0), Fy = T(0);
            M incl = 0;
            if (C.needs_forces) {
                M am = 0;
                uint64_t om = 0;
                bool wl = false, far = false;
                incl = forces<T, PA, BOXES>(C, g, L, sl, lr, st, s, s == 0 || !ok, cand, Fx, Fy,
                                            ocs, lbx, lcsb + s * 128, &am, &om, &wl, &far);
                if (BOXES) {
                    lact[s * 64 + L.lane] = am;
                    lom[s * 64 + L.lane] = om;
                    lwf[s * 64 + L.lane] = (wl ? 1 : 0) | (far ? 2 : 0);
                }
            }
            sl[F_FX * 64 + L.lane] = Fx;
            sl[F_FY * 64 + L.lane] = Fy;
            lmask[s * 64 + L.lane] = incl;
            St<T> nx;
            integrate<T, DRONE>(C, L.pr, st, a, Fx, Fy, nx);
            if (C.use_skin) {
                D += (m_abs(nx.px - st.px) + m_abs(nx.py - st.py)) * T(1.0001);
                ok = env_all<PA>(!L.real || D <= C.half_margin, L.base);
            }
            st = nx;
        }

        // ---- reverse pass
        T ga[4] = {T(0), T(0), T(0), T(0)};
        for (int s = C.S - 1; s >= 0; --s) {
            T *sl = slots + (size_t)s * NF * 64;
            __syncthreads();
            St<T> in;
            slot_get<T, DRONE>(sl, L.lane, in);
            const T Fx = sl[F_FX * 64 + L.lane], Fy = sl[F_FY * 64 + L.lane];
            St<T> gi;
            T gFx, gFy;
            integrate_adj<T, DRONE>(C, L.pr, in, a, Fx, Fy, gs, gi, ga, gFx, gFy);
            if (C.needs_forces) {
                // the slot now carries the force adjoint divided by the damping denominator
                const T wFx = gFx * L.inv_dd, wFy = gFy * L.inv_dd;
                __syncthreads();
                sl[F_FX * 64 + L.lane] = wFx;
                sl[F_FY * 64 + L.lane] = wFy;
                __syncthreads();
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
                        for (int o = 0; o < C.N; ++o)
                            obstacle_force_adj(C, g.obs, eN, o, in.px, in.py, in.vx, in.vy,
                                               L.pr.radius, L.dd, gFx, gFy, gi, ocs);
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

}  // namespace swarp
#include "lean.hpp"
#include "bodies.hpp"
#include "nav.hpp"
namespace swarp {

// --------------------------------------------------------------- neighbour lists

template <typename T, int PA>
__global__ __launch_bounds__(64) void k_neighbors(const Cst<T> C, const T *pos, int32_t *idx,
                                                  int32_t *cnt, int32_t *tru)
{
    typedef typename MaskT<PA>::type M;
    constexpr int EPW = 64 / PA;
    __shared__ T lx[64], ly[64];
    const int lane = threadIdx.x, agent = lane % PA, base = lane - agent;
    const int env = blockIdx.x * EPW + lane / PA;
    const bool active = agent < C.A && env < C.E;
    const size_t i = active ? (size_t)env * C.A + agent : 0;
    const bool real = agent < C.A;
    const T px = real ? pos[2 * i] : (T)__builtin_nan(""), py = real ? pos[2 * i + 1] : (T)__builtin_nan("");
    lx[lane] = px;
    ly[lane] = py;
    __syncthreads();
    M cd;
    const M incl = scan_all<T, PA>(lx, ly, base, C.A, agent, px, py, C.t_nbr, C.t_nbr, cd);
    if (!active) return;
    M m = cap_list(incl, C.K);
    const int n = m_popc(m);
    int32_t *row = idx + i * C.K;
    for (int k = 0; k < C.K; ++k) {
        int v = 0;
        if (k < n) {
            v = m_ctz(m);
            m &= m - 1;
        }
        row[k] = v;
    }
    cnt[i] = n;
    if (tru) tru[i] = m_popc(incl);
}

__global__ void k_edge_index(int E, int A, int K, const int32_t *idx, const int32_t *cnt,
                             const int64_t *off, int64_t n_edges, int64_t *out)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)E * A) return;
    const int64_t e = (int64_t)(i / A);
    const int64_t n = cnt[i];
    const int64_t o = off[i];
    for (int64_t s = 0; s < n && o + s < n_edges; ++s) {
        out[o + s] = e * A + idx[i * K + s];
        out[n_edges + o + s] = (int64_t)i;
    }
}

}  // namespace swarp

// ====================================================================== host side

using namespace swarp;

static thread_local char g_err[512];

static int fail(const char *msg)
{
    snprintf(g_err, sizeof g_err, "%s", msg);
    return -1;
}

static float h_sqrt(float x) { return sqrtf(x); }
static double h_sqrt(double x) { return sqrt(x); }
static float h_next(float x, float to) { return nextafterf(x, to); }
static double h_next(double x, double to) { return nextafter(x, to); }

// Largest x with fl(sqrt(x)) <= r: the exact replacement of sqrt(d2) <= r.  The host's
// sqrt is IEEE correctly rounded, like the device's, so the two tests agree bit for bit.
template <typename T> static T exact_threshold(double radius)
{
    const T r = (T)radius;
    if (r != r || r < T(0)) return (T)-INFINITY;
    if (isinf(r)) return (T)INFINITY;
    T t = r * r;
    for (;;) {
        T nx = h_next(t, (T)INFINITY);
        if (isinf(nx) || !(h_sqrt(nx) <= r)) break;
        t = nx;
    }
    while (t > T(0) && h_sqrt(t) > r) t = h_next(t, (T)-INFINITY);
    return t;
}

template <typename T> static int fill_cst(const swarp_desc_t *d, double skin, Cst<T> &C)
{
    memset(&C, 0, sizeof C);
    C.k = (T)d->k;
    C.c = (T)d->c;
    C.margin = (T)d->margin;
    C.sub_dt = (T)(d->dt / d->substeps);
    C.max_overlap = (T)d->max_overlap;
    C.eps2 = (T)1.0e-10;
    C.t_nbr = exact_threshold<T>(d->neighbor_radius);
    const double r = (double)(T)d->neighbor_radius;
    const double rs = r + (skin > 0.0 ? skin : 0.0);
    T ts = (T)(rs * rs);
    if (ts < C.t_nbr) ts = C.t_nbr;
    C.t_skin = ts;
    C.half_margin = (T)(0.5 * (sqrt((double)ts) - sqrt((double)C.t_nbr)) * (1.0 - 1e-3));
    if (C.half_margin < T(0)) C.half_margin = T(0);
    C.bmin_x = (T)d->bounds_min[0];
    C.bmin_y = (T)d->bounds_min[1];
    C.bmax_x = (T)d->bounds_max[0];
    C.bmax_y = (T)d->bounds_max[1];
    C.E = d->n_envs;
    C.A = d->n_agents;
    C.ad = d->act_dim;
    C.S = d->substeps;
    C.K = d->max_neighbors;
    C.N = d->n_obstacles;
    C.collisions = d->collisions;
    C.soft_walls = d->soft_walls;
    C.clamp = d->clamp_bounds;
    C.boxes = d->has_boxes ? 1 : 0;
    C.per_env = d->params_per_env ? 1 : 0;
    C.wheel = d->wheel_contacts ? 1 : 0;
    C.lat_grip = (T)d->lat_grip;
    C.turn_cap = (T)d->turn_cap;
    C.needs_forces = (d->collisions || d->soft_walls || d->n_obstacles > 0) ? 1 : 0;
    C.use_skin = (d->collisions && d->substeps > 1 && skin > 0.0) ? 1 : 0;
    // contact distances lie in [sqrt(eps2), neighbour radius]: within the range of the
    // short exact division when the radius is at most 2^20
    C.fast_div = d->neighbor_radius <= 0x1p20 ? 1 : 0;
    C.rk4 = d->integrator == SWARP_RK4 ? 1 : 0;
    return 0;
}

static int check_desc(const swarp_desc_t *d, bool need_params = true)
{
    if (!d) return fail("desc is NULL");
    if (d->abi_version != SWARP_ABI_VERSION) return fail("desc->abi_version mismatch");
    if (d->dtype != SWARP_F32 && d->dtype != SWARP_F64) return fail("desc->dtype must be SWARP_F32 or SWARP_F64");
    if (d->n_envs < 1) return fail("n_envs must be >= 1");
    if (d->n_agents < 1 || d->n_agents > 64) return fail("n_agents must lie in [1, 64] in this build");
    if (d->act_dim < 1) return fail("act_dim must be >= 1");
    if (d->substeps < 1) return fail("substeps must be >= 1");
    if (d->collisions && d->max_neighbors < 1) return fail("max_neighbors must be >= 1");
    if (d->n_obstacles < 0) return fail("n_obstacles must be >= 0");
    if (d->integrator != SWARP_EULER && d->integrator != SWARP_RK4)
        return fail("desc->integrator must be SWARP_EULER or SWARP_RK4");
    if (d->clamp_bounds < 0 || d->clamp_bounds > 2) return fail("desc->clamp_bounds must be 0, 1 or 2");
    if (d->clamp_bounds == 2 && !d->has_boxes)
        return fail("the footprint clamp (clamp_bounds 2) is for worlds holding box agents");
    if (d->has_boxes && d->has_drone) return fail("a drone cannot be a box agent");
    if (d->wheel_contacts && (d->has_drone || d->integrator != SWARP_EULER))
        return fail("wheel contacts run on the Euler 2-D path only (no drones, no RK4)");
    if (need_params && (!d->params || !d->model_tag || !d->ctrl_mode))
        return fail("params/model_tag/ctrl_mode must be set");
    if (d->n_obstacles > 0 && (!d->obs_pos || !d->obs_radius || !d->obs_angle || !d->obs_half ||
                               !d->obs_vel || !d->obs_ang_vel || !d->obs_type))
        return fail("obstacle arrays must be set when n_obstacles > 0");
    return 0;
}

static int pad_agents(int A)
{
    int p = 4;
    while (p < A) p <<= 1;
    return p;
}

static double skin_of(const swarp_desc_t *d)
{
    // Candidate-list skin: room for (S-1) substeps of motion of both agents of a pair
    // at about 1.5x the fleet's top speed.  Only speed depends on it; exactness does not.
    if (d->substeps < 2) return 0.0;
    double vmax = 1.0;
    if (getenv("SWARP_SKIN_VMAX")) vmax = atof(getenv("SWARP_SKIN_VMAX"));
    return 2.0 * 1.5 * vmax * (d->substeps - 1) * (d->dt / d->substeps);
}

template <typename T> static void fill_args(const swarp_desc_t *d, Args<T> &a)
{
    memset(&a, 0, sizeof a);
    a.params = (const T *)d->params;
    a.tag = d->model_tag;
    a.mode = d->ctrl_mode;
    a.obs.pos = (const T *)d->obs_pos;
    a.obs.rad = (const T *)d->obs_radius;
    a.obs.ang = (const T *)d->obs_angle;
    a.obs.half = (const T *)d->obs_half;
    a.obs.vel = (const T *)d->obs_vel;
    a.obs.om = (const T *)d->obs_ang_vel;
    a.obs.type = d->obs_type;
}

template <typename T> static void copy_fields(const swarp_state_t *s, T **f)
{
    void *const src[9] = {s->pos, s->theta, s->vel, s->speed, s->ang_vel,
                          s->z, s->vz, s->attitude, s->body_rates};
    for (int k = 0; k < 9; ++k) f[k] = (T *)src[k];
}

static bool fields_ok(const swarp_state_t *s, int n)
{
    if (!s) return false;
    void *const src[9] = {s->pos, s->theta, s->vel, s->speed, s->ang_vel,
                          s->z, s->vz, s->attitude, s->body_rates};
    for (int k = 0; k < n; ++k)
        if (!src[k]) return false;
    return true;
}

#define SWARP_DISPATCH_PA(PA_, KERNEL, ...)                                        \
    switch (PA_) {                                                                 \
    case 4: hipLaunchKernelGGL((KERNEL<T, 4, __VA_ARGS__>), grid4, dim3(64), shm, st, C, a); break; \
    case 8: hipLaunchKernelGGL((KERNEL<T, 8, __VA_ARGS__>), grid8, dim3(64), shm, st, C, a); break; \
    case 16: hipLaunchKernelGGL((KERNEL<T, 16, __VA_ARGS__>), grid16, dim3(64), shm, st, C, a); break; \
    case 32: hipLaunchKernelGGL((KERNEL<T, 32, __VA_ARGS__>), grid32, dim3(64), shm, st, C, a); break; \
    default: hipLaunchKernelGGL((KERNEL<T, 64, __VA_ARGS__>), grid64, dim3(64), shm, st, C, a); break; \
    }

template <typename T, bool DRONE, bool BOXES>
static void launch_fwd(int PA, const Cst<T> &C, const Args<T> &a, hipStream_t st)
{
    const size_t shm = 0;
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    SWARP_DISPATCH_PA(PA, k_rollout_fwd, DRONE, BOXES)
}

template <typename T, bool DRONE, bool BOXES>
static void launch_bwd(int PA, const Cst<T> &C, const Args<T> &a, size_t shm, hipStream_t st)
{
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    SWARP_DISPATCH_PA(PA, k_rollout_bwd, DRONE, BOXES)
}

static bool lean_ok(const swarp_desc_t *d)
{
    return d->holo_velocity_only && !d->has_drone && d->n_obstacles == 0 && !d->clamp_bounds &&
           d->integrator == SWARP_EULER && !d->has_boxes && !d->wheel_contacts &&
           !d->params_per_env;
}

// Byte offsets of the tape regions (see lean.hpp); total == 0: no tape.
struct TapeLayout {
    uint64_t rec, vl, total;
};

static uint64_t align256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

template <typename T> static uint64_t tape_rec_bytes(int PA)
{
    switch (PA) {
    case 4: return TapeRec<T, 4>::R;
    case 8: return TapeRec<T, 8>::R;
    case 16: return TapeRec<T, 16>::R;
    case 32: return TapeRec<T, 32>::R;
    default: return TapeRec<T, 64>::R;
    }
}

static TapeLayout tape_layout(const swarp_desc_t *d, int32_t nT)
{
    TapeLayout L = {0, 0, 0};
    const bool forces = d->collisions || d->soft_walls;
    if (!lean_ok(d) || !forces || d->substeps > TAPE_MAX_S || nT < 1) return L;
    const bool f32 = d->dtype == SWARP_F32;
    const int PA = pad_agents(d->n_agents);
    const uint64_t R = f32 ? tape_rec_bytes<float>(PA) : tape_rec_bytes<double>(PA);
    // one record per step and lane of every workgroup (64 / PA envs each)
    const uint64_t lanes = (uint64_t)((d->n_envs + 64 / PA - 1) / (64 / PA)) * 64;
    L.rec = 0;
    L.vl = align256((uint64_t)nT * lanes * R);
    L.total = align256(L.vl + lanes * 2 * (f32 ? 4 : 8));
    return L;
}

template <typename T> static Tape<T> tape_ptrs(const TapeLayout &L, void *base)
{
    Tape<T> tp = {nullptr, nullptr};
    if (!base || L.total == 0) return tp;
    unsigned char *b = (unsigned char *)base;
    tp.rec = (void *)(b + L.rec);
    tp.vl = (T *)(b + L.vl);
    return tp;
}

template <typename T, bool TAPE>
static void launch_holo_fwd(int PA, const Cst<T> &C, const Args<T> &a, const Tape<T> &tp,
                            hipStream_t st)
{
    const size_t shm = 0;
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_holo_fwd<T, 4, TAPE>), grid4, dim3(64), shm, st, C, a, tp); break;
    case 8: hipLaunchKernelGGL((k_holo_fwd<T, 8, TAPE>), grid8, dim3(64), shm, st, C, a, tp); break;
    case 16: hipLaunchKernelGGL((k_holo_fwd<T, 16, TAPE>), grid16, dim3(64), shm, st, C, a, tp); break;
    case 32: hipLaunchKernelGGL((k_holo_fwd<T, 32, TAPE>), grid32, dim3(64), shm, st, C, a, tp); break;
    default: hipLaunchKernelGGL((k_holo_fwd<T, 64, TAPE>), grid64, dim3(64), shm, st, C, a, tp); break;
    }
}

template <typename T, bool TAPE>
static void launch_holo_bwd(int PA, const Cst<T> &C, const Args<T> &a, const Tape<T> &tp,
                            size_t shm, hipStream_t st)
{
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_holo_bwd<T, 4, TAPE>), grid4, dim3(64), shm, st, C, a, tp); break;
    case 8: hipLaunchKernelGGL((k_holo_bwd<T, 8, TAPE>), grid8, dim3(64), shm, st, C, a, tp); break;
    case 16: hipLaunchKernelGGL((k_holo_bwd<T, 16, TAPE>), grid16, dim3(64), shm, st, C, a, tp); break;
    case 32: hipLaunchKernelGGL((k_holo_bwd<T, 32, TAPE>), grid32, dim3(64), shm, st, C, a, tp); break;
    default: hipLaunchKernelGGL((k_holo_bwd<T, 64, TAPE>), grid64, dim3(64), shm, st, C, a, tp); break;
    }
}

template <typename T>
static int rollout_fwd(const swarp_desc_t *d, int32_t nT, const swarp_state_t *s0,
                       const void *act, const swarp_state_t *traj, const swarp_state_t *fin,
                       void *tape, uint64_t tape_bytes, hipStream_t st)
{
    const TapeLayout TL = tape_layout(d, nT);
    if (tape && tape_bytes != TL.total) return fail("tape_bytes does not match swarp_tape_bytes");
    Cst<T> C;
    fill_cst<T>(d, skin_of(d), C);
    Args<T> a;
    fill_args<T>(d, a);
    const int nf = d->has_drone ? 9 : 5;
    if (!fields_ok(s0, nf)) return fail("state0 is missing a field");
    if (!fields_ok(fin, nf)) return fail("final_state is missing a field");
    if (nT > 1 && !fields_ok(traj, nf)) return fail("traj is missing a field (T > 1)");
    if (!act) return fail("actions is NULL");
    copy_fields<T>(s0, (T **)a.s0.f);
    copy_fields<T>(fin, a.fin.f);
    if (nT > 1) copy_fields<T>(traj, a.traj.f);
    a.act = (const T *)act;
    a.nsteps = nT;
    const int PA = pad_agents(d->n_agents);
    if (lean_ok(d))
        if (tape && TL.total)
            launch_holo_fwd<T, true>(PA, C, a, tape_ptrs<T>(TL, tape), st);
        else
            launch_holo_fwd<T, false>(PA, C, a, tape_ptrs<T>(TL, nullptr), st);
    else if (d->has_drone)
        launch_fwd<T, true, false>(PA, C, a, st);
    else if (d->has_boxes || d->wheel_contacts)
        launch_fwd<T, false, true>(PA, C, a, st);
    else
        launch_fwd<T, false, false>(PA, C, a, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

template <typename T>
static int rollout_bwd(const swarp_desc_t *d, int32_t nT, const swarp_state_t *s0,
                       const void *act, const swarp_state_t *traj, const swarp_state_t *atraj,
                       const swarp_state_t *afin, const swarp_state_t *a0, void *aact,
                       const void *tape, uint64_t tape_bytes, hipStream_t st)
{
    const TapeLayout TL = tape_layout(d, nT);
    if (tape && tape_bytes != TL.total) return fail("tape_bytes does not match swarp_tape_bytes");
    Cst<T> C;
    fill_cst<T>(d, skin_of(d), C);
    Args<T> a;
    fill_args<T>(d, a);
    const int nf = d->has_drone ? 9 : 5;
    if (!fields_ok(s0, nf)) return fail("state0 is missing a field");
    if (nT > 1 && !fields_ok(traj, nf)) return fail("traj is missing a field (T > 1)");
    if (!act || !aact) return fail("actions / adj_actions is NULL");
    copy_fields<T>(s0, (T **)a.s0.f);
    if (nT > 1) copy_fields<T>(traj, a.traj.f);
    if (atraj) copy_fields<T>(atraj, (T **)a.atraj.f);
    if (afin) copy_fields<T>(afin, (T **)a.afin.f);
    if (a0) copy_fields<T>(a0, a.a0.f);
    a.act = (const T *)act;
    a.aact = (T *)aact;
    a.nsteps = nT;
    const int PA = pad_agents(d->n_agents);
    if (lean_ok(d)) {
        const size_t msz = PA == 64 ? 8 : 4;
        const size_t lshm = (size_t)d->substeps * 128 * 2 * sizeof(T) +
                            (size_t)d->substeps * 64 * msz * 2 + 64 * 2 * sizeof(T) +
                            2 * 64 * sizeof(T) + (size_t)d->substeps * 64;
        if (lshm > 65536) return fail("substeps too large for the backward LDS staging (limit 64 KiB per wave)");
        if (tape && TL.total)
            launch_holo_bwd<T, true>(PA, C, a, tape_ptrs<T>(TL, (void *)tape), lshm, st);
        else
            launch_holo_bwd<T, false>(PA, C, a, tape_ptrs<T>(TL, nullptr), lshm, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(hipGetErrorString(e));
        return 0;
    }
    const int NF = d->has_drone ? NF_DRONE : NF_2D;
    const size_t msz = PA == 64 ? 8 : 4;
    size_t shm = 2 * 64 * sizeof(T) + (size_t)d->substeps * NF * 64 * sizeof(T) +
                 (size_t)d->substeps * 64 * msz;
    if (d->has_boxes)  // contact masks, heading cos / sin, static-contact flags per substep
        shm += (size_t)d->substeps * 64 * (msz + 2 * sizeof(T) + 8 + 1);
    if (shm > 65536) return fail("substeps too large for the backward LDS staging (limit 64 KiB per wave)");
    if (d->has_drone)
        launch_bwd<T, true, false>(PA, C, a, shm, st);
    else if (d->has_boxes)
        launch_bwd<T, false, true>(PA, C, a, shm, st);
    else
        launch_bwd<T, false, false>(PA, C, a, shm, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

template <typename T> static int fill_obtab(const swarp_desc_t *d, ObTab<T> &tb)
{
    if (d->n_obstacles < 1 || d->n_obstacles > NOB_MAX)
        return fail("the body path takes 1 to 16 obstacles per env");
    if (!d->obs_kind || !d->obs_body || !d->obs_mass || !d->obs_inertia || !d->obs_body_off)
        return fail("obs_kind/obs_body/obs_mass/obs_inertia/obs_body_off must be set");
    if (d->has_drone) return fail("the body path steps 2-D fleets only");
    tb.rad = (const T *)d->obs_radius;
    tb.half = (const T *)d->obs_half;
    tb.mass = (const T *)d->obs_mass;
    tb.inertia = (const T *)d->obs_inertia;
    tb.off = (const T *)d->obs_body_off;
    tb.type = d->obs_type;
    tb.kind = d->obs_kind;
    tb.body = d->obs_body;
    tb.lin_damp = (T)d->lin_damping;
    tb.ang_damp = (T)d->ang_damping;
    tb.N = d->n_obstacles;
    return 0;
}

template <typename T>
static int rollout_fwd_ob(const swarp_desc_t *d, int32_t nT, const swarp_state_t *s0,
                          const void *ob0, const void *act, const swarp_state_t *traj,
                          const swarp_state_t *fin, void *ob_traj, hipStream_t st)
{
    Cst<T> C;
    fill_cst<T>(d, skin_of(d), C);
    Args<T> a;
    fill_args<T>(d, a);
    ObTab<T> tb;
    if (fill_obtab<T>(d, tb)) return -1;
    if (!fields_ok(s0, 5)) return fail("state0 is missing a field");
    if (!fields_ok(fin, 5)) return fail("final_state is missing a field");
    if (nT > 1 && !fields_ok(traj, 5)) return fail("traj is missing a field (T > 1)");
    if (!act || !ob0 || !ob_traj) return fail("actions / ob0 / ob_traj is NULL");
    copy_fields<T>(s0, (T **)a.s0.f);
    copy_fields<T>(fin, a.fin.f);
    if (nT > 1) copy_fields<T>(traj, a.traj.f);
    a.act = (const T *)act;
    a.nsteps = nT;
    ObIO<T> io = {(const T *)ob0, (T *)ob_traj, nullptr, nullptr};
    const int PA = pad_agents(d->n_agents);
    const dim3 grid((C.E + 64 / PA - 1) / (64 / PA));
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_body_fwd<T, 4>), grid, dim3(64), 0, st, C, a, tb, io); break;
    case 8: hipLaunchKernelGGL((k_body_fwd<T, 8>), grid, dim3(64), 0, st, C, a, tb, io); break;
    case 16: hipLaunchKernelGGL((k_body_fwd<T, 16>), grid, dim3(64), 0, st, C, a, tb, io); break;
    case 32: hipLaunchKernelGGL((k_body_fwd<T, 32>), grid, dim3(64), 0, st, C, a, tb, io); break;
    default: hipLaunchKernelGGL((k_body_fwd<T, 64>), grid, dim3(64), 0, st, C, a, tb, io); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

template <typename T> static size_t body_bwd_lds_of(int PA, int S, int N)
{
    switch (PA) {
    case 4: return body_bwd_lds<T, 4>(S, N);
    case 8: return body_bwd_lds<T, 8>(S, N);
    case 16: return body_bwd_lds<T, 16>(S, N);
    case 32: return body_bwd_lds<T, 32>(S, N);
    default: return body_bwd_lds<T, 64>(S, N);
    }
}

template <typename T>
static int rollout_bwd_ob(const swarp_desc_t *d, int32_t nT, const swarp_state_t *s0,
                          const void *ob0, const void *act, const swarp_state_t *traj,
                          const void *ob_traj, const swarp_state_t *atraj,
                          const swarp_state_t *afin, const void *aob_traj,
                          const swarp_state_t *a0, void *aob0, void *aact, hipStream_t st)
{
    Cst<T> C;
    fill_cst<T>(d, skin_of(d), C);
    Args<T> a;
    fill_args<T>(d, a);
    ObTab<T> tb;
    if (fill_obtab<T>(d, tb)) return -1;
    if (!fields_ok(s0, 5)) return fail("state0 is missing a field");
    if (nT > 1 && !fields_ok(traj, 5)) return fail("traj is missing a field (T > 1)");
    if (!act || !aact || !ob0 || !ob_traj) return fail("actions / adj_actions / ob0 / ob_traj is NULL");
    copy_fields<T>(s0, (T **)a.s0.f);
    if (nT > 1) copy_fields<T>(traj, a.traj.f);
    if (atraj) copy_fields<T>(atraj, (T **)a.atraj.f);
    if (afin) copy_fields<T>(afin, (T **)a.afin.f);
    if (a0) copy_fields<T>(a0, a.a0.f);
    a.act = (const T *)act;
    a.aact = (T *)aact;
    a.nsteps = nT;
    ObIO<T> io = {(const T *)ob0, (T *)ob_traj, (const T *)aob_traj, (T *)aob0};
    const int PA = pad_agents(d->n_agents);
    const size_t shm = body_bwd_lds_of<T>(PA, d->substeps, d->n_obstacles);
    if (shm > 65536) return fail("substeps too large for the body backward's LDS staging (limit 64 KiB per wave)");
    const dim3 grid((C.E + 64 / PA - 1) / (64 / PA));
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_body_bwd<T, 4>), grid, dim3(64), shm, st, C, a, tb, io); break;
    case 8: hipLaunchKernelGGL((k_body_bwd<T, 8>), grid, dim3(64), shm, st, C, a, tb, io); break;
    case 16: hipLaunchKernelGGL((k_body_bwd<T, 16>), grid, dim3(64), shm, st, C, a, tb, io); break;
    case 32: hipLaunchKernelGGL((k_body_bwd<T, 32>), grid, dim3(64), shm, st, C, a, tb, io); break;
    default: hipLaunchKernelGGL((k_body_bwd<T, 64>), grid, dim3(64), shm, st, C, a, tb, io); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

template <typename T> static int nav_obs(const swarp_desc_t *d, const swarp_nav_t *v, hipStream_t st)
{
    Cst<T> C;
    fill_cst<T>(d, 0.0, C);
    NavArgs<T> g;
    memset(&g, 0, sizeof g);
    g.pos = (const T *)v->pos;
    g.vel = (const T *)v->vel;
    g.th = (const T *)v->theta;
    g.om = (const T *)v->ang_vel;
    g.goal = (const T *)v->goals;
    g.params = (const T *)d->params;
    g.rmask = v->reset_mask;
    g.prev = (T *)v->prev_dist;
    g.obs = (T *)v->obs;
    g.touch = (T *)v->touching;
    g.dist = (T *)v->dist;
    g.shaping = (T *)v->shaping;
    g.reward = (T *)v->reward;
    g.idx = v->nbr_idx;
    g.cnt = v->nbr_cnt;
    g.tru = v->nbr_true;
    g.ongoal = v->on_goal;
    g.overflow = v->overflow;
    g.done = v->done;
    g.shaping_factor = (T)v->pos_shaping_factor;
    g.goal_tol = (T)v->goal_tolerance;
    g.coll_pen = (T)v->collision_penalty;
    g.final_rew = (T)v->final_reward;
    g.k_obs = v->k_obs;
    g.W = 9 + 5 * v->k_obs;
    g.advance_prev = v->advance_prev ? 1 : 0;
    g.full_pass = v->full_pass ? 1 : 0;
    g.shared = v->shared_reward ? 1 : 0;
    g.step_count = v->step_count;
    g.truncated = v->truncated;
    g.max_steps = v->max_steps;
    const size_t lds = (size_t)64 * g.W * sizeof(T) + (size_t)64 * d->max_neighbors * 4;
    g.stage = lds <= 48 * 1024 ? 1 : 0;  // rows leave through LDS when they fit
    const unsigned dyn = g.stage ? (unsigned)lds : 0u;
    const int PA = pad_agents(d->n_agents);
    const dim3 grid((d->n_envs + (64 / PA) - 1) / (64 / PA));
    switch (PA) {
    case 4: hipLaunchKernelGGL((k_nav<T, 4>), grid, dim3(64), dyn, st, C, g); break;
    case 8: hipLaunchKernelGGL((k_nav<T, 8>), grid, dim3(64), dyn, st, C, g); break;
    case 16: hipLaunchKernelGGL((k_nav<T, 16>), grid, dim3(64), dyn, st, C, g); break;
    case 32: hipLaunchKernelGGL((k_nav<T, 32>), grid, dim3(64), dyn, st, C, g); break;
    default: hipLaunchKernelGGL((k_nav<T, 64>), grid, dim3(64), dyn, st, C, g); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

extern "C" {

int swarp_abi_version(void) { return SWARP_ABI_VERSION; }

int swarp_rollout_fwd_ob(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                         const void *ob0, const void *actions, const swarp_state_t *traj,
                         const swarp_state_t *final_state, void *ob_traj, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (desc->has_boxes || desc->wheel_contacts || desc->params_per_env)
        return fail("box agents, wheel contacts and per-env parameters with movable bodies are "
                    "not supported in this build");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_fwd_ob<float>(desc, T, state0, ob0, actions, traj, final_state, ob_traj, st);
    return rollout_fwd_ob<double>(desc, T, state0, ob0, actions, traj, final_state, ob_traj, st);
}

int swarp_rollout_bwd_ob(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                         const void *ob0, const void *actions, const swarp_state_t *traj,
                         const void *ob_traj, const swarp_state_t *adj_traj,
                         const swarp_state_t *adj_final, const void *adj_ob_traj,
                         const swarp_state_t *adj_state0, void *adj_ob0, void *adj_actions,
                         void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (desc->has_boxes || desc->wheel_contacts || desc->params_per_env)
        return fail("box agents, wheel contacts and per-env parameters with movable bodies are "
                    "not supported in this build");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_bwd_ob<float>(desc, T, state0, ob0, actions, traj, ob_traj, adj_traj,
                                     adj_final, adj_ob_traj, adj_state0, adj_ob0, adj_actions, st);
    return rollout_bwd_ob<double>(desc, T, state0, ob0, actions, traj, ob_traj, adj_traj,
                                  adj_final, adj_ob_traj, adj_state0, adj_ob0, adj_actions, st);
}

const char *swarp_last_error(void) { return g_err; }

int swarp_rollout_fwd(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                      const void *actions, const swarp_state_t *traj,
                      const swarp_state_t *final_state, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_fwd<float>(desc, T, state0, actions, traj, final_state, nullptr, 0, st);
    return rollout_fwd<double>(desc, T, state0, actions, traj, final_state, nullptr, 0, st);
}

int swarp_tape_bytes(const swarp_desc_t *desc, int32_t T, uint64_t *bytes)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (!bytes) return fail("bytes is NULL");
    *bytes = tape_layout(desc, T).total;
    return 0;
}

int swarp_rollout_fwd_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                           const void *actions, const swarp_state_t *traj,
                           const swarp_state_t *final_state, void *tape, uint64_t tape_bytes,
                           void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (!tape && tape_bytes) return fail("tape is NULL");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_fwd<float>(desc, T, state0, actions, traj, final_state, tape, tape_bytes, st);
    return rollout_fwd<double>(desc, T, state0, actions, traj, final_state, tape, tape_bytes, st);
}

int swarp_rollout_bwd(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                      const void *actions, const swarp_state_t *traj,
                      const swarp_state_t *adj_traj, const swarp_state_t *adj_final,
                      const swarp_state_t *adj_state0, void *adj_actions, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (desc->wheel_contacts)
        return fail("wheel contacts have no reverse pass (the reference runs them untaped only)");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_bwd<float>(desc, T, state0, actions, traj, adj_traj, adj_final, adj_state0,
                                  adj_actions, nullptr, 0, st);
    return rollout_bwd<double>(desc, T, state0, actions, traj, adj_traj, adj_final, adj_state0,
                               adj_actions, nullptr, 0, st);
}

int swarp_rollout_bwd_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                           const void *actions, const swarp_state_t *traj,
                           const swarp_state_t *adj_traj, const swarp_state_t *adj_final,
                           const swarp_state_t *adj_state0, void *adj_actions,
                           const void *tape, uint64_t tape_bytes, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (!tape && tape_bytes) return fail("tape is NULL");
    if (desc->wheel_contacts)
        return fail("wheel contacts have no reverse pass (the reference runs them untaped only)");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_bwd<float>(desc, T, state0, actions, traj, adj_traj, adj_final, adj_state0,
                                  adj_actions, tape, tape_bytes, st);
    return rollout_bwd<double>(desc, T, state0, actions, traj, adj_traj, adj_final, adj_state0,
                               adj_actions, tape, tape_bytes, st);
}

int swarp_neighbors(const swarp_desc_t *desc, const void *pos, int32_t *idx, int32_t *cnt,
                    int32_t *true_cnt, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc, false)) return -1;
    if (desc->max_neighbors < 1) return fail("max_neighbors must be >= 1");
    if (!pos || !idx || !cnt) return fail("pos/idx/cnt must be set");
    hipStream_t st = (hipStream_t)stream;
    const int PA = pad_agents(desc->n_agents);
    const int E = desc->n_envs;
    const dim3 grid((E + (64 / PA) - 1) / (64 / PA));
#define SWARP_NB(TT)                                                                          \
    {                                                                                         \
        Cst<TT> C;                                                                            \
        fill_cst<TT>(desc, 0.0, C);                                                           \
        const TT *p = (const TT *)pos;                                                        \
        switch (PA) {                                                                         \
        case 4: hipLaunchKernelGGL((k_neighbors<TT, 4>), grid, dim3(64), 0, st, C, p, idx, cnt, true_cnt); break; \
        case 8: hipLaunchKernelGGL((k_neighbors<TT, 8>), grid, dim3(64), 0, st, C, p, idx, cnt, true_cnt); break; \
        case 16: hipLaunchKernelGGL((k_neighbors<TT, 16>), grid, dim3(64), 0, st, C, p, idx, cnt, true_cnt); break; \
        case 32: hipLaunchKernelGGL((k_neighbors<TT, 32>), grid, dim3(64), 0, st, C, p, idx, cnt, true_cnt); break; \
        default: hipLaunchKernelGGL((k_neighbors<TT, 64>), grid, dim3(64), 0, st, C, p, idx, cnt, true_cnt); break; \
        }                                                                                     \
    }
    if (desc->dtype == SWARP_F32)
        SWARP_NB(float)
    else
        SWARP_NB(double)
#undef SWARP_NB
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

int swarp_nav_obs(const swarp_desc_t *desc, const swarp_nav_t *nav, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (!nav) return fail("nav is NULL");
    if (desc->max_neighbors < 1) return fail("max_neighbors must be >= 1");
    if (nav->k_obs < 0 || nav->k_obs > desc->max_neighbors)
        return fail("k_obs must lie in [0, max_neighbors]");
    if (!nav->pos || !nav->vel || !nav->theta || !nav->ang_vel || !nav->goals || !nav->prev_dist ||
        !nav->nbr_idx || !nav->nbr_cnt || !nav->obs || !nav->touching || !nav->dist ||
        !nav->shaping || !nav->on_goal || !nav->overflow || !nav->reward || !nav->done)
        return fail("every swarp_nav_t pointer except reset_mask and nbr_true must be set");
    if (!nav->full_pass && !nav->reset_mask)
        return fail("an obs-only pass (full_pass == 0) needs reset_mask");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32) return nav_obs<float>(desc, nav, st);
    return nav_obs<double>(desc, nav, st);
}

int swarp_edge_index(int32_t n_envs, int32_t n_agents, int32_t max_neighbors, const int32_t *idx,
                     const int32_t *cnt, const int64_t *offsets, int64_t n_edges,
                     int64_t *edge_index, void *stream)
{
    g_err[0] = 0;
    if (n_envs < 1 || n_agents < 1 || max_neighbors < 1) return fail("bad sizes");
    if (n_edges < 0) return fail("n_edges must be >= 0");
    if (n_edges == 0) return 0;
    if (!idx || !cnt || !offsets || !edge_index) return fail("pointer arguments must be set");
    const size_t n = (size_t)n_envs * n_agents;
    hipLaunchKernelGGL(k_edge_index, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, n_envs, n_agents, max_neighbors, idx, cnt, offsets,
                       n_edges, edge_index);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

}  // extern "C"
