// wide_bodies.hpp -- movable compound bodies in envs of more than 64 agents, and with
// grid-ordered lists: the body pass of bodies.hpp (obstacle_dynamics_kernel,
// swarp/core/bodies.py:367-568) on the wide kernels' layout, one workgroup of
// ceil(A / 64) waves per env (wide.hpp).  Instantiated by k_wbodies.hip.
//
// The env's obstacle state (12 scalars per obstacle index, as in bodies.hpp) lives in LDS
// for the whole launch, double-buffered across substeps, and goes to HBM once per step.
// The body pass's sums over the env's agents (a body's contact force and torque, the
// adjoints of a body's pose and of a moving shape's state) span the workgroup's waves:
// each flagged agent's values go to LDS with one flag mask per wave, and every thread
// then adds them in ascending agent order (WideEnv::ordered), so the forward's sums keep
// the reference's order and every thread holds them.
//
// The backward recomputes, for each substep in reverse, the substeps before it from the
// step's checkpoint (agent state and obstacle state), as the wide backward does.
#pragma once
#include "bodies.hpp"
#include "wide.hpp"

namespace swarp {

// The body pass's env policy on the wide kernels (see NarrowEnv): the env's AP slots are
// the workgroup's threads.
template <typename T> struct WideEnv {
    int i, AP;
    bool act;
    T *scr;           // [4][AP] values of the flagged agents
    uint64_t *flags;  // [AP / 64] flag mask of each wave

    __device__ __forceinline__ int me() const { return i; }
    __device__ __forceinline__ int stride() const { return AP; }
    __device__ __forceinline__ bool active() const { return act; }
    template <int NV>
    __device__ __forceinline__ void ordered(T (&acc)[NV], const T (&v)[NV], bool flag) const
    {
        const uint64_t bal = __ballot(flag);
        for (int q0 = 0; q0 < NV; q0 += 4) {
            __syncthreads();  // the previous readers of scr / flags are done
            if ((i & 63) == 0) flags[i >> 6] = bal;
            if (flag) {
#pragma unroll
                for (int q = q0; q < NV && q < q0 + 4; ++q) scr[(q - q0) * AP + i] = v[q];
            }
            __syncthreads();
            for (int w = 0; w < AP / 64; ++w) {
                for (uint64_t m = flags[w]; m; m &= m - 1) {
                    const int j = w * 64 + __builtin_ctzll(m);
#pragma unroll
                    for (int q = q0; q < NV && q < q0 + 4; ++q) acc[q] += scr[(q - q0) * AP + j];
                }
            }
        }
    }
    __device__ __forceinline__ bool any(bool f) const
    {
        const uint64_t bal = __ballot(f);
        __syncthreads();
        if ((i & 63) == 0) flags[i >> 6] = bal;
        __syncthreads();
        bool r = false;
        for (int w = 0; w < AP / 64; ++w) r = r || flags[w] != 0;
        return r;
    }
    __device__ __forceinline__ void sync() const { __syncthreads(); }
};

// LDS of a wide body workgroup after the wide kernels' own (wide_lds_bytes): the wave
// flag masks, the ordered sums' values, and obstacle states -- forward: two (substep
// input / output); backward: the step's checkpoint, two recompute buffers and two
// adjoints -- then the static extent of each body root.
template <typename T> struct WBodyLds {
    uint64_t *flags;
    T *scr, *ob, *ext;
};

__host__ __device__ constexpr size_t wbody_align16(size_t b) { return (b + 15) / 16 * 16; }

template <typename T>
__host__ __device__ inline size_t wbody_lds_bytes(int AP, int NC, int N, bool bwd)
{
    return wbody_align16(wide_lds_bytes<T>(AP, NC)) + (size_t)(AP / 64) * sizeof(uint64_t) +
           ((size_t)4 * AP + (size_t)(bwd ? 5 : 2) * OB_W * N + N) * sizeof(T);
}

template <typename T>
__device__ __forceinline__ WBodyLds<T> wbody_lds(unsigned char *smem, int AP, int NC, int N,
                                                 bool bwd)
{
    WBodyLds<T> B;
    unsigned char *p = smem + wbody_align16(wide_lds_bytes<T>(AP, NC));
    B.flags = (uint64_t *)p;
    B.scr = (T *)(p + (size_t)(AP / 64) * sizeof(uint64_t));
    B.ob = B.scr + 4 * AP;
    B.ext = B.ob + (size_t)(bwd ? 5 : 2) * OB_W * N;
    return B;
}

// The agent as the body pass sees it (body_row of the narrow kernels).
template <typename T>
__device__ __forceinline__ BodyRow<T> wbody_row(const Cst<T> &C, const ObTab<T> &tb,
                                                const WLane<T> &L)
{
    if (!tb.bprm) return BodyRow<T>{L.pr.radius, L.dd, L.ddv};
    const int ag = L.active ? L.i : 0;
    const T m = tb.bprm[(size_t)ag * 22 + 1];
    const T dd = T(1) + C.c * C.sub_dt / m;
    return BodyRow<T>{tb.bprm[(size_t)ag * 22], dd, divisor(dd, true)};
}

// Forces of the lane's agent against the env's obstacle state `od` (listed pairs, the
// obstacles in index order, walls).
template <typename T, bool GRID>
__device__ __forceinline__ void wbody_forces(const Cst<T> &C, const ObTab<T> &tb,
                                             const WideLds<T> &W, const GridFrame<T> &G,
                                             const WLane<T> &L, const St<T> &st, const T *od,
                                             T &Fx, T &Fy, int32_t &cut)
{
    wide_forces_with<T, GRID>(C, W, G, L, st, Fx, Fy, cut, [&](T &sx, T &sy) {
        for (int o = 0; o < tb.N; ++o) {
            T gx, gy;
            ob_force(C, tb, od, o, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx, gy);
            sx += gx;
            sy += gy;
        }
    });
}

// One substep of the env: lists and forces on the input state, the body pass (obc -> obn),
// the agents' integration.  Every thread of the workgroup calls it.
template <typename T, bool DRONE, bool GRID, bool SM>
__device__ __forceinline__ void wbody_substep(const Cst<T> &C, const ObTab<T> &tb,
                                              const ShapeSets<T, SM> &SS, const WideEnv<T> &X,
                                              const BodyRow<T> &br, const WideLds<T> &W,
                                              const GridFrame<T> &G, const WLane<T> &L,
                                              const T (&a)[4], St<T> &st, const T *obc, T *obn,
                                              const T *ext, int32_t *wsum)
{
    if (C.collisions) wide_publish<T, GRID>(C, W, G, L, st, wsum);
    T Fx, Fy;
    int32_t cut;
    wbody_forces<T, GRID>(C, tb, W, G, L, st, obc, Fx, Fy, cut);
    body_pass<T>(C, tb, SS, X, br, st, obc, obn, ext, nullptr, nullptr, nullptr);
    X.sync();  // obn complete, obc read by every thread
    St<T> nx;
    integrate<T, DRONE>(C, L.pr, st, a, Fx, Fy, nx);
    st = nx;
}

// ------------------------------------------------------------------ forward rollout

template <typename T, bool DRONE, bool GRID, unsigned F>
__global__ __launch_bounds__(1024) void k_wbody_fwd(const Cst<T> Cin, const Args<T> g,
                                                    const ObTab<T> tb, const ObIO<T> io)
{
    const Cst<T> C = fold_cst<F>(Cin);
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t wsum[16];
    const int AP = blockDim.x, N = tb.N, NW = OB_W * N;
    const int NC = C.grid_bins > 0 ? C.grid_bins * C.grid_bins : 0;
    const WideLds<T> W = wide_lds<T>(smem, AP);
    const WBodyLds<T> B = wbody_lds<T>(smem, AP, NC, N, false);
    const GridFrame<T> G = grid_frame(C, (const T *)nullptr);
    WLane<T> L;
    wide_init<T, F>(C, g, L);
    W.rad[L.i] = L.pr.radius;
    ShapeSets<T, !(F & FT_MANYSH)> SS;
    SS.init(tb, L.i & 63);
    const WideEnv<T> X{L.i, AP, L.active, B.scr, B.flags};
    const BodyRow<T> br = wbody_row(C, tb, L);
    for (int o = L.i; o < N; o += AP) B.ext[o] = body_ext(tb, o);
    const size_t eo = (size_t)L.env * NW, ENW = (size_t)C.E * NW;
    for (int q = L.i; q < NW; q += AP) B.ob[q] = io.ob0[eo + q];
    __syncthreads();
    St<T> st;
    load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
    if (!L.active) st.px = st.py = __builtin_nan("");
    const size_t EA = (size_t)C.E * C.A;
    int cur = 0;
    for (int t = 0; t < g.nsteps; ++t) {
        T a[4];
        load_act(g.act, (size_t)t * EA + L.idx, C.ad, a);
        for (int s = 0; s < C.S; ++s) {
            wbody_substep<T, DRONE, GRID>(C, tb, SS, X, br, W, G, L, a, st, B.ob + cur * NW,
                                          B.ob + (cur ^ 1) * NW, B.ext, wsum);
            cur ^= 1;
        }
        if (L.active) {
            if (t + 1 < g.nsteps)
                store_state<T, DRONE>(g.traj.f, (size_t)t * EA + L.idx, st);
            else
                store_state<T, DRONE>(g.fin.f, L.idx, st);
        }
        for (int q = L.i; q < NW; q += AP) io.traj[(size_t)t * ENW + eo + q] = B.ob[cur * NW + q];
    }
}

// ------------------------------------------------------------------ backward rollout

template <typename T, bool DRONE, bool GRID, unsigned F>
__global__ __launch_bounds__(1024) void k_wbody_bwd(const Cst<T> Cin, const Args<T> g,
                                                    const ObTab<T> tb, const ObIO<T> io)
{
    const Cst<T> C = fold_cst<F>(Cin);
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t wsum[16];
    const int AP = blockDim.x, N = tb.N, NW = OB_W * N;
    const int NC = C.grid_bins > 0 ? C.grid_bins * C.grid_bins : 0;
    const WideLds<T> W = wide_lds<T>(smem, AP);
    const WBodyLds<T> B = wbody_lds<T>(smem, AP, NC, N, true);
    T *const obk = B.ob;                 // the step's checkpoint obstacle state
    T *const obr[2] = {B.ob + NW, B.ob + 2 * NW};  // recompute buffers
    T *gob = B.ob + 3 * NW;              // adjoint of the current substep's output
    T *gprev = B.ob + 4 * NW;            // adjoint of its input
    const GridFrame<T> G = grid_frame(C, (const T *)nullptr);
    WLane<T> L;
    wide_init<T, F>(C, g, L);
    W.rad[L.i] = L.pr.radius;
    ShapeSets<T, !(F & FT_MANYSH)> SS;
    SS.init(tb, L.i & 63);
    const WideEnv<T> X{L.i, AP, L.active, B.scr, B.flags};
    const BodyRow<T> br = wbody_row(C, tb, L);
    for (int o = L.i; o < N; o += AP) B.ext[o] = body_ext(tb, o);
    const size_t eo = (size_t)L.env * NW, ENW = (size_t)C.E * NW;
    for (int q = L.i; q < NW; q += AP) gob[q] = T(0);
    const size_t EA = (size_t)C.E * C.A;
    St<T> gs;
    st_zero(gs);
    for (int t = g.nsteps - 1; t >= 0; --t) {
        if (L.active) {
            if (t == g.nsteps - 1)
                add_adj<T, DRONE>(g.afin.f, L.idx, gs);
            else
                add_adj<T, DRONE>(g.atraj.f, (size_t)t * EA + L.idx, gs);
        }
        __syncthreads();
        if (io.atraj)
            for (int q = L.i; q < NW; q += AP) gob[q] += io.atraj[(size_t)t * ENW + eo + q];
        {
            const T *src = t == 0 ? io.ob0 + eo : io.traj + (size_t)(t - 1) * ENW + eo;
            for (int q = L.i; q < NW; q += AP) obk[q] = src[q];
        }
        St<T> st0;
        if (t == 0)
            load_state<T, DRONE>(g.s0.f, L.idx, 0, st0);
        else
            load_state<T, DRONE>(g.traj.f, L.idx, (size_t)(t - 1) * EA, st0);
        if (!L.active) st0.px = st0.py = __builtin_nan("");
        T a[4];
        load_act(g.act, (size_t)t * EA + L.idx, C.ad, a);
        __syncthreads();
        T ga[4] = {T(0), T(0), T(0), T(0)};
        for (int s = C.S - 1; s >= 0; --s) {
            // the substep's input (agents and obstacles), recomputed from the checkpoint
            St<T> in = st0;
            const T *obc = obk;
            for (int q = 0; q < s; ++q) {
                wbody_substep<T, DRONE, GRID>(C, tb, SS, X, br, W, G, L, a, in, obc, obr[q & 1],
                                              B.ext, wsum);
                obc = obr[q & 1];
            }
            T Fx, Fy;
            int32_t cut;
            if (C.collisions) wide_publish<T, GRID>(C, W, G, L, in, wsum);
            wbody_forces<T, GRID>(C, tb, W, G, L, in, obc, Fx, Fy, cut);
            St<T> gi;
            T gFx, gFy;
            integrate_adj<T, DRONE>(C, L.pr, in, a, Fx, Fy, gs, gi, ga, gFx, gFy);
            // the body pass: adjoint of its input obstacle state into gprev
            body_pass_adj<T>(C, tb, SS, X, br, in, obc, gob, gprev, gi, B.ext, nullptr, nullptr,
                             nullptr);
            if (C.collisions) {
                const T wFx = gFx * L.inv_dd, wFy = gFy * L.inv_dd;
                W.wfx[L.i] = wFx;
                W.wfy[L.i] = wFy;
                W.cut[L.i] = cut;
                __syncthreads();
                if (L.active) {
                    // every in-radius pair, both sides: own (j in i's list), rev (i in j's)
                    visit_list<T, GRID>(
                        W, C.A, G, L.i, in.px, in.py, C.t_nbr, C.A, false,
                        [&](int j, int32_t key) {
                            const bool own = key <= cut;
                            const int32_t kin = GRID ? grid_key_in(W, G.bins, L.i, j) : L.i;
                            const bool rev = kin <= W.cut[j];
                            if (!own && !rev) return;
                            const T wx = (own ? wFx : T(0)) - (rev ? W.wfx[j] : T(0));
                            const T wy = (own ? wFy : T(0)) - (rev ? W.wfy[j] : T(0));
                            pair_adj_combined(C, in.px - W.px[j], in.py - W.py[j],
                                              in.vx - W.vx[j], in.vy - W.vy[j],
                                              L.pr.radius + W.rad[j] + C.margin, wx, wy, gi.px,
                                              gi.py, gi.vx, gi.vy);
                        });
                }
            }
            // obstacles: the agent's adjoint, and the moving shapes' over the env's agents
            for (int o = 0; o < N; ++o) {
                const bool mv = SS.moves(tb, o);
                T op[6];
                if (L.active) {
                    ob_force_adj(C, tb, obc, o, in.px, in.py, in.vx, in.vy, L.pr.radius, L.dd,
                                 gFx, gFy, gi, mv, op);
                } else {
#pragma unroll
                    for (int q = 0; q < 6; ++q) op[q] = T(0);
                }
                if (!mv) continue;
                bool fl = false;
#pragma unroll
                for (int q = 0; q < 6; ++q) fl = fl || op[q] != T(0);
                if (!X.any(fl)) continue;  // no agent of the env touches it
                T *g2 = gprev + 6 * o;
                T acc[6] = {g2[0], g2[1], g2[2], g2[3], g2[4], g2[5]};
                X.template ordered<6>(acc, op, fl);
                __syncthreads();  // every thread has read g2
                if (L.i == 0) {
#pragma unroll
                    for (int q = 0; q < 6; ++q) g2[q] = acc[q];
                }
            }
            if (C.soft_walls && L.active)
                wall_force_adj(C, in.px, in.py, in.vx, in.vy, L.pr.radius, L.dd, gFx, gFy, gi);
            gs = gi;
            __syncthreads();
            T *tmp = gob;
            gob = gprev;
            gprev = tmp;
        }
        if (L.active) {
            T *pa = g.aact + ((size_t)t * EA + L.idx) * C.ad;
            for (int k = 0; k < C.ad; ++k) pa[k] = k < 4 ? ga[k] : T(0);
        }
    }
    if (L.active) store_adj<T, DRONE>(g.a0.f, L.idx, gs);
    __syncthreads();
    if (io.a0)
        for (int q = L.i; q < NW; q += AP) io.a0[eo + q] = gob[q];
}

// ---------------------------------------------------------------------- launchers

// LDS of one workgroup of the wide body kernels: dynamic staging plus the static wsum[16].
template <typename T> size_t wbody_shm(const Cst<T> &C, int N, bool bwd)
{
    return wbody_lds_bytes<T>(wide_threads<T>(C.A), C.grid_bins > 0 ? C.grid_bins * C.grid_bins : 0,
                              N, bwd);
}

#define SWARP_WBODY_DISPATCH(KERNEL, SHM)                                                       \
    if (drone) {                                                                                \
        if (grid) hipLaunchKernelGGL((KERNEL<T, true, true, FT_ALL>), g, b, SHM, st, C, a, tb, io); \
        else hipLaunchKernelGGL((KERNEL<T, true, false, FT_ALL>), g, b, SHM, st, C, a, tb, io);     \
    } else {                                                                                    \
        if (grid) hipLaunchKernelGGL((KERNEL<T, false, true, FT_ALL>), g, b, SHM, st, C, a, tb, io);\
        else hipLaunchKernelGGL((KERNEL<T, false, false, FT_ALL>), g, b, SHM, st, C, a, tb, io);    \
    }

template <typename T>
void launch_wbody_fwd(bool drone, const Cst<T> &C, const Args<T> &a, const ObTab<T> &tb,
                      const ObIO<T> &io, hipStream_t st)
{
    const dim3 g(C.E), b(wide_threads<T>(C.A));
    const bool grid = C.grid_bins > 0;
    const size_t shm = wbody_shm<T>(C, tb.N, false);
    SWARP_WBODY_DISPATCH(k_wbody_fwd, shm)
}

template <typename T>
void launch_wbody_bwd(bool drone, const Cst<T> &C, const Args<T> &a, const ObTab<T> &tb,
                      const ObIO<T> &io, hipStream_t st)
{
    const dim3 g(C.E), b(wide_threads<T>(C.A));
    const bool grid = C.grid_bins > 0;
    const size_t shm = wbody_shm<T>(C, tb.N, true);
    SWARP_WBODY_DISPATCH(k_wbody_bwd, shm)
}
#undef SWARP_WBODY_DISPATCH

}  // namespace swarp
