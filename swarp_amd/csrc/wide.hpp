// wide.hpp -- envs of up to 4096 agents, and the uniform-grid list order.
//
// The generic and specialised kernels put a whole env into one wave (at most 64 agents,
// the lists as 64-bit masks).  These kernels give each env one workgroup of up to 16
// waves, one lane per agent up to 1024 agents and 2 or 4 agents per lane beyond
// (wide_geom: agent i = thread + k * threads), with the env's positions, velocities and
// radii in LDS.  They serve every 2-D or drone fleet (any model, control mode, obstacles,
// walls, clamp, integrator, box agents, wheel contacts) of more than 64 agents per env,
// and every fleet whose lists follow the uniform grid, as far as the env's staging fits
// the 160 KiB of LDS of a workgroup.
//
// List order (which K in-radius neighbours a capped list keeps, and the order the pair
// forces are summed in):
//   brute  ascending agent index (_brute_force, swarp/core/neighbors.py:76-97);
//   grid   the uniform grid's (_query_uniform, swarp/core/neighbors.py:214-251): the cells
//          of the 3x3 block around the agent's cell row by row (dy outer, dx inner), the
//          agents of a cell in ascending index (the stable sort of the (env, cell) keys,
//          :184-211, 663-666).  A cell is (int)((p - origin) / cell_size) per axis,
//          clamped to [0, bins); the frame (origin, cell size) is pinned by the world
//          bounds or, for list builds, reduced over the batch (:149-181).
// Every list position has a traversal key -- the agent index (brute), or slot * 4096 +
// rank in its cell with slot = 3 (dy + 1) + (dx + 1) (grid) -- increasing along the
// traversal, so "j is in i's capped list" is "j within radius of i and key_i(j) <=
// cut_i", where cut_i is the key of i's K-th listed neighbour (INT_MAX when fewer).  The
// backward gathers each pair's two sides with that test, as the generic kernels do with
// their masks.
//
// The backward recomputes, for each substep in reverse, the substeps before it from the
// step's checkpoint (S (S + 1) / 2 forward substeps per step): no per-substep state of
// the env has to fit in LDS.
//
// Box worlds (BOXES: some agent is a box, or wheel contacts) also stage each agent's
// heading, spin and heading cos / sin per substep and its footprint per launch (WBoxLds):
// a pair with a box takes the box law, a box agent its obstacles and walls through the
// box statics, as the one-wave kernels do; their reverse evaluates each listed box pair
// (both sides, as for discs) and a box agent's statics with the forward-mode tangents of
// box_item_adj / box_static_adj.
#pragma once
#include "common.hpp"

namespace swarp {

constexpr int WIDE_MAX_AGENTS = 4096;
constexpr int32_t CUT_ALL = 0x7fffffff;

// Uniform-grid frame of one launch: origin and cell size (from Cst for a pinned frame,
// from `frame` [3] on the device for a batch-reduced one).
template <typename T> struct GridFrame {
    T ox, oy, cs;
    int bins;
};

// One axis of a cell index (_compute_keys / _query_uniform, swarp/core/neighbors.py:
// 188-193, 230-232): truncation toward zero of (p - o) / cs, clamped to [0, bins).
template <typename T> __device__ __forceinline__ int grid_axis(T p, T o, T cs, int bins)
{
    const T q = (p - o) / cs;
    int c = (int)q;
    if (!(q == q)) c = 0;
    return c < 0 ? 0 : (c > bins - 1 ? bins - 1 : c);
}

// LDS of one wide workgroup (AP = waves * 64 agent slots, NC = cells or 0).
template <typename T> struct WideLds {
    T *px, *py, *vx, *vy, *rad, *wfx, *wfy;
    int32_t *cut, *key, *rank, *sorted, *cstart;
};

template <typename T> __host__ __device__ inline size_t wide_lds_bytes(int AP, int NC)
{
    return (size_t)AP * (7 * sizeof(T) + 4 * sizeof(int32_t)) + (size_t)(NC + 1) * sizeof(int32_t);
}

template <typename T> __device__ __forceinline__ WideLds<T> wide_lds(unsigned char *smem, int AP)
{
    WideLds<T> W;
    T *t = (T *)smem;
    W.px = t;
    W.py = t + AP;
    W.vx = t + 2 * AP;
    W.vy = t + 3 * AP;
    W.rad = t + 4 * AP;
    W.wfx = t + 5 * AP;
    W.wfy = t + 6 * AP;
    int32_t *q = (int32_t *)(t + 7 * AP);
    W.cut = q;
    W.key = q + AP;
    W.rank = q + 2 * AP;
    W.sorted = q + 3 * AP;
    W.cstart = q + 4 * AP;
    return W;
}

// Box worlds: each agent's heading, spin and heading cos / sin this substep and its
// footprint (shape, half-extents), after the staging above (16-byte aligned).
template <typename T> struct WBoxLds {
    T *th, *w, *cs, *sn, *shp, *hx, *hy;
};

template <typename T> __host__ __device__ inline size_t wide_box_offset(int AP, int NC)
{
    return (wide_lds_bytes<T>(AP, NC) + 15) / 16 * 16;
}

template <typename T> __host__ __device__ inline size_t wide_box_lds_bytes(int AP, int NC)
{
    return wide_box_offset<T>(AP, NC) + (size_t)7 * AP * sizeof(T);
}

template <typename T>
__device__ __forceinline__ WBoxLds<T> wide_box_lds(unsigned char *smem, int AP, int NC)
{
    T *b = (T *)(smem + wide_box_offset<T>(AP, NC));
    WBoxLds<T> B;
    B.th = b;
    B.w = b + AP;
    B.cs = b + 2 * AP;
    B.sn = b + 3 * AP;
    B.shp = b + 4 * AP;
    B.hx = b + 5 * AP;
    B.hy = b + 6 * AP;
    return B;
}

// Exclusive prefix sum of v[0 .. n) in place over the workgroup; v[n] = the total.
__device__ inline void block_exclusive_scan(int32_t *v, int n, int32_t *wsum)
{
    const int nt = blockDim.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int per = (n + nt - 1) / nt;
    const int lo = tid * per, hi = min(n, lo + per);
    int32_t s = 0;
    for (int c = lo; c < hi; ++c) s += v[c];
    int32_t x = s;  // inclusive scan of the per-thread sums
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    int32_t before = 0;
    for (int w = 0; w < wv; ++w) before += wsum[w];
    int32_t run = before + x - s;
    __syncthreads();
    for (int c = lo; c < hi; ++c) {
        const int32_t t = v[c];
        v[c] = run;
        run += t;
    }
    if (tid == nt - 1) v[n] = before + x;
    __syncthreads();
}

// Cells of the env's agents: key[i] (cell id), rank[i] (agents of the same cell with a
// smaller index), cstart[c] (first sorted slot of cell c, cstart[NC] = A), sorted[]
// (agent indices cell by cell, ascending within a cell).  The
// positions are in W.px / W.py.  Every thread of the workgroup calls it.
template <typename T>
__device__ inline void grid_build(const WideLds<T> &W, int A, const GridFrame<T> &G,
                                  int32_t *wsum)
{
    const int tid = threadIdx.x, nt = blockDim.x, NC = G.bins * G.bins;
    for (int c = tid; c < NC; c += nt) W.cstart[c] = 0;
    __syncthreads();
    for (int i = tid; i < A; i += nt) {
        const int cx = grid_axis(W.px[i], G.ox, G.cs, G.bins);
        const int cy = grid_axis(W.py[i], G.oy, G.cs, G.bins);
        const int k = cy * G.bins + cx;
        W.key[i] = k;
        atomicAdd(&W.cstart[k], 1);
    }
    __syncthreads();
    block_exclusive_scan(W.cstart, NC, wsum);
    for (int i = tid; i < A; i += nt) {
        const int k = W.key[i];
        int r = 0;  // agents of the same cell with a smaller index
        for (int j = 0; j < i; ++j) r += W.key[j] == k ? 1 : 0;
        W.rank[i] = r;
        W.sorted[W.cstart[k] + r] = i;
    }
    __syncthreads();
}

// Visits agent i's in-radius neighbours in list order: f(j, traversal key) for each of the
// first `limit` of them.  Returns the number of in-radius neighbours visited (all of them
// when count_all, else at most limit).  Positions from W.
template <typename T, bool GRID, typename Fn>
__device__ __forceinline__ int visit_list(const WideLds<T> &W, int A, const GridFrame<T> &G,
                                          int i, T px, T py, T t_nbr, int limit, bool count_all,
                                          Fn &&f)
{
    int n = 0;
    if (!GRID) {
        for (int j0 = 0; j0 < A; j0 += 64) {
            uint64_t m = 0;
            const int jn = min(64, A - j0);
            for (int b = 0; b < jn; ++b) {
                const int j = j0 + b;
                const T dx = W.px[j] - px, dy = W.py[j] - py;
                const T d2 = dx * dx + dy * dy;
                m |= (d2 <= t_nbr && j != i) ? (1ull << b) : 0ull;
            }
            while (m && n < limit) {
                const int b = __builtin_ctzll(m);
                m &= m - 1;
                f(j0 + b, j0 + b);
                ++n;
            }
            if (count_all) n += __builtin_popcountll(m);
            if (!count_all && n >= limit) break;
        }
        return n;
    }
    const int k = W.key[i], cx = k % G.bins, cy = k / G.bins;
    for (int sy = 0; sy < 3; ++sy) {
        const int ny = cy + sy - 1;
        if (ny < 0 || ny >= G.bins) continue;
        for (int sx = 0; sx < 3; ++sx) {
            const int nx = cx + sx - 1;
            if (nx < 0 || nx >= G.bins) continue;
            const int c = ny * G.bins + nx, c0 = W.cstart[c], c1 = W.cstart[c + 1];
            for (int si = c0; si < c1; ++si) {
                const int j = W.sorted[si];
                const T dx = W.px[j] - px, dy = W.py[j] - py;
                const T d2 = dx * dx + dy * dy;
                if (!(d2 <= t_nbr) || j == i) continue;
                if (n < limit) f(j, (3 * sy + sx) * WIDE_MAX_AGENTS + (si - c0));
                ++n;
                if (!count_all && n >= limit) return n;
            }
        }
    }
    return n;
}

// Traversal key of agent i's position in agent j's grid list (i within radius of j, so
// i's cell lies in the 3x3 block around j's).
template <typename T>
__device__ __forceinline__ int32_t grid_key_in(const WideLds<T> &W, int bins, int i, int j)
{
    const int ki = W.key[i], kj = W.key[j];
    const int sx = ki % bins - kj % bins + 1, sy = ki / bins - kj / bins + 1;
    return (3 * sy + sx) * WIDE_MAX_AGENTS + W.rank[i];
}

// Frame of this launch.
template <typename T>
__device__ __forceinline__ GridFrame<T> grid_frame(const Cst<T> &C, const T *frame)
{
    GridFrame<T> G;
    G.bins = C.grid_bins;
    if (frame) {
        G.ox = frame[0];
        G.oy = frame[1];
        G.cs = frame[2];
    } else {
        G.ox = C.grid_ox;
        G.oy = C.grid_oy;
        G.cs = C.grid_cs;
    }
    return G;
}

// ------------------------------------------------------------------ frame reduction

// _bounds_init / _bounds_reduce / _finalize_grid (swarp/core/neighbors.py:149-181): the
// batch's min corner, extent max(dx, dy), cell size max(radius, extent / bins), in T.
template <typename T>
__global__ __launch_bounds__(1024) void k_grid_frame(const T *pos, int64_t n, T radius, int bins,
                                                     T *frame)
{
    __shared__ T red[4][16];
    const T big = T(1e30);
    T mnx = big, mny = big, mxx = -big, mxy = -big;
    for (int64_t q = threadIdx.x; q < n; q += 1024) {
        const T x = pos[2 * q], y = pos[2 * q + 1];
        mnx = x < mnx ? x : mnx;
        mny = y < mny ? y : mny;
        mxx = x > mxx ? x : mxx;
        mxy = y > mxy ? y : mxy;
    }
    for (int d = 32; d > 0; d >>= 1) {
        const T a = __shfl_down(mnx, d, 64), b = __shfl_down(mny, d, 64);
        const T c = __shfl_down(mxx, d, 64), e = __shfl_down(mxy, d, 64);
        mnx = a < mnx ? a : mnx;
        mny = b < mny ? b : mny;
        mxx = c > mxx ? c : mxx;
        mxy = e > mxy ? e : mxy;
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][wv] = mnx;
        red[1][wv] = mny;
        red[2][wv] = mxx;
        red[3][wv] = mxy;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w) {
            mnx = red[0][w] < mnx ? red[0][w] : mnx;
            mny = red[1][w] < mny ? red[1][w] : mny;
            mxx = red[2][w] > mxx ? red[2][w] : mxx;
            mxy = red[3][w] > mxy ? red[3][w] : mxy;
        }
        const T ex = mxx - mnx, ey = mxy - mny;
        const T ext = ex > ey ? ex : ey;
        const T q = ext / T(bins);
        frame[0] = mnx;
        frame[1] = mny;
        frame[2] = radius > q ? radius : q;
    }
}

// ------------------------------------------------------------------ neighbour lists

// Launch geometry of the workgroup of an env of A agents: `apt` agents per thread (1, 2
// or 4; agent i = thread + k * threads), `threads` a multiple of 64 up to 1024, `slots` =
// threads * apt >= A staging entries per array.
struct WideGeom {
    int apt, threads, slots;
};

__host__ __device__ inline WideGeom wide_geom(int A)
{
    const int ap = (A + 63) / 64 * 64;
    int apt = (ap + 1023) / 1024;
    if (apt == 3) apt = 4;
    const int th = ((ap + apt - 1) / apt + 63) / 64 * 64;
    return {apt, th, th * apt};
}

// Padded lists, counts and true counts of one env per workgroup (brute or grid order).
template <typename T, bool GRID>
__global__ __launch_bounds__(1024) void k_wide_lists(const Cst<T> C, const T *pos, const T *frame,
                                                     int32_t *idx, int32_t *cnt, int32_t *tru)
{
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t wsum[16];
    const int nt = blockDim.x, A = C.A, env = blockIdx.x;
    const int AP = nt * wide_geom(A).apt;
    const WideLds<T> W = wide_lds<T>(smem, AP);
    const GridFrame<T> G = grid_frame(C, frame);
    for (int i = threadIdx.x; i < AP; i += nt) {
        const size_t row = (size_t)env * A + (i < A ? i : 0);
        W.px[i] = i < A ? pos[2 * row] : T(0);
        W.py[i] = i < A ? pos[2 * row + 1] : T(0);
    }
    __syncthreads();
    if (GRID) grid_build(W, A, G, wsum);
    for (int i = threadIdx.x; i < A; i += nt) {
        const size_t row = (size_t)env * A + i;
        int32_t *out = idx + row * C.K;
        const int n = visit_list<T, GRID>(W, A, G, i, W.px[i], W.py[i], C.t_nbr, C.K, true,
                                          [&](int j, int32_t) { *out++ = j; });
        const int c = n < C.K ? n : C.K;
        for (int q = c; q < C.K; ++q) idx[row * C.K + q] = 0;
        cnt[row] = c;
        if (tru) tru[row] = n;
    }
}

// ------------------------------------------------------------------ rollout kernels

template <typename T> struct WLane {
    int i, env;
    bool active;
    size_t idx;
    Prm<T> pr;
    T dd, inv_dd;
    Dv<T> ddv;
};

template <typename T, unsigned F>
__device__ __forceinline__ void wide_init(const Cst<T> &C, const Args<T> &g, WLane<T> &L,
                                          int i = (int)threadIdx.x)
{
    L.i = i;
    L.env = blockIdx.x;
    L.active = L.i < C.A;
    const int ag = L.active ? L.i : 0;
    L.idx = (size_t)L.env * C.A + ag;
    load_prm(g, C.per_env ? L.idx : (size_t)ag, ag, L.pr);
    fold_prm<F>(L.pr);
    L.dd = T(1) + C.c * C.sub_dt / L.pr.mass;
    L.inv_dd = T(1) / L.dd;
    L.ddv = divisor(L.dd, true);
}

// Publishes the substep's positions and velocities (and the grid) -- every thread.  `B`
// (box worlds, else NULL): also the headings, spins and heading cos / sin.
template <typename T, bool GRID>
__device__ __forceinline__ void wide_publish(const Cst<T> &C, const WideLds<T> &W,
                                             const GridFrame<T> &G, const WLane<T> &L,
                                             const St<T> &st, int32_t *wsum,
                                             const WBoxLds<T> *B = nullptr)
{
    __syncthreads();
    wide_put(W, L, st, B);
    __syncthreads();
    if (GRID && C.collisions) grid_build(W, C.A, G, wsum);
}

// Contact and static forces of the lane's agent (collision_forces_kernel, swarp/core/
// collisions.py:818-881: listed pairs in list order, then obstacles, then walls); `cut`
// receives the key of the K-th listed neighbour (CUT_ALL when the list is not full).
// `obst(sx, sy)` adds the obstacle forces of an active lane (the static obstacles of
// `g.obs` in wide_forces; the env's obstacle state in the movable-body kernels).
template <typename T, bool GRID, typename ObF>
__device__ __forceinline__ void wide_forces_with(const Cst<T> &C, const WideLds<T> &W,
                                                 const GridFrame<T> &G, const WLane<T> &L,
                                                 const St<T> &st, T &Fx, T &Fy, int32_t &cut,
                                                 ObF &&obst)
{
    T fx = T(0), fy = T(0);
    cut = CUT_ALL;
    if (C.collisions && L.active) {
        const T ra = L.pr.radius;
        int n = 0;
        int32_t last = CUT_ALL;
        visit_list<T, GRID>(W, C.A, G, L.i, st.px, st.py, C.t_nbr, C.K, false,
                            [&](int j, int32_t key) {
                                T gx, gy;
                                pair_force(C, st.px - W.px[j], st.py - W.py[j], st.vx - W.vx[j],
                                           st.vy - W.vy[j], ra + W.rad[j] + C.margin, L.ddv, gx, gy);
                                fx += gx;
                                fy += gy;
                                last = key;
                                ++n;
                            });
        if (n >= C.K) cut = last;
    }
    T sx = T(0), sy = T(0);
    if (L.active) obst(sx, sy);
    if (C.soft_walls) {
        T gx, gy;
        unsigned wb;
        wall_force_axes(C, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx, gy, wb);
        sx += gx;
        sy += gy;
    }
    Fx = fx + sx;
    Fy = fy + sy;
}

template <typename T, bool GRID>
__device__ __forceinline__ void wide_forces(const Cst<T> &C, const Args<T> &g,
                                            const WideLds<T> &W, const GridFrame<T> &G,
                                            const WLane<T> &L, const St<T> &st, T &Fx, T &Fy,
                                            int32_t &cut)
{
    wide_forces_with<T, GRID>(C, W, G, L, st, Fx, Fy, cut, [&](T &sx, T &sy) {
        const size_t eN = (size_t)L.env * C.N;
        for (int o = 0; o < C.N; ++o) {
            T gx, gy;
            obstacle_force(C, g.obs, eN, o, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx, gy);
            sx += gx;
            sy += gy;
        }
    });
}

// The forces of a box world (collision_forces_box_kernel, swarp/core/collisions.py:
// 999-1059; the order of forces(): listed pairs, then a box agent's statics -- obstacles
// then walls, _static_forces_shaped :950-996 -- or a disc's obstacles and walls).  A pair
// with a box takes the box law with the lower index as box A.  `tq` (nullable): the
// contact torque about the agent's centre (wheel contacts, :1128-1403).
template <typename T, bool GRID>
__device__ __forceinline__ void wide_forces_box(const Cst<T> &C, const Args<T> &g,
                                                const WideLds<T> &W, const WBoxLds<T> &B,
                                                const GridFrame<T> &G, const WLane<T> &L,
                                                const St<T> &st, T &Fx, T &Fy, int32_t &cut,
                                                T *tq)
{
    const bool box_me = L.pr.shape > T(0.5);
    const T cme = m_cos(st.th), sme = m_sin(st.th);
    const T me[6] = {st.px, st.py, st.th, st.vx, st.vy, st.w};
    const Foot<T> fa = {L.pr.shape, L.pr.radius, L.pr.hx, L.pr.hy};
    T fx = T(0), fy = T(0), tau = T(0);
    cut = CUT_ALL;
    if (C.collisions && L.active) {
        int n = 0;
        int32_t last = CUT_ALL;
        visit_list<T, GRID>(W, C.A, G, L.i, st.px, st.py, C.t_nbr, C.K, false,
                            [&](int j, int32_t key) {
                                T gx, gy;
                                if (box_me || B.shp[j] > T(0.5)) {
                                    const Foot<T> fb = {B.shp[j], W.rad[j], B.hx[j], B.hy[j]};
                                    const T ob[6] = {W.px[j], W.py[j], B.th[j],
                                                     W.vx[j], W.vy[j], B.w[j]};
                                    agent_pair_force_box<T, T>(C, L.i, j, fa, me, cme, sme, fb,
                                                               ob, B.cs[j], B.sn[j], L.dd, gx,
                                                               gy);
                                    if (tq)
                                        tau += pair_torque(C, L.i, j, fa, me, cme, sme, fb, ob,
                                                           B.cs[j], B.sn[j], gx, gy);
                                } else {
                                    pair_force(C, st.px - W.px[j], st.py - W.py[j],
                                               st.vx - W.vx[j], st.vy - W.vy[j],
                                               L.pr.radius + W.rad[j] + C.margin, L.ddv, gx, gy);
                                }
                                fx += gx;
                                fy += gy;
                                last = key;
                                ++n;
                            });
        if (n >= C.K) cut = last;
    }
    T sx = T(0), sy = T(0);
    if (L.active) {
        const size_t eN = (size_t)L.env * C.N;
        if (box_me) {
            box_static_forces<T, T>(C, g.obs, eN, nullptr, L.pr.hx, L.pr.hy, me, cme, sme, L.dd,
                                    sx, sy);
            if (tq)
                tau = tau + box_static_torque(C, g.obs, eN, (const T *)nullptr, L.pr.hx, L.pr.hy,
                                              me, cme, sme, L.dd);
        } else {
            for (int o = 0; o < C.N; ++o) {
                T gx, gy;
                obstacle_force(C, g.obs, eN, o, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv,
                               gx, gy);
                sx += gx;
                sy += gy;
            }
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
    if (tq) *tq = tau;
}

// Stores one agent's state of this substep in the env's staging (box worlds: also its
// heading, spin and heading cos / sin).
template <typename T>
__device__ __forceinline__ void wide_put(const WideLds<T> &W, const WLane<T> &L, const St<T> &st,
                                         const WBoxLds<T> *B)
{
    W.px[L.i] = st.px;
    W.py[L.i] = st.py;
    W.vx[L.i] = st.vx;
    W.vy[L.i] = st.vy;
    if (B) {
        B->th[L.i] = st.th;
        B->w[L.i] = st.w;
        B->cs[L.i] = m_cos(st.th);
        B->sn[L.i] = m_sin(st.th);
    }
}

// One agent's forces of a substep whose state is published.
template <typename T, bool GRID, bool BOXES>
__device__ __forceinline__ void wide_agent_forces(const Cst<T> &C, const Args<T> &g,
                                                  const WideLds<T> &W, const WBoxLds<T> &B,
                                                  const GridFrame<T> &G, const WLane<T> &L,
                                                  const St<T> &st, T &Fx, T &Fy, int32_t &cut,
                                                  T *tq)
{
    if constexpr (BOXES)
        wide_forces_box<T, GRID>(C, g, W, B, G, L, st, Fx, Fy, cut, tq);
    else
        wide_forces<T, GRID>(C, g, W, G, L, st, Fx, Fy, cut);
}

// One substep of the APT agents of each thread (agent i = thread + k * threads).  Box
// worlds with wheel contacts integrate unclamped, rework the step with wheel_contact, then
// clamp (integrate2d_wheel_kernel, swarp/dynamics/kernels.py:1389-1478).
template <typename T, bool DRONE, bool GRID, bool BOXES, int APT>
__device__ __forceinline__ void wide_substep(const Cst<T> &C, const Args<T> &g,
                                             const WideLds<T> &W, const WBoxLds<T> &B,
                                             const GridFrame<T> &G, const WLane<T> (&L)[APT],
                                             const T (&a)[APT][4], St<T> (&st)[APT],
                                             int32_t *wsum)
{
    T Fx[APT], Fy[APT], Tq[APT];
#pragma unroll
    for (int k = 0; k < APT; ++k) Fx[k] = Fy[k] = Tq[k] = T(0);
    if (C.needs_forces) {
        if (C.collisions) {
            __syncthreads();
#pragma unroll
            for (int k = 0; k < APT; ++k) wide_put(W, L[k], st[k], BOXES ? &B : nullptr);
            __syncthreads();
            if (GRID) grid_build(W, C.A, G, wsum);
        }
#pragma unroll
        for (int k = 0; k < APT; ++k) {
            int32_t cut;
            wide_agent_forces<T, GRID, BOXES>(C, g, W, B, G, L[k], st[k], Fx[k], Fy[k], cut,
                                              BOXES && C.wheel ? &Tq[k] : nullptr);
        }
    }
#pragma unroll
    for (int k = 0; k < APT; ++k) {
        St<T> nx;
        if constexpr (BOXES) {
            if (C.wheel) {
                Cst<T> C0 = C;
                C0.clamp = 0;
                integrate<T, DRONE>(C0, L[k].pr, st[k], a[k], Fx[k], Fy[k], nx);
                wheel_contact(C, L[k].pr, st[k], Fx[k], Fy[k], Tq[k], nx);
                if (C.clamp) clamp_position(C, L[k].pr, nx.th, nx.px, nx.py);
                st[k] = nx;
                continue;
            }
        }
        integrate<T, DRONE>(C, L[k].pr, st[k], a[k], Fx[k], Fy[k], nx);
        st[k] = nx;
    }
}

// Footprints of a box world's agents, once per launch.
template <typename T>
__device__ __forceinline__ void wide_box_init(const WBoxLds<T> &B, const WLane<T> &L)
{
    B.shp[L.i] = L.pr.shape;
    B.hx[L.i] = L.pr.hx;
    B.hy[L.i] = L.pr.hy;
}

template <typename T> __device__ __forceinline__ int wide_cells(const Cst<T> &C)
{
    return C.grid_bins > 0 ? C.grid_bins * C.grid_bins : 0;
}

// The lanes of the launch: APT agents per thread, thread + k * threads.
template <typename T, bool BOXES, int APT, unsigned F>
__device__ __forceinline__ void wide_lanes(const Cst<T> &C, const Args<T> &g, const WideLds<T> &W,
                                           const WBoxLds<T> &B, WLane<T> (&L)[APT])
{
#pragma unroll
    for (int k = 0; k < APT; ++k) {
        wide_init<T, F>(C, g, L[k], (int)(threadIdx.x + k * blockDim.x));
        W.rad[L[k].i] = L[k].pr.radius;
        if (BOXES) wide_box_init(B, L[k]);
    }
}

template <typename T, bool DRONE, bool GRID, bool BOXES, int APT, unsigned F>
__global__ __launch_bounds__(1024) void k_wide_fwd(const Cst<T> Cin, const Args<T> g)
{
    const Cst<T> C = fold_cst<F>(Cin);
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t wsum[16];
    const int AP = (int)blockDim.x * APT;
    const WideLds<T> W = wide_lds<T>(smem, AP);
    const WBoxLds<T> B = wide_box_lds<T>(smem, AP, wide_cells(C));
    const GridFrame<T> G = grid_frame(C, (const T *)nullptr);
    WLane<T> L[APT];
    wide_lanes<T, BOXES, APT, F>(C, g, W, B, L);
    St<T> st[APT];
#pragma unroll
    for (int k = 0; k < APT; ++k) load_state<T, DRONE>(g.s0.f, L[k].idx, 0, st[k]);
    const size_t EA = (size_t)C.E * C.A;
    for (int t = 0; t < g.nsteps; ++t) {
        T a[APT][4];
#pragma unroll
        for (int k = 0; k < APT; ++k) load_act(g.act, (size_t)t * EA + L[k].idx, C.ad, a[k]);
        for (int s = 0; s < C.S; ++s)
            wide_substep<T, DRONE, GRID, BOXES, APT>(C, g, W, B, G, L, a, st, wsum);
#pragma unroll
        for (int k = 0; k < APT; ++k) {
            if (!L[k].active) continue;
            if (t + 1 < g.nsteps)
                store_state<T, DRONE>(g.traj.f, (size_t)t * EA + L[k].idx, st[k]);
            else
                store_state<T, DRONE>(g.fin.f, L[k].idx, st[k]);
        }
    }
}

// Reverse of one agent's forces of a substep (published state and force adjoints /
// damping denominators `wF`, cut keys): every in-radius pair, both sides -- own (j in
// i's list), rev (i in j's) -- then the obstacles and walls.
template <typename T, bool GRID, bool BOXES>
__device__ __forceinline__ void wide_agent_adj(const Cst<T> &C, const Args<T> &g,
                                               const WideLds<T> &W, const WBoxLds<T> &B,
                                               const GridFrame<T> &G, const WLane<T> &L,
                                               const St<T> &in, T gFx, T gFy, int32_t cut,
                                               St<T> &gi)
{
    if (!L.active) return;
    const bool box_me = BOXES && L.pr.shape > T(0.5);
    const Foot<T> fa = {L.pr.shape, L.pr.radius, L.pr.hx, L.pr.hy};
    if (C.collisions) {
        const T wFx = W.wfx[L.i], wFy = W.wfy[L.i];
        visit_list<T, GRID>(
            W, C.A, G, L.i, in.px, in.py, C.t_nbr, C.A, false, [&](int j, int32_t key) {
                const bool own = key <= cut;
                const int32_t kin = GRID ? grid_key_in(W, G.bins, L.i, j) : L.i;
                const bool rev = kin <= W.cut[j];
                if (!own && !rev) return;
                const T wx = (own ? wFx : T(0)) - (rev ? W.wfx[j] : T(0));
                const T wy = (own ? wFy : T(0)) - (rev ? W.wfy[j] : T(0));
                if constexpr (BOXES) {
                    if (box_me || B.shp[j] > T(0.5)) {
                        // one box contact seen from both sides; a contact that exerts no
                        // force has zero derivatives
                        const Foot<T> fb = {B.shp[j], W.rad[j], B.hx[j], B.hy[j]};
                        const T ob[6] = {W.px[j], W.py[j], B.th[j], W.vx[j], W.vy[j], B.w[j]};
                        box_item_adj(C, g.obs, (size_t)0, (const T *)nullptr, BI_PAIR, L.i, fa, in,
                                     j, fb, ob, B.cs[j], B.sn[j], 0, T(1), wx, wy, gi);
                        return;
                    }
                }
                pair_adj_combined(C, in.px - W.px[j], in.py - W.py[j], in.vx - W.vx[j],
                                  in.vy - W.vy[j], L.pr.radius + W.rad[j] + C.margin, wx, wy,
                                  gi.px, gi.py, gi.vx, gi.vy);
            });
    }
    if constexpr (BOXES) {
        if (box_me) {
            // a box agent's obstacles and walls
            box_static_adj(C, g.obs, (size_t)L.env * C.N, (const T *)nullptr, fa, in, L.dd, gFx,
                           gFy, gi);
            return;
        }
    }
    if (C.N > 0) {
        const size_t eN = (size_t)L.env * C.N;
        for (int o = 0; o < C.N; ++o)
            obstacle_force_adj(C, g.obs, eN, o, in.px, in.py, in.vx, in.vy, L.pr.radius, L.dd,
                               gFx, gFy, gi);
    }
    if (C.soft_walls)
        wall_force_adj(C, in.px, in.py, in.vx, in.vy, L.pr.radius, L.dd, gFx, gFy, gi);
}

template <typename T, bool DRONE, bool GRID, bool BOXES, int APT, unsigned F>
__global__ __launch_bounds__(1024) void k_wide_bwd(const Cst<T> Cin, const Args<T> g)
{
    const Cst<T> C = fold_cst<F>(Cin);
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int32_t wsum[16];
    const int AP = (int)blockDim.x * APT;
    const WideLds<T> W = wide_lds<T>(smem, AP);
    const WBoxLds<T> B = wide_box_lds<T>(smem, AP, wide_cells(C));
    const GridFrame<T> G = grid_frame(C, (const T *)nullptr);
    WLane<T> L[APT];
    wide_lanes<T, BOXES, APT, F>(C, g, W, B, L);
    const size_t EA = (size_t)C.E * C.A;
    St<T> gs[APT];
#pragma unroll
    for (int k = 0; k < APT; ++k) st_zero(gs[k]);
    for (int t = g.nsteps - 1; t >= 0; --t) {
        St<T> st0[APT];
        T a[APT][4], ga[APT][4];
#pragma unroll
        for (int k = 0; k < APT; ++k) {
            if (L[k].active) {
                if (t == g.nsteps - 1)
                    add_adj<T, DRONE>(g.afin.f, L[k].idx, gs[k]);
                else
                    add_adj<T, DRONE>(g.atraj.f, (size_t)t * EA + L[k].idx, gs[k]);
            }
            if (t == 0)
                load_state<T, DRONE>(g.s0.f, L[k].idx, 0, st0[k]);
            else
                load_state<T, DRONE>(g.traj.f, L[k].idx, (size_t)(t - 1) * EA, st0[k]);
            load_act(g.act, (size_t)t * EA + L[k].idx, C.ad, a[k]);
            for (int q = 0; q < 4; ++q) ga[k][q] = T(0);
        }
        for (int s = C.S - 1; s >= 0; --s) {
            // the substep's input, recomputed from the step's checkpoint
            St<T> in[APT];
#pragma unroll
            for (int k = 0; k < APT; ++k) in[k] = st0[k];
            for (int q = 0; q < s; ++q)
                wide_substep<T, DRONE, GRID, BOXES, APT>(C, g, W, B, G, L, a, in, wsum);
            T Fx[APT], Fy[APT];
            int32_t cut[APT];
#pragma unroll
            for (int k = 0; k < APT; ++k) {
                Fx[k] = Fy[k] = T(0);
                cut[k] = CUT_ALL;
            }
            if (C.needs_forces) {
                if (C.collisions) {
                    __syncthreads();
#pragma unroll
                    for (int k = 0; k < APT; ++k) wide_put(W, L[k], in[k], BOXES ? &B : nullptr);
                    __syncthreads();
                    if (GRID) grid_build(W, C.A, G, wsum);
                }
#pragma unroll
                for (int k = 0; k < APT; ++k)
                    wide_agent_forces<T, GRID, BOXES>(C, g, W, B, G, L[k], in[k], Fx[k], Fy[k],
                                                      cut[k], nullptr);
            }
            St<T> gi[APT];
            T gFx[APT], gFy[APT];
#pragma unroll
            for (int k = 0; k < APT; ++k)
                integrate_adj<T, DRONE>(C, L[k].pr, in[k], a[k], Fx[k], Fy[k], gs[k], gi[k], ga[k],
                                        gFx[k], gFy[k]);
            if (C.needs_forces) {
                if (C.collisions) {
#pragma unroll
                    for (int k = 0; k < APT; ++k) {
                        // the force adjoint divided by the damping denominator
                        W.wfx[L[k].i] = gFx[k] * L[k].inv_dd;
                        W.wfy[L[k].i] = gFy[k] * L[k].inv_dd;
                        W.cut[L[k].i] = cut[k];
                    }
                    __syncthreads();
                }
#pragma unroll
                for (int k = 0; k < APT; ++k)
                    wide_agent_adj<T, GRID, BOXES>(C, g, W, B, G, L[k], in[k], gFx[k], gFy[k],
                                                   cut[k], gi[k]);
            }
#pragma unroll
            for (int k = 0; k < APT; ++k) gs[k] = gi[k];
        }
#pragma unroll
        for (int k = 0; k < APT; ++k) {
            if (!L[k].active) continue;
            T *pa = g.aact + ((size_t)t * EA + L[k].idx) * C.ad;
            for (int q = 0; q < C.ad; ++q) pa[q] = q < 4 ? ga[k][q] : T(0);
        }
    }
#pragma unroll
    for (int k = 0; k < APT; ++k)
        if (L[k].active) store_adj<T, DRONE>(g.a0.f, L[k].idx, gs[k]);
}

// ---------------------------------------------------------------------- launchers

// Threads of the movable-body kernels' workgroup (one per agent slot, at most 1024 agents).
template <typename T> inline int wide_threads(int A) { return ((A + 63) / 64) * 64; }

template <typename T> size_t wide_shm(const Cst<T> &C, bool boxes = false)
{
    const int AP = wide_geom(C.A).slots, NC = C.grid_bins > 0 ? C.grid_bins * C.grid_bins : 0;
    return boxes ? wide_box_lds_bytes<T>(AP, NC) : wide_lds_bytes<T>(AP, NC);
}

template <typename T>
void launch_wide_lists(const Cst<T> &C, const T *pos, const T *frame, int32_t *idx, int32_t *cnt,
                       int32_t *tru, hipStream_t st)
{
    const dim3 grid(C.E), block(wide_geom(C.A).threads);
    const size_t shm = wide_shm<T>(C);
    if (C.grid_bins > 0)
        hipLaunchKernelGGL((k_wide_lists<T, true>), grid, block, shm, st, C, pos, frame, idx, cnt, tru);
    else
        hipLaunchKernelGGL((k_wide_lists<T, false>), grid, block, shm, st, C, pos, frame, idx, cnt, tru);
}

template <typename T>
void launch_grid_frame(const T *pos, int64_t n, T radius, int bins, T *frame, hipStream_t st)
{
    hipLaunchKernelGGL((k_grid_frame<T>), dim3(1), dim3(1024), 0, st, pos, n, radius, bins, frame);
}

// boxes: a box world (box agents or wheel contacts; never with drones).
#define SWARP_WIDE_DISPATCH_APT(KERNEL, APT)                                                           \
    if (drone) {                                                                                       \
        if (grid) hipLaunchKernelGGL((KERNEL<T, true, true, false, APT, FT_ALL>), g, b, shm, st, C, a);  \
        else hipLaunchKernelGGL((KERNEL<T, true, false, false, APT, FT_ALL>), g, b, shm, st, C, a);      \
    } else if (boxes) {                                                                                \
        if (grid) hipLaunchKernelGGL((KERNEL<T, false, true, true, APT, FT_ALL>), g, b, shm, st, C, a);  \
        else hipLaunchKernelGGL((KERNEL<T, false, false, true, APT, FT_ALL>), g, b, shm, st, C, a);      \
    } else {                                                                                           \
        if (grid) hipLaunchKernelGGL((KERNEL<T, false, true, false, APT, FT_ALL>), g, b, shm, st, C, a); \
        else hipLaunchKernelGGL((KERNEL<T, false, false, false, APT, FT_ALL>), g, b, shm, st, C, a);     \
    }
// The launchers of one agents-per-thread count (each count its own compilation unit).
template <typename T, int APT>
void launch_wide_fwd_apt(bool drone, bool boxes, const Cst<T> &C, const Args<T> &a,
                         hipStream_t st)
{
    const dim3 g(C.E), b(wide_geom(C.A).threads);
    const size_t shm = wide_shm<T>(C, boxes);
    const bool grid = C.grid_bins > 0;
    SWARP_WIDE_DISPATCH_APT(k_wide_fwd, APT)
}

template <typename T, int APT>
void launch_wide_bwd_apt(bool drone, bool boxes, const Cst<T> &C, const Args<T> &a,
                         hipStream_t st)
{
    const dim3 g(C.E), b(wide_geom(C.A).threads);
    const size_t shm = wide_shm<T>(C, boxes);
    const bool grid = C.grid_bins > 0;
    SWARP_WIDE_DISPATCH_APT(k_wide_bwd, APT)
}
#undef SWARP_WIDE_DISPATCH_APT

template <typename T>
inline void launch_wide_fwd(bool drone, bool boxes, const Cst<T> &C, const Args<T> &a,
                            hipStream_t st)
{
    switch (wide_geom(C.A).apt) {
    case 1: launch_wide_fwd_apt<T, 1>(drone, boxes, C, a, st); break;
    case 2: launch_wide_fwd_apt<T, 2>(drone, boxes, C, a, st); break;
    default: launch_wide_fwd_apt<T, 4>(drone, boxes, C, a, st); break;
    }
}

template <typename T>
inline void launch_wide_bwd(bool drone, bool boxes, const Cst<T> &C, const Args<T> &a,
                            hipStream_t st)
{
    switch (wide_geom(C.A).apt) {
    case 1: launch_wide_bwd_apt<T, 1>(drone, boxes, C, a, st); break;
    case 2: launch_wide_bwd_apt<T, 2>(drone, boxes, C, a, st); break;
    default: launch_wide_bwd_apt<T, 4>(drone, boxes, C, a, st); break;
    }
}

}  // namespace swarp
