// bodies.hpp -- rollout kernels for worlds with movable compound bodies: the body pass of
// obstacle_dynamics_kernel (swarp/core/bodies.py:367-568, disc variant: disc agents, body
// shapes of any type) inside the fused substep chain, and this build's own adjoint
// of it (the reference never tapes the body pass, swarp/core/stepper.py:952).
// Instantiated by k_bodies.hip.
//
// Per-env obstacle state, 12 scalars per obstacle index o (the reference's obs_* and
// body_* arrays, swarp/core/stepper.py:418-431):
//   [6o .. 6o+5]          shape o:       pos x, pos y, angle, vel x, vel y, ang_vel
//   [6N+6o .. 6N+6o+5]    body rooted at o: pos x, pos y, angle, vel x, vel y, ang_vel
// It lives in LDS for the substeps of a step (double-buffered: substep input / output)
// and goes to HBM once per step as the step's obstacle output, which is also the
// backward's checkpoint.  Static scenery keeps its installed state.
//
// Substep order (swarp/core/stepper.py:908-991): lists on the input positions, agent
// forces against the input obstacle state, the body pass (every movable body integrated
// from the reactions of the input agent state), then the agents' integration.
//
// Sums over agents (a body's contact force and torque, the adjoints of a body's pose)
// are formed in agent order by one loop over the contributing lanes of the env, which
// keeps them in the reference's summation order; a contribution that is exactly zero is
// skipped, which does not change a sum that starts at +0.
//
// Both kernels run one wave per workgroup: lanes exchange values through LDS behind
// wave_lds_sync (a wavefront-scope fence), not a workgroup barrier, whose fence would
// also wait for every outstanding global load and store.
#pragma once
#include "common.hpp"

namespace swarp {

constexpr int OB_W = 12;       // scalars per obstacle index in the per-env state

// Static obstacle tables of the body path.
template <typename T> struct ObTab {
    const SWARP_RO T *rad, *half, *mass, *inertia, *off;  // [N], [N,2], [N], [N], [N,2]
    const SWARP_RO int32_t *type, *kind, *body;            // [N]
    // [A, 22] parameter rows the body pass reads for the agents' reactions when the
    // agents' own rows are per env (NULL: the agents' rows).  The reference's body pass
    // takes the shared table whatever the agent side uses (swarp/core/stepper.py:961-964).
    const SWARP_RO T *bprm;
    T lin_damp, ang_damp;
    int N;
    int cache;   // backward: 1 keeps each substep's body cos / sin and contact sums in LDS
};

// Obstacle-state inputs / outputs of a rollout.
template <typename T> struct ObIO {
    const T *ob0;       // [E, 12N] state entering the rollout
    T *traj;            // [T, E, 12N] state after each step
    const T *atraj;     // [T, E, 12N] adjoint arriving at each step's output (nullable)
    T *a0;              // [E, 12N] adjoint of ob0 (nullable)
    // Body tape (nullable): [T][S][tape_roots][E][BODY_REC] records of the body pass, one
    // per substep and movable body (in root order, the first tape_roots of them): written
    // by the forward, read by the backward in place of evaluating the pass again.
    T *tape;
    int tape_roots;
};

// Body-tape record of one body and substep: its new pose and velocity (x, y, angle,
// vel x, vel y, ang_vel), the new angle's cos and sin, its contact sum (fx, fy, tau); one
// pad entry keeps records 16-byte aligned.
constexpr int BODY_REC = 12;

// An agent as the body pass sees it: the radius and the implicit damping denominator
// 1 + c sub_dt / m of its parameter row in the table the pass reads.
template <typename T> struct BodyRow {
    T r, dd;
    Dv<T> ddv;  // dd as a prepared divisor
};

template <typename T, int PA>
__device__ __forceinline__ BodyRow<T> body_row(const Cst<T> &C, const ObTab<T> &tb,
                                               const Lane<T, PA> &L)
{
    if (!tb.bprm) return BodyRow<T>{L.pr.radius, L.dd, L.ddv};
    const int ag = L.real ? L.agent : 0;
    const T m = tb.bprm[(size_t)ag * 22 + 1];
    const T dd = T(1) + C.c * C.sub_dt / m;
    return BodyRow<T>{tb.bprm[(size_t)ag * 22], dd, divisor(dd, true)};
}

// sin and cos of a body angle (the portable evaluation of swarp_pmath.h, as the oracle's)
template <typename T> __device__ __forceinline__ void psincos(T xr, T &so, T &co)
{
    double s, c;
    swarp_psincos((double)xr, &s, &c);
    so = (T)s;
    co = (T)c;
}

// bounds_apart (swarp/core/collisions.py:73-84)
template <typename T> __device__ __forceinline__ bool b_apart(T dx, T dy, T reach)
{
    const T lim = reach * T(1.0001) + T(1.0e-6);
    return dx * dx + dy * dy > lim * lim;
}

// Whether shape s belongs to a movable body (the body pass re-installs it).
template <typename T> __device__ __forceinline__ bool shape_moves(const ObTab<T> &tb, int s)
{
    const int r = tb.body[s];
    return tb.body[r] == r && tb.kind[r] == 1;
}

// The env's shapes as index sets, for the loops of the body pass.  Instances compiled
// without FT_MANYSH (SM) hold at most 64 shapes: lane s of the wave keeps shape s's body
// root, a set is a 64-bit mask -- body o's shapes one ballot, the movable roots and the
// moving shapes masks formed once per launch -- and a loop visits the set bits in
// ascending order, the index order of a loop over all shapes, with no table reads on
// its way.  Otherwise the loops test the shapes one by one from the tables.
template <typename T, bool SM> struct ShapeSets {
    int32_t root = -1;    // SM: the body root of this lane's shape (-1: no shape)
    uint64_t roots = 0;   // SM: movable body roots
    uint64_t moving = 0;  // SM: shapes of movable bodies
    uint64_t all = 0;     // SM: every shape

    // with the whole wave active
    __device__ __forceinline__ void init(const ObTab<T> &tb, int lane)
    {
        if constexpr (SM) {
            const bool has = lane < tb.N;
            root = has ? tb.body[lane] : -1;
            roots = __ballot(has && root == lane && tb.kind[lane] == 1);
            moving = __ballot(has && ((roots >> ((uint32_t)root & 63u)) & 1ull) != 0);
            all = __ballot(has);
        }
    }
    // the shapes of body root o; SM: with the whole wave active
    __device__ __forceinline__ uint64_t of(int o) const
    {
        if constexpr (SM) return __ballot(root == o);
        return 0;
    }
    __device__ __forceinline__ bool moves(const ObTab<T> &tb, int s) const
    {
        if constexpr (SM) return ((moving >> s) & 1ull) != 0;
        return shape_moves(tb, s);
    }
    __device__ __forceinline__ bool is_root(const ObTab<T> &tb, int o) const
    {
        if constexpr (SM) return ((roots >> o) & 1ull) != 0;
        return tb.body[o] == o && tb.kind[o] == 1;
    }
    // whether shape s belongs to body root o (bm = of(o))
    __device__ __forceinline__ bool in_body(const ObTab<T> &tb, int o, uint64_t bm, int s) const
    {
        if constexpr (SM) return ((bm >> s) & 1ull) != 0;
        return tb.body[s] == o;
    }
    // f(o) for every movable body root o, in index order
    template <typename Fn> __device__ __forceinline__ void each_root(const ObTab<T> &tb, Fn &&f) const
    {
        if constexpr (SM) {
            for (uint64_t m = roots; m; m &= m - 1) f(__builtin_ctzll(m));
        } else {
            for (int o = 0; o < tb.N; ++o)
                if (tb.body[o] == o && tb.kind[o] == 1) f(o);
        }
    }
    // f(s) for every shape of body root o (bm = of(o)), in index order
    template <typename Fn>
    __device__ __forceinline__ void each_of(const ObTab<T> &tb, int o, uint64_t bm, Fn &&f) const
    {
        if constexpr (SM) {
            for (uint64_t m = bm; m; m &= m - 1) f(__builtin_ctzll(m));
        } else {
            for (int s = 0; s < tb.N; ++s)
                if (tb.body[s] == o) f(s);
        }
    }
    // f(s) for every shape not of body root o (bm = of(o)), in index order
    template <typename Fn>
    __device__ __forceinline__ void each_other(const ObTab<T> &tb, int o, uint64_t bm, Fn &&f) const
    {
        if constexpr (SM) {
            for (uint64_t m = all & ~bm; m; m &= m - 1) f(__builtin_ctzll(m));
        } else {
            for (int s = 0; s < tb.N; ++s)
                if (tb.body[s] != o) f(s);
        }
    }
};

// ------------------------------------------------ body-pass terms of any shape type
//
// Written once over the value type V: plain T in the forward pass, a one-tangent Dual in
// the reverse pass, which evaluates them once per seeded input (a column of the term's
// Jacobian) for the boxes and segments.  Circles keep the plain contact law and its
// hand-written reverse.

// pair_force over V (the same operations)
template <typename T, typename V>
__device__ __forceinline__ void pair_force_v(const Cst<T> &C, V dx, V dy, V rvx, V rvy, T md, T dd,
                                             V &fx, V &fy)
{
    const V dist = m_sqrt(wmax(dx * dx + dy * dy, V(C.eps2)));
    const V ov = V(md) - dist;
    fx = V(T(0));
    fy = V(T(0));
    if (val(ov) > T(0)) {
        const V nx = dx / dist, ny = dy / dist;
        const V coef = normal_coeff_v(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
}

// closest_on_segment (swarp/core/collisions.py:157-171): the point of the core (centre c,
// direction (ux, uy), half length hl) closest to p
template <typename T, typename V>
__device__ __forceinline__ void closest_seg_v(V px, V py, V cx, V cy, V ux, V uy, T hl, V &qx,
                                              V &qy)
{
    const V t = wclamp((px - cx) * ux + (py - cy) * uy, V(-hl), V(hl));
    qx = cx + t * ux;
    qy = cy + t * uy;
}

// _reaction (swarp/core/bodies.py:80-127): force on the body from one disc agent (p, v,
// radius ra, damping denominator dd) touching shape `ty` (radius ro, half extents hx, hy)
// centred at c, oriented by (ca, sa) = cos / sin of the body angle, its centre moving
// with vs, spinning with om; and the lever from the shape centre (r0, r1).
template <typename T, typename V>
__device__ __forceinline__ void body_reaction_v(const Cst<T> &C, int ty, T ro, T hx, T hy, T ra,
                                                T dd, V px, V py, V vx, V vy, V cx, V cy, V ca,
                                                V sa, V vsx, V vsy, V om, V &f0, V &f1, V &r0,
                                                V &r1)
{
    V fx, fy;
    if (ty == 1) {
        box_force_v<T, V>(C, px, py, vx, vy, cx, cy, ca, sa, hx, hy, ra + C.margin, dd, vsx, vsy,
                          om, fx, fy);
        r0 = px - cx;
        r1 = py - cy;
    } else if (ty == 2) {
        V qx, qy;
        closest_seg_v<T, V>(px, py, cx, cy, ca, sa, hx, qx, qy);
        const V rrx = qx - cx, rry = qy - cy;
        const V sx = vsx + (-om) * rry, sy = vsy + om * rrx;
        pair_force_v<T, V>(C, px - qx, py - qy, vx - sx, vy - sy, ra + ro + C.margin, dd, fx, fy);
        r0 = rrx;
        r1 = rry;
    } else {
        pair_force_v<T, V>(C, px - cx, py - cy, vx - vsx, vy - vsy, ra + ro + C.margin, dd, fx, fy);
        r0 = V(T(0));
        r1 = V(T(0));
    }
    f0 = -fx;
    f1 = -fy;
}

// _body_body (swarp/core/bodies.py:183-253): force on shape `ty` of a body (radius rs,
// half extents hs, centre q moving with tv, orientation (ca, sa), spin om) from shape ty2
// of another body or of the scenery (q2, tv2, (ca2, sa2), om2), and its lever from the
// shape centre.  A box against a box exerts nothing (the reference models no box-box
// obstacle contact); a round body meets a box as a disc of its radius at its centre.
template <typename T, typename V>
__device__ __forceinline__ void body_body_v(const Cst<T> &C, int ty, T rs, T hsx, T hsy, int ty2,
                                            T r2, T h2x, T h2y, T dd, V qx, V qy, V tvx, V tvy,
                                            V ca, V sa, V om, V q2x, V q2y, V tv2x, V tv2y, V ca2,
                                            V sa2, V om2, V &f0, V &f1, V &r0, V &r1)
{
    f0 = f1 = r0 = r1 = V(T(0));
    if (ty == 1) {
        if (ty2 == 1) return;
        V c2x = q2x, c2y = q2y, v2x = tv2x, v2y = tv2y;
        if (ty2 == 2) {
            closest_seg_v<T, V>(qx, qy, q2x, q2y, ca2, sa2, h2x, c2x, c2y);
            const V rrx = c2x - q2x, rry = c2y - q2y;
            v2x = tv2x + (-om2) * rry;
            v2y = tv2y + om2 * rrx;
        }
        V fox, foy;
        box_force_v<T, V>(C, c2x, c2y, v2x, v2y, qx, qy, ca, sa, hsx, hsy, r2 + C.margin, dd, tvx,
                          tvy, om, fox, foy);
        f0 = -fox;
        f1 = -foy;
        // _closest_in_box (:168-180): c2 - q clamped onto this box, in world axes
        const V dx = c2x - qx, dy = c2y - qy;
        const V lx = ca * dx + sa * dy, ly = (-sa) * dx + ca * dy;
        const V kx = wclamp(lx, V(-hsx), V(hsx)), ky = wclamp(ly, V(-hsy), V(hsy));
        r0 = ca * kx - sa * ky;
        r1 = sa * kx + ca * ky;
    } else if (ty2 == 1) {
        box_force_v<T, V>(C, qx, qy, tvx, tvy, q2x, q2y, ca2, sa2, h2x, h2y, rs + C.margin, dd,
                          tv2x, tv2y, om2, f0, f1);
    } else if (ty2 == 2) {
        V cpx, cpy;
        closest_seg_v<T, V>(qx, qy, q2x, q2y, ca2, sa2, h2x, cpx, cpy);
        const V rrx = cpx - q2x, rry = cpy - q2y;
        const V s2x = tv2x + (-om2) * rry, s2y = tv2y + om2 * rrx;
        pair_force_v<T, V>(C, qx - cpx, qy - cpy, tvx - s2x, tvy - s2y, rs + r2 + C.margin, dd, f0,
                           f1);
    } else {
        pair_force_v<T, V>(C, qx - q2x, qy - q2y, tvx - tv2x, tvy - tv2y, rs + r2 + C.margin, dd,
                           f0, f1);
    }
}

// shape_bound (swarp/core/collisions.py:61-70): radius of the disc about a shape's centre
// that holds it
template <typename T> __device__ __forceinline__ T shape_bound(int ty, T r, T hx, T hy)
{
    return ty == 1 ? m_sqrt(hx * hx + hy * hy) : (ty == 2 ? hx + r : r);
}

// A one-tangent dual of x, seeded when k == seed.
template <typename T> __device__ __forceinline__ Dual<T, 1> dseed(T x, int k, int seed)
{
    Dual<T, 1> r(x);
    r.d[0] = k == seed ? T(1) : T(0);
    return r;
}

// One obstacle's force on an agent, the obstacle's pose read from the env's state `od`
// (_obstacle_forces body, swarp/core/collisions.py:690-743).  DD: the damping denominator
// as a value or a prepared divisor (the same bits).
template <typename T, typename DD>
__device__ __forceinline__ void ob_force(const Cst<T> &C, const ObTab<T> &tb, const T *od, int o,
                                         T px, T py, T vx, T vy, T ra, const DD &dd, T &fx,
                                         T &fy)
{
    fx = T(0);
    fy = T(0);
    const T *sh = od + 6 * o;
    const T cx = sh[0], cy = sh[1];
    const int st = (C.round_only ? 0 : tb.type[o]);
    const T ro = tb.rad[o], hx = tb.half[2 * o], hy = tb.half[2 * o + 1];
    const T bound = st == 1 ? m_sqrt(hx * hx + hy * hy) : (st == 2 ? hx + ro : ro);
    if (b_apart(px - cx, py - cy, ra + C.margin + bound)) return;
    const T vox = sh[3], voy = sh[4], om = sh[5], ang = sh[2];
    if (st == 1) {
        box_force(C, px, py, vx, vy, cx, cy, ang, hx, hy, ra + C.margin, dd, vox, voy, om, fx,
                  fy);
    } else if (st == 2) {
        T ux = m_cos(ang), uy = m_sin(ang);
        T t = wclamp((px - cx) * ux + (py - cy) * uy, -hx, hx);
        T qx = cx + t * ux, qy = cy + t * uy;
        T rx = qx - cx, ry = qy - cy;
        pair_force(C, px - qx, py - qy, vx - (vox + -om * ry), vy - (voy + om * rx),
                   ra + ro + C.margin, dd, fx, fy);
    } else {
        pair_force(C, px - cx, py - cy, vx - vox, vy - voy, ra + ro + C.margin, dd, fx, fy);
    }
}

// Reverse of ob_force: the agent's adjoint into `a`; with `shape` set (a moving shape) the
// adjoint of the shape's state (pos x, pos y, angle, vel x, vel y, ang_vel) is returned in
// op[0..5] (zero otherwise).
template <typename T>
__device__ __forceinline__ void ob_force_adj(const Cst<T> &C, const ObTab<T> &tb, const T *od,
                                             int o, T px, T py, T vx, T vy, T ra, T dd, T gx,
                                             T gy, St<T> &a, bool shape, T (&op)[6])
{
#pragma unroll
    for (int q = 0; q < 6; ++q) op[q] = T(0);
    const T *sh = od + 6 * o;
    const T cx = sh[0], cy = sh[1];
    const int st = (C.round_only ? 0 : tb.type[o]);
    const T ro = tb.rad[o], hx = tb.half[2 * o], hy = tb.half[2 * o + 1];
    const T bound = st == 1 ? m_sqrt(hx * hx + hy * hy) : (st == 2 ? hx + ro : ro);
    if (b_apart(px - cx, py - cy, ra + C.margin + bound)) return;
    const T vox = sh[3], voy = sh[4], om = sh[5], ang = sh[2];
    if (st != 0 && shape) {
        // a moving box or segment: its state's adjoint, one seeded entry at a time
        for (int k = 0; k < 6; ++k) {
            const Dual<T, 1> c0 = dseed(sh[0], 0, k), c1 = dseed(sh[1], 1, k);
            const Dual<T, 1> an = dseed(sh[2], 2, k), v0 = dseed(sh[3], 3, k);
            const Dual<T, 1> v1 = dseed(sh[4], 4, k), w = dseed(sh[5], 5, k);
            const Dual<T, 1> P0(px), P1(py), U0(vx), U1(vy);
            Dual<T, 1> fx, fy;
            if (st == 1) {
                box_force_v<T, Dual<T, 1>>(C, P0, P1, U0, U1, c0, c1, m_cos(an), m_sin(an), hx,
                                           hy, ra + C.margin, dd, v0, v1, w, fx, fy);
            } else {
                Dual<T, 1> qx, qy;
                closest_seg_v<T, Dual<T, 1>>(P0, P1, c0, c1, m_cos(an), m_sin(an), hx, qx, qy);
                const Dual<T, 1> rx = qx - c0, ry = qy - c1;
                pair_force_v<T, Dual<T, 1>>(C, P0 - qx, P1 - qy, U0 - (v0 + (-w) * ry),
                                            U1 - (v1 + w * rx), ra + ro + C.margin, dd, fx, fy);
            }
            op[k] = gx * fx.d[0] + gy * fy.d[0];
        }
    }
    if (st == 1) {
        box_force_adj(C, px, py, vx, vy, cx, cy, ang, hx, hy, ra + C.margin, dd, vox, voy, om,
                      gx, gy, a);
    } else if (st == 2) {
        T ux = m_cos(ang), uy = m_sin(ang);
        T tr = (px - cx) * ux + (py - cy) * uy;
        T t = wclamp(tr, -hx, hx);
        T qx = cx + t * ux, qy = cy + t * uy;
        T rx = qx - cx, ry = qy - cy;
        T adx = T(0), ady = T(0), arx = T(0), ary = T(0);
        pair_force_adj(C, px - qx, py - qy, vx - (vox + -om * ry), vy - (voy + om * rx),
                       ra + ro + C.margin, dd, gx, gy, adx, ady, arx, ary);
        a.px += adx;
        a.py += ady;
        a.vx += arx;
        a.vy += ary;
        T aqx = -adx - om * ary;
        T aqy = -ady + om * arx;
        T atr = wclamp_g(tr, -hx, hx, aqx * ux + aqy * uy);
        a.px += atr * ux;
        a.py += atr * uy;
    } else {
        T adx = T(0), ady = T(0), arx = T(0), ary = T(0);
        pair_force_adj(C, px - cx, py - cy, vx - vox, vy - voy, ra + ro + C.margin, dd, gx, gy,
                       adx, ady, arx, ary);
        a.px += adx;
        a.py += ady;
        a.vx += arx;
        a.vy += ary;
        if (shape) {
            op[0] = -adx;
            op[1] = -ady;
            op[3] = -arx;
            op[4] = -ary;
        }
    }
}

// Agent forces of one substep on the body path: listed pairs (as the generic kernels),
// obstacles from the env's state, walls.
template <typename T, int PA>
__device__ __forceinline__ typename MaskT<PA>::type forces_b(
    const Cst<T> &C, const ObTab<T> &tb, const Lane<T, PA> &L, const T *sl, const T *lr,
    const T *od, const St<T> &st, int s, bool full, typename MaskT<PA>::type &cand, T &Fx, T &Fy)
{
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
        while (m) {
            const int b = m_ctz(m);
            m &= m - 1;
            const int j = L.base + b;
            const T dx = st.px - lx[j], dy = st.py - ly[j], md = ra + lr[j] + C.margin;
            if (pair_apart(dx, dy, md)) continue;  // adds exactly +0 (fx is never -0)
            T gx, gy;
            pair_force(C, dx, dy, st.vx - lvx[j], st.vy - lvy[j], md, L.ddv, gx, gy);
            fx += gx;
            fy += gy;
        }
    }
    T sx = T(0), sy = T(0);
    for (int o = 0; o < tb.N; ++o) {
        T gx, gy;
        ob_force(C, tb, od, o, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx, gy);
        sx += gx;
        sy += gy;
    }
    if (C.soft_walls) {
        T gx, gy;
        unsigned wb;
        wall_force_axes(C, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx, gy, wb);
        sx += gx;
        sy += gy;
    }
    Fx = fx + sx;
    Fy = fy + sy;
    return incl;
}

// The value x of lane l (l wave-uniform).
__device__ __forceinline__ float read_lane(float x, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ double read_lane(double x, int l)
{
    const long long b = __double_as_longlong(x);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(b & 0xffffffffll), l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// acc[q] += v[q] of every flagged lane of this lane's env, in ascending agent order: the
// additions, in their order, of a loop over the env's agents that skips the unflagged
// ones (skipping a zero contribution leaves a sum that starts at +0 unchanged).  The
// values travel by readlane, their lane indices taken in order from the wave's ballot,
// so the loop runs once per flagged lane of the wave with no LDS round trip; lanes of
// the wave's other envs leave acc alone.
template <int PA, int NV, typename T>
__device__ __forceinline__ void env_ordered_sums(T (&acc)[NV], const T (&v)[NV], bool flag,
                                                 int lane)
{
    uint64_t bal = __ballot(flag);
    const int slot = lane / PA;
    while (bal) {
        const int l = __builtin_ctzll(bal);
        bal &= bal - 1;
        const bool mine = PA == 64 || l / PA == slot;
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            const T x = read_lane(v[q], l);
            if (mine) acc[q] += x;
        }
    }
}

// This env's lanes whose flag is set, as a mask over the env's agent slots.
template <int PA> __device__ __forceinline__ typename MaskT<PA>::type env_ballot(bool f, int base)
{
    typedef typename MaskT<PA>::type M;
    const uint64_t bal = __ballot(f);
    const uint64_t full = PA == 64 ? ~0ull : ((1ull << PA) - 1ull);
    return (M)((bal >> base) & full);
}

// How the body pass reaches the agents of its env.  The narrow kernels put an env on PA
// lanes of one wave (NarrowEnv); the wide kernels on a workgroup of waves (WideEnv,
// wide_bodies.hpp).  Every thread of the env calls the pass together:
//   me()      this thread's agent slot in the env; stride() the env's slots
//   active()  the slot holds a real agent
//   ordered<NV>(acc, v, flag)  acc[q] += v[q] of every flagged agent of the env, in
//             ascending agent order; every thread of the env gets the sums
//   any(flag) whether a thread of the env (narrow: of the wave) has the flag
//   sync()    orders the env's LDS writes before its later LDS reads
template <typename T, int PA> struct NarrowEnv {
    const Lane<T, PA> &L;
    __device__ __forceinline__ int me() const { return L.agent; }
    __device__ __forceinline__ int stride() const { return PA; }
    __device__ __forceinline__ bool active() const { return L.active; }
    template <int NV>
    __device__ __forceinline__ void ordered(T (&acc)[NV], const T (&v)[NV], bool flag) const
    {
        env_ordered_sums<PA, NV>(acc, v, flag, L.lane);
    }
    __device__ __forceinline__ bool any(bool f) const { return __ballot(f) != 0; }
    __device__ __forceinline__ void sync() const { wave_lds_sync(); }
};

// New state of one movable body: the contact sum of body_sum, then the integration of
// bodies_env (the oracle's restatement of obstacle_dynamics_kernel).
template <typename T> struct BodyNew {
    T qx, qy, th, tvx, tvy, om, ca, sa;   // input pose (with its sin / cos)
    T fx, fy, tau, ext;                   // contact sum; static extent of the body
    T nx, ny, nth, nvx, nvy, nom, nca, nsa;
    bool clx, cly;
};

// Farthest point of body root o's shapes from the body origin, each shape axis-aligned in
// the body frame (bodies.py:449-459): it depends on the installed tables only, so the
// kernels evaluate it once per launch.
template <typename T> __device__ __forceinline__ T body_ext(const ObTab<T> &tb, int o)
{
    T ext = T(0);
    for (int s = 0; s < tb.N; ++s) {
        if (tb.body[s] != o) continue;
        const T ax = m_abs(tb.off[2 * s]), ay = m_abs(tb.off[2 * s + 1]);
        const T ro = tb.rad[s], hx = tb.half[2 * s], hy = tb.half[2 * s + 1];
        const int ty = tb.type[s];
        const T reach = ty == 1 ? m_sqrt((ax + hx) * (ax + hx) + (ay + hy) * (ay + hy))
                      : ty == 2 ? m_sqrt((ax + hx) * (ax + hx) + ay * ay) + ro
                                : m_sqrt(ax * ax + ay * ay) + ro;
        ext = wmax(ext, reach);
    }
    return ext;
}

// Per-launch / per-step LDS of the body pass of one env slot:
//   ext[o]                    static extent of body root o (body_ext)
//   cs[2o], cs[2o+1]          cos, sin of body o's angle in the obstacle state they
//                             accompany (one array per obstacle-state buffer)
//   sums[3o .. 3o+2]          fx, fy, tau of body o's contact sum (backward only, per substep)
// The sin / cos of a substep's output angle are those of the next substep's input angle,
// so each angle is evaluated once.

// Input pose of body root o from the env's obstacle state `od`, with its cos / sin (from
// `cs`, or evaluated when cs is NULL).
template <typename T>
__device__ __forceinline__ void body_load(const ObTab<T> &tb, const T *od, const T *cs, int o,
                                          BodyNew<T> &B)
{
    const T *b = od + 6 * tb.N + 6 * o;
    B.qx = b[0];
    B.qy = b[1];
    B.th = b[2];
    B.tvx = b[3];
    B.tvy = b[4];
    B.om = b[5];
    if (cs) {
        B.ca = cs[2 * o];
        B.sa = cs[2 * o + 1];
    } else {
        psincos(B.th, B.sa, B.ca);
    }
}

// Contact sum of movable body root o: every lane of the env computes the same values
// (agent contributions reach all of them by readlane, env_ordered_sums).  Agent state of
// the lane in `st`; `od` = the env's obstacle state at the substep input.  Per shape of
// the body (index order): the agents' reactions in agent order, then the contacts with
// the shapes of other bodies and of the scenery in index order (swarp/core/bodies.py:
// 423-501).  bm = SS.of(o).
template <typename T, typename X, bool SM>
__device__ __forceinline__ void body_sum(const Cst<T> &C, const ObTab<T> &tb,
                                         const ShapeSets<T, SM> &SS, const X &L,
                                         const BodyRow<T> &br, const St<T> &st, const T *od,
                                         int o, uint64_t bm, BodyNew<T> &B)
{
    T fx = T(0), fy = T(0), tau = T(0);
    const T mo = tb.mass[o];
    const T denom_self = T(1) + C.c * C.sub_dt / mo;
    SS.each_of(tb, o, bm, [&](int s) {
        const T offx = tb.off[2 * s], offy = tb.off[2 * s + 1];
        const T owx = B.ca * offx - B.sa * offy;
        const T owy = B.sa * offx + B.ca * offy;
        const T csx = B.qx + owx, csy = B.qy + owy;
        const T vsx = B.tvx - B.om * owy, vsy = B.tvy + B.om * owx;
        const int ty = (C.round_only ? 0 : tb.type[s]);
        const T ro = tb.rad[s], hx = tb.half[2 * s], hy = tb.half[2 * s + 1];
        const T bound = shape_bound(ty, ro, hx, hy);
        // the agents' reactions, in agent order
        T f0 = T(0), f1 = T(0), tq = T(0);
        if (L.active() && !b_apart(st.px - csx, st.py - csy, br.r + bound + C.margin)) {
            T r0 = T(0), r1 = T(0);
            if (ty == 0) {
                T gx, gy;
                pair_force(C, st.px - csx, st.py - csy, st.vx - vsx, st.vy - vsy,
                           br.r + ro + C.margin, br.ddv, gx, gy);
                f0 = -gx;
                f1 = -gy;
            } else {
                body_reaction_v<T, T>(C, ty, ro, hx, hy, br.r, br.dd, st.px, st.py, st.vx, st.vy,
                                      csx, csy, B.ca, B.sa, vsx, vsy, B.om, f0, f1, r0, r1);
            }
            const T lx = owx + r0, ly = owy + r1;
            tq = lx * f1 - ly * f0;
        }
        {
            T acc[3] = {fx, fy, tau};
            const T val[3] = {f0, f1, tq};
            L.template ordered<3>(acc, val, f0 != T(0) || f1 != T(0));
            fx = acc[0];
            fy = acc[1];
            tau = acc[2];
        }
        // contacts with the shapes of other bodies and of the scenery, in index order
        SS.each_other(tb, o, bm, [&](int o2) {
            const T *d2 = od + 6 * o2;
            const int ty2 = (C.round_only ? 0 : tb.type[o2]);
            const T r2 = tb.rad[o2], h2x = tb.half[2 * o2], h2y = tb.half[2 * o2 + 1];
            if (b_apart(d2[0] - csx, d2[1] - csy, bound + shape_bound(ty2, r2, h2x, h2y) + C.margin))
                return;
            T gx, gy, r0 = T(0), r1 = T(0);
            if (ty == 0 && ty2 == 0) {
                pair_force(C, csx - d2[0], csy - d2[1], vsx - d2[3], vsy - d2[4],
                           ro + r2 + C.margin, denom_self, gx, gy);
            } else {
                const T ca2 = ty2 == 0 ? T(1) : m_cos(d2[2]), sa2 = ty2 == 0 ? T(0) : m_sin(d2[2]);
                body_body_v<T, T>(C, ty, ro, hx, hy, ty2, r2, h2x, h2y, denom_self, csx, csy, vsx,
                                  vsy, B.ca, B.sa, B.om, d2[0], d2[1], d2[3], d2[4], ca2, sa2,
                                  d2[5], gx, gy, r0, r1);
            }
            const T lx = owx + r0, ly = owy + r1;
            fx += gx;
            fy += gy;
            tau += lx * gy - ly * gx;
        });
    });
    B.fx = fx;
    B.fy = fy;
    B.tau = tau;
}

// Integration of body root o from its contact sum (B.fx, fy, tau, ext and the input pose
// set): the new pose and velocity, with the clamp; not the new angle's sin / cos.
template <typename T>
__device__ __forceinline__ void body_advance(const Cst<T> &C, const ObTab<T> &tb, int o,
                                             BodyNew<T> &B)
{
    const T sdt = C.sub_dt, one = T(1);
    const T lin_decay = one - tb.lin_damp * sdt;
    const T ang_decay = one - tb.ang_damp * sdt;
    const T mo = tb.mass[o], I = tb.inertia[o], ext = B.ext;
    T nvx = (B.tvx + B.fx / mo * sdt) * lin_decay;
    T nvy = (B.tvy + B.fy / mo * sdt) * lin_decay;
    const T nom = (B.om + B.tau / I * sdt) * ang_decay;
    T nx = B.qx + nvx * sdt;
    T ny = B.qy + nvy * sdt;
    B.clx = B.cly = false;
    if (C.clamp) {
        const T half = T(0.5);
        T lo_x = C.bmin_x + ext, mid_x = (C.bmin_x + C.bmax_x) * half;
        lo_x = lo_x < mid_x ? lo_x : mid_x;
        const T hi_x = wmax(C.bmax_x - ext, lo_x);
        T lo_y = C.bmin_y + ext, mid_y = (C.bmin_y + C.bmax_y) * half;
        lo_y = lo_y < mid_y ? lo_y : mid_y;
        const T hi_y = wmax(C.bmax_y - ext, lo_y);
        const T cx = wclamp(nx, lo_x, hi_x), cy = wclamp(ny, lo_y, hi_y);
        B.clx = cx != nx;
        B.cly = cy != ny;
        if (B.clx) nvx = T(0);
        if (B.cly) nvy = T(0);
        nx = cx;
        ny = cy;
    }
    B.nx = nx;
    B.ny = ny;
    B.nvx = nvx;
    B.nvy = nvy;
    B.nom = nom;
    B.nth = B.th + nom * sdt;
}

// cos / sin of the angle of every movable body root in the obstacle state `od`.  Lane
// `agent` of the env fills roots agent, agent + PA, ...
template <typename T, typename X, bool SM>
__device__ __forceinline__ void body_trig(const ObTab<T> &tb, const ShapeSets<T, SM> &SS,
                                          const X &L, const T *od, T *cs)
{
    for (int o = L.me(); o < tb.N; o += L.stride()) {
        if (!SS.is_root(tb, o)) continue;
        T s, c;
        psincos(od[6 * tb.N + 6 * o + 2], s, c);
        cs[2 * o] = c;
        cs[2 * o + 1] = s;
    }
}

// The body pass of one env: obn = obc with every movable body advanced and its shapes
// re-installed at the new pose; cs_out = the new angles' cos / sin (cs_in: the input
// angles'; both NULL when not kept); sums (nullable) receives each body's contact sum.
// Slot `me` of the env copies the entries me, me + stride, ... that the pass does not
// rewrite, and re-installs the moved body's shapes me, me + stride, ...  Body-tape records of
// this env and substep (BODY_REC entries per body, rstride entries from one body's to
// the next's, the first `rroots` bodies): `rout` receives them (nullable); with `rin`
// they are read instead of evaluating those bodies' contact sums and integration.
template <typename T, typename X, bool SM>
__device__ __forceinline__ void body_pass(const Cst<T> &C, const ObTab<T> &tb,
                                          const ShapeSets<T, SM> &SS, const X &L,
                                          const BodyRow<T> &br, const St<T> &st, const T *obc,
                                          T *obn, const T *ext, const T *cs_in, T *cs_out,
                                          T *sums, const T *rin = nullptr, T *rout = nullptr,
                                          size_t rstride = 0, int rroots = 0)
{
    const int N = tb.N;
    for (int q = L.me(); q < OB_W * N; q += L.stride()) {
        const bool rewritten = q < 6 * N ? SS.moves(tb, q / 6) : SS.is_root(tb, (q - 6 * N) / 6);
        if (!rewritten) obn[q] = obc[q];
    }
    int r = 0;  // the body's place in root order
    SS.each_root(tb, [&](int o) {
        const uint64_t bm = SS.of(o);
        BodyNew<T> B;
        if (rin && r < rroots) {
            const T *rec = rin + (size_t)r * rstride;
            B.nx = rec[0];
            B.ny = rec[1];
            B.nth = rec[2];
            B.nvx = rec[3];
            B.nvy = rec[4];
            B.nom = rec[5];
            B.nca = rec[6];
            B.nsa = rec[7];
            B.fx = rec[8];
            B.fy = rec[9];
            B.tau = rec[10];
        } else {
            body_load(tb, obc, cs_in, o, B);
            B.ext = ext[o];
            body_sum<T>(C, tb, SS, L, br, st, obc, o, bm, B);
            body_advance(C, tb, o, B);
            psincos(B.nth, B.nsa, B.nca);
        }
        if (rout && r < rroots && L.me() == 0) {
            T *rec = rout + (size_t)r * rstride;
            rec[0] = B.nx;
            rec[1] = B.ny;
            rec[2] = B.nth;
            rec[3] = B.nvx;
            rec[4] = B.nvy;
            rec[5] = B.nom;
            rec[6] = B.nca;
            rec[7] = B.nsa;
            rec[8] = B.fx;
            rec[9] = B.fy;
            rec[10] = B.tau;
            rec[11] = T(0);
        }
        ++r;
        if (L.me() == 0) {
            T *bo = obn + 6 * N + 6 * o;
            bo[0] = B.nx;
            bo[1] = B.ny;
            bo[2] = B.nth;
            bo[3] = B.nvx;
            bo[4] = B.nvy;
            bo[5] = B.nom;
            if (cs_out) {
                cs_out[2 * o] = B.nca;
                cs_out[2 * o + 1] = B.nsa;
            }
            if (sums) {
                sums[3 * o] = B.fx;
                sums[3 * o + 1] = B.fy;
                sums[3 * o + 2] = B.tau;
            }
        }
        for (int s = L.me(); s < N; s += L.stride()) {
            if (!SS.in_body(tb, o, bm, s)) continue;
            const T offx = tb.off[2 * s], offy = tb.off[2 * s + 1];
            const T owx = B.nca * offx - B.nsa * offy;
            const T owy = B.nsa * offx + B.nca * offy;
            T *so = obn + 6 * s;
            so[0] = B.nx + owx;
            so[1] = B.ny + owy;
            so[2] = B.nth;
            so[3] = B.nvx - B.nom * owy;
            so[4] = B.nvy + B.nom * owx;
            so[5] = B.nom;
        }
    });
}

// Waves per SIMD the float32 profile instances of the body kernels are compiled for
// (register budget 512 / waves per lane): a 16000-env launch is latency-bound, so more
// resident waves beat the spills the tighter budget costs (measured on the config-5
// workload).  Fewer for 4 and 8 agents per env, where the obstacle-state LDS of 16 and 8
// env slots bounds residency anyway; the general instances keep the compiler's choice.
constexpr int body_fwd_waves(int PA, size_t tsize, unsigned F)
{
    return (tsize != 4 || F == FT_ALL) ? 1 : (PA >= 16 ? 4 : (PA == 8 ? 3 : 2));
}
constexpr int body_bwd_waves(int PA, size_t tsize, unsigned F)
{
    return (tsize != 4 || F == FT_ALL) ? 1 : (PA >= 8 ? 3 : 2);
}

// ------------------------------------------------------------------ forward rollout

template <typename T, int PA, bool DRONE, unsigned F>
__global__ __launch_bounds__(64, body_fwd_waves(PA, sizeof(T), F)) void k_body_fwd(const Cst<T> Cin, const Args<T> g,
                                                 const ObTab<T> tb, const ObIO<T> io)
{
    typedef typename MaskT<PA>::type M;
    const Cst<T> C = fold_cst<F>(Cin);
    constexpr int EPW = 64 / PA;
    __shared__ T sl[4 * 64];                         // px py vx vy of the substep
    __shared__ T lr[64];                             // agent radius per lane
    // dynamic LDS (body_fwd_lds): [2][EPW][NW] obstacle state in / out of a substep,
    // [2][EPW][2N] its bodies' cos / sin (body_pass), [N] static extent per body root
    extern __shared__ __align__(16) unsigned char smem[];
    const int NW = OB_W * tb.N;
    T *const lob = (T *)smem;
    T *const lcs = lob + (size_t)2 * EPW * NW;
    T *const lext = lcs + (size_t)2 * EPW * 2 * tb.N;
    Lane<T, PA> L;
    lane_init<T, PA>(C, g, L);
    ShapeSets<T, !(F & FT_MANYSH)> SS;
    SS.init(tb, L.lane);
    const NarrowEnv<T, PA> X{L};
    fold_prm<F>(L.pr);
    const BodyRow<T> br = body_row<T, PA>(C, tb, L);
    lr[L.lane] = L.pr.radius;
    const int ew = L.lane / PA;
    // this env's obstacle state and body cos / sin in buffer c (0 / 1)
    const auto obs = [&](int c) { return lob + ((size_t)c * EPW + ew) * NW; };
    const auto ocs = [&](int c) { return lcs + ((size_t)c * EPW + ew) * 2 * tb.N; };
    const bool env_ok = L.env < C.E;
    const size_t eo = (size_t)(env_ok ? L.env : 0) * NW;
    for (int q = L.agent; q < NW; q += PA) obs(0)[q] = io.ob0[eo + q];
    for (int o = L.lane; o < tb.N; o += 64) lext[o] = body_ext(tb, o);
    wave_lds_sync();
    body_trig<T>(tb, SS, X, obs(0), ocs(0));
    St<T> st;
    load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
    if (!L.active) st.px = st.py = __builtin_nan("");
    const size_t EA = (size_t)C.E * C.A, ENW = (size_t)C.E * NW;
    int cur = 0;
    // each step's action is loaded one step ahead and taken into registers before the
    // step's stores (memory operations complete in order)
    T a[4];
    load_act(g.act, L.idx, C.ad, a);
    for (int t = 0; t < g.nsteps; ++t) {
        T an[4] = {a[0], a[1], a[2], a[3]};
        if (t + 1 < g.nsteps) load_act(g.act, (size_t)(t + 1) * EA + L.idx, C.ad, an);
        progress_priority(t, g.nsteps);
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            wave_lds_sync();
            sl[F_PX * 64 + L.lane] = st.px;
            sl[F_PY * 64 + L.lane] = st.py;
            sl[F_VX * 64 + L.lane] = st.vx;
            sl[F_VY * 64 + L.lane] = st.vy;
            wave_lds_sync();
            const T *obc = obs(cur);
            T Fx, Fy;
            forces_b<T, PA>(C, tb, L, sl, lr, obc, st, s, s == 0 || !ok, cand, Fx, Fy);
            T *rout = io.tape && env_ok ? io.tape + (((size_t)t * C.S + s) * io.tape_roots * C.E +
                                                     L.env) * BODY_REC
                                        : nullptr;
            body_pass<T>(C, tb, SS, X, br, st, obc, obs(cur ^ 1), lext, ocs(cur), ocs(cur ^ 1),
                             nullptr, nullptr, rout, (size_t)C.E * BODY_REC, io.tape_roots);
            St<T> nx;
            integrate<T, DRONE>(C, L.pr, st, a, Fx, Fy, nx);
            if (C.use_skin) {
                D += (m_abs(nx.px - st.px) + m_abs(nx.py - st.py)) * T(1.0001);
                ok = env_all<PA>(!L.active || D <= C.half_margin, L.base);
            }
            st = nx;
            cur ^= 1;
        }
        asm volatile("" ::"v"(an[0]), "v"(an[1]), "v"(an[2]), "v"(an[3]));
        wave_lds_sync();
        if (L.active) {
            if (t + 1 < g.nsteps)
                store_state<T, DRONE>(g.traj.f, (size_t)t * EA + L.idx, st);
            else
                store_state<T, DRONE>(g.fin.f, L.idx, st);
        }
        if (env_ok)
            for (int q = L.agent; q < NW; q += PA) io.traj[(size_t)t * ENW + eo + q] = obs(cur)[q];
        for (int k = 0; k < 4; ++k) a[k] = an[k];
    }
}

// ----------------------------------------------------------------- backward rollout

// Dynamic LDS of k_body_bwd (host and device agree on this layout).
template <typename T, int PA, bool DRONE>
__host__ __device__ constexpr size_t body_bwd_lds(int S, int N, bool cache)
{
    typedef typename MaskT<PA>::type M;
    return 2 * 64 * sizeof(T)                               // radius, damping divisor
           + (size_t)S * (DRONE ? NF_DRONE : NF_2D) * 64 * sizeof(T)  // substep agent slots
           + (size_t)S * 64 * sizeof(M)                     // inclusion masks
           + (size_t)(S + 1) * (64 / PA) * OB_W * N * sizeof(T)  // obstacle state per substep
           + 2 * (size_t)(64 / PA) * OB_W * N * sizeof(T)        // obstacle adjoint in / out
           + (cache ? (size_t)(S + 1) * (64 / PA) * 2 * N * sizeof(T)   // body cos / sin
                          + (size_t)S * (64 / PA) * 3 * N * sizeof(T)   // body contact sums
                    : 0)
           + (size_t)N * sizeof(T);                         // static extent per body root
}

// Dynamic LDS of k_body_fwd: two obstacle states and two cos / sin tables per env slot of
// the wave, and the extent table.
__host__ __device__ constexpr size_t body_fwd_lds(int PA, int N, size_t tsize)
{
    return ((size_t)2 * (64 / PA) * (OB_W + 2) * N + N) * tsize;
}

// All LDS of one k_body_fwd workgroup: the dynamic part above and the kernel's static
// arrays (sl[4 * 64] and lr[64] scalars).  The LDS limits are checked on this total.
__host__ __device__ constexpr size_t body_fwd_lds_total(int PA, int N, size_t tsize)
{
    return body_fwd_lds(PA, N, tsize) + (size_t)5 * 64 * tsize;
}

// Reverse of body_pass for one env.  gout = adjoint of the pass's output (the env's
// obstacle state after the substep), gin receives the adjoint of its input (overwritten);
// the lane's agent adjoint is accumulated into `ga`.  ext / cs_in / cs_out / sums are what
// the forward body_pass of this substep read and wrote: each body's new state is rebuilt
// from its recorded contact sum, not summed again (NULL cs / sums: recomputed).  Same
// order of terms as the oracle's bodies_env_adj.
template <typename T, typename X, bool SM>
__device__ __forceinline__ void body_pass_adj(const Cst<T> &C, const ObTab<T> &tb,
                                              const ShapeSets<T, SM> &SS,
                                              const X &L, const BodyRow<T> &br,
                                              const St<T> &st, const T *obc, const T *gout,
                                              T *gin, St<T> &ga, const T *ext, const T *cs_in,
                                              const T *cs_out, const T *sums)
{
    const int N = tb.N;
    // pass-through of everything the pass does not rewrite
    for (int q = L.me(); q < OB_W * N; q += L.stride()) {
        const int s = q / 6;
        gin[q] = (q < 6 * N && SS.moves(tb, s)) ? T(0) : gout[q];
    }
    L.sync();
    SS.each_root(tb, [&](int o) {
        const uint64_t bm = SS.of(o);
        BodyNew<T> B;
        body_load(tb, obc, cs_in, o, B);
        B.ext = ext[o];
        if (sums) {
            B.fx = sums[3 * o];
            B.fy = sums[3 * o + 1];
            B.tau = sums[3 * o + 2];
        } else {
            body_sum<T>(C, tb, SS, L, br, st, obc, o, bm, B);
        }
        body_advance(C, tb, o, B);
        if (cs_out) {
            B.nca = cs_out[2 * o];
            B.nsa = cs_out[2 * o + 1];
        } else {
            psincos(B.nth, B.nsa, B.nca);
        }
        const T sdt = C.sub_dt, one = T(1);
        const T lin_decay = one - tb.lin_damp * sdt;
        const T ang_decay = one - tb.ang_damp * sdt;
        const T m = tb.mass[o], I = tb.inertia[o];
        // adjoint of the new body state: its own entry plus every re-installed shape
        const T *gb = gout + 6 * N + 6 * o;
        T g_nx = gb[0], g_ny = gb[1], g_nth = gb[2], g_nvx = gb[3], g_nvy = gb[4], g_nom = gb[5];
        SS.each_of(tb, o, bm, [&](int s) {
            const T offx = tb.off[2 * s], offy = tb.off[2 * s + 1];
            const T owx = B.nca * offx - B.nsa * offy;
            const T owy = B.nsa * offx + B.nca * offy;
            const T *gs = gout + 6 * s;
            g_nx += gs[0];
            g_ny += gs[1];
            g_nth += gs[2];
            g_nvx += gs[3];
            g_nvy += gs[4];
            g_nom += gs[5] - gs[3] * owy + gs[4] * owx;
            const T g_owx = gs[0] + gs[4] * B.nom, g_owy = gs[1] - gs[3] * B.nom;
            g_nth += -g_owx * owy + g_owy * owx;
        });
        T g_th = g_nth;
        g_nom += g_nth * sdt;
        T g_qx = B.clx ? T(0) : g_nx, g_qy = B.cly ? T(0) : g_ny;
        if (B.clx) g_nvx = T(0); else g_nvx += g_nx * sdt;
        if (B.cly) g_nvy = T(0); else g_nvy += g_ny * sdt;
        T g_tvx = g_nvx * lin_decay, g_tvy = g_nvy * lin_decay;
        const T g_fx = g_nvx * lin_decay * sdt / m, g_fy = g_nvy * lin_decay * sdt / m;
        T g_om = g_nom * ang_decay;
        const T g_tau = g_nom * ang_decay * sdt / I;
        const T denom_self = T(1) + C.c * C.sub_dt / m;
        SS.each_of(tb, o, bm, [&](int s) {
            const T offx = tb.off[2 * s], offy = tb.off[2 * s + 1];
            const T owx = B.ca * offx - B.sa * offy;
            const T owy = B.sa * offx + B.ca * offy;
            const T csx = B.qx + owx, csy = B.qy + owy;
            const T vsx = B.tvx - B.om * owy, vsy = B.tvy + B.om * owx;
            const int ty = (C.round_only ? 0 : tb.type[s]);
            const T ro = tb.rad[s], hx = tb.half[2 * s], hy = tb.half[2 * s + 1];
            const T bound = shape_bound(ty, ro, hx, hy);
            const T g_f0 = g_fx - g_tau * owy, g_f1 = g_fy + g_tau * owx;
            // the agents' terms, in agent order: contributions to the adjoints of ow, the
            // shape centre cs, its velocity vs, and (boxes, segments) the shape's own angle
            // and spin
            T cv[8] = {T(0), T(0), T(0), T(0), T(0), T(0), T(0), T(0)};
            if (L.active() && !b_apart(st.px - csx, st.py - csy, br.r + bound + C.margin)) {
                if (ty == 0) {
                    const T dx = st.px - csx, dy = st.py - csy, rvx = st.vx - vsx,
                            rvy = st.vy - vsy;
                    const T md = br.r + ro + C.margin;
                    T gx, gy;
                    pair_force(C, dx, dy, rvx, rvy, md, br.ddv, gx, gy);
                    const T f0 = -gx, f1 = -gy;
                    T adx = T(0), ady = T(0), arx = T(0), ary = T(0);
                    pair_force_adj(C, dx, dy, rvx, rvy, md, br.dd, -g_f0, -g_f1, adx, ady, arx,
                                   ary);
                    ga.px += adx;
                    ga.py += ady;
                    ga.vx += arx;
                    ga.vy += ary;
                    cv[0] = g_tau * f1;    // onto g_owx
                    cv[1] = -(g_tau * f0); // onto g_owy (g_owy -= g_tau * f0)
                    cv[2] = -adx;          // onto g_csx
                    cv[3] = -ady;
                    cv[4] = -arx;          // onto g_vsx
                    cv[5] = -ary;
                } else {
                    // a box or segment: the term's Jacobian, one seeded input at a time
                    T f0, f1, r0, r1;
                    body_reaction_v<T, T>(C, ty, ro, hx, hy, br.r, br.dd, st.px, st.py, st.vx,
                                          st.vy, csx, csy, B.ca, B.sa, vsx, vsy, B.om, f0, f1,
                                          r0, r1);
                    const T L0 = owx + r0, L1 = owy + r1;
                    const T h0 = g_fx - g_tau * L1, h1 = g_fy + g_tau * L0;
                    const T hr0 = g_tau * f1, hr1 = -(g_tau * f0);
                    cv[0] = g_tau * f1;
                    cv[1] = -(g_tau * f0);
                    const T in[10] = {st.px, st.py, st.vx, st.vy, csx, csy, B.th, vsx, vsy, B.om};
                    for (int k = 0; k < 10; ++k) {
                        Dual<T, 1> x[10], o0, o1, l0, l1;
#pragma unroll
                        for (int q = 0; q < 10; ++q) x[q] = dseed(in[q], q, k);
                        body_reaction_v<T, Dual<T, 1>>(C, ty, ro, hx, hy, br.r, br.dd, x[0], x[1],
                                                       x[2], x[3], x[4], x[5], m_cos(x[6]),
                                                       m_sin(x[6]), x[7], x[8], x[9], o0, o1, l0,
                                                       l1);
                        const T adj = h0 * o0.d[0] + h1 * o1.d[0] + hr0 * l0.d[0] + hr1 * l1.d[0];
                        if (k == 0) ga.px += adj;
                        else if (k == 1) ga.py += adj;
                        else if (k == 2) ga.vx += adj;
                        else if (k == 3) ga.vy += adj;
                        else if (k == 4) cv[2] += adj;
                        else if (k == 5) cv[3] += adj;
                        else if (k == 6) cv[6] += adj;
                        else if (k == 7) cv[4] += adj;
                        else if (k == 8) cv[5] += adj;
                        else cv[7] += adj;
                    }
                }
            }
            T acc[8] = {T(0), T(0), T(0), T(0), T(0), T(0), T(0), T(0)};
            {
                bool fl = false;
#pragma unroll
                for (int q = 0; q < 8; ++q) fl = fl || cv[q] != T(0);
                L.template ordered<8>(acc, cv, fl);
            }
            T g_owx = acc[0], g_owy = acc[1], g_csx = acc[2], g_csy = acc[3], g_vsx = acc[4],
              g_vsy = acc[5], g_thd = acc[6], g_omd = acc[7];
            SS.each_other(tb, o, bm, [&](int o2) {
                const T *d2 = obc + 6 * o2;
                const int ty2 = (C.round_only ? 0 : tb.type[o2]);
                const T r2 = tb.rad[o2], h2x = tb.half[2 * o2], h2y = tb.half[2 * o2 + 1];
                if (b_apart(d2[0] - csx, d2[1] - csy, bound + shape_bound(ty2, r2, h2x, h2y) + C.margin))
                    return;
                if (ty != 0 || ty2 != 0) {
                    // the term's Jacobian over both shapes' states, one input at a time
                    const T ca2 = ty2 == 0 ? T(1) : m_cos(d2[2]);
                    const T sa2 = ty2 == 0 ? T(0) : m_sin(d2[2]);
                    T f0, f1, r0, r1;
                    body_body_v<T, T>(C, ty, ro, hx, hy, ty2, r2, h2x, h2y, denom_self, csx, csy,
                                      vsx, vsy, B.ca, B.sa, B.om, d2[0], d2[1], d2[3], d2[4], ca2,
                                      sa2, d2[5], f0, f1, r0, r1);
                    const T L0 = owx + r0, L1 = owy + r1;
                    const T h0 = g_fx - g_tau * L1, h1 = g_fy + g_tau * L0;
                    const T hr0 = g_tau * f1, hr1 = -(g_tau * f0);
                    g_owx += g_tau * f1;
                    g_owy -= g_tau * f0;
                    const T in[12] = {csx, csy, vsx, vsy, B.th, B.om,
                                      d2[0], d2[1], d2[3], d2[4], d2[2], d2[5]};
                    const bool mv = SS.moves(tb, o2) && L.me() == 0;
                    for (int k = 0; k < 12; ++k) {
                        Dual<T, 1> x[12], o0, o1, l0, l1;
#pragma unroll
                        for (int q = 0; q < 12; ++q) x[q] = dseed(in[q], q, k);
                        body_body_v<T, Dual<T, 1>>(C, ty, ro, hx, hy, ty2, r2, h2x, h2y,
                                                   denom_self, x[0], x[1], x[2], x[3],
                                                   m_cos(x[4]), m_sin(x[4]), x[5], x[6], x[7],
                                                   x[8], x[9], m_cos(x[10]), m_sin(x[10]), x[11],
                                                   o0, o1, l0, l1);
                        const T adj = h0 * o0.d[0] + h1 * o1.d[0] + hr0 * l0.d[0] + hr1 * l1.d[0];
                        if (k == 0) g_csx += adj;
                        else if (k == 1) g_csy += adj;
                        else if (k == 2) g_vsx += adj;
                        else if (k == 3) g_vsy += adj;
                        else if (k == 4) g_thd += adj;
                        else if (k == 5) g_omd += adj;
                        else if (mv) {
                            // the other shape's state: pos x, pos y, vel x, vel y, angle, spin
                            const int slot = k == 6 ? 0 : k == 7 ? 1 : k == 8 ? 3 : k == 9 ? 4
                                           : k == 10 ? 2 : 5;
                            gin[6 * o2 + slot] += adj;
                        }
                    }
                    return;
                }
                T gx, gy;
                pair_force(C, csx - d2[0], csy - d2[1], vsx - d2[3], vsy - d2[4],
                           ro + r2 + C.margin, denom_self, gx, gy);
                g_owx += g_tau * gy;
                g_owy -= g_tau * gx;
                T adx = T(0), ady = T(0), arx = T(0), ary = T(0);
                pair_force_adj(C, csx - d2[0], csy - d2[1], vsx - d2[3], vsy - d2[4],
                               ro + r2 + C.margin, denom_self, g_f0, g_f1, adx, ady, arx, ary);
                g_csx += adx;
                g_csy += ady;
                g_vsx += arx;
                g_vsy += ary;
                if (SS.moves(tb, o2) && L.me() == 0) {
                    T *g2 = gin + 6 * o2;
                    g2[0] -= adx;
                    g2[1] -= ady;
                    g2[3] -= arx;
                    g2[4] -= ary;
                }
            });
            g_qx += g_csx;
            g_qy += g_csy;
            g_owx += g_csx + g_vsy * B.om;
            g_owy += g_csy - g_vsx * B.om;
            g_tvx += g_vsx;
            g_tvy += g_vsy;
            g_om += -g_vsx * owy + g_vsy * owx + g_omd;
            g_th += -g_owx * owy + g_owy * owx + g_thd;
        });
        if (L.me() == 0) {
            T *gi = gin + 6 * N + 6 * o;
            gi[0] = g_qx;
            gi[1] = g_qy;
            gi[2] = g_th;
            gi[3] = g_tvx;
            gi[4] = g_tvy;
            gi[5] = g_om;
        }
        L.sync();
    });
}

template <typename T, int PA, bool DRONE, unsigned F>
__global__ __launch_bounds__(64, body_bwd_waves(PA, sizeof(T), F)) void k_body_bwd(const Cst<T> Cin, const Args<T> g,
                                                 const ObTab<T> tb, const ObIO<T> io)
{
    const Cst<T> C = fold_cst<F>(Cin);
    typedef typename MaskT<PA>::type M;
    constexpr int EPW = 64 / PA;
    constexpr int NF = DRONE ? NF_DRONE : NF_2D;
    extern __shared__ __align__(16) unsigned char smem[];
    const int N = tb.N, NW = OB_W * N;
    T *lr = (T *)smem;                                   // radius per lane
    T *ldd = lr + 64;                                    // damping divisor per lane
    T *slots = ldd + 64;                                 // S slots of NF fields
    M *lmask = (M *)(slots + (size_t)C.S * NF * 64);     // S inclusion masks
    T *lobs = (T *)(lmask + (size_t)C.S * 64);           // [S+1][EPW][NW] obstacle states
    T *lgob = lobs + (size_t)(C.S + 1) * EPW * NW;       // [2][EPW][NW] obstacle adjoints
    // with tb.cache: [S+1][EPW][2N] body cos / sin, [S][EPW][3N] body contact sums
    T *lcs = tb.cache ? lgob + (size_t)2 * EPW * NW : nullptr;
    T *lsum = tb.cache ? lcs + (size_t)(C.S + 1) * EPW * 2 * N : nullptr;
    // [N] static extent per body root, after the caches (or the adjoints without them)
    T *lext = tb.cache ? lsum + (size_t)C.S * EPW * 3 * N : lgob + (size_t)2 * EPW * NW;
    for (int o = threadIdx.x; o < N; o += 64) lext[o] = body_ext(tb, o);
    Lane<T, PA> L;
    lane_init<T, PA>(C, g, L);
    ShapeSets<T, !(F & FT_MANYSH)> SS;
    SS.init(tb, L.lane);
    const NarrowEnv<T, PA> X{L};
    fold_prm<F>(L.pr);
    const BodyRow<T> br = body_row<T, PA>(C, tb, L);
    lr[L.lane] = L.pr.radius;
    ldd[L.lane] = L.dd;
    const int ew = L.lane / PA;
    const bool env_ok = L.env < C.E;
    const size_t eo = (size_t)(env_ok ? L.env : 0) * NW;
    const size_t EA = (size_t)C.E * C.A, ENW = (size_t)C.E * NW;
    T *gob = lgob + (size_t)ew * NW;             // adjoint of the current substep's output
    T *gprev = lgob + (size_t)(EPW + ew) * NW;   // adjoint of its input
    for (int q = L.agent; q < NW; q += PA) gob[q] = T(0);
    St<T> gs;
    st_zero(gs);
    for (int t = g.nsteps - 1; t >= 0; --t) {
        if (t == g.nsteps - 1)
            add_adj<T, DRONE>(g.afin.f, L.idx, gs);
        else
            add_adj<T, DRONE>(g.atraj.f, (size_t)t * EA + L.idx, gs);
        progress_priority(g.nsteps - 1 - t, g.nsteps);
        wave_lds_sync();
        if (io.atraj && env_ok)
            for (int q = L.agent; q < NW; q += PA) gob[q] += io.atraj[(size_t)t * ENW + eo + q];
        St<T> st;
        if (t == 0)
            load_state<T, DRONE>(g.s0.f, L.idx, 0, st);
        else
            load_state<T, DRONE>(g.traj.f, L.idx, (size_t)(t - 1) * EA, st);
        if (!L.active) st.px = st.py = __builtin_nan("");
        {
            const T *src = t == 0 ? io.ob0 + eo : io.traj + (size_t)(t - 1) * ENW + eo;
            T *dst = lobs + (size_t)ew * NW;
            for (int q = L.agent; q < NW; q += PA) dst[q] = src[q];
            wave_lds_sync();
            if (lcs) body_trig<T>(tb, SS, X, dst, lcs + (size_t)ew * 2 * N);
        }
        T a[4];
        load_act(g.act, (size_t)t * EA + L.idx, C.ad, a);

        // ---- recompute the substep chain of this step into LDS
        M cand = 0;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < C.S; ++s) {
            T *sl = slots + (size_t)s * NF * 64;
            wave_lds_sync();
            slot_put<T, DRONE>(sl, L.lane, st);
            wave_lds_sync();
            const T *obc = lobs + ((size_t)s * EPW + ew) * NW;
            T Fx, Fy;
            const M incl = forces_b<T, PA>(C, tb, L, sl, lr, obc, st, s, s == 0 || !ok, cand, Fx, Fy);
            sl[F_FX * 64 + L.lane] = Fx;
            sl[F_FY * 64 + L.lane] = Fy;
            lmask[s * 64 + L.lane] = incl;
            const T *rin = io.tape ? io.tape + (((size_t)t * C.S + s) * io.tape_roots * C.E +
                                                (env_ok ? L.env : 0)) * BODY_REC
                                   : nullptr;
            body_pass<T>(C, tb, SS, X, br, st, obc, lobs + ((size_t)(s + 1) * EPW + ew) * NW, lext,
                             lcs ? lcs + ((size_t)s * EPW + ew) * 2 * N : nullptr,
                             lcs ? lcs + ((size_t)(s + 1) * EPW + ew) * 2 * N : nullptr,
                             lsum ? lsum + ((size_t)s * EPW + ew) * 3 * N : nullptr, rin, nullptr,
                             (size_t)C.E * BODY_REC, io.tape_roots);
            // the last substep's agent output is the step's checkpoint: not needed here
            if (s + 1 < C.S) {
                St<T> nx;
                integrate<T, DRONE>(C, L.pr, st, a, Fx, Fy, nx);
                if (C.use_skin) {
                    D += (m_abs(nx.px - st.px) + m_abs(nx.py - st.py)) * T(1.0001);
                    ok = env_all<PA>(!L.active || D <= C.half_margin, L.base);
                }
                st = nx;
            }
        }

        // ---- reverse pass
        T ga[4] = {T(0), T(0), T(0), T(0)};
        for (int s = C.S - 1; s >= 0; --s) {
            T *sl = slots + (size_t)s * NF * 64;
            const T *obc = lobs + ((size_t)s * EPW + ew) * NW;
            wave_lds_sync();
            St<T> in;
            slot_get<T, DRONE>(sl, L.lane, in);
            const T Fx = sl[F_FX * 64 + L.lane], Fy = sl[F_FY * 64 + L.lane];
            St<T> gi;
            T gFx, gFy;
            integrate_adj<T, DRONE>(C, L.pr, in, a, Fx, Fy, gs, gi, ga, gFx, gFy);
            // the body pass: adjoint of its input obstacle state into gprev
            body_pass_adj<T>(C, tb, SS, X, br, in, obc, gob, gprev, gi, lext,
                                 lcs ? lcs + ((size_t)s * EPW + ew) * 2 * N : nullptr,
                                 lcs ? lcs + ((size_t)(s + 1) * EPW + ew) * 2 * N : nullptr,
                                 lsum ? lsum + ((size_t)s * EPW + ew) * 3 * N : nullptr);
            if (C.needs_forces) {
                const T wFx = gFx * L.inv_dd, wFy = gFy * L.inv_dd;
                wave_lds_sync();
                sl[F_FX * 64 + L.lane] = wFx;
                sl[F_FY * 64 + L.lane] = wFy;
                wave_lds_sync();
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
                        const T dx = in.px - lx[j], dy = in.py - ly[j];
                        const T md = L.pr.radius + lr[j] + C.margin;
                        if (pair_apart(dx, dy, md)) continue;  // no contact: nothing to add
                        const bool own = in_list(mine, b, C.K);
                        const bool rev = in_list(lmask[s * 64 + j], L.agent, C.K);
                        if (!own && !rev) continue;
                        const T wx = (own ? wFx : T(0)) - (rev ? lgx[j] : T(0));
                        const T wy = (own ? wFy : T(0)) - (rev ? lgy[j] : T(0));
                        pair_adj_combined(C, dx, dy, in.vx - lvx[j], in.vy - lvy[j], md, wx, wy,
                                          gi.px, gi.py, gi.vx, gi.vy);
                    }
                }
                // obstacles: the agent's adjoint, and the moving shapes' in agent order
                for (int o = 0; o < N; ++o) {
                    const bool mv = SS.moves(tb, o);
                    T op[6];
                    if (L.active) {
                        ob_force_adj(C, tb, obc, o, in.px, in.py, in.vx, in.vy, L.pr.radius,
                                     L.dd, gFx, gFy, gi, mv, op);
                    } else {
#pragma unroll
                        for (int q = 0; q < 6; ++q) op[q] = T(0);
                    }
                    if (!mv) continue;
                    bool fl = false;
#pragma unroll
                    for (int q = 0; q < 6; ++q) fl = fl || op[q] != T(0);
                    if (__ballot(fl) == 0) continue;  // no agent of the wave touches it
                    // the env's agent-0 lane keeps the shape's adjoint; the other lanes'
                    // copies of the sums are not used
                    T *g2 = gprev + 6 * o;
                    T acc[6] = {g2[0], g2[1], g2[2], g2[3], g2[4], g2[5]};
                    env_ordered_sums<PA, 6>(acc, op, fl, L.lane);
                    if (L.agent == 0) {
#pragma unroll
                        for (int q = 0; q < 6; ++q) g2[q] = acc[q];
                    }
                }
                if (C.soft_walls)
                    wall_force_adj(C, in.px, in.py, in.vx, in.vy, L.pr.radius, L.dd, gFx, gFy, gi);
            }
            gs = gi;
            wave_lds_sync();
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
    wave_lds_sync();
    if (io.a0 && env_ok)
        for (int q = L.agent; q < NW; q += PA) io.a0[eo + q] = gob[q];
}

// ---------------------------------------------------------------------- launchers

template <typename T, bool DRONE> size_t body_bwd_lds_pa(int PA, int S, int N, bool cache)
{
    switch (PA) {
    case 4: return body_bwd_lds<T, 4, DRONE>(S, N, cache);
    case 8: return body_bwd_lds<T, 8, DRONE>(S, N, cache);
    case 16: return body_bwd_lds<T, 16, DRONE>(S, N, cache);
    case 32: return body_bwd_lds<T, 32, DRONE>(S, N, cache);
    default: return body_bwd_lds<T, 64, DRONE>(S, N, cache);
    }
}

template <typename T> size_t body_bwd_lds_of(int PA, int S, int N, bool drone, bool cache)
{
    return drone ? body_bwd_lds_pa<T, true>(PA, S, N, cache)
                 : body_bwd_lds_pa<T, false>(PA, S, N, cache);
}

#define SWARP_BODY_DISPATCH(KERNEL, DR, FP, SHM)                                       \
    switch (PA) {                                                                      \
    case 4: hipLaunchKernelGGL((KERNEL<T, 4, DR, FP>), grid, dim3(64), SHM, st, C, a, tb, io); break; \
    case 8: hipLaunchKernelGGL((KERNEL<T, 8, DR, FP>), grid, dim3(64), SHM, st, C, a, tb, io); break; \
    case 16: hipLaunchKernelGGL((KERNEL<T, 16, DR, FP>), grid, dim3(64), SHM, st, C, a, tb, io); break; \
    case 32: hipLaunchKernelGGL((KERNEL<T, 32, DR, FP>), grid, dim3(64), SHM, st, C, a, tb, io); break; \
    default: hipLaunchKernelGGL((KERNEL<T, 64, DR, FP>), grid, dim3(64), SHM, st, C, a, tb, io); break; \
    }

// The profile besides FT_ALL the body kernels compile for float32 (0: none).
template <typename T> constexpr unsigned body_profile()
{
    return sizeof(T) == 4 ? FT_PROF_BODY : 0u;
}

// feat: the FT_* paths the world uses; the profile runs when it covers them.  A fleet
// holding a drone (all nine state fields stepped) runs the general DRONE instances.
template <typename T>
void launch_body_fwd(int PA, const Cst<T> &C, const Args<T> &a, const ObTab<T> &tb,
                     const ObIO<T> &io, unsigned feat, bool drone, hipStream_t st)
{
    const dim3 grid((C.E + 64 / PA - 1) / (64 / PA));
    constexpr unsigned P = body_profile<T>();
    const size_t shm = body_fwd_lds(PA, tb.N, sizeof(T));
    if (drone) {
        SWARP_BODY_DISPATCH(k_body_fwd, true, FT_ALL, shm)
    } else if (P != 0u && (feat & ~P) == 0u) {
        SWARP_BODY_DISPATCH(k_body_fwd, false, (P ? P : FT_ALL), shm)
    } else {
        SWARP_BODY_DISPATCH(k_body_fwd, false, FT_ALL, shm)
    }
}

template <typename T>
void launch_body_bwd(int PA, const Cst<T> &C, const Args<T> &a, const ObTab<T> &tb,
                     const ObIO<T> &io, unsigned feat, bool drone, size_t shm, hipStream_t st)
{
    const dim3 grid((C.E + 64 / PA - 1) / (64 / PA));
    constexpr unsigned P = body_profile<T>();
    if (drone) {
        SWARP_BODY_DISPATCH(k_body_bwd, true, FT_ALL, shm)
    } else if (P != 0u && (feat & ~P) == 0u) {
        SWARP_BODY_DISPATCH(k_body_bwd, false, (P ? P : FT_ALL), shm)
    } else {
        SWARP_BODY_DISPATCH(k_body_bwd, false, FT_ALL, shm)
    }
}
#undef SWARP_BODY_DISPATCH

}  // namespace swarp
