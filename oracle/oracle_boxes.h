/*
 * oracle_boxes.h -- box agents: oriented-rectangle footprints in the contact pass and
 * the footprint clamp.  TEST INFRASTRUCTURE ONLY (part of the oracle, see
 * swarp_oracle.c).  Included by oracle_impl.h with REAL / FN / the math macros set.
 *
 * Restates, from the reference's source text:
 *   _cross_w, _point_box, _vertex_vs_box   swarp/core/collisions.py:266-310
 *   obb_contact, obb_force                 swarp/core/collisions.py:312-487
 *   _agent_pair_force                      swarp/core/collisions.py:489-541
 *   _box_obstacle_force, _obstacle_forces_box   swarp/core/collisions.py:543-626
 *   _sgn0, _wall_forces_box                swarp/core/collisions.py:628-688
 *   _static_forces_shaped                  swarp/core/collisions.py:950-996
 *   collision_forces_box_kernel            swarp/core/collisions.py:999-1059
 *   clamp_footprint                        swarp/dynamics/kernels.py:79-99
 *
 * Every function is written once, on forward-mode dual numbers with one tangent: the
 * value part is the forward pass (same operations in the same order as the reference),
 * and one evaluation per seeded input gives one column of the force's Jacobian.  The
 * reverse pass of the contact (forces_env_adj) contracts those columns with the force
 * adjoint, which is the derivative warp-lang's generated adjoint computes: both follow the
 * branch the forward pass took, and both differentiate
 *   max(a, b) -> the operand returned, clamp(x, a, b) -> the operand returned,
 *   abs(x) -> sign(x) (+1 at 0), sqrt(x) -> 1 / (2 sqrt(x)).
 */

typedef struct {
    REAL v, d; /* value, tangent */
} FN(dn);

#define D FN(dn)
static inline D FN(dk)(REAL v)
{
    D r = {v, (REAL)0};
    return r;
}
static inline D FN(dadd)(D a, D b)
{
    D r = {a.v + b.v, a.d + b.d};
    return r;
}
static inline D FN(dsub)(D a, D b)
{
    D r = {a.v - b.v, a.d - b.d};
    return r;
}
static inline D FN(dmul)(D a, D b)
{
    D r = {a.v * b.v, a.d * b.v + a.v * b.d};
    return r;
}
static inline D FN(dscale)(D a, REAL k) /* a * k */
{
    D r = {a.v * k, a.d * k};
    return r;
}
static inline D FN(ddivk)(D a, REAL k) /* a / k */
{
    D r = {a.v / k, a.d / k};
    return r;
}
static inline D FN(ddiv)(D a, D b)
{
    REAL q = a.v / b.v;
    D r = {q, (a.d - q * b.d) / b.v};
    return r;
}
static inline D FN(dneg)(D a)
{
    D r = {-a.v, -a.d};
    return r;
}
static inline D FN(dsqrt)(D a)
{
    REAL s = SQRT(a.v);
    D r = {s, s > (REAL)0 ? a.d * (REAL)0.5 / s : (REAL)0};
    return r;
}
static inline D FN(dabs)(D a)
{
    D r = {FABS(a.v), a.v < (REAL)0 ? -a.d : a.d};
    return r;
}
static inline D FN(dcos)(D a)
{
    D r = {COS(a.v), -SIN(a.v) * a.d};
    return r;
}
static inline D FN(dsin)(D a)
{
    D r = {SIN(a.v), COS(a.v) * a.d};
    return r;
}
static inline D FN(dtanh)(D a)
{
    REAL t = TANH(a.v);
    D r = {t, ((REAL)1 - t * t) * a.d};
    return r;
}
static inline D FN(dmax)(D a, D b) { return a.v > b.v ? a : b; }
static inline D FN(dmin)(D a, D b) { return a.v < b.v ? a : b; }
/* clamp(x, a, b) = min(max(a, x), b) */
static inline D FN(dclamp)(D x, D a, D b)
{
    D m = a.v > x.v ? a : x;
    return m.v < b.v ? m : b;
}
static inline D FN(ddot)(D ax, D ay, D bx, D by)
{
    return FN(dadd)(FN(dmul)(ax, bx), FN(dmul)(ay, by));
}

/* Agent state as seen by the contact pass: px py th vx vy w (defined once for both
   precisions) */
#ifndef ORACLE_BOXES_ENUM
#define ORACLE_BOXES_ENUM
enum { BX_PX, BX_PY, BX_TH, BX_VX, BX_VY, BX_W, BX_N };
#endif

static inline void FN(dstate)(const FN(agent_t) *s, int seed, D *o)
{
    o[BX_PX] = FN(dk)(s->px);
    o[BX_PY] = FN(dk)(s->py);
    o[BX_TH] = FN(dk)(s->th);
    o[BX_VX] = FN(dk)(s->vx);
    o[BX_VY] = FN(dk)(s->vy);
    o[BX_W] = FN(dk)(s->w);
    if (seed >= 0) o[seed].d = (REAL)1;
}

/* adjoint of field `k` of an agent state */
static inline REAL *FN(bx_field)(FN(agent_t) *a, int k)
{
    switch (k) {
    case BX_PX: return &a->px;
    case BX_PY: return &a->py;
    case BX_TH: return &a->th;
    case BX_VX: return &a->vx;
    case BX_VY: return &a->vy;
    default: return &a->w;
    }
}

/* _normal_coeff (collisions.py:87-105) */
static inline D FN(d_normal_coeff)(const FN(ctx_t) *C, D ov, D vn, REAL dd)
{
    D o = ov;
    if (C->max_overlap > (REAL)0)
        o = FN(dscale)(FN(dtanh)(FN(ddivk)(ov, C->max_overlap)), C->max_overlap);
    D num = FN(dsub)(FN(dscale)(o, C->k), FN(dscale)(vn, C->c));
    return FN(dmax)(FN(ddivk)(num, dd), FN(dk)((REAL)0));
}

/* box_force (collisions.py:174-260) with every input a dual: point (p, v) against the
   box (center, angle, half) moving with (vo, om); reach = point radius + margin. */
static void FN(d_box_force)(const FN(ctx_t) *C, D px, D py, D vx, D vy, D cx0, D cy0, D ang,
                            REAL hx, REAL hy, REAL reach, REAL dd, D vox, D voy, D om, D *fx,
                            D *fy)
{
    D ca = FN(dcos)(ang), sa = FN(dsin)(ang);
    D dx = FN(dsub)(px, cx0), dy = FN(dsub)(py, cy0);
    D lx = FN(dadd)(FN(dmul)(ca, dx), FN(dmul)(sa, dy));
    D ly = FN(dadd)(FN(dmul)(FN(dneg)(sa), dx), FN(dmul)(ca, dy));
    D qx = FN(dsub)(FN(dabs)(lx), FN(dk)(hx)), qy = FN(dsub)(FN(dabs)(ly), FN(dk)(hy));
    D cx = FN(dclamp)(lx, FN(dk)(-hx), FN(dk)(hx)), cy = FN(dclamp)(ly, FN(dk)(-hy), FN(dk)(hy));
    D ox = FN(dsub)(lx, cx), oy = FN(dsub)(ly, cy);
    D od2 = FN(dadd)(FN(dmul)(ox, ox), FN(dmul)(oy, oy));
    D s, nlx, nly;
    if (od2.v > C->eps2) {
        s = FN(dsqrt)(od2);
        nlx = FN(ddiv)(ox, s);
        nly = FN(ddiv)(oy, s);
    } else if (qx.v > qy.v) {
        s = qx;
        nlx = FN(dk)(lx.v >= (REAL)0 ? (REAL)1 : (REAL)-1);
        nly = FN(dk)((REAL)0);
    } else {
        s = qy;
        nlx = FN(dk)((REAL)0);
        nly = FN(dk)(ly.v >= (REAL)0 ? (REAL)1 : (REAL)-1);
    }
    *fx = FN(dk)((REAL)0);
    *fy = FN(dk)((REAL)0);
    D ov = FN(dsub)(FN(dk)(reach), s);
    if (ov.v > (REAL)0) {
        D nx = FN(dsub)(FN(dmul)(ca, nlx), FN(dmul)(sa, nly));
        D ny = FN(dadd)(FN(dmul)(sa, nlx), FN(dmul)(ca, nly));
        D spx = FN(dsub)(lx, FN(dmul)(s, nlx)), spy = FN(dsub)(ly, FN(dmul)(s, nly));
        D rx = FN(dsub)(FN(dmul)(ca, spx), FN(dmul)(sa, spy));
        D ry = FN(dadd)(FN(dmul)(sa, spx), FN(dmul)(ca, spy));
        D vsx = FN(dadd)(vox, FN(dmul)(FN(dneg)(om), ry)), vsy = FN(dadd)(voy, FN(dmul)(om, rx));
        D rvx = FN(dsub)(vx, vsx), rvy = FN(dsub)(vy, vsy);
        D coef = FN(d_normal_coeff)(C, ov, FN(ddot)(rvx, rvy, nx, ny), dd);
        *fx = FN(dmul)(coef, nx);
        *fy = FN(dmul)(coef, ny);
    }
}

/* _point_box (collisions.py:273-290): distance (floored) and closest point from a point
   outside an oriented box */
static void FN(d_point_box)(const FN(ctx_t) *C, D vx, D vy, D cx, D cy, D ca, D sa, REAL hx,
                            REAL hy, D *dist, D *qx, D *qy)
{
    D dx = FN(dsub)(vx, cx), dy = FN(dsub)(vy, cy);
    D lx = FN(dadd)(FN(dmul)(ca, dx), FN(dmul)(sa, dy));
    D ly = FN(dadd)(FN(dmul)(FN(dneg)(sa), dx), FN(dmul)(ca, dy));
    D kx = FN(dclamp)(lx, FN(dk)(-hx), FN(dk)(hx)), ky = FN(dclamp)(ly, FN(dk)(-hy), FN(dk)(hy));
    D ox = FN(dsub)(lx, kx), oy = FN(dsub)(ly, ky);
    *dist = FN(dsqrt)(FN(dmax)(FN(dadd)(FN(dmul)(ox, ox), FN(dmul)(oy, oy)), FN(dk)(C->eps2)));
    *qx = FN(dadd)(cx, FN(dsub)(FN(dmul)(ca, kx), FN(dmul)(sa, ky)));
    *qy = FN(dadd)(cy, FN(dadd)(FN(dmul)(sa, kx), FN(dmul)(ca, ky)));
}

/* _vertex_vs_box (collisions.py:293-310): keep (best, normal, point) or replace it by
   vertex v against a box; flip = +1 for a vertex of A, -1 for a vertex of B */
static void FN(d_vertex_vs_box)(const FN(ctx_t) *C, D vx, D vy, D cx, D cy, D ca, D sa,
                                REAL hx, REAL hy, REAL flip, D *best, D *nx, D *ny, D *xx,
                                D *xy)
{
    D dist, qx, qy;
    FN(d_point_box)(C, vx, vy, cx, cy, ca, sa, hx, hy, &dist, &qx, &qy);
    if (dist.v < best->v) {
        D sc = FN(ddiv)(FN(dk)(flip), dist);
        *best = dist;
        *nx = FN(dmul)(FN(dsub)(vx, qx), sc);
        *ny = FN(dmul)(FN(dsub)(vy, qy), sc);
        *xx = FN(dscale)(FN(dadd)(vx, qx), (REAL)0.5);
        *xy = FN(dscale)(FN(dadd)(vy, qy), (REAL)0.5);
    }
}

/* obb_contact (collisions.py:312-447): signed distance s, unit normal n (B -> A) and
   contact point x of two oriented boxes */
static void FN(d_obb_contact)(const FN(ctx_t) *C, D cAx, D cAy, D thA, REAL hA0, REAL hA1,
                              D cBx, D cBy, D thB, REAL hB0, REAL hB1, REAL reach, D *s_o,
                              D *nx_o, D *ny_o, D *xx_o, D *xy_o)
{
    D caA = FN(dcos)(thA), saA = FN(dsin)(thA), caB = FN(dcos)(thB), saB = FN(dsin)(thB);
    D uA0x = caA, uA0y = saA, uA1x = FN(dneg)(saA), uA1y = caA;
    D uB0x = caB, uB0y = saB, uB1x = FN(dneg)(saB), uB1y = caB;
    D dx = FN(dsub)(cAx, cBx), dy = FN(dsub)(cAy, cBy);
    D a00 = FN(dabs)(FN(ddot)(uA0x, uA0y, uB0x, uB0y));
    D a01 = FN(dabs)(FN(ddot)(uA0x, uA0y, uB1x, uB1y));
    D a10 = FN(dabs)(FN(ddot)(uA1x, uA1y, uB0x, uB0y));
    D a11 = FN(dabs)(FN(ddot)(uA1x, uA1y, uB1x, uB1y));
    D dA0 = FN(ddot)(dx, dy, uA0x, uA0y), dA1 = FN(ddot)(dx, dy, uA1x, uA1y);
    D dB0 = FN(ddot)(dx, dy, uB0x, uB0y), dB1 = FN(ddot)(dx, dy, uB1x, uB1y);

    /* projection gap along each face normal; the largest is the SAT separation */
    D s = FN(dsub)(FN(dsub)(FN(dabs)(dA0), FN(dk)(hA0)),
                   FN(dadd)(FN(dscale)(a00, hB0), FN(dscale)(a01, hB1)));
    int axis = 0;
    D t = FN(dsub)(FN(dsub)(FN(dabs)(dA1), FN(dk)(hA1)),
                   FN(dadd)(FN(dscale)(a10, hB0), FN(dscale)(a11, hB1)));
    if (t.v > s.v) {
        s = t;
        axis = 1;
    }
    t = FN(dsub)(FN(dsub)(FN(dabs)(dB0), FN(dk)(hB0)),
                 FN(dadd)(FN(dscale)(a00, hA0), FN(dscale)(a10, hA1)));
    if (t.v > s.v) {
        s = t;
        axis = 2;
    }
    t = FN(dsub)(FN(dsub)(FN(dabs)(dB1), FN(dk)(hB1)),
                 FN(dadd)(FN(dscale)(a01, hA0), FN(dscale)(a11, hA1)));
    if (t.v > s.v) {
        s = t;
        axis = 3;
    }

    D nx = FN(dk)((REAL)0), ny = FN(dk)((REAL)0), xx = cAx, xy = cAy;
    if (s.v > reach) {
        /* no contact; s is a lower bound on the gap */
    } else if (s.v > (REAL)0) {
        /* disjoint: the exact distance, attained at a vertex of one box */
        D eA0x = FN(dscale)(uA0x, hA0), eA0y = FN(dscale)(uA0y, hA0);
        D eA1x = FN(dscale)(uA1x, hA1), eA1y = FN(dscale)(uA1y, hA1);
        D eB0x = FN(dscale)(uB0x, hB0), eB0y = FN(dscale)(uB0y, hB0);
        D eB1x = FN(dscale)(uB1x, hB1), eB1y = FN(dscale)(uB1y, hB1);
        D best = FN(dk)((REAL)1.0e30);
        const REAL one = (REAL)1;
        /* vertex signs (+,+) (-,+) (-,-) (+,-) of e0, e1 */
        for (int q = 0; q < 8; ++q) {
            int k = q & 3;
            REAL s0 = (k == 0 || k == 3) ? one : -one;
            REAL s1 = (k < 2) ? one : -one;
            if (q < 4) {
                D e0x = s0 > 0 ? eA0x : FN(dneg)(eA0x), e0y = s0 > 0 ? eA0y : FN(dneg)(eA0y);
                D e1x = s1 > 0 ? eA1x : FN(dneg)(eA1x), e1y = s1 > 0 ? eA1y : FN(dneg)(eA1y);
                D vx = FN(dadd)(FN(dadd)(cAx, e0x), e1x), vy = FN(dadd)(FN(dadd)(cAy, e0y), e1y);
                FN(d_vertex_vs_box)(C, vx, vy, cBx, cBy, caB, saB, hB0, hB1, one, &best, &nx,
                                    &ny, &xx, &xy);
            } else {
                D e0x = s0 > 0 ? eB0x : FN(dneg)(eB0x), e0y = s0 > 0 ? eB0y : FN(dneg)(eB0y);
                D e1x = s1 > 0 ? eB1x : FN(dneg)(eB1x), e1y = s1 > 0 ? eB1y : FN(dneg)(eB1y);
                D vx = FN(dadd)(FN(dadd)(cBx, e0x), e1x), vy = FN(dadd)(FN(dadd)(cBy, e0y), e1y);
                FN(d_vertex_vs_box)(C, vx, vy, cAx, cAy, caA, saA, hA0, hA1, -one, &best, &nx,
                                    &ny, &xx, &xy);
            }
        }
        s = best;
    } else {
        /* overlapping: the axis of least overlap (oriented B -> A) and its reference face */
        D ux = uA0x, uy = uA0y, tx = uA1x, ty = uA1y, dn = dA0;
        REAL h_n = hA0, h_t = hA1;
        D r_t = FN(dadd)(FN(dscale)(a10, hB0), FN(dscale)(a11, hB1));
        if (axis == 1) {
            ux = uA1x; uy = uA1y; tx = uA0x; ty = uA0y; dn = dA1;
            h_n = hA1; h_t = hA0;
            r_t = FN(dadd)(FN(dscale)(a00, hB0), FN(dscale)(a01, hB1));
        } else if (axis == 2) {
            ux = uB0x; uy = uB0y; tx = uB1x; ty = uB1y; dn = dB0;
            h_n = hB0; h_t = hB1;
            r_t = FN(dadd)(FN(dscale)(a01, hA0), FN(dscale)(a11, hA1));
        } else if (axis == 3) {
            ux = uB1x; uy = uB1y; tx = uB0x; ty = uB0y; dn = dB1;
            h_n = hB1; h_t = hB0;
            r_t = FN(dadd)(FN(dscale)(a00, hA0), FN(dscale)(a10, hA1));
        }
        REAL sgn = dn.v < (REAL)0 ? (REAL)-1 : (REAL)1;
        nx = FN(dscale)(ux, sgn);
        ny = FN(dscale)(uy, sgn);
        D crx = cAx, cry = cAy, cix = cBx, ciy = cBy;
        D xn = FN(dsub)(FN(ddot)(cAx, cAy, nx, ny), FN(dk)(h_n));
        if (axis >= 2) {
            crx = cBx; cry = cBy; cix = cAx; ciy = cAy;
            xn = FN(dadd)(FN(ddot)(cBx, cBy, nx, ny), FN(dk)(h_n));
        }
        D ct_ref = FN(ddot)(crx, cry, tx, ty), ct_inc = FN(ddot)(cix, ciy, tx, ty);
        D lo = FN(dmax)(FN(dsub)(ct_ref, FN(dk)(h_t)), FN(dsub)(ct_inc, r_t));
        D hi = FN(dmin)(FN(dadd)(ct_ref, FN(dk)(h_t)), FN(dadd)(ct_inc, r_t));
        D mid = FN(dmul)(FN(dk)((REAL)0.5), FN(dadd)(lo, hi));
        xx = FN(dadd)(FN(dmul)(nx, xn), FN(dmul)(tx, mid));
        xy = FN(dadd)(FN(dmul)(ny, xn), FN(dmul)(ty, mid));
    }
    *s_o = s;
    *nx_o = nx;
    *ny_o = ny;
    *xx_o = xx;
    *xy_o = xy;
}

/* obb_force (collisions.py:449-487): force on box A from box B */
static void FN(d_obb_force)(const FN(ctx_t) *C, D cAx, D cAy, D thA, REAL hA0, REAL hA1, D vAx,
                            D vAy, D wA, D cBx, D cBy, D thB, REAL hB0, REAL hB1, D vBx, D vBy,
                            D wB, REAL reach, REAL dd, D *fx, D *fy, D *xo, D *yo)
{
    D s, nx, ny, xx, xy;
    FN(d_obb_contact)(C, cAx, cAy, thA, hA0, hA1, cBx, cBy, thB, hB0, hB1, reach, &s, &nx, &ny,
                      &xx, &xy);
    *fx = FN(dk)((REAL)0);
    *fy = FN(dk)((REAL)0);
    D ov = FN(dsub)(FN(dk)(reach), s);
    if (ov.v > (REAL)0) {
        /* material-point velocities at x: v + w x (x - c), w x r = (-w r_y, w r_x) */
        D rAx = FN(dsub)(xx, cAx), rAy = FN(dsub)(xy, cAy);
        D rBx = FN(dsub)(xx, cBx), rBy = FN(dsub)(xy, cBy);
        D pax = FN(dadd)(vAx, FN(dmul)(FN(dneg)(wA), rAy)), pay = FN(dadd)(vAy, FN(dmul)(wA, rAx));
        D pbx = FN(dadd)(vBx, FN(dmul)(FN(dneg)(wB), rBy)), pby = FN(dadd)(vBy, FN(dmul)(wB, rBx));
        D rvx = FN(dsub)(pax, pbx), rvy = FN(dsub)(pay, pby);
        D coef = FN(d_normal_coeff)(C, ov, FN(ddot)(rvx, rvy, nx, ny), dd);
        *fx = FN(dmul)(coef, nx);
        *fy = FN(dmul)(coef, ny);
    }
    if (xo) *xo = xx;
    if (yo) *yo = xy;
}

/* _agent_pair_force (collisions.py:489-541): force on agent a (state sa) from agent b
   (state sb); disc-disc pairs take pair_force directly and never come here. */
static void FN(d_agent_pair_force)(const FN(ctx_t) *C, int a, int b, const FN(prm_t) *Pa,
                                   const FN(prm_t) *Pb, const D *sa, const D *sb, REAL dd,
                                   D *fx, D *fy)
{
    const REAL half = (REAL)0.5;
    if (Pa->shape < half) {
        /* disc a against box b: box_force with a as the point */
        FN(d_box_force)(C, sa[BX_PX], sa[BX_PY], sa[BX_VX], sa[BX_VY], sb[BX_PX], sb[BX_PY],
                        sb[BX_TH], Pb->hx, Pb->hy, Pa->radius + C->margin, dd, sb[BX_VX],
                        sb[BX_VY], sb[BX_W], fx, fy);
    } else if (Pb->shape < half) {
        /* box a against disc b: minus the disc's box_force */
        D gx, gy;
        FN(d_box_force)(C, sb[BX_PX], sb[BX_PY], sb[BX_VX], sb[BX_VY], sa[BX_PX], sa[BX_PY],
                        sa[BX_TH], Pa->hx, Pa->hy, Pb->radius + C->margin, dd, sa[BX_VX],
                        sa[BX_VY], sa[BX_W], &gx, &gy);
        *fx = FN(dneg)(gx);
        *fy = FN(dneg)(gy);
    } else if (a < b) {
        FN(d_obb_force)(C, sa[BX_PX], sa[BX_PY], sa[BX_TH], Pa->hx, Pa->hy, sa[BX_VX], sa[BX_VY],
                        sa[BX_W], sb[BX_PX], sb[BX_PY], sb[BX_TH], Pb->hx, Pb->hy, sb[BX_VX],
                        sb[BX_VY], sb[BX_W], C->margin, dd, fx, fy, NULL, NULL);
    } else {
        /* the lower index is box A on both threads: one contact, opposite signs */
        D gx, gy;
        FN(d_obb_force)(C, sb[BX_PX], sb[BX_PY], sb[BX_TH], Pb->hx, Pb->hy, sb[BX_VX], sb[BX_VY],
                        sb[BX_W], sa[BX_PX], sa[BX_PY], sa[BX_TH], Pa->hx, Pa->hy, sa[BX_VX],
                        sa[BX_VY], sa[BX_W], C->margin, dd, &gx, &gy, NULL, NULL);
        *fx = FN(dneg)(gx);
        *fy = FN(dneg)(gy);
    }
}

/* _obstacle_forces_box + _box_obstacle_force (collisions.py:543-626) and, with soft
   walls, _wall_forces_box (:641-688): the static forces on a box agent, obstacles in
   index order, then the walls (_static_forces_shaped, :950-996).  od: this env's
   obstacle state (6 reals per shape: pos, angle, vel, ang_vel). */
static void FN(d_box_static_forces)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                                    const D *s, REAL dd, D *fx_o, D *fy_o)
{
    const REAL hx = P->hx, hy = P->hy;
    const REAL ra = SQRT(hx * hx + hy * hy);
    D fx = FN(dk)((REAL)0), fy = FN(dk)((REAL)0);
    for (int o = 0; o < C->n_obs; ++o) {
        const REAL *sh = od + 6 * o;
        int st = C->o_type[o];
        REAL ro = C->o_rad[o], ohx = C->o_half[o * 2], ohy = C->o_half[o * 2 + 1];
        if (FN(bounds_apart)(s[BX_PX].v - sh[0], s[BX_PY].v - sh[1],
                             ra + C->margin + FN(shape_bound)(st, ro, ohx, ohy)))
            continue;
        D cx = FN(dk)(sh[0]), cy = FN(dk)(sh[1]), ang = FN(dk)(sh[2]);
        D vox = FN(dk)(sh[3]), voy = FN(dk)(sh[4]), om = FN(dk)(sh[5]);
        D gx, gy;
        if (st == 1) {
            FN(d_obb_force)(C, s[BX_PX], s[BX_PY], s[BX_TH], hx, hy, s[BX_VX], s[BX_VY], s[BX_W],
                            cx, cy, ang, ohx, ohy, vox, voy, om, C->margin, dd, &gx, &gy, NULL, NULL);
        } else if (st == 2) {
            /* a capsule: the degenerate box (half_len, 0), reach grown by its radius */
            FN(d_obb_force)(C, s[BX_PX], s[BX_PY], s[BX_TH], hx, hy, s[BX_VX], s[BX_VY], s[BX_W],
                            cx, cy, ang, ohx, (REAL)0, vox, voy, om, ro + C->margin, dd, &gx,
                            &gy, NULL, NULL);
        } else {
            /* a circle: minus box_force with the circle centre as the point */
            D hxv, hyv;
            FN(d_box_force)(C, cx, cy, vox, voy, s[BX_PX], s[BX_PY], s[BX_TH], hx, hy,
                            ro + C->margin, dd, s[BX_VX], s[BX_VY], s[BX_W], &hxv, &hyv);
            gx = FN(dneg)(hxv);
            gy = FN(dneg)(hyv);
        }
        fx = FN(dadd)(fx, gx);
        fy = FN(dadd)(fy, gy);
    }
    if (C->soft_walls) {
        /* _wall_forces_box: support extents replace the radius; the damper reads the
           velocity of the support vertex touching each wall */
        D ca = FN(dcos)(s[BX_TH]), sa = FN(dsin)(s[BX_TH]);
        D ex = FN(dadd)(FN(dscale)(FN(dabs)(ca), hx), FN(dscale)(FN(dabs)(sa), hy));
        D ey = FN(dadd)(FN(dscale)(FN(dabs)(sa), hx), FN(dscale)(FN(dabs)(ca), hy));
        REAL sc = ca.v > (REAL)0 ? (REAL)1 : (ca.v < (REAL)0 ? (REAL)-1 : (REAL)0);
        REAL ss = sa.v > (REAL)0 ? (REAL)1 : (sa.v < (REAL)0 ? (REAL)-1 : (REAL)0);
        D rl_y = FN(dadd)(FN(dscale)(sa, -sc * hx), FN(dscale)(ca, ss * hy));
        D rb_x = FN(dadd)(FN(dscale)(ca, -ss * hx), FN(dscale)(sa, sc * hy));
        D wx = FN(dk)((REAL)0), wy = FN(dk)((REAL)0);
        D px = s[BX_PX], py = s[BX_PY], vx = s[BX_VX], vy = s[BX_VY], w = s[BX_W];
        D em = FN(dadd)(ex, FN(dk)(C->margin)), eym = FN(dadd)(ey, FN(dk)(C->margin));
        D pen = FN(dsub)(em, FN(dsub)(px, FN(dk)(C->bmin_x)));
        if (pen.v > (REAL)0)
            wx = FN(dadd)(wx, FN(d_normal_coeff)(C, pen, FN(dsub)(vx, FN(dmul)(w, rl_y)), dd));
        pen = FN(dsub)(em, FN(dsub)(FN(dk)(C->bmax_x), px));
        if (pen.v > (REAL)0)
            wx = FN(dadd)(wx, FN(dneg)(FN(d_normal_coeff)(
                                  C, pen, FN(dneg)(FN(dadd)(vx, FN(dmul)(w, rl_y))), dd)));
        pen = FN(dsub)(eym, FN(dsub)(py, FN(dk)(C->bmin_y)));
        if (pen.v > (REAL)0)
            wy = FN(dadd)(wy, FN(d_normal_coeff)(C, pen, FN(dadd)(vy, FN(dmul)(w, rb_x)), dd));
        pen = FN(dsub)(eym, FN(dsub)(FN(dk)(C->bmax_y), py));
        if (pen.v > (REAL)0)
            wy = FN(dadd)(wy, FN(dneg)(FN(d_normal_coeff)(
                                  C, pen, FN(dneg)(FN(dsub)(vy, FN(dmul)(w, rb_x))), dd)));
        fx = FN(dadd)(fx, wx);
        fy = FN(dadd)(fy, wy);
    }
    *fx_o = fx;
    *fy_o = fy;
}

#undef D

/* ---------------------------------------------------------- the box-world force pass */

/* collision_forces_box_kernel (collisions.py:999-1059) for one env: pairs dispatch on
   the two shapes, disc-disc pairs and disc agents' static forces exactly as in the disc
   kernel. */
static void FN(forces_env_box)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                               const FN(agent_t) *st, const int32_t *idx, const int32_t *cnt,
                               REAL *F)
{
    int A = C->n_agents, K = C->max_nbr;
    const REAL half = (REAL)0.5;
    for (int a = 0; a < A; ++a) {
        REAL px = st[a].px, py = st[a].py, vx = st[a].vx, vy = st[a].vy;
        REAL ra = P[a].radius;
        REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
        FN(dn) sa[BX_N];
        FN(dstate)(st + a, -1, sa);
        REAL fx = 0, fy = 0;
        int n = C->collisions ? cnt[a] : 0;
        for (int i = 0; i < n; ++i) {
            int b = idx[a * K + i];
            REAL gx, gy;
            if (P[a].shape < half && P[b].shape < half) {
                FN(pair_force)(C, px - st[b].px, py - st[b].py, vx - st[b].vx, vy - st[b].vy,
                               ra + P[b].radius + C->margin, dd, &gx, &gy);
            } else {
                FN(dn) sb[BX_N], dx, dy;
                FN(dstate)(st + b, -1, sb);
                FN(d_agent_pair_force)(C, a, b, P + a, P + b, sa, sb, dd, &dx, &dy);
                gx = dx.v;
                gy = dy.v;
            }
            fx += gx;
            fy += gy;
        }
        REAL sx = 0, sy = 0;
        if (P[a].shape < half) {
            for (int o = 0; o < C->n_obs; ++o) {
                REAL gx, gy;
                FN(obstacle_force)(C, od, o, px, py, vx, vy, ra, dd, &gx, &gy);
                sx += gx;
                sy += gy;
            }
            if (C->soft_walls) {
                REAL gx, gy;
                FN(wall_force)(C, px, py, vx, vy, ra, dd, &gx, &gy);
                sx += gx;
                sy += gy;
            }
        } else {
            FN(dn) dx, dy;
            FN(d_box_static_forces)(C, od, P + a, sa, dd, &dx, &dy);
            sx = dx.v;
            sy = dy.v;
        }
        F[a * 2] = fx + sx;
        F[a * 2 + 1] = fy + sy;
    }
}

/* Reverse of forces_env_box: aF = adjoint of the forces; accumulates into adj.  A pair
   or static force involving a box is differentiated by seeding each of the six state
   fields (px py th vx vy w) of both agents in turn. */
static void FN(forces_env_box_adj)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                                   const FN(agent_t) *st, const int32_t *idx,
                                   const int32_t *cnt, const REAL *aF, FN(agent_t) *adj)
{
    int A = C->n_agents, K = C->max_nbr;
    const REAL half = (REAL)0.5;
    for (int a = 0; a < A; ++a) {
        REAL gfx = aF[a * 2], gfy = aF[a * 2 + 1];
        if (gfx == (REAL)0 && gfy == (REAL)0) continue;
        REAL px = st[a].px, py = st[a].py, vx = st[a].vx, vy = st[a].vy;
        REAL ra = P[a].radius;
        REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
        int n = C->collisions ? cnt[a] : 0;
        for (int i = 0; i < n; ++i) {
            int b = idx[a * K + i];
            if (P[a].shape < half && P[b].shape < half) {
                REAL adx = 0, ady = 0, arvx = 0, arvy = 0;
                FN(pair_force_adj)(C, px - st[b].px, py - st[b].py, vx - st[b].vx,
                                   vy - st[b].vy, ra + P[b].radius + C->margin, dd, gfx, gfy,
                                   &adx, &ady, &arvx, &arvy);
                adj[a].px += adx;
                adj[a].py += ady;
                adj[a].vx += arvx;
                adj[a].vy += arvy;
                adj[b].px -= adx;
                adj[b].py -= ady;
                adj[b].vx -= arvx;
                adj[b].vy -= arvy;
                continue;
            }
            for (int side = 0; side < 2; ++side) {
                for (int k = 0; k < BX_N; ++k) {
                    FN(dn) sa[BX_N], sb[BX_N], dx, dy;
                    FN(dstate)(st + a, side == 0 ? k : -1, sa);
                    FN(dstate)(st + b, side == 1 ? k : -1, sb);
                    FN(d_agent_pair_force)(C, a, b, P + a, P + b, sa, sb, dd, &dx, &dy);
                    *FN(bx_field)(adj + (side == 0 ? a : b), k) += gfx * dx.d + gfy * dy.d;
                }
            }
        }
        if (P[a].shape < half) {
            for (int o = 0; o < C->n_obs; ++o)
                FN(obstacle_force_adj)(C, od, o, px, py, vx, vy, ra, dd, gfx, gfy, &adj[a].px,
                                       &adj[a].py, &adj[a].vx, &adj[a].vy, NULL);
            if (C->soft_walls)
                FN(wall_force_adj)(C, px, py, vx, vy, ra, dd, gfx, gfy, &adj[a].px, &adj[a].py,
                                   &adj[a].vx, &adj[a].vy);
        } else {
            for (int k = 0; k < BX_N; ++k) {
                FN(dn) sa[BX_N], dx, dy;
                FN(dstate)(st + a, k, sa);
                FN(d_box_static_forces)(C, od, P + a, sa, dd, &dx, &dy);
                *FN(bx_field)(adj + a, k) += gfx * dx.d + gfy * dy.d;
            }
        }
    }
}

/* ------------------------------------------------------------- wheel contacts */
/* WorldConfig.wheel_contacts (no-grad Euler 2-D path only): the force pass also returns
   each agent's contact torque about its centre (collision_forces_wheel_kernel,
   swarp/core/collisions.py:1128-1403) and a diff-drive agent's step is reworked by
   wheel_contact (swarp/dynamics/kernels.py:1328-1387). */

static inline REAL FN(cross2)(REAL rx, REAL ry, REAL fx, REAL fy) { return rx * fy - ry * fx; }

/* _box_sd (collisions.py:1133-1141): signed distance from a point to an oriented box */
static REAL FN(box_sd)(REAL vx, REAL vy, REAL cx, REAL cy, REAL ca, REAL sa, REAL h0, REAL h1)
{
    REAL dx = vx - cx, dy = vy - cy;
    REAL lx = FABS(ca * dx + sa * dy) - h0;
    REAL ly = FABS(-sa * dx + ca * dy) - h1;
    REAL ox = FN(rmax)(lx, (REAL)0), oy = FN(rmax)(ly, (REAL)0);
    REAL m = FN(rmax)(lx, ly);
    m = m < (REAL)0 ? m : (REAL)0;
    return SQRT(ox * ox + oy * oy) + m;
}

/* _manifold_point (collisions.py:1144-1185): the in-reach vertices of either box averaged
   with their depths as weights; (x, y) when none is in reach */
static void FN(manifold_point)(REAL cAx, REAL cAy, REAL thA, REAL hA0, REAL hA1, REAL cBx,
                               REAL cBy, REAL thB, REAL hB0, REAL hB1, REAL reach, REAL *x,
                               REAL *y)
{
    REAL caA = COS(thA), saA = SIN(thA), caB = COS(thB), saB = SIN(thB);
    REAL eA0x = caA * hA0, eA0y = saA * hA0, eA1x = -saA * hA1, eA1y = caA * hA1;
    REAL eB0x = caB * hB0, eB0y = saB * hB0, eB1x = -saB * hB1, eB1y = caB * hB1;
    REAL ax = 0, ay = 0, ws = 0;
    for (int i = 0; i < 4; ++i) {
        REAL sx = (i == 1 || i == 2) ? (REAL)-1 : (REAL)1, sy = i >= 2 ? (REAL)-1 : (REAL)1;
        REAL vax = (cAx + eA0x * sx) + eA1x * sy, vay = (cAy + eA0y * sx) + eA1y * sy;
        REAL da = FN(rmax)(reach - FN(box_sd)(vax, vay, cBx, cBy, caB, saB, hB0, hB1), (REAL)0);
        ax += vax * da;
        ay += vay * da;
        ws += da;
        REAL vbx = (cBx + eB0x * sx) + eB1x * sy, vby = (cBy + eB0y * sx) + eB1y * sy;
        REAL db = FN(rmax)(reach - FN(box_sd)(vbx, vby, cAx, cAy, caA, saA, hA0, hA1), (REAL)0);
        ax += vbx * db;
        ay += vby * db;
        ws += db;
    }
    if (ws > (REAL)0) {
        *x = ax / ws;
        *y = ay / ws;
    }
}

/* _agent_pair_force_torque (collisions.py:1188-1243): the pair force on a and its torque
   about a's centre (0 for a disc a) */
static void FN(pair_force_torque)(const FN(ctx_t) *C, int a, int b, const FN(prm_t) *Pa,
                                  const FN(prm_t) *Pb, const FN(agent_t) *A,
                                  const FN(agent_t) *B, REAL dd, REAL *fx, REAL *fy, REAL *tau)
{
    const REAL half = (REAL)0.5;
    *tau = 0;
    if (Pa->shape < half && Pb->shape < half) {
        FN(pair_force)(C, A->px - B->px, A->py - B->py, A->vx - B->vx, A->vy - B->vy,
                       Pa->radius + Pb->radius + C->margin, dd, fx, fy);
        return;
    }
    FN(dn) sa[BX_N], sb[BX_N], gx, gy, xx, xy;
    FN(dstate)(A, -1, sa);
    FN(dstate)(B, -1, sb);
    if (Pa->shape < half) {
        FN(d_agent_pair_force)(C, a, b, Pa, Pb, sa, sb, dd, &gx, &gy);
        *fx = gx.v;
        *fy = gy.v;
    } else if (Pb->shape < half) {
        FN(d_agent_pair_force)(C, a, b, Pa, Pb, sa, sb, dd, &gx, &gy);
        *fx = gx.v;
        *fy = gy.v;
        REAL fn = SQRT(*fx * *fx + *fy * *fy);
        if (fn > (REAL)0) {  /* at the disc's point nearest to a */
            REAL k = Pb->radius / fn;
            *tau = FN(cross2)((B->px + *fx * k) - A->px, (B->py + *fy * k) - A->py, *fx, *fy);
        }
    } else {
        if (a < b) {
            FN(d_obb_force)(C, sa[BX_PX], sa[BX_PY], sa[BX_TH], Pa->hx, Pa->hy, sa[BX_VX],
                            sa[BX_VY], sa[BX_W], sb[BX_PX], sb[BX_PY], sb[BX_TH], Pb->hx, Pb->hy,
                            sb[BX_VX], sb[BX_VY], sb[BX_W], C->margin, dd, &gx, &gy, &xx, &xy);
            *fx = gx.v;
            *fy = gy.v;
        } else {
            FN(d_obb_force)(C, sb[BX_PX], sb[BX_PY], sb[BX_TH], Pb->hx, Pb->hy, sb[BX_VX],
                            sb[BX_VY], sb[BX_W], sa[BX_PX], sa[BX_PY], sa[BX_TH], Pa->hx, Pa->hy,
                            sa[BX_VX], sa[BX_VY], sa[BX_W], C->margin, dd, &gx, &gy, &xx, &xy);
            *fx = -gx.v;
            *fy = -gy.v;
        }
        if (*fx * *fx + *fy * *fy > (REAL)0) {
            REAL x = xx.v, y = xy.v;
            FN(manifold_point)(A->px, A->py, A->th, Pa->hx, Pa->hy, B->px, B->py, B->th, Pb->hx,
                               Pb->hy, C->margin, &x, &y);
            *tau = FN(cross2)(x - A->px, y - A->py, *fx, *fy);
        }
    }
}

/* _static_forces_torque (collisions.py:1246-1340) for a box agent: obstacles (each force
   at its contact point: a circle's point nearest the box, a box's or capsule core's
   manifold point) and the walls one by one at their support vertices */
static void FN(box_static_torque)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                                  const FN(agent_t) *A, REAL dd, REAL *fx_o, REAL *fy_o,
                                  REAL *tau_o)
{
    const REAL hx = P->hx, hy = P->hy, rb = SQRT(hx * hx + hy * hy);
    REAL fx = 0, fy = 0, tau = 0;
    FN(dn) s[BX_N];
    FN(dstate)(A, -1, s);
    for (int o = 0; o < C->n_obs; ++o) {
        const REAL *sh = od + 6 * o;
        int st = C->o_type[o];
        REAL ro = C->o_rad[o], ohx = C->o_half[o * 2], ohy = C->o_half[o * 2 + 1];
        if (FN(bounds_apart)(A->px - sh[0], A->py - sh[1], rb + C->margin + FN(shape_bound)(st, ro, ohx, ohy)))
            continue;
        FN(dn) cx = FN(dk)(sh[0]), cy = FN(dk)(sh[1]), ang = FN(dk)(sh[2]);
        FN(dn) vox = FN(dk)(sh[3]), voy = FN(dk)(sh[4]), om = FN(dk)(sh[5]);
        FN(dn) gx, gy, xx = cx, xy = cy;
        if (st == 1 || st == 2) {
            FN(d_obb_force)(C, s[BX_PX], s[BX_PY], s[BX_TH], hx, hy, s[BX_VX], s[BX_VY], s[BX_W],
                            cx, cy, ang, ohx, st == 1 ? ohy : (REAL)0, vox, voy, om,
                            st == 1 ? C->margin : ro + C->margin, dd, &gx, &gy, &xx, &xy);
        } else {
            FN(dn) hxv, hyv;
            FN(d_box_force)(C, cx, cy, vox, voy, s[BX_PX], s[BX_PY], s[BX_TH], hx, hy,
                            ro + C->margin, dd, s[BX_VX], s[BX_VY], s[BX_W], &hxv, &hyv);
            gx = FN(dneg)(hxv);
            gy = FN(dneg)(hyv);
        }
        REAL fox = gx.v, foy = gy.v, x = xx.v, y = xy.v;
        if (fox * fox + foy * foy > (REAL)0) {
            if (st == 0) {
                REAL k = ro / SQRT(fox * fox + foy * foy);
                x = x + fox * k;
                y = y + foy * k;
            } else {
                FN(manifold_point)(A->px, A->py, A->th, hx, hy, sh[0], sh[1], sh[2], ohx,
                                   st == 1 ? ohy : (REAL)0, st == 1 ? C->margin : ro + C->margin,
                                   &x, &y);
            }
        }
        fx += fox;
        fy += foy;
        tau += FN(cross2)(x - A->px, y - A->py, fox, foy);
    }
    if (C->soft_walls) {
        REAL ca = COS(A->th), sa = SIN(A->th);
        REAL ex = hx * FABS(ca) + hy * FABS(sa), ey = hx * FABS(sa) + hy * FABS(ca);
        REAL sc = ca > 0 ? (REAL)1 : (ca < 0 ? (REAL)-1 : (REAL)0);
        REAL ss = sa > 0 ? (REAL)1 : (sa < 0 ? (REAL)-1 : (REAL)0);
        REAL rl_y = -sc * hx * sa + ss * hy * ca, rb_x = -ss * hx * ca + sc * hy * sa;
        REAL wx = 0, wy = 0, pen;
        pen = ex + C->margin - (A->px - C->bmin_x);
        if (pen > 0) {
            REAL fl = FN(normal_coeff)(C, pen, A->vx - A->w * rl_y, dd);
            wx += fl;
            tau += -rl_y * fl;
        }
        pen = ex + C->margin - (C->bmax_x - A->px);
        if (pen > 0) {
            REAL fr = -FN(normal_coeff)(C, pen, -(A->vx + A->w * rl_y), dd);
            wx += fr;
            tau += rl_y * fr;
        }
        pen = ey + C->margin - (A->py - C->bmin_y);
        if (pen > 0) {
            REAL fb = FN(normal_coeff)(C, pen, A->vy + A->w * rb_x, dd);
            wy += fb;
            tau += rb_x * fb;
        }
        pen = ey + C->margin - (C->bmax_y - A->py);
        if (pen > 0) {
            REAL ft = -FN(normal_coeff)(C, pen, -(A->vy - A->w * rb_x), dd);
            wy += ft;
            tau += -rb_x * ft;
        }
        fx += wx;
        fy += wy;
    }
    *fx_o = fx;
    *fy_o = fy;
    *tau_o = tau;
}

/* Torques of the wheel-contact force pass (the forces are forces_env_box's) */
static void FN(torques_env)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                            const FN(agent_t) *st, const int32_t *idx, const int32_t *cnt,
                            REAL *tq)
{
    int A = C->n_agents, K = C->max_nbr;
    for (int a = 0; a < A; ++a) {
        REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
        REAL tau = 0;
        int n = C->collisions ? cnt[a] : 0;
        for (int i = 0; i < n; ++i) {
            int b = idx[a * K + i];
            REAL fx, fy, tb;
            FN(pair_force_torque)(C, a, b, P + a, P + b, st + a, st + b, dd, &fx, &fy, &tb);
            tau += tb;
        }
        REAL ts = 0;
        if (P[a].shape > (REAL)0.5) {
            REAL fx, fy;
            FN(box_static_torque)(C, od, P + a, st + a, dd, &fx, &fy, &ts);
        }
        tq[a] = tau + ts;
    }
}

/* wheel_contact (swarp/dynamics/kernels.py:1328-1387): a diff-drive agent's step output
   (*out, unclamped) reworked: sideways force only beyond the wheels' grip, the contact
   torque turning it only beyond turn_cap; other models pass through */
static void FN(wheel_contact)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                              REAL Fx, REAL Fy, REAL torque, FN(agent_t) *out)
{
    if (P->tag != 1) return;
    REAL dt = C->sub_dt, zero = 0;
    REAL ca = COS(in->th), sa = SIN(in->th);
    REAL f_lat = -Fx * sa + Fy * ca;
    REAL slip = FN(rmax)(FABS(f_lat) - C->lat_grip * P->mass, zero);
    if (f_lat < zero) slip = -slip;
    REAL dv = (slip - f_lat) * (dt / P->mass);
    REAL cx = -sa * dv, cy = ca * dv;
    out->vx = out->vx + cx;
    out->vy = out->vy + cy;
    out->px = out->px + cx * dt;
    out->py = out->py + cy * dt;
    REAL inertia = P->mass * (P->hx * P->hx + P->hy * P->hy) / (REAL)3;
    REAL excess = FN(rmax)(FABS(torque) - C->turn_cap, zero);
    if (torque < zero) excess = -excess;
    REAL w_drive = out->w;
    if (torque * out->w < zero && FABS(torque) > C->turn_cap) w_drive = zero;
    /* a disc has no footprint inertia: the torque term is skipped when there is no
       excess (the reference's 0 * (dt / 0) = NaN), keeping the signed zero */
    REAL turn = excess != zero ? excess * (dt / inertia) : excess;
    out->th = in->th + (w_drive + turn) * dt;
}

/* ------------------------------------------------------------ the footprint clamp */

/* clamp_footprint (swarp/dynamics/kernels.py:79-99): inset of the position clamp along x
   and y; a disc by its radius, a box at heading th by its support extents. */
static inline void FN(clamp_insets)(const FN(ctx_t) *C, const FN(prm_t) *P, REAL th, REAL *ex,
                                    REAL *ey)
{
    *ex = P->radius;
    *ey = P->radius;
    if (C->clamp_bounds == 2 && P->shape > (REAL)0.5) {
        REAL ca = FABS(COS(th)), sa = FABS(SIN(th));
        *ex = P->hx * ca + P->hy * sa;
        *ey = P->hx * sa + P->hy * ca;
    }
}

/* the position clamp of a substep's output (disc clamp, or the footprint clamp of a
   world holding box agents) */
static inline void FN(clamp_position)(const FN(ctx_t) *C, const FN(prm_t) *P, REAL th,
                                      REAL *px, REAL *py)
{
    REAL ex, ey;
    FN(clamp_insets)(C, P, th, &ex, &ey);
    *px = FN(rclamp)(*px, C->bmin_x + ex, C->bmax_x - ex);
    *py = FN(rclamp)(*py, C->bmin_y + ey, C->bmax_y - ey);
}

/* Reverse of clamp_position at the unclamped output (px, py, th): rewrites the position
   adjoint and adds the heading's share (through the footprint's bounds) to *gth. */
static inline void FN(clamp_position_adj)(const FN(ctx_t) *C, const FN(prm_t) *P, REAL px,
                                          REAL py, REAL th, REAL *gpx, REAL *gpy, REAL *gth)
{
    REAL ex, ey;
    FN(clamp_insets)(C, P, th, &ex, &ey);
    REAL lox = C->bmin_x + ex, hix = C->bmax_x - ex, loy = C->bmin_y + ey, hiy = C->bmax_y - ey;
    /* clamp(x, a, b): x < a -> a, x > b -> b, else x */
    REAL aex = 0, aey = 0;
    if (px < lox) aex += *gpx;
    else if (px > hix) aex -= *gpx;
    if (py < loy) aey += *gpy;
    else if (py > hiy) aey -= *gpy;
    *gpx = FN(rclamp_gx)(px, lox, hix, *gpx);
    *gpy = FN(rclamp_gx)(py, loy, hiy, *gpy);
    if (C->clamp_bounds == 2 && P->shape > (REAL)0.5 && (aex != (REAL)0 || aey != (REAL)0)) {
        /* ex = hx |cos| + hy |sin|, ey = hx |sin| + hy |cos| */
        REAL c = COS(th), s = SIN(th);
        REAL dca = c < (REAL)0 ? s : -s;  /* d|cos th| / dth */
        REAL dsa = s < (REAL)0 ? -c : c;  /* d|sin th| / dth */
        *gth += aex * (P->hx * dca + P->hy * dsa) + aey * (P->hx * dsa + P->hy * dca);
    }
}
