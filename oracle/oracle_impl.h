/*
 * oracle_impl.h -- body of the CPU restatement, included once per precision by
 * swarp_oracle.c with REAL (float or double), FN(name) (name suffix) and the
 * math macros SQRT/COS/SIN/TAN/ATAN/TANH/FABS defined.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity checker for the HIP product
 * (swarp_amd/csrc) and the CPU baseline timed by bench.py.  Nothing in the
 * product may include, link or call it.
 *
 * Every function restates the reference algorithm from its source text, in the
 * same operation order (no FMA contraction: the build uses -ffp-contract=off),
 * so that a float32 run with no transcendental functions (holonomic agents,
 * circle obstacles, walls) is bit-identical to any other IEEE implementation of
 * the same op sequence.  Citations are relative to the reference checkout.
 *
 * The adjoint ("backward") functions are hand-derived reverse mode of the
 * forward functions below; the reference gets the same from warp-lang's code
 * generator.  Kink conventions follow warp-lang's documented builtins:
 *   max(a, b):      a > b -> gradient to a, else to b
 *   clamp(x, a, b): x < a -> a, x > b -> b, else x
 *   length(v):      zero gradient at v == 0
 * and a branch taken in the forward pass is taken again in the adjoint.
 */

typedef struct {
    REAL px, py, th, vx, vy, s, w, z, vz, qx, qy, qz, qw, bx, by, bz;
} FN(agent_t);

typedef struct {
    /* per-agent constants resolved from the [A, 22] parameter row */
    REAL radius, mass, max_speed, max_accel, max_ang_vel, max_ang_accel;
    REAL l_f, l_r, max_steer, thrust_max, arm, ixx, iyy, izz, kappa, gravity, min_speed;
    REAL shape, hx, hy; /* footprint: 0 disc, 1 box of half-extents (hx, hy) */
    REAL gain_v, gain_w; /* ControlMode.SERVO command gains */
    int tag, mode;
} FN(prm_t);

typedef struct {
    REAL k, c, margin, sub_dt, max_overlap, nbr_radius, eps2;
    REAL bmin_x, bmin_y, bmax_x, bmax_y;
    int n_envs, n_agents, act_dim, substeps, max_nbr;
    int collisions, soft_walls, needs_forces, n_obs;
    int clamp_bounds; /* 0 off, 1 disc clamp, 2 footprint clamp (a world holding boxes) */
    int boxes;        /* some agent is a box: the box-aware contact pass */
    int wheel;        /* WorldConfig.wheel_contacts (no-grad Euler 2-D only) */
    REAL lat_grip, turn_cap;
    /* obstacles: pos [E,N,2], radius [N], type [N], angle [E,N], half [N,2],
       vel [E,N,2], ang_vel [E,N] */
    const REAL *o_pos, *o_rad, *o_ang, *o_half, *o_vel, *o_om;
    const int32_t *o_type;
    /* movable compound bodies (swarp/core/config.py:70-78): kind [N] (1 = MOVABLE),
       mass [N], inertia [N], body [N] (root shape of each shape), body_off [N,2] */
    const int32_t *o_kind, *o_body;
    const REAL *o_mass, *o_inertia, *o_off;
    REAL lin_damping, ang_damping;
    int any_movable;
    int rk4;  /* Integrator.RK4 for the 2-D models */
    int grid_bins;          /* lists in uniform-grid order (0: index order) */
    REAL g_ox, g_oy, g_cs;  /* the grid's frame: origin, cell size */
    /* agent rows the body pass reads, when they differ from the agents' own (NULL): the
       reference's launch_obstacle_dynamics takes the shared table even where the agent
       side runs per-env rows (swarp/core/stepper.py:961-964) */
    const FN(prm_t) *PB;
} FN(ctx_t);

/* Per-env obstacle state, 12 reals per obstacle index o:
     [6*o .. 6*o+5]        shape o:  pos x, pos y, angle, vel x, vel y, ang_vel
     [6*N+6*o .. 6*N+6*o+5] body rooted at o: pos x, pos y, angle, vel x, vel y, ang_vel
   (the reference's obs_* and body_* arrays, swarp/core/stepper.py:418-431). */
#define OB_W 12

/* ------------------------------------------------------------ small helpers */

static inline REAL FN(rmax)(REAL a, REAL b) { return a > b ? a : b; }
static inline REAL FN(rclamp)(REAL x, REAL a, REAL b)
{
    /* clamp(x, a, b) = min(max(a, x), b) */
    REAL m = a > x ? a : x;
    return m < b ? m : b;
}
/* gradient of clamp(x, a, b) with respect to x */
static inline REAL FN(rclamp_gx)(REAL x, REAL a, REAL b, REAL g)
{
    if (x < a) return (REAL)0;
    if (x > b) return (REAL)0;
    return g;
}

/* sin and cos of a body angle: the portable evaluation (swarp_pmath.h) */
static inline void FN(psincos)(REAL xr, REAL *so, REAL *co)
{
    double s, c;
    swarp_psincos((double)xr, &s, &c);
    *so = (REAL)s;
    *co = (REAL)c;
}

/* clamp_norm (swarp/dynamics/kernels.py:68-71): v * (limit / max(length(v), limit)) */
static inline void FN(clamp_norm)(REAL x, REAL y, REAL lim, REAL *ox, REAL *oy)
{
    REAL len = SQRT(x * x + y * y);
    REAL m = FN(rmax)(len, lim);
    REAL sc = lim / m;
    *ox = x * sc;
    *oy = y * sc;
}

static inline void FN(clamp_norm_adj)(REAL x, REAL y, REAL lim, REAL gx, REAL gy,
                                      REAL *ax, REAL *ay)
{
    REAL len = SQRT(x * x + y * y);
    REAL m = FN(rmax)(len, lim);
    REAL sc = lim / m;
    REAL adj_sc = gx * x + gy * y;
    REAL rx = gx * sc, ry = gy * sc;
    if (len > lim) {
        /* sc = lim / m, d sc / d m = -lim / m^2 ; m = len */
        REAL adj_m = -adj_sc * lim / (m * m);
        if (len > (REAL)0) {
            rx += adj_m * x / len;
            ry += adj_m * y / len;
        }
    }
    *ax += rx;
    *ay += ry;
}

/* _normal_coeff (swarp/core/collisions.py:87-105) */
static inline REAL FN(normal_coeff)(const FN(ctx_t) *C, REAL ov, REAL vn, REAL dd)
{
    REAL o = ov;
    if (C->max_overlap > (REAL)0) o = C->max_overlap * TANH(ov / C->max_overlap);
    return FN(rmax)((C->k * o - C->c * vn) / dd, (REAL)0);
}

static inline void FN(normal_coeff_adj)(const FN(ctx_t) *C, REAL ov, REAL vn, REAL dd,
                                        REAL g, REAL *adj_ov, REAL *adj_vn)
{
    REAL o = ov, dodov = (REAL)1;
    if (C->max_overlap > (REAL)0) {
        REAL t = TANH(ov / C->max_overlap);
        o = C->max_overlap * t;
        dodov = (REAL)1 - t * t;
    }
    REAL x = (C->k * o - C->c * vn) / dd;
    if (x > (REAL)0) {
        REAL an = g / dd;
        *adj_ov += C->k * an * dodov;
        *adj_vn += -C->c * an;
    }
}

/* pair_force (swarp/core/collisions.py:108-143) */
static inline void FN(pair_force)(const FN(ctx_t) *C, REAL dx, REAL dy, REAL rvx, REAL rvy,
                                  REAL md, REAL dd, REAL *fx, REAL *fy)
{
    REAL dist = SQRT(FN(rmax)(dx * dx + dy * dy, C->eps2));
    REAL ov = md - dist;
    *fx = (REAL)0;
    *fy = (REAL)0;
    if (ov > (REAL)0) {
        REAL nx = dx / dist, ny = dy / dist;
        REAL coef = FN(normal_coeff)(C, ov, rvx * nx + rvy * ny, dd);
        *fx = coef * nx;
        *fy = coef * ny;
    }
}

/* reverse mode of pair_force: accumulates d/d(d) and d/d(rel_v) */
static inline void FN(pair_force_adj)(const FN(ctx_t) *C, REAL dx, REAL dy, REAL rvx, REAL rvy,
                                      REAL md, REAL dd, REAL gfx, REAL gfy,
                                      REAL *adx, REAL *ady, REAL *arvx, REAL *arvy)
{
    REAL d2 = dx * dx + dy * dy;
    REAL m = FN(rmax)(d2, C->eps2);
    REAL dist = SQRT(m);
    REAL ov = md - dist;
    if (!(ov > (REAL)0)) return;
    REAL nx = dx / dist, ny = dy / dist;
    REAL vn = rvx * nx + rvy * ny;
    REAL coef = FN(normal_coeff)(C, ov, vn, dd);
    REAL adj_coef = gfx * nx + gfy * ny;
    REAL anx = coef * gfx, any = coef * gfy;
    REAL adj_ov = 0, adj_vn = 0;
    FN(normal_coeff_adj)(C, ov, vn, dd, adj_coef, &adj_ov, &adj_vn);
    *arvx += adj_vn * nx;
    *arvy += adj_vn * ny;
    anx += adj_vn * rvx;
    any += adj_vn * rvy;
    REAL gdx = anx / dist, gdy = any / dist;
    REAL adj_dist = -(anx * nx + any * ny) / dist - adj_ov;
    if (d2 > C->eps2) {
        REAL adj_d2 = adj_dist * (REAL)0.5 / dist;
        gdx += (REAL)2 * dx * adj_d2;
        gdy += (REAL)2 * dy * adj_d2;
    }
    *adx += gdx;
    *ady += gdy;
}

/* Whether the body pass re-installs shape s (it belongs to a movable body). */
static inline int FN(shape_moves)(const FN(ctx_t) *C, int s)
{
    if (!C->any_movable) return 0;
    int r = C->o_body[s];
    return C->o_body[r] == r && C->o_kind[r] == 1;
}

/* shape_bound / bounds_apart (swarp/core/collisions.py:61-84) */
static inline REAL FN(shape_bound)(int st, REAL r, REAL hx, REAL hy)
{
    if (st == 1) return SQRT(hx * hx + hy * hy);
    if (st == 2) return hx + r;
    return r;
}
static inline int FN(bounds_apart)(REAL dx, REAL dy, REAL reach)
{
    REAL lim = reach * (REAL)1.0001 + (REAL)1.0e-6;
    return dx * dx + dy * dy > lim * lim;
}

/* box_force (swarp/core/collisions.py:174-260); returns the force */
static inline void FN(box_force)(const FN(ctx_t) *C, REAL px, REAL py, REAL vx, REAL vy,
                                 REAL cx0, REAL cy0, REAL ang, REAL hx, REAL hy, REAL reach,
                                 REAL dd, REAL vox, REAL voy, REAL om, REAL *fx, REAL *fy)
{
    REAL ca = COS(ang), sa = SIN(ang);
    REAL dx = px - cx0, dy = py - cy0;
    REAL lx = ca * dx + sa * dy;
    REAL ly = -sa * dx + ca * dy;
    REAL qx = FABS(lx) - hx, qy = FABS(ly) - hy;
    REAL cx = FN(rclamp)(lx, -hx, hx), cy = FN(rclamp)(ly, -hy, hy);
    REAL ox = lx - cx, oy = ly - cy;
    REAL od2 = ox * ox + oy * oy;
    REAL s, nlx, nly;
    if (od2 > C->eps2) {
        s = SQRT(od2);
        nlx = ox / s;
        nly = oy / s;
    } else if (qx > qy) {
        s = qx;
        nlx = lx >= (REAL)0 ? (REAL)1 : (REAL)-1;
        nly = (REAL)0;
    } else {
        s = qy;
        nlx = (REAL)0;
        nly = ly >= (REAL)0 ? (REAL)1 : (REAL)-1;
    }
    *fx = (REAL)0;
    *fy = (REAL)0;
    REAL ov = reach - s;
    if (ov > (REAL)0) {
        REAL nx = ca * nlx - sa * nly, ny = sa * nlx + ca * nly;
        REAL spx = lx - s * nlx, spy = ly - s * nly;
        REAL rx = ca * spx - sa * spy, ry = sa * spx + ca * spy;
        REAL vsx = vox + -om * ry, vsy = voy + om * rx;
        REAL rvx = vx - vsx, rvy = vy - vsy;
        REAL coef = FN(normal_coeff)(C, ov, rvx * nx + rvy * ny, dd);
        *fx = coef * nx;
        *fy = coef * ny;
    }
}

static inline void FN(box_force_adj)(const FN(ctx_t) *C, REAL px, REAL py, REAL vx, REAL vy,
                                     REAL cx0, REAL cy0, REAL ang, REAL hx, REAL hy, REAL reach,
                                     REAL dd, REAL vox, REAL voy, REAL om, REAL gfx, REAL gfy,
                                     REAL *apx, REAL *apy, REAL *avx, REAL *avy)
{
    REAL ca = COS(ang), sa = SIN(ang);
    REAL dx = px - cx0, dy = py - cy0;
    REAL lx = ca * dx + sa * dy;
    REAL ly = -sa * dx + ca * dy;
    REAL qx = FABS(lx) - hx, qy = FABS(ly) - hy;
    REAL cx = FN(rclamp)(lx, -hx, hx), cy = FN(rclamp)(ly, -hy, hy);
    REAL ox = lx - cx, oy = ly - cy;
    REAL od2 = ox * ox + oy * oy;
    REAL s, nlx, nly;
    int branch;
    if (od2 > C->eps2) {
        s = SQRT(od2);
        nlx = ox / s;
        nly = oy / s;
        branch = 0;
    } else if (qx > qy) {
        s = qx;
        nlx = lx >= (REAL)0 ? (REAL)1 : (REAL)-1;
        nly = (REAL)0;
        branch = 1;
    } else {
        s = qy;
        nlx = (REAL)0;
        nly = ly >= (REAL)0 ? (REAL)1 : (REAL)-1;
        branch = 2;
    }
    REAL ov = reach - s;
    if (!(ov > (REAL)0)) return;
    REAL nx = ca * nlx - sa * nly, ny = sa * nlx + ca * nly;
    REAL spx = lx - s * nlx, spy = ly - s * nly;
    REAL rx = ca * spx - sa * spy, ry = sa * spx + ca * spy;
    REAL vsx = vox + -om * ry, vsy = voy + om * rx;
    REAL rvx = vx - vsx, rvy = vy - vsy;
    REAL vn = rvx * nx + rvy * ny;
    REAL coef = FN(normal_coeff)(C, ov, vn, dd);
    /* f = coef * n */
    REAL adj_coef = gfx * nx + gfy * ny;
    REAL anx = coef * gfx, any = coef * gfy;
    REAL adj_ov = 0, adj_vn = 0;
    FN(normal_coeff_adj)(C, ov, vn, dd, adj_coef, &adj_ov, &adj_vn);
    /* vn = rv . n */
    REAL arvx = adj_vn * nx, arvy = adj_vn * ny;
    anx += adj_vn * rvx;
    any += adj_vn * rvy;
    /* rv = v - vs ; vs = vo + (-om*ry, om*rx) */
    *avx += arvx;
    *avy += arvy;
    REAL arx = -arvy * om;   /* d vsy / d rx = om, adj_vs = -adj_rv */
    REAL ary = arvx * om;    /* d vsx / d ry = -om */
    /* r = R sp */
    REAL aspx = ca * arx + sa * ary, aspy = -sa * arx + ca * ary;
    /* sp = l - s * nl */
    REAL alx = aspx, aly = aspy;
    REAL as = -(aspx * nlx + aspy * nly);
    REAL anlx = -s * aspx, anly = -s * aspy;
    /* n = R nl */
    anlx += ca * anx + sa * any;
    anly += -sa * anx + ca * any;
    /* ov = reach - s */
    as += -adj_ov;
    if (branch == 0) {
        /* nl = o / s ; s = sqrt(od2) */
        REAL aox = anlx / s, aoy = anly / s;
        as += -(anlx * nlx + anly * nly) / s;
        REAL aod2 = as * (REAL)0.5 / s;
        aox += (REAL)2 * ox * aod2;
        aoy += (REAL)2 * oy * aod2;
        /* o = l - clamp(l) */
        alx += aox - FN(rclamp_gx)(lx, -hx, hx, aox);
        aly += aoy - FN(rclamp_gx)(ly, -hy, hy, aoy);
    } else if (branch == 1) {
        /* s = |lx| - hx ; warp-lang adj_abs: x > 0 -> +g else -g */
        alx += lx > (REAL)0 ? as : -as;
    } else {
        aly += ly > (REAL)0 ? as : -as;
    }
    /* l = R^T d */
    REAL adx = ca * alx - sa * aly, ady = sa * alx + ca * aly;
    *apx += adx;
    *apy += ady;
}

/* closest_on_segment (swarp/core/collisions.py:156-171) */
static inline void FN(closest_on_segment)(REAL px, REAL py, REAL cx, REAL cy, REAL ang, REAL hl,
                                          REAL *ox, REAL *oy, REAL *t_out, REAL *tr_out)
{
    REAL dxu = COS(ang), dyu = SIN(ang);
    REAL tr = (px - cx) * dxu + (py - cy) * dyu;
    REAL t = FN(rclamp)(tr, -hl, hl);
    *ox = cx + t * dxu;
    *oy = cy + t * dyu;
    if (t_out) *t_out = t;
    if (tr_out) *tr_out = tr;
}

/* One obstacle's force on an agent; returns 0 if skipped by the broad phase. */
static inline void FN(obstacle_force)(const FN(ctx_t) *C, const REAL *od, int o, REAL px,
                                      REAL py, REAL vx, REAL vy, REAL ra, REAL dd, REAL *fx,
                                      REAL *fy)
{
    const REAL *sh = od + 6 * o;  /* this env's shape state: pos, angle, vel, ang_vel */
    REAL cx = sh[0], cy = sh[1];
    int st = C->o_type[o];
    REAL ro = C->o_rad[o], hx = C->o_half[o * 2], hy = C->o_half[o * 2 + 1];
    *fx = (REAL)0;
    *fy = (REAL)0;
    if (FN(bounds_apart)(px - cx, py - cy, ra + C->margin + FN(shape_bound)(st, ro, hx, hy)))
        return;
    REAL vox = sh[3], voy = sh[4];
    REAL om = sh[5];
    REAL ang = sh[2];
    if (st == 1) {
        FN(box_force)(C, px, py, vx, vy, cx, cy, ang, hx, hy, ra + C->margin, dd, vox, voy, om,
                      fx, fy);
    } else if (st == 2) {
        REAL qx, qy;
        FN(closest_on_segment)(px, py, cx, cy, ang, hx, &qx, &qy, 0, 0);
        REAL rx = qx - cx, ry = qy - cy;
        REAL vsx = vox + -om * ry, vsy = voy + om * rx;
        FN(pair_force)(C, px - qx, py - qy, vx - vsx, vy - vsy, ra + ro + C->margin, dd, fx, fy);
    } else {
        FN(pair_force)(C, px - cx, py - cy, vx - vox, vy - voy, ra + ro + C->margin, dd, fx, fy);
    }
}

/* Reverse of obstacle_force.  `god` (nullable) receives the adjoint of a MOVABLE shape's
   state; static obstacles are constants of the step. */
static void FN(obstacle_shape_adj)(const FN(ctx_t) *C, const REAL *sh, int st, REAL ro, REAL hx,
                                   REAL hy, REAL px, REAL py, REAL vx, REAL vy, REAL ra, REAL dd,
                                   REAL gfx, REAL gfy, REAL *g);
static inline void FN(obstacle_force_adj)(const FN(ctx_t) *C, const REAL *od, int o, REAL px,
                                          REAL py, REAL vx, REAL vy, REAL ra, REAL dd, REAL gfx,
                                          REAL gfy, REAL *apx, REAL *apy, REAL *avx, REAL *avy,
                                          REAL *god)
{
    const REAL *sh = od + 6 * o;
    REAL cx = sh[0], cy = sh[1];
    int st = C->o_type[o];
    REAL ro = C->o_rad[o], hx = C->o_half[o * 2], hy = C->o_half[o * 2 + 1];
    if (FN(bounds_apart)(px - cx, py - cy, ra + C->margin + FN(shape_bound)(st, ro, hx, hy)))
        return;
    REAL vox = sh[3], voy = sh[4];
    REAL om = sh[5];
    REAL ang = sh[2];
    if (st != 0 && god && FN(shape_moves)(C, o))
        FN(obstacle_shape_adj)(C, sh, st, ro, hx, hy, px, py, vx, vy, ra, dd, gfx, gfy, god + 6 * o);
    if (st == 1) {
        FN(box_force_adj)(C, px, py, vx, vy, cx, cy, ang, hx, hy, ra + C->margin, dd, vox, voy,
                          om, gfx, gfy, apx, apy, avx, avy);
    } else if (st == 2) {
        REAL qx, qy, t, tr;
        FN(closest_on_segment)(px, py, cx, cy, ang, hx, &qx, &qy, &t, &tr);
        REAL rx = qx - cx, ry = qy - cy;
        REAL vsx = vox + -om * ry, vsy = voy + om * rx;
        REAL adx = 0, ady = 0, arvx = 0, arvy = 0;
        FN(pair_force_adj)(C, px - qx, py - qy, vx - vsx, vy - vsy, ra + ro + C->margin, dd,
                           gfx, gfy, &adx, &ady, &arvx, &arvy);
        /* d = p - q ; rv = v - vs ; vs = vo + (-om*ry, om*rx) ; r = q - c */
        *apx += adx;
        *apy += ady;
        *avx += arvx;
        *avy += arvy;
        REAL aqx = -adx + (-arvy) * om;   /* through rx: vsy = voy + om*rx */
        REAL aqy = -ady + arvx * om;      /* through ry: vsx = vox - om*ry */
        /* q = c + t * u ; t = clamp(tr) ; tr = (p - c) . u */
        REAL ux = COS(ang), uy = SIN(ang);
        REAL at = aqx * ux + aqy * uy;
        REAL atr = FN(rclamp_gx)(tr, -hx, hx, at);
        *apx += atr * ux;
        *apy += atr * uy;
    } else {
        REAL adx = 0, ady = 0, arvx = 0, arvy = 0;
        FN(pair_force_adj)(C, px - cx, py - cy, vx - vox, vy - voy, ra + ro + C->margin, dd,
                           gfx, gfy, &adx, &ady, &arvx, &arvy);
        *apx += adx;
        *apy += ady;
        *avx += arvx;
        *avy += arvy;
        if (god && FN(shape_moves)(C, o)) {
            REAL *g = god + 6 * o;
            g[0] -= adx;
            g[1] -= ady;
            g[3] -= arvx;
            g[4] -= arvy;
        }
    }
}

/* _wall_forces (swarp/core/collisions.py:746-778) */
static inline void FN(wall_force)(const FN(ctx_t) *C, REAL px, REAL py, REAL vx, REAL vy,
                                  REAL ra, REAL dd, REAL *fx_o, REAL *fy_o)
{
    REAL reach = ra + C->margin;
    REAL fx = 0, fy = 0, pen;
    pen = reach - (px - C->bmin_x);
    if (pen > (REAL)0) fx += FN(normal_coeff)(C, pen, vx, dd);
    pen = reach - (C->bmax_x - px);
    if (pen > (REAL)0) fx += -FN(normal_coeff)(C, pen, -vx, dd);
    pen = reach - (py - C->bmin_y);
    if (pen > (REAL)0) fy += FN(normal_coeff)(C, pen, vy, dd);
    pen = reach - (C->bmax_y - py);
    if (pen > (REAL)0) fy += -FN(normal_coeff)(C, pen, -vy, dd);
    *fx_o = fx;
    *fy_o = fy;
}

static inline void FN(wall_force_adj)(const FN(ctx_t) *C, REAL px, REAL py, REAL vx, REAL vy,
                                      REAL ra, REAL dd, REAL gfx, REAL gfy,
                                      REAL *apx, REAL *apy, REAL *avx, REAL *avy)
{
    REAL reach = ra + C->margin, pen, aov, avn;
    pen = reach - (px - C->bmin_x);
    if (pen > (REAL)0) {
        aov = 0; avn = 0;
        FN(normal_coeff_adj)(C, pen, vx, dd, gfx, &aov, &avn);
        *apx += -aov;
        *avx += avn;
    }
    pen = reach - (C->bmax_x - px);
    if (pen > (REAL)0) {
        aov = 0; avn = 0;
        FN(normal_coeff_adj)(C, pen, -vx, dd, -gfx, &aov, &avn);
        *apx += aov;
        *avx += -avn;
    }
    pen = reach - (py - C->bmin_y);
    if (pen > (REAL)0) {
        aov = 0; avn = 0;
        FN(normal_coeff_adj)(C, pen, vy, dd, gfy, &aov, &avn);
        *apy += -aov;
        *avy += avn;
    }
    pen = reach - (C->bmax_y - py);
    if (pen > (REAL)0) {
        aov = 0; avn = 0;
        FN(normal_coeff_adj)(C, pen, -vy, dd, -gfy, &aov, &avn);
        *apy += aov;
        *avy += -avn;
    }
}

#include "oracle_boxes.h"

/* ------------------------------------------------------------------ neighbours */

/* _brute_force (swarp/core/neighbors.py:76-97) for one env */
static void FN(neighbors_env)(int A, int K, const FN(agent_t) *st, REAL radius,
                              int32_t *idx, int32_t *cnt, int32_t *tru)
{
    for (int a = 0; a < A; ++a) {
        REAL px = st[a].px, py = st[a].py;
        int32_t count = 0, total = 0;
        for (int b = 0; b < A; ++b) {
            if (b == a) continue;
            REAL dx = st[b].px - px, dy = st[b].py - py;
            if (SQRT(dx * dx + dy * dy) <= radius) {
                total += 1;
                if (count < K) idx[a * K + count++] = b;
            }
        }
        cnt[a] = count;
        if (tru) tru[a] = total;
    }
}

/* One axis of a uniform-grid cell (_compute_keys / _query_uniform, swarp/core/neighbors.py:
   188-193, 230-232): truncation toward zero of (p - o) / cs, clamped to [0, bins). */
static int FN(grid_axis)(REAL p, REAL o, REAL cs, int bins)
{
    REAL q = (p - o) / cs;
    int c = q == q ? (int)q : 0;
    return c < 0 ? 0 : (c > bins - 1 ? bins - 1 : c);
}

/* _query_uniform (swarp/core/neighbors.py:214-251) for one env with the frame (ox, oy,
   cs): the cells of the 3x3 block around the agent's cell row by row (dy outer, dx
   inner), the agents of a cell in ascending index -- the order of the stable sort of the
   (env, cell) keys (:184-211, :663-666) -- tested with |p_b - p| <= radius. */
static void FN(neighbors_env_grid)(int A, int K, const FN(agent_t) *st, REAL radius, int bins,
                                   REAL ox, REAL oy, REAL cs, int32_t *idx, int32_t *cnt,
                                   int32_t *tru)
{
    int *cx = (int *)malloc(sizeof(int) * 2 * (size_t)A), *cy = cx + A;
    for (int a = 0; a < A; ++a) {
        cx[a] = FN(grid_axis)(st[a].px, ox, cs, bins);
        cy[a] = FN(grid_axis)(st[a].py, oy, cs, bins);
    }
    for (int a = 0; a < A; ++a) {
        REAL px = st[a].px, py = st[a].py;
        int32_t count = 0, total = 0;
        for (int dy = -1; dy <= 1; ++dy) {
            int ny = cy[a] + dy;
            if (ny < 0 || ny >= bins) continue;
            for (int dx = -1; dx <= 1; ++dx) {
                int nx = cx[a] + dx;
                if (nx < 0 || nx >= bins) continue;
                for (int b = 0; b < A; ++b) {
                    if (cx[b] != nx || cy[b] != ny || b == a) continue;
                    REAL ex = st[b].px - px, ey = st[b].py - py;
                    if (SQRT(ex * ex + ey * ey) <= radius) {
                        total += 1;
                        if (count < K) idx[a * K + count++] = b;
                    }
                }
            }
        }
        cnt[a] = count;
        if (tru) tru[a] = total;
    }
    free(cx);
}

/* The lists of one env in the world's order. */
static void FN(lists_env)(const FN(ctx_t) *C, const FN(agent_t) *st, int32_t *idx, int32_t *cnt)
{
    if (C->grid_bins > 0)
        FN(neighbors_env_grid)(C->n_agents, C->max_nbr, st, C->nbr_radius, C->grid_bins, C->g_ox,
                               C->g_oy, C->g_cs, idx, cnt, NULL);
    else
        FN(neighbors_env)(C->n_agents, C->max_nbr, st, C->nbr_radius, idx, cnt, NULL);
}

/* --------------------------------------------------------------- the force pass */

/* collision_forces_kernel (swarp/core/collisions.py:818-881) for one env */
static void FN(forces_env)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                           const FN(agent_t) *st, const int32_t *idx, const int32_t *cnt, REAL *F)
{
    if (C->boxes || C->wheel) {
        FN(forces_env_box)(C, od, P, st, idx, cnt, F);
        return;
    }
    int A = C->n_agents, K = C->max_nbr;
    for (int a = 0; a < A; ++a) {
        REAL px = st[a].px, py = st[a].py, vx = st[a].vx, vy = st[a].vy;
        REAL ra = P[a].radius;
        REAL fx = 0, fy = 0;
        REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
        int n = C->collisions ? cnt[a] : 0;
        for (int i = 0; i < n; ++i) {
            int b = idx[a * K + i];
            REAL gx, gy;
            FN(pair_force)(C, px - st[b].px, py - st[b].py, vx - st[b].vx, vy - st[b].vy,
                           ra + P[b].radius + C->margin, dd, &gx, &gy);
            fx += gx;
            fy += gy;
        }
        /* _static_forces: obstacles in index order, then the walls */
        REAL sx = 0, sy = 0;
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
        F[a * 2] = fx + sx;
        F[a * 2 + 1] = fy + sy;
    }
}

static void FN(forces_env_adj)(const FN(ctx_t) *C, const REAL *od, const FN(prm_t) *P,
                               const FN(agent_t) *st, const int32_t *idx, const int32_t *cnt,
                               const REAL *aF, FN(agent_t) *adj, REAL *god)
{
    if (C->boxes) {
        FN(forces_env_box_adj)(C, od, P, st, idx, cnt, aF, adj);
        return;
    }
    int A = C->n_agents, K = C->max_nbr;
    for (int a = 0; a < A; ++a) {
        REAL gfx = aF[a * 2], gfy = aF[a * 2 + 1];
        if (gfx == (REAL)0 && gfy == (REAL)0) continue;
        REAL px = st[a].px, py = st[a].py, vx = st[a].vx, vy = st[a].vy;
        REAL ra = P[a].radius;
        REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
        int n = C->collisions ? cnt[a] : 0;
        for (int i = 0; i < n; ++i) {
            int b = idx[a * K + i];
            REAL adx = 0, ady = 0, arvx = 0, arvy = 0;
            FN(pair_force_adj)(C, px - st[b].px, py - st[b].py, vx - st[b].vx, vy - st[b].vy,
                               ra + P[b].radius + C->margin, dd, gfx, gfy,
                               &adx, &ady, &arvx, &arvy);
            adj[a].px += adx;
            adj[a].py += ady;
            adj[a].vx += arvx;
            adj[a].vy += arvy;
            adj[b].px -= adx;
            adj[b].py -= ady;
            adj[b].vx -= arvx;
            adj[b].vy -= arvy;
        }
        for (int o = 0; o < C->n_obs; ++o)
            FN(obstacle_force_adj)(C, od, o, px, py, vx, vy, ra, dd, gfx, gfy,
                                   &adj[a].px, &adj[a].py, &adj[a].vx, &adj[a].vy, god);
        if (C->soft_walls)
            FN(wall_force_adj)(C, px, py, vx, vy, ra, dd, gfx, gfy,
                               &adj[a].px, &adj[a].py, &adj[a].vx, &adj[a].vy);
    }
}

/* ---------------------------------------------------------------- integration */

/* ------------------------------------------------------------------------- RK4 */

/* The 16 agent fields a - b * h, componentwise: o = x + k * h */
static void FN(ag_axpy)(const FN(agent_t) *x, const FN(agent_t) *k, REAL h, FN(agent_t) *o)
{
    o->px = x->px + k->px * h; o->py = x->py + k->py * h; o->th = x->th + k->th * h;
    o->vx = x->vx + k->vx * h; o->vy = x->vy + k->vy * h;
    o->s = x->s + k->s * h; o->w = x->w + k->w * h;
    o->z = x->z + k->z * h; o->vz = x->vz + k->vz * h;
    o->qx = x->qx + k->qx * h; o->qy = x->qy + k->qy * h;
    o->qz = x->qz + k->qz * h; o->qw = x->qw + k->qw * h;
    o->bx = x->bx + k->bx * h; o->by = x->by + k->by * h; o->bz = x->bz + k->bz * h;
}

/* _deriv (swarp/dynamics/kernels.py:416-517): the state derivative with the actions held
   constant.  Holonomic integrates (pos, vel), diff-drive (pos, theta, speed, ang_vel),
   the bicycle (pos, theta, speed), the drone (pos, vel, z, vz, attitude, body_rates,
   with _drone_rates :129-163 and _quat_deriv :117-126); every other field has rate 0. */
static void FN(rk_deriv)(const FN(prm_t) *P, const FN(agent_t) *x, const REAL *a,
                         FN(agent_t) *k)
{
    memset(k, 0, sizeof *k);
    if (P->tag == 0) {
        k->px = x->vx;
        k->py = x->vy;
        if (P->mode != 0) FN(clamp_norm)(a[0], a[1], P->max_accel, &k->vx, &k->vy);
    } else if (P->tag == 1) {
        k->px = x->s * COS(x->th);
        k->py = x->s * SIN(x->th);
        k->th = x->w;
        if (P->mode != 0) {
            k->s = FN(rclamp)(a[0], -P->max_accel, P->max_accel);
            k->w = FN(rclamp)(a[1], -P->max_ang_accel, P->max_ang_accel);
        }
    } else if (P->tag == 2) {
        REAL wb = P->l_f + P->l_r;
        REAL del = FN(rclamp)(a[1], -P->max_steer, P->max_steer);
        REAL beta = ATAN(TAN(del) * P->l_r / wb);
        k->px = x->s * COS(x->th + beta);
        k->py = x->s * SIN(x->th + beta);
        k->th = x->s / wb * COS(beta) * TAN(del);
        k->s = FN(rclamp)(a[0], -P->max_accel, P->max_accel);
    } else if (P->tag == 3) {
        REAL zero = 0, half = (REAL)0.5;
        REAL f0 = FN(rclamp)(a[0], zero, P->thrust_max), f1 = FN(rclamp)(a[1], zero, P->thrust_max);
        REAL f2 = FN(rclamp)(a[2], zero, P->thrust_max), f3 = FN(rclamp)(a[3], zero, P->thrust_max);
        REAL thr = f0 + f1 + f2 + f3;
        REAL qx = x->qx, qy = x->qy, qz = x->qz, qw = x->qw;
        REAL vx3 = 0, vy3 = 0, vz3 = thr;
        REAL c1x = qy * vz3 - qz * vy3, c1y = qz * vx3 - qx * vz3, c1z = qx * vy3 - qy * vx3;
        REAL tx = (REAL)2 * c1x, ty = (REAL)2 * c1y, tz = (REAL)2 * c1z;
        REAL c2x = qy * tz - qz * ty, c2y = qz * tx - qx * tz, c2z = qx * ty - qy * tx;
        REAL fwx = vx3 + qw * tx + c2x, fwy = vy3 + qw * ty + c2y, fwz = vz3 + qw * tz + c2z;
        REAL bx = x->bx, by = x->by, bz = x->bz;
        k->px = x->vx;
        k->py = x->vy;
        k->vx = fwx / P->mass - zero;
        k->vy = fwy / P->mass - zero;
        k->vz = fwz / P->mass - P->gravity;
        k->z = x->vz;
        k->bx = (P->arm * (f1 - f3) - (P->izz - P->iyy) * by * bz) / P->ixx;
        k->by = (P->arm * (f2 - f0) - (P->ixx - P->izz) * bz * bx) / P->iyy;
        k->bz = (P->kappa * (f0 - f1 + f2 - f3) - (P->iyy - P->ixx) * bx * by) / P->izz;
        k->qx = half * (qw * bx + qy * bz - qz * by);
        k->qy = half * (qw * by - qx * bz + qz * bx);
        k->qz = half * (qw * bz + qx * by - qy * bx);
        k->qw = half * (-qx * bx - qy * by - qz * bz);
    }
}

/* Reverse of rk_deriv: gk = adjoint of k; accumulates into gx and ga[0..3]. */
static void FN(rk_deriv_adj)(const FN(prm_t) *P, const FN(agent_t) *x, const REAL *a,
                             const FN(agent_t) *gk, FN(agent_t) *gx, REAL *ga)
{
    if (P->tag == 0) {
        gx->vx += gk->px;
        gx->vy += gk->py;
        if (P->mode != 0) FN(clamp_norm_adj)(a[0], a[1], P->max_accel, gk->vx, gk->vy, &ga[0], &ga[1]);
    } else if (P->tag == 1) {
        REAL c = COS(x->th), sn = SIN(x->th);
        gx->s += gk->px * c + gk->py * sn;
        gx->th += -gk->px * x->s * sn + gk->py * x->s * c;
        gx->w += gk->th;
        if (P->mode != 0) {
            ga[0] += FN(rclamp_gx)(a[0], -P->max_accel, P->max_accel, gk->s);
            ga[1] += FN(rclamp_gx)(a[1], -P->max_ang_accel, P->max_ang_accel, gk->w);
        }
    } else if (P->tag == 2) {
        REAL wb = P->l_f + P->l_r;
        REAL del = FN(rclamp)(a[1], -P->max_steer, P->max_steer);
        REAL td = TAN(del);
        REAL u = td * P->l_r / wb;
        REAL beta = ATAN(u);
        REAL cb = COS(beta), sb = SIN(beta);
        REAL c = COS(x->th + beta), sn = SIN(x->th + beta);
        gx->s += gk->px * c + gk->py * sn + gk->th * (cb * td / wb);
        REAL gang = -gk->px * x->s * sn + gk->py * x->s * c;   /* d / d(th + beta) */
        gx->th += gang;
        REAL gbeta = gang + gk->th * (x->s / wb * (-sb) * td);
        REAL gdel = gk->th * (x->s / wb * cb * ((REAL)1 + td * td))
                    + gbeta / ((REAL)1 + u * u) * ((REAL)1 + td * td) * P->l_r / wb;
        ga[1] += FN(rclamp_gx)(a[1], -P->max_steer, P->max_steer, gdel);
        ga[0] += FN(rclamp_gx)(a[0], -P->max_accel, P->max_accel, gk->s);
    } else if (P->tag == 3) {
        REAL zero = 0, half = (REAL)0.5;
        REAL f0 = FN(rclamp)(a[0], zero, P->thrust_max), f1 = FN(rclamp)(a[1], zero, P->thrust_max);
        REAL f2 = FN(rclamp)(a[2], zero, P->thrust_max), f3 = FN(rclamp)(a[3], zero, P->thrust_max);
        REAL thr = f0 + f1 + f2 + f3;
        REAL qx = x->qx, qy = x->qy, qz = x->qz, qw = x->qw;
        REAL bx = x->bx, by = x->by, bz = x->bz;
        REAL vx3 = 0, vy3 = 0, vz3 = thr;
        REAL tx = (REAL)2 * (qy * vz3 - qz * vy3), ty = (REAL)2 * (qz * vx3 - qx * vz3);
        REAL tz = (REAL)2 * (qx * vy3 - qy * vx3);
        gx->vx += gk->px;
        gx->vy += gk->py;
        gx->vz += gk->z;
        /* fw = v3 + qw t + u x t ; acc = fw / m */
        REAL gfx = gk->vx / P->mass, gfy = gk->vy / P->mass, gfz = gk->vz / P->mass;
        REAL gqx = 0, gqy = 0, gqz = 0, gqw = 0;
        gqw += gfx * tx + gfy * ty + gfz * tz;
        REAL gtx = qw * gfx + (gfy * qz - gfz * qy);
        REAL gty = qw * gfy + (gfz * qx - gfx * qz);
        REAL gtz = qw * gfz + (gfx * qy - gfy * qx);
        gqx += ty * gfz - tz * gfy;
        gqy += tz * gfx - tx * gfz;
        gqz += tx * gfy - ty * gfx;
        /* t = 2 (u x v3) */
        REAL g1x = (REAL)2 * gtx, g1y = (REAL)2 * gty, g1z = (REAL)2 * gtz;
        gqx += vy3 * g1z - vz3 * g1y;
        gqy += vz3 * g1x - vx3 * g1z;
        gqz += vx3 * g1y - vy3 * g1x;
        REAL gthr = gfz + (g1x * qy - g1y * qx);
        /* body-rate derivative (Euler's equation) */
        REAL gax = gk->bx / P->ixx, gay = gk->by / P->iyy, gaz = gk->bz / P->izz;
        REAL gbx = 0, gby = 0, gbz = 0;
        gby -= (P->izz - P->iyy) * bz * gax;
        gbz -= (P->izz - P->iyy) * by * gax;
        gbz -= (P->ixx - P->izz) * bx * gay;
        gbx -= (P->ixx - P->izz) * bz * gay;
        gbx -= (P->iyy - P->ixx) * by * gaz;
        gby -= (P->iyy - P->ixx) * bx * gaz;
        REAL gf0 = gthr - P->arm * gay + P->kappa * gaz;
        REAL gf1 = gthr + P->arm * gax - P->kappa * gaz;
        REAL gf2 = gthr + P->arm * gay + P->kappa * gaz;
        REAL gf3 = gthr - P->arm * gax - P->kappa * gaz;
        /* quaternion derivative 0.5 q (x) (b, 0) */
        REAL Dx = half * gk->qx, Dy = half * gk->qy, Dz = half * gk->qz, Dw = half * gk->qw;
        gqw += Dx * bx + Dy * by + Dz * bz;
        gqx += -Dy * bz + Dz * by - Dw * bx;
        gqy += Dx * bz - Dz * bx - Dw * by;
        gqz += -Dx * by + Dy * bx - Dw * bz;
        gbx += Dx * qw + Dy * qz - Dz * qy - Dw * qx;
        gby += -Dx * qz + Dy * qw + Dz * qx - Dw * qy;
        gbz += Dx * qy - Dy * qx + Dz * qw - Dw * qz;
        gx->qx += gqx; gx->qy += gqy; gx->qz += gqz; gx->qw += gqw;
        gx->bx += gbx; gx->by += gby; gx->bz += gbz;
        ga[0] += FN(rclamp_gx)(a[0], zero, P->thrust_max, gf0);
        ga[1] += FN(rclamp_gx)(a[1], zero, P->thrust_max, gf1);
        ga[2] += FN(rclamp_gx)(a[2], zero, P->thrust_max, gf2);
        ga[3] += FN(rclamp_gx)(a[3], zero, P->thrust_max, gf3);
    }
}

/* The RK4 stage states (x1 = the start), their derivatives and the combine
   x + (k1 + 2 k2 + 2 k3 + k4) dt / 6 (swarp/dynamics/kernels.py:584-738). */
typedef struct {
    FN(agent_t) x1, x2, x3, x4, k1, k2, k3, k4, xi;
} FN(rk_t);

static void FN(rk_stages)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                          const REAL *a, FN(rk_t) *R)
{
    REAL dt = C->sub_dt, half = (REAL)0.5, two = (REAL)2;
    REAL dt2 = dt * half, sixth = dt / (REAL)6;
    FN(agent_t) x = *in;
    /* velocity control sets the velocity-level state from the command (:588-595) */
    if (P->mode == 0) {
        if (P->tag == 0) {
            FN(clamp_norm)(a[0], a[1], P->max_speed, &x.vx, &x.vy);
        } else if (P->tag == 1) {
            x.s = FN(rclamp)(a[0], -P->max_speed, P->max_speed);
            x.w = FN(rclamp)(a[1], -P->max_ang_vel, P->max_ang_vel);
        }
    }
    R->x1 = x;
    FN(rk_deriv)(P, &R->x1, a, &R->k1);
    FN(ag_axpy)(&x, &R->k1, dt2, &R->x2);
    FN(rk_deriv)(P, &R->x2, a, &R->k2);
    FN(ag_axpy)(&x, &R->k2, dt2, &R->x3);
    FN(rk_deriv)(P, &R->x3, a, &R->k3);
    FN(ag_axpy)(&x, &R->k3, dt, &R->x4);
    FN(rk_deriv)(P, &R->x4, a, &R->k4);
#define RK_COMB(f) R->xi.f = x.f + (R->k1.f + R->k2.f * two + R->k3.f * two + R->k4.f) * sixth
    RK_COMB(px); RK_COMB(py); RK_COMB(th); RK_COMB(vx); RK_COMB(vy); RK_COMB(s); RK_COMB(w);
    RK_COMB(z); RK_COMB(vz); RK_COMB(qx); RK_COMB(qy); RK_COMB(qz); RK_COMB(qw);
    RK_COMB(bx); RK_COMB(by); RK_COMB(bz);
#undef RK_COMB
}

/* _integrate_rk4 (swarp/dynamics/kernels.py:520-793): limits on the combined result,
   the contact force as dv = F * (dt / m) after the combine, the attitude renormalised. */
static void FN(rk4_agent)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                          const REAL *a, REAL Fx, REAL Fy, FN(agent_t) *out)
{
    REAL dt = C->sub_dt;
    FN(rk_t) R;
    FN(rk_stages)(C, P, in, a, &R);
    REAL dfx = Fx * (dt / P->mass), dfy = Fy * (dt / P->mass);
    *out = *in;
    REAL pnx = R.xi.px + dfx * dt, pny = R.xi.py + dfy * dt;
    if (P->tag == 0) {
        REAL vx, vy;
        FN(clamp_norm)(R.xi.vx, R.xi.vy, P->max_speed, &vx, &vy);
        vx = vx + dfx;
        vy = vy + dfy;
        out->vx = vx; out->vy = vy;
        out->s = SQRT(vx * vx + vy * vy);
        out->w = 0;
    } else if (P->tag == 1) {
        REAL so = FN(rclamp)(R.xi.s, -P->max_speed, P->max_speed);
        REAL th = R.xi.th;
        out->th = th;
        out->vx = so * COS(th) + dfx;
        out->vy = so * SIN(th) + dfy;
        out->s = so;
        out->w = FN(rclamp)(R.xi.w, -P->max_ang_vel, P->max_ang_vel);
    } else if (P->tag == 2) {
        REAL so = FN(rclamp)(R.xi.s, P->min_speed, P->max_speed);
        REAL th = R.xi.th;
        REAL del = FN(rclamp)(a[1], -P->max_steer, P->max_steer);
        REAL wb = P->l_f + P->l_r;
        REAL beta = ATAN(TAN(del) * P->l_r / wb);
        out->w = so / wb * COS(beta) * TAN(del);
        out->th = th;
        out->vx = so * COS(th + beta) + dfx;
        out->vy = so * SIN(th + beta) + dfy;
        out->s = so;
    } else if (P->tag == 3) {
        out->vx = R.xi.vx + dfx;
        out->vy = R.xi.vy + dfy;
        out->z = R.xi.z;
        out->vz = R.xi.vz;
        REAL l = SQRT(R.xi.qx * R.xi.qx + R.xi.qy * R.xi.qy + R.xi.qz * R.xi.qz + R.xi.qw * R.xi.qw);
        if (l > (REAL)0) {
            out->qx = R.xi.qx / l; out->qy = R.xi.qy / l; out->qz = R.xi.qz / l; out->qw = R.xi.qw / l;
        } else {
            out->qx = 0; out->qy = 0; out->qz = 0; out->qw = 1;
        }
        out->bx = R.xi.bx; out->by = R.xi.by; out->bz = R.xi.bz;
    } else {
        return; /* unknown tag: the state passes through */
    }
    if (C->clamp_bounds) FN(clamp_position)(C, P, out->th, &pnx, &pny);
    out->px = pnx;
    out->py = pny;
}

/* Reverse of rk4_agent: g = adjoint of *out; accumulates into gin, gact[0..3], gF. */
static void FN(rk4_agent_adj)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                              const REAL *a, REAL Fx, REAL Fy, const FN(agent_t) *g,
                              FN(agent_t) *gin, REAL *gact, REAL *gFx, REAL *gFy)
{
    REAL dt = C->sub_dt, half = (REAL)0.5, two = (REAL)2;
    REAL dt2 = dt * half, sixth = dt / (REAL)6;
    if (P->tag > 3) {
        FN(ag_axpy)(gin, g, (REAL)1, gin);
        return;
    }
    FN(rk_t) R;
    FN(rk_stages)(C, P, in, a, &R);
    REAL dfx = Fx * (dt / P->mass), dfy = Fy * (dt / P->mass);
    REAL gpx = g->px, gpy = g->py; /* the clamp is reversed by integrate_agent_adj */
    FN(agent_t) gxi;
    memset(&gxi, 0, sizeof gxi);
    gxi.px = gpx;
    gxi.py = gpy;
    REAL gdfx = gpx * dt + g->vx, gdfy = gpy * dt + g->vy;
    if (P->tag == 0) {
        REAL vx, vy;
        FN(clamp_norm)(R.xi.vx, R.xi.vy, P->max_speed, &vx, &vy);
        vx = vx + dfx;
        vy = vy + dfy;
        REAL gvx = g->vx, gvy = g->vy;
        REAL sp = SQRT(vx * vx + vy * vy);
        if (sp > (REAL)0) {
            gvx += g->s * vx / sp;
            gvy += g->s * vy / sp;
            gdfx += g->s * vx / sp;
            gdfy += g->s * vy / sp;
        }
        FN(clamp_norm_adj)(R.xi.vx, R.xi.vy, P->max_speed, gvx, gvy, &gxi.vx, &gxi.vy);
        gin->th += g->th;
    } else if (P->tag == 1) {
        REAL so = FN(rclamp)(R.xi.s, -P->max_speed, P->max_speed);
        REAL th = R.xi.th, c = COS(th), sn = SIN(th);
        REAL gso = g->s + g->vx * c + g->vy * sn;
        gxi.th = g->th - g->vx * so * sn + g->vy * so * c;
        gxi.s = FN(rclamp_gx)(R.xi.s, -P->max_speed, P->max_speed, gso);
        gxi.w = FN(rclamp_gx)(R.xi.w, -P->max_ang_vel, P->max_ang_vel, g->w);
    } else if (P->tag == 2) {
        REAL so = FN(rclamp)(R.xi.s, P->min_speed, P->max_speed);
        REAL th = R.xi.th;
        REAL del = FN(rclamp)(a[1], -P->max_steer, P->max_steer);
        REAL wb = P->l_f + P->l_r;
        REAL td = TAN(del), u = td * P->l_r / wb;
        REAL beta = ATAN(u), cb = COS(beta), sb = SIN(beta);
        REAL c = COS(th + beta), sn = SIN(th + beta);
        REAL gso = g->s + g->w * (cb * td / wb) + g->vx * c + g->vy * sn;
        REAL gang = -g->vx * so * sn + g->vy * so * c;
        gxi.th = g->th + gang;
        REAL gbeta = gang + g->w * (so / wb * (-sb) * td);
        REAL gdel = g->w * (so / wb * cb * ((REAL)1 + td * td))
                    + gbeta / ((REAL)1 + u * u) * ((REAL)1 + td * td) * P->l_r / wb;
        gact[1] += FN(rclamp_gx)(a[1], -P->max_steer, P->max_steer, gdel);
        gxi.s = FN(rclamp_gx)(R.xi.s, P->min_speed, P->max_speed, gso);
    } else {
        gxi.vx = g->vx;
        gxi.vy = g->vy;
        gxi.z = g->z;
        gxi.vz = g->vz;
        gxi.bx = g->bx; gxi.by = g->by; gxi.bz = g->bz;
        REAL l = SQRT(R.xi.qx * R.xi.qx + R.xi.qy * R.xi.qy + R.xi.qz * R.xi.qz + R.xi.qw * R.xi.qw);
        if (l > (REAL)0) {
            REAL nx = R.xi.qx / l, ny = R.xi.qy / l, nz = R.xi.qz / l, nw = R.xi.qw / l;
            REAL dq = g->qx * nx + g->qy * ny + g->qz * nz + g->qw * nw;
            gxi.qx = (g->qx - nx * dq) / l;
            gxi.qy = (g->qy - ny * dq) / l;
            gxi.qz = (g->qz - nz * dq) / l;
            gxi.qw = (g->qw - nw * dq) / l;
        }
        gin->th += g->th;
        gin->s += g->s;
        gin->w += g->w;
    }
    *gFx += gdfx * (dt / P->mass);
    *gFy += gdfy * (dt / P->mass);
    /* the combine and the stages, in reverse */
    FN(agent_t) gx = gxi, gk1, gk2, gk3, gk4, gs;
    memset(&gk1, 0, sizeof gk1);
    FN(ag_axpy)(&gk1, &gxi, sixth, &gk1);
    memset(&gk2, 0, sizeof gk2);
    FN(ag_axpy)(&gk2, &gxi, two * sixth, &gk2);
    gk3 = gk2;
    gk4 = gk1;
    memset(&gs, 0, sizeof gs);
    FN(rk_deriv_adj)(P, &R.x4, a, &gk4, &gs, gact);
    FN(ag_axpy)(&gx, &gs, (REAL)1, &gx);
    FN(ag_axpy)(&gk3, &gs, dt, &gk3);
    memset(&gs, 0, sizeof gs);
    FN(rk_deriv_adj)(P, &R.x3, a, &gk3, &gs, gact);
    FN(ag_axpy)(&gx, &gs, (REAL)1, &gx);
    FN(ag_axpy)(&gk2, &gs, dt2, &gk2);
    memset(&gs, 0, sizeof gs);
    FN(rk_deriv_adj)(P, &R.x2, a, &gk2, &gs, gact);
    FN(ag_axpy)(&gx, &gs, (REAL)1, &gx);
    FN(ag_axpy)(&gk1, &gs, dt2, &gk1);
    memset(&gs, 0, sizeof gs);
    FN(rk_deriv_adj)(P, &R.x1, a, &gk1, &gs, gact);
    FN(ag_axpy)(&gx, &gs, (REAL)1, &gx);
    /* velocity control: the commanded velocity-level state replaces the input's */
    if (P->mode == 0 && P->tag == 0) {
        FN(clamp_norm_adj)(a[0], a[1], P->max_speed, gx.vx, gx.vy, &gact[0], &gact[1]);
        gx.vx = gx.vy = 0;
    } else if (P->mode == 0 && P->tag == 1) {
        gact[0] += FN(rclamp_gx)(a[0], -P->max_speed, P->max_speed, gx.s);
        gact[1] += FN(rclamp_gx)(a[1], -P->max_ang_vel, P->max_ang_vel, gx.w);
        gx.s = gx.w = 0;
    }
    /* fields no model integrates pass their adjoint through */
    if (P->tag != 3) {
        gx.z += g->z; gx.vz += g->vz;
        gx.qx += g->qx; gx.qy += g->qy; gx.qz += g->qz; gx.qw += g->qw;
        gx.bx += g->bx; gx.by += g->by; gx.bz += g->bz;
    }
    FN(ag_axpy)(gin, &gx, (REAL)1, gin);
}

/* _integrate_agent + _step_2d (swarp/dynamics/kernels.py:194-413), Euler */
/* servo_command (swarp/dynamics/kernels.py:165-191): a SERVO agent's command as the
   VELOCITY command it amounts to this substep (the integrate kernels' :849-863) */
static void FN(servo_command)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                              const REAL *act, REAL *as)
{
    REAL dt = C->sub_dt;
    REAL tv = FN(rclamp)(act[0], -P->max_speed, P->max_speed) * P->gain_v;
    REAL tw = FN(rclamp)(act[1], -P->max_ang_vel, P->max_ang_vel) * P->gain_w;
    REAL dv = P->max_accel * dt, dw = P->max_ang_accel * dt;
    as[0] = in->s + FN(rclamp)(tv - in->s, -dv, dv);
    as[1] = in->w + FN(rclamp)(tw - in->w, -dw, dw);
    for (int k = 2; k < 4; ++k) as[k] = C->act_dim > k ? act[k] : (REAL)0;
}

static void FN(integrate_agent)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                                const REAL *act, REAL Fx, REAL Fy, FN(agent_t) *out)
{
    if (P->mode == 2) {
        FN(prm_t) Pv = *P;
        Pv.mode = 0;
        REAL as[4];
        FN(servo_command)(C, P, in, act, as);
        FN(integrate_agent)(C, &Pv, in, as, Fx, Fy, out);
        return;
    }
    REAL dt = C->sub_dt;
    REAL a0 = act[0], a1 = C->act_dim > 1 ? act[1] : (REAL)0;
    REAL a2 = C->act_dim > 2 ? act[2] : (REAL)0;
    REAL a3 = C->act_dim > 3 ? act[3] : (REAL)0;
    if (C->rk4) {
        REAL a[4] = {a0, a1, a2, a3};
        FN(rk4_agent)(C, P, in, a, Fx, Fy, out);
        return;
    }
    *out = *in; /* drone fields (and unknown tags) pass through */
    REAL pnx, pny;
    if (P->tag == 3) {
        /* DRONE branch (:349-369) with _drone_rates (:129-163) */
        REAL dtm = dt / P->mass;
        REAL dvx = Fx * dtm, dvy = Fy * dtm;
        REAL zero = 0;
        REAL f0 = FN(rclamp)(a0, zero, P->thrust_max), f1 = FN(rclamp)(a1, zero, P->thrust_max);
        REAL f2 = FN(rclamp)(a2, zero, P->thrust_max), f3 = FN(rclamp)(a3, zero, P->thrust_max);
        REAL thrust = f0 + f1 + f2 + f3;
        REAL qx = in->qx, qy = in->qy, qz = in->qz, qw = in->qw;
        REAL vx3 = 0, vy3 = 0, vz3 = thrust;
        /* t = 2 * cross(u, v) */
        REAL c1x = qy * vz3 - qz * vy3, c1y = qz * vx3 - qx * vz3, c1z = qx * vy3 - qy * vx3;
        REAL tx_ = (REAL)2 * c1x, ty_ = (REAL)2 * c1y, tz_ = (REAL)2 * c1z;
        REAL c2x = qy * tz_ - qz * ty_, c2y = qz * tx_ - qx * tz_, c2z = qx * ty_ - qy * tx_;
        REAL fwx = vx3 + qw * tx_ + c2x, fwy = vy3 + qw * ty_ + c2y, fwz = vz3 + qw * tz_ + c2z;
        REAL accx = fwx / P->mass - zero, accy = fwy / P->mass - zero;
        REAL accz = fwz / P->mass - P->gravity;
        REAL tqx = P->arm * (f1 - f3), tqy = P->arm * (f2 - f0);
        REAL tqz = P->kappa * (f0 - f1 + f2 - f3);
        REAL bx = in->bx, by = in->by, bz = in->bz;
        REAL angx = (tqx - (P->izz - P->iyy) * by * bz) / P->ixx;
        REAL angy = (tqy - (P->ixx - P->izz) * bz * bx) / P->iyy;
        REAL angz = (tqz - (P->iyy - P->ixx) * bx * by) / P->izz;
        REAL nbx = bx + angx * dt, nby = by + angy * dt, nbz = bz + angz * dt;
        REAL nvz = in->vz + accz * dt;
        REAL vxy_x = in->vx + accx * dt + dvx, vxy_y = in->vy + accy * dt + dvy;
        /* _quat_deriv(q, br_new) (:117-126) */
        REAL half = (REAL)0.5;
        REAL dqx = half * (qw * nbx + qy * nbz - qz * nby);
        REAL dqy = half * (qw * nby - qx * nbz + qz * nbx);
        REAL dqz = half * (qw * nbz + qx * nby - qy * nbx);
        REAL dqw = half * (-qx * nbx - qy * nby - qz * nbz);
        REAL ux = qx + dqx * dt, uy = qy + dqy * dt, uz = qz + dqz * dt, uw = qw + dqw * dt;
        REAL l = SQRT(ux * ux + uy * uy + uz * uz + uw * uw);
        if (l > (REAL)0) {
            out->qx = ux / l; out->qy = uy / l; out->qz = uz / l; out->qw = uw / l;
        } else {
            out->qx = 0; out->qy = 0; out->qz = 0; out->qw = 1;
        }
        pnx = in->px + vxy_x * dt;
        pny = in->py + vxy_y * dt;
        out->z = in->z + nvz * dt;
        out->vz = nvz;
        out->bx = nbx; out->by = nby; out->bz = nbz;
        out->vx = vxy_x; out->vy = vxy_y;
    } else {
        REAL dtm = dt / P->mass;
        REAL dvx = Fx * dtm, dvy = Fy * dtm;
        REAL px = in->px, py = in->py, th = in->th;
        if (P->tag == 0) {
            REAL vnx, vny;
            if (P->mode == 0) {
                FN(clamp_norm)(a0, a1, P->max_speed, &vnx, &vny);
            } else {
                REAL accx, accy;
                FN(clamp_norm)(a0, a1, P->max_accel, &accx, &accy);
                FN(clamp_norm)(in->vx + accx * dt, in->vy + accy * dt, P->max_speed, &vnx, &vny);
            }
            vnx = vnx + dvx;
            vny = vny + dvy;
            pnx = px + vnx * dt;
            pny = py + vny * dt;
            out->th = th;
            out->vx = vnx; out->vy = vny;
            out->s = SQRT(vnx * vnx + vny * vny);
            out->w = 0;
        } else if (P->tag == 1) {
            REAL sn, wn;
            if (P->mode == 0) {
                sn = FN(rclamp)(a0, -P->max_speed, P->max_speed);
                wn = FN(rclamp)(a1, -P->max_ang_vel, P->max_ang_vel);
            } else {
                REAL acc = FN(rclamp)(a0, -P->max_accel, P->max_accel);
                REAL alp = FN(rclamp)(a1, -P->max_ang_accel, P->max_ang_accel);
                sn = FN(rclamp)(in->s + acc * dt, -P->max_speed, P->max_speed);
                wn = FN(rclamp)(in->w + alp * dt, -P->max_ang_vel, P->max_ang_vel);
            }
            REAL vtx = sn * COS(th) + dvx, vty = sn * SIN(th) + dvy;
            pnx = px + vtx * dt;
            pny = py + vty * dt;
            out->th = th + wn * dt;
            out->vx = vtx; out->vy = vty;
            out->s = sn;
            out->w = wn;
        } else if (P->tag == 2) {
            REAL acc = FN(rclamp)(a0, -P->max_accel, P->max_accel);
            REAL del = FN(rclamp)(a1, -P->max_steer, P->max_steer);
            REAL sn = FN(rclamp)(in->s + acc * dt, P->min_speed, P->max_speed);
            REAL wb = P->l_f + P->l_r;
            REAL beta = ATAN(TAN(del) * P->l_r / wb);
            REAL vtx = sn * COS(th + beta) + dvx, vty = sn * SIN(th + beta) + dvy;
            REAL wn = sn / wb * COS(beta) * TAN(del);
            pnx = px + vtx * dt;
            pny = py + vty * dt;
            out->th = th + wn * dt;
            out->vx = vtx; out->vy = vty;
            out->s = sn;
            out->w = wn;
        } else {
            pnx = px;
            pny = py;
        }
    }
    if (C->clamp_bounds) FN(clamp_position)(C, P, out->th, &pnx, &pny);
    out->px = pnx;
    out->py = pny;
}

/* Reverse mode of integrate_agent: g = adjoint of *out (all 16 fields);
   accumulates into gin (adjoint of *in), gact and gF. */
static void FN(integrate_agent_adj)(const FN(ctx_t) *C, const FN(prm_t) *P,
                                    const FN(agent_t) *in, const REAL *act, REAL Fx, REAL Fy,
                                    const FN(agent_t) *g, FN(agent_t) *gin, REAL *gact,
                                    REAL *gFx, REAL *gFy)
{
    if (P->mode == 2) {
        /* as0 = s + clamp(tv - s, -dv, dv), tv = clamp(a0, +-max_speed) gain_v; likewise w */
        FN(prm_t) Pv = *P;
        Pv.mode = 0;
        REAL as[4], gs[4] = {0, 0, 0, 0};
        FN(servo_command)(C, P, in, act, as);
        FN(integrate_agent_adj)(C, &Pv, in, as, Fx, Fy, g, gin, gs, gFx, gFy);
        REAL dt = C->sub_dt;
        REAL tv = FN(rclamp)(act[0], -P->max_speed, P->max_speed) * P->gain_v;
        REAL tw = FN(rclamp)(act[1], -P->max_ang_vel, P->max_ang_vel) * P->gain_w;
        REAL dv = P->max_accel * dt, dw = P->max_ang_accel * dt;
        REAL xv = tv - in->s, xw = tw - in->w;
        int iv = !(xv < -dv) && !(xv > dv), iw = !(xw < -dw) && !(xw > dw);
        if (!iv) gin->s += gs[0];
        if (!iw) gin->w += gs[1];
        if (iv) gact[0] += FN(rclamp_gx)(act[0], -P->max_speed, P->max_speed, gs[0] * P->gain_v);
        if (iw) gact[1] += FN(rclamp_gx)(act[1], -P->max_ang_vel, P->max_ang_vel, gs[1] * P->gain_w);
        for (int k = 2; k < C->act_dim && k < 4; ++k) gact[k] += gs[k];
        return;
    }
    REAL dt = C->sub_dt;
    REAL a0 = act[0], a1 = C->act_dim > 1 ? act[1] : (REAL)0;
    REAL a2 = C->act_dim > 2 ? act[2] : (REAL)0;
    REAL a3 = C->act_dim > 3 ? act[3] : (REAL)0;
    if (C->clamp_bounds) {
        /* the position clamp, reversed at the unclamped output (its bounds move with the
           heading under the footprint clamp); the rest is differentiated without it */
        FN(ctx_t) C2 = *C;
        C2.clamp_bounds = 0;
        FN(agent_t) raw, g2 = *g;
        FN(integrate_agent)(&C2, P, in, act, Fx, Fy, &raw);
        FN(clamp_position_adj)(C, P, raw.px, raw.py, raw.th, &g2.px, &g2.py, &g2.th);
        FN(integrate_agent_adj)(&C2, P, in, act, Fx, Fy, &g2, gin, gact, gFx, gFy);
        return;
    }
    if (C->rk4) {
        REAL a[4] = {a0, a1, a2, a3}, ga[4] = {0, 0, 0, 0};
        FN(rk4_agent_adj)(C, P, in, a, Fx, Fy, g, gin, ga, gFx, gFy);
        for (int j = 0; j < C->act_dim && j < 4; ++j) gact[j] += ga[j];
        return;
    }
    FN(agent_t) fwd;
    FN(integrate_agent)(C, P, in, act, Fx, Fy, &fwd);
    REAL gpx = g->px, gpy = g->py;
    REAL dtm = dt / P->mass;
    if (P->tag == 3) {
        REAL zero = 0;
        REAL f0 = FN(rclamp)(a0, zero, P->thrust_max), f1 = FN(rclamp)(a1, zero, P->thrust_max);
        REAL f2 = FN(rclamp)(a2, zero, P->thrust_max), f3 = FN(rclamp)(a3, zero, P->thrust_max);
        REAL thrust = f0 + f1 + f2 + f3;
        REAL qx = in->qx, qy = in->qy, qz = in->qz, qw = in->qw;
        REAL vx3 = 0, vy3 = 0, vz3 = thrust;
        REAL c1x = qy * vz3 - qz * vy3, c1y = qz * vx3 - qx * vz3, c1z = qx * vy3 - qy * vx3;
        REAL tx_ = (REAL)2 * c1x, ty_ = (REAL)2 * c1y, tz_ = (REAL)2 * c1z;
        REAL bx = in->bx, by = in->by, bz = in->bz;
        REAL angx = (P->arm * (f1 - f3) - (P->izz - P->iyy) * by * bz) / P->ixx;
        REAL angy = (P->arm * (f2 - f0) - (P->ixx - P->izz) * bz * bx) / P->iyy;
        REAL angz = (P->kappa * (f0 - f1 + f2 - f3) - (P->iyy - P->ixx) * bx * by) / P->izz;
        REAL nbx = bx + angx * dt, nby = by + angy * dt, nbz = bz + angz * dt;
        REAL half = (REAL)0.5;
        REAL dqx = half * (qw * nbx + qy * nbz - qz * nby);
        REAL dqy = half * (qw * nby - qx * nbz + qz * nbx);
        REAL dqz = half * (qw * nbz + qx * nby - qy * nbx);
        REAL dqw = half * (-qx * nbx - qy * nby - qz * nbz);
        REAL ux = qx + dqx * dt, uy = qy + dqy * dt, uz = qz + dqz * dt, uw = qw + dqw * dt;
        REAL l = SQRT(ux * ux + uy * uy + uz * uz + uw * uw);

        /* outputs: p, z, v_xy, vz, q, br ; th, s, w pass through */
        gin->th += g->th;
        gin->s += g->s;
        gin->w += g->w;
        /* p_new = p + vxy*dt ; z_new = z + vz_new*dt */
        gin->px += gpx;
        gin->py += gpy;
        REAL gvx = g->vx + gpx * dt, gvy = g->vy + gpy * dt;
        gin->z += g->z;
        REAL gnvz = g->vz + g->z * dt;
        /* q_new = u / l */
        REAL gux = 0, guy = 0, guz = 0, guw = 0;
        if (l > (REAL)0) {
            REAL nx = ux / l, ny = uy / l, nz = uz / l, nw = uw / l;
            REAL dot = g->qx * nx + g->qy * ny + g->qz * nz + g->qw * nw;
            gux = (g->qx - nx * dot) / l;
            guy = (g->qy - ny * dot) / l;
            guz = (g->qz - nz * dot) / l;
            guw = (g->qw - nw * dot) / l;
        }
        /* u = q + dq*dt */
        REAL gqx = gux, gqy = guy, gqz = guz, gqw = guw;
        REAL gdqx = gux * dt, gdqy = guy * dt, gdqz = guz * dt, gdqw = guw * dt;
        /* dq = 0.5 * quat_deriv(q, nb) */
        gdqx *= half; gdqy *= half; gdqz *= half; gdqw *= half;
        gqw += gdqx * nbx + gdqy * nby + gdqz * nbz;
        gqy += gdqx * nbz - gdqz * nbx - gdqw * nby;
        gqz += -gdqx * nby + gdqy * nbx - gdqw * nbz;
        gqx += -gdqy * nbz + gdqz * nby - gdqw * nbx;
        REAL gnbx = g->bx + gdqx * qw + gdqy * qz - gdqz * qy - gdqw * qx;
        REAL gnby = g->by - gdqx * qz + gdqy * qw + gdqz * qx - gdqw * qy;
        REAL gnbz = g->bz + gdqx * qy - gdqy * qx + gdqz * qw - gdqw * qz;
        /* nb = b + ang*dt */
        REAL gangx = gnbx * dt, gangy = gnby * dt, gangz = gnbz * dt;
        REAL gbx = gnbx, gby = gnby, gbz = gnbz;
        /* angx = (tqx - (izz-iyy)*by*bz)/ixx etc. */
        REAL gtqx = gangx / P->ixx, gtqy = gangy / P->iyy, gtqz = gangz / P->izz;
        gby += -(P->izz - P->iyy) * bz * gtqx;
        gbz += -(P->izz - P->iyy) * by * gtqx;
        gbz += -(P->ixx - P->izz) * bx * gtqy;
        gbx += -(P->ixx - P->izz) * bz * gtqy;
        gbx += -(P->iyy - P->ixx) * by * gtqz;
        gby += -(P->iyy - P->ixx) * bx * gtqz;
        REAL gf0 = -P->arm * gtqy + P->kappa * gtqz;
        REAL gf1 = P->arm * gtqx - P->kappa * gtqz;
        REAL gf2 = P->arm * gtqy + P->kappa * gtqz;
        REAL gf3 = -P->arm * gtqx - P->kappa * gtqz;
        /* nvz = vz + accz*dt ; vxy = v + acc_xy*dt + F*dtm */
        gin->vz += gnvz;
        REAL gaccz = gnvz * dt;
        gin->vx += gvx;
        gin->vy += gvy;
        REAL gaccx = gvx * dt, gaccy = gvy * dt;
        *gFx += gvx * dtm;
        *gFy += gvy * dtm;
        /* acc = fw / m - (0,0,g) */
        REAL gfwx = gaccx / P->mass, gfwy = gaccy / P->mass, gfwz = gaccz / P->mass;
        /* fw = v3 + qw*t + cross(u, t) */
        REAL gv3x = gfwx, gv3y = gfwy, gv3z = gfwz;
        gqw += gfwx * tx_ + gfwy * ty_ + gfwz * tz_;
        REAL gtx = qw * gfwx, gty = qw * gfwy, gtz = qw * gfwz;
        /* c2 = u x t : gu += t x gc2 ; gt += gc2 x u */
        gqx += ty_ * gfwz - tz_ * gfwy;
        gqy += tz_ * gfwx - tx_ * gfwz;
        gqz += tx_ * gfwy - ty_ * gfwx;
        gtx += gfwy * qz - gfwz * qy;
        gty += gfwz * qx - gfwx * qz;
        gtz += gfwx * qy - gfwy * qx;
        /* t = 2 * (u x v3) */
        REAL gc1x = (REAL)2 * gtx, gc1y = (REAL)2 * gty, gc1z = (REAL)2 * gtz;
        gqx += vy3 * gc1z - vz3 * gc1y;
        gqy += vz3 * gc1x - vx3 * gc1z;
        gqz += vx3 * gc1y - vy3 * gc1x;
        gv3x += gc1y * qz - gc1z * qy;
        gv3y += gc1z * qx - gc1x * qz;
        gv3z += gc1x * qy - gc1y * qx;
        (void)gv3x; (void)gv3y;
        REAL gthrust = gv3z;
        gf0 += gthrust; gf1 += gthrust; gf2 += gthrust; gf3 += gthrust;
        gact[0] += FN(rclamp_gx)(a0, zero, P->thrust_max, gf0);
        gact[1] += FN(rclamp_gx)(a1, zero, P->thrust_max, gf1);
        if (C->act_dim > 2) gact[2] += FN(rclamp_gx)(a2, zero, P->thrust_max, gf2);
        if (C->act_dim > 3) gact[3] += FN(rclamp_gx)(a3, zero, P->thrust_max, gf3);
        gin->qx += gqx; gin->qy += gqy; gin->qz += gqz; gin->qw += gqw;
        gin->bx += gbx; gin->by += gby; gin->bz += gbz;
        return;
    }
    /* 2-D models: drone fields pass through */
    gin->z += g->z; gin->vz += g->vz;
    gin->qx += g->qx; gin->qy += g->qy; gin->qz += g->qz; gin->qw += g->qw;
    gin->bx += g->bx; gin->by += g->by; gin->bz += g->bz;
    REAL th = in->th;
    if (P->tag == 0) {
        REAL vnx = fwd.vx, vny = fwd.vy, sp = fwd.s;
        /* p_new = p + vn*dt ; s = length(vn) ; th passthrough ; w = 0 */
        gin->px += gpx;
        gin->py += gpy;
        gin->th += g->th;
        REAL gvx = g->vx + gpx * dt, gvy = g->vy + gpy * dt;
        if (sp > (REAL)0) {
            gvx += g->s * vnx / sp;
            gvy += g->s * vny / sp;
        }
        *gFx += gvx * dtm;
        *gFy += gvy * dtm;
        if (P->mode == 0) {
            FN(clamp_norm_adj)(a0, a1, P->max_speed, gvx, gvy, &gact[0], &gact[1]);
        } else {
            REAL accx, accy;
            FN(clamp_norm)(a0, a1, P->max_accel, &accx, &accy);
            REAL v0x = in->vx + accx * dt, v0y = in->vy + accy * dt;
            REAL g0x = 0, g0y = 0;
            FN(clamp_norm_adj)(v0x, v0y, P->max_speed, gvx, gvy, &g0x, &g0y);
            gin->vx += g0x;
            gin->vy += g0y;
            FN(clamp_norm_adj)(a0, a1, P->max_accel, g0x * dt, g0y * dt, &gact[0], &gact[1]);
        }
    } else if (P->tag == 1) {
        REAL sn = fwd.s;
        REAL c = COS(th), sn_ = SIN(th);
        gin->px += gpx;
        gin->py += gpy;
        REAL gvtx = g->vx + gpx * dt, gvty = g->vy + gpy * dt;
        gin->th += g->th;
        REAL gwn = g->w + g->th * dt;
        *gFx += gvtx * dtm;
        *gFy += gvty * dtm;
        REAL gsn = g->s + gvtx * c + gvty * sn_;
        gin->th += gvtx * sn * -sn_ + gvty * sn * c;
        if (P->mode == 0) {
            gact[0] += FN(rclamp_gx)(a0, -P->max_speed, P->max_speed, gsn);
            gact[1] += FN(rclamp_gx)(a1, -P->max_ang_vel, P->max_ang_vel, gwn);
        } else {
            REAL acc = FN(rclamp)(a0, -P->max_accel, P->max_accel);
            REAL alp = FN(rclamp)(a1, -P->max_ang_accel, P->max_ang_accel);
            REAL gx = FN(rclamp_gx)(in->s + acc * dt, -P->max_speed, P->max_speed, gsn);
            REAL gy = FN(rclamp_gx)(in->w + alp * dt, -P->max_ang_vel, P->max_ang_vel, gwn);
            gin->s += gx;
            gin->w += gy;
            gact[0] += FN(rclamp_gx)(a0, -P->max_accel, P->max_accel, gx * dt);
            gact[1] += FN(rclamp_gx)(a1, -P->max_ang_accel, P->max_ang_accel, gy * dt);
        }
    } else if (P->tag == 2) {
        REAL acc = FN(rclamp)(a0, -P->max_accel, P->max_accel);
        REAL del = FN(rclamp)(a1, -P->max_steer, P->max_steer);
        REAL sn = fwd.s;
        REAL wb = P->l_f + P->l_r;
        REAL td = TAN(del);
        REAL bu = td * P->l_r / wb;
        REAL beta = ATAN(bu);
        REAL ang = th + beta;
        REAL ca = COS(ang), sa = SIN(ang), cb = COS(beta);
        gin->px += gpx;
        gin->py += gpy;
        REAL gvtx = g->vx + gpx * dt, gvty = g->vy + gpy * dt;
        gin->th += g->th;
        REAL gwn = g->w + g->th * dt;
        *gFx += gvtx * dtm;
        *gFy += gvty * dtm;
        /* vt = sn*(cos(ang), sin(ang)) + dv */
        REAL gsn = g->s + gvtx * ca + gvty * sa;
        REAL gang = -gvtx * sn * sa + gvty * sn * ca;
        /* wn = sn / wb * cos(beta) * td */
        gsn += gwn * cb * td / wb;
        REAL gbeta = gang - gwn * (sn / wb) * SIN(beta) * td;
        REAL gtd = gwn * (sn / wb) * cb;
        gin->th += gang;
        /* beta = atan(bu) ; bu = td * l_r / wb ; td = tan(del) */
        REAL gbu = gbeta / ((REAL)1 + bu * bu);
        gtd += gbu * P->l_r / wb;
        REAL gdel = gtd * ((REAL)1 + td * td);
        REAL gx = FN(rclamp_gx)(in->s + acc * dt, P->min_speed, P->max_speed, gsn);
        gin->s += gx;
        gact[0] += FN(rclamp_gx)(a0, -P->max_accel, P->max_accel, gx * dt);
        gact[1] += FN(rclamp_gx)(a1, -P->max_steer, P->max_steer, gdel);
    } else {
        gin->px += gpx; gin->py += gpy; gin->th += g->th;
        gin->vx += g->vx; gin->vy += g->vy; gin->s += g->s; gin->w += g->w;
    }
}

/* ------------------------------------------------- body-pass terms of any shape type */

#define D FN(dn)

/* pair_force on duals (the same operations as FN(pair_force)) */
static void FN(d_pair_force)(const FN(ctx_t) *C, D dx, D dy, D rvx, D rvy, REAL md, REAL dd,
                             D *fx, D *fy)
{
    D d2 = FN(dadd)(FN(dmul)(dx, dx), FN(dmul)(dy, dy));
    D dist = FN(dsqrt)(FN(dmax)(d2, FN(dk)(C->eps2)));
    D ov = FN(dsub)(FN(dk)(md), dist);
    *fx = FN(dk)((REAL)0);
    *fy = FN(dk)((REAL)0);
    if (ov.v > (REAL)0) {
        D nx = FN(ddiv)(dx, dist), ny = FN(ddiv)(dy, dist);
        D coef = FN(d_normal_coeff)(C, ov, FN(ddot)(rvx, rvy, nx, ny), dd);
        *fx = FN(dmul)(coef, nx);
        *fy = FN(dmul)(coef, ny);
    }
}

/* closest_on_segment (swarp/core/collisions.py:157-171) on duals: the point of the core
   (centre c, direction (ux, uy), half length hl) closest to p */
static void FN(d_closest_on_segment)(D px, D py, D cx, D cy, D ux, D uy, REAL hl, D *qx, D *qy)
{
    D t = FN(dclamp)(FN(dadd)(FN(dmul)(FN(dsub)(px, cx), ux), FN(dmul)(FN(dsub)(py, cy), uy)),
                     FN(dk)(-hl), FN(dk)(hl));
    *qx = FN(dadd)(cx, FN(dmul)(t, ux));
    *qy = FN(dadd)(cy, FN(dmul)(t, uy));
}

/* _reaction (swarp/core/bodies.py:80-127): force on the body from one disc agent (p, v,
   radius ra, damping denominator dd) touching shape `ty` (radius ro, half extents hx, hy)
   centred at c, oriented by (ca, sa) = cos / sin of the body angle, its centre moving
   with vs and spinning with om; and the lever from the shape centre (r0, r1). */
static void FN(d_body_reaction)(const FN(ctx_t) *C, int ty, REAL ro, REAL hx, REAL hy, REAL ra,
                                REAL dd, D px, D py, D vx, D vy, D cx, D cy, D th, D vsx, D vsy,
                                D om, D *f0, D *f1, D *r0, D *r1)
{
    D fx, fy;
    if (ty == 1) {
        FN(d_box_force)(C, px, py, vx, vy, cx, cy, th, hx, hy, ra + C->margin, dd, vsx, vsy, om,
                        &fx, &fy);
        *r0 = FN(dsub)(px, cx);
        *r1 = FN(dsub)(py, cy);
    } else if (ty == 2) {
        D ux = FN(dcos)(th), uy = FN(dsin)(th), qx, qy;
        FN(d_closest_on_segment)(px, py, cx, cy, ux, uy, hx, &qx, &qy);
        D rrx = FN(dsub)(qx, cx), rry = FN(dsub)(qy, cy);
        D sx = FN(dadd)(vsx, FN(dmul)(FN(dneg)(om), rry)), sy = FN(dadd)(vsy, FN(dmul)(om, rrx));
        FN(d_pair_force)(C, FN(dsub)(px, qx), FN(dsub)(py, qy), FN(dsub)(vx, sx),
                         FN(dsub)(vy, sy), ra + ro + C->margin, dd, &fx, &fy);
        *r0 = rrx;
        *r1 = rry;
    } else {
        FN(d_pair_force)(C, FN(dsub)(px, cx), FN(dsub)(py, cy), FN(dsub)(vx, vsx),
                         FN(dsub)(vy, vsy), ra + ro + C->margin, dd, &fx, &fy);
        *r0 = FN(dk)((REAL)0);
        *r1 = FN(dk)((REAL)0);
    }
    *f0 = FN(dneg)(fx);
    *f1 = FN(dneg)(fy);
}

/* _body_body (swarp/core/bodies.py:183-253): force on shape `ty` of a body (radius rs,
   half extents hs, centre q moving with tv, angle th, spin om) from shape `ty2` of another
   body or of the scenery (q2, tv2, th2, om2), and its lever from the shape centre.  A
   box against a box exerts nothing (the reference models no box-box obstacle contact). */
static void FN(d_body_body)(const FN(ctx_t) *C, int ty, REAL rs, REAL hsx, REAL hsy, int ty2,
                            REAL r2, REAL h2x, REAL h2y, REAL dd, D qx, D qy, D tvx, D tvy, D th,
                            D om, D q2x, D q2y, D tv2x, D tv2y, D th2, D om2, D *f0, D *f1,
                            D *r0, D *r1)
{
    *f0 = *f1 = *r0 = *r1 = FN(dk)((REAL)0);
    if (ty == 1) {
        if (ty2 == 1) return;
        D c2x = q2x, c2y = q2y, v2x = tv2x, v2y = tv2y;
        if (ty2 == 2) {
            FN(d_closest_on_segment)(qx, qy, q2x, q2y, FN(dcos)(th2), FN(dsin)(th2), h2x, &c2x,
                                     &c2y);
            D rrx = FN(dsub)(c2x, q2x), rry = FN(dsub)(c2y, q2y);
            v2x = FN(dadd)(tv2x, FN(dmul)(FN(dneg)(om2), rry));
            v2y = FN(dadd)(tv2y, FN(dmul)(om2, rrx));
        }
        D fox, foy;
        FN(d_box_force)(C, c2x, c2y, v2x, v2y, qx, qy, th, hsx, hsy, r2 + C->margin, dd, tvx, tvy,
                        om, &fox, &foy);
        *f0 = FN(dneg)(fox);
        *f1 = FN(dneg)(foy);
        /* _closest_in_box (:168-180): c2 - q clamped onto this box, in world axes */
        D ca = FN(dcos)(th), sa = FN(dsin)(th);
        D dx = FN(dsub)(c2x, qx), dy = FN(dsub)(c2y, qy);
        D lx = FN(dadd)(FN(dmul)(ca, dx), FN(dmul)(sa, dy));
        D ly = FN(dadd)(FN(dmul)(FN(dneg)(sa), dx), FN(dmul)(ca, dy));
        D kx = FN(dclamp)(lx, FN(dk)(-hsx), FN(dk)(hsx));
        D ky = FN(dclamp)(ly, FN(dk)(-hsy), FN(dk)(hsy));
        *r0 = FN(dsub)(FN(dmul)(ca, kx), FN(dmul)(sa, ky));
        *r1 = FN(dadd)(FN(dmul)(sa, kx), FN(dmul)(ca, ky));
    } else if (ty2 == 1) {
        FN(d_box_force)(C, qx, qy, tvx, tvy, q2x, q2y, th2, h2x, h2y, rs + C->margin, dd, tv2x,
                        tv2y, om2, f0, f1);
    } else if (ty2 == 2) {
        D cpx, cpy;
        FN(d_closest_on_segment)(qx, qy, q2x, q2y, FN(dcos)(th2), FN(dsin)(th2), h2x, &cpx, &cpy);
        D rrx = FN(dsub)(cpx, q2x), rry = FN(dsub)(cpy, q2y);
        D s2x = FN(dadd)(tv2x, FN(dmul)(FN(dneg)(om2), rry));
        D s2y = FN(dadd)(tv2y, FN(dmul)(om2, rrx));
        FN(d_pair_force)(C, FN(dsub)(qx, cpx), FN(dsub)(qy, cpy), FN(dsub)(tvx, s2x),
                         FN(dsub)(tvy, s2y), rs + r2 + C->margin, dd, f0, f1);
    } else {
        FN(d_pair_force)(C, FN(dsub)(qx, q2x), FN(dsub)(qy, q2y), FN(dsub)(tvx, tv2x),
                         FN(dsub)(tvy, tv2y), rs + r2 + C->margin, dd, f0, f1);
    }
}

/* Farthest point of shape s from its body's origin, the shape axis-aligned in the body
   frame (swarp/core/bodies.py:449-459) */
static inline REAL FN(shape_reach)(const FN(ctx_t) *C, int s)
{
    REAL ax = FABS(C->o_off[2 * s]), ay = FABS(C->o_off[2 * s + 1]);
    REAL ro = C->o_rad[s], hx = C->o_half[2 * s], hy = C->o_half[2 * s + 1];
    int ty = C->o_type[s];
    if (ty == 1) return SQRT((ax + hx) * (ax + hx) + (ay + hy) * (ay + hy));
    if (ty == 2) return SQRT((ax + hx) * (ax + hx) + ay * ay) + ro;
    return SQRT(ax * ax + ay * ay) + ro;
}

static inline D FN(dseed)(REAL v, int k, int seed)
{
    D r = {v, k == seed ? (REAL)1 : (REAL)0};
    return r;
}

/* The adjoint, added into g[0..5], of a moving box or segment shape's state sh (pos,
   angle, vel, ang_vel) through its force on one disc agent (obstacle_force), the force
   adjoint being (gfx, gfy): one Jacobian column per state entry. */
static void FN(obstacle_shape_adj)(const FN(ctx_t) *C, const REAL *sh, int st, REAL ro, REAL hx,
                                   REAL hy, REAL px, REAL py, REAL vx, REAL vy, REAL ra, REAL dd,
                                   REAL gfx, REAL gfy, REAL *g)
{
    for (int k = 0; k < 6; ++k) {
        D c0 = FN(dseed)(sh[0], 0, k), c1 = FN(dseed)(sh[1], 1, k), an = FN(dseed)(sh[2], 2, k);
        D v0 = FN(dseed)(sh[3], 3, k), v1 = FN(dseed)(sh[4], 4, k), om = FN(dseed)(sh[5], 5, k);
        D fx, fy;
        if (st == 1) {
            FN(d_box_force)(C, FN(dk)(px), FN(dk)(py), FN(dk)(vx), FN(dk)(vy), c0, c1, an, hx, hy,
                            ra + C->margin, dd, v0, v1, om, &fx, &fy);
        } else {
            D qx, qy;
            FN(d_closest_on_segment)(FN(dk)(px), FN(dk)(py), c0, c1, FN(dcos)(an), FN(dsin)(an),
                                     hx, &qx, &qy);
            D rx = FN(dsub)(qx, c0), ry = FN(dsub)(qy, c1);
            D sx = FN(dadd)(v0, FN(dmul)(FN(dneg)(om), ry)), sy = FN(dadd)(v1, FN(dmul)(om, rx));
            FN(d_pair_force)(C, FN(dsub)(FN(dk)(px), qx), FN(dsub)(FN(dk)(py), qy),
                             FN(dsub)(FN(dk)(vx), sx), FN(dsub)(FN(dk)(vy), sy),
                             ra + ro + C->margin, dd, &fx, &fy);
        }
        g[k] += gfx * fx.d + gfy * fy.d;
    }
}

#undef D

/* ------------------------------------------------------------- movable bodies */

/* One movable body's contact sum, for the forward pass and its reverse.  Body rooted at
   o.  Per shape s of the body (index order) the reaction of every agent not bounds_apart
   from it, in agent order, then the contacts with the shapes of other bodies and of the
   scenery (index order), exactly the loops of obstacle_dynamics_kernel
   (swarp/core/bodies.py:423-501).  Circles take the plain contact law; boxes and
   segments the dual-number terms above, evaluated without a tangent. */
typedef struct {
    REAL qx, qy, th, tvx, tvy, om, ca, sa;
    REAL fx, fy, tau, ext;
} FN(bodysum_t);

static void FN(body_sum)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *st,
                         const REAL *od, const REAL *bd, int o, FN(bodysum_t) *B)
{
    int N = C->n_obs, A = C->n_agents;
    const REAL *b = bd + 6 * N + 6 * o;
    B->qx = b[0]; B->qy = b[1]; B->th = b[2]; B->tvx = b[3]; B->tvy = b[4]; B->om = b[5];
    FN(psincos)(B->th, &B->sa, &B->ca);
    REAL fx = 0, fy = 0, tau = 0, ext = 0;
    REAL denom_self = (REAL)1 + C->c * C->sub_dt / C->o_mass[o];
    for (int s = 0; s < N; ++s) {
        if (C->o_body[s] != o) continue;
        REAL offx = C->o_off[2 * s], offy = C->o_off[2 * s + 1];
        REAL owx = B->ca * offx - B->sa * offy;
        REAL owy = B->sa * offx + B->ca * offy;
        REAL csx = B->qx + owx, csy = B->qy + owy;
        REAL vsx = B->tvx - B->om * owy, vsy = B->tvy + B->om * owx;
        int ty = C->o_type[s];
        REAL ro = C->o_rad[s], hx = C->o_half[2 * s], hy = C->o_half[2 * s + 1];
        ext = FN(rmax)(ext, FN(shape_reach)(C, s));
        REAL bound = FN(shape_bound)(ty, ro, hx, hy);
        for (int a = 0; a < A; ++a) {
            REAL ra = P[a].radius;
            if (FN(bounds_apart)(st[a].px - csx, st[a].py - csy, ra + bound + C->margin)) continue;
            REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
            REAL f0, f1, r0 = 0, r1 = 0;
            if (ty == 0) {
                REAL gx, gy;
                FN(pair_force)(C, st[a].px - csx, st[a].py - csy, st[a].vx - vsx,
                               st[a].vy - vsy, ra + ro + C->margin, dd, &gx, &gy);
                f0 = -gx;
                f1 = -gy;
            } else {
                FN(dn) g0, g1, l0, l1;
                FN(d_body_reaction)(C, ty, ro, hx, hy, ra, dd, FN(dk)(st[a].px), FN(dk)(st[a].py),
                                    FN(dk)(st[a].vx), FN(dk)(st[a].vy), FN(dk)(csx), FN(dk)(csy),
                                    FN(dk)(B->th), FN(dk)(vsx), FN(dk)(vsy), FN(dk)(B->om), &g0,
                                    &g1, &l0, &l1);
                f0 = g0.v; f1 = g1.v; r0 = l0.v; r1 = l1.v;
            }
            REAL lx = owx + r0, ly = owy + r1;
            fx += f0;
            fy += f1;
            tau += lx * f1 - ly * f0;
        }
        for (int o2 = 0; o2 < N; ++o2) {
            if (C->o_body[o2] == o) continue;
            const REAL *d2 = od + 6 * o2;
            int ty2 = C->o_type[o2];
            REAL r2 = C->o_rad[o2], h2x = C->o_half[2 * o2], h2y = C->o_half[2 * o2 + 1];
            if (FN(bounds_apart)(d2[0] - csx, d2[1] - csy,
                                 bound + FN(shape_bound)(ty2, r2, h2x, h2y) + C->margin))
                continue;
            REAL gx, gy, r0 = 0, r1 = 0;
            if (ty == 0 && ty2 == 0) {
                FN(pair_force)(C, csx - d2[0], csy - d2[1], vsx - d2[3], vsy - d2[4],
                               ro + r2 + C->margin, denom_self, &gx, &gy);
            } else {
                FN(dn) g0, g1, l0, l1;
                FN(d_body_body)(C, ty, ro, hx, hy, ty2, r2, h2x, h2y, denom_self, FN(dk)(csx),
                                FN(dk)(csy), FN(dk)(vsx), FN(dk)(vsy), FN(dk)(B->th),
                                FN(dk)(B->om), FN(dk)(d2[0]), FN(dk)(d2[1]), FN(dk)(d2[3]),
                                FN(dk)(d2[4]), FN(dk)(d2[2]), FN(dk)(d2[5]), &g0, &g1, &l0, &l1);
                gx = g0.v; gy = g1.v; r0 = l0.v; r1 = l1.v;
            }
            REAL lx = owx + r0, ly = owy + r1;
            fx += gx;
            fy += gy;
            tau += lx * gy - ly * gx;
        }
    }
    B->fx = fx; B->fy = fy; B->tau = tau; B->ext = ext;
}

/* The body pass of one env (obstacle_dynamics_kernel, disc variant,
   swarp/core/bodies.py:367-568): every movable body integrated from the reactions of the
   agents of the substep's input state `st`, reading the shape state `ob` of the substep
   input; writes the step's new obstacle state `ob_out` (static shapes copied, each
   movable shape re-installed at its body's new pose).  Other bodies' shapes are read
   from the input snapshot. */
static void FN(bodies_env)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *st,
                           const REAL *ob, REAL *ob_out)
{
    int N = C->n_obs;
    memcpy(ob_out, ob, sizeof(REAL) * OB_W * N);
    for (int o = 0; o < N; ++o) {
        if (C->o_body[o] != o || C->o_kind[o] != 1) continue;
        FN(bodysum_t) B;
        FN(body_sum)(C, P, st, ob, ob, o, &B);
        REAL sdt = C->sub_dt, one = 1;
        REAL lin_decay = one - C->lin_damping * sdt;
        REAL ang_decay = one - C->ang_damping * sdt;
        REAL m = C->o_mass[o], I = C->o_inertia[o];
        REAL nvx = (B.tvx + B.fx / m * sdt) * lin_decay;
        REAL nvy = (B.tvy + B.fy / m * sdt) * lin_decay;
        REAL nom = (B.om + B.tau / I * sdt) * ang_decay;
        REAL nx = B.qx + nvx * sdt;
        REAL ny = B.qy + nvy * sdt;
        if (C->clamp_bounds) {
            REAL half = (REAL)0.5;
            REAL lo_x = C->bmin_x + B.ext, mid_x = (C->bmin_x + C->bmax_x) * half;
            lo_x = lo_x < mid_x ? lo_x : mid_x;
            REAL hi_x = FN(rmax)(C->bmax_x - B.ext, lo_x);
            REAL lo_y = C->bmin_y + B.ext, mid_y = (C->bmin_y + C->bmax_y) * half;
            lo_y = lo_y < mid_y ? lo_y : mid_y;
            REAL hi_y = FN(rmax)(C->bmax_y - B.ext, lo_y);
            REAL cx = FN(rclamp)(nx, lo_x, hi_x), cy = FN(rclamp)(ny, lo_y, hi_y);
            if (cx != nx) nvx = 0;
            if (cy != ny) nvy = 0;
            nx = cx;
            ny = cy;
        }
        REAL nth = B.th + nom * sdt;
        REAL *bo = ob_out + 6 * N + 6 * o;
        bo[0] = nx; bo[1] = ny; bo[2] = nth; bo[3] = nvx; bo[4] = nvy; bo[5] = nom;
        REAL nsa, nca;
        FN(psincos)(nth, &nsa, &nca);
        for (int s = 0; s < N; ++s) {
            if (C->o_body[s] != o) continue;
            REAL offx = C->o_off[2 * s], offy = C->o_off[2 * s + 1];
            REAL owx = nca * offx - nsa * offy;
            REAL owy = nsa * offx + nca * offy;
            REAL *so = ob_out + 6 * s;
            so[0] = nx + owx; so[1] = ny + owy; so[2] = nth;
            so[3] = nvx - nom * owy; so[4] = nvy + nom * owx; so[5] = nom;
        }
    }
}

/* Reverse of bodies_env (this build's own adjoint: the reference never tapes the body
   pass).  gout = adjoint of ob_out; accumulates the agents' adjoint into gst and writes
   the adjoint of the input obstacle state into gob (overwritten). */
static void FN(bodies_env_adj)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *st,
                               const REAL *ob, const REAL *gout, FN(agent_t) *gst, REAL *gob)
{
    int N = C->n_obs, A = C->n_agents;
    /* pass-through of everything the pass does not rewrite */
    memcpy(gob, gout, sizeof(REAL) * OB_W * N);
    for (int s = 0; s < N; ++s)
        if (FN(shape_moves)(C, s)) memset(gob + 6 * s, 0, sizeof(REAL) * 6);
    for (int o = 0; o < N; ++o) {
        if (C->o_body[o] != o || C->o_kind[o] != 1) continue;
        FN(bodysum_t) B;
        FN(body_sum)(C, P, st, ob, ob, o, &B);
        REAL sdt = C->sub_dt, one = 1;
        REAL lin_decay = one - C->lin_damping * sdt;
        REAL ang_decay = one - C->ang_damping * sdt;
        REAL m = C->o_mass[o], I = C->o_inertia[o];
        REAL nvx = (B.tvx + B.fx / m * sdt) * lin_decay;
        REAL nvy = (B.tvy + B.fy / m * sdt) * lin_decay;
        REAL nom = (B.om + B.tau / I * sdt) * ang_decay;
        REAL nx = B.qx + nvx * sdt, ny = B.qy + nvy * sdt;
        int clx = 0, cly = 0;
        if (C->clamp_bounds) {
            REAL half = (REAL)0.5;
            REAL lo_x = C->bmin_x + B.ext, mid_x = (C->bmin_x + C->bmax_x) * half;
            lo_x = lo_x < mid_x ? lo_x : mid_x;
            REAL hi_x = FN(rmax)(C->bmax_x - B.ext, lo_x);
            REAL lo_y = C->bmin_y + B.ext, mid_y = (C->bmin_y + C->bmax_y) * half;
            lo_y = lo_y < mid_y ? lo_y : mid_y;
            REAL hi_y = FN(rmax)(C->bmax_y - B.ext, lo_y);
            clx = FN(rclamp)(nx, lo_x, hi_x) != nx;
            cly = FN(rclamp)(ny, lo_y, hi_y) != ny;
            if (clx) nvx = 0;
            if (cly) nvy = 0;
        }
        REAL nth = B.th + nom * sdt;
        REAL nsa, nca;
        FN(psincos)(nth, &nsa, &nca);
        /* adjoint of the new body state: its own entry plus every re-installed shape */
        const REAL *gb = gout + 6 * N + 6 * o;
        REAL g_nx = gb[0], g_ny = gb[1], g_nth = gb[2], g_nvx = gb[3], g_nvy = gb[4];
        REAL g_nom = gb[5];
        for (int s = 0; s < N; ++s) {
            if (C->o_body[s] != o) continue;
            REAL offx = C->o_off[2 * s], offy = C->o_off[2 * s + 1];
            REAL owx = nca * offx - nsa * offy;
            REAL owy = nsa * offx + nca * offy;
            const REAL *g = gout + 6 * s;
            g_nx += g[0];
            g_ny += g[1];
            g_nth += g[2];
            g_nvx += g[3];
            g_nvy += g[4];
            g_nom += g[5] - g[3] * owy + g[4] * owx;
            REAL g_owx = g[0] + g[4] * nom, g_owy = g[1] - g[3] * nom;
            g_nth += -g_owx * owy + g_owy * owx;
        }
        /* nth = th + nom * sdt */
        REAL g_th = g_nth;
        g_nom += g_nth * sdt;
        /* nx = qx + nvx * sdt (a clamped axis is a constant with zero velocity) */
        REAL g_qx = clx ? (REAL)0 : g_nx, g_qy = cly ? (REAL)0 : g_ny;
        if (clx) g_nvx = 0; else g_nvx += g_nx * sdt;
        if (cly) g_nvy = 0; else g_nvy += g_ny * sdt;
        REAL g_tvx = g_nvx * lin_decay, g_tvy = g_nvy * lin_decay;
        REAL g_fx = g_nvx * lin_decay * sdt / m, g_fy = g_nvy * lin_decay * sdt / m;
        REAL g_om = g_nom * ang_decay;
        REAL g_tau = g_nom * ang_decay * sdt / I;
        /* the contact sum, term by term */
        REAL denom_self = (REAL)1 + C->c * C->sub_dt / m;
        for (int s = 0; s < N; ++s) {
            if (C->o_body[s] != o) continue;
            REAL offx = C->o_off[2 * s], offy = C->o_off[2 * s + 1];
            REAL owx = B.ca * offx - B.sa * offy;
            REAL owy = B.sa * offx + B.ca * offy;
            REAL csx = B.qx + owx, csy = B.qy + owy;
            REAL vsx = B.tvx - B.om * owy, vsy = B.tvy + B.om * owx;
            int ty = C->o_type[s];
            REAL ro = C->o_rad[s], hx = C->o_half[2 * s], hy = C->o_half[2 * s + 1];
            REAL bound = FN(shape_bound)(ty, ro, hx, hy);
            REAL g_owx = 0, g_owy = 0, g_csx = 0, g_csy = 0, g_vsx = 0, g_vsy = 0;
            REAL g_thd = 0, g_omd = 0;  /* through the shape's own angle and spin */
            for (int a = 0; a < A; ++a) {
                REAL ra = P[a].radius;
                if (FN(bounds_apart)(st[a].px - csx, st[a].py - csy, ra + bound + C->margin)) continue;
                REAL dd = (REAL)1 + C->c * C->sub_dt / P[a].mass;
                if (ty != 0) {
                    /* a box or segment: the term's Jacobian column by column */
                    const REAL in[10] = {st[a].px, st[a].py, st[a].vx, st[a].vy, csx, csy, B.th,
                                         vsx, vsy, B.om};
                    REAL f0 = 0, f1 = 0, r0 = 0, r1 = 0, g_f0 = 0, g_f1 = 0, g_r0 = 0, g_r1 = 0;
                    for (int k = -1; k < 10; ++k) {
                        FN(dn) x[10], o0, o1, l0, l1;
                        for (int q = 0; q < 10; ++q) x[q] = FN(dseed)(in[q], q, k);
                        FN(d_body_reaction)(C, ty, ro, hx, hy, ra, dd, x[0], x[1], x[2], x[3],
                                            x[4], x[5], x[6], x[7], x[8], x[9], &o0, &o1, &l0,
                                            &l1);
                        if (k < 0) {
                            f0 = o0.v; f1 = o1.v; r0 = l0.v; r1 = l1.v;
                            REAL L0 = owx + r0, L1 = owy + r1;
                            g_f0 = g_fx - g_tau * L1;
                            g_f1 = g_fy + g_tau * L0;
                            g_r0 = g_tau * f1;
                            g_r1 = -(g_tau * f0);
                            g_owx += g_tau * f1;
                            g_owy -= g_tau * f0;
                            continue;
                        }
                        REAL adj = g_f0 * o0.d + g_f1 * o1.d + g_r0 * l0.d + g_r1 * l1.d;
                        switch (k) {
                        case 0: gst[a].px += adj; break;
                        case 1: gst[a].py += adj; break;
                        case 2: gst[a].vx += adj; break;
                        case 3: gst[a].vy += adj; break;
                        case 4: g_csx += adj; break;
                        case 5: g_csy += adj; break;
                        case 6: g_thd += adj; break;
                        case 7: g_vsx += adj; break;
                        case 8: g_vsy += adj; break;
                        default: g_omd += adj; break;
                        }
                    }
                    continue;
                }
                REAL gx, gy;
                FN(pair_force)(C, st[a].px - csx, st[a].py - csy, st[a].vx - vsx, st[a].vy - vsy,
                               ra + ro + C->margin, dd, &gx, &gy);
                REAL f0 = -gx, f1 = -gy;
                /* tau += lx f1 - ly f0, lever (lx, ly) = (owx, owy) */
                REAL g_f0 = g_fx - g_tau * owy, g_f1 = g_fy + g_tau * owx;
                g_owx += g_tau * f1;
                g_owy -= g_tau * f0;
                REAL adx = 0, ady = 0, arx = 0, ary = 0;
                FN(pair_force_adj)(C, st[a].px - csx, st[a].py - csy, st[a].vx - vsx,
                                   st[a].vy - vsy, ra + ro + C->margin, dd, -g_f0, -g_f1,
                                   &adx, &ady, &arx, &ary);
                gst[a].px += adx;
                gst[a].py += ady;
                gst[a].vx += arx;
                gst[a].vy += ary;
                g_csx -= adx;
                g_csy -= ady;
                g_vsx -= arx;
                g_vsy -= ary;
            }
            for (int o2 = 0; o2 < N; ++o2) {
                if (C->o_body[o2] == o) continue;
                const REAL *d2 = ob + 6 * o2;
                int ty2 = C->o_type[o2];
                REAL r2 = C->o_rad[o2], h2x = C->o_half[2 * o2], h2y = C->o_half[2 * o2 + 1];
                if (FN(bounds_apart)(d2[0] - csx, d2[1] - csy,
                                     bound + FN(shape_bound)(ty2, r2, h2x, h2y) + C->margin))
                    continue;
                if (ty != 0 || ty2 != 0) {
                    const REAL in[12] = {csx, csy, vsx, vsy, B.th, B.om,
                                         d2[0], d2[1], d2[3], d2[4], d2[2], d2[5]};
                    static const int to_state[6] = {0, 1, 3, 4, 2, 5};
                    REAL f0 = 0, f1 = 0, g_f0 = 0, g_f1 = 0, g_r0 = 0, g_r1 = 0;
                    for (int k = -1; k < 12; ++k) {
                        FN(dn) x[12], o0, o1, l0, l1;
                        for (int q = 0; q < 12; ++q) x[q] = FN(dseed)(in[q], q, k);
                        FN(d_body_body)(C, ty, ro, hx, hy, ty2, r2, h2x, h2y, denom_self, x[0],
                                        x[1], x[2], x[3], x[4], x[5], x[6], x[7], x[8], x[9],
                                        x[10], x[11], &o0, &o1, &l0, &l1);
                        if (k < 0) {
                            f0 = o0.v; f1 = o1.v;
                            REAL L0 = owx + l0.v, L1 = owy + l1.v;
                            g_f0 = g_fx - g_tau * L1;
                            g_f1 = g_fy + g_tau * L0;
                            g_r0 = g_tau * f1;
                            g_r1 = -(g_tau * f0);
                            g_owx += g_tau * f1;
                            g_owy -= g_tau * f0;
                            continue;
                        }
                        REAL adj = g_f0 * o0.d + g_f1 * o1.d + g_r0 * l0.d + g_r1 * l1.d;
                        if (k == 0) g_csx += adj;
                        else if (k == 1) g_csy += adj;
                        else if (k == 2) g_vsx += adj;
                        else if (k == 3) g_vsy += adj;
                        else if (k == 4) g_thd += adj;
                        else if (k == 5) g_omd += adj;
                        else if (FN(shape_moves)(C, o2)) gob[6 * o2 + to_state[k - 6]] += adj;
                    }
                    continue;
                }
                REAL gx, gy;
                FN(pair_force)(C, csx - d2[0], csy - d2[1], vsx - d2[3], vsy - d2[4],
                               ro + r2 + C->margin, denom_self, &gx, &gy);
                REAL g_f0 = g_fx - g_tau * owy, g_f1 = g_fy + g_tau * owx;
                g_owx += g_tau * gy;
                g_owy -= g_tau * gx;
                REAL adx = 0, ady = 0, arx = 0, ary = 0;
                FN(pair_force_adj)(C, csx - d2[0], csy - d2[1], vsx - d2[3], vsy - d2[4],
                                   ro + r2 + C->margin, denom_self, g_f0, g_f1, &adx, &ady, &arx,
                                   &ary);
                g_csx += adx;
                g_csy += ady;
                g_vsx += arx;
                g_vsy += ary;
                if (FN(shape_moves)(C, o2)) {
                    REAL *g2 = gob + 6 * o2;
                    g2[0] -= adx;
                    g2[1] -= ady;
                    g2[3] -= arx;
                    g2[4] -= ary;
                }
            }
            /* cs = q + ow ; vs = tv + om x ow ; ow = R(th) off */
            g_qx += g_csx;
            g_qy += g_csy;
            g_owx += g_csx + g_vsy * B.om;
            g_owy += g_csy - g_vsx * B.om;
            g_tvx += g_vsx;
            g_tvy += g_vsy;
            g_om += -g_vsx * owy + g_vsy * owx + g_omd;
            g_th += -g_owx * owy + g_owy * owx + g_thd;
        }
        REAL *gi = gob + 6 * N + 6 * o;
        gi[0] = g_qx; gi[1] = g_qy; gi[2] = g_th; gi[3] = g_tvx; gi[4] = g_tvy; gi[5] = g_om;
    }
}

/* ------------------------------------------------------------ one env, one step */

typedef struct {
    FN(agent_t) *st;    /* (S+1) * A states of the substep chain */
    REAL *F;            /* S * A * 2 forces */
    int32_t *idx, *cnt; /* S * A * K and S * A lists */
    REAL *ob;           /* (S+1) * OB_W * N obstacle states (NULL without obstacles) */
} FN(chain_t);

/* Stepper.launch_substeps (swarp/core/stepper.py:784-1011): per substep neighbours on
   the substep input, forces, then the body pass (swarp/core/stepper.py:952-991), then
   integrate.  Movable bodies are integrated on every step here, taped or not. */
static void FN(step_env)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                         const REAL *ob_in, const REAL *act, FN(agent_t) *out, REAL *ob_out,
                         FN(chain_t) *ch)
{
    int A = C->n_agents, S = C->substeps, K = C->max_nbr, ad = C->act_dim, N = C->n_obs;
    size_t nob = (size_t)OB_W * N;
    FN(agent_t) *st = ch->st;
    memcpy(st, in, sizeof(FN(agent_t)) * A);
    if (N) memcpy(ch->ob, ob_in, sizeof(REAL) * nob);
    for (int s = 0; s < S; ++s) {
        FN(agent_t) *cur = st + s * A, *nxt = st + (s + 1) * A;
        const REAL *obc = N ? ch->ob + s * nob : NULL;
        REAL *obn = N ? ch->ob + (s + 1) * nob : NULL;
        REAL *F = ch->F + s * A * 2;
        int32_t *idx = ch->idx + s * A * K, *cnt = ch->cnt + s * A;
        if (C->needs_forces) {
            if (C->collisions)
                FN(lists_env)(C, cur, idx, cnt);
            else
                for (int a = 0; a < A; ++a) cnt[a] = 0;
            FN(forces_env)(C, obc, P, cur, idx, cnt, F);
        } else {
            for (int a = 0; a < 2 * A; ++a) F[a] = 0;
        }
        if (C->any_movable)
            FN(bodies_env)(C, C->PB ? C->PB : P, cur, obc, obn);
        else if (N)
            memcpy(obn, obc, sizeof(REAL) * nob);
        if (C->wheel) {
            /* contact torques, the unclamped step, wheel_contact, then the clamp */
            REAL *tq = (REAL *)malloc(sizeof(REAL) * (size_t)A);
            FN(ctx_t) C2 = *C;
            C2.clamp_bounds = 0;
            if (C->needs_forces && C->collisions + C->n_obs + C->soft_walls > 0)
                FN(torques_env)(C, obc, P, cur, idx, cnt, tq);
            else
                for (int a = 0; a < A; ++a) tq[a] = 0;
            for (int a = 0; a < A; ++a) {
                FN(integrate_agent)(&C2, P + a, cur + a, act + a * ad, F[a * 2], F[a * 2 + 1], nxt + a);
                FN(wheel_contact)(C, P + a, cur + a, F[a * 2], F[a * 2 + 1], tq[a], nxt + a);
                if (C->clamp_bounds) FN(clamp_position)(C, P + a, nxt[a].th, &nxt[a].px, &nxt[a].py);
            }
            free(tq);
        } else {
            for (int a = 0; a < A; ++a)
                FN(integrate_agent)(C, P + a, cur + a, act + a * ad, F[a * 2], F[a * 2 + 1], nxt + a);
        }
    }
    memcpy(out, st + S * A, sizeof(FN(agent_t)) * A);
    if (N && ob_out) memcpy(ob_out, ch->ob + S * nob, sizeof(REAL) * nob);
}

/* reverse of step_env: gout / gob_out = adjoint of the step output; writes gin / gob_in,
   accumulates gact.  tmp: A agents; gF: 2A; obw: 2 * OB_W * N scratch. */
static void FN(step_env_adj)(const FN(ctx_t) *C, const FN(prm_t) *P, const FN(agent_t) *in,
                             const REAL *ob_in, const REAL *act, const FN(agent_t) *gout,
                             const REAL *gob_out, FN(agent_t) *gin, REAL *gob_in, REAL *gact,
                             FN(chain_t) *ch, FN(agent_t) *tmp, REAL *gF, REAL *obw)
{
    int A = C->n_agents, S = C->substeps, K = C->max_nbr, ad = C->act_dim, N = C->n_obs;
    size_t nob = (size_t)OB_W * N;
    /* tmp / obw receive the (unused) step output; the chain keeps every substep input */
    FN(step_env)(C, P, in, ob_in, act, tmp, obw, ch);
    FN(agent_t) *g = gin;
    memcpy(g, gout, sizeof(FN(agent_t)) * A);
    REAL *gob = obw, *gprev = obw + nob;
    if (N) {
        if (gob_out)
            memcpy(gob, gob_out, sizeof(REAL) * nob);
        else
            memset(gob, 0, sizeof(REAL) * nob);
    }
    for (int s = S - 1; s >= 0; --s) {
        FN(agent_t) *cur = ch->st + s * A;
        const REAL *obc = N ? ch->ob + s * nob : NULL;
        REAL *F = ch->F + s * A * 2;
        int32_t *idx = ch->idx + s * A * K, *cnt = ch->cnt + s * A;
        memset(tmp, 0, sizeof(FN(agent_t)) * A);
        for (int a = 0; a < 2 * A; ++a) gF[a] = 0;
        for (int a = 0; a < A; ++a)
            FN(integrate_agent_adj)(C, P + a, cur + a, act + a * ad, F[a * 2], F[a * 2 + 1],
                                    g + a, tmp + a, gact + a * ad, gF + a * 2, gF + a * 2 + 1);
        if (C->any_movable)
            FN(bodies_env_adj)(C, C->PB ? C->PB : P, cur, obc, gob, tmp, gprev);
        else if (N)
            memcpy(gprev, gob, sizeof(REAL) * nob);
        if (C->needs_forces) FN(forces_env_adj)(C, obc, P, cur, idx, cnt, gF, tmp, N ? gprev : NULL);
        memcpy(g, tmp, sizeof(FN(agent_t)) * A);
        if (N) {
            REAL *t = gob;
            gob = gprev;
            gprev = t;
        }
    }
    if (N && gob_in) memcpy(gob_in, gob, sizeof(REAL) * nob);
}

/* ------------------------------------------------------------------ entry points */

static void FN(make_ctx)(const oracle_cfg_t *cfg, const oracle_obs_t *obs, FN(ctx_t) *C)
{
    memset(C, 0, sizeof(*C));
    C->k = (REAL)cfg->k;
    C->c = (REAL)cfg->c;
    C->margin = (REAL)cfg->margin;
    C->sub_dt = (REAL)(cfg->dt / cfg->substeps);
    C->max_overlap = (REAL)cfg->max_overlap;
    C->nbr_radius = (REAL)cfg->neighbor_radius;
    C->eps2 = (REAL)1.0e-10;
    C->bmin_x = (REAL)cfg->bmin_x;
    C->bmin_y = (REAL)cfg->bmin_y;
    C->bmax_x = (REAL)cfg->bmax_x;
    C->bmax_y = (REAL)cfg->bmax_y;
    C->n_envs = cfg->n_envs;
    C->n_agents = cfg->n_agents;
    C->act_dim = cfg->act_dim;
    C->substeps = cfg->substeps;
    C->max_nbr = cfg->max_neighbors > 0 ? cfg->max_neighbors : 1;
    C->collisions = cfg->collisions;
    C->soft_walls = cfg->soft_walls;
    C->clamp_bounds = cfg->clamp_bounds;
    C->lin_damping = (REAL)cfg->lin_damping;
    C->ang_damping = (REAL)cfg->ang_damping;
    C->rk4 = cfg->rk4;
    C->wheel = cfg->wheel;
    C->lat_grip = (REAL)cfg->lat_grip;
    C->turn_cap = (REAL)cfg->turn_cap;
    C->grid_bins = cfg->grid_bins;
    C->g_ox = (REAL)cfg->grid_ox;
    C->g_oy = (REAL)cfg->grid_oy;
    C->g_cs = (REAL)cfg->grid_cell;
    C->n_obs = obs ? obs->n_obstacles : 0;
    C->needs_forces = C->collisions || C->soft_walls || C->n_obs > 0;
    if (C->n_obs > 0) {
        C->o_pos = (const REAL *)obs->pos;
        C->o_rad = (const REAL *)obs->radius;
        C->o_type = obs->type;
        C->o_ang = (const REAL *)obs->angle;
        C->o_half = (const REAL *)obs->half;
        C->o_vel = (const REAL *)obs->vel;
        C->o_om = (const REAL *)obs->ang_vel;
        C->o_kind = obs->kind;
        C->o_body = obs->body;
        C->o_mass = (const REAL *)obs->mass;
        C->o_inertia = (const REAL *)obs->inertia;
        C->o_off = (const REAL *)obs->body_off;
        if (C->o_kind && C->o_body && C->o_mass && C->o_inertia && C->o_off)
            for (int o = 0; o < C->n_obs; ++o)
                if (C->o_body[o] == o && C->o_kind[o] == 1) C->any_movable = 1;
    }
}

/* The obstacle state of env e as installed (shapes from the obstacle arrays, bodies 0). */
static void FN(static_ob)(const FN(ctx_t) *C, int e, REAL *ob)
{
    int N = C->n_obs;
    memset(ob, 0, sizeof(REAL) * OB_W * N);
    for (int o = 0; o < N; ++o) {
        REAL *sh = ob + 6 * o;
        sh[0] = C->o_pos[(e * N + o) * 2];
        sh[1] = C->o_pos[(e * N + o) * 2 + 1];
        sh[2] = C->o_ang[e * N + o];
        sh[3] = C->o_vel[(e * N + o) * 2];
        sh[4] = C->o_vel[(e * N + o) * 2 + 1];
        sh[5] = C->o_om[e * N + o];
    }
}

static void FN(make_prm)(const REAL *params, const int32_t *tags, const int32_t *modes, int A,
                         FN(prm_t) *P, FN(ctx_t) *C)
{
    C->boxes = 0;
    for (int a = 0; a < A; ++a) {
        const REAL *r = params + a * 22;
        P[a].radius = r[0]; P[a].mass = r[1]; P[a].max_speed = r[2]; P[a].max_accel = r[3];
        P[a].max_ang_vel = r[4]; P[a].max_ang_accel = r[5]; P[a].l_f = r[6]; P[a].l_r = r[7];
        P[a].max_steer = r[8]; P[a].thrust_max = r[9]; P[a].arm = r[10]; P[a].ixx = r[11];
        P[a].iyy = r[12]; P[a].izz = r[13]; P[a].kappa = r[14]; P[a].gravity = r[15];
        P[a].min_speed = r[16];
        P[a].shape = r[17]; P[a].hx = r[18]; P[a].hy = r[19];
        P[a].gain_v = r[20]; P[a].gain_w = r[21];
        if (P[a].shape > (REAL)0.5) C->boxes = 1;
        P[a].tag = tags[a];
        P[a].mode = modes[a];
    }
}

int FN(oracle_neighbors)(int E, int A, int K, const REAL *pos, double radius, int32_t *idx,
                         int32_t *cnt, int32_t *tru)
{
    FN(agent_t) *st = (FN(agent_t) *)calloc((size_t)A, sizeof(FN(agent_t)));
    if (!st) return -1;
    for (int e = 0; e < E; ++e) {
        for (int a = 0; a < A; ++a) {
            st[a].px = pos[(e * A + a) * 2];
            st[a].py = pos[(e * A + a) * 2 + 1];
        }
        FN(neighbors_env)(A, K, st, (REAL)radius, idx + (size_t)e * A * K, cnt + (size_t)e * A,
                          tru + (size_t)e * A);
    }
    free(st);
    return 0;
}

/* Lists in the uniform grid's order.  pinned: the frame is (ox, oy, cs) rounded to REAL
   (NeighborGrid._fill_static_grid, swarp/core/neighbors.py:476-490); else it is reduced
   over the batch in REAL (_bounds_init / _bounds_reduce / _finalize_grid, :149-181):
   origin = the min corner, cell size = max(radius, max(extent x, extent y) / bins).
   frame_out (nullable) receives the frame used. */
int FN(oracle_neighbors_grid)(int E, int A, int K, const REAL *pos, double radius, int bins,
                              int pinned, double ox, double oy, double cs, int32_t *idx,
                              int32_t *cnt, int32_t *tru, REAL *frame_out)
{
    REAL fo_x, fo_y, fcs;
    REAL r = (REAL)radius;
    if (pinned) {
        fo_x = (REAL)ox;
        fo_y = (REAL)oy;
        fcs = (REAL)cs;
    } else {
        REAL big = (REAL)1e30, mnx = big, mny = big, mxx = -big, mxy = -big;
        for (size_t q = 0; q < (size_t)E * A; ++q) {
            REAL x = pos[2 * q], y = pos[2 * q + 1];
            mnx = x < mnx ? x : mnx;
            mny = y < mny ? y : mny;
            mxx = x > mxx ? x : mxx;
            mxy = y > mxy ? y : mxy;
        }
        REAL ex = mxx - mnx, ey = mxy - mny;
        REAL ext = ex > ey ? ex : ey;
        REAL qd = ext / (REAL)bins;
        fo_x = mnx;
        fo_y = mny;
        fcs = r > qd ? r : qd;
    }
    if (frame_out) {
        frame_out[0] = fo_x;
        frame_out[1] = fo_y;
        frame_out[2] = fcs;
    }
    FN(agent_t) *st = (FN(agent_t) *)calloc((size_t)A, sizeof(FN(agent_t)));
    if (!st) return -1;
    for (int e = 0; e < E; ++e) {
        for (int a = 0; a < A; ++a) {
            st[a].px = pos[(e * A + a) * 2];
            st[a].py = pos[(e * A + a) * 2 + 1];
        }
        FN(neighbors_env_grid)(A, K, st, r, bins, fo_x, fo_y, fcs, idx + (size_t)e * A * K,
                               cnt + (size_t)e * A, tru + (size_t)e * A);
    }
    free(st);
    return 0;
}

/* The rows the body pass reads when obs->body_params is set (installed in C->PB; free
   the result), else NULL. */
static FN(prm_t) *FN(body_rows)(const oracle_obs_t *obs, const int32_t *tags,
                                const int32_t *modes, int A, FN(ctx_t) *C)
{
    if (!obs || !obs->body_params) return NULL;
    FN(prm_t) *PB = (FN(prm_t) *)calloc((size_t)A, sizeof(FN(prm_t)));
    FN(ctx_t) scratch = *C;
    FN(make_prm)((const REAL *)obs->body_params, tags, modes, A, PB, &scratch);
    C->PB = PB;
    return PB;
}

static int FN(chain_alloc)(FN(chain_t) *ch, int A, int S, int K, int N)
{
    ch->st = (FN(agent_t) *)malloc(sizeof(FN(agent_t)) * (size_t)(S + 1) * A);
    ch->F = (REAL *)malloc(sizeof(REAL) * (size_t)S * A * 2);
    ch->idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)S * A * K);
    ch->cnt = (int32_t *)malloc(sizeof(int32_t) * (size_t)S * A);
    ch->ob = N ? (REAL *)malloc(sizeof(REAL) * (size_t)(S + 1) * OB_W * N) : NULL;
    return !ch->st || !ch->F || !ch->idx || !ch->cnt || (N && !ch->ob);
}

static void FN(chain_free)(FN(chain_t) *ch)
{
    free(ch->st); free(ch->F); free(ch->idx); free(ch->cnt); free(ch->ob);
}

/* T-step rollout.  state0 [E,A,16], actions [T,E,A,ad], states out [T,E,A,16].
   ob0 [E, 12N] is the initial obstacle state (NULL = as installed); ob_states
   [T, E, 12N] (nullable) receives each step's obstacle state. */
int FN(oracle_rollout_ob)(const oracle_cfg_t *cfg, const REAL *params, const int32_t *tags,
                          const int32_t *modes, const oracle_obs_t *obs, int T,
                          const REAL *state0, const REAL *ob0, const REAL *actions, REAL *states,
                          REAL *ob_states)
{
    FN(ctx_t) C;
    FN(make_ctx)(cfg, obs, &C);
    int E = C.n_envs, A = C.n_agents, S = C.substeps, K = C.max_nbr, ad = C.act_dim, N = C.n_obs;
    size_t nob = (size_t)OB_W * N;
    FN(prm_t) *P = (FN(prm_t) *)calloc((size_t)A, sizeof(FN(prm_t)));
    FN(make_prm)(params, tags, modes, A, P, &C);
    FN(prm_t) *PB = FN(body_rows)(obs, tags, modes, A, &C);
    int nth = cfg->n_threads > 0 ? cfg->n_threads : 1;
    int err = 0;
#pragma omp parallel num_threads(nth)
    {
        FN(chain_t) ch;
        REAL *obw = N ? (REAL *)malloc(sizeof(REAL) * 2 * nob) : NULL;
        if (FN(chain_alloc)(&ch, A, S, K, N) || (N && !obw)) err = 1;
#pragma omp for schedule(static)
        for (int e = 0; e < E; ++e) {
            if (err) continue;
            const FN(agent_t) *cur = (const FN(agent_t) *)(state0 + (size_t)e * A * 16);
            REAL *obc = obw, *obn = N ? obw + nob : NULL;
            if (N) {
                if (ob0)
                    memcpy(obc, ob0 + (size_t)e * nob, sizeof(REAL) * nob);
                else
                    FN(static_ob)(&C, e, obc);
            }
            for (int t = 0; t < T; ++t) {
                FN(agent_t) *out = (FN(agent_t) *)(states + ((size_t)t * E + e) * A * 16);
                FN(step_env)(&C, P, cur, obc, actions + ((size_t)t * E + e) * A * ad, out, obn,
                             &ch);
                cur = out;
                if (N) {
                    if (ob_states) memcpy(ob_states + ((size_t)t * E + e) * nob, obn, sizeof(REAL) * nob);
                    REAL *x = obc;
                    obc = obn;
                    obn = x;
                }
            }
        }
        FN(chain_free)(&ch);
        free(obw);
    }
    free(P);
    free(PB);
    return err ? -1 : 0;
}

int FN(oracle_rollout)(const oracle_cfg_t *cfg, const REAL *params, const int32_t *tags,
                       const int32_t *modes, const oracle_obs_t *obs, int T, const REAL *state0,
                       const REAL *actions, REAL *states)
{
    return FN(oracle_rollout_ob)(cfg, params, tags, modes, obs, T, state0, NULL, actions, states,
                                 NULL);
}

/* Reverse of oracle_rollout_ob.  `states` / `ob_states` are the forward outputs (the
   per-step checkpoints); adj_states [T,E,A,16] / adj_ob_states [T,E,12N] are the adjoints
   injected at every step output (NULL = zero), adj_final [E,A,16] / adj_ob_final [E,12N]
   the adjoints of the last state (NULL = zero).  Writes adj_state0 [E,A,16], adj_ob0
   [E,12N] (nullable) and adj_actions. */
int FN(oracle_rollout_adj_ob)(const oracle_cfg_t *cfg, const REAL *params, const int32_t *tags,
                              const int32_t *modes, const oracle_obs_t *obs, int T,
                              const REAL *state0, const REAL *ob0, const REAL *actions,
                              const REAL *states, const REAL *ob_states, const REAL *adj_states,
                              const REAL *adj_final, const REAL *adj_ob_states,
                              const REAL *adj_ob_final, REAL *adj_state0, REAL *adj_ob0,
                              REAL *adj_actions)
{
    FN(ctx_t) C;
    FN(make_ctx)(cfg, obs, &C);
    if (C.wheel) return -3; /* wheel contacts have no reverse mode (the reference's too) */
    int E = C.n_envs, A = C.n_agents, S = C.substeps, K = C.max_nbr, ad = C.act_dim, N = C.n_obs;
    size_t nob = (size_t)OB_W * N;
    FN(prm_t) *P = (FN(prm_t) *)calloc((size_t)A, sizeof(FN(prm_t)));
    FN(make_prm)(params, tags, modes, A, P, &C);
    FN(prm_t) *PB = FN(body_rows)(obs, tags, modes, A, &C);
    int nth = cfg->n_threads > 0 ? cfg->n_threads : 1;
    int err = 0;
    memset(adj_actions, 0, sizeof(REAL) * (size_t)T * E * A * ad);
#pragma omp parallel num_threads(nth)
    {
        FN(chain_t) ch;
        FN(agent_t) *g = (FN(agent_t) *)malloc(sizeof(FN(agent_t)) * (size_t)A);
        FN(agent_t) *gn = (FN(agent_t) *)malloc(sizeof(FN(agent_t)) * (size_t)A);
        FN(agent_t) *tmp = (FN(agent_t) *)malloc(sizeof(FN(agent_t)) * (size_t)A);
        REAL *gF = (REAL *)malloc(sizeof(REAL) * (size_t)A * 2);
        REAL *ow = (REAL *)malloc(sizeof(REAL) * (4 * nob + 1));
        if (FN(chain_alloc)(&ch, A, S, K, N) || !g || !gn || !tmp || !gF || !ow) err = 1;
#pragma omp for schedule(static)
        for (int e = 0; e < E; ++e) {
            if (err) continue;
            REAL *gob = ow, *gobn = ow + nob, *obw = ow + 2 * nob, *obin = ow + 3 * nob;
            memset(g, 0, sizeof(FN(agent_t)) * A);
            if (N) memset(gob, 0, sizeof(REAL) * nob);
            for (int t = T - 1; t >= 0; --t) {
                if (adj_states) {
                    const REAL *src = adj_states + ((size_t)t * E + e) * A * 16;
                    REAL *gd = (REAL *)g;
                    for (int i = 0; i < A * 16; ++i) gd[i] += src[i];
                }
                if (t == T - 1 && adj_final) {
                    const REAL *src = adj_final + (size_t)e * A * 16;
                    REAL *gd = (REAL *)g;
                    for (int i = 0; i < A * 16; ++i) gd[i] += src[i];
                }
                if (N && adj_ob_states) {
                    const REAL *src = adj_ob_states + ((size_t)t * E + e) * nob;
                    for (size_t i = 0; i < nob; ++i) gob[i] += src[i];
                }
                if (N && t == T - 1 && adj_ob_final) {
                    const REAL *src = adj_ob_final + (size_t)e * nob;
                    for (size_t i = 0; i < nob; ++i) gob[i] += src[i];
                }
                const FN(agent_t) *in =
                    t == 0 ? (const FN(agent_t) *)(state0 + (size_t)e * A * 16)
                           : (const FN(agent_t) *)(states + ((size_t)(t - 1) * E + e) * A * 16);
                if (N) {
                    if (t > 0)
                        memcpy(obin, ob_states + ((size_t)(t - 1) * E + e) * nob, sizeof(REAL) * nob);
                    else if (ob0)
                        memcpy(obin, ob0 + (size_t)e * nob, sizeof(REAL) * nob);
                    else
                        FN(static_ob)(&C, e, obin);
                }
                FN(step_env_adj)(&C, P, in, N ? obin : NULL,
                                 actions + ((size_t)t * E + e) * A * ad, g, N ? gob : NULL, gn,
                                 N ? gobn : NULL, adj_actions + ((size_t)t * E + e) * A * ad,
                                 &ch, tmp, gF, obw);
                memcpy(g, gn, sizeof(FN(agent_t)) * A);
                if (N) memcpy(gob, gobn, sizeof(REAL) * nob);
            }
            memcpy(adj_state0 + (size_t)e * A * 16, g, sizeof(FN(agent_t)) * A);
            if (N && adj_ob0) memcpy(adj_ob0 + (size_t)e * nob, gob, sizeof(REAL) * nob);
        }
        FN(chain_free)(&ch);
        free(g); free(gn); free(tmp); free(gF); free(ow);
    }
    free(P);
    free(PB);
    return err ? -1 : 0;
}

int FN(oracle_rollout_adj)(const oracle_cfg_t *cfg, const REAL *params, const int32_t *tags,
                           const int32_t *modes, const oracle_obs_t *obs, int T,
                           const REAL *state0, const REAL *actions, const REAL *states,
                           const REAL *adj_states, const REAL *adj_final, REAL *adj_state0,
                           REAL *adj_actions)
{
    FN(ctx_t) C;
    FN(make_ctx)(cfg, obs, &C);
    if (C.any_movable) return -2; /* bodies need the obstacle-state entry point */
    /* without movable bodies the obstacle state is constant: its checkpoints are the
       installed arrays, rebuilt per step by the _ob entry point from ob0 = NULL */
    int E = C.n_envs, N = C.n_obs;
    REAL *obs_st = NULL;
    if (N) {
        obs_st = (REAL *)malloc(sizeof(REAL) * (size_t)T * E * OB_W * N);
        if (!obs_st) return -1;
        for (int t = 0; t < T; ++t)
            for (int e = 0; e < E; ++e) FN(static_ob)(&C, e, obs_st + ((size_t)t * E + e) * OB_W * N);
    }
    int rc = FN(oracle_rollout_adj_ob)(cfg, params, tags, modes, obs, T, state0, NULL, actions,
                                       states, obs_st, adj_states, adj_final, NULL, NULL,
                                       adj_state0, NULL, adj_actions);
    free(obs_st);
    return rc;
}

/* The force pass alone on one state (for the closed-form pins). F out [E,A,2]. */
int FN(oracle_forces)(const oracle_cfg_t *cfg, const REAL *params, const int32_t *tags,
                      const int32_t *modes, const oracle_obs_t *obs, const REAL *state,
                      REAL *F)
{
    FN(ctx_t) C;
    FN(make_ctx)(cfg, obs, &C);
    int E = C.n_envs, A = C.n_agents, K = C.max_nbr;
    FN(prm_t) *P = (FN(prm_t) *)calloc((size_t)A, sizeof(FN(prm_t)));
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)A * K);
    int32_t *cnt = (int32_t *)malloc(sizeof(int32_t) * (size_t)A);
    FN(make_prm)(params, tags, modes, A, P, &C);
    REAL *od = C.n_obs ? (REAL *)malloc(sizeof(REAL) * OB_W * C.n_obs) : NULL;
    for (int e = 0; e < E; ++e) {
        const FN(agent_t) *st = (const FN(agent_t) *)(state + (size_t)e * A * 16);
        if (C.collisions)
            FN(lists_env)(&C, st, idx, cnt);
        else
            for (int a = 0; a < A; ++a) cnt[a] = 0;
        if (od) FN(static_ob)(&C, e, od);
        FN(forces_env)(&C, od, P, st, idx, cnt, F + (size_t)e * A * 2);
    }
    free(P); free(idx); free(cnt); free(od);
    return 0;
}
