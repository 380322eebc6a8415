// boxes.hpp -- box agents: oriented-rectangle footprints in the contact pass.
//
// Counterpart of the reference's box-agent kernel (collision_forces_box_kernel,
// swarp/core/collisions.py:999-1059) and the functions it calls: obb_contact / obb_force
// (:312-487), _agent_pair_force (:489-541), _box_obstacle_force / _obstacle_forces_box
// (:543-626), _wall_forces_box (:641-688), _static_forces_shaped (:950-996).
//
// Every function here is written once over a value type V: V = T in the forward pass,
// V = Dual<T, N> in the reverse pass, where N forward-mode tangents seeded on N of the
// six fields of the lane's own state the contact reads give the force's Jacobian
// columns for those fields (6 / N evaluations per contact).  Dual comparisons read the value part,
// so the reverse pass takes the branches the forward pass took, and the value part is
// the forward arithmetic itself (same operations, same order).  The derivative rules
// are those of the generated adjoint the reference differentiates with: max/min/clamp
// pass the tangent of the operand they return, abs(x) has slope sign(x) (+1 at 0).
//
// Included by swarp_hip.hip after physics.hpp.

namespace swarp {

template <typename T, int N> struct Dual {
    T v;
    T d[N];
    __device__ __forceinline__ Dual() {}
    __device__ __forceinline__ Dual(T x) : v(x)
    {
#pragma unroll
        for (int i = 0; i < N; ++i) d[i] = T(0);
    }
};

template <typename T> __device__ __forceinline__ T val(T x) { return x; }
template <typename T, int N> __device__ __forceinline__ T val(const Dual<T, N> &x) { return x.v; }

#define SWARP_DUAL_LOOP _Pragma("unroll") for (int i = 0; i < N; ++i)

template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator+(const Dual<T, N> &a, const Dual<T, N> &b)
{
    Dual<T, N> r;
    r.v = a.v + b.v;
    SWARP_DUAL_LOOP r.d[i] = a.d[i] + b.d[i];
    return r;
}
template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator-(const Dual<T, N> &a, const Dual<T, N> &b)
{
    Dual<T, N> r;
    r.v = a.v - b.v;
    SWARP_DUAL_LOOP r.d[i] = a.d[i] - b.d[i];
    return r;
}
template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator-(const Dual<T, N> &a)
{
    Dual<T, N> r;
    r.v = -a.v;
    SWARP_DUAL_LOOP r.d[i] = -a.d[i];
    return r;
}
template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator*(const Dual<T, N> &a, const Dual<T, N> &b)
{
    Dual<T, N> r;
    r.v = a.v * b.v;
    SWARP_DUAL_LOOP r.d[i] = a.d[i] * b.v + a.v * b.d[i];
    return r;
}
template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator*(const Dual<T, N> &a, T k)
{
    Dual<T, N> r;
    r.v = a.v * k;
    SWARP_DUAL_LOOP r.d[i] = a.d[i] * k;
    return r;
}
// The value part divides exactly (it is the forward arithmetic); the tangents scale by one
// hardware reciprocal (1 ulp in fp32, exact in fp64), accurate far beyond what a
// gradient needs.
template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator/(const Dual<T, N> &a, const Dual<T, N> &b)
{
    Dual<T, N> r;
    r.v = a.v / b.v;
    const T inv = m_rcp(b.v);
    SWARP_DUAL_LOOP r.d[i] = (a.d[i] - r.v * b.d[i]) * inv;
    return r;
}
template <typename T, int N>
__device__ __forceinline__ Dual<T, N> operator/(const Dual<T, N> &a, T k)
{
    Dual<T, N> r;
    r.v = a.v / k;
    const T inv = m_rcp(k);
    SWARP_DUAL_LOOP r.d[i] = a.d[i] * inv;
    return r;
}
template <typename T, int N>
__device__ __forceinline__ bool operator>(const Dual<T, N> &a, const Dual<T, N> &b)
{
    return a.v > b.v;
}
template <typename T, int N>
__device__ __forceinline__ bool operator<(const Dual<T, N> &a, const Dual<T, N> &b)
{
    return a.v < b.v;
}
template <typename T, int N> __device__ __forceinline__ Dual<T, N> m_sqrt(const Dual<T, N> &a)
{
    Dual<T, N> r;
    r.v = m_sqrt(a.v);
    const T h = r.v > T(0) ? T(0.5) * m_rcp(r.v) : T(0);
    SWARP_DUAL_LOOP r.d[i] = a.d[i] * h;
    return r;
}
template <typename T, int N> __device__ __forceinline__ Dual<T, N> m_abs(const Dual<T, N> &a)
{
    return a.v < T(0) ? -a : a;
}
template <typename T, int N> __device__ __forceinline__ Dual<T, N> m_cos(const Dual<T, N> &a)
{
    Dual<T, N> r;
    r.v = m_cos(a.v);
    const T s = -m_sin(a.v);
    SWARP_DUAL_LOOP r.d[i] = s * a.d[i];
    return r;
}
template <typename T, int N> __device__ __forceinline__ Dual<T, N> m_sin(const Dual<T, N> &a)
{
    Dual<T, N> r;
    r.v = m_sin(a.v);
    const T c = m_cos(a.v);
    SWARP_DUAL_LOOP r.d[i] = c * a.d[i];
    return r;
}
template <typename T, int N> __device__ __forceinline__ Dual<T, N> m_tanh(const Dual<T, N> &a)
{
    Dual<T, N> r;
    r.v = m_tanh(a.v);
    const T s = T(1) - r.v * r.v;
    SWARP_DUAL_LOOP r.d[i] = s * a.d[i];
    return r;
}
#undef SWARP_DUAL_LOOP

// Lane state as the contact pass sees it.
enum { BX_PX = 0, BX_PY, BX_TH, BX_VX, BX_VY, BX_W };

template <typename T> __device__ __forceinline__ T wmin(T a, T b) { return a < b ? a : b; }

// _normal_coeff (collisions.py:87-105) over V; the same arithmetic as normal_coeff.
template <typename T, typename V>
__device__ __forceinline__ V normal_coeff_v(const Cst<T> &C, V ov, V vn, T dd)
{
    V o = ov;
    if (C.max_overlap > T(0)) o = m_tanh(ov / C.max_overlap) * C.max_overlap;
    return wmax((o * C.k - vn * C.c) / dd, V(T(0)));
}

// box_force (collisions.py:174-260): the point (p, v) against the box (c, angle given as
// ca = cos, sa = sin, half-extents h) moving with (vo, om); reach = point radius + margin.
template <typename T, typename V>
__device__ __forceinline__ void box_force_v(const Cst<T> &C, V px, V py, V vx, V vy, V cx0, V cy0,
                                            V ca, V sa, T hx, T hy, T reach, T dd, V vox, V voy,
                                            V om, V &fx, V &fy)
{
    const V dx = px - cx0, dy = py - cy0;
    const V lx = ca * dx + sa * dy;
    const V ly = (-sa) * dx + ca * dy;
    const V qx = m_abs(lx) - V(hx), qy = m_abs(ly) - V(hy);
    const V ox = lx - wclamp(lx, V(-hx), V(hx)), oy = ly - wclamp(ly, V(-hy), V(hy));
    const V od2 = ox * ox + oy * oy;
    V s, nlx, nly;
    if (val(od2) > C.eps2) {
        s = m_sqrt(od2);
        nlx = ox / s;
        nly = oy / s;
    } else if (val(qx) > val(qy)) {
        s = qx;
        nlx = V(val(lx) >= T(0) ? T(1) : T(-1));
        nly = V(T(0));
    } else {
        s = qy;
        nlx = V(T(0));
        nly = V(val(ly) >= T(0) ? T(1) : T(-1));
    }
    fx = V(T(0));
    fy = V(T(0));
    const V ov = V(reach) - s;
    if (val(ov) > T(0)) {
        const V nx = ca * nlx - sa * nly, ny = sa * nlx + ca * nly;
        const V spx = lx - s * nlx, spy = ly - s * nly;
        const V rx = ca * spx - sa * spy, ry = sa * spx + ca * spy;
        const V rvx = vx - (vox + (-om) * ry), rvy = vy - (voy + om * rx);
        const V coef = normal_coeff_v(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
}

// _point_box + _vertex_vs_box (collisions.py:273-310): vertex v against a box; keeps or
// replaces (best distance, normal, contact point).  flip = +1 for a vertex of box A.
template <typename T, typename V>
__device__ __forceinline__ void vertex_vs_box(const Cst<T> &C, V vx, V vy, V cx, V cy, V ca, V sa,
                                              T hx, T hy, T flip, V &best, V &nx, V &ny, V &xx,
                                              V &xy)
{
    const V dx = vx - cx, dy = vy - cy;
    const V lx = ca * dx + sa * dy;
    const V ly = (-sa) * dx + ca * dy;
    const V kx = wclamp(lx, V(-hx), V(hx)), ky = wclamp(ly, V(-hy), V(hy));
    const V ox = lx - kx, oy = ly - ky;
    const V dist = m_sqrt(wmax(ox * ox + oy * oy, V(C.eps2)));
    if (val(dist) < val(best)) {
        const V qx = cx + (ca * kx - sa * ky), qy = cy + (sa * kx + ca * ky);
        const V sc = V(flip) / dist;
        best = dist;
        nx = (vx - qx) * sc;
        ny = (vy - qy) * sc;
        xx = (vx + qx) * T(0.5);
        xy = (vy + qy) * T(0.5);
    }
}

// obb_contact (collisions.py:312-447): signed distance s, unit normal n (from B to A) and
// contact point x of box A (centre cA, heading cos/sin caA/saA, half-extents hA) and box B.
template <typename T, typename V>
__device__ __forceinline__ void obb_contact(const Cst<T> &C, V cAx, V cAy, V caA, V saA, T hA0,
                                            T hA1, V cBx, V cBy, V caB, V saB, T hB0, T hB1,
                                            T reach, V &s, V &nx, V &ny, V &xx, V &xy)
{
    const V uA0x = caA, uA0y = saA, uA1x = -saA, uA1y = caA;
    const V uB0x = caB, uB0y = saB, uB1x = -saB, uB1y = caB;
    const V dx = cAx - cBx, dy = cAy - cBy;
    const V a00 = m_abs(uA0x * uB0x + uA0y * uB0y);
    const V a01 = m_abs(uA0x * uB1x + uA0y * uB1y);
    const V a10 = m_abs(uA1x * uB0x + uA1y * uB0y);
    const V a11 = m_abs(uA1x * uB1x + uA1y * uB1y);
    const V dA0 = dx * uA0x + dy * uA0y, dA1 = dx * uA1x + dy * uA1y;
    const V dB0 = dx * uB0x + dy * uB0y, dB1 = dx * uB1x + dy * uB1y;

    // projection gap along each face normal; the largest one is the SAT separation
    s = (m_abs(dA0) - V(hA0)) - (a00 * hB0 + a01 * hB1);
    int axis = 0;
    V t = (m_abs(dA1) - V(hA1)) - (a10 * hB0 + a11 * hB1);
    if (val(t) > val(s)) {
        s = t;
        axis = 1;
    }
    t = (m_abs(dB0) - V(hB0)) - (a00 * hA0 + a10 * hA1);
    if (val(t) > val(s)) {
        s = t;
        axis = 2;
    }
    t = (m_abs(dB1) - V(hB1)) - (a01 * hA0 + a11 * hA1);
    if (val(t) > val(s)) {
        s = t;
        axis = 3;
    }

    nx = V(T(0));
    ny = V(T(0));
    xx = cAx;
    xy = cAy;
    if (val(s) > reach) {
        // no contact; s is a lower bound on the gap
    } else if (val(s) > T(0)) {
        // disjoint: the exact distance, attained at a vertex of one box against the other
        const V eA0x = uA0x * hA0, eA0y = uA0y * hA0, eA1x = uA1x * hA1, eA1y = uA1y * hA1;
        const V eB0x = uB0x * hB0, eB0y = uB0y * hB0, eB1x = uB1x * hB1, eB1y = uB1y * hB1;
        V best = V(T(1.0e30));
        const T one = T(1);
        vertex_vs_box(C, (cAx + eA0x) + eA1x, (cAy + eA0y) + eA1y, cBx, cBy, caB, saB, hB0, hB1,
                      one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cAx - eA0x) + eA1x, (cAy - eA0y) + eA1y, cBx, cBy, caB, saB, hB0, hB1,
                      one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cAx - eA0x) - eA1x, (cAy - eA0y) - eA1y, cBx, cBy, caB, saB, hB0, hB1,
                      one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cAx + eA0x) - eA1x, (cAy + eA0y) - eA1y, cBx, cBy, caB, saB, hB0, hB1,
                      one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cBx + eB0x) + eB1x, (cBy + eB0y) + eB1y, cAx, cAy, caA, saA, hA0, hA1,
                      -one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cBx - eB0x) + eB1x, (cBy - eB0y) + eB1y, cAx, cAy, caA, saA, hA0, hA1,
                      -one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cBx - eB0x) - eB1x, (cBy - eB0y) - eB1y, cAx, cAy, caA, saA, hA0, hA1,
                      -one, best, nx, ny, xx, xy);
        vertex_vs_box(C, (cBx + eB0x) - eB1x, (cBy + eB0y) - eB1y, cAx, cAy, caA, saA, hA0, hA1,
                      -one, best, nx, ny, xx, xy);
        s = best;
    } else {
        // overlapping: the axis of least overlap, oriented B -> A, and its reference face
        V ux = uA0x, uy = uA0y, tx = uA1x, ty = uA1y, dn = dA0;
        T h_n = hA0, h_t = hA1;
        V r_t = a10 * hB0 + a11 * hB1;  // the incident box's reach along tdir
        if (axis == 1) {
            ux = uA1x; uy = uA1y; tx = uA0x; ty = uA0y; dn = dA1;
            h_n = hA1; h_t = hA0;
            r_t = a00 * hB0 + a01 * hB1;
        } else if (axis == 2) {
            ux = uB0x; uy = uB0y; tx = uB1x; ty = uB1y; dn = dB0;
            h_n = hB0; h_t = hB1;
            r_t = a01 * hA0 + a11 * hA1;
        } else if (axis == 3) {
            ux = uB1x; uy = uB1y; tx = uB0x; ty = uB0y; dn = dB1;
            h_n = hB1; h_t = hB0;
            r_t = a00 * hA0 + a10 * hA1;
        }
        const T sgn = val(dn) < T(0) ? T(-1) : T(1);
        nx = ux * sgn;
        ny = uy * sgn;
        // reference face: A's face toward B for an A axis, B's face toward A for a B axis
        V crx = cAx, cry = cAy, cix = cBx, ciy = cBy;
        V xn = (cAx * nx + cAy * ny) - V(h_n);
        if (axis >= 2) {
            crx = cBx; cry = cBy; cix = cAx; ciy = cAy;
            xn = (cBx * nx + cBy * ny) + V(h_n);
        }
        const V ct_ref = crx * tx + cry * ty, ct_inc = cix * tx + ciy * ty;
        const V lo = wmax(ct_ref - V(h_t), ct_inc - r_t);
        const V hi = wmin(ct_ref + V(h_t), ct_inc + r_t);
        const V mid = V(T(0.5)) * (lo + hi);
        xx = nx * xn + tx * mid;
        xy = ny * xn + ty * mid;
    }
}

// obb_force (collisions.py:449-487): force on box A from box B; the damper reads the
// closing velocity of the two material points at the contact point.
template <typename T, typename V>
__device__ __forceinline__ void obb_force(const Cst<T> &C, V cAx, V cAy, V caA, V saA, T hA0,
                                          T hA1, V vAx, V vAy, V wA, V cBx, V cBy, V caB, V saB,
                                          T hB0, T hB1, V vBx, V vBy, V wB, T reach, T dd, V &fx,
                                          V &fy, V *xo = nullptr, V *yo = nullptr)
{
    V s, nx, ny, xx, xy;
    obb_contact(C, cAx, cAy, caA, saA, hA0, hA1, cBx, cBy, caB, saB, hB0, hB1, reach, s, nx, ny,
                xx, xy);
    if (xo) *xo = xx;
    if (yo) *yo = xy;
    fx = V(T(0));
    fy = V(T(0));
    const V ov = V(reach) - s;
    if (val(ov) > T(0)) {
        const V rAx = xx - cAx, rAy = xy - cAy, rBx = xx - cBx, rBy = xy - cBy;
        const V pax = vAx + (-wA) * rAy, pay = vAy + wA * rAx;
        const V pbx = vBx + (-wB) * rBy, pby = vBy + wB * rBx;
        const V rvx = pax - pbx, rvy = pay - pby;
        const V coef = normal_coeff_v(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
}

// Footprint of one agent as the contact pass needs it.
template <typename T> struct Foot {
    T shape, radius, hx, hy;
};

// _agent_pair_force (collisions.py:489-541) for a pair with at least one box: the force
// on agent a (state sa, heading cos/sin ca/sn_a) from agent b.  Box-box evaluates the one
// contact with the lower index as box A on both sides.
template <typename T, typename V>
__device__ __forceinline__ void agent_pair_force_box(const Cst<T> &C, int a, int b,
                                                     const Foot<T> &Fa, const V (&sa)[6], V caa,
                                                     V saa, const Foot<T> &Fb, const V (&sb)[6],
                                                     V cab, V sab, T dd, V &fx, V &fy)
{
    const T half = T(0.5);
    if (Fa.shape < half) {
        box_force_v(C, sa[BX_PX], sa[BX_PY], sa[BX_VX], sa[BX_VY], sb[BX_PX], sb[BX_PY], cab, sab,
                    Fb.hx, Fb.hy, Fa.radius + C.margin, dd, sb[BX_VX], sb[BX_VY], sb[BX_W], fx, fy);
    } else if (Fb.shape < half) {
        V gx, gy;
        box_force_v(C, sb[BX_PX], sb[BX_PY], sb[BX_VX], sb[BX_VY], sa[BX_PX], sa[BX_PY], caa, saa,
                    Fa.hx, Fa.hy, Fb.radius + C.margin, dd, sa[BX_VX], sa[BX_VY], sa[BX_W], gx, gy);
        fx = -gx;
        fy = -gy;
    } else if (a < b) {
        obb_force(C, sa[BX_PX], sa[BX_PY], caa, saa, Fa.hx, Fa.hy, sa[BX_VX], sa[BX_VY], sa[BX_W],
                  sb[BX_PX], sb[BX_PY], cab, sab, Fb.hx, Fb.hy, sb[BX_VX], sb[BX_VY], sb[BX_W],
                  C.margin, dd, fx, fy);
    } else {
        V gx, gy;
        obb_force(C, sb[BX_PX], sb[BX_PY], cab, sab, Fb.hx, Fb.hy, sb[BX_VX], sb[BX_VY], sb[BX_W],
                  sa[BX_PX], sa[BX_PY], caa, saa, Fa.hx, Fa.hy, sa[BX_VX], sa[BX_VY], sa[BX_W],
                  C.margin, dd, gx, gy);
        fx = -gx;
        fy = -gy;
    }
}

// One obstacle's force on a box agent (state s, heading cos / sin ca / sa), the body of
// _box_obstacle_force (:543-586): a BOX obstacle is obb_force with reach = margin, a
// SEGMENT the degenerate box (half_len, 0) with reach = radius + margin (the exact
// capsule), a CIRCLE minus box_force with the circle's centre as the point.
template <typename T, typename V>
__device__ __forceinline__ void box_obstacle_v(const Cst<T> &C, const Obs<T> &O, size_t j, int o,
                                               const T *ocs, T hx, T hy, const V (&s)[6], V ca,
                                               V sa, T dd, V &gx, V &gy)
{
    const T cx = O.pos[2 * j], cy = O.pos[2 * j + 1];
    const int st = O.type[o];
    const T ro = O.rad[o], ohx = O.half[2 * o], ohy = O.half[2 * o + 1];
    T oc, os;
    ob_trig(O, j, o, ocs, oc, os);
    const V vox = V(O.vel[2 * j]), voy = V(O.vel[2 * j + 1]), om = V(O.om[j]);
    if (st == 1 || st == 2) {
        obb_force(C, s[BX_PX], s[BX_PY], ca, sa, hx, hy, s[BX_VX], s[BX_VY], s[BX_W], V(cx), V(cy),
                  V(oc), V(os), ohx, st == 1 ? ohy : T(0), vox, voy, om,
                  st == 1 ? C.margin : ro + C.margin, dd, gx, gy);
    } else {
        V hxv, hyv;
        box_force_v(C, V(cx), V(cy), vox, voy, s[BX_PX], s[BX_PY], ca, sa, hx, hy, ro + C.margin,
                    dd, s[BX_VX], s[BX_VY], s[BX_W], hxv, hyv);
        gx = -hxv;
        gy = -hyv;
    }
}

// Whether obstacle o can touch a box agent of circumradius ra at (px, py): the reference's
// broad phase (bounds_apart with shape_bound, collisions.py:61-84).
template <typename T>
__device__ __forceinline__ bool box_obstacle_near(const Cst<T> &C, const Obs<T> &O, size_t j,
                                                  int o, T ra, T px, T py)
{
    const int st = O.type[o];
    const T ro = O.rad[o], ohx = O.half[2 * o], ohy = O.half[2 * o + 1];
    const T bound = st == 1 ? m_sqrt(ohx * ohx + ohy * ohy) : (st == 2 ? ohx + ro : ro);
    const T lim = (ra + C.margin + bound) * T(1.0001) + T(1.0e-6);
    const T ddx = px - O.pos[2 * j], ddy = py - O.pos[2 * j + 1];
    return !(ddx * ddx + ddy * ddy > lim * lim);
}

// The soft walls on a box agent (_wall_forces_box, :641-688): the support extents replace
// the radius, the damper reads the velocity of the vertex touching each wall.  `active`
// (nullable) is set when a wall exerts a force.
template <typename T, typename V>
__device__ __forceinline__ void box_walls_v(const Cst<T> &C, T hx, T hy, const V (&s)[6], V ca,
                                            V sa, T dd, V &wx, V &wy, bool *active = nullptr)
{
    const V ex = m_abs(ca) * hx + m_abs(sa) * hy;
    const V ey = m_abs(sa) * hx + m_abs(ca) * hy;
    const T vc = val(ca), vs = val(sa);
    const T sc = vc > T(0) ? T(1) : (vc < T(0) ? T(-1) : T(0));
    const T ss = vs > T(0) ? T(1) : (vs < T(0) ? T(-1) : T(0));
    const V rl_y = sa * (-sc * hx) + ca * (ss * hy);
    const V rb_x = ca * (-ss * hx) + sa * (sc * hy);
    const V em = ex + V(C.margin), eym = ey + V(C.margin);
    bool act = false;
    wx = V(T(0));
    wy = V(T(0));
    V pen = em - (s[BX_PX] - V(C.bmin_x));
    if (val(pen) > T(0)) {
        const V q = normal_coeff_v(C, pen, s[BX_VX] - s[BX_W] * rl_y, dd);
        act |= val(q) != T(0);
        wx = wx + q;
    }
    pen = em - (V(C.bmax_x) - s[BX_PX]);
    if (val(pen) > T(0)) {
        const V q = normal_coeff_v(C, pen, -(s[BX_VX] + s[BX_W] * rl_y), dd);
        act |= val(q) != T(0);
        wx = wx + (-q);
    }
    pen = eym - (s[BX_PY] - V(C.bmin_y));
    if (val(pen) > T(0)) {
        const V q = normal_coeff_v(C, pen, s[BX_VY] + s[BX_W] * rb_x, dd);
        act |= val(q) != T(0);
        wy = wy + q;
    }
    pen = eym - (V(C.bmax_y) - s[BX_PY]);
    if (val(pen) > T(0)) {
        const V q = normal_coeff_v(C, pen, -(s[BX_VY] - s[BX_W] * rb_x), dd);
        act |= val(q) != T(0);
        wy = wy + (-q);
    }
    if (active) *active = act;
}

// Static forces on a box agent (state s, heading cos/sin ca/sa): obstacles in index order
// (_obstacle_forces_box, :589-626), then the soft walls (_static_forces_shaped,
// :950-996).  `ocs`: this env's obstacle angles as (cos, sin) pairs, or NULL.  Recording
// (all nullable): `omask` gets bit o for each of the first 64 obstacles exerting a force,
// `wall` whether a wall does, `beyond` whether an obstacle past the 64th does.
template <typename T, typename V>
__device__ __forceinline__ void box_static_forces(const Cst<T> &C, const Obs<T> &O, size_t eN,
                                                  const T *ocs, T hx, T hy, const V (&s)[6], V ca,
                                                  V sa, T dd, V &fx_o, V &fy_o,
                                                  uint64_t *omask = nullptr, bool *wall = nullptr,
                                                  bool *beyond = nullptr)
{
    V fx = V(T(0)), fy = V(T(0));
    const T ra = m_sqrt(hx * hx + hy * hy);
    uint64_t om = 0;
    bool far = false;
    for (int o = 0; o < C.N; ++o) {
        const size_t j = eN + o;
        if (!box_obstacle_near(C, O, j, o, ra, val(s[BX_PX]), val(s[BX_PY]))) continue;
        V gx, gy;
        box_obstacle_v(C, O, j, o, ocs, hx, hy, s, ca, sa, dd, gx, gy);
        if (val(gx) != T(0) || val(gy) != T(0)) {
            if (o < 64) om |= 1ull << o;
            else far = true;
        }
        fx = fx + gx;
        fy = fy + gy;
    }
    bool won = false;
    if (C.soft_walls) {
        V wx, wy;
        box_walls_v(C, hx, hy, s, ca, sa, dd, wx, wy, &won);
        fx = fx + wx;
        fy = fy + wy;
    }
    fx_o = fx;
    fy_o = fy;
    if (omask) *omask = om;
    if (wall) *wall = won;
    if (beyond) *beyond = far;
}

// ------------------------------------------------------------------ wheel contacts
// WorldConfig.wheel_contacts (no-grad Euler 2-D path only): the force pass also returns
// each agent's contact torque about its centre (collision_forces_wheel_kernel,
// swarp/core/collisions.py:1128-1403), which wheel_contact (swarp/dynamics/kernels.py:
// 1328-1387) turns into heading change beyond the drive's turn_cap.

template <typename T> __device__ __forceinline__ T cross2(T rx, T ry, T fx, T fy)
{
    return rx * fy - ry * fx;
}

// _box_sd (:1133-1141): signed distance from a point to an oriented box.
template <typename T>
__device__ __forceinline__ T box_sd(T vx, T vy, T cx, T cy, T ca, T sa, T h0, T h1)
{
    const T dx = vx - cx, dy = vy - cy;
    const T lx = m_abs(ca * dx + sa * dy) - h0;
    const T ly = m_abs((-sa) * dx + ca * dy) - h1;
    const T ox = wmax(lx, T(0)), oy = wmax(ly, T(0));
    return m_sqrt(ox * ox + oy * oy) + wmin(wmax(lx, ly), T(0));
}

// _manifold_point (:1144-1185): the in-reach vertices of either box, averaged with their
// depths as weights; (x, y) is kept when none is in reach.
template <typename T>
__device__ __forceinline__ void manifold_point(T cAx, T cAy, T caA, T saA, T hA0, T hA1, T cBx,
                                               T cBy, T caB, T saB, T hB0, T hB1, T reach, T &x,
                                               T &y)
{
    const T eA0x = caA * hA0, eA0y = saA * hA0, eA1x = (-saA) * hA1, eA1y = caA * hA1;
    const T eB0x = caB * hB0, eB0y = saB * hB0, eB1x = (-saB) * hB1, eB1y = caB * hB1;
    T ax = T(0), ay = T(0), ws = T(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const T sx = (i == 1 || i == 2) ? T(-1) : T(1), sy = i >= 2 ? T(-1) : T(1);
        const T vax = (cAx + eA0x * sx) + eA1x * sy, vay = (cAy + eA0y * sx) + eA1y * sy;
        const T da = wmax(reach - box_sd(vax, vay, cBx, cBy, caB, saB, hB0, hB1), T(0));
        ax += vax * da;
        ay += vay * da;
        ws += da;
        const T vbx = (cBx + eB0x * sx) + eB1x * sy, vby = (cBy + eB0y * sx) + eB1y * sy;
        const T db = wmax(reach - box_sd(vbx, vby, cAx, cAy, caA, saA, hA0, hA1), T(0));
        ax += vbx * db;
        ay += vby * db;
        ws += db;
    }
    if (ws > T(0)) {
        x = ax / ws;
        y = ay / ws;
    }
}

// Torque about agent a's centre of the pair force (fx, fy) on a (_agent_pair_force_torque,
// :1188-1243): 0 for a disc a; a box against a disc b at the disc's point nearest to a; a
// box against a box at the contact's manifold point.
template <typename T>
__device__ __forceinline__ T pair_torque(const Cst<T> &C, int a, int b, const Foot<T> &Fa,
                                         const T (&sa)[6], T caa, T saa, const Foot<T> &Fb,
                                         const T (&sb)[6], T cab, T sab, T fx, T fy)
{
    const T half = T(0.5);
    if (Fa.shape < half) return T(0);
    if (Fb.shape < half) {
        const T fn = m_sqrt(fx * fx + fy * fy);
        if (!(fn > T(0))) return T(0);
        const T k = Fb.radius / fn;
        return cross2((sb[BX_PX] + fx * k) - sa[BX_PX], (sb[BX_PY] + fy * k) - sa[BX_PY], fx, fy);
    }
    if (!(fx * fx + fy * fy > T(0))) return T(0);
    // the contact point obb_force computed (the lower index is box A)
    T gx, gy, x, y;
    if (a < b)
        obb_force(C, sa[BX_PX], sa[BX_PY], caa, saa, Fa.hx, Fa.hy, sa[BX_VX], sa[BX_VY], sa[BX_W],
                  sb[BX_PX], sb[BX_PY], cab, sab, Fb.hx, Fb.hy, sb[BX_VX], sb[BX_VY], sb[BX_W],
                  C.margin, T(1), gx, gy, &x, &y);
    else
        obb_force(C, sb[BX_PX], sb[BX_PY], cab, sab, Fb.hx, Fb.hy, sb[BX_VX], sb[BX_VY], sb[BX_W],
                  sa[BX_PX], sa[BX_PY], caa, saa, Fa.hx, Fa.hy, sa[BX_VX], sa[BX_VY], sa[BX_W],
                  C.margin, T(1), gx, gy, &x, &y);
    manifold_point(sa[BX_PX], sa[BX_PY], caa, saa, Fa.hx, Fa.hy, sb[BX_PX], sb[BX_PY], cab, sab,
                   Fb.hx, Fb.hy, C.margin, x, y);
    return cross2(x - sa[BX_PX], y - sa[BX_PY], fx, fy);
}

// Torque of a box agent's static contacts about its centre (_static_forces_torque,
// :1246-1340): each obstacle's force at its point (a circle's point nearest the box, a
// box's or capsule core's manifold point), each wall's at its support vertex.
template <typename T>
__device__ __forceinline__ T box_static_torque(const Cst<T> &C, const Obs<T> &O, size_t eN,
                                               const T *ocs, T hx, T hy, const T (&s)[6], T ca,
                                               T sa, T dd)
{
    const T ra = m_sqrt(hx * hx + hy * hy);
    T tau = T(0);
    for (int o = 0; o < C.N; ++o) {
        const size_t j = eN + o;
        if (!box_obstacle_near(C, O, j, o, ra, s[BX_PX], s[BX_PY])) continue;
        const int st = O.type[o];
        const T cx = O.pos[2 * j], cy = O.pos[2 * j + 1];
        const T ro = O.rad[o], ohx = O.half[2 * o], ohy = st == 1 ? O.half[2 * o + 1] : T(0);
        T oc, os;
        ob_trig(O, j, o, ocs, oc, os);
        T fx, fy, x = cx, y = cy;
        if (st == 1 || st == 2) {
            obb_force(C, s[BX_PX], s[BX_PY], ca, sa, hx, hy, s[BX_VX], s[BX_VY], s[BX_W], cx, cy,
                      oc, os, ohx, ohy, O.vel[2 * j], O.vel[2 * j + 1], O.om[j],
                      st == 1 ? C.margin : ro + C.margin, dd, fx, fy, &x, &y);
        } else {
            box_obstacle_v(C, O, j, o, ocs, hx, hy, s, ca, sa, dd, fx, fy);
        }
        if (fx * fx + fy * fy > T(0)) {
            if (st == 0) {
                const T k = ro / m_sqrt(fx * fx + fy * fy);
                x = x + fx * k;
                y = y + fy * k;
            } else {
                manifold_point(s[BX_PX], s[BX_PY], ca, sa, hx, hy, cx, cy, oc, os, ohx, ohy,
                               st == 1 ? C.margin : ro + C.margin, x, y);
            }
        }
        tau += cross2(x - s[BX_PX], y - s[BX_PY], fx, fy);
    }
    if (C.soft_walls) {
        const T ex = hx * m_abs(ca) + hy * m_abs(sa), ey = hx * m_abs(sa) + hy * m_abs(ca);
        const T sc = ca > T(0) ? T(1) : (ca < T(0) ? T(-1) : T(0));
        const T ss = sa > T(0) ? T(1) : (sa < T(0) ? T(-1) : T(0));
        const T rl_y = (-sc * hx) * sa + (ss * hy) * ca, rb_x = (-ss * hx) * ca + (sc * hy) * sa;
        T pen = (ex + C.margin) - (s[BX_PX] - C.bmin_x);
        if (pen > T(0)) tau += (-rl_y) * normal_coeff(C, pen, s[BX_VX] - s[BX_W] * rl_y, dd);
        pen = (ex + C.margin) - (C.bmax_x - s[BX_PX]);
        if (pen > T(0)) tau += rl_y * (-normal_coeff(C, pen, -(s[BX_VX] + s[BX_W] * rl_y), dd));
        pen = (ey + C.margin) - (s[BX_PY] - C.bmin_y);
        if (pen > T(0)) tau += rb_x * normal_coeff(C, pen, s[BX_VY] + s[BX_W] * rb_x, dd);
        pen = (ey + C.margin) - (C.bmax_y - s[BX_PY]);
        if (pen > T(0)) tau += (-rb_x) * (-normal_coeff(C, pen, -(s[BX_VY] - s[BX_W] * rb_x), dd));
    }
    return tau;
}

// wheel_contact (swarp/dynamics/kernels.py:1328-1387): a diff-drive agent's unclamped step
// output `o` from input `in` reworked -- sideways force only beyond the wheels' grip, the
// contact torque turning it only beyond turn_cap; other models pass through.
template <typename T>
__device__ __forceinline__ void wheel_contact(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                              T Fx, T Fy, T torque, St<T> &o)
{
    if (P.tag != 1) return;
    const T dt = C.sub_dt, zero = T(0);
    const T ca = m_cos(in.th), sa = m_sin(in.th);
    const T f_lat = (-Fx) * sa + Fy * ca;
    T slip = wmax(m_abs(f_lat) - C.lat_grip * P.mass, zero);
    if (f_lat < zero) slip = -slip;
    const T dv = (slip - f_lat) * (dt / P.mass);
    const T cx = (-sa) * dv, cy = ca * dv;
    o.vx = o.vx + cx;
    o.vy = o.vy + cy;
    o.px = o.px + cx * dt;
    o.py = o.py + cy * dt;
    const T inertia = P.mass * (P.hx * P.hx + P.hy * P.hy) / T(3);
    T excess = wmax(m_abs(torque) - C.turn_cap, zero);
    if (torque < zero) excess = -excess;
    T w_drive = o.w;
    if (torque * o.w < zero && m_abs(torque) > C.turn_cap) w_drive = zero;
    // a disc has no footprint inertia (0): skip the torque term when there is no excess
    // torque -- the reference's 0 * (dt / 0) -- keeping the signed zero, so the bits equal
    // the reference's wherever it is finite
    const T turn = excess != zero ? excess * (dt / inertia) : excess;
    o.th = in.th + (w_drive + turn) * dt;
}

// ------------------------------------------------------------------ reverse helpers

// Tangents carried per reverse evaluation: the six state fields a contact reads (px py th
// vx vy w) are seeded SWARP_BOX_TANGENTS at a time, 6 / SWARP_BOX_TANGENTS evaluations.
// All six in one evaluation measured fastest (the value arithmetic is shared; config-3
// box fleet backward 6.7 ms against 11.1 ms with two and 16.6 ms with one).
#ifndef SWARP_BOX_TANGENTS
#define SWARP_BOX_TANGENTS 6
#endif
constexpr int BOX_NT = SWARP_BOX_TANGENTS;
static_assert(6 % BOX_NT == 0, "the box tangent count must divide 6");

// Adds J^T w to the lane's adjoint, where J holds the Jacobian columns of (fx, fy) with
// respect to the seeded fields k0 .. k0 + N - 1 of the lane's state.
template <typename T, int N>
__device__ __forceinline__ void add_cols(const Dual<T, N> &fx, const Dual<T, N> &fy, T wx, T wy,
                                         int k0, St<T> &g)
{
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const T c = wx * fx.d[i] + wy * fy.d[i];
        switch (k0 + i) {
        case BX_PX: g.px += c; break;
        case BX_PY: g.py += c; break;
        case BX_TH: g.th += c; break;
        case BX_VX: g.vx += c; break;
        case BX_VY: g.vy += c; break;
        default: g.w += c; break;
        }
    }
}

// The lane's state as duals with fields k0 .. k0 + N - 1 seeded (one tangent each).
template <typename T, int N>
__device__ __forceinline__ void seed_state(const St<T> &s, int k0, Dual<T, N> (&o)[6])
{
    const T f[6] = {s.px, s.py, s.th, s.vx, s.vy, s.w};
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        o[k] = Dual<T, N>(f[k]);
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (k == k0 + i) o[k].d[i] = T(1);
    }
}

// The reverse evaluations are out-of-line calls when SWARP_BOX_NOINLINE is defined.
#ifdef SWARP_BOX_NOINLINE
#define SWARP_BOX_ADJ __device__ __noinline__
#else
#define SWARP_BOX_ADJ __device__ __forceinline__
#endif

// Kinds of work item of the box reverse pass (see box_item_adj).
enum { BI_PAIR = 0, BI_OBST = 1, BI_WALL = 2, BI_FULL = 3 };

// Reverse of one box contact of agent a (state `in`): adds J_a(f)^T w.  The contact is
//   BI_PAIR  a pair with neighbour b (`sb`, cos / sin cb, snb of its heading), f the pair
//            function with a unit damping denominator, w the caller's combined cotangent
//            (a's force adjoint / dd_a minus, where a is in b's list, b's / dd_b);
//   BI_OBST  obstacle o (index j = env * N + o) on box agent a, dd = a's, w = a's force
//            adjoint; likewise BI_WALL (the walls) and BI_FULL (every static contact).
// Pairs and obstacles are routed to one of two evaluation sites -- the box-box law
// (obb_force, box A / box B) or the point-box law (box_force, point / box) -- with the
// seeded agent as either operand, so the lanes of a wave evaluating different kinds of
// contact share those two sites.
template <typename T>
SWARP_BOX_ADJ void box_item_adj(const Cst<T> &C, const Obs<T> &O, size_t eN, const T *ocs,
                                int kind, int ag, const Foot<T> &Fa, const St<T> &in, int b,
                                const Foot<T> &Fb, const T (&sb)[6], T cb, T snb, int o, T dd,
                                T wx, T wy, St<T> &g)
{
    typedef Dual<T, BOX_NT> DN;
    const T half = T(0.5);
    // operands as plain values: X = the other agent or the obstacle
    T xs[6] = {T(0), T(0), T(0), T(0), T(0), T(0)}, xc = T(1), xsn = T(0), xh0 = T(0), xh1 = T(0);
    T reach = C.margin, sgn = T(1);
    bool obb = false, me_first = true;  // obb: box-box law; me_first: a is box A / the point
    if (kind == BI_PAIR) {
#pragma unroll
        for (int k = 0; k < 6; ++k) xs[k] = sb[k];
        xc = cb;
        xsn = snb;
        xh0 = Fb.hx;
        xh1 = Fb.hy;
        if (Fa.shape > half && Fb.shape > half) {  // the lower index is box A
            obb = true;
            me_first = ag < b;
            sgn = me_first ? T(1) : T(-1);
        } else if (Fa.shape < half) {               // disc a: the point of box b
            reach = Fa.radius + C.margin;
        } else {                                    // box a against disc b
            me_first = false;
            sgn = T(-1);
            reach = Fb.radius + C.margin;
        }
    } else if (kind == BI_OBST) {
        const size_t j = eN + o;
        const int st = O.type[o];
        const T ro = O.rad[o];
        xs[BX_PX] = O.pos[2 * j];
        xs[BX_PY] = O.pos[2 * j + 1];
        xs[BX_VX] = O.vel[2 * j];
        xs[BX_VY] = O.vel[2 * j + 1];
        xs[BX_W] = O.om[j];
        ob_trig(O, j, o, ocs, xc, xsn);
        xh0 = O.half[2 * o];
        xh1 = st == 1 ? O.half[2 * o + 1] : T(0);
        if (st == 1 || st == 2) {
            obb = true;
            reach = st == 1 ? C.margin : ro + C.margin;
        } else {                                    // circle: minus box_force, its centre the point
            me_first = false;
            sgn = T(-1);
            reach = ro + C.margin;
        }
    }
    const T vx = sgn * wx, vy = sgn * wy;
#pragma unroll 1
    for (int k0 = 0; k0 < 6; k0 += BOX_NT) {
        DN me[6];
        seed_state(in, k0, me);
        const DN ca = m_cos(me[BX_TH]), sa = m_sin(me[BX_TH]);
        DN fx, fy;
        if (kind == BI_WALL) {
            box_walls_v<T, DN>(C, Fa.hx, Fa.hy, me, ca, sa, dd, fx, fy);
        } else if (kind == BI_FULL) {
            box_static_forces<T, DN>(C, O, eN, ocs, Fa.hx, Fa.hy, me, ca, sa, dd, fx, fy);
        } else {
            // operand 1 (box A / the point) and operand 2 (box B / the box)
            DN p1[6], p2[6];
#pragma unroll
            for (int k = 0; k < 6; ++k) {
                p1[k] = me_first ? me[k] : DN(xs[k]);
                p2[k] = me_first ? DN(xs[k]) : me[k];
            }
            const DN c1 = me_first ? ca : DN(xc), s1 = me_first ? sa : DN(xsn);
            const DN c2 = me_first ? DN(xc) : ca, s2 = me_first ? DN(xsn) : sa;
            const T h10 = me_first ? Fa.hx : xh0, h11 = me_first ? Fa.hy : xh1;
            const T h20 = me_first ? xh0 : Fa.hx, h21 = me_first ? xh1 : Fa.hy;
            if (obb)
                obb_force(C, p1[BX_PX], p1[BX_PY], c1, s1, h10, h11, p1[BX_VX], p1[BX_VY],
                          p1[BX_W], p2[BX_PX], p2[BX_PY], c2, s2, h20, h21, p2[BX_VX], p2[BX_VY],
                          p2[BX_W], reach, dd, fx, fy);
            else
                box_force_v(C, p1[BX_PX], p1[BX_PY], p1[BX_VX], p1[BX_VY], p2[BX_PX], p2[BX_PY],
                            c2, s2, h20, h21, reach, dd, p2[BX_VX], p2[BX_VY], p2[BX_W], fx, fy);
        }
        add_cols(fx, fy, vx, vy, k0, g);
    }
}

// Reverse of a box agent's static forces: adds J(f)^T g_F.
template <typename T>
SWARP_BOX_ADJ void box_static_adj(const Cst<T> &C, const Obs<T> &O, size_t eN,
                                               const T *ocs, const Foot<T> &Fa, const St<T> &in,
                                               T dd, T gx, T gy, St<T> &g)
{
    typedef Dual<T, BOX_NT> DN;
#pragma unroll 1
    for (int k0 = 0; k0 < 6; k0 += BOX_NT) {
        DN me[6];
        seed_state(in, k0, me);
        const DN ca = m_cos(me[BX_TH]), sa = m_sin(me[BX_TH]);
        DN fx, fy;
        box_static_forces<T, DN>(C, O, eN, ocs, Fa.hx, Fa.hy, me, ca, sa, dd, fx, fy);
        add_cols(fx, fy, gx, gy, k0, g);
    }
}

}  // namespace swarp
