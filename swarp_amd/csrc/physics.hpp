// physics.hpp -- per-agent device physics of the swarp step for gfx950: contact
// forces, walls, obstacles and the Euler integrator of the four dynamics models, plus
// their hand-written reverse mode.  Included by swarp_hip.hip only.
//
// Operation order follows the reference source text so that float32 results with no
// transcendental functions are bit-identical to any IEEE restatement of it; the build
// disables FMA contraction and keeps divide/sqrt correctly rounded.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "swarp_pmath.h"

namespace swarp {

__device__ __forceinline__ float m_sqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double m_sqrt(double x) { return sqrt(x); }
// Transcendental functions: the portable double-precision evaluations of swarp_pmath.h
// (float results rounded once), bit-identical to the CPU oracle's.
__device__ __forceinline__ float m_cos(float x) { return (float)swarp_pcos((double)x); }
__device__ __forceinline__ double m_cos(double x) { return swarp_pcos(x); }
__device__ __forceinline__ float m_sin(float x) { return (float)swarp_psin((double)x); }
__device__ __forceinline__ double m_sin(double x) { return swarp_psin(x); }
__device__ __forceinline__ float m_tan(float x) { return (float)swarp_ptan((double)x); }
__device__ __forceinline__ double m_tan(double x) { return swarp_ptan(x); }
__device__ __forceinline__ float m_atan(float x) { return (float)swarp_patan((double)x); }
__device__ __forceinline__ double m_atan(double x) { return swarp_patan(x); }
__device__ __forceinline__ float m_tanh(float x) { return (float)swarp_ptanh((double)x); }
__device__ __forceinline__ double m_tanh(double x) { return swarp_ptanh(x); }
__device__ __forceinline__ float m_abs(float x) { return fabsf(x); }
__device__ __forceinline__ double m_abs(double x) { return fabs(x); }

// warp-lang semantics: max(a,b) = a > b ? a : b ; clamp(x,a,b) = min(max(a,x),b)
template <typename T> __device__ __forceinline__ T wmax(T a, T b) { return a > b ? a : b; }
template <typename T> __device__ __forceinline__ T wclamp(T x, T a, T b)
{
    T m = a > x ? a : x;
    return m < b ? m : b;
}
// gradient of clamp(x, a, b) w.r.t. x (x < a -> a, x > b -> b, else x)
template <typename T> __device__ __forceinline__ T wclamp_g(T x, T a, T b, T g)
{
    return (x < a || x > b) ? T(0) : g;
}

// One agent's full state: the nine TorchState fields flattened (16 scalars).
template <typename T> struct St {
    T px, py, th, vx, vy, s, w, z, vz, qx, qy, qz, qw, bx, by, bz;
};

template <typename T> __device__ __forceinline__ void st_zero(St<T> &g)
{
    g.px = g.py = g.th = g.vx = g.vy = g.s = g.w = g.z = g.vz = T(0);
    g.qx = g.qy = g.qz = g.qw = g.bx = g.by = g.bz = T(0);
}

// Per-agent constants of one parameter row (PARAM_FIELDS column order).
template <typename T> struct Prm {
    T radius, mass, max_speed, max_accel, max_ang_vel, max_ang_accel, l_f, l_r, max_steer;
    T thrust_max, arm, ixx, iyy, izz, kappa, gravity, min_speed;
    T shape, hx, hy;  // footprint: 0 disc, 1 box of half-extents (hx, hy)
    T gain_v, gain_w; // ControlMode.SERVO command gains
    int tag, mode;
};

// Step-wide constants, already rounded to T on the host exactly as the reference's
// `dtype(x)` conversions do.
template <typename T> struct Cst {
    T k, c, margin, sub_dt, max_overlap, eps2;
    T t_nbr;        // largest T with sqrt(t_nbr) <= neighbor_radius (exact membership test)
    T t_skin;       // candidate threshold of the per-step skin list (>= t_nbr)
    T half_margin;  // per-agent displacement budget that keeps the skin list exact
    T bmin_x, bmin_y, bmax_x, bmax_y;
    int E, A, ad, S, K, N;
    int collisions, soft_walls, needs_forces, use_skin;
    int clamp;     // 0 off, 1 disc clamp, 2 footprint clamp (a world holding box agents)
    int boxes;     // some agent is a box: the box-aware contact pass
    int wheel;     // WorldConfig.wheel_contacts: contact torques + wheel_contact (no grad)
    int per_env;   // parameter rows per (env, agent) instead of per agent
    int round_only;  // every obstacle is a circle (the body pass takes no box / segment terms)
    T lat_grip, turn_cap;
    int fast_div;  // neighbour radius <= 2^20: contact distances are short-division divisors
    int rk4;       // Integrator.RK4 instead of semi-implicit Euler
    int grid_bins;          // lists in uniform-grid order over bins x bins cells (0: index order)
    T grid_ox, grid_oy, grid_cs;  // the grid's pinned frame: origin and cell size
};

// Read-only tables that no launch writes, read through the constant address space in
// device code: a load at a wave-uniform index (the loops over obstacles and shapes) then
// becomes a scalar load through the scalar cache instead of a vector load per lane.  The
// host sees plain pointers of the same size.
#if defined(__HIP_DEVICE_COMPILE__)
#define SWARP_RO __attribute__((address_space(4)))
#else
#define SWARP_RO
#endif

// Obstacle arrays (device); shared extents [N], per-env poses [E,N].
template <typename T> struct Obs {
    const SWARP_RO T *pos, *rad, *ang, *half, *vel, *om;
    const SWARP_RO int32_t *type;
};

// ---------------------------------------------- exact fp32 arithmetic, restricted ranges
//
// The build keeps fp32 division and sqrt correctly rounded; the compiler's general
// sequences also scale tiny or huge operands and fix up special values.  Where the
// operands are known to lie in a range in which those steps are identities, shorter
// sequences below give the same bits, and a division by a per-lane constant reuses one
// prepared reciprocal.  fp64 keeps the plain operators.

// Correctly rounded sqrt(x) for finite x >= 2^-96: hardware estimate, then the two
// one-ulp residual corrections.
__device__ __forceinline__ float sqrt_rn_big(float x)
{
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sm = __int_as_float(__float_as_int(s) - 1);
    const float sp = __int_as_float(__float_as_int(s) + 1);
    const float rm = __builtin_fmaf(-sm, s, x);
    const float rp = __builtin_fmaf(-sp, s, x);
    const float s1 = rm <= 0.0f ? sm : s;
    return rp > 0.0f ? sp : s1;
}
__device__ __forceinline__ double sqrt_rn_big(double x) { return sqrt(x); }

// Reciprocal of a float32 divisor in double precision: the hardware estimate (relative
// error about 2^-24) and two Newton steps, which bring the relative error to the
// rounding limit of double precision (2^-53; 2^-51 suffices below).
__device__ __forceinline__ double rcp_d(float d)
{
    const double x = (double)d;
    double y = __builtin_amdgcn_rcp(x);
    double e = __builtin_fma(-x, y, 1.0);
    y = __builtin_fma(y, e, y);
    e = __builtin_fma(-x, y, 1.0);
    return __builtin_fma(y, e, y);
}

// A prepared divisor.  float: n / d = RN(n * y) evaluated in double precision with
// y = rcp_d(d) is the correctly rounded float quotient whenever the quotient is not
// subnormal.  Proof: with n = N 2^a, d = D 2^b (N, D < 2^24) and a float rounding
// boundary m = M 2^c next to x = n / d (M odd, M < 2^25), x - m = (n - m d) / d where
// n - m d is a non-zero multiple of 2^(b + c) >= n / (M D) (1 - 2^-23), so
// |x - m| > 2^-49.01 |x|; the double product is within (2^-51 + 2^-53) |x| of x, hence on
// the same side of every boundary (x itself is a boundary only for d a power of two, where
// y and the product are exact).  Subnormal quotients (a coarser grid) are excluded by
// sending |n| < 2^-100 (and NaN) to the general division when d <= 2^20; a divisor outside
// [2^-60, 2^20] sends every numerator there.
template <typename T> struct Dv {
    T d, lo;
};
template <> struct Dv<float> {
    float d, lo;
    double y;
};
template <typename T> __device__ __forceinline__ Dv<T> divisor(T d, bool ok)
{
    Dv<T> v;
    v.d = d;
    v.lo = T(0);
    return v;
}
__device__ __forceinline__ Dv<float> divisor(float d, bool ok)
{
    Dv<float> v;
    v.d = d;
    v.y = rcp_d(d);
    v.lo = (ok && d >= 0x1p-60f && d <= 0x1p20f) ? 0x1p-100f : __builtin_inff();
    return v;
}

// A divisor known to lie in [2^-60, 2^20] whenever `ok` holds.
template <typename T> __device__ __forceinline__ Dv<T> divisor_in_range(T d, bool ok)
{
    return divisor(d, ok);
}
__device__ __forceinline__ Dv<float> divisor_in_range(float d, bool ok)
{
    Dv<float> v;
    v.d = d;
    v.y = rcp_d(d);
    v.lo = ok ? 0x1p-100f : __builtin_inff();
    return v;
}

// n / d, correctly rounded; tiny or NaN numerators take the general division.
template <typename T> __device__ __forceinline__ T div_rn(T n, const Dv<T> &v) { return n / v.d; }
__device__ __forceinline__ float div_rn(float n, const Dv<float> &v)
{
    float q = (float)((double)n * v.y);
    if (__builtin_expect(!(fabsf(n) >= v.lo), 0)) q = n / v.d;
    return q;
}

// Division policies of the drone branches, which divide by the same few values many
// times (mass, the inertias, the quaternion norm): ArithIEEE divides and takes square
// roots with the correctly rounded IEEE operations (any T); ArithPrep computes the same
// float results through prepared divisors (rcp_d once per divisor, then three short
// operations per quotient) and sqrt_rn_big, without branches -- a numerator or radicand
// outside the range where those are exact only raises `bad`, after which the caller
// recomputes with ArithIEEE (zero numerators are exact for every divisor).
template <typename T> struct ArithIEEE {
    typedef T D;
    __device__ __forceinline__ D prep(T d) const { return d; }
    __device__ __forceinline__ T div(T n, const D &d) const { return n / d; }
    __device__ __forceinline__ T sqrt(T x) const { return m_sqrt(x); }
};
struct ArithPrep {
    bool bad = false;
    typedef Dv<float> D;
    __device__ __forceinline__ D prep(float d) const { return divisor(d, true); }
    __device__ __forceinline__ float div(float n, const D &d)
    {
        bad |= !(fabsf(n) >= d.lo) && n != 0.0f;
        return (float)((double)n * d.y);
    }
    __device__ __forceinline__ float sqrt(float x)
    {
        bad |= !(x >= 0x1p-96f && x < __builtin_inff());
        return sqrt_rn_big(x);
    }
};

// ------------------------------------------------------------- contact law

// _normal_coeff (swarp/core/collisions.py:87-105).  SAT = false compiles the tanh
// saturation out (callers that know contact_max_overlap == 0).
template <typename T, bool SAT = true>
__device__ __forceinline__ T normal_coeff(const Cst<T> &C, T ov, T vn, T dd)
{
    T o = ov;
    if (SAT && C.max_overlap > T(0)) o = C.max_overlap * m_tanh(ov / C.max_overlap);
    return wmax((C.k * o - C.c * vn) / dd, T(0));
}

// normal_coeff with the damping denominator as a prepared divisor (same result)
template <typename T, bool SAT = true>
__device__ __forceinline__ T normal_coeff_r(const Cst<T> &C, T ov, T vn, const Dv<T> &dd)
{
    T o = ov;
    if (SAT && C.max_overlap > T(0)) o = C.max_overlap * m_tanh(ov / C.max_overlap);
    return wmax(div_rn(C.k * o - C.c * vn, dd), T(0));
}

// normal_coeff given the damping denominator as a prepared divisor (same result)
template <typename T, bool SAT = true>
__device__ __forceinline__ T normal_coeff(const Cst<T> &C, T ov, T vn, const Dv<T> &dd)
{
    return normal_coeff_r<T, SAT>(C, ov, vn, dd);
}

template <typename T, bool SAT = true>
__device__ __forceinline__ void normal_coeff_adj(const Cst<T> &C, T ov, T vn, T dd, T g,
                                                 T &a_ov, T &a_vn)
{
    T o = ov, slope = T(1);
    if (SAT && C.max_overlap > T(0)) {
        T th = m_tanh(ov / C.max_overlap);
        o = C.max_overlap * th;
        slope = T(1) - th * th;
    }
    if ((C.k * o - C.c * vn) / dd > T(0)) {
        T q = g / dd;
        a_ov += C.k * q * slope;
        a_vn -= C.c * q;
    }
}

// Whether a pair at offset (dx, dy) is certainly apart at contact distance md: its
// squared distance, computed as pair_force computes it, exceeds md^2 by more than the
// roundings of md * md, so the correctly rounded distance is at least md and neither
// pair_force nor its reverses take their contact branch.  Lets a list wider than the
// contact reach skip its far members before their square root.
template <typename T> __device__ __forceinline__ bool pair_apart(T dx, T dy, T md)
{
    return dx * dx + dy * dy > md * md * T(1.000001);
}

// pair_force (swarp/core/collisions.py:108-143): force on self, d = self - other.
// Returns whether the contact branch ran (overlap > 0), the test pair_force_adj repeats
// on the same operands: it contributes only then.
template <typename T>
__device__ __forceinline__ bool pair_force(const Cst<T> &C, T dx, T dy, T rvx, T rvy, T md,
                                           T dd, T &fx, T &fy)
{
    T dist = m_sqrt(wmax(dx * dx + dy * dy, C.eps2));
    T ov = md - dist;
    fx = T(0);
    fy = T(0);
    if (ov > T(0)) {
        T nx = dx / dist, ny = dy / dist;
        T coef = normal_coeff(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
    return ov > T(0);
}

// pair_force with the damping denominator as a prepared divisor, in the exact fast
// arithmetic: the distance (at least sqrt(eps2)) through sqrt_rn_big, the normal through
// one prepared divisor (a distance outside [2^-60, 2^20] takes the general division).
// Same bits as pair_force.
template <typename T>
__device__ __forceinline__ bool pair_force(const Cst<T> &C, T dx, T dy, T rvx, T rvy, T md,
                                           const Dv<T> &dd, T &fx, T &fy)
{
    T dist = sqrt_rn_big(wmax(dx * dx + dy * dy, C.eps2));
    T ov = md - dist;
    fx = T(0);
    fy = T(0);
    if (ov > T(0)) {
        const Dv<T> ds = divisor(dist, true);
        T nx = div_rn(dx, ds), ny = div_rn(dy, ds);
        T coef = normal_coeff_r(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
    return ov > T(0);
}

// pair_force that also reports whether the contact is active (overlap and a positive
// coefficient), the branch the reverse pass must follow.
template <typename T>
__device__ __forceinline__ bool pair_force_rec(const Cst<T> &C, T dx, T dy, T rvx, T rvy, T md,
                                               T dd, T &fx, T &fy)
{
    T dist = m_sqrt(wmax(dx * dx + dy * dy, C.eps2));
    T ov = md - dist;
    fx = T(0);
    fy = T(0);
    bool on = false;
    if (ov > T(0)) {
        T nx = dx / dist, ny = dy / dist;
        T coef = normal_coeff(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
        on = coef > T(0);
    }
    return on;
}

// pair_force_rec with the range-restricted exact arithmetic: the distance is at least
// sqrt(eps2) and at most the neighbour radius, |d| <= distance; dd is a prepared divisor.
template <typename T, bool SAT = true>
__device__ __forceinline__ bool pair_force_rec_r(const Cst<T> &C, T dx, T dy, T rvx, T rvy,
                                                 T md, const Dv<T> &dd, T &fx, T &fy)
{
    T dist = sqrt_rn_big(wmax(dx * dx + dy * dy, C.eps2));
    T ov = md - dist;
    fx = T(0);
    fy = T(0);
    bool on = false;
    if (ov > T(0)) {
        const Dv<T> ds = divisor_in_range(dist, C.fast_div != 0);  // sqrt(eps2) <= dist
        T nx = div_rn(dx, ds), ny = div_rn(dy, ds);
        T coef = normal_coeff_r<T, SAT>(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
        on = coef > T(0);
    }
    return on;
}

__device__ __forceinline__ float m_rsqrt(float x) { return rsqrtf(x); }
__device__ __forceinline__ double m_rsqrt(double x) { return rsqrt(x); }

// Adjoint of one active contact pair, both forces at once (see pair_adj_combined), with
// the branch already known from the recomputed forward pass: the arithmetic only has to
// be accurate, so the distance comes from one reciprocal square root.
template <typename T, bool SAT = true>
__device__ __forceinline__ void pair_adj_active(const Cst<T> &C, T dx, T dy, T rvx, T rvy, T md,
                                                T wx, T wy, T &adx, T &ady, T &arx, T &ary)
{
    const T d2 = dx * dx + dy * dy;
    const T m2 = wmax(d2, C.eps2);
    const T inv = m_rsqrt(m2);
    const T dist = m2 * inv;
    const T nx = dx * inv, ny = dy * inv;
    const T vn = rvx * nx + rvy * ny;
    const T ov = md - dist;
    T o = ov, slope = T(1);
    if (SAT && C.max_overlap > T(0)) {
        const T th = m_tanh(ov / C.max_overlap);
        o = C.max_overlap * th;
        slope = T(1) - th * th;
    }
    const T num = C.k * o - C.c * vn;
    const T a_num = wx * nx + wy * ny;
    T anx = num * wx, any = num * wy;
    const T a_ov = C.k * a_num * slope;
    const T a_vn = -C.c * a_num;
    arx += a_vn * nx;
    ary += a_vn * ny;
    anx += a_vn * rvx;
    any += a_vn * rvy;
    const T a_dist = -(anx * nx + any * ny) * inv - a_ov;
    T ex = anx * inv, ey = any * inv;
    if (d2 > C.eps2) {
        const T h = a_dist * T(0.5) * inv;
        ex += T(2) * dx * h;
        ey += T(2) * dy * h;
    }
    adx += ex;
    ady += ey;
}

// reverse of pair_force: accumulates the adjoints of d and rel_v
template <typename T>
__device__ __forceinline__ void pair_force_adj(const Cst<T> &C, T dx, T dy, T rvx, T rvy, T md,
                                               T dd, T gx, T gy, T &adx, T &ady, T &arx,
                                               T &ary)
{
    T d2 = dx * dx + dy * dy;
    T dist = m_sqrt(wmax(d2, C.eps2));
    T ov = md - dist;
    if (!(ov > T(0))) return;
    T nx = dx / dist, ny = dy / dist;
    T vn = rvx * nx + rvy * ny;
    T coef = normal_coeff(C, ov, vn, dd);
    T a_ov = T(0), a_vn = T(0);
    normal_coeff_adj(C, ov, vn, dd, gx * nx + gy * ny, a_ov, a_vn);
    T anx = coef * gx + a_vn * rvx;
    T any = coef * gy + a_vn * rvy;
    arx += a_vn * nx;
    ary += a_vn * ny;
    T a_dist = -(anx * nx + any * ny) / dist - a_ov;
    T ex = anx / dist, ey = any / dist;
    if (d2 > C.eps2) {
        T h = a_dist * T(0.5) / dist;
        ex += T(2) * dx * h;
        ey += T(2) * dy * h;
    }
    adx += ex;
    ady += ey;
}

// Reverse of the contact pair (a, b) seen from agent a, for both forces the pair exerts.
// With d = p_a - p_b and rv = v_a - v_b, a's force is G(d, rv) / dd_a and b's force is
// -G(d, rv) / dd_b, where G = max(num, 0) * n, n = d / |d|, num = k*ov' - c*(rv.n) (the
// contact law is symmetric under (d, rv) -> (-d, -rv)).  So the adjoint of both is one
// evaluation of G's adjoint with the cotangent w = [b in a's list] g_a/dd_a
// - [a in b's list] g_b/dd_b (the caller passes w).  The distance, the normal and num are
// recomputed exactly as in the forward pass so every branch is taken as it was there; the
// arithmetic after the branches uses one reciprocal of the distance.
template <typename T>
__device__ __forceinline__ void pair_adj_combined(const Cst<T> &C, T dx, T dy, T rvx, T rvy, T md,
                                                  T wx, T wy, T &adx, T &ady, T &arx, T &ary)
{
    const T d2 = dx * dx + dy * dy;
    const T dist = m_sqrt(wmax(d2, C.eps2));
    const T ov = md - dist;
    if (!(ov > T(0))) return;
    const T nx = dx / dist, ny = dy / dist;
    const T vn = rvx * nx + rvy * ny;
    T o = ov, slope = T(1);
    if (C.max_overlap > T(0)) {
        const T th = m_tanh(ov / C.max_overlap);
        o = C.max_overlap * th;
        slope = T(1) - th * th;
    }
    const T num = C.k * o - C.c * vn;
    if (!(num > T(0))) return;  // clamped repulsive: no gradient (dd >= 1 keeps the sign)
    const T a_num = wx * nx + wy * ny;
    T anx = num * wx, any = num * wy;
    const T a_ov = C.k * a_num * slope;
    const T a_vn = -C.c * a_num;
    arx += a_vn * nx;
    ary += a_vn * ny;
    anx += a_vn * rvx;
    any += a_vn * rvy;
    const T inv = T(1) / dist;
    const T a_dist = -(anx * nx + any * ny) * inv - a_ov;
    T ex = anx * inv, ey = any * inv;
    if (d2 > C.eps2) {
        const T h = a_dist * T(0.5) * inv;
        ex += T(2) * dx * h;
        ey += T(2) * dy * h;
    }
    adx += ex;
    ady += ey;
}

// ------------------------------------------------------------------- walls

// _wall_forces (swarp/core/collisions.py:746-778)
template <typename T, bool SAT = true>
__device__ __forceinline__ void wall_force(const Cst<T> &C, T px, T py, T vx, T vy, T ra, T dd,
                                           T &fx, T &fy)
{
    T reach = ra + C.margin;
    T ax = T(0), ay = T(0), pen;
    pen = reach - (px - C.bmin_x);
    if (pen > T(0)) ax += normal_coeff<T, SAT>(C, pen, vx, dd);
    pen = reach - (C.bmax_x - px);
    if (pen > T(0)) ax += -normal_coeff<T, SAT>(C, pen, -vx, dd);
    pen = reach - (py - C.bmin_y);
    if (pen > T(0)) ay += normal_coeff<T, SAT>(C, pen, vy, dd);
    pen = reach - (C.bmax_y - py);
    if (pen > T(0)) ay += -normal_coeff<T, SAT>(C, pen, -vy, dd);
    fx = ax;
    fy = ay;
}

// _wall_forces with one contact evaluation per axis.  When the bounds are at least two
// reaches wide an agent cannot touch both walls of an axis, so at most one of the two
// `fx +=` terms of the reference is non-zero and the sum is that term alone (0 + x).
// Falls back to the four-term form otherwise.  `bits` records which axes are in
// contact with a positive coefficient (bit 0: x, bit 1: y) for the reverse pass.
template <typename T, bool SAT = true>
__device__ __forceinline__ void wall_force_axes(const Cst<T> &C, T px, T py, T vx, T vy, T ra,
                                                const Dv<T> &dv, T &fx, T &fy, unsigned &bits)
{
    const T dd = dv.d;
    const T reach = ra + C.margin;
    const T w2 = T(2) * reach * T(1.00001);
    bits = 0u;
    if (!(C.bmax_x - C.bmin_x >= w2) || !(C.bmax_y - C.bmin_y >= w2)) {
        wall_force<T, SAT>(C, px, py, vx, vy, ra, dd, fx, fy);
        bits = 3u;  // reverse pass re-derives every side
        return;
    }
    const T pl = reach - (px - C.bmin_x), pr = reach - (C.bmax_x - px);
    const T pb = reach - (py - C.bmin_y), pt = reach - (C.bmax_y - py);
    T ax = T(0), ay = T(0);
    if (pl > T(0) || pr > T(0)) {
        const bool lo = pl > T(0);
        const T cf = normal_coeff_r<T, SAT>(C, lo ? pl : pr, lo ? vx : -vx, dv);
        ax += lo ? cf : -cf;
        bits |= cf > T(0) ? 1u : 0u;
    }
    if (pb > T(0) || pt > T(0)) {
        const bool lo = pb > T(0);
        const T cf = normal_coeff_r<T, SAT>(C, lo ? pb : pt, lo ? vy : -vy, dv);
        ay += lo ? cf : -cf;
        bits |= cf > T(0) ? 2u : 0u;
    }
    fx = ax;
    fy = ay;
}

template <typename T, bool SAT = true>
__device__ __forceinline__ void wall_force_adj(const Cst<T> &C, T px, T py, T vx, T vy, T ra,
                                               T dd, T gx, T gy, St<T> &a);

// Reverse of wall_force_axes given its recorded contact bits; g * inv_dd = cotangent / dd.
// For either wall of an axis d(coef)/d(p) = -k*slope/dd along the inward normal and
// d(coef)/d(v) = -c/dd, so the side only enters through the overlap of the slope.
template <typename T, bool SAT = true>
__device__ __forceinline__ void wall_axes_adj(const Cst<T> &C, T px, T py, T vx, T vy, T ra,
                                              T dd, T inv_dd, T gx, T gy, unsigned bits,
                                              T &apx, T &apy, T &avx, T &avy)
{
    const T reach = ra + C.margin;
    const T w2 = T(2) * reach * T(1.00001);
    if (!(C.bmax_x - C.bmin_x >= w2) || !(C.bmax_y - C.bmin_y >= w2)) {
        St<T> a;
        a.px = apx; a.py = apy; a.vx = avx; a.vy = avy;
        wall_force_adj<T, SAT>(C, px, py, vx, vy, ra, dd, gx, gy, a);
        apx = a.px; apy = a.py; avx = a.vx; avy = a.vy;
        return;
    }
    if (bits & 1u) {
        const T pl = reach - (px - C.bmin_x), pr = reach - (C.bmax_x - px);
        T slope = T(1);
        if (SAT && C.max_overlap > T(0)) {
            const T th = m_tanh((pl > T(0) ? pl : pr) / C.max_overlap);
            slope = T(1) - th * th;
        }
        const T q = gx * inv_dd;
        apx -= C.k * slope * q;
        avx -= C.c * q;
    }
    if (bits & 2u) {
        const T pb = reach - (py - C.bmin_y), pt = reach - (C.bmax_y - py);
        T slope = T(1);
        if (SAT && C.max_overlap > T(0)) {
            const T th = m_tanh((pb > T(0) ? pb : pt) / C.max_overlap);
            slope = T(1) - th * th;
        }
        const T q = gy * inv_dd;
        apy -= C.k * slope * q;
        avy -= C.c * q;
    }
}

template <typename T, bool SAT>
__device__ __forceinline__ void wall_force_adj(const Cst<T> &C, T px, T py, T vx, T vy, T ra,
                                               T dd, T gx, T gy, St<T> &a)
{
    T reach = ra + C.margin, pen;
    pen = reach - (px - C.bmin_x);
    if (pen > T(0)) {
        T o = T(0), v = T(0);
        normal_coeff_adj<T, SAT>(C, pen, vx, dd, gx, o, v);
        a.px -= o;
        a.vx += v;
    }
    pen = reach - (C.bmax_x - px);
    if (pen > T(0)) {
        T o = T(0), v = T(0);
        normal_coeff_adj<T, SAT>(C, pen, -vx, dd, -gx, o, v);
        a.px += o;
        a.vx -= v;
    }
    pen = reach - (py - C.bmin_y);
    if (pen > T(0)) {
        T o = T(0), v = T(0);
        normal_coeff_adj<T, SAT>(C, pen, vy, dd, gy, o, v);
        a.py -= o;
        a.vy += v;
    }
    pen = reach - (C.bmax_y - py);
    if (pen > T(0)) {
        T o = T(0), v = T(0);
        normal_coeff_adj<T, SAT>(C, pen, -vy, dd, -gy, o, v);
        a.py += o;
        a.vy -= v;
    }
}

// --------------------------------------------------------------- obstacles

// box_force (swarp/core/collisions.py:174-260); reach = agent radius + margin
// (ca, sa) = cos / sin of the box angle.  Returns whether the contact branch ran, the
// test box_force_adj_cs repeats on the same operands.
template <typename T>
__device__ __forceinline__ bool box_force_cs(const Cst<T> &C, T px, T py, T vx, T vy, T cx0,
                                             T cy0, T ca, T sa, T hx, T hy, T reach, T dd,
                                             T vox, T voy, T om, T &fx, T &fy)
{
    T dx = px - cx0, dy = py - cy0;
    T lx = ca * dx + sa * dy;
    T ly = -sa * dx + ca * dy;
    T qx = m_abs(lx) - hx, qy = m_abs(ly) - hy;
    T ox = lx - wclamp(lx, -hx, hx), oy = ly - wclamp(ly, -hy, hy);
    T od2 = ox * ox + oy * oy;
    T s, nlx, nly;
    if (od2 > C.eps2) {
        s = m_sqrt(od2);
        nlx = ox / s;
        nly = oy / s;
    } else if (qx > qy) {
        s = qx;
        nlx = lx >= T(0) ? T(1) : T(-1);
        nly = T(0);
    } else {
        s = qy;
        nlx = T(0);
        nly = ly >= T(0) ? T(1) : T(-1);
    }
    fx = T(0);
    fy = T(0);
    T ov = reach - s;
    if (ov > T(0)) {
        T nx = ca * nlx - sa * nly, ny = sa * nlx + ca * nly;
        T spx = lx - s * nlx, spy = ly - s * nly;
        T rx = ca * spx - sa * spy, ry = sa * spx + ca * spy;
        T rvx = vx - (vox + -om * ry), rvy = vy - (voy + om * rx);
        T coef = normal_coeff(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
    return ov > T(0);
}

// box_force_cs with the damping denominator as a prepared divisor, in the exact fast
// arithmetic of pair_force's overload (same bits).
template <typename T>
__device__ __forceinline__ bool box_force_cs(const Cst<T> &C, T px, T py, T vx, T vy, T cx0,
                                             T cy0, T ca, T sa, T hx, T hy, T reach,
                                             const Dv<T> &dd, T vox, T voy, T om, T &fx, T &fy)
{
    T dx = px - cx0, dy = py - cy0;
    T lx = ca * dx + sa * dy;
    T ly = -sa * dx + ca * dy;
    T qx = m_abs(lx) - hx, qy = m_abs(ly) - hy;
    T ox = lx - wclamp(lx, -hx, hx), oy = ly - wclamp(ly, -hy, hy);
    T od2 = ox * ox + oy * oy;
    T s, nlx, nly;
    if (od2 > C.eps2) {
        s = sqrt_rn_big(od2);
        const Dv<T> ds = divisor(s, true);
        nlx = div_rn(ox, ds);
        nly = div_rn(oy, ds);
    } else if (qx > qy) {
        s = qx;
        nlx = lx >= T(0) ? T(1) : T(-1);
        nly = T(0);
    } else {
        s = qy;
        nlx = T(0);
        nly = ly >= T(0) ? T(1) : T(-1);
    }
    fx = T(0);
    fy = T(0);
    T ov = reach - s;
    if (ov > T(0)) {
        T nx = ca * nlx - sa * nly, ny = sa * nlx + ca * nly;
        T spx = lx - s * nlx, spy = ly - s * nly;
        T rx = ca * spx - sa * spy, ry = sa * spx + ca * spy;
        T rvx = vx - (vox + -om * ry), rvy = vy - (voy + om * rx);
        T coef = normal_coeff_r(C, ov, rvx * nx + rvy * ny, dd);
        fx = coef * nx;
        fy = coef * ny;
    }
    return ov > T(0);
}

template <typename T, typename DD>
__device__ __forceinline__ void box_force(const Cst<T> &C, T px, T py, T vx, T vy, T cx0, T cy0,
                                          T ang, T hx, T hy, T reach, const DD &dd, T vox, T voy,
                                          T om, T &fx, T &fy)
{
    box_force_cs(C, px, py, vx, vy, cx0, cy0, m_cos(ang), m_sin(ang), hx, hy, reach, dd, vox,
                 voy, om, fx, fy);
}

template <typename T>
__device__ __forceinline__ void box_force_adj_cs(const Cst<T> &C, T px, T py, T vx, T vy, T cx0,
                                                 T cy0, T ca, T sa, T hx, T hy, T reach, T dd,
                                                 T vox, T voy, T om, T gx, T gy, St<T> &a)
{
    T dx = px - cx0, dy = py - cy0;
    T lx = ca * dx + sa * dy;
    T ly = -sa * dx + ca * dy;
    T qx = m_abs(lx) - hx, qy = m_abs(ly) - hy;
    T ox = lx - wclamp(lx, -hx, hx), oy = ly - wclamp(ly, -hy, hy);
    T od2 = ox * ox + oy * oy;
    T s, nlx, nly;
    int face;
    if (od2 > C.eps2) {
        s = m_sqrt(od2);
        nlx = ox / s;
        nly = oy / s;
        face = 0;
    } else if (qx > qy) {
        s = qx;
        nlx = lx >= T(0) ? T(1) : T(-1);
        nly = T(0);
        face = 1;
    } else {
        s = qy;
        nlx = T(0);
        nly = ly >= T(0) ? T(1) : T(-1);
        face = 2;
    }
    T ov = reach - s;
    if (!(ov > T(0))) return;
    T nx = ca * nlx - sa * nly, ny = sa * nlx + ca * nly;
    T spx = lx - s * nlx, spy = ly - s * nly;
    T rx = ca * spx - sa * spy, ry = sa * spx + ca * spy;
    T rvx = vx - (vox + -om * ry), rvy = vy - (voy + om * rx);
    T vn = rvx * nx + rvy * ny;
    T coef = normal_coeff(C, ov, vn, dd);
    T a_ov = T(0), a_vn = T(0);
    normal_coeff_adj(C, ov, vn, dd, gx * nx + gy * ny, a_ov, a_vn);
    T anx = coef * gx + a_vn * rvx, any = coef * gy + a_vn * rvy;
    T arvx = a_vn * nx, arvy = a_vn * ny;
    a.vx += arvx;
    a.vy += arvy;
    // surface velocity: vs = vo + (-om*ry, om*rx), rel_v = v - vs
    T arx = -om * arvy, ary = om * arvx;
    T aspx = ca * arx + sa * ary, aspy = -sa * arx + ca * ary;
    T alx = aspx, aly = aspy;
    T as = -(aspx * nlx + aspy * nly) - a_ov;
    T anlx = -s * aspx + (ca * anx + sa * any);
    T anly = -s * aspy + (-sa * anx + ca * any);
    if (face == 0) {
        T aox = anlx / s, aoy = anly / s;
        as += -(anlx * nlx + anly * nly) / s;
        T h = as * T(0.5) / s;
        aox += T(2) * ox * h;
        aoy += T(2) * oy * h;
        alx += aox - wclamp_g(lx, -hx, hx, aox);
        aly += aoy - wclamp_g(ly, -hy, hy, aoy);
    } else if (face == 1) {
        alx += lx > T(0) ? as : -as;
    } else {
        aly += ly > T(0) ? as : -as;
    }
    a.px += ca * alx - sa * aly;
    a.py += sa * alx + ca * aly;
}

template <typename T>
__device__ __forceinline__ void box_force_adj(const Cst<T> &C, T px, T py, T vx, T vy, T cx0,
                                              T cy0, T ang, T hx, T hy, T reach, T dd, T vox,
                                              T voy, T om, T gx, T gy, St<T> &a)
{
    box_force_adj_cs(C, px, py, vx, vy, cx0, cy0, m_cos(ang), m_sin(ang), hx, hy, reach, dd, vox,
                     voy, om, gx, gy, a);
}

// cos / sin of obstacle j's angle: from the per-launch table when there is one.
template <typename T>
__device__ __forceinline__ void ob_trig(const Obs<T> &O, size_t j, int o, const T *cs, T &c, T &s)
{
    if (cs != nullptr) {
        c = cs[2 * o];
        s = cs[2 * o + 1];
    } else {
        const T ang = O.ang[j];
        c = m_cos(ang);
        s = m_sin(ang);
    }
}

// The broad phase of _obstacle_forces (swarp/core/collisions.py:717-720, with shape_bound
// :62-70 and bounds_apart :74-84): whether obstacle o's bounding disc comes within reach
// of an agent of radius ra at (px, py).  A NaN position is in reach (the comparison that
// would cull it fails), so a NaN state still propagates through the contact code.
// PT: the env's obstacle poses and bounding radii come from a per-launch table `pose`
// (OPOSE_W scalars per obstacle index: pos x, pos y, vel x, vel y, ang_vel, the bound
// below), the same values read once per launch.
constexpr int OPOSE_W = 8;

template <typename T> __device__ __forceinline__ T ob_bound(const Obs<T> &O, int o)
{
    const int st = O.type[o];
    const T ro = O.rad[o], hx = O.half[2 * o], hy = O.half[2 * o + 1];
    return st == 1 ? m_sqrt(hx * hx + hy * hy) : (st == 2 ? hx + ro : ro);
}

template <typename T, bool PT = false>
__device__ __forceinline__ bool obstacle_in_reach(const Cst<T> &C, const Obs<T> &O, size_t eN,
                                                  int o, T px, T py, T ra, const T *pose = nullptr)
{
    const size_t j = eN + o;
    const T cx = PT ? pose[OPOSE_W * o] : O.pos[2 * j];
    const T cy = PT ? pose[OPOSE_W * o + 1] : O.pos[2 * j + 1];
    T bound = PT ? pose[OPOSE_W * o + 5] : ob_bound(O, o);
    T lim = (ra + C.margin + bound) * T(1.0001) + T(1.0e-6);
    T ddx = px - cx, ddy = py - cy;
    return !(ddx * ddx + ddy * ddy > lim * lim);
}

// One obstacle on one agent (_obstacle_forces body, swarp/core/collisions.py:690-743).
// Returns whether its narrow phase took the contact branch: obstacle_force_adj on the
// same state contributes only then (elsewhere it adds zeros at most).
// `cs`: this env's obstacle angles as (cos, sin) pairs [N][2], computed once per launch
// (the angles do not change within one), or NULL to evaluate them here.
// DD: the damping denominator as a plain value or as a prepared divisor (Dv<T>, the
// exact fast arithmetic of the force overloads that take one); the same bits either way.
template <typename T, typename DD, bool PT = false>
__device__ __forceinline__ bool obstacle_force(const Cst<T> &C, const Obs<T> &O, size_t eN, int o,
                                               T px, T py, T vx, T vy, T ra, const DD &dd, T &fx,
                                               T &fy, const T *cs = nullptr,
                                               const T *pose = nullptr)
{
    fx = T(0);
    fy = T(0);
    if (!obstacle_in_reach<T, PT>(C, O, eN, o, px, py, ra, pose)) return false;
    const size_t j = eN + o;
    const T *pp = pose + OPOSE_W * o;
    const T cx = PT ? pp[0] : O.pos[2 * j], cy = PT ? pp[1] : O.pos[2 * j + 1];
    const int st = O.type[o];
    const T ro = O.rad[o], hx = O.half[2 * o], hy = O.half[2 * o + 1];
    const T vox = PT ? pp[2] : O.vel[2 * j], voy = PT ? pp[3] : O.vel[2 * j + 1];
    const T om = PT ? pp[4] : O.om[j];
    if (st == 1) {
        T ca, sa;
        ob_trig(O, j, o, cs, ca, sa);
        return box_force_cs(C, px, py, vx, vy, cx, cy, ca, sa, hx, hy, ra + C.margin, dd, vox,
                            voy, om, fx, fy);
    } else if (st == 2) {
        T ux, uy;
        ob_trig(O, j, o, cs, ux, uy);
        T t = wclamp((px - cx) * ux + (py - cy) * uy, -hx, hx);
        T qx = cx + t * ux, qy = cy + t * uy;
        T rx = qx - cx, ry = qy - cy;
        return pair_force(C, px - qx, py - qy, vx - (vox + -om * ry), vy - (voy + om * rx),
                          ra + ro + C.margin, dd, fx, fy);
    } else {
        return pair_force(C, px - cx, py - cy, vx - vox, vy - voy, ra + ro + C.margin, dd, fx,
                          fy);
    }
}

template <typename T>
__device__ __forceinline__ void obstacle_force_adj(const Cst<T> &C, const Obs<T> &O, size_t eN,
                                                   int o, T px, T py, T vx, T vy, T ra, T dd,
                                                   T gx, T gy, St<T> &a, const T *cs = nullptr)
{
    if (!obstacle_in_reach(C, O, eN, o, px, py, ra)) return;
    const size_t j = eN + o;
    const T cx = O.pos[2 * j], cy = O.pos[2 * j + 1];
    const int st = O.type[o];
    const T ro = O.rad[o], hx = O.half[2 * o], hy = O.half[2 * o + 1];
    const T vox = O.vel[2 * j], voy = O.vel[2 * j + 1], om = O.om[j];
    if (st == 1) {
        T ca, sa;
        ob_trig(O, j, o, cs, ca, sa);
        box_force_adj_cs(C, px, py, vx, vy, cx, cy, ca, sa, hx, hy, ra + C.margin, dd, vox, voy,
                         om, gx, gy, a);
    } else if (st == 2) {
        T ux, uy;
        ob_trig(O, j, o, cs, ux, uy);
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
        // closest point q(p): d = p - q, rel_v through the lever r = q - c
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
    }
}

// ------------------------------------------------------------- integration

// Inset of the position clamp along x and y (clamp_footprint, swarp/dynamics/kernels.py:
// 79-99): a disc by its radius; under the footprint clamp a box at heading th by its
// support extents hx |cos| + hy |sin| and hx |sin| + hy |cos|.
template <typename T>
__device__ __forceinline__ void clamp_insets(const Cst<T> &C, const Prm<T> &P, T th, T &ex, T &ey)
{
    ex = P.radius;
    ey = P.radius;
    if (C.clamp == 2 && P.shape > T(0.5)) {
        const T ca = m_abs(m_cos(th)), sa = m_abs(m_sin(th));
        ex = P.hx * ca + P.hy * sa;
        ey = P.hx * sa + P.hy * ca;
    }
}

// The position clamp of a substep's output (kernels.py:395-403).
template <typename T>
__device__ __forceinline__ void clamp_position(const Cst<T> &C, const Prm<T> &P, T th, T &px, T &py)
{
    T ex, ey;
    clamp_insets(C, P, th, ex, ey);
    px = wclamp(px, C.bmin_x + ex, C.bmax_x - ex);
    py = wclamp(py, C.bmin_y + ey, C.bmax_y - ey);
}

// Reverse of clamp_position at the unclamped output (px, py, th): rewrites the position
// adjoint (clamp(x, a, b): x < a -> a, x > b -> b, else x) and adds the heading's share,
// through the footprint's bounds, to gth.
template <typename T>
__device__ __forceinline__ void clamp_position_adj(const Cst<T> &C, const Prm<T> &P, T px, T py,
                                                   T th, T &gpx, T &gpy, T &gth)
{
    T ex, ey;
    clamp_insets(C, P, th, ex, ey);
    const T lox = C.bmin_x + ex, hix = C.bmax_x - ex, loy = C.bmin_y + ey, hiy = C.bmax_y - ey;
    T aex = T(0), aey = T(0);
    if (px < lox) aex += gpx;
    else if (px > hix) aex -= gpx;
    if (py < loy) aey += gpy;
    else if (py > hiy) aey -= gpy;
    gpx = wclamp_g(px, lox, hix, gpx);
    gpy = wclamp_g(py, loy, hiy, gpy);
    if (C.clamp == 2 && P.shape > T(0.5) && (aex != T(0) || aey != T(0))) {
        const T c = m_cos(th), s = m_sin(th);
        const T dca = c < T(0) ? s : -s;  // d|cos th| / dth
        const T dsa = s < T(0) ? -c : c;  // d|sin th| / dth
        gth += aex * (P.hx * dca + P.hy * dsa) + aey * (P.hx * dsa + P.hy * dca);
    }
}

// clamp_norm (swarp/dynamics/kernels.py:68-71)
template <typename T>
__device__ __forceinline__ void clamp_norm(T x, T y, T lim, T &ox, T &oy)
{
    T sc = lim / wmax(m_sqrt(x * x + y * y), lim);
    ox = x * sc;
    oy = y * sc;
}

template <typename T>
__device__ __forceinline__ void clamp_norm_adj(T x, T y, T lim, T gx, T gy, T &ax, T &ay)
{
    T len = m_sqrt(x * x + y * y);
    T m = wmax(len, lim);
    T sc = lim / m;
    T rx = gx * sc, ry = gy * sc;
    if (len > lim) {
        T am = -(gx * x + gy * y) * lim / (m * m);
        rx += am * x / len;
        ry += am * y / len;
    }
    ax += rx;
    ay += ry;
}

__device__ __forceinline__ float m_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ double m_rcp(double x) { return 1.0 / x; }

// clamp_norm_adj with reciprocal estimates in place of the correctly rounded divisions:
// the branch (len > lim) is decided on the exact length, as the forward pass decided it;
// the adjoint values only need to be accurate (a few ulp in float32, exact in float64).
template <typename T>
__device__ __forceinline__ void clamp_norm_adj_rcp(T x, T y, T lim, T gx, T gy, T &ax, T &ay)
{
    const T len = m_sqrt(x * x + y * y);
    if (len > lim) {
        const T il = m_rcp(len);
        const T sc = lim * il;
        const T am = -(gx * x + gy * y) * sc * il;
        ax += gx * sc + am * x * il;
        ay += gy * sc + am * y * il;
    } else {
        ax += gx;
        ay += gy;
    }
}

// ------------------------------------------------------------------------------ RK4

// o = x + k * h over the 16 state fields.
template <typename T>
__device__ __forceinline__ void st_axpy(const St<T> &x, const St<T> &k, T h, St<T> &o)
{
    o.px = x.px + k.px * h; o.py = x.py + k.py * h; o.th = x.th + k.th * h;
    o.vx = x.vx + k.vx * h; o.vy = x.vy + k.vy * h; o.s = x.s + k.s * h; o.w = x.w + k.w * h;
    o.z = x.z + k.z * h; o.vz = x.vz + k.vz * h;
    o.qx = x.qx + k.qx * h; o.qy = x.qy + k.qy * h; o.qz = x.qz + k.qz * h; o.qw = x.qw + k.qw * h;
    o.bx = x.bx + k.bx * h; o.by = x.by + k.by * h; o.bz = x.bz + k.bz * h;
}

// _deriv (swarp/dynamics/kernels.py:416-517): the state derivative with the actions held
// constant.  Holonomic integrates (pos, vel), diff-drive (pos, theta, speed, ang_vel), the
// bicycle (pos, theta, speed), the drone (pos, vel, z, vz, attitude, body_rates; _drone_rates
// :129-163, _quat_deriv :117-126); every other field has rate 0.
template <typename T, bool DRONE>
__device__ __forceinline__ void rk_deriv(const Prm<T> &P, const St<T> &x, const T (&a)[4], St<T> &k)
{
    st_zero(k);
    if (DRONE && P.tag == 3) {
        const T z0 = T(0), h = T(0.5);
        T f0 = wclamp(a[0], z0, P.thrust_max), f1 = wclamp(a[1], z0, P.thrust_max);
        T f2 = wclamp(a[2], z0, P.thrust_max), f3 = wclamp(a[3], z0, P.thrust_max);
        T thr = f0 + f1 + f2 + f3;
        T vx3 = T(0), vy3 = T(0), vz3 = thr;
        T c1x = x.qy * vz3 - x.qz * vy3, c1y = x.qz * vx3 - x.qx * vz3, c1z = x.qx * vy3 - x.qy * vx3;
        T tx = T(2) * c1x, ty = T(2) * c1y, tz = T(2) * c1z;
        T c2x = x.qy * tz - x.qz * ty, c2y = x.qz * tx - x.qx * tz, c2z = x.qx * ty - x.qy * tx;
        T fwx = vx3 + x.qw * tx + c2x, fwy = vy3 + x.qw * ty + c2y, fwz = vz3 + x.qw * tz + c2z;
        k.px = x.vx;
        k.py = x.vy;
        k.vx = fwx / P.mass - z0;
        k.vy = fwy / P.mass - z0;
        k.vz = fwz / P.mass - P.gravity;
        k.z = x.vz;
        k.bx = (P.arm * (f1 - f3) - (P.izz - P.iyy) * x.by * x.bz) / P.ixx;
        k.by = (P.arm * (f2 - f0) - (P.ixx - P.izz) * x.bz * x.bx) / P.iyy;
        k.bz = (P.kappa * (f0 - f1 + f2 - f3) - (P.iyy - P.ixx) * x.bx * x.by) / P.izz;
        k.qx = h * (x.qw * x.bx + x.qy * x.bz - x.qz * x.by);
        k.qy = h * (x.qw * x.by - x.qx * x.bz + x.qz * x.bx);
        k.qz = h * (x.qw * x.bz + x.qx * x.by - x.qy * x.bx);
        k.qw = h * (-x.qx * x.bx - x.qy * x.by - x.qz * x.bz);
    } else if (P.tag == 0) {
        k.px = x.vx;
        k.py = x.vy;
        if (P.mode != 0) clamp_norm(a[0], a[1], P.max_accel, k.vx, k.vy);
    } else if (P.tag == 1) {
        k.px = x.s * m_cos(x.th);
        k.py = x.s * m_sin(x.th);
        k.th = x.w;
        if (P.mode != 0) {
            k.s = wclamp(a[0], -P.max_accel, P.max_accel);
            k.w = wclamp(a[1], -P.max_ang_accel, P.max_ang_accel);
        }
    } else if (P.tag == 2) {
        T wb = P.l_f + P.l_r;
        T del = wclamp(a[1], -P.max_steer, P.max_steer);
        T beta = m_atan(m_tan(del) * P.l_r / wb);
        k.px = x.s * m_cos(x.th + beta);
        k.py = x.s * m_sin(x.th + beta);
        k.th = x.s / wb * m_cos(beta) * m_tan(del);
        k.s = wclamp(a[0], -P.max_accel, P.max_accel);
    }
}

// Reverse of rk_deriv: gk = adjoint of k; accumulates into gx and ga.
template <typename T, bool DRONE>
__device__ __forceinline__ void rk_deriv_adj(const Prm<T> &P, const St<T> &x, const T (&a)[4],
                                             const St<T> &gk, St<T> &gx, T (&ga)[4])
{
    if (DRONE && P.tag == 3) {
        const T z0 = T(0), h = T(0.5);
        T f0 = wclamp(a[0], z0, P.thrust_max), f1 = wclamp(a[1], z0, P.thrust_max);
        T f2 = wclamp(a[2], z0, P.thrust_max), f3 = wclamp(a[3], z0, P.thrust_max);
        T thr = f0 + f1 + f2 + f3;
        T qx = x.qx, qy = x.qy, qz = x.qz, qw = x.qw, bx = x.bx, by = x.by, bz = x.bz;
        T vx3 = T(0), vy3 = T(0), vz3 = thr;
        T tx = T(2) * (qy * vz3 - qz * vy3), ty = T(2) * (qz * vx3 - qx * vz3);
        T tz = T(2) * (qx * vy3 - qy * vx3);
        gx.vx += gk.px;
        gx.vy += gk.py;
        gx.vz += gk.z;
        // fw = v3 + qw t + u x t ; acc = fw / m
        T gfx = gk.vx / P.mass, gfy = gk.vy / P.mass, gfz = gk.vz / P.mass;
        T gqx = T(0), gqy = T(0), gqz = T(0), gqw = T(0);
        gqw += gfx * tx + gfy * ty + gfz * tz;
        T gtx = qw * gfx + (gfy * qz - gfz * qy);
        T gty = qw * gfy + (gfz * qx - gfx * qz);
        T gtz = qw * gfz + (gfx * qy - gfy * qx);
        gqx += ty * gfz - tz * gfy;
        gqy += tz * gfx - tx * gfz;
        gqz += tx * gfy - ty * gfx;
        // t = 2 (u x v3)
        T g1x = T(2) * gtx, g1y = T(2) * gty, g1z = T(2) * gtz;
        gqx += vy3 * g1z - vz3 * g1y;
        gqy += vz3 * g1x - vx3 * g1z;
        gqz += vx3 * g1y - vy3 * g1x;
        T gthr = gfz + (g1x * qy - g1y * qx);
        // body-rate derivative (Euler's equation)
        T gax = gk.bx / P.ixx, gay = gk.by / P.iyy, gaz = gk.bz / P.izz;
        T gbx = T(0), gby = T(0), gbz = T(0);
        gby -= (P.izz - P.iyy) * bz * gax;
        gbz -= (P.izz - P.iyy) * by * gax;
        gbz -= (P.ixx - P.izz) * bx * gay;
        gbx -= (P.ixx - P.izz) * bz * gay;
        gbx -= (P.iyy - P.ixx) * by * gaz;
        gby -= (P.iyy - P.ixx) * bx * gaz;
        T gf0 = gthr - P.arm * gay + P.kappa * gaz;
        T gf1 = gthr + P.arm * gax - P.kappa * gaz;
        T gf2 = gthr + P.arm * gay + P.kappa * gaz;
        T gf3 = gthr - P.arm * gax - P.kappa * gaz;
        // quaternion derivative 0.5 q (x) (b, 0)
        T Dx = h * gk.qx, Dy = h * gk.qy, Dz = h * gk.qz, Dw = h * gk.qw;
        gqw += Dx * bx + Dy * by + Dz * bz;
        gqx += -Dy * bz + Dz * by - Dw * bx;
        gqy += Dx * bz - Dz * bx - Dw * by;
        gqz += -Dx * by + Dy * bx - Dw * bz;
        gbx += Dx * qw + Dy * qz - Dz * qy - Dw * qx;
        gby += -Dx * qz + Dy * qw + Dz * qx - Dw * qy;
        gbz += Dx * qy - Dy * qx + Dz * qw - Dw * qz;
        gx.qx += gqx; gx.qy += gqy; gx.qz += gqz; gx.qw += gqw;
        gx.bx += gbx; gx.by += gby; gx.bz += gbz;
        ga[0] += wclamp_g(a[0], z0, P.thrust_max, gf0);
        ga[1] += wclamp_g(a[1], z0, P.thrust_max, gf1);
        ga[2] += wclamp_g(a[2], z0, P.thrust_max, gf2);
        ga[3] += wclamp_g(a[3], z0, P.thrust_max, gf3);
    } else if (P.tag == 0) {
        gx.vx += gk.px;
        gx.vy += gk.py;
        if (P.mode != 0) clamp_norm_adj(a[0], a[1], P.max_accel, gk.vx, gk.vy, ga[0], ga[1]);
    } else if (P.tag == 1) {
        T c = m_cos(x.th), sn = m_sin(x.th);
        gx.s += gk.px * c + gk.py * sn;
        gx.th += -gk.px * x.s * sn + gk.py * x.s * c;
        gx.w += gk.th;
        if (P.mode != 0) {
            ga[0] += wclamp_g(a[0], -P.max_accel, P.max_accel, gk.s);
            ga[1] += wclamp_g(a[1], -P.max_ang_accel, P.max_ang_accel, gk.w);
        }
    } else if (P.tag == 2) {
        T wb = P.l_f + P.l_r;
        T del = wclamp(a[1], -P.max_steer, P.max_steer);
        T td = m_tan(del);
        T u = td * P.l_r / wb;
        T beta = m_atan(u);
        T cb = m_cos(beta), sb = m_sin(beta);
        T c = m_cos(x.th + beta), sn = m_sin(x.th + beta);
        gx.s += gk.px * c + gk.py * sn + gk.th * (cb * td / wb);
        T gang = -gk.px * x.s * sn + gk.py * x.s * c;  // d / d(th + beta)
        gx.th += gang;
        T gbeta = gang + gk.th * (x.s / wb * (-sb) * td);
        T gdel = gk.th * (x.s / wb * cb * (T(1) + td * td))
                 + gbeta / (T(1) + u * u) * (T(1) + td * td) * P.l_r / wb;
        ga[1] += wclamp_g(a[1], -P.max_steer, P.max_steer, gdel);
        ga[0] += wclamp_g(a[0], -P.max_accel, P.max_accel, gk.s);
    }
}

// The stage states x2..x4 (x1 = x0) and the combine x0 + (k1 + 2 k2 + 2 k3 + k4) dt / 6
// (swarp/dynamics/kernels.py:584-738).  x0 is the input with the velocity-control command
// written into the velocity-level state (:588-595).
template <typename T> struct RkSt {
    St<T> x0, x2, x3, x4, xi;
};

template <typename T, bool DRONE>
__device__ __forceinline__ void rk_stages(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                          const T (&a)[4], RkSt<T> &R)
{
    const T dt = C.sub_dt, two = T(2);
    const T dt2 = dt * T(0.5), sixth = dt / T(6);
    R.x0 = in;
    if (P.mode == 0) {
        if (P.tag == 0) {
            clamp_norm(a[0], a[1], P.max_speed, R.x0.vx, R.x0.vy);
        } else if (P.tag == 1) {
            R.x0.s = wclamp(a[0], -P.max_speed, P.max_speed);
            R.x0.w = wclamp(a[1], -P.max_ang_vel, P.max_ang_vel);
        }
    }
    St<T> k1, k2, k3, k4;
    rk_deriv<T, DRONE>(P, R.x0, a, k1);
    st_axpy(R.x0, k1, dt2, R.x2);
    rk_deriv<T, DRONE>(P, R.x2, a, k2);
    st_axpy(R.x0, k2, dt2, R.x3);
    rk_deriv<T, DRONE>(P, R.x3, a, k3);
    st_axpy(R.x0, k3, dt, R.x4);
    rk_deriv<T, DRONE>(P, R.x4, a, k4);
#define SWARP_RK_COMB(f) R.xi.f = R.x0.f + (k1.f + k2.f * two + k3.f * two + k4.f) * sixth
    SWARP_RK_COMB(px); SWARP_RK_COMB(py); SWARP_RK_COMB(th); SWARP_RK_COMB(vx);
    SWARP_RK_COMB(vy); SWARP_RK_COMB(s); SWARP_RK_COMB(w); SWARP_RK_COMB(z);
    SWARP_RK_COMB(vz); SWARP_RK_COMB(qx); SWARP_RK_COMB(qy); SWARP_RK_COMB(qz);
    SWARP_RK_COMB(qw); SWARP_RK_COMB(bx); SWARP_RK_COMB(by); SWARP_RK_COMB(bz);
#undef SWARP_RK_COMB
}

// RK4 substep of one agent: _integrate_rk4 (swarp/dynamics/kernels.py:520-793).  Limits on
// the combined result only, the contact force as dv = F * (dt / m) after the combine, the
// attitude renormalised.
template <typename T, bool DRONE>
__device__ __forceinline__ void integrate_rk4(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                              const T (&a)[4], T Fx, T Fy, St<T> &o)
{
    const T dt = C.sub_dt;
    RkSt<T> R;
    rk_stages<T, DRONE>(C, P, in, a, R);
    const T dfx = Fx * (dt / P.mass), dfy = Fy * (dt / P.mass);
    o = in;
    T pnx = R.xi.px + dfx * dt, pny = R.xi.py + dfy * dt;
    if (DRONE && P.tag == 3) {
        o.vx = R.xi.vx + dfx;
        o.vy = R.xi.vy + dfy;
        o.z = R.xi.z;
        o.vz = R.xi.vz;
        T l = m_sqrt(R.xi.qx * R.xi.qx + R.xi.qy * R.xi.qy + R.xi.qz * R.xi.qz + R.xi.qw * R.xi.qw);
        if (l > T(0)) {
            o.qx = R.xi.qx / l; o.qy = R.xi.qy / l; o.qz = R.xi.qz / l; o.qw = R.xi.qw / l;
        } else {
            o.qx = T(0); o.qy = T(0); o.qz = T(0); o.qw = T(1);
        }
        o.bx = R.xi.bx; o.by = R.xi.by; o.bz = R.xi.bz;
    } else if (P.tag == 0) {
        T vx, vy;
        clamp_norm(R.xi.vx, R.xi.vy, P.max_speed, vx, vy);
        vx = vx + dfx;
        vy = vy + dfy;
        o.vx = vx; o.vy = vy;
        o.s = m_sqrt(vx * vx + vy * vy);
        o.w = T(0);
    } else if (P.tag == 1) {
        T so = wclamp(R.xi.s, -P.max_speed, P.max_speed);
        T th = R.xi.th;
        o.th = th;
        o.vx = so * m_cos(th) + dfx;
        o.vy = so * m_sin(th) + dfy;
        o.s = so;
        o.w = wclamp(R.xi.w, -P.max_ang_vel, P.max_ang_vel);
    } else if (P.tag == 2) {
        T so = wclamp(R.xi.s, P.min_speed, P.max_speed);
        T th = R.xi.th;
        T del = wclamp(a[1], -P.max_steer, P.max_steer);
        T wb = P.l_f + P.l_r;
        T beta = m_atan(m_tan(del) * P.l_r / wb);
        o.w = so / wb * m_cos(beta) * m_tan(del);
        o.th = th;
        o.vx = so * m_cos(th + beta) + dfx;
        o.vy = so * m_sin(th + beta) + dfy;
        o.s = so;
    } else {
        return;
    }
    if (C.clamp) clamp_position(C, P, o.th, pnx, pny);
    o.px = pnx;
    o.py = pny;
}

// Reverse of integrate_rk4 with integrate_adj's contract: overwrites gi (adjoint of the
// input) and gF, accumulates ga.  The stages are recomputed from the input.
template <typename T, bool DRONE>
__device__ __forceinline__ void integrate_rk4_adj(const Cst<T> &C, const Prm<T> &P,
                                                  const St<T> &in, const T (&a)[4], T Fx, T Fy,
                                                  const St<T> &g, St<T> &gi, T (&ga)[4], T &gFx,
                                                  T &gFy)
{
    const T dt = C.sub_dt, two = T(2);
    const T dt2 = dt * T(0.5), sixth = dt / T(6);
    gFx = T(0);
    gFy = T(0);
    if (P.tag > 3 || (!DRONE && P.tag == 3)) {
        gi = g;
        return;
    }
    RkSt<T> R;
    rk_stages<T, DRONE>(C, P, in, a, R);
    const T dfx = Fx * (dt / P.mass), dfy = Fy * (dt / P.mass);
    T gpx = g.px, gpy = g.py;
    St<T> gxi;
    st_zero(gxi);
    gxi.px = gpx;
    gxi.py = gpy;
    T gdfx = gpx * dt + g.vx, gdfy = gpy * dt + g.vy;
    T pass_th = T(0), pass_s = T(0), pass_w = T(0);
    if (DRONE && P.tag == 3) {
        gxi.vx = g.vx;
        gxi.vy = g.vy;
        gxi.z = g.z;
        gxi.vz = g.vz;
        gxi.bx = g.bx; gxi.by = g.by; gxi.bz = g.bz;
        T l = m_sqrt(R.xi.qx * R.xi.qx + R.xi.qy * R.xi.qy + R.xi.qz * R.xi.qz + R.xi.qw * R.xi.qw);
        if (l > T(0)) {
            T nx = R.xi.qx / l, ny = R.xi.qy / l, nz = R.xi.qz / l, nw = R.xi.qw / l;
            T dq = g.qx * nx + g.qy * ny + g.qz * nz + g.qw * nw;
            gxi.qx = (g.qx - nx * dq) / l;
            gxi.qy = (g.qy - ny * dq) / l;
            gxi.qz = (g.qz - nz * dq) / l;
            gxi.qw = (g.qw - nw * dq) / l;
        }
        pass_th = g.th;
        pass_s = g.s;
        pass_w = g.w;
    } else if (P.tag == 0) {
        T vx, vy;
        clamp_norm(R.xi.vx, R.xi.vy, P.max_speed, vx, vy);
        vx = vx + dfx;
        vy = vy + dfy;
        T gvx = g.vx, gvy = g.vy;
        T sp = m_sqrt(vx * vx + vy * vy);
        if (sp > T(0)) {
            gvx += g.s * vx / sp;
            gvy += g.s * vy / sp;
            gdfx += g.s * vx / sp;
            gdfy += g.s * vy / sp;
        }
        clamp_norm_adj(R.xi.vx, R.xi.vy, P.max_speed, gvx, gvy, gxi.vx, gxi.vy);
        pass_th = g.th;
    } else if (P.tag == 1) {
        T so = wclamp(R.xi.s, -P.max_speed, P.max_speed);
        T th = R.xi.th, c = m_cos(th), sn = m_sin(th);
        T gso = g.s + g.vx * c + g.vy * sn;
        gxi.th = g.th - g.vx * so * sn + g.vy * so * c;
        gxi.s = wclamp_g(R.xi.s, -P.max_speed, P.max_speed, gso);
        gxi.w = wclamp_g(R.xi.w, -P.max_ang_vel, P.max_ang_vel, g.w);
    } else {
        T so = wclamp(R.xi.s, P.min_speed, P.max_speed);
        T th = R.xi.th;
        T del = wclamp(a[1], -P.max_steer, P.max_steer);
        T wb = P.l_f + P.l_r;
        T td = m_tan(del), u = td * P.l_r / wb;
        T beta = m_atan(u), cb = m_cos(beta), sb = m_sin(beta);
        T c = m_cos(th + beta), sn = m_sin(th + beta);
        T gso = g.s + g.w * (cb * td / wb) + g.vx * c + g.vy * sn;
        T gang = -g.vx * so * sn + g.vy * so * c;
        gxi.th = g.th + gang;
        T gbeta = gang + g.w * (so / wb * (-sb) * td);
        T gdel = g.w * (so / wb * cb * (T(1) + td * td))
                 + gbeta / (T(1) + u * u) * (T(1) + td * td) * P.l_r / wb;
        ga[1] += wclamp_g(a[1], -P.max_steer, P.max_steer, gdel);
        gxi.s = wclamp_g(R.xi.s, P.min_speed, P.max_speed, gso);
    }
    gFx = gdfx * (dt / P.mass);
    gFy = gdfy * (dt / P.mass);
    // the combine and the stages, in reverse
    St<T> gx = gxi, gk1, gk2, gk3, gs, z;
    st_zero(z);
    st_axpy(z, gxi, sixth, gk1);
    st_axpy(z, gxi, two * sixth, gk2);
    gk3 = gk2;
    st_zero(gs);
    rk_deriv_adj<T, DRONE>(P, R.x4, a, gk1, gs, ga);  // k4 carries gk1's weight
    st_axpy(gx, gs, T(1), gx);
    st_axpy(gk3, gs, dt, gk3);
    st_zero(gs);
    rk_deriv_adj<T, DRONE>(P, R.x3, a, gk3, gs, ga);
    st_axpy(gx, gs, T(1), gx);
    st_axpy(gk2, gs, dt2, gk2);
    st_zero(gs);
    rk_deriv_adj<T, DRONE>(P, R.x2, a, gk2, gs, ga);
    st_axpy(gx, gs, T(1), gx);
    st_axpy(gk1, gs, dt2, gk1);
    st_zero(gs);
    rk_deriv_adj<T, DRONE>(P, R.x0, a, gk1, gs, ga);
    st_axpy(gx, gs, T(1), gx);
    // velocity control: the commanded velocity-level state replaces the input's
    if (P.mode == 0 && P.tag == 0) {
        clamp_norm_adj(a[0], a[1], P.max_speed, gx.vx, gx.vy, ga[0], ga[1]);
        gx.vx = gx.vy = T(0);
    } else if (P.mode == 0 && P.tag == 1) {
        ga[0] += wclamp_g(a[0], -P.max_speed, P.max_speed, gx.s);
        ga[1] += wclamp_g(a[1], -P.max_ang_vel, P.max_ang_vel, gx.w);
        gx.s = gx.w = T(0);
    }
    gi = gx;
    gi.th += pass_th;
    gi.s += pass_s;
    gi.w += pass_w;
    // fields no 2-D model integrates pass their adjoint through
    if (!(DRONE && P.tag == 3)) {
        gi.z += g.z; gi.vz += g.vz;
        gi.qx += g.qx; gi.qy += g.qy; gi.qz += g.qz; gi.qw += g.qw;
        gi.bx += g.bx; gi.by += g.by; gi.bz += g.bz;
    }
}

// The drone branch of the Euler substep (_integrate_agent TAG_DRONE,
// swarp/dynamics/kernels.py:349-369): "+" quadrotor, rotor clamp, body rates, vz, planar
// velocity (+ contact dv), attitude q = normalize(q + qdot(br_new) dt), position, z.
// Writes the fields it steps into o (and the new planar position into pnx / pny).
template <typename T, typename Ar>
__device__ __forceinline__ void drone_euler(const Prm<T> &P, const St<T> &in, const T (&a)[4],
                                            T dt, T dvx, T dvy, Ar &&A, St<T> &o, T &pnx,
                                            T &pny)
{
    const T z0 = T(0);
    T f0 = wclamp(a[0], z0, P.thrust_max), f1 = wclamp(a[1], z0, P.thrust_max);
    T f2 = wclamp(a[2], z0, P.thrust_max), f3 = wclamp(a[3], z0, P.thrust_max);
    T thr = f0 + f1 + f2 + f3;
    const auto dm = A.prep(P.mass), dix = A.prep(P.ixx), diy = A.prep(P.iyy), diz = A.prep(P.izz);
    // _quat_rotate_vec(q, (0,0,thrust)) written generically (kernels.py:108-114)
    T vx3 = T(0), vy3 = T(0), vz3 = thr;
    T c1x = in.qy * vz3 - in.qz * vy3, c1y = in.qz * vx3 - in.qx * vz3;
    T c1z = in.qx * vy3 - in.qy * vx3;
    T tx = T(2) * c1x, ty = T(2) * c1y, tz = T(2) * c1z;
    T c2x = in.qy * tz - in.qz * ty, c2y = in.qz * tx - in.qx * tz, c2z = in.qx * ty - in.qy * tx;
    T fwx = vx3 + in.qw * tx + c2x, fwy = vy3 + in.qw * ty + c2y, fwz = vz3 + in.qw * tz + c2z;
    T accx = A.div(fwx, dm) - z0, accy = A.div(fwy, dm) - z0, accz = A.div(fwz, dm) - P.gravity;
    T tqx = P.arm * (f1 - f3), tqy = P.arm * (f2 - f0), tqz = P.kappa * (f0 - f1 + f2 - f3);
    T nbx = in.bx + A.div(tqx - (P.izz - P.iyy) * in.by * in.bz, dix) * dt;
    T nby = in.by + A.div(tqy - (P.ixx - P.izz) * in.bz * in.bx, diy) * dt;
    T nbz = in.bz + A.div(tqz - (P.iyy - P.ixx) * in.bx * in.by, diz) * dt;
    T nvz = in.vz + accz * dt;
    T vxx = in.vx + accx * dt + dvx, vxy = in.vy + accy * dt + dvy;
    const T h = T(0.5);
    T dqx = h * (in.qw * nbx + in.qy * nbz - in.qz * nby);
    T dqy = h * (in.qw * nby - in.qx * nbz + in.qz * nbx);
    T dqz = h * (in.qw * nbz + in.qx * nby - in.qy * nbx);
    T dqw = h * (-in.qx * nbx - in.qy * nby - in.qz * nbz);
    T ux = in.qx + dqx * dt, uy = in.qy + dqy * dt, uz = in.qz + dqz * dt, uw = in.qw + dqw * dt;
    T l = A.sqrt(ux * ux + uy * uy + uz * uz + uw * uw);
    if (l > T(0)) {
        const auto dl = A.prep(l);
        o.qx = A.div(ux, dl); o.qy = A.div(uy, dl); o.qz = A.div(uz, dl); o.qw = A.div(uw, dl);
    } else {
        o.qx = T(0); o.qy = T(0); o.qz = T(0); o.qw = T(1);
    }
    pnx = in.px + vxx * dt;
    pny = in.py + vxy * dt;
    o.z = in.z + nvz * dt;
    o.vz = nvz;
    o.bx = nbx; o.by = nby; o.bz = nbz;
    o.vx = vxx; o.vy = vxy;
}

// Semi-implicit Euler substep of one agent: _integrate_agent + _step_2d
// (swarp/dynamics/kernels.py:194-413).  `o` receives the new state.
template <typename T, bool DRONE>
__device__ __forceinline__ void integrate_core(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                               const T (&a)[4], T Fx, T Fy, St<T> &o)
{
    if (C.rk4) {
        integrate_rk4<T, DRONE>(C, P, in, a, Fx, Fy, o);
        return;
    }
    const T dt = C.sub_dt;
    const T dtm = dt / P.mass;
    const T dvx = Fx * dtm, dvy = Fy * dtm;
    o = in;
    T pnx = in.px, pny = in.py;
    if (DRONE && P.tag == 3) {
        if constexpr (sizeof(T) == 4) {
            ArithPrep A;
            drone_euler(P, in, a, dt, dvx, dvy, A, o, pnx, pny);
            if (__builtin_expect(A.bad, 0)) drone_euler(P, in, a, dt, dvx, dvy, ArithIEEE<T>(), o, pnx, pny);
        } else {
            drone_euler(P, in, a, dt, dvx, dvy, ArithIEEE<T>(), o, pnx, pny);
        }
    } else if (P.tag == 0) {
        T vnx, vny;
        if (P.mode == 0) {
            clamp_norm(a[0], a[1], P.max_speed, vnx, vny);
        } else {
            T acx, acy;
            clamp_norm(a[0], a[1], P.max_accel, acx, acy);
            clamp_norm(in.vx + acx * dt, in.vy + acy * dt, P.max_speed, vnx, vny);
        }
        vnx = vnx + dvx;
        vny = vny + dvy;
        pnx = in.px + vnx * dt;
        pny = in.py + vny * dt;
        o.vx = vnx; o.vy = vny;
        o.s = m_sqrt(vnx * vnx + vny * vny);
        o.w = T(0);
    } else if (P.tag == 1) {
        T sn, wn;
        if (P.mode == 0) {
            sn = wclamp(a[0], -P.max_speed, P.max_speed);
            wn = wclamp(a[1], -P.max_ang_vel, P.max_ang_vel);
        } else {
            T acc = wclamp(a[0], -P.max_accel, P.max_accel);
            T alp = wclamp(a[1], -P.max_ang_accel, P.max_ang_accel);
            sn = wclamp(in.s + acc * dt, -P.max_speed, P.max_speed);
            wn = wclamp(in.w + alp * dt, -P.max_ang_vel, P.max_ang_vel);
        }
        T vtx = sn * m_cos(in.th) + dvx, vty = sn * m_sin(in.th) + dvy;
        pnx = in.px + vtx * dt;
        pny = in.py + vty * dt;
        o.th = in.th + wn * dt;
        o.vx = vtx; o.vy = vty;
        o.s = sn;
        o.w = wn;
    } else if (P.tag == 2) {
        T acc = wclamp(a[0], -P.max_accel, P.max_accel);
        T del = wclamp(a[1], -P.max_steer, P.max_steer);
        T sn = wclamp(in.s + acc * dt, P.min_speed, P.max_speed);
        T wb = P.l_f + P.l_r;
        T beta = m_atan(m_tan(del) * P.l_r / wb);
        T vtx = sn * m_cos(in.th + beta) + dvx, vty = sn * m_sin(in.th + beta) + dvy;
        T wn = sn / wb * m_cos(beta) * m_tan(del);
        pnx = in.px + vtx * dt;
        pny = in.py + vty * dt;
        o.th = in.th + wn * dt;
        o.vx = vtx; o.vy = vty;
        o.s = sn;
        o.w = wn;
    }
    if (C.clamp) clamp_position(C, P, o.th, pnx, pny);
    o.px = pnx;
    o.py = pny;
}

// servo_command (swarp/dynamics/kernels.py:165-191): ControlMode.SERVO as the VELOCITY
// command it amounts to this substep -- the drive's speed and turn rate move toward the
// gained command by at most max_accel dt and max_ang_accel dt.
template <typename T>
__device__ __forceinline__ void servo_command(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                              const T (&a)[4], T (&as)[4])
{
    const T dt = C.sub_dt;
    const T tv = wclamp(a[0], -P.max_speed, P.max_speed) * P.gain_v;
    const T tw = wclamp(a[1], -P.max_ang_vel, P.max_ang_vel) * P.gain_w;
    const T dv = P.max_accel * dt, dw = P.max_ang_accel * dt;
    as[0] = in.s + wclamp(tv - in.s, -dv, dv);
    as[1] = in.w + wclamp(tw - in.w, -dw, dw);
    as[2] = a[2];
    as[3] = a[3];
}

// One substep of integration (integrate_kernel, swarp/dynamics/kernels.py:812-971): a
// SERVO agent's command turned into the VELOCITY command first (:849-863).
template <typename T, bool DRONE>
__device__ __forceinline__ void integrate(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                          const T (&a)[4], T Fx, T Fy, St<T> &o)
{
    T as[4] = {a[0], a[1], a[2], a[3]};
    Prm<T> Pv = P;
    if (P.mode == 2) {
        servo_command(C, P, in, a, as);
        Pv.mode = 0;
    }
    integrate_core<T, DRONE>(C, Pv, in, as, Fx, Fy, o);
}

// Reverse of drone_euler (gi = g on entry: the fields the drone does not step pass
// through).  g = adjoint of the substep output; writes the adjoints of the fields it
// steps into gi, the force adjoint into gFx / gFy and each rotor's action adjoint into
// gact (to be added to the action adjoint).
template <typename T, typename Ar>
__device__ __forceinline__ void drone_euler_adj(const Prm<T> &P, const St<T> &in, const T (&a)[4],
                                                T dt, T dtm, const St<T> &g, Ar &&A, St<T> &gi,
                                                T &gFx, T &gFy, T (&gact)[4])
{
    const T gpx = g.px, gpy = g.py;
    const T z0 = T(0);
    T f0 = wclamp(a[0], z0, P.thrust_max), f1 = wclamp(a[1], z0, P.thrust_max);
    T f2 = wclamp(a[2], z0, P.thrust_max), f3 = wclamp(a[3], z0, P.thrust_max);
    T thr = f0 + f1 + f2 + f3;
    const auto dm = A.prep(P.mass), dix = A.prep(P.ixx), diy = A.prep(P.iyy), diz = A.prep(P.izz);
    T vx3 = T(0), vy3 = T(0), vz3 = thr;
    T qx = in.qx, qy = in.qy, qz = in.qz, qw = in.qw;
    T c1x = qy * vz3 - qz * vy3, c1y = qz * vx3 - qx * vz3, c1z = qx * vy3 - qy * vx3;
    T tx = T(2) * c1x, ty = T(2) * c1y, tz = T(2) * c1z;
    T nbx = in.bx + A.div(P.arm * (f1 - f3) - (P.izz - P.iyy) * in.by * in.bz, dix) * dt;
    T nby = in.by + A.div(P.arm * (f2 - f0) - (P.ixx - P.izz) * in.bz * in.bx, diy) * dt;
    T nbz = in.bz + A.div(P.kappa * (f0 - f1 + f2 - f3) - (P.iyy - P.ixx) * in.bx * in.by, diz) * dt;
    const T h = T(0.5);
    T ux = qx + h * (qw * nbx + qy * nbz - qz * nby) * dt;
    T uy = qy + h * (qw * nby - qx * nbz + qz * nbx) * dt;
    T uz = qz + h * (qw * nbz + qx * nby - qy * nbx) * dt;
    T uw = qw + h * (-qx * nbx - qy * nby - qz * nbz) * dt;
    T l = A.sqrt(ux * ux + uy * uy + uz * uz + uw * uw);
    gi.px = gpx;
    gi.py = gpy;
    T gvx = g.vx + gpx * dt, gvy = g.vy + gpy * dt;
    gi.z = g.z;
    T gnvz = g.vz + g.z * dt;
    T gux = T(0), guy = T(0), guz = T(0), guw = T(0);
    if (l > T(0)) {
        const auto dl = A.prep(l);
        T nx = A.div(ux, dl), ny = A.div(uy, dl), nz = A.div(uz, dl), nw = A.div(uw, dl);
        T dq = g.qx * nx + g.qy * ny + g.qz * nz + g.qw * nw;
        gux = A.div(g.qx - nx * dq, dl);
        guy = A.div(g.qy - ny * dq, dl);
        guz = A.div(g.qz - nz * dq, dl);
        guw = A.div(g.qw - nw * dq, dl);
    }
    T gqx = gux, gqy = guy, gqz = guz, gqw = guw;
    T Dx = h * gux * dt, Dy = h * guy * dt, Dz = h * guz * dt, Dw = h * guw * dt;
    gqw += Dx * nbx + Dy * nby + Dz * nbz;
    gqx += -Dy * nbz + Dz * nby - Dw * nbx;
    gqy += Dx * nbz - Dz * nbx - Dw * nby;
    gqz += -Dx * nby + Dy * nbx - Dw * nbz;
    T gnbx = g.bx + Dx * qw + Dy * qz - Dz * qy - Dw * qx;
    T gnby = g.by - Dx * qz + Dy * qw + Dz * qx - Dw * qy;
    T gnbz = g.bz + Dx * qy - Dy * qx + Dz * qw - Dw * qz;
    T gbx = gnbx, gby = gnby, gbz = gnbz;
    T gtx = A.div(gnbx * dt, dix), gty = A.div(gnby * dt, diy), gtz = A.div(gnbz * dt, diz);
    gby -= (P.izz - P.iyy) * in.bz * gtx;
    gbz -= (P.izz - P.iyy) * in.by * gtx;
    gbz -= (P.ixx - P.izz) * in.bx * gty;
    gbx -= (P.ixx - P.izz) * in.bz * gty;
    gbx -= (P.iyy - P.ixx) * in.by * gtz;
    gby -= (P.iyy - P.ixx) * in.bx * gtz;
    T gf0 = -P.arm * gty + P.kappa * gtz;
    T gf1 = P.arm * gtx - P.kappa * gtz;
    T gf2 = P.arm * gty + P.kappa * gtz;
    T gf3 = -P.arm * gtx - P.kappa * gtz;
    gi.vz = gnvz;
    gi.vx = gvx;
    gi.vy = gvy;
    gFx = gvx * dtm;
    gFy = gvy * dtm;
    T gfx = A.div(gvx * dt, dm), gfy = A.div(gvy * dt, dm), gfz = A.div(gnvz * dt, dm);
    gqw += gfx * tx + gfy * ty + gfz * tz;
    T gtx2 = qw * gfx + (gfy * qz - gfz * qy);
    T gty2 = qw * gfy + (gfz * qx - gfx * qz);
    T gtz2 = qw * gfz + (gfx * qy - gfy * qx);
    gqx += ty * gfz - tz * gfy;
    gqy += tz * gfx - tx * gfz;
    gqz += tx * gfy - ty * gfx;
    T g1x = T(2) * gtx2, g1y = T(2) * gty2, g1z = T(2) * gtz2;
    gqx += vy3 * g1z - vz3 * g1y;
    gqy += vz3 * g1x - vx3 * g1z;
    gqz += vx3 * g1y - vy3 * g1x;
    T gthr = gfz + (g1x * qy - g1y * qx);
    gf0 += gthr; gf1 += gthr; gf2 += gthr; gf3 += gthr;
    gact[0] = wclamp_g(a[0], z0, P.thrust_max, gf0);
    gact[1] = wclamp_g(a[1], z0, P.thrust_max, gf1);
    gact[2] = wclamp_g(a[2], z0, P.thrust_max, gf2);
    gact[3] = wclamp_g(a[3], z0, P.thrust_max, gf3);
    gi.qx = gqx; gi.qy = gqy; gi.qz = gqz; gi.qw = gqw;
    gi.bx = gbx; gi.by = gby; gi.bz = gbz;
}

// Reverse of integrate without its position clamp (integrate_adj reverses that first).
// g = adjoint of the substep output.  Overwrites gi with the adjoint of the substep
// input, accumulates ga (actions) and returns gF (force).
template <typename T, bool DRONE>
__device__ __forceinline__ void integrate_adj_core(const Cst<T> &C, const Prm<T> &P,
                                                   const St<T> &in, const T (&a)[4], T Fx, T Fy,
                                                   const St<T> &g, St<T> &gi, T (&ga)[4], T &gFx,
                                                   T &gFy)
{
    if (C.rk4) {
        integrate_rk4_adj<T, DRONE>(C, P, in, a, Fx, Fy, g, gi, ga, gFx, gFy);
        return;
    }
    const T dt = C.sub_dt;
    const T dtm = dt / P.mass;
    const T dvx = Fx * dtm, dvy = Fy * dtm;
    gi = g;  // default: every field passes through
    T gpx = g.px, gpy = g.py;
    gFx = T(0);
    gFy = T(0);
    if (DRONE && P.tag == 3) {
        T gact[4];
        if constexpr (sizeof(T) == 4) {
            ArithPrep A;
            drone_euler_adj(P, in, a, dt, dtm, g, A, gi, gFx, gFy, gact);
            if (__builtin_expect(A.bad, 0))
                drone_euler_adj(P, in, a, dt, dtm, g, ArithIEEE<T>(), gi, gFx, gFy, gact);
        } else {
            drone_euler_adj(P, in, a, dt, dtm, g, ArithIEEE<T>(), gi, gFx, gFy, gact);
        }
        ga[0] += gact[0];
        ga[1] += gact[1];
        ga[2] += gact[2];
        ga[3] += gact[3];
        return;
    }
    if (P.tag == 0) {
        T vnx, vny, acx = T(0), acy = T(0), v0x = T(0), v0y = T(0);
        if (P.mode == 0) {
            clamp_norm(a[0], a[1], P.max_speed, vnx, vny);
        } else {
            clamp_norm(a[0], a[1], P.max_accel, acx, acy);
            v0x = in.vx + acx * dt;
            v0y = in.vy + acy * dt;
            clamp_norm(v0x, v0y, P.max_speed, vnx, vny);
        }
        vnx = vnx + dvx;
        vny = vny + dvy;
        T sp = m_sqrt(vnx * vnx + vny * vny);
        gi.px = gpx;
        gi.py = gpy;
        gi.th = g.th;
        gi.vx = T(0);
        gi.vy = T(0);
        gi.s = T(0);
        gi.w = T(0);
        T gvx = g.vx + gpx * dt, gvy = g.vy + gpy * dt;
        if (sp > T(0)) {
            gvx += g.s * vnx / sp;
            gvy += g.s * vny / sp;
        }
        gFx = gvx * dtm;
        gFy = gvy * dtm;
        if (P.mode == 0) {
            clamp_norm_adj(a[0], a[1], P.max_speed, gvx, gvy, ga[0], ga[1]);
        } else {
            T g0x = T(0), g0y = T(0);
            clamp_norm_adj(v0x, v0y, P.max_speed, gvx, gvy, g0x, g0y);
            gi.vx = g0x;
            gi.vy = g0y;
            clamp_norm_adj(a[0], a[1], P.max_accel, g0x * dt, g0y * dt, ga[0], ga[1]);
        }
    } else if (P.tag == 1) {
        T sn, wn, acc = T(0), alp = T(0);
        if (P.mode == 0) {
            sn = wclamp(a[0], -P.max_speed, P.max_speed);
            wn = wclamp(a[1], -P.max_ang_vel, P.max_ang_vel);
        } else {
            acc = wclamp(a[0], -P.max_accel, P.max_accel);
            alp = wclamp(a[1], -P.max_ang_accel, P.max_ang_accel);
            sn = wclamp(in.s + acc * dt, -P.max_speed, P.max_speed);
            wn = wclamp(in.w + alp * dt, -P.max_ang_vel, P.max_ang_vel);
        }
        T c = m_cos(in.th), sg = m_sin(in.th);
        gi.px = gpx;
        gi.py = gpy;
        T gvx = g.vx + gpx * dt, gvy = g.vy + gpy * dt;
        T gwn = g.w + g.th * dt;
        gFx = gvx * dtm;
        gFy = gvy * dtm;
        T gsn = g.s + gvx * c + gvy * sg;
        gi.th = g.th + (gvx * sn * -sg + gvy * sn * c);
        gi.vx = T(0);
        gi.vy = T(0);
        gi.s = T(0);
        gi.w = T(0);
        if (P.mode == 0) {
            ga[0] += wclamp_g(a[0], -P.max_speed, P.max_speed, gsn);
            ga[1] += wclamp_g(a[1], -P.max_ang_vel, P.max_ang_vel, gwn);
        } else {
            T gx = wclamp_g(in.s + acc * dt, -P.max_speed, P.max_speed, gsn);
            T gy = wclamp_g(in.w + alp * dt, -P.max_ang_vel, P.max_ang_vel, gwn);
            gi.s = gx;
            gi.w = gy;
            ga[0] += wclamp_g(a[0], -P.max_accel, P.max_accel, gx * dt);
            ga[1] += wclamp_g(a[1], -P.max_ang_accel, P.max_ang_accel, gy * dt);
        }
    } else if (P.tag == 2) {
        T acc = wclamp(a[0], -P.max_accel, P.max_accel);
        T del = wclamp(a[1], -P.max_steer, P.max_steer);
        T sn = wclamp(in.s + acc * dt, P.min_speed, P.max_speed);
        T wb = P.l_f + P.l_r;
        T td = m_tan(del);
        T bu = td * P.l_r / wb;
        T beta = m_atan(bu);
        T ang = in.th + beta;
        T ca = m_cos(ang), sa = m_sin(ang), cb = m_cos(beta);
        gi.px = gpx;
        gi.py = gpy;
        T gvx = g.vx + gpx * dt, gvy = g.vy + gpy * dt;
        T gwn = g.w + g.th * dt;
        gFx = gvx * dtm;
        gFy = gvy * dtm;
        T gsn = g.s + gvx * ca + gvy * sa + gwn * cb * td / wb;
        T gang = -gvx * sn * sa + gvy * sn * ca;
        T gbeta = gang - gwn * (sn / wb) * m_sin(beta) * td;
        T gtd = gwn * (sn / wb) * cb + gbeta / (T(1) + bu * bu) * P.l_r / wb;
        gi.th = g.th + gang;
        gi.vx = T(0);
        gi.vy = T(0);
        gi.w = T(0);
        T gx = wclamp_g(in.s + acc * dt, P.min_speed, P.max_speed, gsn);
        gi.s = gx;
        ga[0] += wclamp_g(a[0], -P.max_accel, P.max_accel, gx * dt);
        ga[1] += wclamp_g(a[1], -P.max_steer, P.max_steer, gtd * (T(1) + td * td));
    }
}

// Reverse of integrate: a SERVO agent's command conversion around the rest; the position
// clamp, reversed at the unclamped output (its bounds move with the heading under the
// footprint clamp); then the step itself.
template <typename T, bool DRONE>
__device__ __forceinline__ void integrate_adj(const Cst<T> &C, const Prm<T> &P, const St<T> &in,
                                              const T (&a)[4], T Fx, T Fy, const St<T> &g,
                                              St<T> &gi, T (&ga)[4], T &gFx, T &gFy)
{
    const bool servo = P.mode == 2;
    T as[4] = {a[0], a[1], a[2], a[3]};
    Prm<T> Pv = P;
    if (servo) {
        servo_command(C, P, in, a, as);
        Pv.mode = 0;
    }
    Cst<T> C0 = C;
    C0.clamp = 0;
    St<T> g2 = g;
    if (C.clamp) {
        St<T> raw;
        integrate_core<T, DRONE>(C0, Pv, in, as, Fx, Fy, raw);
        clamp_position_adj(C, Pv, raw.px, raw.py, raw.th, g2.px, g2.py, g2.th);
    }
    T gs[4] = {T(0), T(0), T(0), T(0)};
    integrate_adj_core<T, DRONE>(C0, Pv, in, as, Fx, Fy, g2, gi, gs, gFx, gFy);
    if (servo) {
        // as0 = s + clamp(tv - s, -dv, dv), tv = clamp(a0, +-max_speed) gain_v; likewise w
        const T dt = C.sub_dt;
        const T tv = wclamp(a[0], -P.max_speed, P.max_speed) * P.gain_v;
        const T tw = wclamp(a[1], -P.max_ang_vel, P.max_ang_vel) * P.gain_w;
        const T dv = P.max_accel * dt, dw = P.max_ang_accel * dt;
        const T xv = tv - in.s, xw = tw - in.w;
        const bool iv = !(xv < -dv) && !(xv > dv), iw = !(xw < -dw) && !(xw > dw);
        gi.s += iv ? T(0) : gs[0];
        gi.w += iw ? T(0) : gs[1];
        ga[0] += iv ? wclamp_g(a[0], -P.max_speed, P.max_speed, gs[0] * P.gain_v) : T(0);
        ga[1] += iw ? wclamp_g(a[1], -P.max_ang_vel, P.max_ang_vel, gs[1] * P.gain_w) : T(0);
    } else {
        ga[0] += gs[0];
        ga[1] += gs[1];
    }
    ga[2] += gs[2];
    ga[3] += gs[3];
}

}  // namespace swarp
