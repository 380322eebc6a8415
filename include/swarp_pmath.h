/*
 * swarp_pmath.h -- portable sin, cos, tan, atan and tanh: the same bits on every IEEE
 * platform.
 *
 * The step's float32 results depend on the transcendental functions of the diff-drive
 * and bicycle models, the obstacle and box geometry and the saturated contact law
 * (swarp/dynamics/kernels.py:194-275, swarp/core/collisions.py:87-105, 156-260).
 * Vendor math libraries differ by an ulp between host and device, and contact-rich
 * rollouts amplify an ulp to 1e-5 and more within twenty steps.  These functions are
 * evaluated in double precision with additions, subtractions, multiplications, exact
 * divisions, rint and fabs only, written out in a fixed order (no fused operations:
 * callers compile with -ffp-contract=off), so the HIP kernels and the C oracle compute
 * them identically; a float32 caller rounds the double result once.
 *
 * Method (from the mathematics; the coefficients are Taylor coefficients):
 *   sin, cos  Cody-Waite reduction by pi/2 (pi/2 split into a 33-bit head, so k * head
 *             is exact for |k| < 2^20, and a tail); Taylor series of sin and cos on
 *             |r| <= pi/4 to r^17 / r^18.
 *   tan       sin / cos of one reduction.
 *   atan      odd symmetry, atan(x) = pi/2 - atan(1/x) for |x| > 1, then
 *             atan(t) = atan(c) + atan((t - c) / (1 + t c)) with c the nearest of
 *             0, 1/4, 1/2, 3/4, 1 (|u| <= 1/8), and the Taylor series of atan(u) to u^21.
 *   tanh      odd symmetry, tanh(a) = e / (e + 2) with e = expm1(2a); expm1(y) by its
 *             Taylor series to y^17 for y < 1/2, else exp(y) - 1 with exp(y) = 2^k exp(r),
 *             r = y - k ln2 (ln2 split into a 41-bit head and a tail), exp(r) by its
 *             Taylor series to r^17; tanh(a) = 1 for a > 22.
 * Accuracy against float64 libm (tests/test_pmath.py): float32 results within 1 ulp of
 * the correctly rounded value (equal to it on all but a tiny fraction of inputs);
 * float64 results within 4 ulps, or within 2^-80 (1 + |x|) absolute next to the zeros of
 * sin and cos, where the two-part pi/2 bounds the reduction's absolute error.
 *
 * Included by the HIP kernels (device functions) and by the CPU oracle (plain C).
 */
#ifndef SWARP_PMATH_H
#define SWARP_PMATH_H

#if defined(__HIP__)
#define SWARP_PM static __host__ __device__ __forceinline__
#else
#define SWARP_PM static inline
#endif

/* sin and cos of x */
SWARP_PM void swarp_psincos(double x, double *so, double *co)
{
    const double k = __builtin_rint(x * 0x1.45f306dc9c883p-1);
    const double r = (x - k * 0x1.921fb544p+0) - k * 0x1.0b4611a626331p-34;
    const double z = r * r;
    double ps = 0x1.952c77030ad4ap-49;
    ps = ps * z - 0x1.ae7f3e733b81fp-41;
    ps = ps * z + 0x1.6124613a86d09p-33;
    ps = ps * z - 0x1.ae64567f544e4p-26;
    ps = ps * z + 0x1.71de3a556c734p-19;
    ps = ps * z - 0x1.a01a01a01a01ap-13;
    ps = ps * z + 0x1.1111111111111p-7;
    ps = ps * z - 0x1.5555555555555p-3;
    const double sn = r + r * (z * ps);
    double pc = -0x1.6827863b97d97p-53;
    pc = pc * z + 0x1.ae7f3e733b81fp-45;
    pc = pc * z - 0x1.93974a8c07c9dp-37;
    pc = pc * z + 0x1.1eed8eff8d898p-29;
    pc = pc * z - 0x1.27e4fb7789f5cp-22;
    pc = pc * z + 0x1.a01a01a01a01ap-16;
    pc = pc * z - 0x1.6c16c16c16c17p-10;
    pc = pc * z + 0x1.5555555555555p-5;
    const double cn = (1.0 - z * 0.5) + (z * z) * pc;
    const double q = k - 4.0 * __builtin_floor(k * 0.25); /* quadrant 0..3 (NaN: NaN) */
    *so = q == 0.0 ? sn : (q == 1.0 ? cn : (q == 2.0 ? -sn : -cn));
    *co = q == 0.0 ? cn : (q == 1.0 ? -sn : (q == 2.0 ? -cn : sn));
    if (x == 0.0) *so = x; /* sin keeps the sign of a zero */
}

SWARP_PM double swarp_psin(double x)
{
    double s, c;
    swarp_psincos(x, &s, &c);
    return s;
}

SWARP_PM double swarp_pcos(double x)
{
    double s, c;
    swarp_psincos(x, &s, &c);
    return c;
}

SWARP_PM double swarp_ptan(double x)
{
    double s, c;
    swarp_psincos(x, &s, &c);
    return s / c;
}

SWARP_PM double swarp_patan(double x)
{
    const double a = __builtin_fabs(x);
    const int inv = a > 1.0;
    const double t = inv ? 1.0 / a : a; /* in [0, 1] (NaN stays NaN) */
    const double j = __builtin_rint(t * 4.0);
    const double c = j * 0.25;
    const double u = (t - c) / (1.0 + t * c);
    const double z = u * u;
    double p = 0x1.8618618618618p-5; /* 1/21 */
    p = p * z - 0x1.af286bca1af28p-5;
    p = p * z + 0x1.e1e1e1e1e1e1ep-5;
    p = p * z - 0x1.1111111111111p-4;
    p = p * z + 0x1.3b13b13b13b14p-4;
    p = p * z - 0x1.745d1745d1746p-4;
    p = p * z + 0x1.c71c71c71c71cp-4;
    p = p * z - 0x1.2492492492492p-3;
    p = p * z + 0x1.999999999999ap-3;
    p = p * z - 0x1.5555555555555p-2; /* -1/3 */
    const double at = u + u * (z * p);
    /* atan(0), atan(1/4), atan(1/2), atan(3/4), atan(1) */
    const double base = j < 0.5 ? 0.0
                        : j < 1.5 ? 0x1.f5b75f92c80ddp-3
                        : j < 2.5 ? 0x1.dac670561bb4fp-2
                        : j < 3.5 ? 0x1.4978fa3269ee1p-1
                                  : 0x1.921fb54442d18p-1;
    double r = base + at;
    if (inv) r = 0x1.921fb54442d18p+0 - r;
    return __builtin_copysign(r, x);
}

/* e^y - 1 for y >= 0 (the only use: tanh) */
SWARP_PM double swarp_pexpm1_pos(double y)
{
    if (y < 0.5) {
        double p = 0x1.952c77030ad4ap-49; /* 1/17! */
        p = p * y + 0x1.ae7f3e733b81fp-45;
        p = p * y + 0x1.ae7f3e733b81fp-41;
        p = p * y + 0x1.93974a8c07c9dp-37;
        p = p * y + 0x1.6124613a86d09p-33;
        p = p * y + 0x1.1eed8eff8d898p-29;
        p = p * y + 0x1.ae64567f544e4p-26;
        p = p * y + 0x1.27e4fb7789f5cp-22;
        p = p * y + 0x1.71de3a556c734p-19;
        p = p * y + 0x1.a01a01a01a01ap-16;
        p = p * y + 0x1.a01a01a01a01ap-13;
        p = p * y + 0x1.6c16c16c16c17p-10;
        p = p * y + 0x1.1111111111111p-7;
        p = p * y + 0x1.5555555555555p-5;
        p = p * y + 0x1.5555555555555p-3;
        p = p * y + 0x1.0000000000000p-1;
        return y + y * (y * p);
    }
    const double k = __builtin_rint(y * 0x1.71547652b82fep+0);
    const double r = (y - k * 0x1.62e42fefa3800p-1) - k * 0x1.ef35793c76730p-45;
    double p = 0x1.952c77030ad4ap-49;
    p = p * r + 0x1.ae7f3e733b81fp-45;
    p = p * r + 0x1.ae7f3e733b81fp-41;
    p = p * r + 0x1.93974a8c07c9dp-37;
    p = p * r + 0x1.6124613a86d09p-33;
    p = p * r + 0x1.1eed8eff8d898p-29;
    p = p * r + 0x1.ae64567f544e4p-26;
    p = p * r + 0x1.27e4fb7789f5cp-22;
    p = p * r + 0x1.71de3a556c734p-19;
    p = p * r + 0x1.a01a01a01a01ap-16;
    p = p * r + 0x1.a01a01a01a01ap-13;
    p = p * r + 0x1.6c16c16c16c17p-10;
    p = p * r + 0x1.1111111111111p-7;
    p = p * r + 0x1.5555555555555p-5;
    p = p * r + 0x1.5555555555555p-3;
    p = p * r + 0x1.0000000000000p-1;
    const double er = 1.0 + (r + r * (r * p));
    return __builtin_ldexp(er, (int)k) - 1.0; /* exact scaling by 2^k, 1 <= k <= 64 */
}

SWARP_PM double swarp_ptanh(double x)
{
    const double a = __builtin_fabs(x);
    double r;
    if (a > 22.0) {
        r = 1.0;
    } else {
        const double e = swarp_pexpm1_pos(2.0 * a);
        r = e / (e + 2.0);
    }
    if (!(a == a)) r = x; /* NaN */
    return __builtin_copysign(r, x);
}

#endif /* SWARP_PMATH_H */
