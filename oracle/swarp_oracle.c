/*
 * swarp_oracle.c -- CPU restatement of swarp's differentiable physics step.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker of the HIP product and the CPU
 * baseline timed by bench.py.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it (through oracle/oracle.py).
 *
 * Restates, from the reference's source text:
 *   neighbours     swarp/core/neighbors.py:76-97 (_brute_force)
 *   contact forces swarp/core/collisions.py:48-260, 690-881
 *   integration    swarp/dynamics/kernels.py:68-413 (Euler, all four models),
                  :416-793 (RK4, the three 2-D models)
 *   step ordering  swarp/core/stepper.py:784-1011 (taped path)
 * and the reverse mode warp-lang generates for them (swarp/interop/autograd.py:277-296).
 *
 * Built with -ffp-contract=off so every a*b+c rounds twice, as written.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* sin, cos, tan, atan, tanh: the portable double-precision evaluations shared with the
   HIP kernels (include/swarp_pmath.h, pinned against libm by tests/test_pmath.py), so a
   float32 restatement computes the same transcendental values as the device. */
#include "swarp_pmath.h"

typedef struct {
    int n_envs, n_agents, act_dim, substeps, max_neighbors;
    int collisions, soft_walls, clamp_bounds, n_threads;
    double dt, k, c, margin, max_overlap, neighbor_radius;
    double bmin_x, bmin_y, bmax_x, bmax_y;
    double lin_damping, ang_damping; /* movable bodies' viscous decay rates */
    int rk4;                         /* Integrator.RK4 (2-D models) instead of Euler */
    int wheel;                       /* WorldConfig.wheel_contacts (forward only) */
    double lat_grip, turn_cap;       /* wheel_lateral_friction * gravity, wheel_turn_torque */
    /* list order: grid_bins = 0 ascending index (_brute_force); > 0 the uniform grid's
       (_query_uniform) over grid_bins^2 cells with the pinned frame (origin, cell size)
       grid_ox, grid_oy, grid_cell, rounded to REAL */
    int grid_bins;
    double grid_ox, grid_oy, grid_cell;
} oracle_cfg_t;

typedef struct {
    int n_obstacles;
    const void *pos, *radius, *angle, *half, *vel, *ang_vel;
    const int32_t *type;
    /* movable compound bodies (NULL = every obstacle immovable): kind [N] (1 = MOVABLE),
       body [N] (root shape), mass [N], inertia [N], body_off [N,2] */
    const int32_t *kind, *body;
    const void *mass, *inertia, *body_off;
    /* [A, 22] agent rows the body pass reads (NULL: the agents' own rows): the shared
       table when the agents' rows are per env (swarp/core/stepper.py:961-964) */
    const void *body_params;
} oracle_obs_t;

int oracle_abi_version(void) { return 1; }

#define REAL double
#define FN(x) x##_f64
#define SQRT sqrt
#define COS swarp_pcos
#define SIN swarp_psin
#define TAN swarp_ptan
#define ATAN swarp_patan
#define TANH swarp_ptanh
#define FABS fabs
#include "oracle_impl.h"
#undef REAL
#undef FN
#undef SQRT
#undef COS
#undef SIN
#undef TAN
#undef ATAN
#undef TANH
#undef FABS

#define REAL float
#define FN(x) x##_f32
#define SQRT sqrtf
#define COS(x) ((float)swarp_pcos((double)(x)))
#define SIN(x) ((float)swarp_psin((double)(x)))
#define TAN(x) ((float)swarp_ptan((double)(x)))
#define ATAN(x) ((float)swarp_patan((double)(x)))
#define TANH(x) ((float)swarp_ptanh((double)(x)))
#define FABS fabsf
#include "oracle_impl.h"

/* The portable transcendental functions over arrays (fn: 0 sin, 1 cos, 2 tan, 3 atan,
   4 tanh), for their accuracy tests. */
static double pm_eval(int fn, double x)
{
    switch (fn) {
    case 0: return swarp_psin(x);
    case 1: return swarp_pcos(x);
    case 2: return swarp_ptan(x);
    case 3: return swarp_patan(x);
    default: return swarp_ptanh(x);
    }
}

void oracle_pmath_f64(int fn, const double *x, double *y, long n)
{
    for (long i = 0; i < n; ++i) y[i] = pm_eval(fn, x[i]);
}

void oracle_pmath_f32(int fn, const float *x, float *y, long n)
{
    for (long i = 0; i < n; ++i) y[i] = (float)pm_eval(fn, (double)x[i]);
}
