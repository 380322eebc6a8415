// swarp_hip.hip -- host side and C ABI of the swarp physics step (include/swarp_hip.h).
// The kernels live in the family units k_*.hip (one object per family and dtype, built
// in parallel); this unit validates descriptors, derives the step constants and calls
// their launchers.
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
#include <stdlib.h>
#include <string.h>

#include "launch.hpp"
#include "swarp_hip.h"

// ====================================================================== host side

using namespace swarp;

static thread_local char g_err[512];

static int fail(const char *msg)
{
    snprintf(g_err, sizeof g_err, "%s", msg);
    return -1;
}

namespace swarp {
// The error channel of the entry points defined in other units (coo_noalloc.hip).
int set_error(const char *msg) { return msg[0] ? fail(msg) : (g_err[0] = 0, 0); }
}  // namespace swarp

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
    C.round_only = d->obstacle_types == 1 ? 1 : 0;
    C.wheel = d->wheel_contacts ? 1 : 0;
    C.lat_grip = (T)d->lat_grip;
    C.turn_cap = (T)d->turn_cap;
    C.needs_forces = (d->collisions || d->soft_walls || d->n_obstacles > 0) ? 1 : 0;
    C.use_skin = (d->collisions && d->substeps > 1 && skin > 0.0) ? 1 : 0;
    // contact distances lie in [sqrt(eps2), neighbour radius]: within the range of the
    // short exact division when the radius is at most 2^20
    C.fast_div = d->neighbor_radius <= 0x1p20 ? 1 : 0;
    C.rk4 = d->integrator == SWARP_RK4 ? 1 : 0;
    C.grid_bins = d->neighbor_method == SWARP_LISTS_GRID ? d->grid_bins : 0;
    C.grid_ox = (T)d->grid_origin[0];
    C.grid_oy = (T)d->grid_origin[1];
    C.grid_cs = (T)d->grid_cell;
    return 0;
}

static int check_desc(const swarp_desc_t *d, bool need_params = true)
{
    if (!d) return fail("desc is NULL");
    if (d->abi_version != SWARP_ABI_VERSION) return fail("desc->abi_version mismatch");
    if (d->dtype != SWARP_F32 && d->dtype != SWARP_F64) return fail("desc->dtype must be SWARP_F32 or SWARP_F64");
    if (d->n_envs < 1) return fail("n_envs must be >= 1");
    if (d->n_agents < 1 || d->n_agents > SWARP_WIDE_MAX_AGENTS)
        return fail("n_agents must lie in [1, 4096]");
    if (d->neighbor_method != SWARP_LISTS_BRUTE && d->neighbor_method != SWARP_LISTS_GRID)
        return fail("desc->neighbor_method must be SWARP_LISTS_BRUTE or SWARP_LISTS_GRID");
    if (d->neighbor_method == SWARP_LISTS_GRID) {
        // the cell table's LDS bounds the bins (wide_lds_check); 1024 bounds bins^2's range
        if (d->grid_bins < 1 || d->grid_bins > 1024) return fail("grid_bins must lie in [1, 1024]");
        if (d->grid_pinned && !(d->grid_cell > 0.0)) return fail("grid_cell must be positive");
    }
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
    const double vmax = d->skin_speed > 0.0 ? d->skin_speed : 1.0;
    return 2.0 * 1.5 * vmax * (d->substeps - 1) * (d->dt / d->substeps);
}

template <typename T> static void fill_args(const swarp_desc_t *d, Args<T> &a)
{
    memset(&a, 0, sizeof a);
    a.params = (const T *)d->params;
    a.tag = d->model_tag;
    a.mode = d->ctrl_mode;
    a.obs.pos = (decltype(a.obs.pos))d->obs_pos;
    a.obs.rad = (decltype(a.obs.rad))d->obs_radius;
    a.obs.ang = (decltype(a.obs.ang))d->obs_angle;
    a.obs.half = (decltype(a.obs.half))d->obs_half;
    a.obs.vel = (decltype(a.obs.vel))d->obs_vel;
    a.obs.om = (decltype(a.obs.om))d->obs_ang_vel;
    a.obs.type = (decltype(a.obs.type))d->obs_type;
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

// The optional kernel paths (FT_* bits) the world uses, which select the kernel instance.
// body: the obstacles are the movable bodies of the body kernels, not static obstacles.
static unsigned world_features(const swarp_desc_t *d, bool body)
{
    unsigned f = 0;
    if (d->integrator == SWARP_RK4) f |= FT_RK4;
    if (d->max_overlap > 0.0) f |= FT_SAT;
    if (!body && d->n_obstacles > 0) f |= FT_OBST;
    // box or segment shapes among the obstacles of a body world (0: not known)
    if (body && d->obstacle_types != 1) f |= FT_SHAPES;
    if (body && d->n_obstacles > 64) f |= FT_MANYSH;
    if (d->soft_walls) f |= FT_WALL;
    if (d->clamp_bounds) f |= FT_CLAMP;
    const unsigned models = d->fleet_models ? (unsigned)d->fleet_models : ~0u;
    const unsigned modes = d->fleet_modes ? (unsigned)d->fleet_modes : ~0u;
    if (models & ~0xfu) return FT_ALL;
    // the control mode only changes holonomic and diff-drive agents (bicycles and drones
    // read their actions one way)
    if ((modes & ~1u) && (models & 3u)) f |= FT_MODES;
    if (models & 1u) f |= FT_HOLO;
    if (models & 2u) f |= FT_DIFF;
    if (models & 4u) f |= FT_BICY;
    if (models & 8u) f |= FT_DRONE;
    return f;
}

// The wide-env kernels (one workgroup per env): more than 64 agents, or grid-ordered lists.
static bool wide_path(const swarp_desc_t *d)
{
    return d->n_agents > 64 || d->neighbor_method == SWARP_LISTS_GRID;
}

// What the wide-env kernels do not step, as an error message (NULL: they step it).
static const char *wide_unsupported(const swarp_desc_t *d)
{
    if (d->neighbor_method == SWARP_LISTS_GRID && d->collisions && !d->grid_pinned)
        return "stepping with uniform-grid lists needs the grid frame pinned by the world bounds "
               "(an adaptive frame reduces over every env at every substep)";
    return nullptr;
}

// lists_only: the list builder's staging (no box fields).
template <typename T> static int wide_lds_check(const swarp_desc_t *d, bool lists_only = false)
{
    const int NC = d->neighbor_method == SWARP_LISTS_GRID ? d->grid_bins * d->grid_bins : 0;
    const int AP = wide_geom(d->n_agents).slots;
    // dynamic staging + the kernels' static wsum[16]: the workgroup's whole LDS; box worlds
    // also stage headings, spins and footprints
    if (!lists_only && (d->has_boxes || d->wheel_contacts)) {
        if (wide_box_lds_bytes<T>(AP, NC) + 16 * sizeof(int32_t) > LDS_MAX)
            return fail("n_agents / grid_bins too large for the wide-env LDS staging of a box "
                        "world at this dtype (limit 160 KiB)");
    } else if (wide_lds_bytes<T>(AP, NC) + 16 * sizeof(int32_t) > LDS_MAX) {
        return fail("n_agents / grid_bins too large for the wide-env LDS staging at this dtype "
                    "(limit 160 KiB)");
    }
    return 0;
}

static bool lean_ok(const swarp_desc_t *d)
{
    return !wide_path(d) && d->holo_velocity_only && !d->has_drone && d->n_obstacles == 0 && !d->clamp_bounds &&
           d->integrator == SWARP_EULER && !d->has_boxes && !d->wheel_contacts &&
           !d->params_per_env;
}

// Byte offsets of the tape regions (see lean.hpp); total == 0: no tape.  The specialised
// holonomic kernels keep records (rec) and last velocities (vl); the two-wave forward of
// 2-D fleets among static obstacles keeps each substep's total forces (fsum, read by the
// backward's recompute), each substep's neighbour-inclusion masks (nmask, read by the
// recompute in place of its scan) and, for at most 32 obstacles, each substep's obstacle
// contact masks (omask, read by its reverse pass).
struct TapeLayout {
    uint64_t rec, vl, fsum, omask, nmask, total;
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

// Whether rollout_fwd runs the two-wave forward (launch_fwd's condition for it).
static bool split_ok(const swarp_desc_t *d)
{
    if (wide_path(d) || lean_ok(d) || d->has_drone || d->has_boxes || d->wheel_contacts)
        return false;
    if (d->dtype != SWARP_F32 || d->n_obstacles <= 0) return false;
    const unsigned feat = world_features(d, false);
    if ((feat & ~FT_PROF_2D) != 0u || !(feat & FT_OBST)) return false;
    return (64 / pad_agents(d->n_agents)) * d->n_obstacles <= OCS_MAX;
}

// Whether the one-wave generic forward keeps a tape: each substep's total force (fsum) and
// neighbour-inclusion masks (nmask), which its backward reads instead of a force pass.
static bool gen_tape_ok(const swarp_desc_t *d)
{
    return !wide_path(d) && !lean_ok(d) && !split_ok(d) && !d->has_boxes && !d->wheel_contacts &&
           (d->collisions || d->soft_walls || d->n_obstacles > 0);
}

static TapeLayout tape_layout(const swarp_desc_t *d, int32_t nT)
{
    TapeLayout L = {0, 0, 0, 0, 0, 0};
    if (nT >= 1 && split_ok(d)) {
        const uint64_t n = (uint64_t)nT * d->substeps * d->n_envs * d->n_agents;
        L.fsum = 0;
        L.omask = align256(n * 2 * sizeof(float));
        L.nmask = align256(L.omask + n * omask_bytes(d->n_obstacles));
        L.total = align256(L.nmask + n * (pad_agents(d->n_agents) == 64 ? 8 : 4));
        return L;
    }
    if (nT >= 1 && gen_tape_ok(d)) {
        const uint64_t n = (uint64_t)nT * d->substeps * d->n_envs * d->n_agents;
        L.fsum = 0;
        L.omask = L.nmask = align256(n * 2 * (d->dtype == SWARP_F32 ? 4 : 8));
        L.total = align256(L.nmask + n * (pad_agents(d->n_agents) == 64 ? 8 : 4));
        return L;
    }
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
    if (tape && TL.total && (split_ok(d) || gen_tape_ok(d))) {
        a.fsum = (T *)((unsigned char *)tape + TL.fsum);
        if (split_ok(d) && omask_bytes(d->n_obstacles)) a.omask = (unsigned char *)tape + TL.omask;
        a.nmask = (unsigned char *)tape + TL.nmask;
    }
    const int PA = pad_agents(d->n_agents);
    const unsigned feat = world_features(d, false);
    if (wide_path(d)) {
        if (const char *why = wide_unsupported(d)) return fail(why);
        if (wide_lds_check<T>(d)) return -1;
        launch_wide_fwd<T>(d->has_drone != 0, d->has_boxes || d->wheel_contacts, C, a, st);
    } else if (lean_ok(d)) {
        if (tape && TL.total)
            launch_holo_fwd<T, true>(PA, C, a, tape_ptrs<T>(TL, tape), st);
        else
            launch_holo_fwd<T, false>(PA, C, a, tape_ptrs<T>(TL, nullptr), st);
    } else if (d->has_drone) {
        launch_fwd<T, true, false>(PA, C, a, feat, st);
    } else if (d->has_boxes || d->wheel_contacts) {
        launch_fwd<T, false, true>(PA, C, a, feat, st);
    } else {
        launch_fwd<T, false, false>(PA, C, a, feat, st);
    }
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
    if (tape && TL.total && (split_ok(d) || gen_tape_ok(d))) {
        a.fsum = (T *)((unsigned char *)tape + TL.fsum);
        if (split_ok(d) && omask_bytes(d->n_obstacles)) a.omask = (unsigned char *)tape + TL.omask;
        a.nmask = (unsigned char *)tape + TL.nmask;
    }
    const int PA = pad_agents(d->n_agents);
    if (wide_path(d)) {
        if (const char *why = wide_unsupported(d)) return fail(why);
        if (wide_lds_check<T>(d)) return -1;
        launch_wide_bwd<T>(d->has_drone != 0, d->has_boxes != 0, C, a, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(hipGetErrorString(e));
        return 0;
    }
    if (lean_ok(d)) {
        const size_t msz = PA == 64 ? 8 : 4;
        const size_t lshm = (size_t)d->substeps * 128 * 2 * sizeof(T) +
                            (size_t)d->substeps * 64 * msz * 2 + 64 * 2 * sizeof(T) +
                            2 * 64 * sizeof(T) + (size_t)d->substeps * 64;
        if (lshm > LDS_MAX) return fail("substeps too large for the backward LDS staging (limit 160 KiB per wave)");
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
    else if (split_ok(d) && omask_bytes(d->n_obstacles))  // obstacle-contact masks per substep
        shm += (size_t)d->substeps * 64 * sizeof(uint32_t);
    // with k_rollout_bwd's static arrays (ocs_lds[2 OCS_MAX], lbx[3 * 64]): the whole LDS
    if (shm + (2 * OCS_MAX + 3 * 64) * sizeof(T) > LDS_MAX)
        return fail("substeps too large for the backward LDS staging (limit 160 KiB per wave)");
    if (d->has_drone)
        launch_bwd<T, true, false>(PA, C, a, world_features(d, false), shm, st);
    else if (d->has_boxes)
        launch_bwd<T, false, true>(PA, C, a, world_features(d, false), shm, st);
    else
        launch_bwd<T, false, false>(PA, C, a, world_features(d, false), shm, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

// Env slot width of the body kernels: the padded agent count, doubled (fewer env slots per
// wave, more pad lanes) until the obstacle staging of both passes fits 64 KiB of LDS, which
// leaves room for more resident workgroups than a larger staging; 64 when nothing fits (the
// callers then check the 160 KiB a workgroup may hold).
template <typename T> static int body_pa(const swarp_desc_t *d)
{
    const bool dr = d->has_drone != 0;
    int PA = pad_agents(d->n_agents);
    while (PA < 64 && (body_fwd_lds_total(PA, d->n_obstacles, sizeof(T)) > 65536 ||
                       body_bwd_lds_of<T>(PA, d->substeps, d->n_obstacles, dr, false) > 65536))
        PA *= 2;
    return PA;
}

// LDS of the wide body kernels' workgroup (dynamic staging + the static wsum[16]) within
// 160 KiB; bwd: the backward's (three obstacle states and two adjoints instead of two).
template <typename T> static int wbody_lds_check(const swarp_desc_t *d, bool bwd)
{
    const int NC = d->neighbor_method == SWARP_LISTS_GRID ? d->grid_bins * d->grid_bins : 0;
    const int AP = ((d->n_agents + 63) / 64) * 64;
    if (wbody_lds_bytes<T>(AP, NC, d->n_obstacles, bwd) + 16 * sizeof(int32_t) > LDS_MAX)
        return fail(bwd ? "agents and obstacles per env too many for the wide body backward's "
                          "LDS staging (limit 160 KiB per workgroup)"
                        : "agents and obstacles per env too many for the wide body forward's "
                          "LDS staging (limit 160 KiB per workgroup)");
    return 0;
}

template <typename T> static int fill_obtab(const swarp_desc_t *d, ObTab<T> &tb)
{
    if (d->n_obstacles < 1) return fail("the body path takes at least one obstacle per env");
    if (d->n_agents > 1024)
        return fail("movable bodies step at most 1024 agents per env (one thread per agent in "
                    "the env's workgroup)");
    if (wide_path(d)) {
        if (const char *why = wide_unsupported(d)) return fail(why);
        if (wbody_lds_check<T>(d, false)) return -1;
    } else if (body_fwd_lds_total(body_pa<T>(d), d->n_obstacles, sizeof(T)) > LDS_MAX) {
        return fail("too many obstacles per env for the body forward's LDS staging (limit "
                    "160 KiB per wave)");
    }
    if (!d->obs_kind || !d->obs_body || !d->obs_mass || !d->obs_inertia || !d->obs_body_off)
        return fail("obs_kind/obs_body/obs_mass/obs_inertia/obs_body_off must be set");
    tb.rad = (decltype(tb.rad))d->obs_radius;
    tb.half = (decltype(tb.half))d->obs_half;
    tb.mass = (decltype(tb.mass))d->obs_mass;
    tb.inertia = (decltype(tb.inertia))d->obs_inertia;
    tb.off = (decltype(tb.off))d->obs_body_off;
    tb.type = (decltype(tb.type))d->obs_type;
    tb.kind = (decltype(tb.kind))d->obs_kind;
    tb.body = (decltype(tb.body))d->obs_body;
    // per-env rows: the body pass reads the shared table (body_params)
    if (d->params_per_env && !d->body_params)
        return fail("body_params must be set when params_per_env = 1 and bodies move");
    tb.bprm = d->params_per_env ? (decltype(tb.bprm))d->body_params : nullptr;
    tb.lin_damp = (T)d->lin_damping;
    tb.ang_damp = (T)d->ang_damping;
    tb.N = d->n_obstacles;
    tb.cache = 0;
    return 0;
}

// Bodies a body tape of `bytes` holds for a T-step rollout of d (0: not a whole number of
// per-body slices, or none).
template <typename T> static int64_t ob_tape_roots(const swarp_desc_t *d, int32_t nT, uint64_t bytes)
{
    const uint64_t per = (uint64_t)nT * d->substeps * d->n_envs * BODY_REC * sizeof(T);
    if (per == 0 || bytes % per != 0) return 0;
    return (int64_t)(bytes / per);
}

template <typename T>
static int rollout_fwd_ob(const swarp_desc_t *d, int32_t nT, const swarp_state_t *s0,
                          const void *ob0, const void *act, const swarp_state_t *traj,
                          const swarp_state_t *fin, void *ob_traj, void *tape, uint64_t tape_bytes,
                          hipStream_t st)
{
    Cst<T> C;
    fill_cst<T>(d, skin_of(d), C);
    Args<T> a;
    fill_args<T>(d, a);
    ObTab<T> tb;
    if (fill_obtab<T>(d, tb)) return -1;
    const int nf = d->has_drone ? 9 : 5;
    if (!fields_ok(s0, nf)) return fail("state0 is missing a field");
    if (!fields_ok(fin, nf)) return fail("final_state is missing a field");
    if (nT > 1 && !fields_ok(traj, nf)) return fail("traj is missing a field (T > 1)");
    if (!act || !ob0 || !ob_traj) return fail("actions / ob0 / ob_traj is NULL");
    copy_fields<T>(s0, (T **)a.s0.f);
    copy_fields<T>(fin, a.fin.f);
    if (nT > 1) copy_fields<T>(traj, a.traj.f);
    a.act = (const T *)act;
    a.nsteps = nT;
    ObIO<T> io = {(const T *)ob0, (T *)ob_traj, nullptr, nullptr, nullptr, 0};
    if (tape) {
        const int64_t r = ob_tape_roots<T>(d, nT, tape_bytes);
        if (r < 1 || r > d->n_obstacles)
            return fail("tape_bytes is not swarp_ob_tape_bytes of 1..n_obstacles bodies");
        io.tape = (T *)tape;
        io.tape_roots = (int)r;
    }
    if (wide_path(d)) {
        // the wide kernels keep no body tape (their backward evaluates the pass again)
        io.tape = nullptr;
        io.tape_roots = 0;
        launch_wbody_fwd<T>(d->has_drone != 0, C, a, tb, io, st);
    } else {
        launch_body_fwd<T>(body_pa<T>(d), C, a, tb, io, world_features(d, true),
                           d->has_drone != 0, st);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

template <typename T>
static int rollout_bwd_ob(const swarp_desc_t *d, int32_t nT, const swarp_state_t *s0,
                          const void *ob0, const void *act, const swarp_state_t *traj,
                          const void *ob_traj, const swarp_state_t *atraj,
                          const swarp_state_t *afin, const void *aob_traj,
                          const swarp_state_t *a0, void *aob0, void *aact, const void *tape,
                          uint64_t tape_bytes, hipStream_t st)
{
    Cst<T> C;
    fill_cst<T>(d, skin_of(d), C);
    Args<T> a;
    fill_args<T>(d, a);
    ObTab<T> tb;
    if (fill_obtab<T>(d, tb)) return -1;
    const int nf = d->has_drone ? 9 : 5;
    if (!fields_ok(s0, nf)) return fail("state0 is missing a field");
    if (nT > 1 && !fields_ok(traj, nf)) return fail("traj is missing a field (T > 1)");
    if (!act || !aact || !ob0 || !ob_traj) return fail("actions / adj_actions / ob0 / ob_traj is NULL");
    copy_fields<T>(s0, (T **)a.s0.f);
    if (nT > 1) copy_fields<T>(traj, a.traj.f);
    if (atraj) copy_fields<T>(atraj, (T **)a.atraj.f);
    if (afin) copy_fields<T>(afin, (T **)a.afin.f);
    if (a0) copy_fields<T>(a0, a.a0.f);
    a.act = (const T *)act;
    a.aact = (T *)aact;
    a.nsteps = nT;
    ObIO<T> io = {(const T *)ob0, (T *)ob_traj, (const T *)aob_traj, (T *)aob0, nullptr, 0};
    if (tape) {
        const int64_t r = ob_tape_roots<T>(d, nT, tape_bytes);
        if (r < 1 || r > d->n_obstacles)
            return fail("tape_bytes is not swarp_ob_tape_bytes of 1..n_obstacles bodies");
        io.tape = (T *)tape;
        io.tape_roots = (int)r;
    }
    if (wide_path(d)) {
        if (wbody_lds_check<T>(d, true)) return -1;
        io.tape = nullptr;
        io.tape_roots = 0;
        launch_wbody_bwd<T>(d->has_drone != 0, C, a, tb, io, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(hipGetErrorString(e));
        return 0;
    }
    const int PA = body_pa<T>(d);
    // the per-substep body caches (cos / sin, contact sums) when they fit
    const bool dr = d->has_drone != 0;
    size_t shm = body_bwd_lds_of<T>(PA, d->substeps, d->n_obstacles, dr, true);
    // (the caches only where they keep the workgroup within 64 KiB: more resident waves)
    tb.cache = shm <= 65536 ? 1 : 0;
    if (!tb.cache) shm = body_bwd_lds_of<T>(PA, d->substeps, d->n_obstacles, dr, false);
    if (shm > LDS_MAX)
        return fail("obstacle count or substeps too large for the body backward's LDS staging "
                    "(limit 160 KiB per wave)");
    launch_body_bwd<T>(PA, C, a, tb, io, world_features(d, true), d->has_drone != 0, shm, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

// Whether rollout_bwd_ob can run this configuration (the checks it makes before its launch).
template <typename T> static int bwd_ob_fits(const swarp_desc_t *d)
{
    ObTab<T> tb;
    if (fill_obtab<T>(d, tb)) return -1;
    if (wide_path(d)) return wbody_lds_check<T>(d, true);
    if (body_bwd_lds_of<T>(body_pa<T>(d), d->substeps, d->n_obstacles, d->has_drone != 0, false) >
        LDS_MAX)
        return fail("obstacle count or substeps too large for the body backward's LDS staging "
                    "(limit 160 KiB per wave)");
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
    g.radius = (const T *)v->radius;
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
    launch_nav<T>(PA, C, g, dyn, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

// Default drone fields [z n | vz n | attitude 4n | body_rates 3n]: every element 0 except
// the w component of each quaternion.  Each lane writes one 16-byte piece (16 / sizeof(T)
// consecutive elements) with one vector store; the piece at the end of a buffer whose
// length is not a multiple of it is written element by element.  `buf` is 16-byte aligned
// (the caller's allocation).
template <typename T> __global__ void k_state_defaults(int64_t n, T *buf)
{
    constexpr int V = 16 / sizeof(T);
    const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
    const int64_t end = 9 * n;
    if (i0 >= end) return;
    T v[V];
#pragma unroll
    for (int k = 0; k < V; ++k) {
        const int64_t i = i0 + k;
        v[k] = (i >= 2 * n && i < 6 * n && ((i - 2 * n) & 3) == 3) ? T(1) : T(0);
    }
    if (i0 + V <= end) {
        uint4 w;
        __builtin_memcpy(&w, v, 16);
        *(uint4 *)(buf + i0) = w;
    } else {
        for (int k = 0; k < V && i0 + k < end; ++k) buf[i0 + k] = v[k];
    }
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
    if (desc->has_boxes || desc->wheel_contacts)
        return fail("box agents and wheel contacts with movable bodies are not supported in "
                    "this build");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_fwd_ob<float>(desc, T, state0, ob0, actions, traj, final_state, ob_traj,
                                     nullptr, 0, st);
    return rollout_fwd_ob<double>(desc, T, state0, ob0, actions, traj, final_state, ob_traj,
                                  nullptr, 0, st);
}

int swarp_ob_tape_bytes(const swarp_desc_t *desc, int32_t T, int32_t n_bodies, uint64_t *bytes)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (!bytes) return fail("bytes is NULL");
    if (T < 1) return fail("T must be >= 1");
    if (n_bodies < 1 || n_bodies > desc->n_obstacles)
        return fail("n_bodies must lie in [1, n_obstacles]");
    const uint64_t ts = desc->dtype == SWARP_F32 ? 4 : 8;
    *bytes = (uint64_t)T * desc->substeps * desc->n_envs * n_bodies * BODY_REC * ts;
    return 0;
}

int swarp_rollout_fwd_ob_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                              const void *ob0, const void *actions, const swarp_state_t *traj,
                              const swarp_state_t *final_state, void *ob_traj, void *tape,
                              uint64_t tape_bytes, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (!tape) return fail("tape is NULL");
    if (desc->has_boxes || desc->wheel_contacts)
        return fail("box agents and wheel contacts with movable bodies are not supported in "
                    "this build");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_fwd_ob<float>(desc, T, state0, ob0, actions, traj, final_state, ob_traj,
                                     tape, tape_bytes, st);
    return rollout_fwd_ob<double>(desc, T, state0, ob0, actions, traj, final_state, ob_traj,
                                  tape, tape_bytes, st);
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
    if (desc->has_boxes || desc->wheel_contacts)
        return fail("box agents and wheel contacts with movable bodies are not supported in "
                    "this build");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_bwd_ob<float>(desc, T, state0, ob0, actions, traj, ob_traj, adj_traj,
                                     adj_final, adj_ob_traj, adj_state0, adj_ob0, adj_actions,
                                     nullptr, 0, st);
    return rollout_bwd_ob<double>(desc, T, state0, ob0, actions, traj, ob_traj, adj_traj,
                                  adj_final, adj_ob_traj, adj_state0, adj_ob0, adj_actions,
                                  nullptr, 0, st);
}

int swarp_rollout_bwd_ob_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                              const void *ob0, const void *actions, const swarp_state_t *traj,
                              const void *ob_traj, const swarp_state_t *adj_traj,
                              const swarp_state_t *adj_final, const void *adj_ob_traj,
                              const swarp_state_t *adj_state0, void *adj_ob0, void *adj_actions,
                              const void *tape, uint64_t tape_bytes, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (T < 1) return fail("T must be >= 1");
    if (!tape) return fail("tape is NULL");
    if (desc->has_boxes || desc->wheel_contacts)
        return fail("box agents and wheel contacts with movable bodies are not supported in "
                    "this build");
    hipStream_t st = (hipStream_t)stream;
    if (desc->dtype == SWARP_F32)
        return rollout_bwd_ob<float>(desc, T, state0, ob0, actions, traj, ob_traj, adj_traj,
                                     adj_final, adj_ob_traj, adj_state0, adj_ob0, adj_actions,
                                     tape, tape_bytes, st);
    return rollout_bwd_ob<double>(desc, T, state0, ob0, actions, traj, ob_traj, adj_traj,
                                  adj_final, adj_ob_traj, adj_state0, adj_ob0, adj_actions,
                                  tape, tape_bytes, st);
}

int swarp_rollout_bwd_ob_check(const swarp_desc_t *desc)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (desc->has_boxes || desc->wheel_contacts)
        return fail("box agents and wheel contacts with movable bodies are not supported in "
                    "this build");
    return desc->dtype == SWARP_F32 ? bwd_ob_fits<float>(desc) : bwd_ob_fits<double>(desc);
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
    const bool adaptive = desc->neighbor_method == SWARP_LISTS_GRID && !desc->grid_pinned;
    if (adaptive && !desc->grid_frame) return fail("grid_frame must be set for an adaptive grid frame");
    if (desc->dtype == SWARP_F32) {
        if (wide_path(desc) && wide_lds_check<float>(desc, true)) return -1;
        Cst<float> C;
        fill_cst<float>(desc, 0.0, C);
        if (wide_path(desc)) {
            float *fr = adaptive ? (float *)desc->grid_frame : nullptr;
            if (adaptive)
                launch_grid_frame<float>((const float *)pos, (int64_t)C.E * C.A,
                                         (float)desc->neighbor_radius, C.grid_bins, fr, st);
            launch_wide_lists<float>(C, (const float *)pos, fr, idx, cnt, true_cnt, st);
        } else {
            launch_neighbors<float>(PA, C, (const float *)pos, idx, cnt, true_cnt, st);
        }
    } else {
        if (wide_path(desc) && wide_lds_check<double>(desc, true)) return -1;
        Cst<double> C;
        fill_cst<double>(desc, 0.0, C);
        if (wide_path(desc)) {
            double *fr = adaptive ? (double *)desc->grid_frame : nullptr;
            if (adaptive)
                launch_grid_frame<double>((const double *)pos, (int64_t)C.E * C.A,
                                          desc->neighbor_radius, C.grid_bins, fr, st);
            launch_wide_lists<double>(C, (const double *)pos, fr, idx, cnt, true_cnt, st);
        } else {
            launch_neighbors<double>(PA, C, (const double *)pos, idx, cnt, true_cnt, st);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

int swarp_nav_obs(const swarp_desc_t *desc, const swarp_nav_t *nav, void *stream)
{
    g_err[0] = 0;
    if (check_desc(desc)) return -1;
    if (wide_path(desc))
        return fail("the fused navigation pass takes at most 64 agents per env with index-ordered lists");
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

int swarp_state_defaults(int32_t dtype, int64_t n, void *buf, void *stream)
{
    g_err[0] = 0;
    if (dtype != SWARP_F32 && dtype != SWARP_F64) return fail("dtype must be SWARP_F32 or SWARP_F64");
    if (n < 0 || n > (int64_t)1 << 40) return fail("n out of range");
    if (n == 0) return 0;
    if (!buf) return fail("buf must be set");
    if (((uintptr_t)buf & 15u) != 0u) return fail("buf must be 16-byte aligned");
    const int64_t per = dtype == SWARP_F32 ? 4 : 2;  // elements per 16-byte piece
    const int64_t items = (9 * n + per - 1) / per;
    const unsigned blocks = (unsigned)((items + 255) / 256);
    if (dtype == SWARP_F32)
        hipLaunchKernelGGL(k_state_defaults<float>, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                           n, (float *)buf);
    else
        hipLaunchKernelGGL(k_state_defaults<double>, dim3(blocks), dim3(256), 0,
                           (hipStream_t)stream, n, (double *)buf);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
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
    launch_edge_index(n_envs, n_agents, max_neighbors, idx, cnt, offsets, n_edges, edge_index,
                      (hipStream_t)stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(hipGetErrorString(e));
    return 0;
}

}  // extern "C"
