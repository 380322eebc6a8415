// Runs the library's C entry points on host buffers of exactly the extents the ABI
// documents, with the kernels executed by the host emulation (emu/hip/hip_runtime.h),
// under AddressSanitizer and UndefinedBehaviorSanitizer.  Any access outside an input,
// output, workspace, LDS or static array the kernels own is reported and fails the run.
//
// The cases follow the GPU parity tests' shapes (reduced in env count), in the order of
// the run whose GPU memory fault is on record: movable bodies first, then the float32
// drone rollout with every adjoint field, then the other kernel families.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>
#include <vector>

#include "swarp_hip.h"

namespace {

std::mt19937 rng(12345);
bool plant_short_actions = false;  // negative control: actions one element short

template <typename T> struct Buf {
    std::vector<T> v;
    explicit Buf(size_t n = 0) : v(n) {}
    T *p() { return v.empty() ? nullptr : v.data(); }
};

// heap block of exactly n elements (ASan checks its extent)
template <typename T> T *make(size_t n, std::vector<void *> &owned)
{
    T *p = (T *)malloc(n * sizeof(T) + (n == 0));
    owned.push_back(p);
    return p;
}

template <typename T> void fill(T *p, size_t n, double lo, double hi)
{
    std::uniform_real_distribution<double> u(lo, hi);
    for (size_t i = 0; i < n; ++i) p[i] = (T)u(rng);
}

const int WID[9] = {2, 1, 2, 1, 1, 1, 1, 4, 3};

struct Case {
    const char *name;
    int E, A, T, S, K, ad, nobs;
    bool drone, boxes, walls, bodies, rk4, grid;
    int models;  // 0 holonomic, 1 diff/bicycle mix, 3 drone
    bool per_env = false;  // per-env parameter rows (the body pass then reads the shared)
    bool shaped = false;   // movable bodies of box and segment shapes too
    bool fleet = false;    // fleet model / mode bit sets filled in (the profile instances,
                           // and for 2-D fleets among obstacles the two-wave forward)
    bool wheel = false;    // wheel contacts (forward only)
};

template <typename T>
int run_case(const Case &c)
{
    std::vector<void *> own;
    const int E = c.E, A = c.A, nT = c.T, ad = c.ad;
    const size_t EA = (size_t)E * A;
    swarp_desc_t d;
    memset(&d, 0, sizeof d);
    d.abi_version = SWARP_ABI_VERSION;
    d.dtype = sizeof(T) == 4 ? SWARP_F32 : SWARP_F64;
    d.n_envs = E;
    d.n_agents = A;
    d.act_dim = ad;
    d.substeps = c.S;
    d.max_neighbors = c.K;
    d.collisions = 1;
    d.soft_walls = c.walls ? 1 : 0;
    d.has_drone = c.drone ? 1 : 0;
    d.has_boxes = c.boxes ? 1 : 0;
    if (c.wheel) {
        d.wheel_contacts = 1;
        d.lat_grip = 2.94;
        d.turn_cap = 0.02;
    }
    d.dt = 0.05;
    d.k = 100.0;
    d.c = 1.0;
    d.margin = 0.025;
    d.neighbor_radius = 0.3;
    d.bounds_min[0] = d.bounds_min[1] = -1.0;
    d.bounds_max[0] = d.bounds_max[1] = 1.0;
    d.integrator = c.rk4 ? SWARP_RK4 : SWARP_EULER;
    d.skin_speed = 1.0;
    d.lin_damping = 0.5;
    d.ang_damping = 0.5;
    if (c.grid) {
        d.neighbor_method = SWARP_LISTS_GRID;
        d.grid_bins = 8;
        d.grid_pinned = 1;
        d.grid_origin[0] = d.grid_origin[1] = -1.0;
        d.grid_cell = 0.3;
    }
    // parameter rows: radius, mass, max_speed, max_accel, max_ang_vel, max_ang_accel, l_f,
    // l_r, max_steer, thrust_max, arm, ixx, iyy, izz, kappa, gravity, min_speed, shape,
    // hx, hy, gain_v, gain_w
    T *params = make<T>((size_t)A * 22, own);
    int32_t *tag = make<int32_t>(A, own), *mode = make<int32_t>(A, own);
    for (int a = 0; a < A; ++a) {
        const T row[22] = {T(0.05), T(1), T(1), T(2), T(3), T(6), T(0.1), T(0.1), T(0.7), T(10),
                           T(0.1), T(0.01), T(0.01), T(0.02), T(0.01), T(9.81), T(0),
                           T(c.boxes && a % 2 ? 1 : 0), T(0.05), T(0.03), T(2), T(2)};
        memcpy(params + (size_t)a * 22, row, sizeof row);
        tag[a] = c.models == 3 ? 3 : (c.models == 1 ? 1 + a % 2 : 0);
        mode[a] = 0;
    }
    d.params = params;
    if (c.per_env) {
        T *rows = make<T>(EA * 22, own);
        for (size_t q = 0; q < EA; ++q) {
            memcpy(rows + q * 22, params + (q % A) * 22, sizeof(T) * 22);
            rows[q * 22] = T(0.04 + 0.01 * (double)(q % 3));     // radius
            rows[q * 22 + 1] = T(1.0 + 0.5 * (double)(q % 2));  // mass
        }
        d.params = rows;
        d.params_per_env = 1;
        d.body_params = params;
    }
    d.model_tag = tag;
    d.ctrl_mode = mode;
    if (c.fleet) {
        int mb = 0;
        for (int a = 0; a < A; ++a) mb |= 1 << tag[a];
        d.fleet_models = mb;
        d.fleet_modes = 1;  // every agent in VELOCITY mode
    }
    const int N = c.nobs;
    d.n_obstacles = N;
    if (N > 0) {
        T *opos = make<T>((size_t)E * N * 2, own), *orad = make<T>(N, own);
        T *oang = make<T>((size_t)E * N, own), *ohalf = make<T>((size_t)N * 2, own);
        T *ovel = make<T>((size_t)E * N * 2, own), *oom = make<T>((size_t)E * N, own);
        int32_t *otype = make<int32_t>(N, own);
        fill(opos, (size_t)E * N * 2, -0.5, 0.5);
        fill(oang, (size_t)E * N, -3.0, 3.0);
        memset(ovel, 0, sizeof(T) * E * N * 2);
        memset(oom, 0, sizeof(T) * E * N);
        for (int o = 0; o < N; ++o) {
            orad[o] = T(0.1);
            ohalf[2 * o] = T(0.15);
            ohalf[2 * o + 1] = T(c.bodies && !c.shaped ? 0 : 0.08);
            otype[o] = c.bodies && !c.shaped ? 0 : o % 3;
        }
        d.obs_pos = opos;
        d.obs_radius = orad;
        d.obs_angle = oang;
        d.obs_half = ohalf;
        d.obs_vel = ovel;
        d.obs_ang_vel = oom;
        d.obs_type = otype;
        if (c.bodies) {
            int32_t *kind = make<int32_t>(N, own), *body = make<int32_t>(N, own);
            T *mass = make<T>(N, own), *inert = make<T>(N, own), *off = make<T>((size_t)N * 2, own);
            for (int o = 0; o < N; ++o) {
                kind[o] = 1;
                body[o] = 0;
                mass[o] = T(1);
                inert[o] = T(0.05);
                off[2 * o] = T(o == 1 ? 0.2 : (o == 2 ? -0.2 : 0));
                off[2 * o + 1] = T(o == 3 ? 0.2 : (o == 4 ? -0.2 : 0));
            }
            d.obs_kind = kind;
            d.obs_body = body;
            d.obs_mass = mass;
            d.obs_inertia = inert;
            d.obs_body_off = off;
        }
    }
    const int nf = c.drone ? 9 : 5;
    auto fields = [&](size_t lead, bool with_values) {
        swarp_state_t s;
        memset(&s, 0, sizeof s);
        void **f = (void **)&s;
        for (int k = 0; k < nf; ++k) {
            T *p = make<T>(lead * EA * WID[k], own);
            if (with_values) {
                fill(p, lead * EA * WID[k], -0.8, 0.8);
                if (k == 7)  // unit quaternions
                    for (size_t q = 0; q < lead * EA; ++q) {
                        p[4 * q] = p[4 * q + 1] = p[4 * q + 2] = T(0.01);
                        p[4 * q + 3] = T(1);
                    }
                if (k == 5)
                    for (size_t q = 0; q < lead * EA; ++q) p[q] = T(1);
            } else {
                memset(p, 0, sizeof(T) * lead * EA * WID[k]);
            }
            f[k] = p;
        }
        return s;
    };
    swarp_state_t s0 = fields(1, true), fin = fields(1, false);
    swarp_state_t traj = nT > 1 ? fields(nT - 1, false) : swarp_state_t{};
    const size_t nact = (size_t)nT * EA * ad - (plant_short_actions ? 1 : 0);
    T *act = make<T>(nact, own);
    fill(act, nact, c.drone ? 0.0 : -1.0, c.drone ? 10.0 : 1.0);
    int rc;
    if (c.bodies) {
        const size_t NW = (size_t)12 * N;
        T *ob0 = make<T>(EA / A * NW, own), *obt = make<T>((size_t)nT * E * NW, own);
        for (int e = 0; e < E; ++e)
            for (size_t q = 0; q < NW; ++q) ob0[e * NW + q] = T(0);
        rc = swarp_rollout_fwd_ob(&d, nT, &s0, ob0, act, nT > 1 ? &traj : nullptr, &fin, obt, nullptr);
        if (rc) return fprintf(stderr, "%s fwd_ob: %s\n", c.name, swarp_last_error()), 1;
        swarp_state_t atr = nT > 1 ? fields(nT - 1, true) : swarp_state_t{};
        swarp_state_t afin = fields(1, true), a0 = fields(1, false);
        T *aobt = make<T>((size_t)nT * E * NW, own), *aob0 = make<T>((size_t)E * NW, own);
        fill(aobt, (size_t)nT * E * NW, -1, 1);
        T *aact = make<T>((size_t)nT * EA * ad, own);
        rc = swarp_rollout_bwd_ob(&d, nT, &s0, ob0, act, nT > 1 ? &traj : nullptr, obt,
                                  nT > 1 ? &atr : nullptr, &afin, aobt, &a0, aob0, aact, nullptr);
        if (rc) return fprintf(stderr, "%s bwd_ob: %s\n", c.name, swarp_last_error()), 1;
    } else if (c.wheel) {
        rc = swarp_rollout_fwd(&d, nT, &s0, act, nT > 1 ? &traj : nullptr, &fin, nullptr);
        if (rc) return fprintf(stderr, "%s fwd: %s\n", c.name, swarp_last_error()), 1;
    } else {
        rc = swarp_rollout_fwd(&d, nT, &s0, act, nT > 1 ? &traj : nullptr, &fin, nullptr);
        if (rc) return fprintf(stderr, "%s fwd: %s\n", c.name, swarp_last_error()), 1;
        swarp_state_t atr = nT > 1 ? fields(nT - 1, true) : swarp_state_t{};
        swarp_state_t afin = fields(1, true), a0 = fields(1, false);
        T *aact = make<T>((size_t)nT * EA * ad, own);
        rc = swarp_rollout_bwd(&d, nT, &s0, act, nT > 1 ? &traj : nullptr, nT > 1 ? &atr : nullptr,
                               &afin, &a0, aact, nullptr);
        if (rc) return fprintf(stderr, "%s bwd: %s\n", c.name, swarp_last_error()), 1;
        // the adjoint of a nullable field left NULL is not read
        swarp_state_t afin2 = fields(1, true);
        ((void **)&afin2)[1] = nullptr;
        rc = swarp_rollout_bwd(&d, nT, &s0, act, nT > 1 ? &traj : nullptr, nullptr, &afin2, &a0,
                               aact, nullptr);
        if (rc) return fprintf(stderr, "%s bwd (sparse adjoints): %s\n", c.name, swarp_last_error()), 1;
        // the taped pair, where the configuration keeps a tape
        uint64_t tb = 0;
        rc = swarp_tape_bytes(&d, nT, &tb);
        if (rc) return fprintf(stderr, "%s tape_bytes: %s\n", c.name, swarp_last_error()), 1;
        if (tb) {
            void *tape = make<unsigned char>(tb, own);
            rc = swarp_rollout_fwd_tape(&d, nT, &s0, act, nT > 1 ? &traj : nullptr, &fin, tape, tb,
                                        nullptr);
            if (rc) return fprintf(stderr, "%s fwd_tape: %s\n", c.name, swarp_last_error()), 1;
            rc = swarp_rollout_bwd_tape(&d, nT, &s0, act, nT > 1 ? &traj : nullptr,
                                        nT > 1 ? &atr : nullptr, &afin, &a0, aact, tape, tb, nullptr);
            if (rc) return fprintf(stderr, "%s bwd_tape: %s\n", c.name, swarp_last_error()), 1;
        }
    }
    // neighbour lists of the initial state
    int32_t *idx = make<int32_t>(EA * c.K, own), *cnt = make<int32_t>(EA, own), *tru = make<int32_t>(EA, own);
    rc = swarp_neighbors(&d, s0.pos, idx, cnt, tru, nullptr);
    if (rc) return fprintf(stderr, "%s neighbors: %s\n", c.name, swarp_last_error()), 1;
    for (auto p : own) free(p);
    printf("%-28s ok\n", c.name);
    fflush(stdout);
    return 0;
}

}  // namespace

int main(int argc, char **argv)
{
    plant_short_actions = argc > 1 && strcmp(argv[1], "--plant-short-actions") == 0;
    const Case cases[] = {
        // name                 E   A   T  S  K  ad N  drone  boxes  walls  bodies rk4   grid   models
        {"bodies f32 A=12",      5, 12, 4, 2, 8, 2, 5, false, false, true,  true,  false, false, 0},
        {"bodies f32 A=64",      2, 64, 3, 2, 16, 2, 5, false, false, true,  true,  false, false, 0},
        {"bodies drones f32 A=8", 9, 8, 3, 2, 8, 4, 5, true,  false, true,  true,  false, false, 3},
        {"bodies per-env f32",   6, 12, 3, 2, 8, 2, 5, false, false, true,  true,  false, false, 0, true},
        {"bodies shaped f32",    6, 12, 3, 2, 8, 2, 5, false, false, true,  true,  false, false, 0, false, true},
        {"bodies f32 A=64 profile", 2, 64, 3, 2, 16, 2, 5, false, false, true, true, false, false, 0,
         false, false, true},
        {"bodies f32 A=12 profile", 5, 12, 4, 2, 8, 2, 5, false, false, true, true, false, false, 0,
         false, false, true},
        {"drones f32 64x8",     16, 8, 6, 2, 8, 4, 0, true,  false, false, false, false, false, 3},
        {"drones f64 A=3",       4, 3, 5, 1, 4, 4, 0, true,  false, false, false, false, false, 3},
        {"mixed f32 obstacles",  9, 32, 4, 2, 16, 2, 6, false, false, true,  false, false, false, 1},
        {"mixed f32 obstacles profile", 9, 32, 4, 2, 16, 2, 6, false, false, true, false, false, false, 1,
         false, false, true},
        {"mixed f32 rk4",        5, 20, 3, 2, 8, 2, 3, false, false, true,  false, true,  false, 1},
        {"boxes f32",            7, 16, 3, 2, 8, 2, 3, false, true,  true,  false, false, false, 1},
        {"holonomic f64 A=5",   11, 5, 4, 3, 4, 2, 0, false, false, true,  false, false, false, 0},
        {"wide f32 A=100",       2, 100, 3, 2, 12, 2, 3, false, false, true,  false, false, false, 1},
        {"wide grid f32 A=70",   2, 70, 3, 2, 8, 2, 0, false, false, true,  false, false, true,  0},
        {"wide bodies f32 A=100", 2, 100, 3, 2, 12, 2, 5, false, false, true, true, false, false, 0},
        {"wide bodies grid f32 A=70", 2, 70, 3, 2, 8, 2, 5, false, false, true, true, false, true, 0},
        {"wide bodies drones f32 A=72", 2, 72, 3, 2, 8, 4, 5, true, false, true, true, false, false, 3},
        {"wide bodies f64 A=65",  2, 65, 2, 2, 8, 2, 6, false, false, true, true, false, false, 0},
        {"wide boxes f32 A=100",  2, 100, 3, 2, 12, 2, 3, false, true, true, false, false, false, 1},
        {"wide boxes grid f32 A=70", 2, 70, 3, 2, 8, 2, 3, false, true, true, false, false, true, 1},
        {"wide boxes f64 A=66",   2, 66, 2, 2, 8, 2, 2, false, true, true, false, false, false, 1},
        {"wide wheel f32 A=72",   2, 72, 3, 2, 8, 2, 3, false, true, true, false, false, false, 1,
         false, false, false, true},
        {"wide 2 per lane f32 A=1100", 1, 1100, 2, 2, 8, 2, 2, false, false, true, false, false, false, 1},
        {"wide 4 per lane grid f32 A=2100", 1, 2100, 2, 1, 8, 2, 0, false, false, true, false, false, true, 0},
    };
    int bad = 0;
    for (const Case &c : cases) {
        const bool f64 = strstr(c.name, "f64") != nullptr;
        bad += f64 ? run_case<double>(c) : run_case<float>(c);
    }
    printf("%d case(s) failed\n", bad);
    return bad ? 1 : 0;
}
