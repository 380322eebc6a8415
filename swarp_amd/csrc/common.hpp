// common.hpp -- lane layout, state I/O and the contact pass shared by every rollout kernel
// family (generic, holonomic, bodies, navigation).
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
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "physics.hpp"
#include "boxes.hpp"
#include "swarp_hip.h"

namespace swarp {

template <int PA> struct MaskT { typedef uint32_t type; };
template <> struct MaskT<64> { typedef uint64_t type; };

__device__ __forceinline__ int m_ctz(uint32_t m) { return __builtin_ctz(m); }
__device__ __forceinline__ int m_ctz(uint64_t m) { return __builtin_ctzll(m); }
__device__ __forceinline__ int m_popc(uint32_t m) { return __builtin_popcount(m); }
__device__ __forceinline__ int m_popc(uint64_t m) { return __builtin_popcountll(m); }

// Issue priority of a wave from its progress through the rollout (`done` of `total`
// steps), for the rollout kernels that keep several waves per SIMD.  Their waves start
// together and the launch ends with its slowest wave: per-wave timing copies of the
// config-2 forward show wave durations spread from 0.65x to 1.0x of the launch, barely
// correlated with the waves' own contact work (r = 0.26) -- the spread comes from the
// waves a wave shares its SIMD with.  A wave that has fallen behind its neighbours
// therefore issues ahead of them, so the waves of a SIMD finish together instead of
// leaving one to run alone.  Levels by the fraction done: [0, 1/2) 3, [1/2, 3/4) 2,
// [3/4, 7/8) 1, then 0 (measured against even quarters, against later bands and against
// a priority from the step's own contact count).  s_setprio orders instruction issue
// between the waves of one SIMD; no result depends on it.
__device__ __forceinline__ void progress_priority(int done, int total)
{
    const int d8 = 8 * done;  // d8 < k * total <=> the fraction done is below k / 8
    if (d8 < 4 * total) __builtin_amdgcn_s_setprio(3);
    else if (d8 < 6 * total) __builtin_amdgcn_s_setprio(2);
    else if (d8 < 7 * total) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

// Field pointers of one state; strides (in scalars) 2,1,2,1,1,1,1,4,3.
template <typename T> struct Fields {
    T *f[9];
};
template <typename T> struct CFields {
    const T *f[9];
};

template <typename T> struct Args {
    const T *params;
    const int32_t *tag, *mode;
    Obs<T> obs;
    CFields<T> s0;       // rollout input state
    const T *act;        // [T,E,A,ad]
    Fields<T> traj;      // outputs of steps 0..T-2 (stride E*A per step)
    Fields<T> fin;       // output of step T-1
    CFields<T> atraj;    // adjoints arriving at traj (nullable per field)
    CFields<T> afin;     // adjoint arriving at fin (nullable per field)
    Fields<T> a0;        // adjoint of s0 (nullable per field)
    T *aact;             // adjoint of actions
    int nsteps;
    // Force tape (nullable): per step, substep and agent the total force the forward
    // integrated (listed pairs, static obstacles, walls), [T][S][E A] pairs -- written by
    // the generic forward kernels (worlds without box agents or wheel contacts), read by
    // the backward's recompute in place of evaluating the forces again.
    T *fsum;
    // Obstacle-contact tape (nullable, with fsum, at most 32 obstacles): per step, substep
    // and agent a mask of the obstacles whose narrow phase took its contact branch, bit o
    // for obstacle o, [T][S][E A] words of omask_bytes(N) bytes, written by the two-wave
    // forward -- the backward reverses only those obstacles (the others' reverses add
    // zeros at most).
    void *omask;
    // Neighbour tape (nullable, with fsum): per step, substep and agent the uncapped
    // inclusion mask of its neighbour lists (MaskT<PA> words, [T][S][E A]; worlds with
    // agent contacts), written with fsum -- the backward's recompute reads it instead of
    // scanning.
    void *nmask;
};

// Width of one obstacle-contact mask word for N obstacles (0: no mask above 32).
__host__ __device__ constexpr int omask_bytes(int N)
{
    return N <= 8 ? 1 : (N <= 16 ? 2 : (N <= 32 ? 4 : 0));
}

__device__ __forceinline__ void omask_put(void *base, int N, size_t k, uint32_t m)
{
    const int w = omask_bytes(N);
    if (w == 1) ((uint8_t *)base)[k] = (uint8_t)m;
    else if (w == 2) ((uint16_t *)base)[k] = (uint16_t)m;
    else ((uint32_t *)base)[k] = m;
}

__device__ __forceinline__ uint32_t omask_get(const void *base, int N, size_t k)
{
    const int w = omask_bytes(N);
    if (w == 1) return ((const uint8_t *)base)[k];
    if (w == 2) return ((const uint16_t *)base)[k];
    return ((const uint32_t *)base)[k];
}

__device__ __forceinline__ int fstride(int k)
{
    // pos theta vel speed ang_vel z vz attitude body_rates
    return k == 0 || k == 2 ? 2 : (k == 7 ? 4 : (k == 8 ? 3 : 1));
}

// The field-pointer arrays below may hold generic pointers or global ones (see vgpr_ptr).
template <typename T, bool DRONE, typename P>
__device__ __forceinline__ void load_state(const P *f, size_t i, size_t off, St<T> &s)
{
    // `off` = element offset of the state in the trajectory (step * E * A)
    const size_t j = i + off;
    s.px = f[0][2 * j]; s.py = f[0][2 * j + 1];
    s.th = f[1][j];
    s.vx = f[2][2 * j]; s.vy = f[2][2 * j + 1];
    s.s = f[3][j];
    s.w = f[4][j];
    if (DRONE) {
        s.z = f[5][j]; s.vz = f[6][j];
        s.qx = f[7][4 * j]; s.qy = f[7][4 * j + 1]; s.qz = f[7][4 * j + 2]; s.qw = f[7][4 * j + 3];
        s.bx = f[8][3 * j]; s.by = f[8][3 * j + 1]; s.bz = f[8][3 * j + 2];
    } else {
        s.z = s.vz = s.qx = s.qy = s.qz = s.bx = s.by = s.bz = T(0);
        s.qw = T(1);
    }
}

template <typename T, bool DRONE>
__device__ __forceinline__ void store_state(T *const *f, size_t j, const St<T> &s)
{
    f[0][2 * j] = s.px; f[0][2 * j + 1] = s.py;
    f[1][j] = s.th;
    f[2][2 * j] = s.vx; f[2][2 * j + 1] = s.vy;
    f[3][j] = s.s;
    f[4][j] = s.w;
    if (DRONE) {
        f[5][j] = s.z; f[6][j] = s.vz;
        f[7][4 * j] = s.qx; f[7][4 * j + 1] = s.qy; f[7][4 * j + 2] = s.qz; f[7][4 * j + 3] = s.qw;
        f[8][3 * j] = s.bx; f[8][3 * j + 1] = s.by; f[8][3 * j + 2] = s.bz;
    }
}

// Adds a nullable adjoint state (fields may be NULL) at element j.
template <typename T, bool DRONE, typename P>
__device__ __forceinline__ void add_adj(const P *f, size_t j, St<T> &g)
{
    if (f[0]) { g.px += f[0][2 * j]; g.py += f[0][2 * j + 1]; }
    if (f[1]) g.th += f[1][j];
    if (f[2]) { g.vx += f[2][2 * j]; g.vy += f[2][2 * j + 1]; }
    if (f[3]) g.s += f[3][j];
    if (f[4]) g.w += f[4][j];
    if (DRONE) {
        if (f[5]) g.z += f[5][j];
        if (f[6]) g.vz += f[6][j];
        if (f[7]) { g.qx += f[7][4 * j]; g.qy += f[7][4 * j + 1]; g.qz += f[7][4 * j + 2]; g.qw += f[7][4 * j + 3]; }
        if (f[8]) { g.bx += f[8][3 * j]; g.by += f[8][3 * j + 1]; g.bz += f[8][3 * j + 2]; }
    }
}

template <typename T, bool DRONE>
__device__ __forceinline__ void store_adj(T *const *f, size_t j, const St<T> &g)
{
    if (f[0]) { f[0][2 * j] = g.px; f[0][2 * j + 1] = g.py; }
    if (f[1]) f[1][j] = g.th;
    if (f[2]) { f[2][2 * j] = g.vx; f[2][2 * j + 1] = g.vy; }
    if (f[3]) f[3][j] = g.s;
    if (f[4]) f[4][j] = g.w;
    if (DRONE) {
        if (f[5]) f[5][j] = g.z;
        if (f[6]) f[6][j] = g.vz;
        if (f[7]) { f[7][4 * j] = g.qx; f[7][4 * j + 1] = g.qy; f[7][4 * j + 2] = g.qz; f[7][4 * j + 3] = g.qw; }
        if (f[8]) { f[8][3 * j] = g.bx; f[8][3 * j + 1] = g.by; f[8][3 * j + 2] = g.bz; }
    }
}

template <typename T>
__device__ __forceinline__ void load_prm(const Args<T> &g, size_t row, int a, Prm<T> &p)
{
    const T *r = g.params + row * 22;
    p.radius = r[0]; p.mass = r[1]; p.max_speed = r[2]; p.max_accel = r[3];
    p.max_ang_vel = r[4]; p.max_ang_accel = r[5]; p.l_f = r[6]; p.l_r = r[7];
    p.max_steer = r[8]; p.thrust_max = r[9]; p.arm = r[10]; p.ixx = r[11];
    p.iyy = r[12]; p.izz = r[13]; p.kappa = r[14]; p.gravity = r[15]; p.min_speed = r[16];
    p.shape = r[17]; p.hx = r[18]; p.hy = r[19];
    p.gain_v = r[20]; p.gain_w = r[21];
    p.tag = g.tag[a];
    p.mode = g.mode[a];
}

template <typename T>
__device__ __forceinline__ void load_act(const T *act, size_t j, int ad, T (&a)[4])
{
    const T *p = act + j * ad;
    a[0] = p[0];
    a[1] = ad > 1 ? p[1] : T(0);
    a[2] = ad > 2 ? p[2] : T(0);
    a[3] = ad > 3 ? p[3] : T(0);
}

// LDS staging of one substep.  Fields: 0 px, 1 py, 2 vx, 3 vy, 4 th, 5 s, 6 w, 7 Fx, 8 Fy,
// then (drone) 9 z, 10 vz, 11..14 q, 15..17 br.  Each field is 64 consecutive scalars.
constexpr int F_PX = 0, F_PY = 1, F_VX = 2, F_VY = 3, F_TH = 4, F_S = 5, F_W = 6, F_FX = 7,
              F_FY = 8, NF_2D = 9, NF_DRONE = 18;

// Neighbour lists of one agent as a bitmask over the env's agents, ascending bit =
// ascending list order (neighbors.py:90-96).  Full scan over every pair of the env.
// A wave-uniform 32-bit value written into lane L of a per-lane value (v_writelane_b32;
// the lane is an inline constant: a second scalar operand would exceed the instruction's
// one scalar read); the other lanes keep theirs.  The compiler's hazard checks do not see
// into the asm: when v is VCC just written by a compare, the read as a scalar operand
// needs one wait state, which the s_nop provides.
template <int L> __device__ __forceinline__ uint32_t set_lane(uint32_t v, uint32_t old)
{
#if defined(__HIP_DEVICE_COMPILE__)
    asm("s_nop 0\n\tv_writelane_b32 %0, %1, %2" : "+v"(old) : "s"(v), "i"(L));
    return old;
#else
    return (int)(threadIdx.x % 64) == L ? v : old;
#endif
}
template <int L> __device__ __forceinline__ uint64_t set_lane64(uint64_t v, uint64_t old)
{
    const uint32_t lo = set_lane<L>((uint32_t)v, (uint32_t)old);
    const uint32_t hi = set_lane<L>((uint32_t)(v >> 32), (uint32_t)(old >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// f(IntC<B>{}), f(IntC<B + 1>{}), ..., f(IntC<E - 1>{}): a loop whose index is a constant.
template <int V> struct IntC {
    static constexpr int value = V;
};
template <int B, int E, typename Fn> __device__ __forceinline__ void static_for(Fn &&f)
{
    if constexpr (B < E) {
        f(IntC<B>{});
        static_for<B + 1, E>(f);
    }
}

// Same membership, evaluated only on the skin candidates.
template <typename T, int PA>
__device__ __forceinline__ typename MaskT<PA>::type scan_cand(const T *lx, const T *ly, int base,
                                                              T px, T py, T t_nbr,
                                                              typename MaskT<PA>::type cand)
{
    typedef typename MaskT<PA>::type M;
    M incl = 0;
    while (cand) {
        const int b = m_ctz(cand);
        cand &= cand - 1;
        T dx = lx[base + b] - px, dy = ly[base + b] - py;
        T d2 = dx * dx + dy * dy;
        incl |= d2 <= t_nbr ? (M(1) << b) : M(0);
    }
    return incl;
}

template <typename T, int PA>
__device__ __forceinline__ typename MaskT<PA>::type scan_all(const T *lx, const T *ly, int base,
                                                             int A, int me, T px, T py, T t_nbr,
                                                             T t_skin,
                                                             typename MaskT<PA>::type &cand)
{
    typedef typename MaskT<PA>::type M;
    M incl = 0, cd = 0;
    (void)A;  // pad slots (b >= A) hold NaN positions and never pass the test
    if constexpr (PA == 64) {
        // One env per wave, and the env's lanes all run this scan together.  A pair's
        // squared distance has the same bits from either end (x_b - x_a = -(x_a - x_b)
        // exactly), so the wave's ballot over agent b's column is agent b's row: it goes
        // to lane b as a scalar, with no per-lane bit assembly.  Only the skin mask is
        // built so; the inclusion mask is the candidates' test (a subset: t_nbr <= t_skin).
        // (positions read eight at a time, so that one wait covers eight LDS reads)
        static_for<0, 8>([&](auto cc) {
            constexpr int b0 = decltype(cc)::value * 8;
            T qx[8], qy[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                qx[k] = lx[base + b0 + k];
                qy[k] = ly[base + b0 + k];
            }
            static_for<0, 8>([&](auto kc) {
                constexpr int k = decltype(kc)::value, b = b0 + k;
                const T dx = qx[k] - px, dy = qy[k] - py;
                const T d2 = dx * dx + dy * dy;
                cd = (M)set_lane64<b>(__ballot(d2 <= t_skin), (uint64_t)cd);
            });
        });
        const M self = ~(M(1) << me);
        cand = cd & self;
        return t_nbr == t_skin ? cand : scan_cand<T, PA>(lx, ly, base, px, py, t_nbr, cand);
    } else {
#pragma unroll
        for (int b = 0; b < PA; ++b) {
            T dx = lx[base + b] - px, dy = ly[base + b] - py;
            T d2 = dx * dx + dy * dy;
            incl |= d2 <= t_nbr ? (M(1) << b) : M(0);
            cd |= d2 <= t_skin ? (M(1) << b) : M(0);
        }
    }
    const M self = ~(M(1) << me);
    cand = cd & self;
    return incl & self;
}

// First K members of an inclusion mask (the padded list of length K).
template <typename M> __device__ __forceinline__ M cap_list(M incl, int K)
{
    if (m_popc(incl) <= K) return incl;
    M rest = incl;
    for (int i = 0; i < K; ++i) rest &= rest - 1;
    return incl ^ rest;
}

// ------------------------------------------------------------- feature profiles
//
// The generic and body kernels are instantiated per feature profile F: a bit set of the
// optional paths an instance compiles.  fold_cst / fold_prm overwrite, in a kernel's own
// copy of the constants and of each lane's parameter row, every field an absent feature
// reads with the compile-time value that switches it off, so constant propagation removes
// those paths (FT_ALL keeps them all).  The host picks an instance whose profile covers
// the world's features (swarp_desc_t fleet_models / fleet_modes and the constants).
enum : unsigned {
    FT_RK4 = 1u << 0,    // Integrator.RK4
    FT_SAT = 1u << 1,    // contact_max_overlap > 0 (tanh law)
    FT_OBST = 1u << 2,   // static obstacles
    FT_WALL = 1u << 3,   // soft walls
    FT_CLAMP = 1u << 4,  // position clamp
    FT_MODES = 1u << 5,  // ACCELERATION / SERVO control of a holonomic or diff-drive agent
    FT_HOLO = 1u << 6,   // model tags present: holonomic, diff-drive, bicycle, drone
    FT_DIFF = 1u << 7,
    FT_BICY = 1u << 8,
    FT_DRONE = 1u << 9,
    FT_SHAPES = 1u << 10,  // box or segment obstacles in a body world (body kernels only)
    FT_MANYSH = 1u << 11,  // more than 64 obstacle shapes in a body world (body kernels only)
    FT_ALL = 0xfffu,
};
// Profiles compiled besides FT_ALL (float32): 2-D fleets with obstacles and walls under
// Euler, drone fleets (config 4), holonomic fleets with movable bodies
// (config 5).
constexpr unsigned FT_PROF_2D = FT_OBST | FT_WALL | FT_HOLO | FT_DIFF | FT_BICY;
constexpr unsigned FT_PROF_DRONE = FT_WALL | FT_DRONE;
constexpr unsigned FT_PROF_BODY = FT_WALL | FT_HOLO;

template <unsigned F, typename T> __device__ __forceinline__ Cst<T> fold_cst(Cst<T> C)
{
    if (!(F & FT_RK4)) C.rk4 = 0;
    if (!(F & FT_SAT)) C.max_overlap = T(0);
    if (!(F & FT_OBST)) C.N = 0;
    if (!(F & FT_WALL)) C.soft_walls = 0;
    if (!(F & FT_CLAMP)) C.clamp = 0;
    if (!(F & FT_SHAPES)) C.round_only = 1;
    return C;
}

template <unsigned F, typename T> __device__ __forceinline__ void fold_prm(Prm<T> &P)
{
    constexpr unsigned tags = F & (FT_HOLO | FT_DIFF | FT_BICY | FT_DRONE);
    if (tags == FT_HOLO) P.tag = 0;
    if (tags == FT_DIFF) P.tag = 1;
    if (tags == FT_BICY) P.tag = 2;
    if (tags == FT_DRONE) P.tag = 3;
    if (!(F & FT_HOLO)) __builtin_assume(P.tag != 0);
    if (!(F & FT_DIFF)) __builtin_assume(P.tag != 1);
    if (!(F & FT_BICY)) __builtin_assume(P.tag != 2);
    if (!(F & FT_DRONE)) __builtin_assume(P.tag != 3);
    if (!(F & FT_MODES)) P.mode = 0;
}

// Per-lane context shared by the forward and backward kernels.
template <typename T, int PA> struct Lane {
    int lane, agent, base, env;
    bool real;     // agent < A (lane holds a real agent slot of its env)
    bool active;   // real and env < E
    size_t idx;    // env * A + agent (clamped to a valid element for inactive lanes)
    Prm<T> pr;
    T dd;          // implicit damping denominator 1 + c*sub_dt/m (collisions.py:845)
    T inv_dd;      // 1 / dd (adjoint arithmetic only)
    Dv<T> ddv;     // dd as a prepared divisor (exact fp32 division by dd)
};

// `lane`: the work-item's lane within its wave's env slots (the thread index of a
// one-wave workgroup; split kernels pass threadIdx.x % 64, so both waves of a workgroup
// hold the same envs).
template <typename T, int PA>
__device__ __forceinline__ void lane_init(const Cst<T> &C, const Args<T> &g, Lane<T, PA> &L,
                                          int lane = -1)
{
    constexpr int EPW = 64 / PA;
    L.lane = lane < 0 ? (int)threadIdx.x : lane;
    L.agent = L.lane % PA;
    L.base = L.lane - L.agent;
    L.env = blockIdx.x * EPW + L.lane / PA;
    L.real = L.agent < C.A;
    L.active = L.real && L.env < C.E;
    const int ag = L.real ? L.agent : 0;
    const int ev = L.env < C.E ? L.env : 0;
    L.idx = (size_t)ev * C.A + ag;
    // per-env parameter tables (Stepper.set_agent_params_per_env) index [env, agent]
    load_prm(g, C.per_env ? (size_t)ev * C.A + ag : (size_t)ag, ag, L.pr);
    L.dd = T(1) + C.c * C.sub_dt / L.pr.mass;
    L.inv_dd = T(1) / L.dd;
    L.ddv = divisor(L.dd, true);
}

// A wave-uniform global-memory pointer held in vector registers: the value is unchanged,
// but the compiler no longer treats it as uniform, so it does not occupy scalar registers.
// Used for the many state-field pointers a step loop reads: kept in scalar registers they
// overflow the scalar file and are spilled, and every use then re-reads them lane by lane.
// The result is typed as a global (address space 1) pointer: laundered through integers
// a generic pointer would be read with flat loads, which also count as LDS operations, so
// every wait for an LDS result would wait for them too.
#if defined(__HIP_DEVICE_COMPILE__)
#define SWARP_GLOBAL __attribute__((address_space(1)))
#else
#define SWARP_GLOBAL
#endif
template <typename T> __device__ __forceinline__ const SWARP_GLOBAL T *vgpr_ptr(const T *p)
{
    const uint64_t u = (uint64_t)p;
    uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    asm volatile("" : "+v"(lo), "+v"(hi));
    return (const SWARP_GLOBAL T *)(((uint64_t)hi << 32) | lo);
}

// Orders one wave's LDS stores before its later LDS loads across lanes, for kernels whose
// workgroup is that one wave: the LDS executes a wave's instructions in the order they
// are issued, so the exchange needs only a wavefront-scope fence that keeps the compiler
// from moving accesses across it -- no s_barrier and no wait for the stores to complete.
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Whether every real agent of this lane's env stayed within the skin budget.
template <int PA> __device__ __forceinline__ bool env_all(bool ok, int base)
{
    const uint64_t bal = __ballot(ok);
    const uint64_t full = PA == 64 ? ~0ull : ((1ull << PA) - 1ull);
    return ((bal >> base) & full) == full;
}

// Contact + static forces of one substep, reading the env's positions/velocities from
// the LDS slot `sl`.  Returns the uncapped inclusion mask (for the true count).
// Obstacle angles as (cos, sin) per env slot of the wave, filled once per launch when
// 64/PA envs x N obstacles fit (OCS_MAX pairs); NULL table otherwise.
constexpr int OCS_MAX = 256;

// LDS one gfx950 workgroup may allocate, static and dynamic together (160 KiB); a launch
// of more than 64 KiB needs no opt-in on this runtime.
constexpr size_t LDS_MAX = 163840;

template <typename T, int PA>
__device__ __forceinline__ const T *ob_trig_table(const Cst<T> &C, const Args<T> &g,
                                                  const Lane<T, PA> &L, T *ocs)
{
    if (C.N <= 0 || (64 / PA) * C.N > OCS_MAX) return nullptr;
    const int ew = L.lane / PA;
    const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
    for (int q = L.agent; q < C.N; q += PA) {
        const T ang = g.obs.ang[eN + q];
        ocs[2 * (ew * C.N + q)] = m_cos(ang);
        ocs[2 * (ew * C.N + q) + 1] = m_sin(ang);
    }
    __syncthreads();
    return ocs + 2 * ew * C.N;
}

// This env's obstacle poses and bounding radii (OPOSE_W scalars per obstacle, see
// obstacle_in_reach) staged once per launch under ob_trig_table's condition, and before
// it: its barrier publishes both.  NULL when they do not fit.
template <typename T, int PA>
__device__ __forceinline__ const T *ob_pose_table(const Cst<T> &C, const Args<T> &g,
                                                  const Lane<T, PA> &L, T *opos)
{
    if (C.N <= 0 || (64 / PA) * C.N > OCS_MAX) return nullptr;
    const int ew = L.lane / PA;
    const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
    T *dst = opos + OPOSE_W * ew * C.N;
    for (int q = L.agent; q < C.N; q += PA) {
        const size_t j = eN + q;
        dst[OPOSE_W * q] = g.obs.pos[2 * j];
        dst[OPOSE_W * q + 1] = g.obs.pos[2 * j + 1];
        dst[OPOSE_W * q + 2] = g.obs.vel[2 * j];
        dst[OPOSE_W * q + 3] = g.obs.vel[2 * j + 1];
        dst[OPOSE_W * q + 4] = g.obs.om[j];
        dst[OPOSE_W * q + 5] = ob_bound(g.obs, q);
    }
    return dst;
}

// Box worlds (BOXES; false compiles the box paths out): `lbx` holds per lane the
// footprint (shape, hx, hy rows of 64), `lcs` the cos and sin of every lane's heading
// (rows of 64), and the slot `sl` also carries the headings and spins (F_TH, F_W rows).
// `act` (nullable) receives the mask of listed neighbours whose box contact exerts a
// force; for a box agent `om` / `wall` / `beyond` which of its first 64 obstacles, its
// walls, and any later obstacle do: the contacts without force have zero derivatives.
// `fsum` (nullable, worlds without box agents): the substep's total force as a forward
// recorded it -- then only the neighbour lists are built.
template <typename T, int PA, bool BOXES>
__device__ __forceinline__ typename MaskT<PA>::type forces(
    const Cst<T> &C, const Args<T> &g, const Lane<T, PA> &L, const T *sl, const T *lr,
    const St<T> &st, int s, bool full, typename MaskT<PA>::type &cand, T &Fx, T &Fy,
    const T *ocs = nullptr, const T *lbx = nullptr, const T *lcs = nullptr,
    typename MaskT<PA>::type *act = nullptr, uint64_t *om = nullptr, bool *wall = nullptr,
    bool *beyond = nullptr, T *tq = nullptr, const T *fsum = nullptr)
{
    const bool box_me = BOXES && L.pr.shape > T(0.5);
    T me[6] = {st.px, st.py, st.th, st.vx, st.vy, st.w};
    T cme = T(1), sme = T(0);
    if (BOXES) {
        cme = lcs[L.lane];
        sme = lcs[64 + L.lane];
    }
    typename MaskT<PA>::type am = 0;
    const bool wheel = BOXES && tq != nullptr;  // contact torques (wheel contacts)
    T tau = T(0);
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
    }
    if (!BOXES && fsum) {
        // the total force as the forward recorded it (the same bits): only the lists
        Fx = fsum[0];
        Fy = fsum[1];
        return incl;
    }
    if (C.collisions) {
        M m = cap_list(incl, C.K);
        const T ra = L.pr.radius;
        const Foot<T> fa = {L.pr.shape, ra, L.pr.hx, L.pr.hy};
        const T *lth = sl + F_TH * 64, *lw = sl + F_W * 64;
        while (m) {
            const int b = m_ctz(m);
            m &= m - 1;
            const int j = L.base + b;
            T gx, gy;
            if (BOXES && (box_me || lbx[j] > T(0.5))) {
                // a pair with a box (collision_forces_box_kernel, collisions.py:1044-1052)
                const Foot<T> fb = {lbx[j], lr[j], lbx[64 + j], lbx[128 + j]};
                const T ob[6] = {lx[j], ly[j], lth[j], lvx[j], lvy[j], lw[j]};
                agent_pair_force_box<T, T>(C, L.agent, b, fa, me, cme, sme, fb, ob, lcs[j],
                                           lcs[64 + j], L.dd, gx, gy);
                if (gx != T(0) || gy != T(0)) am |= typename MaskT<PA>::type(1) << b;
                if (wheel)
                    tau += pair_torque(C, L.agent, b, fa, me, cme, sme, fb, ob, lcs[j], lcs[64 + j],
                                       gx, gy);
            } else {
                pair_force(C, st.px - lx[j], st.py - ly[j], st.vx - lvx[j], st.vy - lvy[j],
                           ra + lr[j] + C.margin, L.ddv, gx, gy);
            }
            fx += gx;
            fy += gy;
        }
    }
    T sx = T(0), sy = T(0);
    if (box_me) {
        // a box agent's obstacles and walls (_static_forces_shaped, collisions.py:950-996)
        const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
        box_static_forces<T, T>(C, g.obs, eN, ocs, L.pr.hx, L.pr.hy, me, cme, sme, L.dd, sx, sy,
                                om, wall, beyond);
        if (wheel)
            tau = tau + box_static_torque(C, g.obs, eN, ocs, L.pr.hx, L.pr.hy, me, cme, sme, L.dd);
    } else if (C.N > 0) {
        const size_t eN = (size_t)(L.env < C.E ? L.env : 0) * C.N;
        for (int o = 0; o < C.N; ++o) {
            T gx, gy;
            obstacle_force(C, g.obs, eN, o, st.px, st.py, st.vx, st.vy, L.pr.radius, L.ddv, gx,
                           gy, ocs);
            sx += gx;
            sy += gy;
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
    if (act) *act = am;
    if (wheel) *tq = tau;
    return incl;
}

// ----------------------------------------------------------------- backward rollout

template <typename T, bool DRONE>
__device__ __forceinline__ void slot_put(T *sl, int lane, const St<T> &s)
{
    sl[F_PX * 64 + lane] = s.px; sl[F_PY * 64 + lane] = s.py;
    sl[F_VX * 64 + lane] = s.vx; sl[F_VY * 64 + lane] = s.vy;
    sl[F_TH * 64 + lane] = s.th; sl[F_S * 64 + lane] = s.s; sl[F_W * 64 + lane] = s.w;
    if (DRONE) {
        sl[9 * 64 + lane] = s.z; sl[10 * 64 + lane] = s.vz;
        sl[11 * 64 + lane] = s.qx; sl[12 * 64 + lane] = s.qy;
        sl[13 * 64 + lane] = s.qz; sl[14 * 64 + lane] = s.qw;
        sl[15 * 64 + lane] = s.bx; sl[16 * 64 + lane] = s.by; sl[17 * 64 + lane] = s.bz;
    }
}

template <typename T, bool DRONE>
__device__ __forceinline__ void slot_get(const T *sl, int lane, St<T> &s)
{
    s.px = sl[F_PX * 64 + lane]; s.py = sl[F_PY * 64 + lane];
    s.vx = sl[F_VX * 64 + lane]; s.vy = sl[F_VY * 64 + lane];
    s.th = sl[F_TH * 64 + lane]; s.s = sl[F_S * 64 + lane]; s.w = sl[F_W * 64 + lane];
    if (DRONE) {
        s.z = sl[9 * 64 + lane]; s.vz = sl[10 * 64 + lane];
        s.qx = sl[11 * 64 + lane]; s.qy = sl[12 * 64 + lane];
        s.qz = sl[13 * 64 + lane]; s.qw = sl[14 * 64 + lane];
        s.bx = sl[15 * 64 + lane]; s.by = sl[16 * 64 + lane]; s.bz = sl[17 * 64 + lane];
    } else {
        s.z = s.vz = s.qx = s.qy = s.qz = s.bx = s.by = s.bz = T(0);
        s.qw = T(1);
    }
}

// Whether agent `me` is among the first K members of inclusion mask `incl`.
template <typename M> __device__ __forceinline__ bool in_list(M incl, int me, int K)
{
    return ((incl >> me) & M(1)) && m_popc(incl & ((M(1) << me) - M(1))) < K;
}

}  // namespace swarp
