// lean.hpp -- specialised rollout kernels for fleets of holonomic agents in velocity
// mode without obstacles (the reference's NavigationScenario default, BASELINE config 1/2).
// Instantiated by k_holo.hip; the host side sizes the tape with TapeRec.  A workgroup is one
// wave, so lanes exchange values through LDS with wave_lds_sync instead of a barrier.
//
// Same arithmetic, in the same order, as the generic kernels (so the results are
// bit-identical), with what this fleet does not need removed:
//   * clamp_norm(action) is computed once per step (the action is constant over the
//     substeps) instead of once per substep;
//   * only pos / vel are carried through the substeps; theta passes through, speed is
//     the length of the last substep's velocity, ang_vel is zero;
//   * the neighbour scan has a compile-time trip count: pad lanes of a partially filled
//     env slot hold NaN positions, which fail every membership test, so the LDS reads of
//     a scan are issued back to back and waited on once;
//   * the next step's inputs are loaded one step ahead.
#pragma once
#include "common.hpp"

namespace swarp {

template <typename T> struct alignas(2 * sizeof(T)) P2 {
    T x, y;
};

template <typename T> __device__ __forceinline__ P2<T> ld2(const T *p, size_t j)
{
    return *reinterpret_cast<const P2<T> *>(p + 2 * j);
}
template <typename T> __device__ __forceinline__ void st2(T *p, size_t j, T x, T y)
{
    P2<T> v;
    v.x = x;
    v.y = y;
    *reinterpret_cast<P2<T> *>(p + 2 * j) = v;
}

// Full scan of the env's PA slots: inclusion (radius) and skin-candidate masks.
template <typename T, int PA>
__device__ __forceinline__ void lean_scan(const P2<T> *lp, int base, int me, T px, T py,
                                          const Cst<T> &C, typename MaskT<PA>::type &incl,
                                          typename MaskT<PA>::type &cand)
{
    typedef typename MaskT<PA>::type M;
    M in = 0, cd = 0;
    constexpr int CH = PA < 16 ? PA : 16;  // LDS reads batched per chunk, one wait each
#pragma unroll
    for (int b0 = 0; b0 < PA; b0 += CH) {
        P2<T> q[CH];
#pragma unroll
        for (int k = 0; k < CH; ++k) q[k] = lp[base + b0 + k];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const T dx = q[k].x - px, dy = q[k].y - py;
            const T d2 = dx * dx + dy * dy;
            in |= d2 <= C.t_nbr ? (M(1) << (b0 + k)) : M(0);
            cd |= d2 <= C.t_skin ? (M(1) << (b0 + k)) : M(0);
        }
    }
    const M self = ~(M(1) << me);
    incl = in & self;
    cand = cd & self;
}

template <typename T, int PA>
__device__ __forceinline__ typename MaskT<PA>::type lean_cand(const P2<T> *lp, int base, T px,
                                                              T py, T t_nbr,
                                                              typename MaskT<PA>::type cand)
{
    typedef typename MaskT<PA>::type M;
    M in = 0;
    while (cand) {
        const int b = m_ctz(cand);
        cand &= cand - 1;
        const P2<T> q = lp[base + b];
        const T dx = q.x - px, dy = q.y - py;
        const T d2 = dx * dx + dy * dy;
        in |= d2 <= t_nbr ? (M(1) << b) : M(0);
    }
    return in;
}

// ---------------------------------------------- skin scan of 16-agent envs by row rotation
//
// An env of PA = 16 agents is one DPP row of 16 lanes, and row_ror:k hands lane a the
// value of lane (a - k) mod 16 without touching LDS.  The distance of a pair is the same
// bits seen from either end (the subtraction only changes sign), so each lane evaluates 8
// of its 15 pairs: offsets k = 1..8 towards (a - k), whose result is its bit for
// neighbour a - k; lanes a + k (k = 1..7) evaluated the pairs towards a, and their compare
// bits come back by row_ror:(16 - k).  Bits are collected relative to the lane (bit j =
// neighbour (a + j) mod 16) and rotated into agent order at the end.
// (bound_ctrl set: every source lane of a row rotation exists, and the flag lets the
// compiler fold the move into its user as a DPP operand)
template <int K> __device__ __forceinline__ float ror16(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 0x120 + K, 0xf, 0xf, true));
}
template <int K> __device__ __forceinline__ uint32_t ror16u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + K, 0xf, 0xf, true);
}

template <int K>
__device__ __forceinline__ void skin_offset(float px, float py, float t, uint32_t &own,
                                            uint32_t &got)
{
    const float dx = ror16<K>(px) - px, dy = ror16<K>(py) - py;  // neighbour (a - K)
    const float d2 = dx * dx + dy * dy;
    const bool in = d2 <= t;
    own |= in ? (1u << (16 - K)) : 0u;
    if (K < 8) got |= ror16u<16 - K>(in ? (1u << K) : 0u);  // lane a + K's pair with a
}

// Mask (agent order, self excluded) of the env's agents within squared distance t, for
// PA = 16 float lanes; `rot` = 16 - (agent index of this lane).
__device__ __forceinline__ uint32_t skin_dpp16(float px, float py, float t, uint32_t rot)
{
    uint32_t own = 0u, got = 0u;
    skin_offset<1>(px, py, t, own, got);
    skin_offset<2>(px, py, t, own, got);
    skin_offset<3>(px, py, t, own, got);
    skin_offset<4>(px, py, t, own, got);
    skin_offset<5>(px, py, t, own, got);
    skin_offset<6>(px, py, t, own, got);
    skin_offset<7>(px, py, t, own, got);
    skin_offset<8>(px, py, t, own, got);
    const uint32_t r = own | got;  // bit j: neighbour (a + j) mod 16
    return __builtin_amdgcn_ubfe(r | (r << 16), rot, 16u);
}

// One substep of the force pass: neighbour lists (into `incl`) and the total force.
// Also records which listed contacts are active (`act`) and the wall contact bits, the
// branches the reverse pass follows.  SAT: contact_max_overlap > 0 (the tanh law).
// For 16-agent float envs a full scan builds only the skin mask (skin_dpp16) and the
// lists come from the candidate check, as on the other substeps.
template <typename T, int PA, bool SAT>
__device__ __forceinline__ void lean_forces(const Cst<T> &C, const P2<T> *lp, const P2<T> *lv,
                                            const T *lr, int base, int me, T ra,
                                            const Dv<T> &dd, T px, T py, T vx, T vy, bool full,
                                            bool first,
                                            typename MaskT<PA>::type &cand,
                                            typename MaskT<PA>::type &incl,
                                            typename MaskT<PA>::type &act, unsigned &wbits,
                                            T &Fx, T &Fy)
{
    typedef typename MaskT<PA>::type M;
    constexpr bool DPP16 = PA == 16 && sizeof(T) == 4;
    T fx = T(0), fy = T(0);
    incl = 0;
    act = 0;
    wbits = 0u;
    if (C.collisions) {
        if (DPP16 && full) {
            const M cd = (M)skin_dpp16((float)px, (float)py, (float)C.t_skin, 16u - (uint32_t)me);
            if (first) cand = cd;
            incl = lean_cand<T, PA>(lp, base, px, py, C.t_nbr, cd);
        } else if (full) {
            M cd;
            lean_scan<T, PA>(lp, base, me, px, py, C, incl, cd);
            if (first) cand = cd;
        } else {
            incl = lean_cand<T, PA>(lp, base, px, py, C.t_nbr, cand);
        }
        M m = cap_list(incl, C.K);
        while (m) {
            const int b = m_ctz(m);
            m &= m - 1;
            const int j = base + b;
            const P2<T> q = lp[j], w = lv[j];
            T gx, gy;
            const bool on = pair_force_rec_r<T, SAT>(C, px - q.x, py - q.y, vx - w.x, vy - w.y,
                                             ra + lr[j] + C.margin, dd, gx, gy);
            act |= on ? (M(1) << b) : M(0);
            fx += gx;
            fy += gy;
        }
    }
    T sx = T(0), sy = T(0);
    if (C.soft_walls) wall_force_axes<T, SAT>(C, px, py, vx, vy, ra, dd, sx, sy, wbits);
    Fx = fx + sx;
    Fy = fy + sy;
}

// ------------------------------------------------------------------ rollout tape
//
// What the reverse pass of a step reads besides the step's input checkpoint, written by
// the forward so that the backward does not recompute the step (substep count <= 4):
//   rec [T][workgroup][chunk][lane] 16-byte chunks: per step and lane one record of
//       TapeRec::R bytes (NC = R / 16 chunks) holding
//       TAPE_MAX_S mask words   per substep the inclusion mask (uncapped lists) and the
//                               active-contact mask, packed as one TapeW word; an agent is
//                               never its own neighbour, so its own bit carries the
//                               substep's wall-contact bits (x in the inclusion mask, y in
//                               the active mask)
//       TAPE_MAX_S - 1 pairs    input velocity of substeps 1..S-1 (positions follow exactly
//                               as p_{s+1} = p_s + v_{s+1} * sub_dt, the forward's own update)
//   vl  [workgroup][lane] pairs output velocity of the last step (the backward takes no
//                               final state; every other step's output velocity is a
//                               checkpoint)
// The velocity after substep s is the step's clamped command plus F_s dt / m, and F_s is
// exactly +0 when substep s has no active contact and no wall bit (every term is +-0 and
// the sum starts at +0).  Such velocities are not stored: the forward writes a velocity
// chunk only for the lanes whose masks say a force acted, the backward loads it only
// for those lanes and otherwise rebuilds the velocity as command + 0 -- the same bits.
// Most lanes feel no force in most steps, so most velocity cache lines are never moved.
// Slots past the configuration's substep count are left unwritten.  The tape is private
// to the two kernels, so it is indexed by lane rather than by agent: each 16-byte chunk
// store of the forward and load of the backward moves 1 KB of contiguous memory per wave.
// Lanes without an agent write records the backward never reads.
constexpr int TAPE_MAX_S = 4;

template <typename T> struct Tape {
    void *rec;
    T *vl;
};

// Mask word of one agent and substep: inclusion bits, then active-contact bits.
template <int PA> struct TapeW {
    typedef uint32_t type;  // PA <= 16: incl | act << 16
    static __device__ __forceinline__ type pack(uint32_t in, uint32_t ac) { return in | ac << 16; }
    static __device__ __forceinline__ uint32_t incl(type w) { return w & 0xffffu; }
    static __device__ __forceinline__ uint32_t act(type w) { return w >> 16; }
};
template <> struct TapeW<32> {
    typedef uint64_t type;
    static __device__ __forceinline__ type pack(uint32_t in, uint32_t ac)
    {
        return (uint64_t)in | (uint64_t)ac << 32;
    }
    static __device__ __forceinline__ uint32_t incl(type w) { return (uint32_t)w; }
    static __device__ __forceinline__ uint32_t act(type w) { return (uint32_t)(w >> 32); }
};
struct alignas(16) MaskPair64 {
    uint64_t in, ac;
};
template <> struct TapeW<64> {
    typedef MaskPair64 type;
    static __device__ __forceinline__ type pack(uint64_t in, uint64_t ac) { return {in, ac}; }
    static __device__ __forceinline__ uint64_t incl(type w) { return w.in; }
    static __device__ __forceinline__ uint64_t act(type w) { return w.ac; }
};

// Byte layout of one tape record.
template <typename T, int PA> struct TapeRec {
    typedef typename TapeW<PA>::type W;
    static constexpr int OM = 0;
    static constexpr int OV = TAPE_MAX_S * (int)sizeof(W);  // a multiple of 16
    static constexpr int R = (OV + (TAPE_MAX_S - 1) * (int)sizeof(P2<T>) + 15) / 16 * 16;
    static constexpr int NC = R / 16;
    static constexpr int NM = OV / 16;  // chunks of mask words, always stored and loaded
    // chunk holding the velocity of substep j + 1
    static constexpr __device__ __forceinline__ int vchunk(int j)
    {
        return (OV + j * (int)sizeof(P2<T>)) / 16;
    }
};

// Whether the velocity after substep s was stored: a force may have acted (an active
// contact or a wall bit; the record's own-bit convention above).
template <int PA, typename W>
__device__ __forceinline__ bool vel_stored(const W &w, int me)
{
    return TapeW<PA>::act(w) != 0 || ((TapeW<PA>::incl(w) >> me) & 1) != 0;
}

struct alignas(16) Chunk16 {
    uint32_t d[4];
};

// Write `v` at byte `off` of this lane's record staged in LDS as [chunk][lane] 16-byte
// cells (every field lies inside one chunk).
template <typename X>
__device__ __forceinline__ void stage_put(unsigned char *st, int lane, int off, const X &v)
{
    __builtin_memcpy(st + (((off >> 4) * 64 + lane) << 4) + (off & 15), &v, sizeof(X));
}

// Read the field of type X at byte `off` of a record held in registers.
template <typename X, int NC>
__device__ __forceinline__ X rec_get(const Chunk16 (&r)[NC], int off)
{
    X x;
    __builtin_memcpy(&x, (const unsigned char *)r + off, sizeof(X));
    return x;
}

// SC: the substep count when fixed at compile time (the substep loops unroll), 0: C.S.
template <typename T, int PA, bool TAPE, bool SAT, int SC>
__global__ __launch_bounds__(64) void k_holo_fwd(const Cst<T> C, const Args<T> g,
                                                 const Tape<T> tp)
{
    const int S = SC > 0 ? SC : C.S;
    typedef typename MaskT<PA>::type M;
    typedef TapeW<PA> TW;
    typedef TapeRec<T, PA> TR;
    __shared__ P2<T> lp[64], lv[64];
    __shared__ T lr[64];
    // tape staging: each lane writes and reads back only its own record, so the step's
    // tape goes to memory with the state stores, after the prefetched action is used
    __shared__ Chunk16 tst[TAPE ? TR::NC * 64 : 1];
    unsigned char *const tsb = (unsigned char *)tst;
    const int lane = threadIdx.x, me = lane % PA, base = lane - me;
    const int env = blockIdx.x * (64 / PA) + lane / PA;
    const bool real = me < C.A;
    const bool active = real && env < C.E;
    const size_t i = (size_t)(env < C.E ? env : 0) * C.A + (real ? me : 0);
    const T *prow = g.params + (real ? me : 0) * 22;
    const T ra = prow[0], mass = prow[1], vmax = prow[2];
    const T dt = C.sub_dt, dtm = dt / mass, dd = T(1) + C.c * C.sub_dt / mass;
    const Dv<T> ddv = divisor(dd, true);
    lr[lane] = ra;
    const T qnan = __builtin_nan("");
    P2<T> p = ld2(g.s0.f[0], i), v = ld2(g.s0.f[2], i);
    if (!real) p.x = p.y = qnan;  // pad slot: never within any radius
    const T th = g.s0.f[1][i];
    const size_t EA = (size_t)C.E * C.A;
    P2<T> a = ld2(g.act, i);
    // resolve the initial loads here: a load still in flight at the loop entry makes every
    // iteration wait for all outstanding memory operations, prefetch and stores included
    __builtin_amdgcn_s_waitcnt(0);
    T cnx, cny;  // the step's clamped velocity command
    clamp_norm(a.x, a.y, vmax, cnx, cny);
    for (int t = 0; t < g.nsteps; ++t) {
        P2<T> an = a;
        if (t + 1 < g.nsteps) an = ld2(g.act, (size_t)(t + 1) * EA + i);
        M cand = 0, incl = 0, act = 0;
        unsigned wb = 0u, vneed = 0u;
        T D = T(0);
        bool ok = false;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            T Fx = T(0), Fy = T(0);
            if (C.needs_forces) {
                if (C.collisions) {
                    wave_lds_sync();
                    lp[lane] = p;
                    lv[lane] = v;
                    wave_lds_sync();
                }
                lean_forces<T, PA, SAT>(C, lp, lv, lr, base, me, ra, ddv, p.x, p.y, v.x, v.y,
                                        s == 0 || !ok, s == 0, cand, incl, act, wb, Fx, Fy);
                if (s == 0) progress_priority(t, g.nsteps);
            }
            const T vnx = cnx + Fx * dtm, vny = cny + Fy * dtm;
            const T pnx = p.x + vnx * dt, pny = p.y + vny * dt;
            if (TAPE) {
                const M own = M(1) << me;
                stage_put(tsb, lane, TR::OM + s * (int)sizeof(typename TW::type),
                          TW::pack(incl | ((wb & 1u) ? own : M(0)), act | ((wb & 2u) ? own : M(0))));
                if (s + 1 < S) {
                    stage_put(tsb, lane, TR::OV + s * (int)sizeof(P2<T>), P2<T>{vnx, vny});
                    vneed |= (act != 0 || wb != 0u) ? 1u << TR::vchunk(s) : 0u;
                }
            }
            if (C.use_skin) {
                D += (m_abs(pnx - p.x) + m_abs(pny - p.y)) * T(1.0001);
                ok = env_all<PA>(!real || D <= C.half_margin, base);
            }
            p.x = pnx;
            p.y = pny;
            v.x = vnx;
            v.y = vny;
        }
        // use the prefetched action before issuing this step's stores: memory operations
        // complete in order, so waiting for it afterwards would also wait for the stores
        clamp_norm(an.x, an.y, vmax, cnx, cny);
        asm volatile("" ::"v"(cnx), "v"(cny));  // keeps the use ahead of the stores
        if (active) {
            const bool last = t + 1 == g.nsteps;
            T *const *f = last ? g.fin.f : g.traj.f;
            const size_t j = last ? i : (size_t)t * EA + i;
            st2(f[0], j, p.x, p.y);
            f[1][j] = th;
            st2(f[2], j, v.x, v.y);
            f[3][j] = m_sqrt(v.x * v.x + v.y * v.y);
            f[4][j] = T(0);
        }
        if (TAPE) {
            Chunk16 c[TR::NC];
#pragma unroll
            for (int k = 0; k < TR::NC; ++k) c[k] = tst[k * 64 + lane];
            Chunk16 *dst = (Chunk16 *)tp.rec + ((size_t)t * gridDim.x + blockIdx.x) * TR::NC * 64 + lane;
#pragma unroll
            for (int k = 0; k < TR::NC; ++k)
                if (k < TR::NM || ((vneed >> k) & 1u)) dst[k * 64] = c[k];
            if (t + 1 == g.nsteps) st2(tp.vl, (size_t)blockIdx.x * 64 + lane, v.x, v.y);
        }
    }
}

template <typename T, int PA, bool TAPE, bool SAT, int SC>
__global__ __launch_bounds__(64) void k_holo_bwd(const Cst<T> C, const Args<T> g,
                                                 const Tape<T> tp)
{
    const int S = SC > 0 ? SC : C.S;
    typedef typename MaskT<PA>::type M;
    typedef TapeW<PA> TW;
    typedef typename TW::type W;
    typedef TapeRec<T, PA> TR;
    extern __shared__ __align__(16) unsigned char smem[];
    // per substep slot: P2 pos[64], P2 vel[64]; then inclusion masks [S][64], active-contact
    // masks [S][64]; then gF[64], r[64], dd[64]; then wall bits [S][64] (bytes)
    P2<T> *slot = (P2<T> *)smem;
    M *lm = (M *)(slot + (size_t)S * 128);
    M *la = lm + (size_t)S * 64;
    P2<T> *lg = (P2<T> *)(la + (size_t)S * 64);
    T *lr = (T *)(lg + 64);
    T *ldd = lr + 64;
    unsigned char *lw = (unsigned char *)(ldd + 64);
    const int lane = threadIdx.x, me = lane % PA, base = lane - me;
    const int env = blockIdx.x * (64 / PA) + lane / PA;
    const bool real = me < C.A;
    const bool active = real && env < C.E;
    const size_t i = (size_t)(env < C.E ? env : 0) * C.A + (real ? me : 0);
    const T *prow = g.params + (real ? me : 0) * 22;
    const T ra = prow[0], mass = prow[1], vmax = prow[2];
    const T dt = C.sub_dt, dtm = dt / mass, dd = T(1) + C.c * C.sub_dt / mass;
    const Dv<T> ddv = divisor(dd, true);
    const T inv_dd = T(1) / dd;
    lr[lane] = ra;
    ldd[lane] = dd;
    const T qnan = __builtin_nan("");
    const size_t EA = (size_t)C.E * C.A;
    // adjoint of the current step's output: pos, theta, vel (speed enters per step)
    T gpx = T(0), gpy = T(0), gth = T(0), gvx = T(0), gvy = T(0);
    int t = g.nsteps - 1;
    // step inputs: checkpoint t-1 (or state0), action t
    P2<T> p = t == 0 ? ld2(g.s0.f[0], i) : ld2(g.traj.f[0], (size_t)(t - 1) * EA + i);
    P2<T> v = t == 0 ? ld2(g.s0.f[2], i) : ld2(g.traj.f[2], (size_t)(t - 1) * EA + i);
    P2<T> a = ld2(g.act, (size_t)t * EA + i);
    // adjoint arriving at step t's outputs (pos, theta, vel, speed); null fields carry none
    struct Arr {
        P2<T> p, v;
        T th, s;
    };
    auto arrival = [&](int tt) {
        Arr r;
        const T *const *f = tt == g.nsteps - 1 ? g.afin.f : g.atraj.f;
        const size_t j = tt == g.nsteps - 1 ? i : (size_t)tt * EA + i;
        const P2<T> z = {T(0), T(0)};
        r.p = f[0] ? ld2(f[0], j) : z;
        r.th = f[1] ? f[1][j] : T(0);
        r.v = f[2] ? ld2(f[2], j) : z;
        r.s = f[3] ? f[3][j] : T(0);
        return r;
    };
    Arr arr = arrival(t);
    // tape record of step tt (TAPE), one step ahead like the checkpoint
    struct Tp {
        Chunk16 c[TR::NC];
    };
    auto rec_of = [&](int tt) {
        return (const Chunk16 *)tp.rec + ((size_t)tt * gridDim.x + blockIdx.x) * TR::NC * 64 + lane;
    };
    // the mask chunks of step tt (issued two steps ahead of use)
    auto masks_into = [&](int tt, Tp &r) {
        const Chunk16 *src = rec_of(tt);
#pragma unroll
        for (int k = 0; k < TR::NM; ++k) r.c[k] = src[k * 64];
    };
    // the velocity chunks of step tt that the forward stored (issued one step ahead)
    auto vels_into = [&](int tt, Tp &r) {
        const Chunk16 *src = rec_of(tt);
        unsigned need = 0u;
#pragma unroll
        for (int j = 0; j + 1 < TAPE_MAX_S; ++j)
            if (j + 1 < S && vel_stored<PA>(rec_get<W>(r.c, TR::OM + j * (int)sizeof(W)), me))
                need |= 1u << TR::vchunk(j);
#pragma unroll
        for (int k = TR::NM; k < TR::NC; ++k) {
            Chunk16 x = {};
            if (((need >> k) & 1u) && active) x = src[k * 64];
            r.c[k] = x;
        }
    };
    Tp tc, tn;
    P2<T> vout = {T(0), T(0)};  // output velocity of step t (TAPE)
    if (TAPE) {
        masks_into(t, tc);
        vels_into(t, tc);
        if (t > 0) masks_into(t - 1, tn);
        vout = ld2(tp.vl, (size_t)blockIdx.x * 64 + lane);
    }
    // resolve the initial loads here: a load still in flight at the loop entry makes every
    // iteration wait for all outstanding memory operations, prefetch and stores included
    __builtin_amdgcn_s_waitcnt(0);
    for (; t >= 0; --t) {
        gpx += arr.p.x;
        gpy += arr.p.y;
        gth += arr.th;
        gvx += arr.v.x;
        gvy += arr.v.y;
        const T gs = arr.s;
        // prefetch the previous step's inputs and arriving adjoint
        P2<T> pn = p, vn = v, an = a;
        Arr arn = arr;
        if (t > 0) {
            pn = t - 1 == 0 ? ld2(g.s0.f[0], i) : ld2(g.traj.f[0], (size_t)(t - 2) * EA + i);
            vn = t - 1 == 0 ? ld2(g.s0.f[2], i) : ld2(g.traj.f[2], (size_t)(t - 2) * EA + i);
            an = ld2(g.act, (size_t)(t - 1) * EA + i);
            arn = arrival(t - 1);
        }
        Tp tnn;
        if (TAPE && t > 0) {
            vels_into(t - 1, tn);
            if (t > 1) masks_into(t - 2, tnn);
        }
        if (!real) p.x = p.y = qnan;
        T cnx, cny;
        clamp_norm(a.x, a.y, vmax, cnx, cny);
        const P2<T> vin = v;
        progress_priority(g.nsteps - 1 - t, g.nsteps);

        // ---- the substeps of step t into LDS: from the tape, or recomputed
        if (TAPE) {
            wave_lds_sync();  // the previous step's reverse pass is done with the slots
            P2<T> pp = p, vv = v;
#pragma unroll
            for (int s = 0; s < TAPE_MAX_S; ++s) {
                if (s < S) {
                    P2<T> *sp = slot + s * 128;
                    sp[lane] = pp;
                    sp[64 + lane] = vv;
                    const W w = rec_get<W>(tc.c, TR::OM + s * (int)sizeof(W));
                    const M own = M(1) << me;
                    const M in = (M)TW::incl(w), ac = (M)TW::act(w);
                    lm[s * 64 + lane] = active ? (in & ~own) : M(0);
                    la[s * 64 + lane] = active ? (ac & ~own) : M(0);
                    lw[s * 64 + lane] = active ? (unsigned char)(((in & own) ? 1u : 0u) |
                                                                 ((ac & own) ? 2u : 0u))
                                               : (unsigned char)0;
                    if (s + 1 < TAPE_MAX_S && s + 1 < S) {
                        // a stored velocity, or the command plus the exactly-zero force term
                        vv = (active && vel_stored<PA>(w, me))
                                 ? rec_get<P2<T>>(tc.c, TR::OV + s * (int)sizeof(P2<T>))
                                 : P2<T>{cnx + T(0), cny + T(0)};
                        pp.x = pp.x + vv.x * dt;
                        pp.y = pp.y + vv.y * dt;
                    }
                }
            }
            wave_lds_sync();
            v = vout;
        }
        M cand = 0, incl, act;
        unsigned wb;
        T D = T(0);
        bool ok = false;
        for (int s = 0; s < (TAPE ? 0 : S); ++s) {
            P2<T> *sp = slot + s * 128;
            wave_lds_sync();
            sp[lane] = p;
            sp[64 + lane] = v;
            wave_lds_sync();
            T Fx = T(0), Fy = T(0);
            if (C.needs_forces) {
                lean_forces<T, PA, SAT>(C, sp, sp + 64, lr, base, me, ra, ddv, p.x, p.y, v.x,
                                        v.y, s == 0 || !ok, s == 0, cand, incl, act, wb, Fx, Fy);
            } else {
                incl = 0;
                act = 0;
                wb = 0u;
            }
            lm[s * 64 + lane] = incl;
            la[s * 64 + lane] = act;
            lw[s * 64 + lane] = (unsigned char)wb;
            const T vnx = cnx + Fx * dtm, vny = cny + Fy * dtm;
            const T pnx = p.x + vnx * dt, pny = p.y + vny * dt;
            if (C.use_skin) {
                D += (m_abs(pnx - p.x) + m_abs(pny - p.y)) * T(1.0001);
                ok = env_all<PA>(!real || D <= C.half_margin, base);
            }
            p.x = pnx;
            p.y = pny;
            v.x = vnx;
            v.y = vny;
        }
        // speed output = |v| of the last substep (zero gradient at v = 0); skipped where no
        // adjoint arrives at it, since it would add exactly zero
        if (gs != T(0)) {
            const T spd = m_sqrt(v.x * v.x + v.y * v.y);
            if (spd > T(0)) {
                gvx += gs * v.x / spd;
                gvy += gs * v.y / spd;
            }
        }

        // ---- reverse pass over the substeps
        T gcx = T(0), gcy = T(0);
#pragma unroll
        for (int s = S - 1; s >= 0; --s) {
            const T gtx = gvx + gpx * dt, gty = gvy + gpy * dt;  // adjoint of v_new
            gcx += gtx;
            gcy += gty;
            const T gFx = gtx * dtm, gFy = gty * dtm;
            T ipx = gpx, ipy = gpy, ivx = T(0), ivy = T(0);
            if (C.needs_forces) {
                const P2<T> *sp = slot + s * 128;
                const P2<T> q0 = sp[lane], w0 = sp[64 + lane];
                if (C.collisions) {
                    // publish the force adjoint pre-divided by the damping denominator
                    wave_lds_sync();
                    P2<T> gg;
                    gg.x = gFx * inv_dd;
                    gg.y = gFy * inv_dd;
                    lg[lane] = gg;
                    wave_lds_sync();
                    const M mact = la[s * 64 + lane];
                    M m = lm[s * 64 + lane];
                    while (m) {
                        const int b = m_ctz(m);
                        m &= m - 1;
                        const int j = base + b;
                        const bool own = (mact >> b) & M(1);
                        const bool rev = (la[s * 64 + j] >> me) & M(1);
                        if (!own && !rev) continue;
                        const P2<T> q = sp[j], w = sp[64 + j];
                        const P2<T> gb = lg[j];
                        const T wx = (own ? gg.x : T(0)) - (rev ? gb.x : T(0));
                        const T wy = (own ? gg.y : T(0)) - (rev ? gb.y : T(0));
                        pair_adj_active<T, SAT>(C, q0.x - q.x, q0.y - q.y, w0.x - w.x, w0.y - w.y,
                                        ra + lr[j] + C.margin, wx, wy, ipx, ipy, ivx, ivy);
                    }
                }
                if (C.soft_walls)
                    wall_axes_adj<T, SAT>(C, q0.x, q0.y, w0.x, w0.y, ra, dd, inv_dd, gFx, gFy,
                                  (unsigned)lw[s * 64 + lane], ipx, ipy, ivx, ivy);
            }
            gpx = ipx;
            gpy = ipy;
            gvx = ivx;
            gvy = ivy;
        }
        // use the prefetched values before issuing this step's stores: memory operations
        // complete in order, so waiting for them afterwards would also wait for the stores
        asm volatile("" ::"v"(pn.x), "v"(pn.y), "v"(vn.x), "v"(vn.y), "v"(an.x), "v"(an.y),
                     "v"(arn.p.x), "v"(arn.p.y), "v"(arn.v.x), "v"(arn.v.y), "v"(arn.th),
                     "v"(arn.s));
        if (active) {
            T ax = T(0), ay = T(0);
            clamp_norm_adj_rcp(a.x, a.y, vmax, gcx, gcy, ax, ay);
            T *pa = g.aact + ((size_t)t * EA + i) * C.ad;
            pa[0] = ax;
            if (C.ad > 1) pa[1] = ay;
            for (int k = 2; k < C.ad; ++k) pa[k] = T(0);
        }
        p = pn;
        v = vn;
        a = an;
        arr = arn;
        if (TAPE) {
            vout = vin;
            tc = tn;
            tn = tnn;
        }
    }
    if (active) {
        T *const *f = g.a0.f;
        if (f[0]) st2(f[0], i, gpx, gpy);
        if (f[1]) f[1][i] = gth;
        if (f[2]) st2(f[2], i, gvx, gvy);
        if (f[3]) f[3][i] = T(0);
        if (f[4]) f[4][i] = T(0);
    }
}

// ---------------------------------------------------------------------- launchers

#define SWARP_HOLO_PA(KERNEL, SATV, SCV, SHM)                                                     \
    switch (PA) {                                                                                 \
    case 4: hipLaunchKernelGGL((KERNEL<T, 4, TAPE, SATV, SCV>), grid4, dim3(64), SHM, st, C, a, tp); break;   \
    case 8: hipLaunchKernelGGL((KERNEL<T, 8, TAPE, SATV, SCV>), grid8, dim3(64), SHM, st, C, a, tp); break;   \
    case 16: hipLaunchKernelGGL((KERNEL<T, 16, TAPE, SATV, SCV>), grid16, dim3(64), SHM, st, C, a, tp); break; \
    case 32: hipLaunchKernelGGL((KERNEL<T, 32, TAPE, SATV, SCV>), grid32, dim3(64), SHM, st, C, a, tp); break; \
    default: hipLaunchKernelGGL((KERNEL<T, 64, TAPE, SATV, SCV>), grid64, dim3(64), SHM, st, C, a, tp); break; \
    }

// The saturated contact law (contact_max_overlap > 0) selects the SAT instances; the others
// carry no tanh code at all.  Without saturation, 1 and 4 substeps have instances with the
// count fixed at compile time (the navigation configurations); other counts loop at run time.
#define SWARP_HOLO_DISPATCH(KERNEL, SHM)                                                           \
    if (C.max_overlap > T(0)) {                                                                   \
        SWARP_HOLO_PA(KERNEL, true, 0, SHM)                                                       \
    } else if (C.S == 4) {                                                                        \
        SWARP_HOLO_PA(KERNEL, false, 4, SHM)                                                      \
    } else if (C.S == 1) {                                                                        \
        SWARP_HOLO_PA(KERNEL, false, 1, SHM)                                                      \
    } else {                                                                                      \
        SWARP_HOLO_PA(KERNEL, false, 0, SHM)                                                      \
    }

template <typename T, bool TAPE>
void launch_holo_fwd(int PA, const Cst<T> &C, const Args<T> &a, const Tape<T> &tp, hipStream_t st)
{
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    SWARP_HOLO_DISPATCH(k_holo_fwd, 0)
}

template <typename T, bool TAPE>
void launch_holo_bwd(int PA, const Cst<T> &C, const Args<T> &a, const Tape<T> &tp, size_t shm,
                     hipStream_t st)
{
    const dim3 grid4((C.E + 15) / 16), grid8((C.E + 7) / 8), grid16((C.E + 3) / 4),
        grid32((C.E + 1) / 2), grid64(C.E);
    SWARP_HOLO_DISPATCH(k_holo_bwd, shm)
}

#undef SWARP_HOLO_DISPATCH

#undef SWARP_HOLO_PA

}  // namespace swarp
