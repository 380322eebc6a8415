/*
 * swarp_hip.h -- C ABI of libswarp_hip.so, the MI355X (gfx950) physics step of swarp.
 *
 * Every pointer is a caller-owned device pointer (HIP device memory) unless stated;
 * nothing here allocates device memory.  All launches go to `stream` (a hipStream_t,
 * NULL = the legacy default stream) and return without synchronising.  Functions
 * return 0 on success and a negative code on a rejected argument; the message is in
 * swarp_last_error() (thread-local).  No function keeps global mutable state.
 *
 * Layouts (row-major, contiguous, scalar type given by desc->dtype):
 *   pos [E,A,2], theta [E,A], vel [E,A,2], speed [E,A], ang_vel [E,A],
 *   z [E,A], vz [E,A], attitude [E,A,4] (x,y,z,w), body_rates [E,A,3]
 *   -- the nine fields of the reference's TorchState (swarp/interop/autograd.py:29-45).
 *   actions [T,E,A,act_dim]; params [A,22] in PARAM_FIELDS column order
 *   (swarp/dynamics/base.py:114-145); model_tag / ctrl_mode [A] int32.
 */
#ifndef SWARP_HIP_H
#define SWARP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SWARP_ABI_VERSION 16

#define SWARP_F32 0
#define SWARP_F64 1

/* desc->integrator (the reference's Integrator, swarp/dynamics/base.py:97-101) */
#define SWARP_EULER 0
#define SWARP_RK4 1

/* Everything the step needs besides the state and the actions.
 * Counterpart of the Stepper's configuration (swarp/core/stepper.py:87-137) plus
 * WorldConfig's contact constants (swarp/core/config.py:181-322) and the obstacle
 * arrays Stepper.set_obstacles installs (swarp/core/stepper.py:295-432). */
typedef struct swarp_desc {
    int32_t abi_version;     /* must equal SWARP_ABI_VERSION */
    int32_t dtype;           /* SWARP_F32 or SWARP_F64 */
    int32_t n_envs, n_agents, act_dim, substeps;
    int32_t max_neighbors;   /* padded list width K (swarp/core/config.py max_neighbors) */
    int32_t n_obstacles;
    int32_t collisions;      /* agent-agent contacts on */
    int32_t soft_walls;      /* bounds_mode == "soft" with bounds set */
    int32_t clamp_bounds;    /* bounds_mode == "clamp" with bounds set: 1 the disc clamp,
                                2 the footprint clamp of a world holding box agents
                                (clamp_footprint, swarp/dynamics/kernels.py:74-99) */
    int32_t has_drone;       /* fleet holds a DRONE: all nine fields are stepped */
    int32_t holo_velocity_only; /* every agent is HOLONOMIC in VELOCITY mode: selects the
                                   specialised kernels (must describe params truthfully) */
    double dt;               /* env step; sub_dt = dt / substeps */
    double k, c, margin, max_overlap;
    double neighbor_radius;
    double bounds_min[2], bounds_max[2];
    const void *params;
    const int32_t *model_tag, *ctrl_mode;
    /* obstacles (NULL when n_obstacles == 0): pos [E,N,2], radius [N], angle [E,N],
       half_extents [N,2], vel [E,N,2], ang_vel [E,N], type [N] int32 */
    const void *obs_pos, *obs_radius, *obs_angle, *obs_half, *obs_vel, *obs_ang_vel;
    const int32_t *obs_type;
    /* movable compound bodies (read by the _ob entry points only; Obstacles' body fields,
       swarp/core/config.py:70-78): kind [N] int32 (1 = MOVABLE), body [N] int32 (root
       index of each shape's body), mass [N], inertia [N], body_offset [N,2]; the linear /
       angular damping of WorldConfig (obstacle_linear_damping, obstacle_angular_damping) */
    const int32_t *obs_kind, *obs_body;
    const void *obs_mass, *obs_inertia, *obs_body_off;
    double lin_damping, ang_damping;
    /* SWARP_EULER: semi-implicit Euler (_integrate_agent, swarp/dynamics/kernels.py:278-413);
       SWARP_RK4: classic RK4 on each substep (_integrate_rk4, :520-793), every model */
    int32_t integrator;
    /* some agent is a BOX (params' shape column, swarp/dynamics/base.py:83-95): the
       box-aware contact pass (collision_forces_box_kernel, swarp/core/collisions.py:
       999-1059) -- oriented-rectangle contacts against discs, boxes, obstacles and walls */
    int32_t has_boxes;
    /* WorldConfig.wheel_contacts (forward only, Euler, no drones; swarp/core/stepper.py:
       851-858): the force pass also computes each agent's contact torque
       (collision_forces_wheel_kernel, swarp/core/collisions.py:1343-1403) and a diff-drive
       agent's step is reworked by wheel_contact (swarp/dynamics/kernels.py:1328-1387);
       lat_grip = wheel_lateral_friction * gravity, turn_cap = wheel_turn_torque.
       swarp_rollout_bwd rejects it. */
    int32_t wheel_contacts;
    double lat_grip, turn_cap;
    /* 1: `params` is [n_envs, n_agents, 22], one row per (env, agent) -- the per-env
       override of Stepper.set_agent_params_per_env (swarp/core/stepper.py:493-575,
       the reference's *_per_env kernel variants); 0: [n_agents, 22] shared by every env. */
    int32_t params_per_env;
    /* The fleet's top speed (the largest max_speed of its parameter rows; <= 0 reads as
       1).  Sizes the per-step skin of the neighbour search, which only affects speed:
       the lists stay exact whatever the agents do. */
    double skin_speed;
    /* The fleet's dynamics models and control modes as bit sets: bit m of fleet_models
       set when some agent's model_tag is m (DynamicsModel, swarp/dynamics/base.py:12-19),
       bit c of fleet_modes when some agent's ctrl_mode is c (ControlMode, :57-78).  They
       select kernel instances compiled without the absent models and modes, so they must
       describe model_tag / ctrl_mode truthfully; 0 reads as "any" (the general
       instances). */
    int32_t fleet_models, fleet_modes;
    /* Neighbour-list order (NeighborGrid's method, swarp/core/neighbors.py:387-389):
       SWARP_LISTS_BRUTE ascending agent index (_brute_force, :76-97); SWARP_LISTS_GRID the
       uniform grid's (_query_uniform, :214-251) over grid_bins x grid_bins cells (their
       table in LDS beside the env's agents, see below).  grid_pinned = 1: the frame is grid_origin / grid_cell (the world
       rectangle's, NeighborGrid._fill_static_grid :476-490, as the reference computes
       them in float64; rounded to dtype here); 0: swarp_neighbors reduces it over the
       batch (:149-181) into grid_frame, a caller-owned device buffer of 3 scalars of
       dtype.  Stepping with grid lists takes a pinned frame. */
    int32_t neighbor_method, grid_bins, grid_pinned;
    double grid_origin[2], grid_cell;
    void *grid_frame;
    /* The shared [n_agents, 22] table (Stepper.params.floats) when params_per_env = 1: the
       body pass of the _ob entry points reads the agents' radius and mass from it, as the
       reference's launch_obstacle_dynamics does whatever table the agent side uses
       (swarp/core/stepper.py:961-964); the agents' own forces and integration read
       `params`.  Ignored when params_per_env = 0. */
    const void *body_params;
    /* The obstacle shape types present as a bit set (bit t set when some obstacle's type
       is t: 0 circle, 1 box, 2 segment); 0 reads as "any".  Lets the movable-body kernels
       run an instance compiled without box and segment terms, so it must be truthful. */
    int32_t obstacle_types;
} swarp_desc_t;

#define SWARP_LISTS_BRUTE 0
#define SWARP_LISTS_GRID 1
/* Agents per env: up to 64 on every path; up to SWARP_WIDE_MAX_AGENTS on the wide-env
   path (one workgroup per env, 1, 2 or 4 agents per thread; movable bodies up to 1024
   agents, one per thread), which steps 2-D and drone fleets with any model,
   control mode, obstacles, walls, clamp and integrator, box agents and wheel contacts,
   and movable bodies (within their staging limits), and serves every fleet with
   grid-ordered lists.  An env's staging (agents, the grid's bins^2 cells, box fields)
   stays within the 160 KiB of LDS of one workgroup: at 1024 agents up to 172 bins per
   axis in float32 (150 in float64; box worlds 150 / 90). */
#define SWARP_WIDE_MAX_AGENTS 4096

/* The nine state fields.  A NULL field means "not provided": an input adjoint that
 * is NULL reads as zero, an output adjoint that is NULL is not written.  For a fleet
 * without drones (desc->has_drone == 0) the last four fields are never touched. */
typedef struct swarp_state {
    void *pos, *theta, *vel, *speed, *ang_vel, *z, *vz, *attitude, *body_rates;
} swarp_state_t;

/* Library / ABI version (SWARP_ABI_VERSION). */
int swarp_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *swarp_last_error(void);

/* T-step forward rollout in one launch.
 * Replaces T calls of Stepper.launch_substeps under _WarpStepFn.forward
 * (swarp/interop/autograd.py:229-275, swarp/core/stepper.py:784-1011): each step runs
 * `substeps` substeps of neighbour search (swarp/core/neighbors.py:76-97), contact
 * forces (swarp/core/collisions.py:818-881) and integration
 * (swarp/dynamics/kernels.py:812-971).
 * `traj` receives the outputs of steps 0..T-2, each field strided by one state
 * (field [T-1, E, A, ...]); it may be NULL when T == 1.  `final` receives the output
 * of step T-1.  Inputs are never written. */
int swarp_rollout_fwd(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                      const void *actions, const swarp_state_t *traj,
                      const swarp_state_t *final_state, void *stream);

/* Reverse of swarp_rollout_fwd in one launch (the adjoints the reference gets from
 * wp.Tape.backward, swarp/interop/autograd.py:277-296).  Step inputs are recomputed
 * from state0 and the checkpoints `traj` (the forward's own outputs); this entry point
 * recomputes each step's substep intermediates in the kernel from its checkpoint
 * (swarp_rollout_bwd_tape reads them from the forward's tape instead).  `adj_traj` (same
 * layout as traj, fields may be NULL) and `adj_final` are the adjoints arriving at
 * each step output.  Writes adj_state0 (fields may be NULL) and adj_actions
 * [T,E,A,act_dim] (every element written). */
int swarp_rollout_bwd(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                      const void *actions, const swarp_state_t *traj,
                      const swarp_state_t *adj_traj, const swarp_state_t *adj_final,
                      const swarp_state_t *adj_state0, void *adj_actions, void *stream);

/* Rollout tape: what the backward's reverse pass reads besides the checkpoints (the
 * input velocity of substeps 1..S-1, each substep's uncapped neighbour mask and
 * active-contact mask, the wall-contact bits, the last step's output velocity), written
 * by the forward so that the backward does not recompute the substeps.  Counterpart of
 * the taped substep buffers the reference keeps alive for wp.Tape.backward
 * (StepBuffers / make_buffers, swarp/core/stepper.py:55-63, 642-678).
 * Writes in *bytes the tape size of a T-step rollout of this configuration; 0 when the
 * configuration keeps no tape, in which case the _tape entry points behave as the plain
 * ones.  Three kinds of configuration keep one: fleets on the specialised holonomic-velocity
 * kernels with substeps <= 4 and contacts or walls (the records above), and float32 2-D
 * fleets among static obstacles whose forward runs the obstacle pass on a wave of its own
 * (at most 256 / (envs per 64 lanes) obstacles, no box agents, wheel contacts or drones):
 * there the tape holds each substep's per-agent total force (listed pairs, obstacles,
 * walls), 8 T S E A bytes, and neighbour-inclusion mask, 4 T S E A bytes (8 at more than
 * 32 agents), which the backward reads instead of evaluating the forces and scanning, and
 * for at most 32 obstacles each substep's per-agent mask of the obstacles in contact,
 * w T S E A bytes more (w = 1, 2 or 4 for up to 8, 16 or 32 obstacles; each part rounded
 * up to 256), so that the backward reverses only those; and the other fleets without box
 * agents or wheel contacts that have contacts, walls or obstacles (drones among them):
 * each substep's total force and neighbour mask as above, no contact masks.  The taped
 * backward gives the
 * untaped one's values; a gradient that is zero may differ in the sign of that zero. */
int swarp_tape_bytes(const swarp_desc_t *desc, int32_t T, uint64_t *bytes);

/* swarp_rollout_fwd that also writes the tape (`tape_bytes` must be
 * swarp_tape_bytes(desc, T); the tape is device memory owned by the caller). */
int swarp_rollout_fwd_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                           const void *actions, const swarp_state_t *traj,
                           const swarp_state_t *final_state, void *tape, uint64_t tape_bytes,
                           void *stream);

/* swarp_rollout_bwd reading the substep intermediates from the tape written by
 * swarp_rollout_fwd_tape on the same inputs (same results; see swarp_tape_bytes for the
 * sign of zero gradients under the obstacle tape). */
int swarp_rollout_bwd_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                           const void *actions, const swarp_state_t *traj,
                           const swarp_state_t *adj_traj, const swarp_state_t *adj_final,
                           const swarp_state_t *adj_state0, void *adj_actions,
                           const void *tape, uint64_t tape_bytes, void *stream);

/* Rollout of a world whose obstacle state evolves: movable compound bodies integrated
 * from the agents' contact reactions inside every substep (the body pass of
 * obstacle_dynamics_kernel, swarp/core/bodies.py:367-568, disc variant: disc agents,
 * body shapes of any type; the reference runs it on untaped steps,
 * swarp/core/stepper.py:952-991).  Replaces T calls of Stepper.launch_substeps with the
 * body pass enabled.  Fleets of any dynamics models including drones, shared or per-env
 * parameter rows (then desc->body_params), disc agents, up to 1024 agents per env with
 * index-ordered or (pinned-frame) uniform-grid lists, and n_obstacles >= 1 up to what the
 * per-env obstacle staging allows: the forward's and the backward's LDS of one workgroup
 * (dynamic and static) stay within the 160 KiB a gfx950 workgroup may hold.  Up to 64
 * agents per env with index-ordered lists an env takes a slot of one wave, widened (fewer
 * envs per wave) while the staging exceeds 64 KiB, as far as one env per wave -- at 64
 * agents, 4 substeps and float32 that is 1401 obstacles forward and 447 backward (float64:
 * 695 / 209); wider envs and grid-ordered lists take a workgroup of ceil(n_agents / 64)
 * waves, whose agent staging shares the 160 KiB (brute lists, float32: 1329 / 544
 * obstacles forward / backward at 512 agents, 1021 / 418 at 1024).  Beyond it the call
 * fails before any launch
 * (swarp_rollout_bwd_ob_check asks the backward's limit).  The _tape entry points keep
 * no body tape on the workgroup-per-env kernels (they accept one and leave it unused).
 * ob0 [E, 12N]: per env and obstacle index o, the shape state (pos x, pos y, angle,
 * vel x, vel y, ang_vel) at [6o..6o+5] and the state of the body rooted at o at
 * [6N+6o..6N+6o+5] (the reference's obs_* and body_* arrays, stepper.py:418-431).
 * ob_traj [T, E, 12N] receives the obstacle state after each step.  Other arguments as
 * swarp_rollout_fwd. */
int swarp_rollout_fwd_ob(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                         const void *ob0, const void *actions, const swarp_state_t *traj,
                         const swarp_state_t *final_state, void *ob_traj, void *stream);

/* Reverse of swarp_rollout_fwd_ob (this build's own adjoint of the body pass; the
 * reference has none).  adj_ob_traj [T, E, 12N] (nullable) is the adjoint arriving at each
 * step's obstacle output; adj_ob0 [E, 12N] (nullable) receives the adjoint of ob0.  Other
 * arguments as swarp_rollout_bwd. */
int swarp_rollout_bwd_ob(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                         const void *ob0, const void *actions, const swarp_state_t *traj,
                         const void *ob_traj, const swarp_state_t *adj_traj,
                         const swarp_state_t *adj_final, const void *adj_ob_traj,
                         const swarp_state_t *adj_state0, void *adj_ob0, void *adj_actions,
                         void *stream);

/* 0 when swarp_rollout_bwd_ob can run a configuration (descriptor valid for the body path,
 * obstacle staging within the backward's LDS), else -1 with the reason in
 * swarp_last_error.  Replaces no reference function: a caller whose forward will be
 * differentiated asks it before swarp_rollout_fwd_ob, so that a configuration the
 * backward refuses is refused before the forward advances any state (the reference's
 * taped forward and its backward accept the same configurations,
 * swarp/interop/autograd.py:229-296). */
int swarp_rollout_bwd_ob_check(const swarp_desc_t *desc);

/* Body tape: per substep and movable body, the body pass's result -- the body's new pose
 * and velocity, the new angle's cos / sin, its contact force and torque -- written by the
 * forward so that the backward's recompute of each step reads it instead of evaluating
 * the pass again (the agents' forces are still recomputed from the checkpoints).  Bodies
 * are counted in root order (the obstacle indices o with body[o] = o and kind[o] = 1);
 * a tape may hold the first n_bodies of them, and the backward evaluates the others.
 * No counterpart in the reference: its body pass runs on untaped steps and is not
 * differentiated (swarp/core/stepper.py:952-991).
 * Writes in *bytes the size of the tape of a T-step rollout holding n_bodies bodies
 * (1 <= n_bodies <= n_obstacles): T * substeps * n_envs * n_bodies * 12 scalars. */
int swarp_ob_tape_bytes(const swarp_desc_t *desc, int32_t T, int32_t n_bodies, uint64_t *bytes);

/* swarp_rollout_fwd_ob that also writes the body tape (device memory owned by the caller;
 * tape_bytes = swarp_ob_tape_bytes(desc, T, n_bodies) for some n_bodies). */
int swarp_rollout_fwd_ob_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                              const void *ob0, const void *actions, const swarp_state_t *traj,
                              const swarp_state_t *final_state, void *ob_traj, void *tape,
                              uint64_t tape_bytes, void *stream);

/* swarp_rollout_bwd_ob reading the body pass of the tape written by
 * swarp_rollout_fwd_ob_tape on the same inputs (same results, bit for bit). */
int swarp_rollout_bwd_ob_tape(const swarp_desc_t *desc, int32_t T, const swarp_state_t *state0,
                              const void *ob0, const void *actions, const swarp_state_t *traj,
                              const void *ob_traj, const swarp_state_t *adj_traj,
                              const swarp_state_t *adj_final, const void *adj_ob_traj,
                              const swarp_state_t *adj_state0, void *adj_ob0, void *adj_actions,
                              const void *tape, uint64_t tape_bytes, void *stream);

/* Padded radius-neighbour lists of one state: replaces NeighborGrid.query_into's
 * brute-force kernel (swarp/core/neighbors.py:76-97, 465-492).  pos [E,A,2] of
 * desc->dtype; idx [E,A,K] int32 (entries past cnt are zero-filled), cnt [E,A] int32,
 * true_cnt [E,A] int32 (uncapped; NULL = not written).  Radius = desc->neighbor_radius,
 * K = desc->max_neighbors. */
int swarp_neighbors(const swarp_desc_t *desc, const void *pos, int32_t *idx, int32_t *cnt,
                    int32_t *true_cnt, void *stream);

/* Inputs and outputs of the navigation scenario's fused per-step pass (swarp_nav_obs).
 * Scalars are in desc->dtype; E = desc->n_envs, A = desc->n_agents, K =
 * desc->max_neighbors, W = 9 + 5 * k_obs (the observation width). */
typedef struct swarp_nav {
    const void *pos, *vel, *theta, *ang_vel; /* state [E,A,2], [E,A,2], [E,A], [E,A] */
    const void *goals;                       /* [E,A,2] */
    const uint8_t *reset_mask;               /* [E]: envs just reset (NULL = none) */
    void *prev_dist;                         /* [E,A] shaping baseline, read and updated */
    int32_t *nbr_idx, *nbr_cnt, *nbr_true;   /* lists of pos: [E,A,K], [E,A], [E,A] (true
                                                may be NULL) */
    void *obs;                               /* [E,A,W] */
    void *touching, *dist, *shaping;         /* [E,A] */
    uint8_t *on_goal, *overflow;             /* [E,A] */
    void *reward;                            /* [E,A] (full passes only) */
    uint8_t *done;                           /* [E]   (full passes only) */
    int32_t k_obs;                           /* neighbour slots in the observation */
    int32_t advance_prev;                    /* 1: the baseline advances to the current
                                                distance (a step pass) */
    int32_t full_pass;                       /* 0: obs-only pass over the envs of
                                                reset_mask (auto-reset); 1: every env,
                                                reward and done included */
    int32_t shared_reward;
    double pos_shaping_factor, goal_tolerance, collision_penalty, final_reward;
    int32_t *step_count;                     /* [E] episode step counter, incremented on
                                                step passes (advance_prev = 1, full_pass =
                                                1); NULL = not counted here */
    uint8_t *truncated;                      /* [E] step_count >= max_steps after the
                                                increment (NULL = not written) */
    int32_t max_steps;                       /* <= 0: no time limit */
    const void *radius;                      /* [A] radii of the touching test: the
                                                scenario's static agent radius, which
                                                the reference hands its navigation
                                                kernels even when parameters are
                                                randomized per env (navigation.py:556-557);
                                                NULL: column P_RADIUS of desc->params */
} swarp_nav_t;

/* The navigation scenario's per-step pass in one launch: radius lists of `pos`
 * (as swarp_neighbors), observation rows, touching count, goal distance, position
 * shaping, on-goal / overflow flags, reward and done.  Replaces the reference's no-grad
 * fast path: the NeighborGrid build + nav_obs_kernel + nav_reward_kernel
 * (swarp/scenarios/navigation.py:539-650, swarp/scenarios/navigation_kernels.py:41-243).
 * Radii for the touching test: nav->radius (else column P_RADIUS of desc->params). */
int swarp_nav_obs(const swarp_desc_t *desc, const swarp_nav_t *nav, void *stream);

/* COO radius graph from padded lists: replaces NeighborGrid.edge_index's torch mask ops
 * (swarp/core/neighbors.py:716-733).  `offsets` [E*A] int64 must hold the exclusive
 * prefix sum of cnt in (env, agent) order (n_edges = offsets[last] + cnt[last]);
 * writes edge_index [2, n_edges] int64: row 0 = e*A + idx[e,a,s] (sender),
 * row 1 = e*A + a (receiver), in (e, a, s) order. */
int swarp_edge_index(int32_t n_envs, int32_t n_agents, int32_t max_neighbors,
                     const int32_t *idx, const int32_t *cnt, const int64_t *offsets,
                     int64_t n_edges, int64_t *edge_index, void *stream);

/* The COO radius graph without any allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same edges in the same order as
 * swarp_edge_index, but the prefix sums of cnt are computed inside -- their per-block
 * partial sums live in a file-scope device array of 65536 int64 (512 KiB per GPU, held
 * until the process ends), so n_envs * n_agents must be <= 16777216 (larger sizes are
 * rejected) -- and the edge count is written to the device scalar *n_edges instead of
 * being passed in.  edge_index is [2, capacity] int64: senders at edge_index[0 .. m),
 * receivers at edge_index[capacity .. capacity + m), m = min(*n_edges, capacity); edges
 * past capacity are dropped (compare *n_edges with capacity).  Counts are read as
 * min(max(cnt, 0), max_neighbors).  Calls that overlap on one GPU share its array and
 * race: serialise them (one stream, or events). */
int swarp_edge_index_noalloc(int32_t n_envs, int32_t n_agents, int32_t max_neighbors,
                             const int32_t *idx, const int32_t *cnt, int64_t capacity,
                             int64_t *edge_index, int64_t *n_edges, void *stream);

/* Default values of the four drone fields of n agents, written in one pass into one
 * contiguous buffer of 9 n elements of `dtype` (SWARP_F32 or SWARP_F64) laid out as
 * [z (n), vz (n), attitude (4 n, x y z w), body_rates (3 n)]: zeros, with the identity
 * quaternion (0, 0, 0, 1) per agent.  `buf` must be 16-byte aligned.  Replaces the zero
 * and identity tensors of fill_state_defaults (swarp/interop/autograd.py:48-68). */
int swarp_state_defaults(int32_t dtype, int64_t n, void *buf, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* SWARP_HIP_H */
