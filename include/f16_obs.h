/* f16_obs.h -- C ABI of the observation / reward / termination kernels and of the fused
 * post-physics environment step (libf16hip.so).
 *
 * Every function launches on `stream` (a hipStream_t, NULL = the default stream), never
 * synchronises and never allocates.  Device pointers only.  Return 0 on success, a negative
 * F16_E* code for a rejected argument, or -(1000 + hipError_t) for a launch failure.
 *
 * Layout.  Aircraft a of engagement e is a = 2e (plane 0) or 2e + 1 (plane 1).  The aircraft
 * state is the structure-of-arrays buffer of f16_fdm.h: field k of aircraft a at
 * states[k * ld + a].  Per-aircraft reconstructor vectors are structure-of-arrays too:
 * component k of aircraft a at X[k * rec->ld + a]; the action history holds the five most
 * recent (aileron, elevator, rudder, throttle) rows, newest first, as component 4*step + channel.
 * Observations are row-major float32, obs[a * obs_dim + j], obs_dim 184 or 214.
 */
#ifndef F16_OBS_H
#define F16_OBS_H

#ifdef __cplusplus
extern "C" {
#endif

/* Reconstructor state of BatchObsReward (research/competition_36500/runtime/cuda_fdm/
 * obs_reward.py:338-353, 471-486): what the observation needs beyond the aircraft states. */
typedef struct F16Recon {
    double *hp;            /* (nac)      hit points, 1 at reset                              */
    double *fuel;          /* (nac)      fuel proxy, 1 at reset                              */
    double *t_sec;         /* (nenv)     engagement time [s]                                 */
    double *prev_att;      /* (3, ld)    roll/pitch/yaw [deg] at the previous decision       */
    unsigned char *prev_valid;   /* (nac) prev_att holds a value                          */
    double *pqr;           /* (3, ld)    attitude-difference body rates [rad/s]              */
    double *dealt;         /* (nac)      damage rate dealt this decision                     */
    double *taken;         /* (nac)      damage rate taken this decision                     */
    double *hp_loss;       /* (nac)      HP lost this decision                               */
    double *act_hist;      /* (20, ld)   action history, newest first                        */
    double *prev_x;        /* (nac)      previous geometry advantage G                       */
    unsigned char *prev_x_valid; /* (nac)                                                    */
    double *prev_alt_log;  /* (nac)      previous log(altitude / 304.8 m)                    */
    double *prev_vel_ned;  /* (3, ld)    214-D only (else NULL): previous NED velocity [m/s] */
    double *accel;         /* (3, ld)    214-D only (else NULL): NED acceleration [m/s^2]    */
    long ld;               /* column stride of the (k, ld) arrays, >= nac                   */
    int nenv;
    double *aux;           /* (nenv, 21) future-aux features of plane 0, or NULL (off): own NED
                              position [m] and velocity [m/s], the partner's, own NED-to-body
                              rotation row-major -- written wherever a row becomes the
                              engagement's observation (R/cuda_fdm/gen/obs_kernel.cu:348-355)  */
} F16Recon;

/* MY_REWARD_CONFIG scalars (claude_code/my_reward.py:45-103) and the kernel_advance options
 * (obs_reward.py:410-441).  mode: 0 final-safe geometry, 1 altitude hunt, 2 attack, 3 defence
 * (cuda_fdm/reward_modes.py). */
typedef struct F16RewardCfg {
    double own_damage_weight, damage_scale, shaping_reward_scale;
    double win_reward, loss_reward;
    double timeout_win_reward, timeout_loss_reward, timeout_draw_reward;
    double min_alt_m, max_time_s, alt_hunt_coef;
    int mode;
    int fuel_exhaustion;         /* 1: an engagement also terminates when either aircraft's
                                    physical fuel (state field 14) is <= 0 (BASELINE league
                                    workload; the reference's rule set has no such term) */
} F16RewardCfg;

/* BatchObsReward.kernel_advance (obs_reward.py:410-441; obs_kernel.cu advance_kernel, and
 * external_observation.cu external_acceleration when rec->accel is set): push `actions`
 * ((nac, 4) float64 rows) into the history, integrate HP / fuel / body rates / time from the
 * post-physics states, decide termination (term) and truncation (trunc) per engagement
 * (uint8), and write the reward of every aircraft (float64). */
int f16_obr_advance(const double *states, long ld, const double *actions, const F16Recon *rec,
                    const F16RewardCfg *cfg, double *reward, unsigned char *term,
                    unsigned char *trunc, void *stream);

/* BatchObsReward.kernel_init_reward_state (obs_reward.py:443-452): re-anchor the geometry
 * advantage and log-altitude of the engagements whose env_mask byte is non-zero (NULL = all). */
int f16_obr_init_reward(const double *states, long ld, const unsigned char *env_mask,
                        const F16Recon *rec, void *stream);

/* BatchObsReward.kernel_build_obs (obs_reward.py:454-469) and, for obs_dim 214, the external
 * 214-D observation (obs_reward.py:487-496, external_observation.cu): write the observation rows
 * of the engagements selected by env_mask (NULL = all).  214 needs rec->accel.  obs must be
 * 16-byte aligned for 184 and 8-byte aligned for 214 (as any tensor allocation is). */
int f16_obr_build_obs(const double *states, long ld, const unsigned char *env_mask,
                      const F16Recon *rec, int obs_dim, float *obs, void *stream);

/* Inputs and outputs of the fused post-physics step.  Output pointers may be NULL unless noted;
 * byte flags are 0/1 (torch.bool compatible). */
typedef struct F16EnvStepIO {
    double *states;              /* SoA states (field k of aircraft a at states[k*ld + a]);
                                    autoreset rewrites finished engagements in place (required) */
    long ld;
    const double *actions;       /* (nac, 4) controls of this decision (required) */
    const double *ic_pool;       /* (pool_size, 2, 101) initial-condition rows (required) */
    long pool_size;
    const long *pick;            /* (nenv) pool row per engagement; NULL: drawn in the kernel as
                                    floor(pool_size x0 / 2^32), x0 = Philox4x32-10 word 0 with key
                                    `seed` and counter (e, step, 0, 0x5EED5EED) */
    unsigned long long seed;
    unsigned int step;
    int obs_dim;                 /* 184 or 214 */
    float *obs;                  /* (nac, obs_dim) observations after autoreset (required) */
    float *terminal_obs;         /* (nac, obs_dim) observations before autoreset */
    double *reward;              /* (nac) */
    float *reward_f32;           /* (nac) the same rewards rounded to float32 */
    unsigned char *term, *trunc, *done;   /* (nenv) */
    float *done_f32;             /* (nenv) term|trunc as 0.0 / 1.0 */
    double *terminal_hp;         /* (nac) HP after the decision, before autoreset */
    double *terminal_alt_m;      /* (nac) (|ECI position| - sea-level radius) in metres */
    unsigned char *terminal_finite;  /* (nenv) every state value of both aircraft finite */
    unsigned char *finite_acc;   /* (nenv) cleared to 0 where terminal_finite is 0, else untouched */
    int *opp_assign;             /* (nenv) opponent id per engagement, redrawn at autoreset as the
                                    first k with opp_cdf[k] > u, u = (x0 >> 8) 2^-24, x0 = Philox
                                    word 0 with counter (e, step, 1, 0x0FF0A55E); or NULL */
    const float *opp_cdf;        /* (n_opp) cumulative opponent weights, last = 1 */
    int n_opp;
    const unsigned int *step_base;   /* device counter added to `step` when non-NULL (captured
                                        rollouts): the counters above use *step_base + step */
    double *norm_partial;        /* RunningNorm partial sums of the new `obs` rows, in the
                                    f16_norm_update workspace layout (per 128-row block: obs_dim
                                    sums, then obs_dim sums of squares), so that f16_norm_merge
                                    completes RunningNorm.update(obs) -- or NULL.  Only where
                                    f16_env_post_step_norm_fusable(nenv, obs_dim) is 1. */
    float *norm_count;           /* with norm_partial: the running count, advanced by nac */
    float *norm_count_snap;      /* with norm_partial: the count before this update (the
                                    workspace's last element, as f16_norm_update keeps it) */
    const unsigned char *state_finite;  /* (nac) per aircraft, 1 if all 101 state values are
                                    finite, as f16_fdm_step_batch_finite wrote them for these
                                    states -- or NULL: the kernel reads the 86 fields beyond the
                                    15 it needs anyway and tests them itself */
    const float *pool_obs;       /* (pool_size, 2, obs_dim): each pool row's observation after an
                                    autoreset (what reset_envs + init_reward + build_obs give
                                    on that row, rl_env.py:559-577), or NULL: the kernel builds
                                    them.  With pool_obs, also: */
    const double *pool_prev_x;   /* (pool_size, 2) the re-anchored geometry advantage */
    const double *pool_prev_alt_log;  /* (pool_size, 2) the re-anchored log altitude */
    const double *pool_aux;      /* (pool_size, 21) plane 0's aux features (used when rec->aux) */
    float *reward0_f32;          /* (nenv) the float32 reward of each engagement's first aircraft
                                    (aircraft 2e), or NULL: a learner-side rollout buffer row */
} F16EnvStepIO;

/* GpuDogfightVecEnv.step after the physics launch (research/competition_36500/runtime/
 * cuda_fdm/rl_env.py:540-580), one launch: the finite flag over the post-physics states,
 * advance + reward + termination, the terminal observation, terminal HP and MSL altitude, then
 * for every engagement with term|trunc: the state rows of ic_pool[pick] are copied into states,
 * the reconstructor is reset, the reward state re-anchored and the observation rebuilt; live
 * engagements keep the terminal observation in `obs`.  A pick outside [0, pool_size) fills that
 * engagement's states with NaN so the error surfaces as a non-finite state instead of an
 * out-of-bounds read.  obs and terminal_obs: 16-byte aligned for 184, 8-byte for 214. */
/* The whole GpuDogfightVecEnv.step after the action decode (research/competition_36500/
 * runtime/cuda_fdm/rl_env.py:511-580): the physics step of f16_fdm_step_batch_keep (`actions`
 * for `substeps` steps at fcs_rate; when `actions` is non-NULL and differs from io->actions, the
 * launch also copies it into io->actions, which must not overlap it) followed by
 * f16_env_post_step of `io`, with `state_finite` ((nac) bytes, required) carrying the physics'
 * per-aircraft finite flags to the post-physics step (io->state_finite is ignored).  Where every
 * workgroup of the post-physics step's full-row tile is resident at once (as
 * f16_env_post_step_norm_fusable reports), one launch does both: each 512-thread workgroup runs
 * the physics of its 128 aircraft on four wavefronts per 64 aircraft, then their post-physics
 * step, again on four (two wavefronts per SIMD at 16,384 engagements); otherwise the two launches
 * are issued.  Results equal the two entry points' bit for bit.  Every argument is checked before
 * anything is launched. */
int f16_env_step(const F16EnvStepIO *io, const F16Recon *rec, const F16RewardCfg *cfg,
                 const double *actions, int substeps, int fcs_rate, unsigned char *state_finite,
                 void *stream);

/* The same step with two wavefronts per 64 aircraft in each phase (256-thread workgroups, one
 * wavefront per SIMD at 16,384 engagements); same arguments, same results bit for bit.  Kept as
 * the cross-check of f16_env_step's four-wavefront kernel. */
int f16_env_step_tworole(const F16EnvStepIO *io, const F16Recon *rec, const F16RewardCfg *cfg,
                         const double *actions, int substeps, int fcs_rate,
                         unsigned char *state_finite, void *stream);

/* The autoreset half of f16_env_post_step alone, for the engagements with mask[e] != 0
 * ((nenv) bytes): pool row (io->pick or the Philox draw at io->step), reconstructor reset,
 * re-anchored reward state (and, with io->opp_assign, an opponent redraw); no observation.  The
 * device-side replacement of the staggered warm-up's host re-seeding (R/cuda_fdm/rl_env.py:
 * 386-434).  Reads io->states, ld, ic_pool, pool_size, pick, seed, step, step_base, obs_dim. */
int f16_env_reseed(const F16EnvStepIO *io, const F16Recon *rec, const unsigned char *mask,
                   void *stream);

int f16_env_post_step(const F16EnvStepIO *io, const F16Recon *rec, const F16RewardCfg *cfg,
                      void *stream);
/* With io->pool_obs set, an autoreset copies the pool row's observation, anchors and aux
 * features from those tables instead of rebuilding them (a pick outside the pool still builds
 * its NaN row); the tables must describe io->ic_pool at this obs_dim.  f16_env_post_step_onewave
 * ignores them and always builds, so the two entry points cross-check the tables. */

/* 1 when f16_env_post_step over nenv engagements can also produce the RunningNorm partial sums
 * of its new observation rows (io->norm_partial): every row's block sits whole in one
 * workgroup's staging tile.  0 otherwise (the caller then runs f16_norm_update). */
int f16_env_post_step_norm_fusable(int nenv, int obs_dim);

/* The same step with one wavefront per 64 aircraft (f16_env_post_step spreads each group's
 * row build over four wavefronts -- advance, scalar block, vector-block frames 0-2 and 3-5 --
 * where the full-row tile is resident, as f16_env_post_step_norm_fusable reports, and over an
 * advance wave and a vector-block wave otherwise); results are identical bit for bit.  Kept as
 * the cross-check of the multi-wave kernels. */
int f16_env_post_step_onewave(const F16EnvStepIO *io, const F16Recon *rec,
                              const F16RewardCfg *cfg, void *stream);

/* GpuDogfightVecEnv.state9_flat (cuda_fdm/rl_env.py:583-592 with kinematics_state and
 * ned_from_ecef_altasl, :88-163): per aircraft N, E, D [m] (D = -MSL altitude; N/E the tangent
 * plane about the official origin of the point at the aircraft's geodetic latitude/longitude),
 * roll, pitch, yaw [deg], body u, v, w [m/s].  s9: (nac, 9) row-major float64. */
int f16_state9(const double *states, long ld, int nac, double *s9, void *stream);

/* build_future_labels (R/cuda_fdm/future_aux.py:29-55): from the (T, nenv, 21) features of a
 * rollout and its (T, nenv) episode-start flags (the done flag entering each step; nonzero =
 * start), labels (T, nenv, 6) float32 and mask (T, nenv, 2) bytes.  Slot 0: the partner 5 steps
 * ahead, slot 1: own 10 steps ahead; each the position change minus the constant-velocity
 * prediction (h * dt * velocity), rotated into the current own body frame, / 100 m; zero and
 * masked when an episode starts within the horizon or the horizon leaves the rollout. */
int f16_future_labels(const double *features, const float *starts, int T, int nenv, double dt,
                      float *labels, unsigned char *mask, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* F16_OBS_H */
