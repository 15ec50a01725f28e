/* f16_policy.h -- C ABI of the rollout-side policy kernels (libf16hip.so): observation
 * running-normalisation update and the fused actor/critic MLP step with categorical sampling.
 *
 * Launch on `stream` (hipStream_t, NULL = default), no synchronisation, no allocation; device
 * pointers only; 0 on success, F16_E* (< 0) for a rejected argument, -(1000 + hipError_t) for a
 * launch failure.
 */
#ifndef F16_POLICY_H
#define F16_POLICY_H

#ifdef __cplusplus
extern "C" {
#endif

/* Packed network of the reference's MLPDiscreteActorCritic with hidden (256, 256), tanh
 * (research/competition_36500/runtime/claude_code/model.py:162-205; BASELINE C4/C5 sizes).
 * bf16 part, each matrix [out][in] (input width padded to kp = round_up(obs_dim, 32)) stored
 * fragment-major: blocks of 512 elements in (32-row tile t, 16-column slice s) order, element
 * (32t + l%32, 16s + 8(l/32) + i) of block (t, s) at 8l + i (l < 64, i < 8):
 *   W1 [512][kp]   actor layer-1 rows 0..255, critic layer-1 rows 256..511 (pad columns 0)
 *   W2a [256][256] actor layer 2,  W2c [256][256] critic layer 2
 *   W3a [96][256]  actor logits head, rows 84..95 zero
 * f32 part: b1 [512], b2a [256], b2c [256], b3a [96] (84..95 zero), w3c [256] critic head
 * weights, b3c [1]  (F16_POLICY_NF = 1377 floats). */
#define F16_POLICY_HID 256
#define F16_POLICY_BINS 21
#define F16_POLICY_CHANNELS 4
#define F16_POLICY_NF 1377

typedef struct F16PolicyGroup {
    const void *wbf;        /* bf16 weight blob of this group's network */
    const float *wf;        /* f32 bias/head blob */
    const float *mean, *var;/* this network's RunningNorm statistics, or NULL for the launch's */
    int row_begin, row_end; /* logical rows [begin, end) evaluated by this network (ignored when
                               F16PolicyArgs.group_offsets is set) */
} F16PolicyGroup;

#define F16_POLICY_MAX_GROUPS 16

typedef struct F16PolicyArgs {
    const float *obs;       /* physical observation rows, row stride obs_ld floats */
    long obs_ld;
    int obs_dim;            /* 184 or 214 */
    const float *mean, *var;/* RunningNorm statistics (obs_dim), NULL = no normalisation */
    float clip, eps;        /* normalisation clip (10) and epsilon (1e-8) */
    const int *rows;        /* logical row -> physical row; NULL = identity */
    int ngroups;            /* networks, each over its own logical row range */
    F16PolicyGroup group[F16_POLICY_MAX_GROUPS];
    const int *group_offsets;  /* device (ngroups + 1) row offsets: group g evaluates logical rows
                                  [offsets[g], offsets[g+1]); NULL = the groups' row_begin/end */
    int max_group_rows;     /* with group_offsets: upper bound of any group's row count */
    int total_group_rows;   /* with group_offsets: upper bound of the groups' row counts summed,
                               or 0.  When set, the launch packs every group's 64-row tiles into
                               one grid dimension (about total / 64 + ngroups workgroups instead
                               of ngroups x max_group_rows / 64) */
    unsigned long long seed;/* Philox4x32-10 key */
    unsigned int step;      /* counter word 1 (rollout step) */
    unsigned int salt;      /* counter word 3 (separates independent draws at one step) */
    int deterministic;      /* 1: per-channel argmax instead of sampling */
    const float *grid;      /* 21 control values of linspace(-1, 1, 21) in float32 */
    float *nobs_out;        /* normalised observations at logical rows (ld nobs_ld), or NULL */
    long nobs_ld;
    long long *act_idx;     /* (logical, 4) sampled bins, or NULL */
    float *logp;            /* (logical) summed log-probability of the sampled bins, or NULL */
    float *value;           /* (logical) critic value, or NULL (the critic is then skipped) */
    double *env_actions;    /* (physical, 4) float64 controls [ail, ele, rud, thr], or NULL */
    float *logits_out;      /* (logical, 84) actor logits, or NULL */
    const unsigned int *step_base;  /* device counter added to `step` when non-NULL, so a
                                       captured (HIP graph) rollout advances its draws on the
                                       device: counter word 1 = *step_base + step */
} F16PolicyArgs;

/* One policy step for every logical row: optional RunningNorm.normalize with clip
 * (cuda_fdm/ppo_gpu.py:210-214), actor logits and critic value of the MLP
 * (claude_code/model.py:195-205), per-channel categorical draw, its summed log-probability
 * (model.py:221-233 / ppo_gpu.py:266-276 actor_step, value_step), and action_to_env
 * (ppo_gpu.py:361-370).  The draw for (physical row r, channel c) inverts the CDF of the
 * channel's softmax at u = (x0 >> 8) * 2^-24, x0 the first word of Philox4x32-10 with key `seed`
 * and counter (r, step, c, salt).  kp = round_up(obs_dim, 32) of the packed weights. */
int f16_policy_step(const F16PolicyArgs *args, void *stream);

/* Stable counting sort of n items by group id (the reference's per-opponent lane partition,
 * R/cuda_fdm/ppo_gpu.py:536-592, without its host synchronisation): item i with id assign[i] in
 * [0, ngroups) gets physical row stride*i + offset; rows[] lists the physical rows group by group
 * in increasing i, group_offsets[0..ngroups] the group boundaries.  Ids outside the range are
 * dropped (counted nowhere).  n <= 2^24, ngroups <= F16_POLICY_MAX_GROUPS; `work` is device
 * scratch of f16_group_workspace_bytes(n). */
long f16_group_workspace_bytes(int n);
int f16_group_rows(const int *assign, int n, int ngroups, int stride, int offset, int *rows,
                   int *group_offsets, void *work, void *stream);

/* sizeof(F16PolicyGroup), sizeof(F16PolicyArgs), and with n >= 4 sizeof(F16PPOArgs),
 * sizeof(F16AdamArgs) (f16_ppo.h) as compiled into the library (out[0..n)), so that a binding
 * can check its struct layouts; no counterpart in the reference. */
int f16_abi_struct_sizes(long *out, int n);

/* RunningNorm.update (cuda_fdm/ppo_gpu.py:194-207) from the batch of `nrows` physical rows
 * (rows[i], or i when rows is NULL) of obs (row stride obs_ld): batch mean and population
 * variance per column, then the parallel-variance merge into mean/var/count (float32, in
 * place).  `work` is device scratch of at least f16_norm_workspace_bytes(nrows, obs_dim). */
long f16_norm_workspace_bytes(int nrows, int obs_dim);
int f16_norm_update(const float *obs, long obs_ld, const int *rows, int nrows, int obs_dim,
                    float *mean, float *var, float *count, void *work, void *stream);

/* f16_norm_update without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  The partial sums live in a fixed 8 MiB device array of the
 * library (one per GPU, held until the process ends; f16_norm_noalloc_max_bytes() returns its
 * size): a batch whose f16_norm_workspace_bytes(nrows, obs_dim) exceeds it is rejected with
 * F16_ETOOBIG (262,144 rows of 214 columns fit).  Calls no allocating routine.  Every call on
 * one GPU shares the array, so calls that overlap on one GPU (two streams, two host threads)
 * race; calls ordered on one stream do not.  Results equal f16_norm_update's bit for bit. */
long f16_norm_noalloc_max_bytes(void);
int f16_norm_update_noalloc(const float *obs, long obs_ld, const int *rows, int nrows,
                            int obs_dim, float *mean, float *var, float *count, void *stream);

/* The second half of f16_norm_update alone: merge the per-block partial sums already in `work`
 * (written by a launch that formed them, e.g. f16_env_post_step with io->norm_partial) into
 * mean/var with the count snapshot kept at the workspace's end.  f16_norm_update(obs, ...) and
 * (partials of the same rows) + f16_norm_merge give identical statistics. */
int f16_norm_merge(int nrows, int obs_dim, float *mean, float *var, void *work, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* F16_POLICY_H */
