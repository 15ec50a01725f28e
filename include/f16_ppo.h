/* f16_ppo.h -- C ABI of the PPO update kernels (libf16hip.so): minibatch gradients of the
 * clipped-surrogate actor loss and the value loss of the discrete actor-critic MLP, gradient-norm
 * clipping plus Adam on fp32 master parameters, and the repacking of the rollout kernel's blobs.
 *
 * Launch on `stream` (hipStream_t, NULL = default), no synchronisation, no allocation; device
 * pointers only; 0 on success, F16_E* (< 0) for a rejected argument, -(1000 + hipError_t) for a
 * launch failure.
 *
 * Flat parameter layout (fp32; the order of the reference's actor_parameters() followed by
 * critic_parameters(), claude_code/model.py:179-185), D = obs_dim:
 *   actor:  W1 [256][D] | b1 [256] | W2 [256][256] | b2 [256] | W3 [84][256] | b3 [84]
 *   critic: W1 [256][D] | b1 [256] | W2 [256][256] | b2 [256] | w3 [256]     | b3 [1]
 * n_actor = 256 D + 87636, n_critic = 256 D + 66305; the critic follows the actor directly.
 */
#ifndef F16_PPO_H
#define F16_PPO_H

#ifdef __cplusplus
extern "C" {
#endif

/* out[0] = n_actor, out[1] = n_critic for obs_dim (184 or 214). */
int f16_ppo_param_counts(int obs_dim, long *out2);

/* Transposed bf16 blob the backward pass reads (elements): W3a^T [256][96] (columns 84..95
 * zero), W2a^T [256][256], W2c^T [256][256], each fragment-major like the f16_policy.h blob. */
#define F16_PPO_WT_ELEMS (256 * 96 + 2 * 256 * 256)

/* Device scratch for f16_ppo_grad over minibatches of up to mb_rows rows (1 .. 2^24; -1
 * beyond, and f16_ppo_grad returns F16_EINVAL for such a minibatch). */
long f16_ppo_workspace_bytes(int obs_dim, int mb_rows);

/* Per-minibatch statistics written by f16_ppo_grad (float32, means over the minibatch). */
#define F16_PPO_STAT_POLICY_LOSS 0   /* mean(max(pg1, pg2)) */
#define F16_PPO_STAT_VALUE_LOSS 1    /* 0.5 mean((v - ret)^2) */
#define F16_PPO_STAT_ENTROPY 2       /* mean summed entropy */
#define F16_PPO_STAT_APPROX_KL 3     /* mean((ratio - 1) - log ratio) */
#define F16_PPO_STAT_CLIPFRAC 4      /* mean(|ratio - 1| > clip) */
#define F16_PPO_STAT_ADV_MEAN 5      /* minibatch advantage mean and std (before normalising) */
#define F16_PPO_STAT_ADV_STD 6
#define F16_PPO_NSTATS 8

typedef struct F16PPOArgs {
    /* rollout buffers flattened over (step, row): `count` transitions */
    const float *obs;            /* normalised observations, row stride obs_ld floats */
    long obs_ld;
    int obs_dim;                 /* 184 or 214 */
    const long long *act;        /* (count, 4) sampled bins */
    const float *old_logp;       /* (count) log-probability at collection */
    const float *adv, *ret;      /* (count) GAE advantages and returns */
    long count;
    /* the minibatch: transitions idx[0 .. mb_rows) (a slice of the epoch's permutation) */
    const long long *idx;
    int mb_rows;
    /* loss (PPOConfig, R/cuda_fdm/ppo_gpu.py:955-978) */
    float clip_coef, ent_coef, vf_coef;
    int norm_adv;
    /* the network as the rollout kernel holds it (f16_policy.h blobs) plus the transposed blob */
    const void *wbf;
    const float *wf;
    const void *wT;
    /* outputs */
    float *grad;                 /* flat (n_actor + n_critic) loss gradients, unclipped */
    float *stats;                /* F16_PPO_NSTATS floats */
    void *work;                  /* f16_ppo_workspace_bytes(obs_dim, >= mb_rows) */
    const float *adv_stats;      /* optional: this minibatch's advantage mean and sample std
                                    (2 floats, f16_ppo_adv_stats); NULL = formed here */
} F16PPOArgs;

/* One minibatch of PPOGPUTrainer.update (R/cuda_fdm/ppo_gpu.py:2059-2109): the actor loss
 * max(-A ratio, -A clamp(ratio, 1 - clip, 1 + clip)).mean() - ent_coef * entropy.mean() with A the
 * minibatch-normalised advantage ((A - mean) / (std + 1e-8), sample std, when norm_adv and
 * mb_rows > 1), the critic loss vf_coef * 0.5 ((v - ret)^2).mean(), and both gradients with
 * respect to the flat parameters (the actor's through log_softmax, the critic's through the value
 * head); bf16 operands on MFMA, fp32 accumulation, deterministic reductions. */
int f16_ppo_grad(const F16PPOArgs *args, void *stream);

/* The advantage mean and sample std of every minibatch of an epoch, in two launches instead of
 * two per minibatch: minibatch j is idx[j mb_rows .. min((j + 1) mb_rows, total)) (the epoch's
 * permutation cut as PPOGPUTrainer.update cuts it, ppo_gpu.py:2055-2078), its mean and std at
 * out[2j], out[2j + 1] (device), the same values f16_ppo_grad forms for it alone.  nmb must be
 * ceil(total / mb_rows); work: f16_ppo_adv_work_bytes(mb_rows, nmb) device bytes. */
long f16_ppo_adv_work_bytes(int mb_rows, int nmb);
int f16_ppo_adv_stats(const float *adv, const long long *idx, long total, long count, int mb_rows,
                      int nmb, float *out, void *work, void *stream);

typedef struct F16AdamArgs {
    int obs_dim;
    float *param;                /* flat fp32 master parameters (n_actor + n_critic) */
    float *exp_avg, *exp_avg_sq; /* Adam moments, same layout */
    float *grad;                 /* flat gradients; scaled in place by the clip coefficient */
    float max_grad_norm;         /* per network (ppo_gpu.py:2089, 2104) */
    double actor_lr, critic_lr;  /* Python floats, as torch.optim.Adam holds them; the step's */
    double beta1, beta2, eps;    /* scalars are formed in double and rounded once, as torch's
                                    foreach Adam does (0.9, 0.999, eps 1e-5: ppo_gpu.py:1303) */
    int step;                    /* optimizer step count after this step (1, 2, ...) */
    float *grad_norms;           /* (2) out: actor and critic total norms before clipping */
    void *wbf;                   /* rollout blobs to refresh from the new parameters, or NULL */
    float *wf;
    void *wT;                    /* transposed blob to refresh, or NULL */
    void *work;                  /* f16_ppo_workspace_bytes scratch (shared with f16_ppo_grad) */
} F16AdamArgs;

/* clip_grad_norm_ of the actor's and the critic's parameters (each its own total 2-norm,
 * coefficient min(1, max_norm / (norm + 1e-6))) followed by torch.optim.Adam's update of each
 * (ppo_gpu.py:2088-2090, 2103-2105; the foreach formulation: lerp of the first moment,
 * bias-corrected denominator sqrt(v) / sqrt(1 - beta2^t) + eps, step lr / (1 - beta1^t)), then the
 * blobs f16_policy_step and f16_ppo_grad read. */
int f16_ppo_adam_step(const F16AdamArgs *args, void *stream);

/* The rollout blobs (f16_policy.h layout, kp = round_up(obs_dim, 32)) and the transposed blob
 * from flat master parameters; wT may be NULL. */
int f16_ppo_pack(const float *param, int obs_dim, void *wbf, float *wf, void *wT, void *stream);

/* The aggregate finite check before an update: one flag for the reference's
 * torch.stack([trajectory_finite] + [torch.isfinite(x).all() for x in (b_obs, b_rew, b_val,
 * b_logp, adv, ret)]).all() (R/cuda_fdm/ppo_gpu.py:2000-2009), read in one pass.  A span is n
 * elements of elem_bytes at ptr (aligned to elem_bytes; n = 0 allowed): 4 = float32 and 8 =
 * float64, each element finite (not inf, not NaN); 1 = uint8/bool flags, each nonzero.  *flag (one
 * device byte) = 1 when every span holds, else 0.  Two launches (the flag set, then the scan). */
#define F16_FINITE_MAX_SPANS 16
typedef struct F16FiniteSpan {
    const void *ptr;
    long n;
    int elem_bytes;
} F16FiniteSpan;
int f16_all_finite(const F16FiniteSpan *spans, int nspans, unsigned char *flag, void *stream);

/* The epoch's shuffle of the transitions, in place of torch.randperm(count)
 * (R/cuda_fdm/ppo_gpu.py:2055): perm[0 .. n) (int64, device) = a permutation of 0 .. n-1 drawn by
 * the 64-bit device word *key -- an eight-round Feistel network (MurmurHash3-finaliser round
 * functions, Philox4x32-10 round keys) with equal halves on the smallest power-of-four domain >= n
 * below 2^15 elements, unequal halves of 8 bits or more on the smallest power of two above,
 * cycle-walked into [0, n).  1 <= n <= 2^31. */
int f16_permutation(long long *perm, long n, const unsigned long long *key, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* F16_PPO_H */
