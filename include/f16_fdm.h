/* f16_fdm.h -- C ABI of the MI355X F-16 flight-dynamics path (libf16hip.so).
 *
 * Plain pointers and sizes only.  All pointers are device pointers unless stated otherwise;
 * `stream` is a hipStream_t (the caller's current stream; nothing is synchronised).
 * Return value: 0 on success, F16_EINVAL (-1) for bad sizes/strides/null pointers,
 * F16_ERATE (-2) for an unsupported FCS rate, -(1000 + hipError_t) for a launch error.
 *
 * State layout: structure-of-arrays, field k (0..100, the reference's FdmState order,
 * cuda_fdm/ic.py:92-114) of aircraft a at states[k * ld + a]; ld >= nac.
 */
#ifndef F16_FDM_H
#define F16_FDM_H
#ifdef __cplusplus
extern "C" {
#endif

/* Advance nac aircraft by `substeps` 1/60-s steps with each aircraft's action held.
 * actions: (nac, 4) row-major [aileron, elevator, rudder in -1..1, throttle in 0..1].
 * obs (optional, may be NULL): (17, obs_ld) structure-of-arrays FDM output of the last substep:
 *   eci_pos(3) eci_vel(3) euler(3) vUVW(3) alpha beta mach Vt alt_asl.
 * fcs_rate: FCS component rate in Hz, 120 (root lineage) or 60 (184-D lineage).
 * Replaces the NVRTC kernel `fdm_step_batch(FdmState*, const double* actions, int nac,
 * int substeps, double* obs)` (cuda_fdm/gen/fdm_kernel.cu:32) as launched by
 * GpuDogfight.step (cuda_fdm/gpu_env.py:95-106). */
int f16_fdm_step_batch(double* states, long ld, const double* actions, int nac, int substeps,
                       int fcs_rate, double* obs, long obs_ld, void* stream);

/* f16_fdm_step_batch that also writes finite[a] = 1 if all 101 state values of aircraft a
 * after the step are finite, else 0 ((nac) bytes), formed from the values the kernel holds in
 * registers as it stores them -- the flag GpuDogfightVecEnv.step computes over `states` after
 * the physics (R/cuda_fdm/rl_env.py:545), without reading the state back.  substeps >= 1.
 * The env step hands it to f16_env_post_step as F16EnvStepIO.state_finite. */
int f16_fdm_step_batch_finite(double* states, long ld, const double* actions, int nac,
                              int substeps, int fcs_rate, double* obs, long obs_ld,
                              unsigned char* finite, void* stream);

/* GpuDogfight.step in one launch: f16_fdm_step_batch (finite NULL) or
 * f16_fdm_step_batch_finite (finite non-NULL, substeps >= 1) that also copies the (nac, 4)
 * actions it reads into actions_keep -- the reference step's `self.actions.copy_(a)` before
 * its launch (cuda_fdm/gpu_env.py:98-99), folded into the kernel.  actions_keep must not
 * overlap actions (F16_EINVAL).  Written for every aircraft, also when substeps is 0. */
int f16_fdm_step_batch_keep(double* states, long ld, const double* actions,
                            double* actions_keep, int nac, int substeps, int fcs_rate,
                            double* obs, long obs_ld, unsigned char* finite, void* stream);

/* The same step with each substep of 64 aircraft spread over two cooperating wavefronts (flight
 * and systems) instead of the four of f16_fdm_step_batch (integrator, aero build-up, FCS, mass /
 * atmosphere / engine).  Results equal f16_fdm_step_batch bit for bit; kept as its
 * cross-check.  Same arguments, contract and reference interface. */
int f16_fdm_step_batch_split(double* states, long ld, const double* actions, int nac,
                             int substeps, int fcs_rate, double* obs, long obs_ld, void* stream);

/* The same step computed with one lane (one wavefront) per aircraft doing the whole substep.
 * Results equal f16_fdm_step_batch bit for bit; f16_fdm_step_batch spreads each substep over
 * four cooperating wavefronts.  Same arguments, contract and reference interface. */
int f16_fdm_step_batch_onelane(double* states, long ld, const double* actions, int nac,
                               int substeps, int fcs_rate, double* obs, long obs_ld,
                               void* stream);

/* Seed aircraft states from initial conditions on the device.
 * ic: (n, 10) rows [lat_deg, lon_deg, alt_ft, vt_fps, phi_deg, theta_deg, psi_deg, alpha_deg,
 *     beta_deg, fuel_lbs] (geodetic latitude, epa = 0, fuel-flow 0).
 * rows (optional): (n,) int64 target aircraft index per IC row; NULL seeds rows 0..n-1.
 *     A row index outside [0, ld) is skipped (nothing written); callers validate first.
 * Replaces the host-side build_seed_vector (cuda_fdm/ic.py:117-138) used by
 * GpuDogfight.reset_ic (cuda_fdm/gpu_env.py:78-92) and the env's IC pools. */
int f16_seed_batch(const double* ic, int n, int fcs_rate, double* states, long ld,
                   const long* rows, void* stream);

/* Host pointer out4 <- {registers per lane, static LDS bytes, scratch bytes per lane,
 * max threads per block} of the kernel f16_fdm_step_batch launches: the four-wave kernel
 * without the 17-value output (cf. cuda_fdm/tests/profile_kernel.py:23-33).  NULL out4 ->
 * F16_EINVAL. */
int f16_fdm_kernel_info(int fcs_rate, int* out4);

/* The same footprint for the one-lane kernel behind f16_fdm_step_batch_onelane
 * (cuda_fdm/tests/profile_kernel.py:23-33 reads one kernel; this build has two). */
int f16_fdm_kernel_info_onelane(int fcs_rate, int* out4);

/* The step in single precision: GpuDogfight(precision="fp32") (cuda_fdm/gpu_env.py:33-58, whose
 * kernel is the fp64 source with every double made float, cuda_fdm/tests/cuda_rt.py:150-160).
 * states (101, ld) and obs (17, obs_ld) float, structure-of-arrays as above; actions (nac, 4)
 * float.  The four-wave kernel of f16_fdm_step_batch, compiled from the same model source in
 * float.  Same argument rules and return codes as f16_fdm_step_batch. */
int f16_fdm_step_batch_f32(float* states, long ld, const float* actions, int nac, int substeps,
                           int fcs_rate, float* obs, long obs_ld, void* stream);

/* Footprint of the kernel behind f16_fdm_step_batch_f32, as f16_fdm_kernel_info. */
int f16_fdm_kernel_info_f32(int fcs_rate, int* out4);

/* Generalized advantage estimation over a rollout buffer (fp32).
 * rew, val, adv, ret: (T, nenv*nagents) time-major, column = env*nagents + agent;
 * done: (T, nenv), done[t] = done flag entering step t; last_val: (nenv*nagents);
 * next_done: (nenv).  gamma_lambda = gamma*lambda rounded once to float.
 * Replaces the reverse Python loop of PPOGPUTrainer.collect_rollout
 * (research/competition_36500/runtime/cuda_fdm/ppo_gpu.py:1979-1995). */
int f16_gae(const float* rew, const float* val, const float* done, const float* last_val,
            const float* next_done, int T, int nenv, int nagents, float gamma,
            float gamma_lambda, float* adv, float* ret, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* F16_FDM_H */
