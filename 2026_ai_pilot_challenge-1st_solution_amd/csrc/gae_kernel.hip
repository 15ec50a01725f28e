// gae_kernel.hip -- generalized advantage estimation over a rollout buffer (gfx950).
//
// One lane per (engagement, agent) column, reverse scan over time with the running advantage in
// a register.  Buffers are time-major: x[t * ncol + c] with c = env * nagents + agent, so every
// time step is one coalesced 4-byte-per-lane load per buffer.  The done mask is per engagement,
// done[t * nenv + env], shared by its agents.
//
// Semantics and fp32 operation order follow the reference learner (research/competition_36500/
// runtime/cuda_fdm/ppo_gpu.py:1979-1995):
//   nnt_t   = 1 - done[t+1]          (t < T-1),   1 - next_done      (t = T-1)
//   V_next  = val[t+1]               (t < T-1),   last_val           (t = T-1)
//   delta   = (rew[t] + (gamma * V_next) * nnt_t) - val[t]
//   A_t     = delta + ((gamma_lambda * nnt_t) * A_{t+1})
//   ret[t]  = A_t + val[t]
// where done[t] is the done flag entering step t and gamma_lambda is gamma*lambda formed in
// double and rounded once to float, as the reference's Python scalars are.
#include <hip/hip_runtime.h>

#include "f16_capi_common.h"

namespace f16 {

constexpr int kGaeBlock = 256;
constexpr int kGaeChunk = 8;   // time steps whose loads are issued together

__global__ __launch_bounds__(kGaeBlock) void gae_kernel(
    const float* __restrict__ rew, const float* __restrict__ val, const float* __restrict__ done,
    const float* __restrict__ last_val, const float* __restrict__ next_done, int T, int nenv,
    int nagents, float gamma, float gamma_lambda, float* __restrict__ adv,
    float* __restrict__ ret) {
  const int ncol = nenv * nagents;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncol) return;
  const int e = c / nagents;
  float a_next = 0.0f;
  float v_next = last_val[c];
  float nnt = 1.0f - next_done[e];
  int t = T - 1;
  // chunks of kGaeChunk steps: issue all loads of the chunk, then the dependent recurrence
  for (; t >= kGaeChunk - 1; t -= kGaeChunk) {
    float r[kGaeChunk], v[kGaeChunk], d[kGaeChunk];
#pragma unroll
    for (int k = 0; k < kGaeChunk; ++k) {
      const long i = (long)(t - k) * ncol + c;
      r[k] = rew[i];
      v[k] = val[i];
      d[k] = done[(long)(t - k) * nenv + e];
    }
#pragma unroll
    for (int k = 0; k < kGaeChunk; ++k) {
      const float g = gamma * v_next;
      const float delta = (r[k] + g * nnt) - v[k];
      a_next = delta + (gamma_lambda * nnt) * a_next;
      const long i = (long)(t - k) * ncol + c;
      adv[i] = a_next;
      ret[i] = a_next + v[k];
      v_next = v[k];
      nnt = 1.0f - d[k];
    }
  }
  for (; t >= 0; --t) {
    const long i = (long)t * ncol + c;
    const float rr = rew[i], vv = val[i];
    const float g = gamma * v_next;
    const float delta = (rr + g * nnt) - vv;
    a_next = delta + (gamma_lambda * nnt) * a_next;
    adv[i] = a_next;
    ret[i] = a_next + vv;
    v_next = vv;
    nnt = 1.0f - done[(long)t * nenv + e];
  }
}

}  // namespace f16

extern "C" int f16_gae(const float* rew, const float* val, const float* done,
                       const float* last_val, const float* next_done, int T, int nenv,
                       int nagents, float gamma, float gamma_lambda, float* adv, float* ret,
                       void* stream) {
  if (T < 0 || nenv < 0 || nagents < 1) return F16_EINVAL;
  const long ncol = (long)nenv * nagents;
  if (T == 0 || ncol == 0) return 0;
  if (ncol > 0x7fffffffL) return F16_EINVAL;
  if (!rew || !val || !done || !last_val || !next_done || !adv || !ret) return F16_EINVAL;
  const dim3 grid((unsigned)((ncol + f16::kGaeBlock - 1) / f16::kGaeBlock)), block(f16::kGaeBlock);
  hipLaunchKernelGGL(f16::gae_kernel, grid, block, 0, (hipStream_t)stream, rew, val, done,
                     last_val, next_done, T, nenv, nagents, gamma, gamma_lambda, adv, ret);
  return f16_last_error();
}
