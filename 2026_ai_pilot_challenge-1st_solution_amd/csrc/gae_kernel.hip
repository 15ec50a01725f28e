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

// 64-thread workgroups: at BASELINE C4 ([64, 16384, 2] = 32,768 columns) that is 512
// workgroups, two per CU, so every CU streams (256-thread workgroups left half of them idle).
constexpr int kGaeBlock = 64;
// Time steps per chunk.  Chunks are double-buffered: the next chunk's loads are issued before
// the current chunk's recurrence runs, so at T = 64 all of a column's loads are in flight at
// once and each lane waits out one memory latency instead of one per chunk.
constexpr int kGaeChunk = 32;

struct GaeChunk {
  float r[kGaeChunk], v[kGaeChunk], d[kGaeChunk];
};

// Steps t_hi, t_hi - 1, ..., t_hi - kGaeChunk + 1 of column c (steps below 0 are not read).
__device__ __forceinline__ void gae_load(GaeChunk& x, const float* __restrict__ rew,
                                         const float* __restrict__ val,
                                         const float* __restrict__ done, int t_hi, int ncol,
                                         int nenv, int c, int e) {
#pragma unroll
  for (int k = 0; k < kGaeChunk; ++k) {
    const int t = t_hi - k;
    if (t >= 0) {
      const long i = (long)t * ncol + c;
      x.r[k] = rew[i];
      x.v[k] = val[i];
      x.d[k] = done[(long)t * nenv + e];
    }
  }
}

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
  GaeChunk cur, nxt;
  gae_load(cur, rew, val, done, T - 1, ncol, nenv, c, e);
  for (int t = T - 1; t >= 0; t -= kGaeChunk) {
    if (t - kGaeChunk >= 0) gae_load(nxt, rew, val, done, t - kGaeChunk, ncol, nenv, c, e);
#pragma unroll
    for (int k = 0; k < kGaeChunk; ++k) {
      if (t - k >= 0) {
        const float g = gamma * v_next;
        const float delta = (cur.r[k] + g * nnt) - cur.v[k];
        a_next = delta + (gamma_lambda * nnt) * a_next;
        const long i = (long)(t - k) * ncol + c;
        adv[i] = a_next;
        ret[i] = a_next + cur.v[k];
        v_next = cur.v[k];
        nnt = 1.0f - cur.d[k];
      }
    }
    cur = nxt;
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
