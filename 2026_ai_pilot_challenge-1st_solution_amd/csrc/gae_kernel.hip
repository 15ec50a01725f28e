// gae_kernel.hip -- generalized advantage estimation over a rollout buffer (gfx950).
//
// One lane per (engagement, agent) column, reverse scan over time with the running advantage in
// a register.  Buffers are time-major: x[t * ncol + c] with c = env * nagents + agent, so every
// time step is one coalesced 4-byte-per-lane load per buffer.  The done mask is per engagement,
// done[t * nenv + env], shared by its agents.
//
// For T <= 256 (gae_segment_kernel) each workgroup takes 64 columns and gives every 16-step
// time segment its own wavefront.  All of a segment's loads and its deltas (which do not depend
// on the advantage) are issued and formed at once, so the whole rollout buffer is in flight;
// only the advantage itself is handed from segment to segment, latest first, through LDS at one
// workgroup barrier per segment.  A wavefront keeps at most 63 loads outstanding, so one lane
// per column holding every step would have kept only 21 steps (8 MB at 32,768 columns) in
// flight.  Longer rollouts, and batches of 65,536 columns or more, use gae_kernel, one lane per
// column over double-buffered chunks: there the columns alone keep enough loads in flight, and
// the segments' hand-off chain only adds time (rocprofv3 kernel trace, MI355X: [64, 16384, 2]
// 8.6 us with segments vs 11.3 us chunked; [128, 65536, 2] 65.7 us vs 57.5 us).
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

// Time steps per wavefront of gae_segment_kernel (3 x 16 + 2 loads in flight per lane).
constexpr int kGaeSeg = 16;
constexpr int kGaeMaxSegs = 16;      // up to 1,024 threads: T <= 256
constexpr long kGaeChunkedCols = 65536;   // from this many columns on, gae_kernel

// One workgroup per 64 columns, one wavefront per kGaeSeg-step segment (blockDim.x = 64 x the
// number of segments).  Per step the operations and their order are gae_kernel's.
__global__ __launch_bounds__(64 * kGaeMaxSegs) void gae_segment_kernel(
    const float* __restrict__ rew, const float* __restrict__ val, const float* __restrict__ done,
    const float* __restrict__ last_val, const float* __restrict__ next_done, int T, int nenv,
    int nagents, float gamma, float gamma_lambda, float* __restrict__ adv,
    float* __restrict__ ret) {
  __shared__ float a_in[kGaeMaxSegs][64];   // the advantage entering each segment's last step
  const int ncol = nenv * nagents;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nseg = blockDim.x >> 6;
  const int c0 = blockIdx.x * 64 + lane;
  const bool live = c0 < ncol;
  const int c = live ? c0 : ncol - 1;       // lanes past the batch shadow the last column
  const int e = c / nagents;
  const int t0 = w * kGaeSeg;
  const int n = min(kGaeSeg, T - t0);       // steps of this segment (>= 1)
  float r[kGaeSeg], v[kGaeSeg], d[kGaeSeg];
#pragma unroll
  for (int k = 0; k < kGaeSeg; ++k) {
    if (k < n) {
      const long i = (long)(t0 + k) * ncol + c;
      r[k] = rew[i];
      v[k] = val[i];
      if (k > 0) d[k] = done[(long)(t0 + k) * nenv + e];
    }
  }
  // the step after the segment: the next segment's first step, or the bootstrap
  float v_end, d_end;
  if (t0 + n < T) {
    v_end = val[(long)(t0 + n) * ncol + c];
    d_end = done[(long)(t0 + n) * nenv + e];
  } else {
    v_end = last_val[c];
    d_end = next_done[e];
  }
  // delta_t and the advantage's coefficient for every step, ahead of the hand-off
  float delta[kGaeSeg], coef[kGaeSeg];
#pragma unroll
  for (int k = 0; k < kGaeSeg; ++k) {
    if (k < n) {
      const float v_next = (k + 1 < n) ? v[k + 1] : v_end;
      const float nnt = 1.0f - ((k + 1 < n) ? d[k + 1] : d_end);
      const float g = gamma * v_next;
      delta[k] = (r[k] + g * nnt) - v[k];
      coef[k] = gamma_lambda * nnt;
    }
  }
  // the recurrence, latest segment first: segment s runs after s + 1 handed over its advantage
  for (int s = nseg - 1; s >= 0; --s) {
    if (w == s) {
      float a = (s == nseg - 1) ? 0.0f : a_in[s + 1][lane];
#pragma unroll
      for (int k = kGaeSeg - 1; k >= 0; --k) {
        if (k < n) {
          a = delta[k] + coef[k] * a;
          if (live) {
            const long i = (long)(t0 + k) * ncol + c;
            adv[i] = a;
            ret[i] = a + v[k];
          }
        }
      }
      a_in[s][lane] = a;
    }
    if (s > 0) __syncthreads();
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
  const int nseg = (T + f16::kGaeSeg - 1) / f16::kGaeSeg;
  if (nseg <= f16::kGaeMaxSegs && ncol < f16::kGaeChunkedCols) {
    const dim3 grid((unsigned)((ncol + 63) / 64)), block(64 * nseg);
    hipLaunchKernelGGL(f16::gae_segment_kernel, grid, block, 0, (hipStream_t)stream, rew, val,
                       done, last_val, next_done, T, nenv, nagents, gamma, gamma_lambda, adv, ret);
  } else {
    const dim3 grid((unsigned)((ncol + f16::kGaeBlock - 1) / f16::kGaeBlock)), block(f16::kGaeBlock);
    hipLaunchKernelGGL(f16::gae_kernel, grid, block, 0, (hipStream_t)stream, rew, val, done,
                       last_val, next_done, T, nenv, nagents, gamma, gamma_lambda, adv, ret);
  }
  return f16_last_error();
}
