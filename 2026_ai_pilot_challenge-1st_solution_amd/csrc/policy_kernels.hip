// policy_kernels.hip -- rollout policy step on gfx950: RunningNorm update and the fused
// normalise -> actor/critic MLP (bf16 MFMA, fp32 accumulate) -> categorical draw -> controls.
//
// Policy workgroup: 64 observation rows, 4 waves.  The rows are normalised once, rounded to bf16
// and kept in LDS; the actor's and critic's first layers run as one 512-wide GEMM over them,
// each wave owning 128 output columns (2 x 4 tiles of v_mfma_f32_32x32x16_bf16).  Hidden layers
// stay in LDS (bf16, row pitch = width + 8 so the 16-byte fragment reads of 16 consecutive rows
// hit 64 distinct banks); layer 2 runs actor and critic halves on two waves each; the logits
// head (84 columns padded to 96) runs on three waves while the fourth forms the critic's
// 256-long dot products.  Weights stream from L2 (every workgroup reads the same 0.5 MB).
// Sampling is one lane per (row, channel).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "f16_capi_common.h"
#include "f16_policy.h"
#include "philox.h"
#include "sample_math.h"

namespace f16pol {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRows = 64;               // observation rows per workgroup
constexpr int kThreads = 256;
constexpr int kHid = F16_POLICY_HID;    // 256
constexpr int kH2 = 2 * kHid;           // actor | critic
constexpr int kHPitch = kH2 + 8;        // bf16 per LDS row of the hidden activations
constexpr int kBins = F16_POLICY_BINS;  // 21
constexpr int kChan = F16_POLICY_CHANNELS;
constexpr int kLogits = kBins * kChan;  // 84
constexpr int kLogitsPad = 96;
constexpr int kLPitch = kLogitsPad + 1; // f32 per LDS row of logits

// offsets (elements) inside the packed blobs
template <int KP>
struct Blob {
  static constexpr long W1 = 0;
  static constexpr long W2A = W1 + (long)kH2 * KP;
  static constexpr long W2C = W2A + (long)kHid * kHid;
  static constexpr long W3A = W2C + (long)kHid * kHid;
  static constexpr long NBF = W3A + (long)kLogitsPad * kHid;
};
constexpr int kB1 = 0, kB2A = 512, kB2C = 768, kB3A = 1024, kW3C = 1120, kB3C = 1376;
static_assert(kB3C + 1 == F16_POLICY_NF, "f32 blob layout");

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Output element r (0..15) of a 32x32 tile held by `lane`: row and column inside the tile.
__device__ __forceinline__ int tile_row(int lane, int r) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

// acc[i][j] += A(rows 32i.., LDS, pitch) x B(cols cb+32j.., global [col][K])^T over K.
template <int NI, int NJ, int K>
__device__ __forceinline__ void gemm_tiles(f32x16 (&acc)[NI][NJ], const __bf16* __restrict__ As,
                                           int a_pitch, int a_col0,
                                           const __bf16* __restrict__ Bg, int col0, int lane) {
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  bf16x8 b[NJ], bn[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    b[j] = *reinterpret_cast<const bf16x8*>(Bg + (long)(col0 + 32 * j + lr) * K + lk);
#pragma unroll 2
  for (int k0 = 0; k0 < K; k0 += 16) {
    if (k0 + 16 < K) {                // prefetch the next K slice of the weights
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        bn[j] = *reinterpret_cast<const bf16x8*>(Bg + (long)(col0 + 32 * j + lr) * K + k0 + 16 + lk);
    }
    bf16x8 a[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
      a[i] = *reinterpret_cast<const bf16x8*>(As + (32 * i + lr) * a_pitch + a_col0 + k0 + lk);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma(a[i], b[j], acc[i][j]);
    if (k0 + 16 < K) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) b[j] = bn[j];
    }
  }
}

template <int NI, int NJ>
__device__ __forceinline__ void zero(f32x16 (&acc)[NI][NJ]) {
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
}

// bias + tanh, rounded to bf16, into the LDS activation rows
template <int NI, int NJ>
__device__ __forceinline__ void store_tanh(const f32x16 (&acc)[NI][NJ], const float* __restrict__ bias,
                                           __bf16* Hs, int col0, int lane) {
  const int lr = lane & 31;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float bj = bias[col0 + 32 * j + lr];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        Hs[(32 * i + tile_row(lane, r)) * kHPitch + col0 + 32 * j + lr] = (__bf16)tanhf(acc[i][j][r] + bj);
  }
}

template <int KP>
__global__ __launch_bounds__(kThreads) void policy_kernel(const F16PolicyArgs p) {
  constexpr int XP = KP + 8;
  static_assert(kRows * kLPitch * 4 <= kRows * XP * 2, "logits reuse the input rows' LDS");
  __shared__ __align__(16) __bf16 Xs[kRows * XP];
  __shared__ __align__(16) __bf16 Hs[kRows * kHPitch];
  const int gi = blockIdx.y;
  if (gi >= p.ngroups) return;
  const F16PolicyGroup G = p.group[gi];
  const int r0 = G.row_begin + blockIdx.x * kRows;
  if (r0 >= G.row_end) return;                        // uniform per workgroup
  const int nr = min(kRows, G.row_end - r0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const __bf16* wbf = static_cast<const __bf16*>(G.wbf);
  const float* wf = G.wf;

  // ---- normalise (RunningNorm.normalize, ppo_gpu.py:210-214) and stage bf16 rows in LDS
  for (int idx = tid; idx < kRows * KP; idx += kThreads) {
    const int r = idx / KP, k = idx - (idx / KP) * KP;
    float v = 0.0f;
    if (r < nr && k < p.obs_dim) {
      const int li = r0 + r;
      const long pr = p.rows ? p.rows[li] : li;
      float x = p.obs[pr * p.obs_ld + k];
      if (p.mean) {
        x = (x - p.mean[k]) / sqrtf(p.var[k] + p.eps);
        x = x < -p.clip ? -p.clip : (x > p.clip ? p.clip : x);
      }
      if (p.nobs_out) p.nobs_out[(long)li * p.nobs_ld + k] = x;
      v = x;
    }
    Xs[r * XP + k] = (__bf16)v;
  }
  __syncthreads();

  // ---- layer 1: [actor | critic] = tanh(X W1^T + b1), wave owns 128 of the 512 columns
  {
    f32x16 acc[2][4];
    zero(acc);
    gemm_tiles<2, 4, KP>(acc, Xs, XP, 0, wbf + Blob<KP>::W1, 128 * wave, lane);
    store_tanh(acc, wf + kB1, Hs, 128 * wave, lane);
  }
  __syncthreads();

  // ---- layer 2: waves 0-1 actor, 2-3 critic; each 128 columns over its half's 256 inputs
  {
    const int half = wave >> 1;
    const int ocol = (wave & 1) * 128;
    f32x16 acc[2][4];
    zero(acc);
    gemm_tiles<2, 4, kHid>(acc, Hs, kHPitch, half * kHid,
                           wbf + (half ? Blob<KP>::W2C : Blob<KP>::W2A), ocol, lane);
    __syncthreads();                                    // every wave has read layer 1
    store_tanh(acc, wf + (half ? kB2C : kB2A) - half * kHid, Hs, half * kHid + ocol, lane);
  }
  __syncthreads();

  // ---- heads: logits on waves 0-2 (32 columns each), critic value on wave 3
  float* Ls = reinterpret_cast<float*>(Xs);
  if (wave < 3) {
    f32x16 acc[2][1];
    zero(acc);
    gemm_tiles<2, 1, kHid>(acc, Hs, kHPitch, 0, wbf + Blob<KP>::W3A, 32 * wave, lane);
    const int col = 32 * wave + (lane & 31);
    const float bc = wf[kB3A + col];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) Ls[(32 * i + tile_row(lane, r)) * kLPitch + col] = acc[i][0][r] + bc;
  } else {
    const int row = lane;
    const float* w3 = wf + kW3C;
    float s = 0.0f;
#pragma unroll 4
    for (int k0 = 0; k0 < kHid; k0 += 8) {
      const bf16x8 h = *reinterpret_cast<const bf16x8*>(Hs + row * kHPitch + kHid + k0);
#pragma unroll
      for (int q = 0; q < 8; ++q) s += (float)h[q] * w3[k0 + q];
    }
    if (row < nr && p.value) p.value[r0 + row] = s + wf[kB3C];
  }
  __syncthreads();

  // ---- per (row, channel): softmax, draw, log-probability, control
  const int row = tid >> 2, ch = tid & 3;
  const float* l = Ls + row * kLPitch + ch * kBins;
  float lg[kBins];
#pragma unroll
  for (int k = 0; k < kBins; ++k) lg[k] = l[k];
  float m = lg[0];
  int amax = 0;
#pragma unroll
  for (int k = 1; k < kBins; ++k)
    if (lg[k] > m) { m = lg[k]; amax = k; }
  float e[kBins], s = 0.0f;
#pragma unroll
  for (int k = 0; k < kBins; ++k) { e[k] = f16rng::exp_nonpos(lg[k] - m); s += e[k]; }
  const int li = r0 + row;
  const long pr = (row < nr) ? (p.rows ? p.rows[li] : li) : 0;
  int idx = amax;
  if (!p.deterministic) {
    uint32_t c[4] = {(uint32_t)pr, p.step, (uint32_t)ch, p.salt};
    f16rng::philox4x32_10(c, (uint32_t)p.seed, (uint32_t)(p.seed >> 32));
    const float u = (float)(c[0] >> 8) * 0x1p-24f;
    const float target = u * s;
    float cum = 0.0f;
    idx = kBins - 1;
#pragma unroll
    for (int k = 0; k < kBins; ++k) {
      cum += e[k];
      if (cum > target) { idx = k; break; }
    }
  }
  float lp = 0.0f;
#pragma unroll
  for (int k = 0; k < kBins; ++k)
    if (k == idx) lp = (lg[k] - m) - logf(s);
  lp += __shfl_xor(lp, 1);
  lp += __shfl_xor(lp, 2);
  if (row < nr) {
    if (p.act_idx) p.act_idx[(long)li * kChan + ch] = idx;
    if (p.logp && ch == 0) p.logp[li] = lp;
    if (p.env_actions) {
      float g = p.grid[idx];
      if (ch == 3) g = 0.5f * g + 0.5f;
      p.env_actions[pr * kChan + ch] = (double)g;
    }
    if (p.logits_out) {
#pragma unroll
      for (int k = 0; k < kBins; ++k) p.logits_out[(long)li * kLogits + ch * kBins + k] = lg[k];
    }
  }
}

// ---- RunningNorm.update: per-block column partial sums, then one fixed-order merge
constexpr int kNormThreads = 256;
constexpr int kNormRowsPerBlock = 128;

__global__ __launch_bounds__(kNormThreads) void norm_partial_kernel(
    const float* __restrict__ obs, long ld, const int* __restrict__ rows, int nrows, int dim,
    double* __restrict__ work) {
  const int c = threadIdx.x;
  const int b = blockIdx.x;
  if (c >= dim) return;
  const int i0 = b * kNormRowsPerBlock, i1 = min(nrows, i0 + kNormRowsPerBlock);
  double s = 0.0, q = 0.0;
  for (int i = i0; i < i1; ++i) {
    const long pr = rows ? rows[i] : i;
    const double x = obs[pr * ld + c];
    s += x;
    q += x * x;
  }
  work[(long)b * 2 * dim + c] = s;
  work[(long)b * 2 * dim + dim + c] = q;
}

__global__ __launch_bounds__(kNormThreads) void norm_merge_kernel(
    const double* __restrict__ work, int nblocks, int nrows, int dim, float* __restrict__ mean,
    float* __restrict__ var, float* __restrict__ count) {
  const int c = threadIdx.x;
  const float cnt = *count;
  __syncthreads();                      // every lane has read the shared count
  if (c < dim) {
    double s = 0.0, q = 0.0;
    for (int b = 0; b < nblocks; ++b) {
      s += work[(long)b * 2 * dim + c];
      q += work[(long)b * 2 * dim + dim + c];
    }
    const double mu = s / nrows;
    double v = q / nrows - mu * mu;
    v = v < 0.0 ? 0.0 : v;
    const float b_mean = (float)mu, b_var = (float)v, b_count = (float)nrows;
    const float delta = b_mean - mean[c];
    const float tot = cnt + b_count;
    mean[c] = mean[c] + delta * (b_count / tot);
    const float m_a = var[c] * cnt;
    const float m_b = b_var * b_count;
    const float M2 = m_a + m_b + (delta * delta) * (cnt * b_count / tot);
    var[c] = M2 / tot;
  }
  if (c == 0) *count = cnt + (float)nrows;
}

static int norm_blocks(int nrows) { return (nrows + kNormRowsPerBlock - 1) / kNormRowsPerBlock; }

}  // namespace f16pol

using namespace f16pol;

extern "C" int f16_policy_step(const F16PolicyArgs* a, void* stream) {
  if (!a || !a->obs || a->ngroups < 1 || a->ngroups > F16_POLICY_MAX_GROUPS) return F16_EINVAL;
  if (a->obs_dim != 184 && a->obs_dim != 214) return F16_EINVAL;
  if (a->obs_ld < a->obs_dim || !a->grid) return F16_EINVAL;
  if (a->mean && !a->var) return F16_EINVAL;
  if (a->nobs_out && a->nobs_ld < a->obs_dim) return F16_EINVAL;
  int max_rows = 0;
  for (int g = 0; g < a->ngroups; ++g) {
    const F16PolicyGroup& G = a->group[g];
    if (G.row_begin < 0 || G.row_end < G.row_begin || !G.wbf || !G.wf) return F16_EINVAL;
    if (((uintptr_t)G.wbf & 15) != 0) return F16_EINVAL;
    max_rows = max(max_rows, G.row_end - G.row_begin);
  }
  if (max_rows == 0) return 0;
  const dim3 grid((unsigned)((max_rows + kRows - 1) / kRows), (unsigned)a->ngroups), block(kThreads);
  if (a->obs_dim == 184)
    hipLaunchKernelGGL(policy_kernel<192>, grid, block, 0, (hipStream_t)stream, *a);
  else
    hipLaunchKernelGGL(policy_kernel<224>, grid, block, 0, (hipStream_t)stream, *a);
  return f16_last_error();
}

extern "C" int f16_abi_struct_sizes(long* out, int n) {
  const long sizes[4] = {(long)sizeof(F16PolicyGroup), (long)sizeof(F16PolicyArgs), 0, 0};
  if (!out || n < 2) return F16_EINVAL;
  for (int i = 0; i < 2; ++i) out[i] = sizes[i];
  return 0;
}

extern "C" long f16_norm_workspace_bytes(int nrows, int obs_dim) {
  if (nrows < 0 || obs_dim < 0) return -1;
  return (long)norm_blocks(nrows) * 2 * obs_dim * (long)sizeof(double);
}

extern "C" int f16_norm_update(const float* obs, long obs_ld, const int* rows, int nrows,
                               int obs_dim, float* mean, float* var, float* count, void* work,
                               void* stream) {
  if (nrows < 0 || obs_dim < 1 || obs_dim > kNormThreads || obs_ld < obs_dim) return F16_EINVAL;
  if (nrows == 0) return 0;
  if (!obs || !mean || !var || !count || !work) return F16_EINVAL;
  const int nb = norm_blocks(nrows);
  hipLaunchKernelGGL(norm_partial_kernel, dim3(nb), dim3(kNormThreads), 0, (hipStream_t)stream,
                     obs, obs_ld, rows, nrows, obs_dim, (double*)work);
  hipLaunchKernelGGL(norm_merge_kernel, dim3(1), dim3(kNormThreads), 0, (hipStream_t)stream,
                     (const double*)work, nb, nrows, obs_dim, mean, var, count);
  return f16_last_error();
}
