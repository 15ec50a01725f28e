// policy_kernels.hip -- rollout policy step on gfx950: RunningNorm update and the fused
// normalise -> actor/critic MLP (bf16 MFMA, fp32 accumulate) -> categorical draw -> controls.
//
// Policy workgroup: 64 observation rows, 8 waves; 71 KB of LDS, so two workgroups share a CU.
// The rows are loaded with every load in flight at once (float4 where the rows allow it, each
// thread keeping one column), normalised with per-column statistics staged in LDS, rounded to
// bf16 and kept in LDS.  Every wave owns 32 units of every hidden layer of both networks (2 tiles
// of v_mfma_f32_32x32x16_bf16 with units as the matrix rows, so a lane's results are 4
// consecutive units of one observation row: one 8-byte LDS store per 4 activations; row pitch
// 264, so 16-byte fragment reads of 16 consecutive rows hit 64 distinct banks).  The two
// networks' layers alternate so that one network's matrix products run beside the other's tanh
// epilogue (the kernel is bound by the vector ALU, which the tanh fills).  The logits head (84
// units padded to 96) runs on six waves and its results overlay an activation buffer for the
// draw; the critic's value is summed from per-wave partials formed in its last epilogue.
// Weights stream from L2 a few K-slices ahead (every workgroup reads the same 0.55 MB).
// Sampling is one lane per (row, channel).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <mutex>

#include "f16_capi_common.h"
#include "f16_policy.h"
#include "f16_ppo.h"
#include "philox.h"
#include "policy_mfma.h"
#include "sample_math.h"

namespace f16pol {

// acc += W x A^T exactly as gemm_t forms it (the same K slices in the same order, so the sums are
// bit-identical), with another layer's epilogue spread over the slices: epilogue step j (of 8)
// follows the MFMAs of slice j * NK / 8.  A wave's matrix products and its vector epilogue then
// interleave instead of alternating, and the SIMD keeps both pipes busy.
template <int NR, int K, class Epi>
__device__ __forceinline__ void gemm_epi(f32x16 (&acc)[NR], const __bf16* __restrict__ Wg, int u0,
                                         const __bf16* __restrict__ As, int a_pitch, int lane,
                                         Epi&& epi) {
  constexpr int PD = 2;                               // weight slices in flight ahead
  constexpr int NK = K / 16;
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  const __bf16* wp = Wg + (long)(u0 >> 5) * (K / 16) * 512 + lane * 8;
  const __bf16* ap = As + lr * a_pitch + lk;
  bf16x8 w[PD + 1];
#pragma unroll
  for (int q = 0; q < PD; ++q) w[q] = *reinterpret_cast<const bf16x8*>(wp + 512 * q);
  // one activation fragment per row tile: the next slice's is read right after this slice's
  // MFMAs take theirs, and the epilogue step between covers the LDS latency
  bf16x8 a[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) a[r] = *reinterpret_cast<const bf16x8*>(ap + 32 * r * a_pitch);
#pragma unroll
  for (int s = 0; s < NK; ++s) {
    if (s + PD < NK) w[(s + PD) % (PD + 1)] =
        *reinterpret_cast<const bf16x8*>(wp + 512 * (s + PD));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = mfma(w[s % (PD + 1)], a[r], acc[r]);
    if (s + 1 < NK) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
        a[r] = *reinterpret_cast<const bf16x8*>(ap + 32 * r * a_pitch + 16 * (s + 1));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if ((j * NK) / 8 == s) epi(j);
  }
}

// Epilogue step j of a hidden layer (two 32-row tiles): tanh of 4 consecutive units of one row,
// rounded to bf16, one 8-byte LDS store at E[row][unit].  Steps 0..7 cover the 32 x 64 block.
struct TanhEpi {
  const f32x16* acc;
  __bf16* E;
  int u0, lane;
  __device__ __forceinline__ void operator()(int j) const {
    const int g = j >> 1, r = j & 1;
    const int unit = u0 + 8 * g + (lane >> 5) * 4;
    bf16x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (__bf16)tanh_act(acc[r][4 * g + i]);
    *reinterpret_cast<bf16x4*>(E + (32 * r + (lane & 31)) * kHPitch + unit) = v;
  }
};

// Epilogue step j of the critic's layer 2: the same tanh and bf16 rounding, then the value
// head's products for those 4 units summed into this lane's row partial vp[r].
struct ValueEpi {
  const f32x16* acc;
  const float4* w3;      // the head weights of this lane's units, group g at w3[g]
  float* vp;
  __device__ __forceinline__ void operator()(int j) const {
    const int g = j >> 1, r = j & 1;
    float s = vp[r];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float h = (float)(__bf16)tanh_act(acc[r][4 * g + i]);
      s += h * w3[g][i];
    }
    vp[r] = s;
  }
};

// threadIdx.x % 64 through an empty asm, so the compiler derives lane values where they are used
// instead of holding them in registers across phases.
__device__ __forceinline__ int fresh_lane() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t & 63;
}

// Row staging: VW floats per load (4 where the rows allow 16-byte access), NC vectors per row,
// RP rows per pass of the 512 threads, NP passes for the 64 rows.  Each thread keeps one vector
// column for every pass, so its normalisation statistics are read once.
template <int D, int VW>
struct Stage {
  static constexpr int NC = D / VW;
  static constexpr int RP = kThreads / NC;
  static constexpr int NP = (kRows + RP - 1) / RP;
};

// One policy workgroup: 64 observation rows, 8 waves.  Wave w owns units [32w, 32w + 32) of
// every hidden layer of both networks (two 32-row MFMA tiles each).  LDS: A holds the
// normalised rows, then the critic's layer-1 activations; B the actor's layer-1, then layer-2
// activations, then the logits.  Phases (barriers between them):
//   1  actor layer 1 products                       (reads A)
//   2  critic layer 1 products + actor layer 1 tanh (reads A, writes B)
//   3  actor layer 2 products  + critic layer 1 tanh (reads B, writes A)
//   4  critic layer 2 products + actor layer 2 tanh (reads A, writes B)
//   5  logits products (waves 0-5) + critic layer 2 tanh and value partials (reads B)
//   6  logits to LDS; 7 draws (waves 0-3) beside the value sums (wave 4).
// Without values asked for (a league's opponents), the critic's work is skipped.  The actor's
// arithmetic is the PPO update's forward (policy_mfma.h), operation for operation.
// (HIP's second launch bound is waves per SIMD: two 8-wave workgroups per CU are four per SIMD,
// which caps the registers at 128.)
template <int KP, int VW>
__global__ __launch_bounds__(kThreads, 4) void policy_kernel(const F16PolicyArgs p) {
  static_assert(kRows * kLPitch * 4 <= kRows * kHPitch * 2, "logits reuse B");
  static_assert(KP <= kHPitch, "rows fit A");
  __shared__ __align__(16) __bf16 As[kRows * kHPitch];
  __shared__ __align__(16) __bf16 Bs[kRows * kHPitch];
  __shared__ __align__(16) float col_mean[KP], col_sd[KP], col_rcp[KP];
  __shared__ float vpart[kWaves][kRows];
  // The workgroup's network and 64-row tile.  The row ranges are uniform: kept in scalar
  // registers (a vector load would hold them, and everything derived from them, in vector
  // registers for the whole kernel).
  int gi, r0, ge;
  if (p.total_group_rows > 0) {
    // packed grid (device offsets): the groups' tiles in group order.  Workgroups go to the 8
    // XCDs round robin (workgroup i to XCD i % 8), each XCD with its own L2, so workgroup i takes
    // tile start(i % 8) + i / 8 of a split of the tiles into 8 contiguous runs: each XCD's L2
    // then holds the weights of one or two of the networks rather than of all of them.
    int t;
    {
      constexpr int kX = 8;
      const int n = gridDim.x, q = n / kX, rem = n % kX, x = blockIdx.x % kX;
      t = x * q + min(x, rem) + (int)(blockIdx.x / kX);
    }
    gi = -1;
    r0 = ge = 0;
    for (int g = 0; g < p.ngroups; ++g) {
      const int b = __builtin_amdgcn_readfirstlane(p.group_offsets[g]);
      const int e = __builtin_amdgcn_readfirstlane(p.group_offsets[g + 1]);
      const int nt = e > b ? (e - b + kRows - 1) / kRows : 0;
      if (t < nt) {
        gi = g;
        r0 = b + t * kRows;
        ge = e;
        break;
      }
      t -= nt;
    }
    if (gi < 0) return;                               // past the last group's last tile
  } else {
    gi = blockIdx.y;
    if (gi >= p.ngroups) return;
    const int gb = __builtin_amdgcn_readfirstlane(p.group_offsets ? p.group_offsets[gi]
                                                                  : p.group[gi].row_begin);
    ge = __builtin_amdgcn_readfirstlane(p.group_offsets ? p.group_offsets[gi + 1]
                                                        : p.group[gi].row_end);
    r0 = gb + blockIdx.x * kRows;
    if (r0 >= ge) return;                             // uniform per workgroup
  }
  const F16PolicyGroup G = p.group[gi];
  const int nr = min(kRows, ge - r0);
  const float* g_mean = G.mean ? G.mean : p.mean;
  const float* g_var = G.mean ? G.var : p.var;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: a scalar register
  const __bf16* wbf = static_cast<const __bf16*>(G.wbf);
  const float* wf = G.wf;
  constexpr int D = KP == 192 ? 184 : 214;              // observation width of this kernel
  const bool critic = p.value != nullptr;             // the same for every workgroup
  const int u0 = 32 * wave;

  // ---- normalise (RunningNorm.normalize, ppo_gpu.py:210-214) and stage bf16 rows in A.
  // Row indices, then every row load (unconditional: items of rows past nr read row nr - 1 and
  // are dropped; a choice or skip inside the load loop made the compiler wait for all
  // outstanding loads at each branch join), then the statistics and their barrier, so both
  // latencies overlap.
  using S = Stage<D, VW>;
  typedef float vec __attribute__((ext_vector_type(VW)));
  vec x[S::NP];                                       // the rows, raw then normalised
  {
    const int cv = tid % S::NC, rb = tid / S::NC;     // vector column, first row
    const bool act = rb < S::RP;                      // threads past RP * NC only load
    long pr[S::NP];
    if (p.rows) {
#pragma unroll
      for (int q = 0; q < S::NP; ++q) pr[q] = p.rows[r0 + min(rb + S::RP * q, nr - 1)];
    } else {
#pragma unroll
      for (int q = 0; q < S::NP; ++q) pr[q] = r0 + min(rb + S::RP * q, nr - 1);
    }
#pragma unroll
    for (int q = 0; q < S::NP; ++q)
      x[q] = *reinterpret_cast<const vec*>(p.obs + pr[q] * p.obs_ld + VW * cv);
    if (tid < KP) {
      const bool on = g_mean && tid < D;
      col_mean[tid] = on ? g_mean[tid] : 0.0f;
      const float sd = on ? sqrtf(g_var[tid] + p.eps) : 1.0f;
      col_sd[tid] = sd;
      col_rcp[tid] = 1.0f / sd;                       // correctly rounded (IEEE division)
    }
    __syncthreads();
    if (act) {
      const vec mu = *reinterpret_cast<const vec*>(col_mean + VW * cv);
      const vec sd = *reinterpret_cast<const vec*>(col_sd + VW * cv);
      const vec rc = *reinterpret_cast<const vec*>(col_rcp + VW * cv);
#pragma unroll
      for (int q = 0; q < S::NP; ++q) {
        const int r = rb + S::RP * q;
        if (r < kRows) {
          vec v = {};
          if (r < nr) {
            v = x[q];
            if (g_mean) {
#pragma unroll
              for (int i = 0; i < VW; ++i) {
                // (v - mu) / sd as the correctly rounded quotient from the correctly rounded
                // reciprocal: q0 = d rc, the exact residual d - q0 sd by one fma, one fma
                // correction (Markstein), three operations in place of the division sequence
                const float d = v[i] - mu[i];
                const float q0 = d * rc[i];
                const float e = __builtin_fmaf(-q0, sd[i], d);
                const float t = __builtin_fmaf(e, rc[i], q0);
                v[i] = t < -p.clip ? -p.clip : (t > p.clip ? p.clip : t);
              }
            }
          }
          x[q] = v;
          typedef __bf16 bvec __attribute__((ext_vector_type(VW)));
          bvec b;
#pragma unroll
          for (int i = 0; i < VW; ++i) b[i] = (__bf16)v[i];
          *reinterpret_cast<bvec*>(As + r * kHPitch + VW * cv) = b;
        }
      }
    }
    for (int idx = tid; idx < kRows * (KP - D); idx += kThreads) {   // zero the K padding
      const int r = idx / (KP - D);
      As[r * kHPitch + D + (idx - r * (KP - D))] = (__bf16)0.0f;
    }
  }
  __syncthreads();

  // ---- phase 1: actor layer 1 products.  Every phase derives its lane values afresh
  // (fresh_lane): held from one phase to the next they took registers the phases need.
  f32x16 a1[2];
  int ln = fresh_lane();
  init_bias(a1, wf + kB1, u0, ln);
  {
    // the normalised rows leave for nobs_out during these products, not in the staging, where
    // every workgroup's row reads are in flight at once
    const int t = fresh_lane() + 64 * wave;
    const int cv = t % S::NC, rb = t / S::NC;
    auto store_rows = [&](int j) {
      if (!p.nobs_out || rb >= S::RP) return;
#pragma unroll
      for (int q = 0; q < S::NP; ++q) {
        const int r = rb + S::RP * q;
        if ((q * 8) / S::NP == j && r < nr)
          *reinterpret_cast<vec*>(p.nobs_out + (long)(r0 + r) * p.nobs_ld + VW * cv) = x[q];
      }
    };
    gemm_epi<2, KP>(a1, wbf + Blob<KP>::W1, u0, As, kHPitch, ln, store_rows);
  }
  // ---- phase 2: critic layer 1 products, actor layer 1 tanh -> B
  f32x16 c1[2];
  ln = fresh_lane();
  if (critic) {
    init_bias(c1, wf + kB1 + kHid, u0, ln);
    gemm_epi<2, KP>(c1, wbf + Blob<KP>::W1C, u0, As, kHPitch, ln, TanhEpi{a1, Bs, u0, ln});
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) TanhEpi{a1, Bs, u0, ln}(j);
  }
  __syncthreads();
  // ---- phase 3: actor layer 2 products, critic layer 1 tanh -> A
  f32x16 a2[2];
  ln = fresh_lane();
  init_bias(a2, wf + kB2A, u0, ln);
  if (critic)
    gemm_epi<2, kHid>(a2, wbf + Blob<KP>::W2A, u0, Bs, kHPitch, ln, TanhEpi{c1, As, u0, ln});
  else
    gemm_epi<2, kHid>(a2, wbf + Blob<KP>::W2A, u0, Bs, kHPitch, ln, [](int) {});
  __syncthreads();
  // ---- phase 4: critic layer 2 products, actor layer 2 tanh -> B
  f32x16 c2[2];
  ln = fresh_lane();
  if (critic) {
    init_bias(c2, wf + kB2C, u0, ln);
    gemm_epi<2, kHid>(c2, wbf + Blob<KP>::W2C, u0, As, kHPitch, ln, TanhEpi{a2, Bs, u0, ln});
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) TanhEpi{a2, Bs, u0, ln}(j);
  }
  __syncthreads();
  // ---- phase 5: the logits head on waves 0-5 (32 units x 32 rows each), beside the critic's
  // layer-2 tanh and its value partials (this wave's 32 units of every row)
  const int ut = wave % 3, rt = wave / 3;
  f32x16 h[1];
  ln = fresh_lane();
  float vp[2] = {0.0f, 0.0f};
  float4 w3[4];
  if (critic) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      w3[g] = *reinterpret_cast<const float4*>(wf + kW3C + u0 + 8 * g + (ln >> 5) * 4);
  }
  if (wave < 6) {
    init_bias(h, wf + kB3A, 32 * ut, ln);
    if (critic)
      gemm_epi<1, kHid>(h, wbf + Blob<KP>::W3A, 32 * ut, Bs + 32 * rt * kHPitch, kHPitch, ln,
                        ValueEpi{c2, w3, vp});
    else
      gemm_t<1, kHid>(h, wbf + Blob<KP>::W3A, 32 * ut, Bs + 32 * rt * kHPitch, kHPitch, 0, ln);
  } else if (critic) {
#pragma unroll
    for (int j = 0; j < 8; ++j) ValueEpi{c2, w3, vp}(j);
  }
  if (critic) {
#pragma unroll
    for (int r = 0; r < 2; ++r) vp[r] += __shfl_xor(vp[r], 32);   // lns l, l + 32: one row
    if (ln < 32) { vpart[wave][ln] = vp[0]; vpart[wave][32 + ln] = vp[1]; }
  }
  __syncthreads();                                    // every wave has read actor layer 2
  ln = fresh_lane();
  float* Ls = reinterpret_cast<float*>(Bs);
  if (wave < 6) {
    const int row = 32 * rt + (ln & 31);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int unit = 32 * ut + 8 * g + (ln >> 5) * 4;
      *reinterpret_cast<float4*>(Ls + row * kLPitch + unit) =
          make_float4(h[0][4 * g + 0], h[0][4 * g + 1], h[0][4 * g + 2], h[0][4 * g + 3]);
    }
  }
  __syncthreads();

  // ---- value: the eight waves' partials in order, plus the bias (wave 4, beside the draws)
  ln = fresh_lane();
  if (critic && wave == 4) {
    float v = vpart[0][ln];
#pragma unroll
    for (int q = 1; q < kWaves; ++q) v += vpart[q][ln];
    if (ln < nr) p.value[r0 + ln] = v + wf[kB3C];
  }

  // ---- per (row, channel): softmax, draw, log-probability, control (waves 0-3)
  const uint32_t step = p.step + (p.step_base ? *p.step_base : 0u);
  if (tid < kRows * kChan) {
    const int row = tid >> 2, ch = tid & 3;
    const float* l = Ls + row * kLPitch + ch * kBins;
    float lg[kBins];
#pragma unroll
    for (int k = 0; k < kBins; ++k) lg[k] = l[k];
    float m = lg[0];
#pragma unroll
    for (int k = 1; k < kBins; ++k) m = fmaxf(m, lg[k]);
    float e[kBins], s = 0.0f;
#pragma unroll
    for (int k = 0; k < kBins; ++k) { e[k] = f16rng::exp_nonpos(lg[k] - m); s += e[k]; }
    const int li = r0 + row;
    const long pr = (row < nr) ? (p.rows ? p.rows[li] : li) : 0;
    int idx = 0;
    if (!p.deterministic) {
      uint32_t c[4] = {(uint32_t)pr, step, (uint32_t)ch, p.salt};
      f16rng::philox4x32_10(c, (uint32_t)p.seed, (uint32_t)(p.seed >> 32));
      const float u = (float)(c[0] >> 8) * 0x1p-24f;
      const float target = u * s;
      // the first k with e_0 + ... + e_k > target (20 if none): the partial sums never
      // decrease (every e_k is a finite value >= 0), so it is the count of the k whose sum
      // is not above the target -- no early exit, no branch per bin
      float cum = 0.0f;
      int below = 0;
#pragma unroll
      for (int k = 0; k < kBins; ++k) {
        cum += e[k];
        below += (cum > target) ? 0 : 1;
      }
      idx = min(below, kBins - 1);
    } else {
#pragma unroll
      for (int k = kBins - 1; k >= 0; --k)         // the first bin at the maximum (0 if none)
        if (lg[k] == m) idx = k;
    }
    float lsel = lg[0];
#pragma unroll
    for (int k = 1; k < kBins; ++k)
      if (k == idx) lsel = lg[k];
    float lp = (lsel - m) - logf(s);
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
}

// ---- RunningNorm.update in two launches.
// (1) norm_partial_kernel: each block sums 128 rows per column in fp64 (four row phases of 32
//     rows, every load of a phase in flight, phases combined in a fixed order) and writes one
//     (sum, sum of squares) per column; block 0 also snapshots the running count into the
//     workspace and advances it by nrows (the merge reads the snapshot, so no block of the
//     merge can see the new count).
// (2) norm_merge_kernel: one block per column; thread t sums partials t, t + 256, ... in order
//     (all of a thread's loads in flight), then a fixed tree, then the reference's float32
//     parallel-variance merge.  Deterministic, no atomics.
constexpr int kNormCols = 256;                   // >= obs_dim
constexpr int kNormPhases = 4;
constexpr int kNormRowsPerPhase = 32;
constexpr int kNormRowsPerBlock = kNormPhases * kNormRowsPerPhase;
constexpr int kNormChunk = 32;
constexpr int kMergeThreads = 256;

__global__ __launch_bounds__(kNormCols * kNormPhases) void norm_partial_kernel(
    const float* __restrict__ obs, long ld, const int* __restrict__ rows, int nrows, int dim,
    double* __restrict__ work, float* __restrict__ count, float* __restrict__ count_snap) {
  __shared__ double ss[kNormPhases][kNormCols], sq[kNormPhases][kNormCols];
  const int c = threadIdx.x % kNormCols, ph = threadIdx.x / kNormCols;
  const int b = blockIdx.x;
  double s = 0.0, q = 0.0;
  if (c < dim) {
    const int i0 = b * kNormRowsPerBlock + ph * kNormRowsPerPhase;
#pragma unroll
    for (int k0 = 0; k0 < kNormRowsPerPhase; k0 += kNormChunk) {
      // row indices first, then every load unconditionally (rows past nrows read row nrows - 1
      // and add 0): a choice or a skip inside the load loop made the compiler wait for all
      // outstanding loads at each branch join, one load at a time
      long src[kNormChunk];
      if (rows) {
#pragma unroll
        for (int i = 0; i < kNormChunk; ++i) src[i] = rows[min(i0 + k0 + i, nrows - 1)];
      } else {
#pragma unroll
        for (int i = 0; i < kNormChunk; ++i) src[i] = min(i0 + k0 + i, nrows - 1);
      }
      float x[kNormChunk];
#pragma unroll
      for (int i = 0; i < kNormChunk; ++i) x[i] = obs[src[i] * ld + c];
#pragma unroll
      for (int i = 0; i < kNormChunk; ++i) {
        const double v = (i0 + k0 + i < nrows) ? (double)x[i] : 0.0;
        s += v;
        q += v * v;
      }
    }
  }
  ss[ph][c] = s;
  sq[ph][c] = q;
  __syncthreads();
  if (ph == 0 && c < dim) {
    double S = ss[0][c], Q = sq[0][c];
#pragma unroll
    for (int k = 1; k < kNormPhases; ++k) { S += ss[k][c]; Q += sq[k][c]; }
    work[(long)b * 2 * dim + c] = S;
    work[(long)b * 2 * dim + dim + c] = Q;
  }
  if (b == 0 && threadIdx.x == 0) {
    const float cnt = *count;
    *count_snap = cnt;
    *count = cnt + (float)nrows;
  }
}

__global__ __launch_bounds__(kMergeThreads) void norm_merge_kernel(
    const double* __restrict__ work, int nblocks, int nrows, int dim, float* __restrict__ mean,
    float* __restrict__ var, const float* __restrict__ count_snap) {
  __shared__ double ss[kMergeThreads], sq[kMergeThreads];
  const int c = blockIdx.x, t = threadIdx.x;
  double s = 0.0, q = 0.0;
  for (int b = t; b < nblocks; b += kMergeThreads) {
    s += work[(long)b * 2 * dim + c];
    q += work[(long)b * 2 * dim + dim + c];
  }
  ss[t] = s;
  sq[t] = q;
  __syncthreads();
  for (int w = kMergeThreads / 2; w > 0; w >>= 1) {
    if (t < w) { ss[t] += ss[t + w]; sq[t] += sq[t + w]; }
    __syncthreads();
  }
  if (t == 0) {
    const double mu = ss[0] / nrows;
    double v = sq[0] / nrows - mu * mu;
    v = v < 0.0 ? 0.0 : v;
    const float cnt = *count_snap;
    const float b_mean = (float)mu, b_var = (float)v, b_count = (float)nrows;
    const float delta = b_mean - mean[c];
    const float tot = cnt + b_count;
    mean[c] = mean[c] + delta * (b_count / tot);
    const float m_a = var[c] * cnt;
    const float m_b = b_var * b_count;
    const float M2 = m_a + m_b + (delta * delta) * (cnt * b_count / tot);
    var[c] = M2 / tot;
  }
}

static int norm_blocks(int nrows) { return (nrows + kNormRowsPerBlock - 1) / kNormRowsPerBlock; }

// ---- stable counting sort of items by group (one workgroup; per-thread contiguous chunks)
constexpr int kGroupThreads = 256;
constexpr int kGroupWaves = kGroupThreads / 64;

// exclusive prefix of v over the workgroup's threads (in thread order) and the total
__device__ __forceinline__ int block_exclusive_scan(int v, int* wave_sum, int& total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_sum[w] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int u = 0; u < kGroupWaves; ++u) {
    const int sw = wave_sum[u];
    before += u < w ? sw : 0;
    all += sw;
  }
  __syncthreads();                                   // wave_sum is reused by the next call
  total = all;
  return before + x - v;
}

// Three passes over blocks of kGroupItems items: (A) per-block group counts, (B) one small
// scan giving each (block, group) its output base -- groups in order, blocks in order within a
// group -- and the group offsets, (C) per-block stable scatter.  Deterministic, no atomics.
constexpr int kGroupItems = 1024;                 // items per block: 4 per thread

__device__ __forceinline__ void block_counts(const int* __restrict__ assign, int n, int ngroups,
                                             int i0, int (&c)[F16_POLICY_MAX_GROUPS], int& j0,
                                             int& j1) {
  constexpr int per = kGroupItems / kGroupThreads;
  j0 = min(n, i0 + threadIdx.x * per);
  j1 = min(n, j0 + per);
#pragma unroll
  for (int g = 0; g < F16_POLICY_MAX_GROUPS; ++g) c[g] = 0;
  for (int i = j0; i < j1; ++i) {
    const int g = assign[i];
#pragma unroll
    for (int q = 0; q < F16_POLICY_MAX_GROUPS; ++q) c[q] += (g == q && q < ngroups) ? 1 : 0;
  }
}

__global__ __launch_bounds__(kGroupThreads) void group_count_kernel(
    const int* __restrict__ assign, int n, int ngroups, int* __restrict__ counts) {
  __shared__ int wave_sum[kGroupWaves];
  int c[F16_POLICY_MAX_GROUPS], j0, j1;
  block_counts(assign, n, ngroups, blockIdx.x * kGroupItems, c, j0, j1);
  for (int g = 0; g < ngroups; ++g) {              // uniform
    int total;
    block_exclusive_scan(c[g], wave_sum, total);
    if (threadIdx.x == 0) counts[blockIdx.x * F16_POLICY_MAX_GROUPS + g] = total;
  }
}

// Exclusive scan of the counts in (group, block) order -- groups in order, blocks in order
// within a group -- written back in place as the (block, group) output bases, with the group
// offsets.  One workgroup; thread t owns a contiguous run of that order, its loads all in flight.
constexpr int kBasePer = 16;                      // (group, block) entries per thread per pass

__global__ __launch_bounds__(kGroupThreads) void group_base_kernel(
    int* __restrict__ counts, int nblocks, int ngroups, int* __restrict__ offsets) {
  __shared__ int wave_sum[kGroupWaves];
  const int total_n = nblocks * ngroups;
  int carry = 0;
  for (int base0 = 0; base0 < total_n; base0 += kGroupThreads * kBasePer) {   // uniform
    const int k0 = base0 + threadIdx.x * kBasePer;
    int v[kBasePer], sum = 0;
#pragma unroll
    for (int j = 0; j < kBasePer; ++j) {
      const int k = k0 + j, g = k / max(nblocks, 1), b = k - g * nblocks;
      v[j] = k < total_n ? counts[b * F16_POLICY_MAX_GROUPS + g] : 0;
      sum += v[j];
    }
    int total;
    int run = carry + block_exclusive_scan(sum, wave_sum, total);
#pragma unroll
    for (int j = 0; j < kBasePer; ++j) {
      const int k = k0 + j, g = k / max(nblocks, 1), b = k - g * nblocks;
      if (k < total_n) {
        if (b == 0) offsets[g] = run;
        counts[b * F16_POLICY_MAX_GROUPS + g] = run;
      }
      run += v[j];
    }
    carry += total;
  }
  if (threadIdx.x == 0) {
    if (nblocks == 0)
      for (int g = 0; g < ngroups; ++g) offsets[g] = 0;
    offsets[ngroups] = carry;
  }
}

__global__ __launch_bounds__(kGroupThreads) void group_scatter_kernel(
    const int* __restrict__ assign, int n, int ngroups, int stride, int offset,
    const int* __restrict__ bases, int* __restrict__ rows) {
  __shared__ int wave_sum[kGroupWaves];
  int c[F16_POLICY_MAX_GROUPS], j0, j1;
  block_counts(assign, n, ngroups, blockIdx.x * kGroupItems, c, j0, j1);
  int pos[F16_POLICY_MAX_GROUPS];
#pragma unroll
  for (int g = 0; g < F16_POLICY_MAX_GROUPS; ++g) {
    if (g >= ngroups) { pos[g] = 0; continue; }    // uniform
    int total;
    pos[g] = bases[blockIdx.x * F16_POLICY_MAX_GROUPS + g] + block_exclusive_scan(c[g], wave_sum, total);
  }
  for (int i = j0; i < j1; ++i) {
    const int g = assign[i];
#pragma unroll
    for (int q = 0; q < F16_POLICY_MAX_GROUPS; ++q)
      if (g == q && q < ngroups) rows[pos[q]++] = stride * i + offset;
  }
}

// Passes (B) and (C) in one launch for up to kBasedBlocks blocks: every block reads all blocks'
// counts (a few KB) and forms its own output bases -- the same sums group_base_kernel forms --
// before its scatter; block 0 also writes the group offsets.  One launch fewer per grouping.
constexpr int kBasedBlocks = kGroupThreads;

__global__ __launch_bounds__(kGroupThreads) void group_scatter_based_kernel(
    const int* __restrict__ assign, int n, int ngroups, int stride, int offset,
    const int* __restrict__ counts, int nblocks, int* __restrict__ rows,
    int* __restrict__ offsets) {
  __shared__ int cnt[F16_POLICY_MAX_GROUPS][kBasedBlocks];
  __shared__ int before[F16_POLICY_MAX_GROUPS], total[F16_POLICY_MAX_GROUPS];
  __shared__ int gbase[F16_POLICY_MAX_GROUPS];
  __shared__ int wave_sum[kGroupWaves];
  const int t = threadIdx.x;
  if (t < nblocks) {
#pragma unroll
    for (int g = 0; g < F16_POLICY_MAX_GROUPS; ++g)
      if (g < ngroups) cnt[g][t] = counts[t * F16_POLICY_MAX_GROUPS + g];
  }
  __syncthreads();
  if (t < ngroups) {                                 // thread g: its group's sums over blocks
    int bf = 0, tot = 0;
    for (int b = 0; b < nblocks; ++b) {
      const int v = cnt[t][b];
      bf += b < (int)blockIdx.x ? v : 0;
      tot += v;
    }
    before[t] = bf;
    total[t] = tot;
  }
  __syncthreads();
  if (t == 0) {                                       // groups in order
    int off = 0;
    for (int g = 0; g < ngroups; ++g) {
      gbase[g] = off + before[g];
      if (blockIdx.x == 0) offsets[g] = off;
      off += total[g];
    }
    if (blockIdx.x == 0) offsets[ngroups] = off;
  }
  __syncthreads();
  int c[F16_POLICY_MAX_GROUPS], j0, j1;
  block_counts(assign, n, ngroups, blockIdx.x * kGroupItems, c, j0, j1);
  int pos[F16_POLICY_MAX_GROUPS];
#pragma unroll
  for (int g = 0; g < F16_POLICY_MAX_GROUPS; ++g) {
    if (g >= ngroups) { pos[g] = 0; continue; }    // uniform
    int tot;
    pos[g] = gbase[g] + block_exclusive_scan(c[g], wave_sum, tot);
  }
  for (int i = j0; i < j1; ++i) {
    const int g = assign[i];
#pragma unroll
    for (int q = 0; q < F16_POLICY_MAX_GROUPS; ++q)
      if (g == q && q < ngroups) rows[pos[q]++] = stride * i + offset;
  }
}

}  // namespace f16pol

using namespace f16pol;

extern "C" long f16_group_workspace_bytes(int n) {
  if (n < 0) return -1;
  return (long)((n + kGroupItems - 1) / kGroupItems + 1) * F16_POLICY_MAX_GROUPS * (long)sizeof(int);
}

extern "C" int f16_group_rows(const int* assign, int n, int ngroups, int stride, int offset,
                              int* rows, int* group_offsets, void* work, void* stream) {
  if (n < 0 || n > (1 << 24) || ngroups < 1 || ngroups > F16_POLICY_MAX_GROUPS) return F16_EINVAL;
  if (!group_offsets || !work || (n > 0 && (!assign || !rows))) return F16_EINVAL;
  const int nb = (n + kGroupItems - 1) / kGroupItems;
  int* counts = static_cast<int*>(work);
  hipStream_t s = (hipStream_t)stream;
  if (nb > 0)
    hipLaunchKernelGGL(group_count_kernel, dim3(nb), dim3(kGroupThreads), 0, s, assign, n,
                       ngroups, counts);
  if (nb > 0 && nb <= kBasedBlocks) {               // up to 262,144 items: two launches
    hipLaunchKernelGGL(group_scatter_based_kernel, dim3(nb), dim3(kGroupThreads), 0, s, assign,
                       n, ngroups, stride, offset, counts, nb, rows, group_offsets);
    return f16_last_error();
  }
  hipLaunchKernelGGL(group_base_kernel, dim3(1), dim3(kGroupThreads), 0, s, counts, nb, ngroups,
                     group_offsets);
  if (nb > 0)
    hipLaunchKernelGGL(group_scatter_kernel, dim3(nb), dim3(kGroupThreads), 0, s, assign, n,
                       ngroups, stride, offset, counts, rows);
  return f16_last_error();
}

extern "C" int f16_policy_step(const F16PolicyArgs* a, void* stream) {
  if (!a || !a->obs || a->ngroups < 1 || a->ngroups > F16_POLICY_MAX_GROUPS) return F16_EINVAL;
  if (a->obs_dim != 184 && a->obs_dim != 214) return F16_EINVAL;
  if (a->obs_ld < a->obs_dim || !a->grid) return F16_EINVAL;
  if (a->mean && !a->var) return F16_EINVAL;
  if (a->nobs_out && a->nobs_ld < a->obs_dim) return F16_EINVAL;
  int max_rows = 0;
  for (int g = 0; g < a->ngroups; ++g) {
    const F16PolicyGroup& G = a->group[g];
    if (!G.wbf || !G.wf || ((uintptr_t)G.wbf & 15) != 0) return F16_EINVAL;
    if ((G.mean == nullptr) != (G.var == nullptr)) return F16_EINVAL;
    if (!a->group_offsets) {
      if (G.row_begin < 0 || G.row_end < G.row_begin) return F16_EINVAL;
      max_rows = max(max_rows, G.row_end - G.row_begin);
    }
  }
  if (a->group_offsets) {
    if (a->max_group_rows < 0 || a->total_group_rows < 0) return F16_EINVAL;
    max_rows = a->max_group_rows;
  } else if (a->total_group_rows != 0) {
    return F16_EINVAL;                                   // the packed grid needs device offsets
  }
  if (max_rows == 0) return 0;
  if (a->obs_ld % 2 || ((uintptr_t)a->obs & 7) || (a->nobs_out && (a->nobs_ld % 2 || ((uintptr_t)a->nobs_out & 7))))
    return F16_EINVAL;                                   // rows are moved as float2 at least
  // float4 rows where every row start is 16-byte aligned (184 columns; 214 is not a multiple of 4)
  const bool v4 = a->obs_dim == 184 && a->obs_ld % 4 == 0 && ((uintptr_t)a->obs & 15) == 0 &&
                  (!a->nobs_out || (a->nobs_ld % 4 == 0 && ((uintptr_t)a->nobs_out & 15) == 0));
  const dim3 grid = a->total_group_rows > 0
      ? dim3((unsigned)((a->total_group_rows + kRows - 1) / kRows + a->ngroups), 1u)
      : dim3((unsigned)((max_rows + kRows - 1) / kRows), (unsigned)a->ngroups);
  const dim3 block(kThreads);
  hipStream_t s = (hipStream_t)stream;
  if (a->obs_dim == 184) {
    if (v4) hipLaunchKernelGGL((policy_kernel<192, 4>), grid, block, 0, s, *a);
    else hipLaunchKernelGGL((policy_kernel<192, 2>), grid, block, 0, s, *a);
  } else {
    hipLaunchKernelGGL((policy_kernel<224, 2>), grid, block, 0, s, *a);
  }
  return f16_last_error();
}

extern "C" int f16_abi_struct_sizes(long* out, int n) {
  const long sizes[4] = {(long)sizeof(F16PolicyGroup), (long)sizeof(F16PolicyArgs),
                         (long)sizeof(F16PPOArgs), (long)sizeof(F16AdamArgs)};
  if (!out || n < 2) return F16_EINVAL;
  for (int i = 0; i < n && i < 4; ++i) out[i] = sizes[i];
  return 0;
}

extern "C" long f16_norm_workspace_bytes(int nrows, int obs_dim) {
  if (nrows < 0 || obs_dim < 0) return -1;
  return (long)norm_blocks(nrows) * 2 * obs_dim * (long)sizeof(double) + (long)sizeof(double);
}

extern "C" int f16_norm_merge(int nrows, int obs_dim, float* mean, float* var, void* work,
                              void* stream) {
  if (nrows < 0 || obs_dim < 1 || obs_dim > kNormCols) return F16_EINVAL;
  if (nrows == 0) return 0;
  if (!mean || !var || !work) return F16_EINVAL;
  const int nb = norm_blocks(nrows);
  const double* partial = static_cast<const double*>(work);
  const float* snap = reinterpret_cast<const float*>(partial + (long)nb * 2 * obs_dim);
  hipLaunchKernelGGL(norm_merge_kernel, dim3(obs_dim), dim3(kMergeThreads), 0,
                     (hipStream_t)stream, partial, nb, nrows, obs_dim, mean, var, snap);
  return f16_last_error();
}

extern "C" int f16_norm_update(const float* obs, long obs_ld, const int* rows, int nrows,
                               int obs_dim, float* mean, float* var, float* count, void* work,
                               void* stream) {
  if (nrows < 0 || obs_dim < 1 || obs_dim > kNormCols || obs_ld < obs_dim) return F16_EINVAL;
  if (nrows == 0) return 0;
  if (!obs || !mean || !var || !count || !work) return F16_EINVAL;
  const int nb = norm_blocks(nrows);
  double* partial = static_cast<double*>(work);
  float* snap = reinterpret_cast<float*>(partial + (long)nb * 2 * obs_dim);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(norm_partial_kernel, dim3(nb), dim3(kNormCols * kNormPhases), 0, s, obs,
                     obs_ld, rows, nrows, obs_dim, partial, count, snap);
  hipLaunchKernelGGL(norm_merge_kernel, dim3(obs_dim), dim3(kMergeThreads), 0, s,
                     (const double*)partial, nb, nrows, obs_dim, mean, var, snap);
  return f16_last_error();
}

// ------------------------------------------------------------------ allocation-free norm update
// f16_norm_update with its workspace in a fixed device array instead of a caller buffer, for
// callers that cannot allocate.  `scratch` is a file-scope __device__ array: the code object
// holds one copy of it on every GPU it is loaded on, kept until the process ends.  Host code
// never passes the symbol itself (on the host it names a stand-in, not device memory): the
// device address is looked up once per device with hipGetSymbolAddress and kept in
// g_scratch_dev[], and only that address reaches kernels.  Both kernels write every workspace
// value they later read (per-block partial sums of every column, the count snapshot), so the
// array needs no clearing between calls.  Calls that overlap on one GPU share the array and
// race.
constexpr long kNoAllocScratchBytes = 8l << 20;          // 8 MiB per GPU
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];   // device address of `scratch` on each device, or null

// The device address of `scratch` on the current device, looked up on the first call there.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(1000 + (int)e);
  if (dev < 0 || dev >= kMaxDevices) return F16_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return -(1000 + (int)e);
    if (!p) return F16_EINVAL;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}
}  // namespace

extern "C" long f16_norm_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int f16_norm_update_noalloc(const float* obs, long obs_ld, const int* rows, int nrows,
                                       int obs_dim, float* mean, float* var, float* count,
                                       void* stream) {
  if (nrows < 0 || obs_dim < 1 || obs_dim > kNormCols || obs_ld < obs_dim) return F16_EINVAL;
  if (nrows == 0) return 0;
  if (!obs || !mean || !var || !count) return F16_EINVAL;
  if (f16_norm_workspace_bytes(nrows, obs_dim) > kNoAllocScratchBytes) return F16_ETOOBIG;
  void* work = nullptr;
  const int rc = scratch_address(&work);
  if (rc) return rc;
  return f16_norm_update(obs, obs_ld, rows, nrows, obs_dim, mean, var, count, work, stream);
}
