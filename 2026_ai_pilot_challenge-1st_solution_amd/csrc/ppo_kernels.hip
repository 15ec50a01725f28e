// ppo_kernels.hip -- the PPO update of the discrete actor-critic MLP on gfx950.
//
// One minibatch (f16_ppo_grad) is seven launches:
//   adv_partial/final  minibatch advantage mean and sample std (shifted fp64 sums, two levels);
//   ppo_fused_kernel   per 64 gathered rows (persistent, one workgroup per CU, the next tile's
//                      rows in flight during the current one): forward of both networks, the loss head (softmax,
//                      log-probability, entropy, ratio, clipped surrogate, value error) and the
//                      backward chain down to the first hidden layer, all with the rows'
//                      activations held in LDS.  The layer inputs and output gradients every
//                      weight gradient needs leave unit-major ([feature][row], bf16), so the
//                      reduction over rows reads them as contiguous MFMA fragments;
//   wgrad_kernel       every weight gradient dW = dY^T X as one split-K launch: 256 x 256 output
//                      tiles of all four products, rows in chunks, 64-row stages double-buffered
//                      through LDS, fp32 partials per chunk (bias gradients are the row sums of
//                      dY, taken while staging);
//   colsum kernels     the partials summed in a fixed order (deterministic, no atomics): the
//                      weight-gradient chunks, then the fused kernel's per-tile rows in two
//                      levels, the second (colsum_tail_kernel) also forming the minibatch means.
// The optimizer step (f16_ppo_adam_step) is three: per-block squared-norm partials, the clipped
// Adam update (every block re-reduces the norm partials in the same order), and the repack of
// the bf16 blobs the rollout and the next minibatch read.
//
// The forward runs the same tiles, the same K order and the same epilogue as the rollout kernel
// (policy_mfma.h), and the log-probability is formed with the same expression sequence, so at
// unchanged weights the update's log-probability equals the rollout's bit for bit (ratio 1).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "f16_capi_common.h"
#include "f16_policy.h"
#include "f16_ppo.h"
#include "philox.h"
#include "policy_mfma.h"
#include "sample_math.h"

namespace f16ppo {

using namespace f16pol;

constexpr int kZPitch = kLogitsPad + 8;          // bf16 per LDS row of logit gradients
constexpr int kStatCols = 8;                     // fused-kernel partial row: 8 sums,
constexpr int kPartCols = kStatCols + kHid + 1 + 7;   // dw3c [256], db3c, pad to 272
constexpr long kWT3 = 0, kWT2A = 256L * 96, kWT2C = kWT2A + 65536;

// ---- flat parameter offsets (f16_ppo.h)
struct Flat {
  long D;
  __host__ __device__ long a_w1() const { return 0; }
  __host__ __device__ long a_b1() const { return 256 * D; }
  __host__ __device__ long a_w2() const { return 256 * D + 256; }
  __host__ __device__ long a_b2() const { return 256 * D + 65792; }
  __host__ __device__ long a_w3() const { return 256 * D + 66048; }
  __host__ __device__ long a_b3() const { return 256 * D + 87552; }
  __host__ __device__ long na() const { return 256 * D + 87636; }
  __host__ __device__ long c_w1() const { return na(); }
  __host__ __device__ long c_b1() const { return na() + 256 * D; }
  __host__ __device__ long c_w2() const { return na() + 256 * D + 256; }
  __host__ __device__ long c_b2() const { return na() + 256 * D + 65792; }
  __host__ __device__ long c_w3() const { return na() + 256 * D + 66048; }
  __host__ __device__ long c_b3() const { return na() + 256 * D + 66304; }
  __host__ __device__ long n() const { return na() + 256 * D + 66305; }
};

// ---- workspace layout; the fixed-size parts come first, so the optimizer's scratch does not
// move with the minibatch size
constexpr int kAdvThreads = 256;
constexpr int kAdvPer = 8;                       // rows per thread of the advantage partials
constexpr int kNormBlockElems = 4096;            // flat elements per squared-norm block
constexpr int kWgradSlots = 256;                 // resident wgrad workgroups when the device
                                                 // cannot be asked (1 per CU x 256 CUs)
constexpr int kMaxChunks = 64;                   // bound on the chunks the partials hold

__host__ __device__ inline long align256(long x) { return (x + 255) & ~255L; }

struct Work {
  float* advs;          // [8]: mean, std, statistics sums
  double* normp;        // [nblk][2] squared-norm partials
  __bf16 *xt, *h1t, *h2t, *dh1t, *dh2t, *dzt;   // unit-major in 64-row blocks (ublock); features
                                                // kp, 512, 256, 512, 512, kLogitsPad
                                                // (h2t: the actor's layer 2; the critic's
                                                // enters only the value head, summed in-kernel)
  float* fpart;         // [nwg][kPartCols]
  double* advp;         // [nadv][2] advantage partial sums
  float* fmid;          // [ceil(nwg / kColRows)][kPartCols] first level of the fpart sums
  float* wpart;         // [nchunk][nflat - 257]
  long ld;              // rows, rounded up to 64
  int nwg, nchunk, chunk_rows, nadv;
  long bytes;
};

// The unit-major buffers are stored in 64-row blocks: feature f of row m of a buffer of NF
// features at (m / 64) NF 64 + 64 f + m % 64, so each tile's output for one buffer is one
// contiguous NF x 128-byte run and a weight-gradient stage (256 features x 64 rows) is one
// contiguous 32 KB read, where a [feature][row] layout over the whole minibatch made every
// 128-byte row segment its own DRAM page.  Within a block the feature stride is 64 elements.
constexpr long kUBlock = 64;
__host__ __device__ inline __bf16* ublock(__bf16* buf, long nf, long m0) {
  return buf + (m0 / kUBlock) * nf * kUBlock;
}

constexpr int kColRows = 64;                     // rows per block of the two-level column sum
inline long kColGroups(long nrows) { return (nrows + kColRows - 1) / kColRows; }

inline int norm_blocks(long n) { return (int)((n + kNormBlockElems - 1) / kNormBlockElems); }

inline int wgrad_tiles(int kp) { return 2 * ((kp + 255) / 256) + 1 + 1 + 1; }

inline Work layout(int obs_dim, long mb_rows, void* base, int wg_slots = kWgradSlots) {
  Work w{};
  const int kp = (obs_dim + 31) / 32 * 32;
  const Flat F{obs_dim};
  w.ld = (mb_rows + 63) / 64 * 64;
  w.nwg = (int)(w.ld / 64);
  const int tiles = wgrad_tiles(kp);
  // chunks of 64-row stages: one workgroup per resident slot (a grid a little above a
  // multiple of the slots leaves a mostly idle last round), at least 4 stages each
  long chunks = std::max(1, std::min(wg_slots / tiles, kMaxChunks));
  long cr = (w.ld + chunks - 1) / chunks;
  cr = (cr + 63) / 64 * 64;
  if (cr < 256) cr = 256;
  w.chunk_rows = (int)cr;
  w.nchunk = (int)((w.ld + cr - 1) / cr);
  // partial rows are allocated for min(ceil(ld / 256), kMaxChunks) chunks: never fewer than
  // nchunk (cr >= 256, nchunk <= chunks) and non-decreasing in ld, so a workspace sized for a
  // minibatch serves every smaller one
  const long cap = std::min((w.ld + 255) / 256, (long)kMaxChunks);
  char* p = static_cast<char*>(base);
  long off = 0;
  auto take = [&](long bytes) { char* q = p ? p + off : nullptr; off += align256(bytes); return q; };
  w.advs = reinterpret_cast<float*>(take(64));
  w.normp = reinterpret_cast<double*>(take((long)norm_blocks(F.n()) * 2 * sizeof(double)));
  w.xt = reinterpret_cast<__bf16*>(take((long)kp * w.ld * 2));
  w.h1t = reinterpret_cast<__bf16*>(take(512L * w.ld * 2));
  w.h2t = reinterpret_cast<__bf16*>(take(256L * w.ld * 2));   // actor layer 2 only
  w.dh1t = reinterpret_cast<__bf16*>(take(512L * w.ld * 2));
  w.dh2t = reinterpret_cast<__bf16*>(take(512L * w.ld * 2));
  w.dzt = reinterpret_cast<__bf16*>(take((long)kLogitsPad * w.ld * 2));
  w.fpart = reinterpret_cast<float*>(take((long)w.nwg * kPartCols * 4));
  w.nadv = (int)((w.ld + kAdvThreads * kAdvPer - 1) / (kAdvThreads * kAdvPer));
  w.advp = reinterpret_cast<double*>(take((long)w.nadv * 2 * sizeof(double)));
  w.fmid = reinterpret_cast<float*>(take((long)kColGroups(w.nwg) * kPartCols * 4));
  w.wpart = reinterpret_cast<float*>(take(cap * (F.n() - 257) * 4));
  w.bytes = off;
  return w;
}

// ---- minibatch advantage mean and sample standard deviation (ppo_gpu.py:2077-2078): each block
// sums (x - K) and (x - K)^2 in fp64 over its rows, K the minibatch's first advantage (shifting
// keeps the one-pass variance exact to fp64 rounding for any mean); one block merges the partials
// in a fixed order.
__device__ __forceinline__ void adv_partial_body(const float* __restrict__ adv,
                                                 const long long* __restrict__ idx, int n,
                                                 long count, double* __restrict__ part, int blk) {
  __shared__ double rs[kAdvThreads], rq[kAdvThreads];
  const int t = threadIdx.x;
  const long long p0 = idx[0];
  const double K = (p0 >= 0 && p0 < count) ? (double)adv[p0] : 0.0;
  double s = 0.0, q = 0.0;
  const int i = blk * kAdvThreads * kAdvPer + t;
  // every index load, then every value load, unconditionally (out-of-range items read element
  // 0 and are not summed): loads chosen or skipped inside the summing loop were issued one at a
  // time, each waiting out the previous ones
  long long p[kAdvPer];
#pragma unroll
  for (int k = 0; k < kAdvPer; ++k) p[k] = idx[min(i + k * kAdvThreads, n - 1)];
  if (count > 0) {
    float v[kAdvPer];
#pragma unroll
    for (int k = 0; k < kAdvPer; ++k) v[k] = adv[(p[k] >= 0 && p[k] < count) ? p[k] : 0];
#pragma unroll
    for (int k = 0; k < kAdvPer; ++k) {
      if (i + k * kAdvThreads < n && p[k] >= 0 && p[k] < count) {
        const double d = (double)v[k] - K;
        s += d;
        q += d * d;
      }
    }
  }
  rs[t] = s;
  rq[t] = q;
  __syncthreads();
  for (int w = kAdvThreads / 2; w > 0; w >>= 1) {
    if (t < w) { rs[t] += rs[t + w]; rq[t] += rq[t + w]; }
    __syncthreads();
  }
  if (t == 0) { part[2L * blk] = rs[0]; part[2L * blk + 1] = rq[0]; }
}

__global__ __launch_bounds__(kAdvThreads) void adv_partial_kernel(const float* __restrict__ adv,
                                                                  const long long* __restrict__ idx,
                                                                  int n, long count,
                                                                  double* __restrict__ part) {
  adv_partial_body(adv, idx, n, count, part, blockIdx.x);
}

__device__ __forceinline__ void adv_final_body(const float* __restrict__ adv,
                                               const long long* __restrict__ idx, int n,
                                               long count, int nblk,
                                               const double* __restrict__ part, float* advs) {
  __shared__ double rs[kAdvThreads], rq[kAdvThreads];
  const int t = threadIdx.x;
  double s = 0.0, q = 0.0;
  for (int b = t; b < nblk; b += kAdvThreads) { s += part[2L * b]; q += part[2L * b + 1]; }
  rs[t] = s;
  rq[t] = q;
  __syncthreads();
  for (int w = kAdvThreads / 2; w > 0; w >>= 1) {
    if (t < w) { rs[t] += rs[t + w]; rq[t] += rq[t + w]; }
    __syncthreads();
  }
  if (t == 0) {
    const long long p0 = idx[0];
    const double K = (p0 >= 0 && p0 < count) ? (double)adv[p0] : 0.0;
    const double ms = rs[0] / n;                       // mean of the shifted values
    double var = n > 1 ? (rq[0] - rs[0] * ms) / (n - 1) : 0.0;
    var = var < 0.0 ? 0.0 : var;
    advs[0] = (float)(K + ms);
    advs[1] = (float)sqrt(var);
  }
}

__global__ __launch_bounds__(kAdvThreads) void adv_final_kernel(const float* __restrict__ adv,
                                                                const long long* __restrict__ idx,
                                                                int n, long count, int nblk,
                                                                const double* __restrict__ part,
                                                                float* advs) {
  adv_final_body(adv, idx, n, count, nblk, part, advs);
}

// The same for every minibatch of an epoch at once: minibatch j (blockIdx.y, then blockIdx.x of
// the final level) is idx[j mb, min((j + 1) mb, total)), its partials at part + 2 nadv j and its
// mean and std at out[2j], out[2j + 1] -- the values f16_ppo_grad forms for that minibatch alone.
__global__ __launch_bounds__(kAdvThreads) void adv_partial_epoch_kernel(
    const float* __restrict__ adv, const long long* __restrict__ idx, int mb, long total,
    long count, int nadv, double* __restrict__ part) {
  const long s0 = (long)blockIdx.y * mb;
  adv_partial_body(adv, idx + s0, (int)min((long)mb, total - s0), count,
                   part + 2L * nadv * blockIdx.y, blockIdx.x);
}

__global__ __launch_bounds__(kAdvThreads) void adv_final_epoch_kernel(
    const float* __restrict__ adv, const long long* __restrict__ idx, int mb, long total,
    long count, int nadv, const double* __restrict__ part, float* __restrict__ out) {
  const long s0 = (long)blockIdx.x * mb;
  adv_final_body(adv, idx + s0, (int)min((long)mb, total - s0), count, nadv,
                 part + 2L * nadv * blockIdx.x, out + 2L * blockIdx.x);
}

// ---- fused forward / loss / backward of 64 gathered rows

// ---- cross-lane data movement by DPP (vector instructions, no LDS round trip)
constexpr int kDppXor1 = 0xB1;          // quad_perm [1, 0, 3, 2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;          // quad_perm [2, 3, 0, 1]: lane ^ 2
constexpr int kDppRor4 = 0x124;         // row_ror:4 within 16 lanes
constexpr int kDppRor8 = 0x128;         // row_ror:8
constexpr int kDppHalfMirror = 0x141;   // lane i <- lane 7 - i within 8 lanes (lane ^ 7)
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, true));
}
// Sum over the 32 lanes of a half-wave (lanes 0-31 and 32-63 separately), every lane getting
// the sum: quad swaps and row rotations, then one exchange across the 16-lane rows.  The fixed
// pattern fixes the summation order.
__device__ __forceinline__ float sum32(float x) {
  x += dpp<kDppXor1>(x);
  x += dpp<kDppXor2>(x);
  x += dpp<kDppRor4>(x);
  x += dpp<kDppRor8>(x);
  return x + __shfl_xor(x, 16);
}
// the same over all 64 lanes
__device__ __forceinline__ float sum64(float x) {
  x = sum32(x);
  return x + __shfl_xor(x, 32);
}

constexpr int kBufWord3 = 0x00020000;   // gfx9 buffer descriptor word 3 (raw, 32-bit data format)
constexpr int kMaxMinibatchRows = 1 << 24;

// LDS [row][pitch] bf16 tile of 64 rows x NF features (NF a multiple of 32) -> unit-major global
// dst[f][m0 + row], transposed by the matrix cores: D = A I over two 16-wide K slices, A the
// tile's rows read as the usual activation operand (16-byte, bank-conflict-free) and I the
// identity split over the slices, so result lane l holds feature l % 32 of rows
// 32r + 8g + 4(l / 32) + 0..3 -- one 8-byte store per 4 rows.  Exact: each output is one
// product x * 1 plus zero products.  Blocks of 32 features x 32 rows go round the waves.
template <int NF>
__device__ __forceinline__ void transpose_t(const __bf16* S, int pitch, __bf16* dst, long ld,
                                            long m0, int wave, int lane) {
  const int lr = lane & 31, kb = (lane >> 5) * 8;
  bf16x8 i0, i1;                                  // identity fragments of the two K slices
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    i0[t] = (__bf16)(kb + t == lr ? 1.0f : 0.0f);
    i1[t] = (__bf16)(kb + t + 16 == lr ? 1.0f : 0.0f);
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(dst + m0, 0, 0x7fffffff, kBufWord3);
  const int lo = 2 * (lr * (int)ld + (lane >> 5) * 4);
  for (int blk = wave; blk < (NF / 32) * 2; blk += kWaves) {
    const int fb = blk >> 1, r = blk & 1;
    const __bf16* ap = S + (32 * r + lr) * pitch + 32 * fb + kb;
    const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(ap);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(ap + 16);
    f32x16 acc = {};
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, i0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, i1, acc, 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (__bf16)acc[4 * g + e];
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), rs,
                                            lo + 2 * (32 * r + 8 * g), 2 * 32 * fb * (int)ld, 0);
    }
  }
}

// Unit-major stores of a 32-unit x 64-row block (unit u0 + 8g + lh + j, row 32r + lr) as buffer
// stores: the block's origin dst + u0 ld + m0 is the (wave-uniform) buffer base, the (g, j)
// offset 2 (8g + j) ld the scalar offset and the lane's 2 (lh ld + lr) + 64 r the vector
// offset, so a store needs no vector address arithmetic.  The buffer's window is 2 GB from the
// base (offsets below 72 ld bytes occur; the kernels pass a 64-row block with ld = 64); u0 must
// be wave-uniform.
struct UnitMajor {
  __amdgpu_buffer_rsrc_t rsrc;
  int ld2;              // bytes between consecutive features
  int lane_off;         // 2 (lh ld + lr)
  __device__ __forceinline__ UnitMajor(__bf16* dst, long ld, long m0, int u0, int lane)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(dst + (long)u0 * ld + m0, 0, 0x7fffffff,
                                               kBufWord3)),
        ld2(2 * (int)ld), lane_off(2 * ((lane >> 5) * 4 * (int)ld + (lane & 31))) {}
  __device__ __forceinline__ void put(int g, int r, int j, __bf16 v) const {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), rsrc,
                                          lane_off + 64 * r, (8 * g + j) * ld2, 0);
  }
};

// tanh epilogue: bf16 activation to LDS Hs[row][unit] and to unit-major dst[unit][m0 + row]
template <int NR>
__device__ __forceinline__ void store_tanh_t(const f32x16 (&acc)[NR], __bf16* Hs, int u0,
                                             __bf16* dst, long ld, long m0, int lane) {
  const int lr = lane & 31, lh = (lane >> 5) * 4;
  const UnitMajor out(dst, ld, m0, u0, lane);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int unit = u0 + 8 * g + lh;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      bf16x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (__bf16)tanh_act(acc[r][4 * g + j]);
      const int row = 32 * r + lr;
      *reinterpret_cast<bf16x4*>(Hs + row * kHPitch + unit) = v;
#pragma unroll
      for (int j = 0; j < 4; ++j) out.put(g, r, j, v[j]);
    }
  }
}

// backward epilogue: d = acc * (1 - h^2) with h the layer's bf16 activation at Hs[row][unit];
// rounded to bf16, to unit-major dst and, when Out is non-null, to Out[row][unit]
template <int NR>
__device__ __forceinline__ void store_dtanh_t(const f32x16 (&acc)[NR], const __bf16* Hs,
                                              __bf16* Out, int u0, __bf16* dst, long ld, long m0,
                                              int lane) {
  const int lr = lane & 31, lh = (lane >> 5) * 4;
  const UnitMajor out(dst, ld, m0, u0, lane);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int unit = u0 + 8 * g + lh;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int row = 32 * r + lr;
      const bf16x4 h = *reinterpret_cast<const bf16x4*>(Hs + row * kHPitch + unit);
      bf16x4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float hv = (float)h[j];
        v[j] = (__bf16)(acc[r][4 * g + j] * (1.0f - hv * hv));
      }
      if (Out) *reinterpret_cast<bf16x4*>(Out + row * kHPitch + unit) = v;
#pragma unroll
      for (int j = 0; j < 4; ++j) out.put(g, r, j, v[j]);
    }
  }
}

// A product's first weight fragments, loaded before the previous phase's epilogue.  vmcnt
// retires loads and stores in issue order, so a weight load issued after that epilogue's global
// stores could only be waited for behind all of them; these are issued ahead of the stores.
template <int K>
struct WPre {
  static constexpr int PF = K / 16 < 4 ? K / 16 : 4;
  bf16x8 w[PF];
};
template <int K>
__device__ __forceinline__ void wprefetch(WPre<K>& p, const __bf16* __restrict__ Wg, int u0,
                                          int lane) {
  const __bf16* wp = Wg + (long)(u0 >> 5) * (K / 16) * 512 + lane * 8;
#pragma unroll
  for (int q = 0; q < WPre<K>::PF; ++q) p.w[q] = *reinterpret_cast<const bf16x8*>(wp + 512 * q);
  __builtin_amdgcn_sched_barrier(0);     // issued here, not sunk towards the product
}
// init_bias from the biases staged in LDS (global loads there would wait behind the previous
// epilogue's stores as well): element e of a tile is unit u0 + 8(e/4) + 4(lane/32) + e%4
template <int NR>
__device__ __forceinline__ void init_bias_lds(f32x16 (&acc)[NR], const float* bias, int u0,
                                              int lane) {
  const int lh = (lane >> 5) * 4;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 b = *reinterpret_cast<const float4*>(bias + u0 + 8 * g + lh);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      acc[r][4 * g + 0] = b.x;
      acc[r][4 * g + 1] = b.y;
      acc[r][4 * g + 2] = b.z;
      acc[r][4 * g + 3] = b.w;
    }
  }
}

// gemm_t's product (the same slices in the same order, so the same sums) with the first
// fragments taken from p; the rest stream PF slices ahead.
template <int NR, int K>
__device__ __forceinline__ void gemm_p(f32x16 (&acc)[NR], const WPre<K>& p,
                                       const __bf16* __restrict__ Wg, int u0,
                                       const __bf16* __restrict__ As, int a_pitch, int lane) {
  constexpr int NK = K / 16, PF = WPre<K>::PF;
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  const __bf16* wp = Wg + (long)(u0 >> 5) * (K / 16) * 512 + lane * 8;
  const __bf16* ap = As + lr * a_pitch + lk;
  bf16x8 w[PF + 1];
#pragma unroll
  for (int q = 0; q < PF; ++q) w[q] = p.w[q];
  bf16x8 a[NR], an[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) a[r] = *reinterpret_cast<const bf16x8*>(ap + 32 * r * a_pitch);
#pragma unroll
  for (int s = 0; s < NK; ++s) {
    if (s + PF < NK) w[(s + PF) % (PF + 1)] =
        *reinterpret_cast<const bf16x8*>(wp + 512 * (s + PF));
    if (s + 1 < NK) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
        an[r] = *reinterpret_cast<const bf16x8*>(ap + 32 * r * a_pitch + 16 * (s + 1));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = mfma(w[s % (PF + 1)], a[r], acc[r]);
#pragma unroll
    for (int r = 0; r < NR; ++r) a[r] = an[r];
  }
}

template <int NR>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[NR]) {
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[r][e] = 0.0f;
}

// rows of tile t: threads < 64 read the minibatch indices (idx_load; kNoRow past the
// minibatch), then idx_store puts them into rowpN (-1: past the minibatch or a bad index, which
// is counted in badN and not read).  Split so that the load is waited for well after its issue.
constexpr long long kNoRow = -(1LL << 62);
__device__ __forceinline__ long long idx_load(const F16PPOArgs& a, int t, int tid) {
  long long p = kNoRow;
  const long r = (long)t * kRows + tid;
  if (tid < kRows && r < a.mb_rows) p = a.idx[r];
  return p;
}
__device__ __forceinline__ void idx_store(const F16PPOArgs& a, long long p, long long* rowpN,
                                          float* badN, int tid) {
  if (tid < kRows) {
    float bad = 0.0f;
    if (p == kNoRow) {
      p = -1;
    } else if (p < 0 || p >= a.count) {
      bad = 1.0f;
      p = -1;
    }
    rowpN[tid] = p;
    badN[tid] = bad;
  }
}

// the rows listed in rowpN as float2 pairs, every load in flight at once
template <int D, int kPer>
__device__ __forceinline__ void issue_rows(const F16PPOArgs& a, const long long* rowpN,
                                           float2 (&xr)[kPer], int tid) {
  constexpr int half = D / 2;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int it = tid + q * kThreads;
    const int r = it / half, c = it - r * half;
    xr[q] = make_float2(0.0f, 0.0f);
    if (r < kRows && rowpN[r] >= 0)
      xr[q] = *reinterpret_cast<const float2*>(a.obs + rowpN[r] * a.obs_ld + 2 * c);
  }
}

// The loss head's per-row inputs for thread tid of the rows listed in rp: the drawn bin of its
// (row, channel) item (two lanes per item), the row's collection log-probability and advantage,
// and for tid < 64 the return of row tid.  Rows with rp < 0 give act -1 and zeros.
struct HeadIn {
  long long act;
  float old_lp, adv, ret;
};
__device__ __forceinline__ HeadIn gather_head(const F16PPOArgs& a, const long long* rp, int tid) {
  HeadIn h{-1, 0.0f, 0.0f, 0.0f};
  const int lrow = tid >> 3, lch = (tid >> 1) & 3;
  const long long pr = rp[lrow];
  if (pr >= 0) {
    h.act = a.act[pr * kChan + lch];
    h.old_lp = a.old_logp[pr];
    h.adv = a.adv[pr];
  }
  if (tid < kRows && rp[tid] >= 0) h.ret = a.ret[rp[tid]];
  return h;
}

// The fused kernel is persistent: one workgroup per CU walks the minibatch's 64-row tiles, and
// the next tile's gathered rows and loss-head inputs are loaded into registers during the
// current tile's loss head, landing while it computes.
template <int KP>
__global__ __launch_bounds__(kThreads, 1) void ppo_fused_kernel(const F16PPOArgs a, const Work w) {
  constexpr int XP = KP + 8;
  constexpr int D = KP == 192 ? 184 : 214;
  constexpr int half = D / 2;                             // float2 per observation row
  constexpr int kPer = (kRows * half + kThreads - 1) / kThreads;
  __shared__ __align__(16) __bf16 Xs[kRows * XP];
  __shared__ __align__(16) __bf16 H1s[kRows * kHPitch];
  __shared__ __align__(16) __bf16 H2s[kRows * kHPitch];
  __shared__ __align__(16) float Ls[kRows * kLPitch];     // logits, then (bf16) their gradients
  __shared__ float rowf[kRows][8];
  __shared__ float vpart[kWaves][kRows];                  // per-wave partial critic values
  __shared__ long long rowp[kRows], rowpN[kRows];
  __shared__ __align__(16) float cst[kB3C];               // biases and the value head, wf[0, kB3C)
  __shared__ float badN[kRows];
  __bf16* Zs = reinterpret_cast<__bf16*>(Ls);
  static_assert(kRows * kZPitch * 2 <= kRows * kLPitch * 4, "logit gradients overlay the logits");

  const long ld = w.ld;
  const __bf16* wbf = static_cast<const __bf16*>(a.wbf);
  const __bf16* wT = static_cast<const __bf16*>(a.wT);
  const float* wf = a.wf;
  const float inv_mb = 1.0f / (float)a.mb_rows;
  // launch constants read once (scalar loads before any store of this kernel)
  const float* const am = a.adv_stats ? a.adv_stats : w.advs;
  const float adv_mean = am[0], adv_std = am[1], b3c = wf[kB3C];
  for (int i = threadIdx.x; i < kB3C / 4; i += kThreads)
    reinterpret_cast<float4*>(cst)[i] = reinterpret_cast<const float4*>(wf)[i];
  const float* w3s = cst + kW3C;

  float2 xr[kPer];
  int tile = blockIdx.x;
  if (tile >= w.nwg) return;                               // uniform per workgroup
  idx_store(a, idx_load(a, tile, (int)threadIdx.x), rowpN, badN, (int)threadIdx.x);
  __syncthreads();
  issue_rows<D, kPer>(a, rowpN, xr, (int)threadIdx.x);
  HeadIn hnext = gather_head(a, rowpN, (int)threadIdx.x);
  WPre<KP> pa1;
  wprefetch(pa1, wbf + Blob<KP>::W1, 32 * __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6),
            (int)threadIdx.x & 63);
  // every load above has landed before the loop, so the loop's own waits for the gathered rows
  // count only the previous tile's loads (they retire by its last product's final wait)
  __builtin_amdgcn_s_waitcnt(0x0F70);                     // vmcnt(0)
  for (; tile < w.nwg; tile += gridDim.x) {
    // the thread index passes through an empty asm each tile, so the per-lane addresses below are
    // formed inside the loop rather than hoisted out of it and held live (they would spill)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31, lh = (lane >> 5) * 4;
    const long m0 = (long)tile * kRows;
    // ---- stage this tile's rows (normalised at collection), rounded to bf16
    if (tid < kRows) { rowp[tid] = rowpN[tid]; rowf[tid][7] = badN[tid]; }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int it = tid + q * kThreads;
      const int r = it / half, c = it - r * half;
      if (r < kRows) {
        bf16x2 b;
        b[0] = (__bf16)xr[q].x;
        b[1] = (__bf16)xr[q].y;
        *reinterpret_cast<bf16x2*>(Xs + r * XP + 2 * c) = b;
      }
    }
    for (int it = tid; it < kRows * (KP - D); it += kThreads) {
      const int r = it / (KP - D);
      Xs[r * XP + D + (it - r * (KP - D))] = (__bf16)0.0f;
    }
    __syncthreads();
    const int next = tile + gridDim.x;
    const long long pnext = next < w.nwg ? idx_load(a, next, tid) : kNoRow;
    // the loss head's per-row inputs, gathered during the previous tile
    const int item = tid >> 1, hb = tid & 1;           // (row, channel) item, bin half
    const int lrow = item >> 2, lch = item & 3;
    const HeadIn hin = hnext;
    transpose_t<KP>(Xs, XP, ublock(w.xt, KP, m0), kUBlock, 0, wave, lane);

    // ---- actor forward
    WPre<kHid> pa2, pl3;
    {
      f32x16 acc[2];
      init_bias_lds(acc, cst + kB1, 32 * wave, lane);
      gemm_p<2, KP>(acc, pa1, wbf + Blob<KP>::W1, 32 * wave, Xs, XP, lane);
      wprefetch(pa2, wbf + Blob<KP>::W2A, 32 * wave, lane);
      store_tanh_t(acc, H1s, 32 * wave, ublock(w.h1t, 2 * kHid, m0), kUBlock, 0, lane);
    }
    __syncthreads();
    {
      f32x16 acc[2];
      init_bias_lds(acc, cst + kB2A, 32 * wave, lane);
      gemm_p<2, kHid>(acc, pa2, wbf + Blob<KP>::W2A, 32 * wave, H1s, kHPitch, lane);
      if (wave < 6) wprefetch(pl3, wbf + Blob<KP>::W3A, 32 * (wave % 3), lane);
      store_tanh_t(acc, H2s, 32 * wave, ublock(w.h2t, kHid, m0), kUBlock, 0, lane);
      idx_store(a, pnext, rowpN, badN, tid);     // the next tile's rows, read after the barrier
    }
    __syncthreads();
    if (wave < 6) {
      const int ut = wave % 3, rt = wave / 3;
      f32x16 acc[1];
      init_bias_lds(acc, cst + kB3A, 32 * ut, lane);
      gemm_p<1, kHid>(acc, pl3, wbf + Blob<KP>::W3A, 32 * ut, H2s + 32 * rt * kHPitch, kHPitch,
                      lane);
      const int row = 32 * rt + lr;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int unit = 32 * ut + 8 * g + lh;
        *reinterpret_cast<float4*>(Ls + row * kLPitch + unit) =
            make_float4(acc[0][4 * g + 0], acc[0][4 * g + 1], acc[0][4 * g + 2], acc[0][4 * g + 3]);
      }
    }
    __syncthreads();

    // ---- loss head (ppo_gpu.py:2065-2090; model.py:207-219).
    // The next tile's rows are gathered from here on, landing while this tile computes.
    // Two lanes per (row, channel) -- lanes 2i, 2i + 1 take bins 0-10 and 11-20 -- so all eight
    // waves share the head.  The maximum (exact, order-free), the numerator sum in the rollout's
    // order (the high half continues from the low half's partial), the chosen bin's
    // log-probability and the channel sum are the rollout kernel's values bit for bit.
    const int k0 = hb ? 11 : 0;                        // this lane's bins: k0 .. k0 + nb - 1
    constexpr int kHalf = 11;
    const int nb = hb ? kBins - kHalf : kHalf;
    const long long act = hin.act;
    const float old_lp = hin.old_lp, adv_r = hin.adv, ret_r = hin.ret;
    if (next < w.nwg) {
      issue_rows<D, kPer>(a, rowpN, xr, tid);
      hnext = gather_head(a, rowpN, tid);
    }
    float dz[kHalf];
    {
      const long long pr = rowp[lrow];
      const bool valid = pr >= 0;
      const float* l = Ls + lrow * kLPitch + lch * kBins + k0;
      float lg[kHalf];
#pragma unroll
      for (int k = 0; k < kHalf; ++k) lg[k] = k < nb ? l[k] : l[0];
      float m = lg[0];
#pragma unroll
      for (int k = 1; k < kHalf; ++k) m = fmaxf(m, lg[k]);
      m = fmaxf(m, dpp<kDppXor1>(m));                 // the rollout's maximum (max is exact)
      float e[kHalf], sp = 0.0f;
#pragma unroll
      for (int k = 0; k < kHalf; ++k) {
        e[k] = k < nb ? f16rng::exp_nonpos(lg[k] - m) : 0.0f;
        if (hb == 0) sp += e[k];                      // the low half's sum, bins in order
      }
      float s = dpp<kDppXor1>(sp);                    // the high lane receives it and continues
#pragma unroll
      for (int k = 0; k < kHalf; ++k)
        if (k < nb) s += e[k];
      const float s_hi = dpp<kDppXor1>(s);            // every lane takes part in the exchange
      s = hb ? s : s_hi;                              // (the low lane's value above is unused)
      const float lse = logf(s), inv_s = 1.0f / s;
      float lp = 0.0f, hc = 0.0f;
      bool mine = false;
#pragma unroll
      for (int k = 0; k < kHalf; ++k) {
        const float lpk = (lg[k] - m) - lse;
        if (k < nb && k0 + k == act) { lp = lpk; mine = true; }
        if (k < nb) hc -= (e[k] * inv_s) * lpk;
      }
      const float lpo = dpp<kDppXor1>(lp);
      lp = mine ? lp : lpo;
      hc += dpp<kDppXor1>(hc);
      // channels (lane bits 1-2; both lanes of an item hold the same value): c + (c ^ 1), then
      // plus the partner pair's sum -- lane ^ 7 holds (c ^ 3) + (c ^ 2) -- which equals the
      // rollout kernel's (c + (c ^ 1)) + ((c ^ 2) + (c ^ 3)) bit for bit (commutative adds)
      lp += dpp<kDppXor2>(lp);
      lp += dpp<kDppHalfMirror>(lp);
      float ent = hc + dpp<kDppXor2>(hc);
      ent += dpp<kDppHalfMirror>(ent);
      float gcoef = 0.0f, pl = 0.0f, kl = 0.0f, cf = 0.0f;
      if (valid) {
        const float logr = lp - old_lp;
        const float ratio = expf(logr);
        float A = adv_r;
        if (a.norm_adv && a.mb_rows > 1) A = (A - adv_mean) / (adv_std + 1e-8f);
        const float lo = (float)(1.0 - (double)a.clip_coef), hi = (float)(1.0 + (double)a.clip_coef);
        const float rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
        const float pg1 = -A * ratio, pg2 = -A * rc;
        const float inr = (ratio >= lo && ratio <= hi) ? 1.0f : 0.0f;
        // d max(pg1, pg2) / d ratio; torch.max of two tensors shares a tie evenly
        float dr;
        if (pg1 > pg2) dr = -A;
        else if (pg1 < pg2) dr = -A * inr;
        else dr = 0.5f * -A + 0.5f * (-A * inr);
        gcoef = dr * ratio * inv_mb;
        pl = pg1 > pg2 ? pg1 : pg2;
        kl = (ratio - 1.0f) - logr;
        cf = fabsf(ratio - 1.0f) > a.clip_coef ? 1.0f : 0.0f;
      }
      const float ec = a.ent_coef * inv_mb;
#pragma unroll
      for (int k = 0; k < kHalf; ++k) {
        const float pk = e[k] * inv_s;
        const float lpk = (lg[k] - m) - lse;
        const float oh = k0 + k == act ? 1.0f : 0.0f;
        dz[k] = valid ? gcoef * (oh - pk) + ec * pk * (lpk + hc) : 0.0f;
      }
      if (lch == 0 && hb == 0) {
        rowf[lrow][0] = pl;
        rowf[lrow][1] = valid ? ent : 0.0f;
        rowf[lrow][2] = kl;
        rowf[lrow][3] = cf;
      }
    }
    __syncthreads();                          // every logit is read
#pragma unroll
    for (int k = 0; k < kHalf; ++k)
      if (k < nb) Zs[lrow * kZPitch + lch * kBins + k0 + k] = (__bf16)dz[k];
    if (lch == 3 && hb == 1) {
#pragma unroll
      for (int k = kLogits; k < kLogitsPad; ++k) Zs[lrow * kZPitch + k] = (__bf16)0.0f;
    }
    __syncthreads();
    WPre<kLogitsPad> pb3;
    wprefetch(pb3, wT + kWT3, 32 * wave, lane);
    transpose_t<kLogitsPad>(Zs, kZPitch, ublock(w.dzt, kLogitsPad, m0), kUBlock, 0, wave, lane);

    // ---- actor backward: dH2 = (dZ W3) (1 - H2^2) in place of H2, dH1 = (dH2 W2) (1 - H1^2)
    WPre<kHid> pb2, pbc, pc2;
    WPre<KP> pc1;
    {
      f32x16 acc[2];
      zero_acc(acc);
      gemm_p<2, kLogitsPad>(acc, pb3, wT + kWT3, 32 * wave, Zs, kZPitch, lane);
      wprefetch(pb2, wT + kWT2A, 32 * wave, lane);
      store_dtanh_t(acc, H2s, H2s, 32 * wave, ublock(w.dh2t, 2 * kHid, m0), kUBlock, 0, lane);
    }
    __syncthreads();
    {
      f32x16 acc[2];
      zero_acc(acc);
      gemm_p<2, kHid>(acc, pb2, wT + kWT2A, 32 * wave, H2s, kHPitch, lane);
      wprefetch(pc1, wbf + Blob<KP>::W1C, 32 * wave, lane);
      store_dtanh_t(acc, H1s, nullptr, 32 * wave, ublock(w.dh1t, 2 * kHid, m0), kUBlock, 0,
                    lane);
    }
    __syncthreads();

    // ---- critic forward; the value head is folded into the second layer's epilogue
    {
      f32x16 acc[2];
      init_bias_lds(acc, cst + kB1 + kHid, 32 * wave, lane);
      gemm_p<2, KP>(acc, pc1, wbf + Blob<KP>::W1C, 32 * wave, Xs, XP, lane);
      wprefetch(pc2, wbf + Blob<KP>::W2C, 32 * wave, lane);
      store_tanh_t(acc, H1s, 32 * wave, ublock(w.h1t, 2 * kHid, m0) + kHid * kUBlock, kUBlock, 0,
                   lane);
    }
    __syncthreads();
    bf16x4 hc2[4][2];                          // this lane's critic layer-2 activations
    {
      f32x16 acc[2];
      init_bias_lds(acc, cst + kB2C, 32 * wave, lane);
      gemm_p<2, kHid>(acc, pc2, wbf + Blob<KP>::W2C, 32 * wave, H1s, kHPitch, lane);
      float vp[2] = {0.0f, 0.0f};
      float4 w4s[4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        w4s[g] = *reinterpret_cast<const float4*>(w3s + 32 * wave + 8 * g + lh);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 w4 = w4s[g];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          bf16x4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = (__bf16)tanh_act(acc[r][4 * g + j]);
          hc2[g][r] = v;
          vp[r] += (float)v[0] * w4.x + (float)v[1] * w4.y + (float)v[2] * w4.z + (float)v[3] * w4.w;
        }
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) vp[r] += __shfl_xor(vp[r], 32);   // lanes l, l + 32: one row
      if (lane < 32) { vpart[wave][lr] = vp[0]; vpart[wave][32 + lr] = vp[1]; }
    }
    __syncthreads();
    if (tid < kRows) {      // wave 0, one lane per row: value, its error, d(loss)/dv; tile sums
      float v = vpart[0][tid];
#pragma unroll
      for (int q = 1; q < kWaves; ++q) v += vpart[q][tid];
      const long long pr = rowp[tid];
      float dv = 0.0f, se = 0.0f;
      if (pr >= 0) {
        const float err = (v + b3c) - ret_r;
        se = err * err;
        dv = a.vf_coef * err * inv_mb;      // d(vf_coef 0.5 mean(err^2)) / dv
      }
      rowf[tid][4] = dv;
      // the tile's sums over its rows: pl, ent, kl, cf, se, bad and db3c = sum dv
      float st[7] = {rowf[tid][0], rowf[tid][1], rowf[tid][2], rowf[tid][3], se, rowf[tid][7], dv};
#pragma unroll
      for (int q = 0; q < 7; ++q) st[q] = sum64(st[q]);
      if (tid == 0) {
        float* part = w.fpart + (long)tile * kPartCols;
        *reinterpret_cast<float4*>(part) = make_float4(st[0], st[1], st[2], st[3]);
        *reinterpret_cast<float4*>(part + 4) = make_float4(0.0f, st[4], 0.0f, st[5]);
        part[kStatCols + kHid] = st[6];
      }
    }
    __syncthreads();
    wprefetch(pbc, wT + kWT2C, 32 * wave, lane);
    // dw3c = sum over rows of dv h2c (this lane's two rows, then the 32 lanes that share its
    // units) and dH2c = dv w3c (1 - h2c^2), both from the registers; dH2c to H2s (no reader
    // left since the actor's backward) and unit-major
    {
      const float dv0 = rowf[lr][4], dv1 = rowf[32 + lr][4];
      const UnitMajor out(ublock(w.dh2t, 2 * kHid, m0) + kHid * kUBlock, kUBlock, 0, 32 * wave,
                          lane);
      float* part = w.fpart + (long)tile * kPartCols + kStatCols;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int unit = 32 * wave + 8 * g + lh;
        const float4 w4v = *reinterpret_cast<const float4*>(w3s + unit);
        const float w4[4] = {w4v.x, w4v.y, w4v.z, w4v.w};
        float sw[4];
        bf16x4 d0, d1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float h0 = (float)hc2[g][0][j], h1 = (float)hc2[g][1][j];
          sw[j] = sum32(dv0 * h0 + dv1 * h1);
          d0[j] = (__bf16)(dv0 * w4[j] * (1.0f - h0 * h0));
          d1[j] = (__bf16)(dv1 * w4[j] * (1.0f - h1 * h1));
        }
        *reinterpret_cast<bf16x4*>(H2s + lr * kHPitch + unit) = d0;
        *reinterpret_cast<bf16x4*>(H2s + (32 + lr) * kHPitch + unit) = d1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          out.put(g, 0, j, d0[j]);
          out.put(g, 1, j, d1[j]);
        }
        if ((lane & 31) == 0)
          *reinterpret_cast<float4*>(part + unit) = make_float4(sw[0], sw[1], sw[2], sw[3]);
      }
    }
    __syncthreads();
    {
      f32x16 acc[2];
      zero_acc(acc);
      gemm_p<2, kHid>(acc, pbc, wT + kWT2C, 32 * wave, H2s, kHPitch, lane);
      wprefetch(pa1, wbf + Blob<KP>::W1, 32 * wave, lane);    // the next tile's first product
      store_dtanh_t(acc, H1s, nullptr, 32 * wave, ublock(w.dh1t, 2 * kHid, m0) + kHid * kUBlock,
                    kUBlock, 0, lane);
    }
    // the next tile first writes Xs, rowp and rowf (read before the syncs above) and H1s only
    // after its first barrier, so no barrier is needed here
  }
}

// ---- weight gradients: C[a][b] = sum over rows of A[a][row] B[b][row], split over row chunks.
// Output tiles are 256 x 256, so each product's operands are read once per row chunk (the
// first layer's input twice, beside the two 256-unit halves of dH1): the kernel streams ~4.5 KB
// per minibatch row against 4.2 KB of distinct operands.  Eight waves, 2 (A halves of 128) x 4
// (B quarters of 64), each accumulating a 128 x 64 block as 4 x 2 MFMA 32x32 tiles; 64-row
// stages double-buffered through LDS (147 KB), one workgroup per CU.
constexpr int kWT = 256;                  // output tile side
constexpr int kWK = 64;                   // rows per stage
constexpr int kWPitch = kWK + 8;          // bf16 per LDS feature row (16-byte aligned, spread over banks)
constexpr int kWThreads = 512;
constexpr int kWPieces = kWT * kWK / 8 / kWThreads;   // 16-byte pieces per thread per operand

struct WJob {
  const __bf16* A;     // feature 0 of row 0 in the 64-row block layout (ublock)
  const __bf16* B;
  long sA, sB;         // elements between consecutive 64-row blocks: the buffer's features x 64
  int nA, nB;          // features present in the buffers (loads beyond read as zero)
  int vA, vB;          // features that are parameters
  long wbase[2];       // flat index of W[0][0] for a < 256 and for a >= 256
  long bbase[2];       // flat index of the bias of a < 256 / a >= 256
  int wld;             // flat row length of W
};

constexpr int kWMaxWG = 8 * kMaxChunks;   // tiles x chunks (at most 8 tiles)

struct WJobs {
  WJob job[4];
  unsigned char tj[8], ta[8], tb[8];
  int ntiles;
  // workgroup i computes tile wg[i] >> 6 of chunk wg[i] & 63.  Workgroups go to the 8 XCDs round
  // robin (i to XCD i % 8): the two tiles that read the same layer-input rows (the two 256-unit
  // halves of dH1 against X) are placed 8 apart, on one XCD, so the second reads them from its L2.
  unsigned short wg[kWMaxWG];
};

static_assert(kWK == kUBlock, "a weight-gradient stage is one 64-row block of each operand");

__global__ __launch_bounds__(kWThreads, 1) void wgrad_kernel(const WJobs J, long mp,
                                                             int chunk_rows, float* __restrict__ wpart,
                                                             long pld) {
  __shared__ __align__(16) __bf16 As[2][kWT * kWPitch];
  __shared__ __align__(16) __bf16 Bs[2][kWT * kWPitch];
  const int tile = J.wg[blockIdx.x] >> 6, c = J.wg[blockIdx.x] & 63;
  const WJob& jb = J.job[J.tj[tile]];
  const int fa0 = kWT * J.ta[tile], fb0 = kWT * J.tb[tile];
  const bool bias = J.tb[tile] == 0;
  const long k0 = (long)c * chunk_rows;
  const long k1 = min(k0 + chunk_rows, mp);
  const int nst = k1 > k0 ? (int)((k1 - k0) / kWK) : 0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wa = wave & 1, wb = wave >> 1;
  const int part = tid & 7;                   // 8-row piece of a feature's 64 rows
  bf16x8 ra[kWPieces], rb[kWPieces];
  float bsum[kWPieces];
#pragma unroll
  for (int q = 0; q < kWPieces; ++q) bsum[q] = 0.0f;
  const bf16x8 zero8 = {};
  auto load = [&](int st) {
    const long blk = k0 / kUBlock + st;         // kWK = 64: one block per stage
    const __bf16* A = jb.A + blk * jb.sA + 8 * part;
    const __bf16* B = jb.B + blk * jb.sB + 8 * part;
#pragma unroll
    for (int q = 0; q < kWPieces; ++q) {
      const int f = (tid >> 3) + (kWThreads / 8) * q;
      ra[q] = fa0 + f < jb.nA ? *reinterpret_cast<const bf16x8*>(A + (long)(fa0 + f) * kUBlock)
                              : zero8;
      rb[q] = fb0 + f < jb.nB ? *reinterpret_cast<const bf16x8*>(B + (long)(fb0 + f) * kUBlock)
                              : zero8;
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int q = 0; q < kWPieces; ++q) {
      const int f = (tid >> 3) + (kWThreads / 8) * q;
      *reinterpret_cast<bf16x8*>(&As[buf][f * kWPitch + 8 * part]) = ra[q];
      *reinterpret_cast<bf16x8*>(&Bs[buf][f * kWPitch + 8 * part]) = rb[q];
      if (bias) {
#pragma unroll
        for (int i = 0; i < 8; ++i) bsum[q] += (float)ra[q][i];
      }
    }
  };
  // MFMA blocks holding parameters or present features: wave-uniform
  bool liveA[4], liveB[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) liveA[i] = fa0 + 128 * wa + 32 * i < jb.nA;
#pragma unroll
  for (int j = 0; j < 2; ++j) liveB[j] = fb0 + 64 * wb + 32 * j < jb.nB;
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  if (nst > 0) {
    load(0);
    stage(0);
  }
  __syncthreads();
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) load(st + 1);
#pragma unroll
    for (int kk = 0; kk < kWK / 16; ++kk) {
      bf16x8 af[4], bfg[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[buf][(128 * wa + 32 * i + lr) * kWPitch +
                                                          16 * kk + lk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfg[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(64 * wb + 32 * j + lr) * kWPitch +
                                                           16 * kk + lk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          if (liveA[i] && liveB[j]) acc[i][j] = mfma(af[i], bfg[j], acc[i][j]);
    }
    if (st + 1 < nst) stage(buf ^ 1);
    __syncthreads();
  }
  float* out = wpart + (long)c * pld;
  // element e of acc[i][j]: a = fa0 + 128wa + 32i + 8(e/4) + 4(lane/32) + e%4, b = fb0 + 64wb + 32j + lane%32
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int b = fb0 + 64 * wb + 32 * j + lr;
      if (b >= jb.vB) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int aa = fa0 + 128 * wa + 32 * i + 8 * (e >> 2) + (lane >> 5) * 4 + (e & 3);
        if (aa < jb.vA)
          out[jb.wbase[aa >> 8] + (long)(aa & 255) * jb.wld + b] = acc[i][j][e];
      }
    }
  if (bias) {
#pragma unroll
    for (int q = 0; q < kWPieces; ++q) {
      float s = bsum[q];
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      const int aa = fa0 + (tid >> 3) + (kWThreads / 8) * q;
      if (part == 0 && aa < jb.vA) out[jb.bbase[aa >> 8] + (aa & 255)] = s;
    }
  }
}

// out[c] = sum over r of part[r * ld + c], rows in a fixed order: PH row phases per column
template <int PH>
__global__ __launch_bounds__(64 * PH) void colsum_kernel(const float* __restrict__ part, int nrows,
                                                         long ld, long ncols,
                                                         float* __restrict__ out) {
  __shared__ float s[PH][64];
  const int t = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const long c = (long)blockIdx.x * 64 + t;
  float acc = 0.0f;
  if (c < ncols)
    for (int r = ph; r < nrows; r += PH) acc += part[(long)r * ld + c];
  s[ph][t] = acc;
  __syncthreads();
  if (ph == 0 && c < ncols) {
    float v = s[0][t];
#pragma unroll
    for (int k = 1; k < PH; ++k) v += s[k][t];
    out[c] = v;
  }
}

// colsum_kernel<4> four columns to a thread (16-byte loads and stores; ncols and ld multiples of
// 4, part and out 16-byte aligned): every column summed in the same row order, the same bits
__global__ __launch_bounds__(256) void colsum4_kernel(const float* __restrict__ part, int nrows,
                                                      long ld, long ncols,
                                                      float* __restrict__ out) {
  __shared__ float4 s[4][64];
  const int t = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const long c = 4 * ((long)blockIdx.x * 64 + t);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (c < ncols)
    for (int r = ph; r < nrows; r += 4) {
      const float4 v = *reinterpret_cast<const float4*>(part + (long)r * ld + c);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
  s[ph][t] = acc;
  __syncthreads();
  if (ph == 0 && c < ncols) {
    float4 v = s[0][t];
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      const float4 u = s[k][t];
      v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
    }
    *reinterpret_cast<float4*>(out + c) = v;
  }
}

// first level over the fused kernel's partial rows: block (x, y) sums rows [64y, 64y + 64) of
// columns [64x, 64x + 64) (4 phases of 16 rows, combined in order)
__global__ __launch_bounds__(256) void colsum_group_kernel(const float* __restrict__ part, int nrows,
                                                           float* __restrict__ mid) {
  __shared__ float sm[4][64];
  const int t = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + t;
  const int r0 = blockIdx.y * kColRows;
  float acc = 0.0f;
  if (c < kPartCols)
    for (int r = r0 + ph; r < min(r0 + kColRows, nrows); r += 4) acc += part[(long)r * kPartCols + c];
  sm[ph][t] = acc;
  __syncthreads();
  if (ph == 0 && c < kPartCols)
    mid[(long)blockIdx.y * kPartCols + c] = (sm[0][t] + sm[1][t]) + (sm[2][t] + sm[3][t]);
}

// second level over the first-level sums `mid` ([ng][kPartCols]): block x sums columns
// [64x, 64x + 64) exactly as colsum_kernel<4> does (row phases r = ph (mod 4), combined in
// order); the statistics columns [0, kStatCols) go to sums, dw3c and db3c to grad; block 0 then
// forms the minibatch means from its statistics sums (ppo_gpu.py:2080-2081, 2098, 2107-2108).
__global__ __launch_bounds__(256) void colsum_tail_kernel(const float* __restrict__ mid, int ng,
                                                          float* __restrict__ sums,
                                                          float* __restrict__ grad_w3c,
                                                          const float* __restrict__ advs, int n,
                                                          float* __restrict__ stats) {
  __shared__ float sm[4][64];
  const int t = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + t;
  constexpr int kCols = kStatCols + kHid + 1;
  float acc = 0.0f;
  if (c < kCols)
    for (int r = ph; r < ng; r += 4) acc += mid[(long)r * kPartCols + c];
  sm[ph][t] = acc;
  __syncthreads();
  if (ph == 0 && c < kCols) {
    float v = sm[0][t];
#pragma unroll
    for (int k = 1; k < 4; ++k) v += sm[k][t];
    if (c < kStatCols) {
      sums[c] = v;
      sm[0][t] = v;
    } else {
      grad_w3c[c - kStatCols] = v;
    }
  }
  if (blockIdx.x != 0) return;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float fn = (float)n;
    stats[F16_PPO_STAT_POLICY_LOSS] = sm[0][0] / fn;
    stats[F16_PPO_STAT_ENTROPY] = sm[0][1] / fn;
    stats[F16_PPO_STAT_APPROX_KL] = sm[0][2] / fn;
    stats[F16_PPO_STAT_CLIPFRAC] = sm[0][3] / fn;
    stats[F16_PPO_STAT_VALUE_LOSS] = 0.5f * (sm[0][5] / fn);
    stats[F16_PPO_STAT_ADV_MEAN] = advs[0];
    stats[F16_PPO_STAT_ADV_STD] = advs[1];
    stats[7] = sm[0][7];
  }
}

// ---- clip_grad_norm_ + Adam
__global__ __launch_bounds__(256) void sumsq_kernel(const float* __restrict__ g, long n, long na,
                                                    double* __restrict__ normp) {
  __shared__ double sa[256], sc[256];
  const long b0 = (long)blockIdx.x * kNormBlockElems;
  double xa = 0.0, xc = 0.0;
  for (int i = threadIdx.x; i < kNormBlockElems; i += 256) {
    const long k = b0 + i;
    if (k < n) {
      const double v = g[k];
      if (k < na) xa += v * v;
      else xc += v * v;
    }
  }
  sa[threadIdx.x] = xa;
  sc[threadIdx.x] = xc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) { sa[threadIdx.x] += sa[threadIdx.x + w]; sc[threadIdx.x] += sc[threadIdx.x + w]; }
    __syncthreads();
  }
  if (threadIdx.x == 0) { normp[2L * blockIdx.x] = sa[0]; normp[2L * blockIdx.x + 1] = sc[0]; }
}

struct AdamScalars {
  float lr_step[2];        // -lr / (1 - beta1^t), actor / critic
  float bc2_sqrt;          // sqrt(1 - beta2^t)
  float one_m_b1, b2, one_m_b2, eps, max_norm;
};

__global__ __launch_bounds__(256) void adam_kernel(float* __restrict__ p, float* __restrict__ m,
                                                   float* __restrict__ v, float* __restrict__ g,
                                                   long n, long na, const double* __restrict__ normp,
                                                   int nblk, const AdamScalars S,
                                                   float* __restrict__ norms_out) {
  __shared__ double sa[256], sc[256];
  __shared__ float clip[2];
  double xa = 0.0, xc = 0.0;
  for (int b = threadIdx.x; b < nblk; b += 256) { xa += normp[2L * b]; xc += normp[2L * b + 1]; }
  sa[threadIdx.x] = xa;
  sc[threadIdx.x] = xc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) { sa[threadIdx.x] += sa[threadIdx.x + w]; sc[threadIdx.x] += sc[threadIdx.x + w]; }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float tn[2] = {(float)sqrt(sa[0]), (float)sqrt(sc[0])};
    for (int k = 0; k < 2; ++k) {
      float cc = S.max_norm / (tn[k] + 1e-6f);
      clip[k] = cc > 1.0f ? 1.0f : cc;
    }
    if (blockIdx.x == 0 && norms_out) { norms_out[0] = tn[0]; norms_out[1] = tn[1]; }
  }
  __syncthreads();
  const long k = (long)blockIdx.x * 256 + threadIdx.x;
  if (k >= n) return;
  const int net = k < na ? 0 : 1;
  const float gk = g[k] * clip[net];
  g[k] = gk;
  float mk = m[k], vk = v[k];
  mk = mk + S.one_m_b1 * (gk - mk);            // exp_avg.lerp_(grad, 1 - beta1)
  vk = vk * S.b2;                              // exp_avg_sq.mul_(beta2)
  vk = vk + S.one_m_b2 * gk * gk;              //   .addcmul_(grad, grad, 1 - beta2)
  const float denom = sqrtf(vk) / S.bc2_sqrt + S.eps;
  p[k] = p[k] + S.lr_step[net] * (mk / denom); // param.addcdiv_(exp_avg, denom, -step_size)
  m[k] = mk;
  v[k] = vk;
}

// ---- blobs from the flat master parameters
template <int KP>
__global__ __launch_bounds__(256) void pack_kernel(const float* __restrict__ P,
                                                   __bf16* __restrict__ wbf, float* __restrict__ wf,
                                                   __bf16* __restrict__ wT) {
  constexpr int D = KP == 192 ? 184 : 214;
  const Flat F{D};
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  constexpr long nbf = Blob<KP>::NBF;
  if (i < nbf) {
    // fragment-major blocks: element q of a matrix [N][K] is (n, k) of block q / 512
    auto unfrag = [](long q, long K, long& n, long& k) {
      const long blk = q >> 9, r = q & 511, l = r >> 3;
      n = (blk / (K >> 4)) * 32 + (l & 31);
      k = (blk % (K >> 4)) * 16 + (l >> 5) * 8 + (r & 7);
    };
    float x = 0.0f;
    long n, k;
    if (i < Blob<KP>::W2A) {
      unfrag(i, KP, n, k);
      if (k < D) x = n < kHid ? P[F.a_w1() + n * D + k] : P[F.c_w1() + (n - kHid) * D + k];
    } else if (i < Blob<KP>::W2C) {
      unfrag(i - Blob<KP>::W2A, kHid, n, k);
      x = P[F.a_w2() + n * kHid + k];
    } else if (i < Blob<KP>::W3A) {
      unfrag(i - Blob<KP>::W2C, kHid, n, k);
      x = P[F.c_w2() + n * kHid + k];
    } else {
      unfrag(i - Blob<KP>::W3A, kHid, n, k);
      if (n < kLogits) x = P[F.a_w3() + n * kHid + k];
    }
    if (wbf) wbf[i] = (__bf16)x;
    return;
  }
  long j = i - nbf;
  if (j < F16_POLICY_NF) {
    float x = 0.0f;
    if (j < kB2A) x = j < kHid ? P[F.a_b1() + j] : P[F.c_b1() + j - kHid];
    else if (j < kB2C) x = P[F.a_b2() + j - kB2A];
    else if (j < kB3A) x = P[F.c_b2() + j - kB2C];
    else if (j < kW3C) x = j - kB3A < kLogits ? P[F.a_b3() + j - kB3A] : 0.0f;
    else if (j < kB3C) x = P[F.c_w3() + j - kW3C];
    else x = P[F.c_b3()];
    if (wf) wf[j] = x;
    return;
  }
  j -= F16_POLICY_NF;
  if (j < F16_PPO_WT_ELEMS && wT) {
    // transposed matrices, fragment-major: W3a^T [256][96], W2a^T and W2c^T [256][256]
    const long base = j < kWT2A ? 0 : (j < kWT2C ? kWT2A : kWT2C);
    const long K = j < kWT2A ? kLogitsPad : kHid;
    const long q = j - base, blk = q >> 9, r = q & 511, l = r >> 3;
    const long nn = (blk / (K >> 4)) * 32 + (l & 31);
    const long kk = (blk % (K >> 4)) * 16 + (l >> 5) * 8 + (r & 7);
    float x = 0.0f;
    if (j < kWT2A) {
      if (kk < kLogits) x = P[F.a_w3() + kk * kHid + nn];
    } else if (j < kWT2C) {
      x = P[F.a_w2() + kk * kHid + nn];
    } else {
      x = P[F.c_w2() + kk * kHid + nn];
    }
    wT[j] = (__bf16)x;
  }
}

template <int KP>
int launch_pack(const float* param, void* wbf, float* wf, void* wT, hipStream_t s) {
  const long total = Blob<KP>::NBF + F16_POLICY_NF + F16_PPO_WT_ELEMS;
  hipLaunchKernelGGL(pack_kernel<KP>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     param, static_cast<__bf16*>(wbf), wf, static_cast<__bf16*>(wT));
  return f16_last_error();
}

// ---- the rollout's aggregate finite check
// One pass over every span, 16-byte loads in the aligned body and single elements at the two
// unaligned ends: the largest exponent field of the float32 words and of the float64 high
// words (all ones only for inf and NaN), and whether any byte of a uint8 flag span is zero
// (((w - 0x01010101) & ~w & 0x80808080) != 0 exactly when a byte of w is zero).
struct FiniteSpans {
  F16FiniteSpan s[F16_FINITE_MAX_SPANS];
  int n;
};
constexpr int kFinBlock = 256;
constexpr int kFinUnroll = 4;
constexpr unsigned kExp32 = 0x7f800000u, kExp64 = 0x7ff00000u;

struct FinAcc {
  unsigned m32 = 0, m64 = 0, zero = 0;
  __device__ __forceinline__ void word(unsigned w, int eb, bool high) {
    if (eb == 4) m32 = max(m32, w & kExp32);
    else if (eb == 8) { if (high) m64 = max(m64, w & kExp64); }
    else zero |= (w - 0x01010101u) & ~w & 0x80808080u;
  }
  __device__ __forceinline__ void chunk(const uint4& q, int eb) {
    word(q.x, eb, false); word(q.y, eb, true); word(q.z, eb, false); word(q.w, eb, true);
  }
  __device__ __forceinline__ void element(const unsigned char* e, int eb) {
    if (eb == 4) m32 = max(m32, *reinterpret_cast<const unsigned*>(e) & kExp32);
    else if (eb == 8) m64 = max(m64, *reinterpret_cast<const unsigned*>(e + 4) & kExp64);
    else zero |= (*e == 0) ? 1u : 0u;
  }
};

__global__ void finite_init_kernel(unsigned char* flag) { flag[0] = 1; }

__global__ __launch_bounds__(kFinBlock) void finite_kernel(FiniteSpans S,
                                                           unsigned char* __restrict__ flag) {
  FinAcc acc;
  const long gt = (long)blockIdx.x * kFinBlock + threadIdx.x;
  const long G = (long)gridDim.x * kFinBlock;
  for (int k = 0; k < S.n; ++k) {
    const int eb = S.s[k].elem_bytes;
    const uintptr_t p = (uintptr_t)S.s[k].ptr;
    const uintptr_t end = p + (uintptr_t)S.s[k].n * (uintptr_t)eb;
    const uintptr_t a = min((p + 15) & ~(uintptr_t)15, end);
    const uintptr_t e = max(a, end & ~(uintptr_t)15);
    const uint4* body = reinterpret_cast<const uint4*>(a);
    const long nchunk = (long)((e - a) >> 4);
    for (long c = gt; c < nchunk; c += kFinUnroll * G) {
      uint4 q[kFinUnroll];
#pragma unroll
      for (int u = 0; u < kFinUnroll; ++u)
        if (c + u * G < nchunk) q[u] = body[c + u * G];
#pragma unroll
      for (int u = 0; u < kFinUnroll; ++u)
        if (c + u * G < nchunk) acc.chunk(q[u], eb);
    }
    // the ends: fewer than 16 bytes each, one element per thread of the first workgroup
    if (gt < 16) {
      const uintptr_t h = p + (uintptr_t)gt * eb, t = e + (uintptr_t)gt * eb;
      if (h < a) acc.element(reinterpret_cast<const unsigned char*>(h), eb);
      if (t < end) acc.element(reinterpret_cast<const unsigned char*>(t), eb);
    }
  }
  if (acc.m32 == kExp32 || acc.m64 == kExp64 || acc.zero != 0) flag[0] = 0;
}

// ---- the epoch's permutation of the transitions
// perm[i] = the image of i under an eight-round Feistel network on la + lb bits (round r maps
// (L, R), L of a bits and R of b, to (R, L ^ F(R ^ k_r)) and swaps a and b; F the low a bits of
// MurmurHash3's 32-bit finaliser, the eight round keys k_r two Philox4x32-10 blocks of the 64-bit
// key), applied again while the image lies outside [0, n) (cycle walking: the walk stays on i's
// cycle of the network's bijection of [0, 2^(la + lb)), so it ends, and the restriction is a
// bijection of [0, n)).  Below 2^15 elements the halves are equal (la = lb = h, 4^h the smallest
// power of four >= n: fewer than four passes per element on average; with four rounds instead of
// eight the positions drawn for small n are measurably non-uniform); above, la + lb is the
// smallest power of two >= n with halves of 8 bits or more: fewer than two passes on average and
// one at a power of two (a wave waits for its longest walk, so the shorter walks count).
constexpr int kPermBlock = 256;
constexpr int kPermRounds = 8;

__device__ __forceinline__ uint32_t fmix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x85EBCA6Bu;
  x ^= x >> 13;
  x *= 0xC2B2AE35u;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ uint64_t feistel(uint64_t x, int la, int lb,
                                            const uint32_t (&k)[kPermRounds]) {
  int a = la, b = lb;
  uint32_t L = (uint32_t)(x >> b), R = (uint32_t)x & ((1u << b) - 1u);
#pragma unroll
  for (int r = 0; r < kPermRounds; ++r) {   // an even count: a and b end as they began
    const uint32_t nr = L ^ (fmix32(R ^ k[r]) & ((1u << a) - 1u));
    L = R;
    R = nr;
    const int t = a;
    a = b;
    b = t;
  }
  return ((uint64_t)L << b) | R;
}

__global__ __launch_bounds__(kPermBlock) void permute_kernel(long long* __restrict__ perm,
                                                             long n, int la, int lb,
                                                             const unsigned long long* key) {
  __shared__ uint32_t ks[kPermRounds];
  if (threadIdx.x < kPermRounds / 4) {
    const unsigned long long k = key[0];
    uint32_t c[4] = {threadIdx.x, 0x243F6A88u, 0x85A308D3u, 0x13198A2Eu};
    f16rng::philox4x32_10(c, (uint32_t)k, (uint32_t)(k >> 32));
#pragma unroll
    for (int j = 0; j < 4; ++j) ks[4 * threadIdx.x + j] = c[j];
  }
  __syncthreads();
  const long i = (long)blockIdx.x * kPermBlock + threadIdx.x;
  if (i >= n) return;
  uint32_t k[kPermRounds];
#pragma unroll
  for (int r = 0; r < kPermRounds; ++r) k[r] = ks[r];
  uint64_t x = feistel((uint64_t)i, la, lb, k);
  while (x >= (uint64_t)n) x = feistel(x, la, lb, k);
  perm[i] = (long long)x;
}

}  // namespace f16ppo

using namespace f16ppo;

// compute units of the current device (the persistent fused kernel runs one workgroup on each)
static int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
    return 256;
  return n;
}

// Resident wgrad workgroups: compute units x the kernel's occupancy (1 per CU on MI355X: 147 KB
// LDS), asked once per process.
static int wgrad_slots() {
  static int slots = 0;
  if (slots == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, wgrad_kernel, kWThreads, 0) !=
            hipSuccess || per_cu < 1)
      per_cu = 1;
    slots = per_cu * device_cus();
  }
  return slots;
}

extern "C" int f16_ppo_param_counts(int obs_dim, long* out2) {
  if (!out2 || (obs_dim != 184 && obs_dim != 214)) return F16_EINVAL;
  const Flat F{obs_dim};
  out2[0] = F.na();
  out2[1] = F.n() - F.na();
  return 0;
}

extern "C" long f16_ppo_workspace_bytes(int obs_dim, int mb_rows) {
  if ((obs_dim != 184 && obs_dim != 214) || mb_rows < 1 || mb_rows > kMaxMinibatchRows) return -1;
  return layout(obs_dim, mb_rows, nullptr).bytes;
}

extern "C" int f16_ppo_grad(const F16PPOArgs* a, void* stream) {
  if (!a || (a->obs_dim != 184 && a->obs_dim != 214)) return F16_EINVAL;
  if (a->mb_rows < 1 || a->count < 1 || a->obs_ld < a->obs_dim) return F16_EINVAL;
  if (a->mb_rows > kMaxMinibatchRows) return F16_EINVAL;   // bound on the minibatch size
  if (!a->obs || !a->act || !a->old_logp || !a->adv || !a->ret || !a->idx) return F16_EINVAL;
  if (!a->wbf || !a->wf || !a->wT || !a->grad || !a->stats || !a->work) return F16_EINVAL;
  if (((uintptr_t)a->wbf & 15) || ((uintptr_t)a->wT & 15) || ((uintptr_t)a->work & 255))
    return F16_EINVAL;
  if ((a->obs_ld & 1) || ((uintptr_t)a->obs & 7)) return F16_EINVAL;   // rows move as float2
  const int D = a->obs_dim, kp = (D + 31) / 32 * 32;
  const Flat F{D};
  const Work w = layout(D, a->mb_rows, a->work, wgrad_slots());
  hipStream_t s = (hipStream_t)stream;
  if (!a->adv_stats) {   // else the epoch's f16_ppo_adv_stats formed them
    hipLaunchKernelGGL(adv_partial_kernel, dim3(w.nadv), dim3(kAdvThreads), 0, s, a->adv, a->idx,
                       a->mb_rows, a->count, w.advp);
    hipLaunchKernelGGL(adv_final_kernel, dim3(1), dim3(kAdvThreads), 0, s, a->adv, a->idx,
                       a->mb_rows, a->count, w.nadv, (const double*)w.advp, w.advs);
  }
  const unsigned fgrid = (unsigned)std::min(w.nwg, device_cus());
  if (kp == 192)
    hipLaunchKernelGGL(ppo_fused_kernel<192>, dim3(fgrid), dim3(kThreads), 0, s, *a, w);
  else
    hipLaunchKernelGGL(ppo_fused_kernel<224>, dim3(fgrid), dim3(kThreads), 0, s, *a, w);
  // the four weight-gradient products and their tiles
  WJobs J{};
  const long na = F.na();
  constexpr long kB512 = 512 * kUBlock, kB256 = 256 * kUBlock;
  J.job[0] = WJob{w.dh1t, w.xt, kB512, kp * kUBlock, 512, kp, 512, D, {F.a_w1(), F.c_w1()},
                  {F.a_b1(), F.c_b1()}, D};
  J.job[1] = WJob{w.dh2t, w.h1t, kB512, kB512, 256, 256, 256, 256, {F.a_w2(), F.a_w2()},
                  {F.a_b2(), F.a_b2()}, 256};
  J.job[2] = WJob{w.dh2t + kB256, w.h1t + kB256, kB512, kB512, 256, 256, 256, 256,
                  {F.c_w2(), F.c_w2()}, {F.c_b2(), F.c_b2()}, 256};
  J.job[3] = WJob{w.dzt, w.h2t, kLogitsPad * kUBlock, kB256, kLogitsPad, 256, kLogits, 256,
                  {F.a_w3(), F.a_w3()},
                  {F.a_b3(), F.a_b3()}, 256};
  (void)na;
  int nt = 0;
  const int ntA[4] = {2, 1, 1, 1}, ntB[4] = {(kp + 255) / 256, 1, 1, 1};
  for (int j = 0; j < 4; ++j)
    for (int ta = 0; ta < ntA[j]; ++ta)
      for (int tb = 0; tb < ntB[j]; ++tb) {
        J.tj[nt] = (unsigned char)j;
        J.ta[nt] = (unsigned char)ta;
        J.tb[nt] = (unsigned char)tb;
        ++nt;
      }
  J.ntiles = nt;
  {
    // tiles 0 and 1 (job 0's A halves, one B) of chunk c at ids 16 (c / 8) + c % 8 and 8 more,
    // the other tiles' work in the ids left, in tile-major order; where the last pair would not
    // fit the grid (few chunks), id c nt + t runs tile t of chunk c
    const int nwg = nt * w.nchunk;
    const int last = 16 * ((w.nchunk - 1) / 8) + (w.nchunk - 1) % 8 + 8;
    if (last < nwg) {
      for (int i = 0; i < nwg; ++i) J.wg[i] = 0xffff;
      for (int c = 0; c < w.nchunk; ++c) {
        const int id0 = 16 * (c / 8) + c % 8;
        J.wg[id0] = (unsigned short)c;
        J.wg[id0 + 8] = (unsigned short)(64 + c);
      }
      int next = 0;
      for (int t = 2; t < nt; ++t)
        for (int c = 0; c < w.nchunk; ++c) {
          while (J.wg[next] != 0xffff) ++next;   // exactly nwg - 2 nchunk free ids remain
          J.wg[next] = (unsigned short)(t * 64 + c);
        }
    } else {
      for (int c = 0; c < w.nchunk; ++c)
        for (int t = 0; t < nt; ++t) J.wg[c * nt + t] = (unsigned short)(t * 64 + c);
    }
  }
  const long pld = F.n() - 257;          // every flat parameter but the critic's value head
  hipLaunchKernelGGL(wgrad_kernel, dim3(nt * w.nchunk), dim3(kWThreads), 0, s, J, w.ld,
                     w.chunk_rows, w.wpart, pld);
  if (pld % 4 == 0 && ((uintptr_t)a->grad & 15) == 0)
    hipLaunchKernelGGL(colsum4_kernel, dim3((unsigned)((pld / 4 + 63) / 64)), dim3(256), 0, s,
                       (const float*)w.wpart, w.nchunk, pld, pld, a->grad);
  else
    hipLaunchKernelGGL(colsum_kernel<4>, dim3((unsigned)((pld + 63) / 64)), dim3(256), 0, s,
                       (const float*)w.wpart, w.nchunk, pld, pld, a->grad);
  // the per-workgroup partials (statistics, dw3c, db3c): groups of kColRows rows, then the groups
  const int ng = (int)kColGroups(w.nwg);
  hipLaunchKernelGGL(colsum_group_kernel, dim3((kPartCols + 63) / 64, ng), dim3(256), 0, s,
                     (const float*)w.fpart, w.nwg, w.fmid);
  hipLaunchKernelGGL(colsum_tail_kernel, dim3((kStatCols + kHid + 1 + 63) / 64), dim3(256), 0, s,
                     (const float*)w.fmid, ng, w.advs + 8, a->grad + F.c_w3(),
                     a->adv_stats ? a->adv_stats : (const float*)w.advs, a->mb_rows, a->stats);
  return f16_last_error();
}

extern "C" int f16_ppo_adam_step(const F16AdamArgs* a, void* stream) {
  if (!a || (a->obs_dim != 184 && a->obs_dim != 214) || a->step < 1) return F16_EINVAL;
  if (!a->param || !a->exp_avg || !a->exp_avg_sq || !a->grad || !a->work) return F16_EINVAL;
  if (((uintptr_t)a->work & 255) || (a->wbf && ((uintptr_t)a->wbf & 15))) return F16_EINVAL;
  if ((a->wbf == nullptr) != (a->wf == nullptr)) return F16_EINVAL;
  const Flat F{a->obs_dim};
  const Work w = layout(a->obs_dim, 1, a->work);
  const long n = F.n();
  const int nblk = norm_blocks(n);
  AdamScalars S;
  const double t = (double)a->step;
  const double bc1 = 1.0 - pow(a->beta1, t), bc2 = 1.0 - pow(a->beta2, t);
  S.lr_step[0] = (float)(-(a->actor_lr / bc1));
  S.lr_step[1] = (float)(-(a->critic_lr / bc1));
  S.bc2_sqrt = (float)sqrt(bc2);
  S.one_m_b1 = (float)(1.0 - a->beta1);
  S.b2 = (float)a->beta2;
  S.one_m_b2 = (float)(1.0 - a->beta2);
  S.eps = (float)a->eps;
  S.max_norm = a->max_grad_norm;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(sumsq_kernel, dim3(nblk), dim3(256), 0, s, (const float*)a->grad, n, F.na(),
                     w.normp);
  hipLaunchKernelGGL(adam_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a->param,
                     a->exp_avg, a->exp_avg_sq, a->grad, n, F.na(), (const double*)w.normp, nblk, S,
                     a->grad_norms);
  int rc = f16_last_error();
  if (rc || (!a->wbf && !a->wT)) return rc;
  return a->obs_dim == 184 ? launch_pack<192>(a->param, a->wbf, a->wf, a->wT, s)
                           : launch_pack<224>(a->param, a->wbf, a->wf, a->wT, s);
}

extern "C" int f16_ppo_pack(const float* param, int obs_dim, void* wbf, float* wf, void* wT,
                            void* stream) {
  if (!param || (obs_dim != 184 && obs_dim != 214)) return F16_EINVAL;
  if ((wbf == nullptr) != (wf == nullptr) || (!wbf && !wT)) return F16_EINVAL;
  if ((wbf && ((uintptr_t)wbf & 15)) || (wT && ((uintptr_t)wT & 15))) return F16_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  return obs_dim == 184 ? launch_pack<192>(param, wbf, wf, wT, s)
                        : launch_pack<224>(param, wbf, wf, wT, s);
}

extern "C" int f16_all_finite(const F16FiniteSpan* spans, int nspans, unsigned char* flag,
                              void* stream) {
  if (!flag || nspans < 0 || nspans > F16_FINITE_MAX_SPANS || (nspans > 0 && !spans))
    return F16_EINVAL;
  FiniteSpans S;
  S.n = nspans;
  long chunks = 0;
  for (int k = 0; k < nspans; ++k) {
    const F16FiniteSpan& sp = spans[k];
    if (sp.n < 0 || (sp.elem_bytes != 1 && sp.elem_bytes != 4 && sp.elem_bytes != 8))
      return F16_EINVAL;
    if (sp.n > 0 && (!sp.ptr || ((uintptr_t)sp.ptr % (uintptr_t)sp.elem_bytes)))
      return F16_EINVAL;
    if (sp.n > (1L << 40) / sp.elem_bytes) return F16_EINVAL;
    S.s[k] = sp;
    chunks = std::max(chunks, sp.n * sp.elem_bytes / 16);
  }
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(finite_init_kernel, dim3(1), dim3(1), 0, s, flag);
  // enough workgroups to keep every CU's loads in flight on the largest span, at most 8 per CU
  const long per_block = (long)kFinBlock * kFinUnroll;
  const long blocks = std::min<long>(std::max<long>(1, (chunks + per_block - 1) / per_block),
                                     8L * device_cus());
  hipLaunchKernelGGL(finite_kernel, dim3((unsigned)blocks), dim3(kFinBlock), 0, s, S, flag);
  return f16_last_error();
}

extern "C" int f16_permutation(long long* perm, long n, const unsigned long long* key,
                               void* stream) {
  if (!perm || !key || n < 1 || n > (1L << 31)) return F16_EINVAL;   // the grid's x extent
  int k = 1;
  while ((1L << k) < n) ++k;
  int la, lb;
  if (k >= 16) {
    la = k - k / 2;
    lb = k / 2;
  } else {
    la = 1;
    while ((1L << (2 * la)) < n) ++la;
    lb = la;
  }
  hipLaunchKernelGGL(permute_kernel, dim3((unsigned)((n + kPermBlock - 1) / kPermBlock)),
                     dim3(kPermBlock), 0, (hipStream_t)stream, perm, n, la, lb, key);
  return f16_last_error();
}

static inline int adv_blocks(int mb_rows) {
  return (mb_rows + kAdvThreads * kAdvPer - 1) / (kAdvThreads * kAdvPer);
}

extern "C" long f16_ppo_adv_work_bytes(int mb_rows, int nmb) {
  if (mb_rows < 1 || mb_rows > kMaxMinibatchRows || nmb < 1) return -1;
  return (long)adv_blocks(mb_rows) * nmb * 2 * (long)sizeof(double);
}

extern "C" int f16_ppo_adv_stats(const float* adv, const long long* idx, long total, long count,
                                 int mb_rows, int nmb, float* out, void* work, void* stream) {
  if (!adv || !idx || !out || !work || total < 1 || count < 1) return F16_EINVAL;
  if (mb_rows < 1 || mb_rows > kMaxMinibatchRows || nmb < 1 || nmb > 65535) return F16_EINVAL;
  if ((long)(nmb - 1) * mb_rows >= total || (long)nmb * mb_rows < total) return F16_EINVAL;
  if ((uintptr_t)work & 7) return F16_EINVAL;
  const int nadv = adv_blocks(mb_rows);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(adv_partial_epoch_kernel, dim3(nadv, nmb), dim3(kAdvThreads), 0, s, adv,
                     idx, mb_rows, total, count, nadv, static_cast<double*>(work));
  hipLaunchKernelGGL(adv_final_epoch_kernel, dim3(nmb), dim3(kAdvThreads), 0, s, adv, idx,
                     mb_rows, total, count, nadv, static_cast<const double*>(work), out);
  return f16_last_error();
}
