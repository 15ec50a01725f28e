// policy_mfma.h -- the bf16 MFMA building blocks shared by the rollout policy kernel and the
// PPO update kernels: packed-blob offsets, the tanh used for the hidden activations, and the
// weight-streaming 32x32x16 tile product with its bias/tanh epilogues.
#pragma once
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "f16_policy.h"

namespace f16pol {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRows = 64;               // observation rows per workgroup
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kHid = F16_POLICY_HID;    // 256
constexpr int kHPitch = kHid + 8;       // bf16 per LDS row of one network's hidden activations
constexpr int kBins = F16_POLICY_BINS;  // 21
constexpr int kChan = F16_POLICY_CHANNELS;
constexpr int kLogits = kBins * kChan;  // 84
constexpr int kLogitsPad = 96;
constexpr int kLPitch = 100;            // f32 per LDS row of logits (16-byte rows)
constexpr int kPrefetch = 3;            // weight K-slices in flight ahead of the MFMAs

// offsets (elements) inside the packed blobs
template <int KP>
struct Blob {
  static constexpr long W1 = 0;
  static constexpr long W1C = (long)kHid * KP;     // critic rows of W1
  static constexpr long W2A = 2L * kHid * KP;
  static constexpr long W2C = W2A + (long)kHid * kHid;
  static constexpr long W3A = W2C + (long)kHid * kHid;
  static constexpr long NBF = W3A + (long)kLogitsPad * kHid;
};
constexpr int kB1 = 0, kB2A = 512, kB2C = 768, kB3A = 1024, kW3C = 1120, kB3C = 1376;
static_assert(kB3C + 1 == F16_POLICY_NF, "f32 blob layout");

// tanh for the bf16 hidden activations: 2 / (1 + t) - 1, t = e^{-2x}, from the hardware exp2
// and reciprocal (~1 ulp each) and one fma 2 r - 1.  Near 0 the difference cancels, but the
// absolute error stays near 2e-7 everywhere (r = 1/2 to ~1e-7), far inside the bf16 rounding
// step the result is stored with; t = inf below x = -44 gives r = 0, -1 exactly.  Five
// instructions per activation, two of them transcendental.
__device__ __forceinline__ float tanh_act(float x) {
  const float t = __builtin_amdgcn_exp2f(x * -2.8853900817779268f);
  const float r = __builtin_amdgcn_rcpf(1.0f + t);
  return __builtin_fmaf(2.0f, r, -1.0f);
}

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Weight matrices [N][K] are stored fragment-major: one 512-element block per (32-unit tile t,
// 16-wide K-slice s), blocks in (t, s) order, holding lane l's 8 operand values at [8l, 8l + 8)
// -- unit 32t + l%32, K columns 16s + 8(l/32) .. +8 -- so a wavefront's fragment load is 1 KB
// contiguous (8 whole cache lines instead of 32 partial ones).

// acc[r] += W(units u0..u0+31, fragment-major [units][K]) x A(rows 32r.., LDS [row][pitch])^T
// over K (u0 a multiple of 32).  Units are the MFMA rows, observation rows the MFMA columns:
// element e of a tile's result held by `lane` is unit 8(e/4) + 4(lane/32) + e%4, row lane%32.
// Weights run PF K-slices ahead (at most K/16 - 1), the LDS activation fragments one slice ahead.
#ifndef F16_GEMM_PIN
#define F16_GEMM_PIN 1
#endif
template <int NR, int K, int PF = kPrefetch, bool PIN = (F16_GEMM_PIN != 0)>
__device__ __forceinline__ void gemm_t(f32x16 (&acc)[NR], const __bf16* __restrict__ Wg, int u0,
                                       const __bf16* __restrict__ As, int a_pitch, int a_col0,
                                       int lane) {
  constexpr int PD = PF < K / 16 ? PF : K / 16 - 1;     // prefetch distance
  const int lr = lane & 31, lk = (lane >> 5) * 8;
  constexpr int NK = K / 16;
  const __bf16* wp = Wg + (long)(u0 >> 5) * (K / 16) * 512 + lane * 8;
  const __bf16* ap = As + lr * a_pitch + a_col0 + lk;
  bf16x8 w[PD + 1];
#pragma unroll
  for (int q = 0; q < PD; ++q) w[q] = *reinterpret_cast<const bf16x8*>(wp + 512 * q);
  bf16x8 a[NR], an[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) a[r] = *reinterpret_cast<const bf16x8*>(ap + 32 * r * a_pitch);
#pragma unroll
  for (int s = 0; s < NK; ++s) {
    if (s + PD < NK) w[(s + PD) % (PD + 1)] =
        *reinterpret_cast<const bf16x8*>(wp + 512 * (s + PD));
    if (s + 1 < NK) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
        an[r] = *reinterpret_cast<const bf16x8*>(ap + 32 * r * a_pitch + 16 * (s + 1));
    }
    // keep the loads above ahead of this slice's MFMAs: left alone, the scheduler sinks each
    // weight load next to its use and waits out a full L2 round trip every other slice
    if constexpr (PIN) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = mfma(w[s % (PD + 1)], a[r], acc[r]);
#pragma unroll
    for (int r = 0; r < NR; ++r) a[r] = an[r];
  }
}

// accumulators start at the layer's bias: element e of a tile is unit u0 + 8(e/4) + 4(lane/32) + e%4
template <int NR>
__device__ __forceinline__ void init_bias(f32x16 (&acc)[NR], const float* __restrict__ bias, int u0,
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

// tanh, rounded to bf16, 4 consecutive units per 8-byte LDS store at Hs[row][unit]
template <int NR>
__device__ __forceinline__ void store_tanh(const f32x16 (&acc)[NR], __bf16* Hs, int u0, int lane) {
  const int lr = lane & 31, lh = (lane >> 5) * 4;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int unit = u0 + 8 * g + lh;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      bf16x4 v;
      v[0] = (__bf16)tanh_act(acc[r][4 * g + 0]);
      v[1] = (__bf16)tanh_act(acc[r][4 * g + 1]);
      v[2] = (__bf16)tanh_act(acc[r][4 * g + 2]);
      v[3] = (__bf16)tanh_act(acc[r][4 * g + 3]);
      *reinterpret_cast<bf16x4*>(Hs + (32 * r + lr) * kHPitch + unit) = v;
    }
  }
}

}  // namespace f16pol
