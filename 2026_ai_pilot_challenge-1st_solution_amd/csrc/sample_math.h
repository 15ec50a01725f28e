// sample_math.h -- softmax numerators for the categorical draw, from IEEE basic operations only,
// so that the draw is reproducible bit-for-bit by any IEEE-754 single-precision implementation of
// the same expression sequence (compiled without contraction).
//
// e^x for x <= 0: Cody-Waite reduction x = n ln2 + r with ln2 split into a 16-bit head (n * head
// exact for |n| < 256) and a tail, |r| <= ln2/2, each step one fused multiply-add; e^r by its
// degree-7 Taylor polynomial in Horner form, one fma per degree (truncation < 2e-8 relative);
// scaling by 2^n with ldexp.  Below -87, 0.  fmaf is exactly rounded on every IEEE
// implementation, so the sequence stays reproducible.
#pragma once

#include <math.h>

#ifndef F16_HD
#define F16_HD __host__ __device__ __forceinline__
#endif

namespace f16rng {

F16_HD float exp_nonpos(float x0) {
  const bool in = x0 >= -87.0f;                      // false below -87 and for NaN
  const float x = in ? x0 : 0.0f;                    // selects, not a branch per call
  const float n = rintf(x * 1.44269504f);
  const float r = fmaf(-n, 1.42860677e-6f, fmaf(-n, 0.693145751953125f, x));
  float p = fmaf(1.0f / 5040.0f, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return in ? ldexpf(p, (int)n) : 0.0f;
}

}  // namespace f16rng
