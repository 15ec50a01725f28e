// fdm_math.h -- short-latency fp64 division, reciprocal, square root, exp and log for the
// dependency chains of the FDM kernels, and the finite-flag accumulator (the FDM's
// precision-specific primitives; fdm_math_f32.h holds the single-precision ones).
//
// Each FDM role runs one wavefront per SIMD, so nothing hides the latency of a dependent
// operation: every division, square root or transcendental on a chain costs its full latency.
// Measured on gfx950 (one wavefront per SIMD, clocks per dependent step): IEEE division 73,
// sqrt 114, exp 116, log 418; the hardware reciprocal and reciprocal square root
// (v_rcp_f64 / v_rsq_f64, relative error <= 5e-8) 27.  The forms below start from those two
// instructions and refine with fused multiply-adds:
//   fm_rcp   Newton-Raphson twice:  r += r (1 - b r)                           (~1 ulp)
//   fm_div   a * fm_rcp(b), then one residual step q += r (a - b q)            (~0.5 ulp;
//            identical to IEEE division on 1M random normal operands)
//   fm_sqrt  Goldschmidt: g = x y, h = y / 2, one coupled step, then one residual step
//            g += h (x - g g)                       (~0.5 ulp for normal x; a subnormal x loses
//            relative accuracy, to ~1e-14, as the residual g g underflows -- the model's square
//            roots are of sums of squares of physical quantities, nowhere near that range)
//   fm_exp   Cody-Waite reduction x = k ln2 + r, |r| <= ln2 / 2, Taylor series of degree 13
//            (truncation < 5e-18 relative) evaluated by Estrin's scheme, scaled by 2^k
//   fm_log   x = 2^k m, m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(s), s = (m - 1) / (m + 1),
//            |s| <= 0.1716, odd series through s^21 (truncation < 3e-17 relative), Estrin
// Every form keeps the IEEE result on the special operands the model can meet (a zero or
// infinite square-root argument, NaN propagating through all of them); division and
// reciprocal assume a finite non-zero divisor whose reciprocal is a normal number, which
// every call site guarantees.  The CPU restatement uses the C library; these forms differ
// from it by at most a couple of roundings per call, far inside the per-step tolerance.
#pragma once

#include <hip/hip_runtime.h>

namespace f16 {

#define F16_DEV __device__ __forceinline__

F16_DEV double fm_rcp(double b) {
  double r = __builtin_amdgcn_rcp(b);
  double e = __builtin_fma(-b, r, 1.0);
  r = __builtin_fma(e, r, r);
  e = __builtin_fma(-b, r, 1.0);
  return __builtin_fma(e, r, r);
}

F16_DEV double fm_div(double a, double b) {
  const double r = fm_rcp(b);
  const double q = a * r;
  return __builtin_fma(__builtin_fma(-b, q, a), r, q);
}

F16_DEV double fm_sqrt(double x) {
  const double y = __builtin_amdgcn_rsq(x);
  double g = x * y, h = 0.5 * y;
  const double e = __builtin_fma(-g, h, 0.5);
  g = __builtin_fma(g, e, g);
  h = __builtin_fma(h, e, h);
  g = __builtin_fma(__builtin_fma(-g, g, x), h, g);
  // sqrt(+0) = +0 and sqrt(+inf) = +inf (the refinement would turn 0 * inf into NaN)
  return (x == 0.0 || x == __builtin_inf()) ? x : g;
}

F16_DEV double fm_exp(double x) {
  constexpr double kLog2e = 1.4426950408889634;        // 1 / ln 2
  constexpr double kLn2Hi = 6.93147180369123816490e-01; // ln 2 rounded to 32 bits: k * kLn2Hi is exact for abs(k) < 2^21
  constexpr double kLn2Lo = 1.90821492927058770002e-10; // ln 2 - kLn2Hi
  const double xc = __builtin_fmin(__builtin_fmax(x, -746.0), 710.0);
  const double k = __builtin_rint(xc * kLog2e);
  double r = __builtin_fma(-k, kLn2Hi, xc);
  r = __builtin_fma(-k, kLn2Lo, r);
  // Taylor coefficients 1/n!, n = 0..13, by Estrin's scheme
  const double r2 = r * r, r4 = r2 * r2, r8 = r4 * r4;
  const double p01 = 1.0 + r;
  const double p23 = __builtin_fma(r, 1.0 / 6.0, 0.5);
  const double p45 = __builtin_fma(r, 1.0 / 120.0, 1.0 / 24.0);
  const double p67 = __builtin_fma(r, 1.0 / 5040.0, 1.0 / 720.0);
  const double p89 = __builtin_fma(r, 1.0 / 362880.0, 1.0 / 40320.0);
  const double pab = __builtin_fma(r, 1.0 / 39916800.0, 1.0 / 3628800.0);
  const double pcd = __builtin_fma(r, 1.0 / 6227020800.0, 1.0 / 479001600.0);
  const double p03 = __builtin_fma(p23, r2, p01);
  const double p47 = __builtin_fma(p67, r2, p45);
  const double p8b = __builtin_fma(pab, r2, p89);
  const double p07 = __builtin_fma(p47, r4, p03);
  const double p8d = __builtin_fma(pcd, r4, p8b);
  const double p = __builtin_fma(p8d, r8, p07);
  const double y = __builtin_ldexp(p, (int)k);
  return x != x ? x : y;
}

F16_DEV double fm_log(double x) {
  constexpr double kLn2Hi = 6.93147180369123816490e-01;
  constexpr double kLn2Lo = 1.90821492927058770002e-10;
  constexpr double kSqrt2 = 1.4142135623730951;
  // subnormal arguments are scaled by 2^54 first so the exponent field is meaningful
  const bool sub = x < 2.2250738585072014e-308;
  const double xs = sub ? x * 18014398509481984.0 : x;
  const unsigned long long bits = __double_as_longlong(xs);
  int k = (int)((bits >> 52) & 0x7ff) - 1023 - (sub ? 54 : 0);
  double m = __longlong_as_double((long long)((bits & 0x000fffffffffffffULL) |
                                              0x3ff0000000000000ULL));   // [1, 2)
  const bool big = m >= kSqrt2;
  m = big ? 0.5 * m : m;
  k += big ? 1 : 0;
  const double s = fm_div(m - 1.0, m + 1.0);
  const double z = s * s;
  // log m = 2 s (1 + z/3 + z^2/5 + ... + z^10/21) = 2s + 2s z Q(z), Q by Estrin's scheme
  const double z2 = z * z, z4 = z2 * z2, z8 = z4 * z4;
  const double q01 = __builtin_fma(z, 1.0 / 5.0, 1.0 / 3.0);
  const double q23 = __builtin_fma(z, 1.0 / 9.0, 1.0 / 7.0);
  const double q45 = __builtin_fma(z, 1.0 / 13.0, 1.0 / 11.0);
  const double q67 = __builtin_fma(z, 1.0 / 17.0, 1.0 / 15.0);
  const double q89 = __builtin_fma(z, 1.0 / 21.0, 1.0 / 19.0);
  const double q03 = __builtin_fma(q23, z2, q01);
  const double q47 = __builtin_fma(q67, z2, q45);
  const double q07 = __builtin_fma(q47, z4, q03);
  const double q = __builtin_fma(q89, z8, q07);
  const double s2 = s + s;
  const double lm = __builtin_fma(s2 * z, q, s2);
  const double kd = (double)k;
  const double y = __builtin_fma(kd, kLn2Hi, __builtin_fma(kd, kLn2Lo, lm));
  // log(+0) = -inf, log(+inf) = +inf, negative or NaN -> NaN
  const double special = x == 0.0 ? -__builtin_inf() : (x == __builtin_inf() ? x : __builtin_nan(""));
  return (x > 0.0 && x < __builtin_inf()) ? y : special;
}

// Finite-flag accumulator: the largest IEEE exponent field seen (high word & 0x7ff00000); every
// value was finite iff the result is below kFinInf.  Two 32-bit VALU operations per value, no
// lane masks.
F16_DEV unsigned fin_acc(unsigned m, double x) {
  const unsigned hi = (unsigned)((unsigned long long)__double_as_longlong(x) >> 32);
  return max(m, hi & 0x7ff00000u);
}
constexpr unsigned kFinInf = 0x7ff00000u;

#undef F16_DEV

}  // namespace f16
