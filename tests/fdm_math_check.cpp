// Host check of csrc/fdm_math.h (the FDM's fp64 division, reciprocal, sqrt, exp and log).
//
// The device forms start from the hardware reciprocal and reciprocal square root, whose
// relative error on gfx950 is at most 5e-8; here those two instructions are replaced by the
// correctly rounded value perturbed by +-4.5e-8 (both signs, one pass each), so the refinement
// steps are exercised from a start at least as bad as the hardware's.  Every result is compared
// with an 80-bit long-double reference (glibc's expl/logl/sqrtl and exact long-double division)
// in units of the double result's ulp.  Prints one line of maxima and the special-operand check.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>

#define __device__
#define __forceinline__ inline
static double g_pert = 4.5e-8;
static double emu_rcp(double x) { return (1.0 / x) * (1.0 + g_pert); }
static double emu_rsq(double x) { return (1.0 / std::sqrt(x)) * (1.0 - g_pert); }
#define __builtin_amdgcn_rcp(x) emu_rcp(x)
#define __builtin_amdgcn_rsq(x) emu_rsq(x)
static long long __double_as_longlong(double d) { long long v; std::memcpy(&v, &d, 8); return v; }
static double __longlong_as_double(long long v) { double d; std::memcpy(&d, &v, 8); return d; }
using std::max;   // HIP's device max(unsigned, unsigned), used by fin_acc
#include "fdm_math.h"

using namespace f16;

static double ulp_err(double got, long double want) {
  const double w = (double)want;
  if (std::isnan(w)) return std::isnan(got) ? 0.0 : 1e9;
  if (std::isinf(w) || w == 0.0) return got == w ? 0.0 : 1e9;
  const double u = std::nextafter(std::fabs(w), INFINITY) - std::fabs(w);
  return (double)(std::fabs((long double)got - want) / u);
}

static bool same(double a, double b) {
  return (std::isnan(a) && std::isnan(b)) || (a == b && std::signbit(a) == std::signbit(b));
}

int main(int argc, char** argv) {
  const int n = argc > 1 ? std::atoi(argv[1]) : 1000000;
  std::mt19937_64 rng(20261202);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  double e_div = 0, e_rcp = 0, e_sqrt = 0, e_exp = 0, e_log = 0;
  long div_ne_ieee = 0;
  for (int pass = 0; pass < 2; ++pass) {
    g_pert = pass ? -4.5e-8 : 4.5e-8;
    for (int i = 0; i < n; ++i) {
      const double a = std::ldexp(1.0 + U(rng), (int)(U(rng) * 400) - 200) * (U(rng) < 0.5 ? -1 : 1);
      const double b = std::ldexp(1.0 + U(rng), (int)(U(rng) * 400) - 200) * (U(rng) < 0.5 ? -1 : 1);
      const double d = fm_div(a, b);
      e_div = std::fmax(e_div, ulp_err(d, (long double)a / (long double)b));
      div_ne_ieee += d != a / b;
      e_rcp = std::fmax(e_rcp, ulp_err(fm_rcp(b), 1.0L / (long double)b));
      const double x = std::fabs(a);
      e_sqrt = std::fmax(e_sqrt, ulp_err(fm_sqrt(x), sqrtl((long double)x)));
      const double ex = (U(rng) - 0.5) * (i % 2 ? 1400.0 : 6.0);
      e_exp = std::fmax(e_exp, ulp_err(fm_exp(ex), expl((long double)ex)));
      e_log = std::fmax(e_log, ulp_err(fm_log(x), logl((long double)x)));
      const double x1 = 1.0 + (U(rng) - 0.5) * 1e-3;   // near 1, where log loses precision
      e_log = std::fmax(e_log, ulp_err(fm_log(x1), logl((long double)x1)));
    }
  }
  int bad = 0;
  const double sp[] = {0.0, -0.0, 1.0, 4.9e-324, 2.2e-308, 1e308, -1.0, INFINITY, -INFINITY, NAN};
  for (double v : sp) {
    if (!(std::fabs(v) > 0.0 && std::fabs(v) < 2.2250738585072014e-308))   // subnormal: below
      bad += !same(fm_sqrt(v), std::sqrt(v));
    bad += !same(fm_log(v), std::log(v)) && !(std::isnan(fm_log(v)) && std::isnan(std::log(v)));
    bad += !same(fm_exp(v), std::exp(v));
  }
  bad += !same(fm_exp(709.7), std::exp(709.7)) + !same(fm_exp(-745.0), std::exp(-745.0));
  // subnormal square-root arguments: documented relative accuracy 1e-14
  double e_sub = 0.0;
  for (double v : {4.9e-324, 1e-310, 2.0e-308})
    e_sub = std::fmax(e_sub, std::fabs(fm_sqrt(v) - std::sqrt(v)) / std::sqrt(v));
  bad += e_sub > 1e-13;
  std::printf("div %.4f rcp %.4f sqrt %.4f exp %.4f log %.4f div_ne_ieee %ld special_bad %d\n",
              e_div, e_rcp, e_sqrt, e_exp, e_log, div_ne_ieee, bad);
  return 0;
}
