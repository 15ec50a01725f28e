// opcount.hpp -- a counting stand-in for `double`, used to build an instrumented copy of the C
// restatement (f16_oracle.c) that tallies the floating-point operations of the flight model.
// TEST INFRASTRUCTURE ONLY (the FLOP-count fixture, tests/golden/make_flops_golden.py).
//
// Convention (the static count it replaces, 1,550 per aircraft-substep): every add, subtract,
// multiply, divide and square root counts one; every other libm call (sin, cos, atan2, exp,
// pow, ...) counts one and is tallied separately; negation, fabs, comparisons, min/max
// selects and conversions count nothing (compares are tallied for information).  Operations
// between two compile-time constants fold away and are not counted, as in the source.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <cmath>

struct OpCounts {
  unsigned long long add, sub, mul, div, sqrt, libm, cmp;
};
extern thread_local OpCounts g_ops;

struct OpDouble {
  double v;
  OpDouble() = default;
  constexpr OpDouble(double x) : v(x) {}
  constexpr OpDouble(float x) : v(x) {}
  constexpr OpDouble(int x) : v(x) {}
  constexpr OpDouble(long x) : v((double)x) {}
  constexpr OpDouble(unsigned x) : v(x) {}
  constexpr OpDouble(unsigned long x) : v((double)x) {}
  constexpr OpDouble(long long x) : v((double)x) {}
  explicit constexpr operator double() const { return v; }
  explicit constexpr operator int() const { return (int)v; }
  explicit constexpr operator long() const { return (long)v; }
  explicit constexpr operator unsigned() const { return (unsigned)v; }
  explicit constexpr operator bool() const { return v != 0.0; }
  OpDouble& operator+=(OpDouble o) { ++g_ops.add; v += o.v; return *this; }
  OpDouble& operator-=(OpDouble o) { ++g_ops.sub; v -= o.v; return *this; }
  OpDouble& operator*=(OpDouble o) { ++g_ops.mul; v *= o.v; return *this; }
  OpDouble& operator/=(OpDouble o) { ++g_ops.div; v /= o.v; return *this; }
};
static_assert(sizeof(OpDouble) == sizeof(double), "layout-compatible with double");

inline OpDouble operator+(OpDouble a, OpDouble b) { ++g_ops.add; return OpDouble(a.v + b.v); }
inline OpDouble operator-(OpDouble a, OpDouble b) { ++g_ops.sub; return OpDouble(a.v - b.v); }
inline OpDouble operator*(OpDouble a, OpDouble b) { ++g_ops.mul; return OpDouble(a.v * b.v); }
inline OpDouble operator/(OpDouble a, OpDouble b) { ++g_ops.div; return OpDouble(a.v / b.v); }
inline OpDouble operator-(OpDouble a) { return OpDouble(-a.v); }
inline OpDouble operator+(OpDouble a) { return a; }
#define OPC_CMP(op)                                                                   \
  inline bool operator op(OpDouble a, OpDouble b) { ++g_ops.cmp; return a.v op b.v; }
OPC_CMP(<) OPC_CMP(>) OPC_CMP(<=) OPC_CMP(>=) OPC_CMP(==) OPC_CMP(!=)
#undef OPC_CMP

inline OpDouble sqrt(OpDouble a) { ++g_ops.sqrt; return OpDouble(std::sqrt(a.v)); }
#define OPC_LIBM1(f) inline OpDouble f(OpDouble a) { ++g_ops.libm; return OpDouble(std::f(a.v)); }
OPC_LIBM1(sin) OPC_LIBM1(cos) OPC_LIBM1(tan) OPC_LIBM1(asin) OPC_LIBM1(acos) OPC_LIBM1(atan)
OPC_LIBM1(exp) OPC_LIBM1(log) OPC_LIBM1(log10) OPC_LIBM1(tanh) OPC_LIBM1(cbrt)
#undef OPC_LIBM1
inline OpDouble atan2(OpDouble a, OpDouble b) { ++g_ops.libm; return OpDouble(std::atan2(a.v, b.v)); }
inline OpDouble pow(OpDouble a, OpDouble b) { ++g_ops.libm; return OpDouble(std::pow(a.v, b.v)); }
inline OpDouble fmod(OpDouble a, OpDouble b) { ++g_ops.libm; return OpDouble(std::fmod(a.v, b.v)); }
inline OpDouble fabs(OpDouble a) { return OpDouble(std::fabs(a.v)); }
inline OpDouble floor(OpDouble a) { return OpDouble(std::floor(a.v)); }
inline OpDouble ceil(OpDouble a) { return OpDouble(std::ceil(a.v)); }
inline OpDouble fmin(OpDouble a, OpDouble b) { ++g_ops.cmp; return OpDouble(std::fmin(a.v, b.v)); }
inline OpDouble fmax(OpDouble a, OpDouble b) { ++g_ops.cmp; return OpDouble(std::fmax(a.v, b.v)); }
inline OpDouble copysign(OpDouble a, OpDouble b) { return OpDouble(std::copysign(a.v, b.v)); }
inline bool isfinite(OpDouble a) { return std::isfinite(a.v); }
inline bool isnan(OpDouble a) { return std::isnan(a.v); }

// from here on, the restatement's `double` is the counting type
#define double OpDouble
