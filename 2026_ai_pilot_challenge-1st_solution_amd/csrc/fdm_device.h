// fdm_device.h -- device-side F-16 six-degree-of-freedom model for gfx950.
//
// One lane owns one aircraft.  Its integrator state lives in VGPRs for all substeps of a
// launch; the aero/engine/FCS/ISA tables are one flat image staged in LDS per workgroup.
// The model is the reference's JSBSim-v1.0.0 restatement (cuda_fdm/ref, model order of
// cuda_fdm/ref/jsb_fdm.py:212-244): propagate -> kinematics -> atmosphere -> mass -> FCS ->
// auxiliary -> engine -> aero -> gravity -> accelerations.
//
// Numerics.  All arithmetic is IEEE double with contraction disabled (-ffp-contract=off).
// Where the reference evaluates a trigonometric function of an angle that was itself produced
// by atan2/asin from a vector, this code uses the vector ratio directly (e.g. sin(atan2(z,rxy))
// = z/r, cos(alpha) = u/sqrt(u^2+w^2)); the angles are still produced wherever they are state
// or output.  These substitutions change results at the last-ulp level only (the per-step
// tolerance against the CPU restatement is 1e-10 relative).
#pragma once

#include <hip/hip_runtime.h>

#include "f16_model_gen.h"
#include "fdm_math.h"
#include "f16_state.h"

// Every model function is host+device so the identical algorithm can also be built for the CPU
// (debugging and unit checks); the kernels are the only production callers.
#define F16_HD __host__ __device__ __forceinline__

namespace f16 {

// ------------------------------------------------------------------ constants
constexpr double kDt = 1.0 / 60.0;                 // integration step (jsb_fdm.py:18)
constexpr double kRot = 0.00007292115;             // Earth rotation, rad/s (jsb_frames.py:14)
constexpr double kSemiMajor = 20925646.32546;      // WGS84 a, ft (jsb_frames.py:10)
constexpr double kGM = 14.0764417572E15;           // ft^3/s^2 (jsb_frames.py:12)
constexpr double kJ2 = 1.08262982E-03;             // (jsb_frames.py:13)
constexpr double kInToFt = 1.0 / 12;               // jsb_const.py:10
constexpr double kLbToSlug = 1.0 / 32.174049;      // jsb_const.py:13
constexpr double kEarthRadiusIsa = F16M_EARTH_RADIUS_ISA;
constexpr double kHbMac = 765.0;                   // aero/h_b-mac-ft (jsb_fdm.py:86)
constexpr double kGearForce = 0.30;                // externally forced gear position (jsb_fdm.py:84)

// ------------------------------------------------------------------ table interpolation
// Bracket for a 1-D table: value = f * (y[hi] - y[lo]) + y[lo].  Keys at or beyond the ends
// select the end value exactly (lo = hi, f = 0), as the reference's Table1D does.  The factor
// is (key - x[r-1]) times the interval's reciprocal width (stored in the image at `riv`), which
// differs from the reference's division by at most one rounding.
struct F16Br1 { int lo, hi; double f; };
// Bracket for one axis of a 2-D table: upper index r in [1, n-1] and the factor clamped to
// [0, 1] (the reference's Table2D has no end special case, so the clamped factor is kept).
struct F16Br2 { int r; double f; };

F16_HD F16Br1 f16_br1(const double* T, int off, int riv, int n, int r, double key,
                      double x0, double xn) {
  const double xl = T[off + r - 1];
  double f = (key - xl) * T[riv + r - 1];
  f = (f > 1.0) ? 1.0 : f;
  F16Br1 b;
  const bool lo_end = key <= x0, hi_end = key >= xn;
  b.lo = lo_end ? 0 : (hi_end ? n - 1 : r - 1);
  b.hi = lo_end ? 0 : (hi_end ? n - 1 : r);
  b.f = (lo_end || hi_end) ? 0.0 : f;
  return b;
}

F16_HD F16Br2 f16_br2(const double* T, int off, int riv, int r, double key) {
  const double xl = T[off + r - 1];
  double f = (key - xl) * T[riv + r - 1];
  f = (f > 1.0) ? 1.0 : ((f < 0.0) ? 0.0 : f);
  F16Br2 b;
  b.r = r;
  b.f = f;
  return b;
}

F16_HD double f16_lerp1(const double* T, int off, const F16Br1& b) {
  const double ylo = T[off + b.lo], yhi = T[off + b.hi];
  return b.f * (yhi - ylo) + ylo;
}

F16_HD double f16_lerp2(const double* T, int off, int nc, const F16Br2& br,
                                            const F16Br2& bc) {
  const int i0 = off + (br.r - 1) * nc + bc.r - 1;
  const double d00 = T[i0], d01 = T[i0 + 1], d10 = T[i0 + nc], d11 = T[i0 + nc + 1];
  const double col1 = br.f * (d10 - d00) + d00;
  const double col2 = br.f * (d11 - d01) + d01;
  return col1 + bc.f * (col2 - col1);
}

#include "f16_grid_gen.inc"
#include "f16_aero_gen.inc"

#define F16_BR1_(g, key)                                                                    \
  f16_br1(T, F16M_##g##_OFF, F16M_##g##_RIV, F16M_##g##_LEN, f16m_upper_##g(key), (key),        \
          F16M_##g##_X0, F16M_##g##_XN)
#define F16_BR1(g, key) F16_BR1_(g, key)
#define F16_BR2_(g, key) f16_br2(T, F16M_##g##_OFF, F16M_##g##_RIV, f16m_upper_##g(key), (key))
#define F16_BR2(g, key) F16_BR2_(g, key)

// ------------------------------------------------------------------ small helpers
F16_HD double clampd(double x, double lo, double hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// |a-b| <= 1e-9 * max(1, |a|, |b|)  (jsb_fcs.py:28-30)
F16_HD bool near_equal(double a, double b) {
  double m = 1.0;
  const double fa = fabs(a), fb = fabs(b);
  m = fa > m ? fa : m;
  m = fb > m ? fb : m;
  return fabs(a - b) <= 1e-9 * m;
}

// Rate-limited actuator with two detents (lo, hi) and one travel time t: the general
// kinematic (jsb_fcs.py:42-78) always brackets into segment 1 for two detents, so it reduces to
// one clipped step of at most dt0.
F16_HD double kinemat2(double input, double output, double lo, double hi,
                                           double t, double dt0) {
  input = clampd(input * hi, lo, hi);
  if (dt0 > 0.0 && !near_equal(input, output)) {
    const double rate = (hi - lo) / t;
    const double this_in = clampd(input, lo, hi);
    // dt0 < |this_in - output| / rate, without the division (a constant product for the
    // callers' literal arguments)
    if (dt0 * rate < fabs(this_in - output))
      output = (output < input) ? output + dt0 * rate : output - dt0 * rate;
    else
      output = this_in;
  }
  return output;
}

// Trailing-edge-flap kinematic: detents (-1, 0, 1), times (3, 0, 3).  Same loop as the
// reference with an iteration cap; three passes always suffice for three detents.
F16_HD double kinemat_tef(double input, double output, double dt0) {
  const double det[3] = {-1.0, 0.0, 1.0}, tim[3] = {3.0, 0.0, 3.0};
  input = clampd(input * det[2], det[0], det[2]);
  for (int it = 0; it < 4 && dt0 > 0.0 && !near_equal(input, output); ++it) {
    int ind = 1;
    const bool down = input < output;
    if (down ? (det[1] < output) : (det[1] <= output)) ind = 2;
    const double dlo = ind == 1 ? det[0] : det[1], dhi = ind == 1 ? det[1] : det[2];
    const double t = ind == 1 ? tim[1] : tim[2];
    if (t <= 0.0) { output = input; break; }
    const double rate = (dhi - dlo) / t;
    const double this_in = clampd(input, dlo, dhi);
    double this_dt = fabs((this_in - output) / rate);
    if (dt0 < this_dt) {
      this_dt = dt0;
      output = (output < input) ? output + this_dt * rate : output - this_dt * rate;
    } else {
      output = this_in;
    }
    dt0 -= this_dt;
  }
  return output;
}

// AEROSURFACE_SCALE, zero-centred (jsb_fcs.py:107-113)
F16_HD double surface_scale(double in, double in_min, double in_max,
                                                double out_min, double out_max) {
  if (in == 0.0) return 0.0;
  return in > 0.0 ? (in / in_max) * out_max : (in / in_min) * out_min;
}

F16_HD double seek(double v, double target, double accel, double decel) {
  if (v > target) {
    v -= kDt * decel;
    v = v < target ? target : v;
  } else if (v < target) {
    v += kDt * accel;
    v = v > target ? target : v;
  }
  return v;
}

// ------------------------------------------------------------------ register-resident state
// The 66 state doubles a substep reads.  The remaining 35 of the 101 are outputs only
// (history slots, PID input_prev2, the rudder and gear kinematic outputs) and are written by
// the kernel straight to memory.
struct Aircraft {
  double p[3], v[3], q[4], wi[3], epa, fuel;
  double ai[3], wdi[3], qd[4];
  double vh1[3], vh2[3];   // velocity history slots 0 and 1 at substep start
  double ah1[3];           // acceleration history slot 0 at substep start
  double pba[3], ppd[3], ppq[3];
  double pa[9];            // alpha, mach, vc_kts, vg_fps, n_py, n_pz, p, q, r (previous frame)
  double n1, n2, n2n, ff;
  double k_tef, k_ail, k_ele, k_lef;
  double pid_ip[3], pid_io[3];
};

// Per-substep results that are not carried state.
struct SubstepOut {
  double k_rud, k_gear;
  double euler[3], uvw[3];
  double alpha, beta, mach, vt, alt;
};

// Atmosphere at geometric altitude h (ft): jsb_atmos.py:43-111.
struct Atmos { double T, P, rho, a, sigma, densalt; };

F16_HD Atmos isa(double h, const double* T) {
  constexpr double kER = kEarthRadiusIsa;
  constexpr double lapse[8] = F16M_ATM_LAPSE_INIT;
  constexpr double alts[9] = F16M_ATM_ALT_INIT;
  constexpr double temps[9] = F16M_ATM_TMP_INIT;
  constexpr double dbrk[9] = F16M_ATM_DBRK_INIT;
  Atmos o;
  const double gp = fm_div(h * kER, kER + h);
  if (gp >= 0.0) {
    const F16Br1 b = F16_BR1(F16M_TG_ISA_TEMP_R, gp);
    o.T = f16_lerp1(T, F16M_T_ISA_TEMP_OFF, b);
  } else {
    o.T = temps[0] + gp * lapse[0];
  }
  // pressure layer: first b with gp < alt[b+1] (b <= 7).  pow(Tb / (Tb + L dH), g0 M / (R* L))
  // is exp(e * log(1 + (L / Tb) dH)); an isothermal layer is exp(e * dH).  Both forms are
  // evaluated with one log and one exp for every lane.
  int b = 0;
#pragma unroll
  for (int i = 1; i < 8; ++i) b += !(gp < alts[i]);
  const double* lb = T + F16M_ATM_LAYER_OFF + F16M_ATM_LAYER_STRIDE * b;
  const double dH = gp - lb[0];
  const double kb = lb[2];
  const double lg = fm_log(1.0 + kb * dH);
  o.P = lb[1] * fm_exp(lb[3] * (kb != 0.0 ? lg : dH));
  o.rho = fm_div(o.P, F16M_RENG * o.T);
  o.a = fm_sqrt(F16M_GAMMA_R * o.T);
  o.sigma = o.rho * (1.0 / F16M_RHO_SL);
  // density altitude: first d with rho >= dbrk[d+1]; pow(rho / rb, x) is exp(x log(rho / rb))
  int d = 0;
#pragma unroll
  for (int i = 1; i < 8; ++i) d += !(o.rho >= dbrk[i]);
  const double* ld = T + F16M_ATM_LAYER_OFF + F16M_ATM_LAYER_STRIDE * d;
  const double lr = fm_log(o.rho * ld[5]);
  const double xd = ld[6];
  const double da = ld[4] + ld[7] * (xd != 0.0 ? fm_exp(xd * lr) - 1.0 : lr);
  o.densalt = fm_div(da * kER, kER - da);
  return o;
}

// Mass, CG, inertia and its inverse for a fuel load (jsb_massbalance.py:49-83); the two
// internal tanks share the fuel equally.
struct Mass { double cg[3], mass, J[6], Jinv[6], rp[3]; };   // J, Jinv: xx yy zz xy xz yz (symmetric)

F16_HD void add_pointmass(double m, double rx, double ry, double rz,
                                              const double cg[3], double mJ[3][3]) {
  const double vx = kInToFt * (cg[0] - rx), vy = kInToFt * (ry - cg[1]), vz = kInToFt * (cg[2] - rz);
  const double sx = m * vx, sy = m * vy, sz = m * vz;
  const double xx = sx * vx, yy = sy * vy, zz = sz * vz;
  const double xy = -sx * vy, xz = -sx * vz, yz = -sy * vz;
  mJ[0][0] = mJ[0][0] + (yy + zz); mJ[0][1] = mJ[0][1] + xy; mJ[0][2] = mJ[0][2] + xz;
  mJ[1][0] = mJ[1][0] + xy; mJ[1][1] = mJ[1][1] + (xx + zz); mJ[1][2] = mJ[1][2] + yz;
  mJ[2][0] = mJ[2][0] + xz; mJ[2][1] = mJ[2][1] + yz; mJ[2][2] = mJ[2][2] + (xx + yy);
}

F16_HD Mass mass_props(double fuel) {
  constexpr double ew = F16M_EMPTYWT, pw = F16M_PILOT_WT;
  constexpr double bcg[3] = {F16M_BASECG_X, F16M_BASECG_Y, F16M_BASECG_Z};
  constexpr double pl[3] = {F16M_PILOT_X, F16M_PILOT_Y, F16M_PILOT_Z};
  constexpr double t0l[3] = {F16M_TANK0_X, F16M_TANK0_Y, F16M_TANK0_Z};
  constexpr double t1l[3] = {F16M_TANK1_X, F16M_TANK1_Y, F16M_TANK1_Z};
  Mass o;
  const double t = fuel / 2.0;
  const double weight = ew + (t + t) + pw;
  const double iw = fm_rcp(weight);
#pragma unroll
  for (int i = 0; i < 3; ++i)
    o.cg[i] = (ew * bcg[i] + pw * pl[i] + t * t0l[i] + t * t1l[i]) * iw;
  double mJ[3][3] = {{F16M_IXX, -F16M_IXY, F16M_IXZ},
                     {-F16M_IXY, F16M_IYY, -F16M_IYZ},
                     {F16M_IXZ, -F16M_IYZ, F16M_IZZ}};
  add_pointmass(kLbToSlug * ew, bcg[0], bcg[1], bcg[2], o.cg, mJ);
  add_pointmass(kLbToSlug * pw, pl[0], pl[1], pl[2], o.cg, mJ);
  const double mt = kLbToSlug * t;
  add_pointmass(mt, t0l[0], t0l[1], t0l[2], o.cg, mJ);
  add_pointmass(mt, t1l[0], t1l[1], t1l[2], o.cg, mJ);
  const double Ixx = mJ[0][0], Iyy = mJ[1][1], Izz = mJ[2][2];
  const double Ixy = -mJ[0][1], Ixz = -mJ[0][2], Iyz = -mJ[1][2];
  double k1 = Iyy * Izz - Iyz * Iyz, k2 = Iyz * Ixz + Ixy * Izz, k3 = Ixy * Iyz + Iyy * Ixz;
  const double den = fm_rcp(Ixx * k1 - Ixy * k2 - Ixz * k3);
  k1 *= den; k2 *= den; k3 *= den;
  o.Jinv[0] = k1; o.Jinv[1] = (Izz * Ixx - Ixz * Ixz) * den; o.Jinv[2] = (Ixx * Iyy - Ixy * Ixy) * den;
  o.Jinv[3] = k2; o.Jinv[4] = k3; o.Jinv[5] = (Ixy * Ixz + Iyz * Ixx) * den;
  o.J[0] = Ixx; o.J[1] = Iyy; o.J[2] = Izz; o.J[3] = -Ixy; o.J[4] = -Ixz; o.J[5] = -Iyz;
  o.mass = kLbToSlug * weight;
  o.rp[0] = kInToFt * (o.cg[0] - F16M_AERORP_X);
  o.rp[1] = kInToFt * (F16M_AERORP_Y - o.cg[1]);
  o.rp[2] = kInToFt * (o.cg[2] - F16M_AERORP_Z);
  return o;
}

// Pitot total pressure and its inverse (jsb_auxiliary.py:20-42) -> calibrated airspeed, ft/s.
F16_HD double vcal_from_mach(double mach, double p) {
  double pt;
  if (mach < 0.0) {
    pt = p;
  } else if (mach < 1.0) {
    const double m2 = 1.0 + 0.2 * mach * mach;   // m2^3.5 = m2^3 sqrt(m2)
    pt = p * (m2 * m2 * m2 * fm_sqrt(m2));
  } else {
    const double m2 = mach * mach, m7 = m2 * m2 * m2 * mach, d = 7.0 * m2 - 1.0;
    pt = fm_div(p * 166.92158009316827 * m7, d * d * fm_sqrt(d));
  }
  const double qc = pt - p;
  const double A = qc * (1.0 / 2116.228) + 1.0;  // StdDaySLpressure (jsb_const.py:24)
  double M = fm_sqrt(5.0 * (fm_exp(fm_log(A) * (1.0 / 3.5)) - 1.0));
  if (M > 1.0) {
    for (int i = 0; i < 10; ++i) {
      const double t = 1.0 - fm_rcp(7.0 * M * M);
      M = 0.8812848543473311 * fm_sqrt(A * (t * t * fm_sqrt(t)));
    }
  }
  return F16M_STD_SL_SOUNDSPEED * M;
}



// ------------------------------------------------------------------ kinematics
// Frames derived from the ECI state (FDM._kinematics_from_state, jsb_fdm.py:121-140).
struct Kin {
  double ce, se;              // cos/sin of the Earth position angle
  double ex, ey, ez, radius, irad, sLat;
  double B[3][3];             // Ti2b: rows are the body axes in ECI
  double uvw[3], wpqr[3];     // body velocity w.r.t. the Earth, body rates w.r.t. the Earth
  double vn, ve;              // local north/east ground velocity
  double ctcp;                // cos(theta) * cos(phi) of the local-NED Euler angles
};

// Ti2b from the ECI->body quaternion (quat_to_T, jsb_frames.py): rows are the body axes in ECI.
// A pure function of q, so a caller may recompute it instead of keeping it live.
F16_HD void body_dcm(const double q[4], double B[3][3]) {
  const double q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
  const double q0q0 = q0 * q0, q1q1 = q1 * q1, q2q2 = q2 * q2, q3q3 = q3 * q3;
  const double q0q1 = q0 * q1, q0q2 = q0 * q2, q0q3 = q0 * q3;
  const double q1q2 = q1 * q2, q1q3 = q1 * q3, q2q3 = q2 * q3;
  B[0][0] = q0q0 + q1q1 - q2q2 - q3q3; B[0][1] = 2.0 * (q1q2 + q0q3); B[0][2] = 2.0 * (q1q3 - q0q2);
  B[1][0] = 2.0 * (q1q2 - q0q3); B[1][1] = q0q0 - q1q1 + q2q2 - q3q3; B[1][2] = 2.0 * (q2q3 + q0q1);
  B[2][0] = 2.0 * (q1q3 + q0q2); B[2][1] = 2.0 * (q2q3 - q0q1); B[2][2] = q0q0 - q1q1 - q2q2 + q3q3;
}

// `want_euler` (wave-uniform) also produces the Euler angles (mat_to_euler,
// jsb_frames.py:140-163) for the output row; the FCS only needs cos(theta)cos(phi), which is
// formed from the DCM without the inverse trigonometry.
F16_HD void kinematics(const double p[3], const double v[3], const double q[4],
                       const double wi[3], double ce, double se, bool want_euler, Kin& k,
                       double euler[3]) {
  k.ce = ce;
  k.se = se;
  k.ex = ce * p[0] + se * p[1];
  k.ey = ce * p[1] - se * p[0];
  k.ez = p[2];
  const double rxy2 = k.ex * k.ex + k.ey * k.ey;
  k.radius = fm_sqrt(rxy2 + k.ez * k.ez);
  const double rxy = fm_sqrt(rxy2);
  double sLon = 0.0, cLon = 1.0, sLat = 0.0, cLat = 1.0;
  if (rxy != 0.0) { const double ir = fm_rcp(rxy); sLon = k.ey * ir; cLon = k.ex * ir; }
  k.irad = fm_rcp(k.radius);
  if (k.radius != 0.0) { sLat = k.ez * k.irad; cLat = rxy * k.irad; }
  k.sLat = sLat;
  // local N, E, D axes in ECI (columns of Tl2i = Tec2i * Tl2ec; Tec2l rows from
  // location_derived, jsb_frames.py:48-51)
  const double n0 = -cLon * sLat, n1 = -sLon * sLat;
  const double d0 = -cLon * cLat, d1 = -sLon * cLat;
  const double N[3] = {ce * n0 - se * n1, se * n0 + ce * n1, cLat};
  const double E[2] = {ce * (-sLon) - se * cLon, se * (-sLon) + ce * cLon};
  const double D[3] = {ce * d0 - se * d1, se * d0 + ce * d1, -sLat};
  body_dcm(q, k.B);
  // Tl2b[i][j] = body_i . local_j
  double L[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    L[i][0] = k.B[i][0] * N[0] + k.B[i][1] * N[1] + k.B[i][2] * N[2];
    L[i][1] = k.B[i][0] * E[0] + k.B[i][1] * E[1];
    L[i][2] = k.B[i][0] * D[0] + k.B[i][1] * D[1] + k.B[i][2] * D[2];
  }
  // body velocity relative to the rotating Earth: Ti2b (v - omega x p)
  const double dv[3] = {v[0] + kRot * p[1], v[1] - kRot * p[0], v[2]};
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    k.uvw[i] = k.B[i][0] * dv[0] + k.B[i][1] * dv[1] + k.B[i][2] * dv[2];
    k.wpqr[i] = wi[i] - k.B[i][2] * kRot;   // vPQR = vPQRi - Ti2b * omega
  }
  k.vn = L[0][0] * k.uvw[0] + L[1][0] * k.uvw[1] + L[2][0] * k.uvw[2];
  k.ve = L[0][1] * k.uvw[0] + L[1][1] * k.uvw[1] + L[2][1] * k.uvw[2];
  const double d6 = L[0][2];
  const bool gimbal = d6 <= -1.0 || d6 >= 1.0;
  if (gimbal) {
    k.ctcp = 6.123233995736766e-17 * cos(atan2(-L[2][1], L[1][1]));   // cos(+-pi/2) in double
  } else {
    const double h = fm_sqrt(L[1][2] * L[1][2] + L[2][2] * L[2][2]);
    k.ctcp = fm_sqrt(1.0 - d6 * d6) * (h != 0.0 ? fm_div(L[2][2], h) : 1.0);
  }
  if (want_euler) {
    if (gimbal) {
      euler[1] = d6 <= -1.0 ? 0.5 * M_PI : -0.5 * M_PI;
      euler[0] = atan2(-L[2][1], L[1][1]);
      euler[2] = 0.0;
    } else {
      euler[1] = asin(-d6);
      euler[0] = atan2(L[1][2], L[2][2]);
      double ps = atan2(L[0][1], L[0][0]);
      euler[2] = ps < 0.0 ? ps + 2.0 * M_PI : ps;
    }
  }
}

// ------------------------------------------------------------------ force path components
// FDM._force_path (jsb_fdm.py:76-119): atmosphere -> mass -> FCS (previous-frame auxiliary
// values, current attitude) -> auxiliary -> engine -> aero -> gravity -> accelerations.  Each
// stage is a function of exactly what it reads, so the same arithmetic can run as one sequence
// (force_path) or spread over cooperating wavefronts (fdm_split.h) with identical results.

// ---- FCS (jsb_fcs.py:143-268) ----
struct FcsOut { double ail, elev, rud, lef, flap, k_rud; };
// Gear kinematic from its forced seed 0.30 toward command 0: one rate-limited step.
template <int FCS_RATE>
constexpr double kGearPos = kGearForce - (1.0 / (double)FCS_RATE) * ((1.0 - 0.0) / 5.0);

// Every channel that reads only previous-frame values: trailing-edge flap, roll loop, flaperon
// mix, yaw loop and rudder kinematic, leading-edge flap, and the pitch schedule (elevator
// command times the alpha schedule), which it returns.  Updates the FCS state in `a`.
template <int FCS_RATE>
F16_HD double fcs_prev_frame(Aircraft& a, double c_ail, double c_ele, double c_rud,
                             const double* __restrict__ T, FcsOut& o) {
  constexpr double fdt = 1.0 / (double)FCS_RATE;
  const double pa_alpha = a.pa[0], pa_mach = a.pa[1], vc = a.pa[2], vg = a.pa[3];
  const double tef_rad = (vc < 250.0) ? 0.349 : ((pa_mach > 0.9) ? -0.0349 : 0.0);
  const double tef = kinemat_tef(2.864789 * tef_rad, a.k_tef, fdt);
  a.k_tef = tef;
  // roll: PID (3, 5e-4, -1.25e-3), integrating only when its trigger is 0 (vc < 20 kt)
  const double rte = c_ail - 0.31821 * a.pa[6];
  double rpid;
  {
    const double ip = a.pid_ip[0];
    const double dval = (rte - ip) * (double)FCS_RATE;   // / fdt
    a.pid_io[0] += 0.00050 * fdt * ((vc < 20.0) ? (1.5 * rte - 0.5 * ip) : 0.0);
    a.pid_ip[0] = rte;
    rpid = 3.00000 * rte + a.pid_io[0] + -0.00125 * dval;
  }
  const double rrc = clampd(rpid + c_ail, -1.0, 1.0);
  o.ail = surface_scale(rrc, -1.0, 1.0, -0.375, 0.375);
  const double lapn = kinemat2(rrc, a.k_ail, -1.0, 1.0, 0.3, fdt);
  a.k_ail = lapn;
  const F16Br1 bm = F16_BR1(F16M_TG_FCS_AIL_SPEED_R, pa_mach);
  const double asc = f16_lerp1(T, F16M_T_FCS_AIL_SPEED_OFF, bm) * lapn;
  const double lf = clampd(-tef - asc, -1.0, 1.0), rf = clampd(tef - asc, -1.0, 1.0);
  o.flap = 1.4324 * (lf + rf);
  // pitch schedule
  const double ecl = clampd(c_ele + 0.0, -1.0, 0.44);
  const F16Br1 ba = F16_BR1(F16M_TG_FCS_ELEV_SCHED_R, pa_alpha);
  const double esch = f16_lerp1(T, F16M_T_FCS_ELEV_SCHED_OFF, ba) * ecl;
  // yaw: PID (0.1055, 1e-5, 5e-5) clipped to +-1, trigger 0 below 10 kt; its output seeds
  // the rudder kinematic
  const F16Br1 bv = F16_BR1(F16M_TG_FCS_YAW_RATE_R, vg);
  const double yrn = f16_lerp1(T, F16M_T_FCS_YAW_RATE_OFF, bv) * a.pa[8];
  const double yte = c_rud + yrn + 0.25 * a.pa[4];
  double ypid;
  {
    const double ip = a.pid_ip[2];
    const double dval = (yte - ip) * (double)FCS_RATE;
    a.pid_io[2] += 0.000010 * fdt * ((vc < 10.0) ? (1.5 * yte - 0.5 * ip) : 0.0);
    a.pid_ip[2] = yte;
    ypid = clampd(0.105500 * yte + a.pid_io[2] + 0.00005 * dval, -1.0, 1.0);
  }
  const double ysch = clampd(c_rud + 0.0 + ypid, -1.0, 1.0);
  const double rpn = kinemat2(ysch, ypid, -1.0, 1.0, 0.4, fdt);
  o.k_rud = rpn;
  o.rud = surface_scale(rpn, -1.0, 1.0, -0.524, 0.524);
  // leading-edge flap switch: the gear is never at 0 and weight-on-wheels is never set
  o.lef = (pa_alpha > 0.0873) ? 0.262 : ((pa_mach > 0.9) ? -0.0349 : 0.0);
  a.k_lef = kinemat2(2.293578 * o.lef, a.k_lef, -1.0, 1.0, 3.0, fdt);
  return esch;
}

// The pitch loop: g-load PID (0.3, 0.025, 0) clipped to +-1, trigger 0 below 5 kt, on the
// schedule plus the current attitude's gravity correction (cos(theta) cos(phi)).
template <int FCS_RATE>
F16_HD void fcs_pitch(Aircraft& a, double esch, double ctcp, FcsOut& o) {
  constexpr double fdt = 1.0 / (double)FCS_RATE;
  const double vc = a.pa[2];
  const double gcorr = a.pa[5] - ctcp;
  const double pte = esch + 6.2 * a.pa[7] - 0.020 * gcorr;
  double gpid;
  {
    const double ip = a.pid_ip[1];
    const double dval = (pte - ip) * (double)FCS_RATE;
    a.pid_io[1] += 0.0250 * fdt * ((vc < 5.0) ? (1.5 * pte - 0.5 * ip) : 0.0);
    a.pid_ip[1] = pte;
    gpid = clampd(0.3000 * pte + a.pid_io[1] + 0.0000 * dval, -1.0, 1.0);
  }
  const double psch = clampd(esch + 1.0472 * a.pa[0] + gpid, -1.0, 1.0);
  const double epn = kinemat2(psch, a.k_ele, -1.0, 1.0, 0.3, fdt);
  a.k_ele = epn;
  o.elev = surface_scale(epn, -1.0, 1.0, -0.436, 0.436);
}

// ---- auxiliary (jsb_auxiliary.py:45-73) ----
struct AuxGeo { double vt2, vt, alpha, beta, ca, sa, cb, sb; };

F16_HD AuxGeo aux_geometry(const double uvw[3]) {
  AuxGeo g;
  const double u = uvw[0], v = uvw[1], w = uvw[2];
  const double muw = u * u + w * w;
  g.vt2 = muw + v * v;
  g.vt = fm_sqrt(g.vt2);
  g.alpha = 0.0; g.beta = 0.0; g.ca = 1.0; g.sa = 0.0; g.cb = 1.0; g.sb = 0.0;
  if (g.vt > 0.001) {
    const double suw = fm_sqrt(muw), ivt = fm_rcp(g.vt);
    g.beta = atan2(v, suw);
    g.cb = suw * ivt;
    g.sb = v * ivt;
    if (muw >= 1e-6) {
      const double isuw = fm_rcp(suw);
      g.alpha = atan2(w, u);
      g.ca = u * isuw;
      g.sa = w * isuw;
    }
  }
  return g;
}

// Pilot-station load factors from the previous frame's body acceleration, angular
// acceleration and rates, about the current CG.
F16_HD void load_factors(const Aircraft& a, const double cg[3], double& npy, double& npz) {
  const double eye[3] = {kInToFt * (cg[0] - F16M_EYEPOINT_X), kInToFt * (F16M_EYEPOINT_Y - cg[1]),
                         kInToFt * (cg[2] - F16M_EYEPOINT_Z)};
  const double* wd = a.ppd;
  const double* wq = a.ppq;
  const double c1y = wd[2] * eye[0] - wd[0] * eye[2], c1z = wd[0] * eye[1] - wd[1] * eye[0];
  const double c2x = wq[1] * eye[2] - wq[2] * eye[1], c2y = wq[2] * eye[0] - wq[0] * eye[2];
  const double c2z = wq[0] * eye[1] - wq[1] * eye[0];
  const double c3y = wq[2] * c2x - wq[0] * c2z, c3z = wq[0] * c2y - wq[1] * c2x;
  npy = (a.pba[1] + c1y + c3y) * (1.0 / F16M_SLGRAVITY);
  npz = (a.pba[2] + c1z + c3z) * (1.0 / F16M_SLGRAVITY);
}

F16_HD double vc_knots(double mach, double P) {
  return (fabs(mach) > 0.0) ? vcal_from_mach(mach, P) * F16M_FPSTOKTS : 0.0;
}

// ---- engine (jsb_propulsion.py:89-128); throttle position = 2 * throttle command ----
// Updates the spool and fuel-flow state in `a`; returns the thrust, and the fuel burnt this
// step in `burn`.
F16_HD double engine(Aircraft& a, double c_thr, const Atmos& at, double mach,
                     const double* __restrict__ T, double& burn) {
  double thr = 2.0 * c_thr, aug = 0.0;
  if (thr > 1.0) { aug = thr - 1.0; thr -= aug; }
  // spool-time constants as the reference forms them: k * 90 / (bypass + 3)
  constexpr double d_up = 1.0 * 90.0 / (F16M_ENG_BYPASSRATIO + 3.0);
  constexpr double d_n2dn = 3.0 * 90.0 / (F16M_ENG_BYPASSRATIO + 3.0);
  constexpr double d_n1dn = 2.4 * 90.0 / (F16M_ENG_BYPASSRATIO + 3.0);
  const double nx = a.n2n + 0.1;
  const double om = 1.0 - (nx < 1.0 ? nx : 1.0);
  const double den = 1.0 + 3.0 * (om * om * om) + (1.0 - at.sigma);
  const double iden = fm_rcp(den);
  const double up = d_up * iden, n2dn = d_n2dn * iden, n1dn = d_n1dn * iden;
  a.n2 = seek(a.n2, F16M_ENG_IDLEN2 + thr * (F16M_ENG_MAXN2 - F16M_ENG_IDLEN2), up, n2dn);
  a.n1 = seek(a.n1, F16M_ENG_IDLEN1 + thr * (F16M_ENG_MAXN1 - F16M_ENG_IDLEN1), up, n1dn);
  a.n2n = (a.n2 - F16M_ENG_IDLEN2) * (1.0 / (F16M_ENG_MAXN2 - F16M_ENG_IDLEN2));
  const F16Br2 bm = F16_BR2(F16M_TG_ENG_IDLE_R, mach);
  const F16Br2 bd = F16_BR2(F16M_TG_ENG_IDLE_C, at.densalt);
  const F16Br2 bm2 = F16_BR2(F16M_TG_ENG_MIL_R, mach);
  const double idle = F16M_ENG_MILTHRUST * f16_lerp2(T, F16M_T_ENG_IDLE_OFF, F16M_T_ENG_IDLE_NC, bm, bd);
  const double mil = (F16M_ENG_MILTHRUST - idle) * f16_lerp2(T, F16M_T_ENG_MIL_OFF, F16M_T_ENG_MIL_NC, bm2, bd);
  double thrust = idle + mil * a.n2n * a.n2n;
  const double on = 1.0 - a.n2n;
  const double tsfc = F16M_ENG_TSFC * fm_sqrt(at.T * (1.0 / 389.7)) * (0.84 + on * on);
  a.ff = seek(a.ff, thrust * tsfc, 1000.0, 10000.0);
  a.ff = a.ff < F16M_IDLEFF ? F16M_IDLEFF : a.ff;
  if (aug > 0.0) {   // afterburner, AugMethod 2
    const F16Br2 bm3 = F16_BR2(F16M_TG_ENG_AUG_R, mach);
    const double tdiff = F16M_ENG_MAXTHRUST * f16_lerp2(T, F16M_T_ENG_AUG_OFF, F16M_T_ENG_AUG_NC, bm3, bd) - thrust;
    thrust += tdiff * aug;
    a.ff = seek(a.ff, thrust * F16M_ENG_ATSFC, 5000.0, 10000.0);
  }
  burn = a.ff * (kDt / 3600.0);
  return thrust;
}

// ---- aerodynamics (jsb_aero.py:75-107): 40 coefficient functions ----
F16_HD void aero_rates(double vt, double& bi2vel, double& ci2vel) {
  const double twovel = 2.0 * vt;
  const double i2v = twovel != 0.0 ? fm_rcp(twovel) : 0.0;
  bi2vel = F16M_BW * i2v;
  ci2vel = F16M_CBAR * i2v;
}
constexpr double kCLge = 1.0;   // kCLge(765 ft): beyond the table's last breakpoint (1.1 -> 1.0)

// Wind-axis aero forces to body forces, moments about the CG, then the engine's thrust at the
// structural origin.
F16_HD void forces_moments(const double ax[6], const AuxGeo& g, const Mass& mb, double thrust,
                           double F[3], double M[3]) {
  const double ca = g.ca, sa = g.sa, cb = g.cb, sb = g.sb;
  const double drag = -ax[0], side = ax[1], lift = -ax[2];
  F[0] = ca * cb * drag + (-ca * sb) * side + (-sa) * lift;
  F[1] = sb * drag + cb * side;
  F[2] = sa * cb * drag + (-sa * sb) * side + ca * lift;
  const double rx = mb.rp[0], ry = mb.rp[1], rz = mb.rp[2];
  M[0] = ax[3] + (ry * F[2] - rz * F[1]);
  M[1] = ax[4] + (rz * F[0] - rx * F[2]);
  M[2] = ax[5] + (rx * F[1] - ry * F[0]);
  const double mz = kInToFt * (mb.cg[2] - 0.0), my = kInToFt * (0.0 - mb.cg[1]);
  F[0] = F[0] + thrust;
  M[1] = M[1] + mz * thrust;
  M[2] = M[2] + (-my) * thrust;
}

// ---- J2 gravity (jsb_frames.py:69-80) ----
F16_HD void gravity(const Kin& k, double gi[3]) {
  const double adivr = kSemiMajor * k.irad;
  const double pc = 1.5 * kJ2 * adivr * adivr;
  const double s2 = k.sLat * k.sLat;   // sin(geocentric latitude) = z / r
  const double kxy = 1.0 + pc * (1.0 - 5.0 * s2), kz = 1.0 + pc * (3.0 - 5.0 * s2);
  const double g = -(kGM * k.irad * k.irad) * k.irad;
  const double gx = g * (kxy * k.ex), gy = g * (kxy * k.ey), gz = g * (kz * k.ez);
  gi[0] = k.ce * gx - k.se * gy;   // Tec2i * g_ecef
  gi[1] = k.se * gx + k.ce * gy;
  gi[2] = gz;
}

// ---- accelerations (jsb_accel.py:10-31) ----
struct Accel { double ai[3], wdi[3], pba[3], ppq[3]; };   // vUVWidot, vPQRidot, vBodyAccel, vPQRi

F16_HD void accelerations(const double B[3][3], const double wpqr[3], const Mass& mb,
                          const double F[3], const double M[3], const double gi[3], Accel& o) {
  double wq[3];   // vPQRi re-formed from vPQR, as the reference's accelerations do
#pragma unroll
  for (int i = 0; i < 3; ++i) wq[i] = wpqr[i] + B[i][2] * kRot;
  const double* J = mb.J;
  const double Jw0 = J[0] * wq[0] + J[3] * wq[1] + J[4] * wq[2];
  const double Jw1 = J[3] * wq[0] + J[1] * wq[1] + J[5] * wq[2];
  const double Jw2 = J[4] * wq[0] + J[5] * wq[1] + J[2] * wq[2];
  const double m0 = M[0] - (wq[1] * Jw2 - wq[2] * Jw1);
  const double m1 = M[1] - (wq[2] * Jw0 - wq[0] * Jw2);
  const double m2 = M[2] - (wq[0] * Jw1 - wq[1] * Jw0);
  const double* Ji = mb.Jinv;
  o.wdi[0] = Ji[0] * m0 + Ji[3] * m1 + Ji[4] * m2;
  o.wdi[1] = Ji[3] * m0 + Ji[1] * m1 + Ji[5] * m2;
  o.wdi[2] = Ji[4] * m0 + Ji[5] * m1 + Ji[2] * m2;
  const double sm = fm_rcp(mb.mass);
#pragma unroll
  for (int i = 0; i < 3; ++i) o.pba[i] = F[i] * sm;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    o.ai[i] = (B[0][i] * o.pba[0] + B[1][i] * o.pba[1] + B[2][i] * o.pba[2]) + gi[i];
    o.ppq[i] = wq[i];
  }
}

// ---- propagate: quaternion rect-Euler + normalize, vPQRi rect-Euler, ECI position AB3 on the
// velocity history, ECI velocity AB2 on the acceleration history, Earth position angle ----
F16_HD void propagate(Aircraft& a) {
  {
    double q0 = a.q[0] + kDt * a.qd[0], q1 = a.q[1] + kDt * a.qd[1];
    double q2 = a.q[2] + kDt * a.qd[2], q3 = a.q[3] + kDt * a.qd[3];
    const double mag = fm_sqrt(q0 * q0 + q1 * q1 + q2 * q2 + q3 * q3);
    if (mag != 0.0) {
      const double inv = fm_rcp(mag);
      q0 = q0 * inv; q1 = q1 * inv; q2 = q2 * inv; q3 = q3 * inv;
    }
    a.q[0] = q0; a.q[1] = q1; a.q[2] = q2; a.q[3] = q3;
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    a.wi[i] = a.wi[i] + kDt * a.wdi[i];
    const double v0 = a.v[i];
    a.p[i] = a.p[i] + (kDt / 12.0) * (23.0 * v0 - 16.0 * a.vh1[i] + 5.0 * a.vh2[i]);
    a.v[i] = v0 + kDt * (1.5 * a.ai[i] - 0.5 * a.ah1[i]);
    a.vh2[i] = a.vh1[i];
    a.vh1[i] = v0;
    a.ah1[i] = a.ai[i];
  }
  a.epa += kRot * kDt;
}

// Quaternion derivative for the next step (quat_qdot, jsb_frames.py:170-176).
F16_HD void quat_rate(Aircraft& a) {
  const double p = a.wi[0], qq = a.wi[1], r = a.wi[2];
  const double q0 = a.q[0], q1 = a.q[1], q2 = a.q[2], q3 = a.q[3];
  a.qd[0] = -0.5 * (q1 * p + q2 * qq + q3 * r);
  a.qd[1] = 0.5 * (q0 * p - q3 * qq + q2 * r);
  a.qd[2] = 0.5 * (q3 * p + q0 * qq - q1 * r);
  a.qd[3] = 0.5 * (-q2 * p + q1 * qq + q0 * r);
}

// Frames at the propagated state; sin/cos of the Earth position angle are evaluated every step
// (a rotation recurrence would bias cos by one rounding per step, which the altitude-dependent
// terms amplify).
F16_HD void frames(const Aircraft& a, bool want_euler, Kin& k, double euler[3]) {
  double ce, se;
  sincos(a.epa, &se, &ce);
  kinematics(a.p, a.v, a.q, a.wi, ce, se, want_euler, k, euler);
}

// ------------------------------------------------------------------ force path (one lane)
struct ForceOut {
  double ai[3], wdi[3], pba[3], ppq[3];   // vUVWidot, vPQRidot, vBodyAccel, vPQRi
  double alpha, beta, vt, mach, vc_kts, vg, npy, npz;
  double fuel_burn, alt, k_rud;
};

template <int FCS_RATE>
F16_HD void force_path(Aircraft& a, double c_ail, double c_ele, double c_rud,
                       double c_thr, const Kin& k, const double* __restrict__ T, ForceOut& o) {
  const double alt = k.radius - kSemiMajor;
  const Atmos at = isa(alt, T);
  const Mass mb = mass_props(a.fuel);
  FcsOut fc;
  const double esch = fcs_prev_frame<FCS_RATE>(a, c_ail, c_ele, c_rud, T, fc);
  fcs_pitch<FCS_RATE>(a, esch, k.ctcp, fc);
  o.k_rud = fc.k_rud;
  const AuxGeo g = aux_geometry(k.uvw);
  const double qbar = 0.5 * at.rho * g.vt2;
  const double mach = fm_div(g.vt, at.a);
  load_factors(a, mb.cg, o.npy, o.npz);
  o.vc_kts = vc_knots(mach, at.P);
  o.vg = fm_sqrt(k.vn * k.vn + k.ve * k.ve);
  o.alpha = g.alpha; o.beta = g.beta; o.vt = g.vt; o.mach = mach; o.alt = alt;
  const double thrust = engine(a, c_thr, at, mach, T, o.fuel_burn);
  double ax[6];
  {
    const double alpha = g.alpha, beta = g.beta;
    double bi2vel, ci2vel;
    aero_rates(g.vt, bi2vel, ci2vel);
    constexpr double kclge = kCLge;
    constexpr double gear = kGearPos<FCS_RATE>;
    const double p = k.wpqr[0], q = k.wpqr[1], r = k.wpqr[2];
    const double ail = fc.ail, elev = fc.elev, rud = fc.rud, lef = fc.lef, flap = fc.flap;
    F16_AERO_BRACKETS;
    F16_AERO_LOOKUPS;
    // each axis as SCALE * (EARLY + LATE), the EARLY sums rounded first exactly as the split
    // kernel forms them a phase ahead
    const double e0 = F16_AERO_DRAG_EARLY, e1 = F16_AERO_SIDE_EARLY, e2 = F16_AERO_LIFT_EARLY;
    const double e3 = F16_AERO_ROLL_EARLY, e4 = F16_AERO_PITCH_EARLY, e5 = F16_AERO_YAW_EARLY;
    ax[0] = F16_AERO_DRAG_SCALE * (e0 + F16_AERO_DRAG_LATE);
    ax[1] = F16_AERO_SIDE_SCALE * (e1 + F16_AERO_SIDE_LATE);
    ax[2] = F16_AERO_LIFT_SCALE * (e2 + F16_AERO_LIFT_LATE);
    ax[3] = F16_AERO_ROLL_SCALE * (e3 + F16_AERO_ROLL_LATE);
    ax[4] = F16_AERO_PITCH_SCALE * (e4 + F16_AERO_PITCH_LATE);
    ax[5] = F16_AERO_YAW_SCALE * (e5 + F16_AERO_YAW_LATE);
  }
  double F[3], M[3], gi[3];
  forces_moments(ax, g, mb, thrust, F, M);
  gravity(k, gi);
  Accel ac;
  accelerations(k.B, k.wpqr, mb, F, M, gi, ac);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    o.ai[i] = ac.ai[i]; o.wdi[i] = ac.wdi[i]; o.pba[i] = ac.pba[i]; o.ppq[i] = ac.ppq[i];
  }
}

// ------------------------------------------------------------------ one integration step
// FDM.step (jsb_fdm.py:212-244).  FCS_RATE: the FCS components' dt is 1/FCS_RATE s (120 for
// cuda_fdm/ref/jsb_fcs.py:19, 60 for the 184-D runtime's copy of that file).
template <int FCS_RATE>
F16_HD void substep(Aircraft& a, double c_ail, double c_ele, double c_rud,
                                        double c_thr, const double* __restrict__ T,
                                        bool want_euler, SubstepOut& out) {
  propagate(a);
  Kin k;
  frames(a, want_euler, k, out.euler);
  quat_rate(a);
  ForceOut f;
  force_path<FCS_RATE>(a, c_ail, c_ele, c_rud, c_thr, k, T, f);
  a.fuel -= f.fuel_burn;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    a.ai[i] = f.ai[i];
    a.wdi[i] = f.wdi[i];
    a.pba[i] = f.pba[i];
    a.ppd[i] = f.wdi[i];
    a.ppq[i] = f.ppq[i];
  }
  a.pa[0] = f.alpha; a.pa[1] = f.mach; a.pa[2] = f.vc_kts; a.pa[3] = f.vg;
  a.pa[4] = f.npy; a.pa[5] = f.npz; a.pa[6] = k.wpqr[0]; a.pa[7] = k.wpqr[1]; a.pa[8] = k.wpqr[2];
  out.k_rud = f.k_rud;
  out.k_gear = kGearPos<FCS_RATE>;
#pragma unroll
  for (int i = 0; i < 3; ++i) out.uvw[i] = k.uvw[i];
  out.alpha = f.alpha; out.beta = f.beta; out.mach = f.mach; out.vt = f.vt; out.alt = f.alt;
}

}  // namespace f16
