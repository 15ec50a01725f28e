// obs_device.h -- per-aircraft observation, reconstructor and reward math (host+device).
//
// Lane layout used by the kernels: aircraft a of engagement e is lane 2e (plane 0) or 2e+1
// (plane 1) of the same wavefront, so a lane reads its partner's values with one cross-lane
// exchange (__shfl_xor(x, 1)) instead of a second state9 evaluation or a second HBM read.
//
// Semantics follow the reference's torch reconstructor (research/competition_36500/runtime/
// cuda_fdm/obs_reward.py:53-819) and state9 bridge (cuda_fdm/rl_env.py:88-163); constants from
// claude_code/my_observation.py:103-160 and MY_REWARD_CONFIG (claude_code/my_reward.py:45-103).
// All geometry is fp64; observations are stored as fp32 with non-finite values mapped to
// 0 / +-10 (torch.nan_to_num).
#pragma once

#include <hip/hip_runtime.h>

#include "f16_state.h"
#include "fdm_math.h"

#ifndef F16_HD
#define F16_HD __host__ __device__ __forceinline__
#endif

namespace f16obs {

using f16::fm_div;
using f16::fm_exp;
using f16::fm_log;
using f16::fm_rcp;
using f16::fm_sqrt;

constexpr double kD2R = 3.141592653589793 / 180.0;
constexpr double kR2D = 180.0 / 3.141592653589793;
constexpr double kFt2M = 0.3048;
constexpr double kM2FtObs = 3.28084;               // the observation's feet conversion
constexpr double kGacc = 9.80665;
constexpr double kRot = 7.292115e-5;
constexpr double kSeaLevelRadiusFt = 20925646.32546;
constexpr double kWgsA = 6378137.0;
constexpr double kWgsE2 = 0.0066943799901411;
constexpr double kMinAltM = 1000.0 * kFt2M;         // hard deck 304.8 m
constexpr double kDtStep = 6.0 / 60.0;              // one decision = 6 simulator frames
constexpr double kTimeTol = 1.0e-8;
constexpr double kAltLogScale = 304.8;
constexpr double kAltLogFloor = 1e-4;
constexpr int kActHist = 20;                        // 5 steps x 4 channels, newest first
constexpr int kAuxDim = 21;                         // future-aux features per engagement

// Official origin (37.240778 N, 131.869556 E, 0 m) in ECEF metres, its trigonometry, and the
// WGS84 polar radius b = a sqrt(1 - e^2) and second eccentricity ep2 = (a^2 - b^2) / b^2 of the
// Bowring step.  Filled on the host (obs_kernels.hip) with the same expressions as the checker.
struct Origin { double ox, oy, oz, slat, clat, slon, clon, b, ep2; };

F16_HD double clampd(double x, double lo, double hi) { return x < lo ? lo : (x > hi ? hi : x); }
F16_HD double norm3(const double v[3]) { return fm_sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]); }
F16_HD void mv3(const double A[3][3], const double v[3], double o[3]) {
  const double a = A[0][0] * v[0] + A[0][1] * v[1] + A[0][2] * v[2];
  const double b = A[1][0] * v[0] + A[1][1] * v[1] + A[1][2] * v[2];
  const double c = A[2][0] * v[0] + A[2][1] * v[1] + A[2][2] * v[2];
  o[0] = a; o[1] = b; o[2] = c;
}
F16_HD void mtv3(const double A[3][3], const double v[3], double o[3]) {   // A^T v
  const double a = A[0][0] * v[0] + A[1][0] * v[1] + A[2][0] * v[2];
  const double b = A[0][1] * v[0] + A[1][1] * v[1] + A[2][1] * v[2];
  const double c = A[0][2] * v[0] + A[1][2] * v[1] + A[2][2] * v[2];
  o[0] = a; o[1] = b; o[2] = c;
}
F16_HD void cross3(const double a[3], const double b[3], double o[3]) {
  const double x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
  o[0] = x; o[1] = y; o[2] = z;
}

// ---------------------------------------------------------------- state9 bridge
// Attitude of one aircraft: R = Tx(roll) Ty(pitch) Tz(yaw) (NED -> body, GeometryInfo
// convention) and the sin/cos of roll, pitch, yaw (observation scalars 27-38 reuse them).
struct Att { double R[3][3]; double sr, cr, sp, cp, sy, cy; };

F16_HD void att_from_trig(Att& A) {
  const double cr = A.cr, sr = A.sr, cp = A.cp, sp = A.sp, cy = A.cy, sy = A.sy;
  A.R[0][0] = cp * cy;                  A.R[0][1] = cp * sy;                  A.R[0][2] = -sp;
  A.R[1][0] = sr * (sp * cy) - cr * sy; A.R[1][1] = sr * (sp * sy) + cr * cy; A.R[1][2] = sr * cp;
  A.R[2][0] = cr * (sp * cy) + sr * sy; A.R[2][1] = cr * (sp * sy) - sr * cy; A.R[2][2] = cr * cp;
}

// sin and cos of atan2(y, x) without the angle (atan2(0, 0) = 0)
F16_HD void sc_atan2(double y, double x, double& s, double& c) {
  const double h = fm_sqrt(x * x + y * y);
  if (h > 0.0) { const double ih = fm_rcp(h); s = y * ih; c = x * ih; } else { s = 0.0; c = 1.0; }
}

// 101-double state (field k at st[k*ld]) -> N/E/D m (D = -MSL), roll/pitch/yaw deg, body u/v/w
// m/s.  N/E are the tangent projection about the origin of the point at the aircraft's
// geodetic latitude/longitude (Bowring) and MSL altitude (rl_env.py:64-85).  The sines and
// cosines of the Bowring angles and, when `att` is given, of the Euler angles come from the
// ratios they are atan2'd from (sin atan2(y, x) = y / hypot(x, y)); the angles themselves are
// produced only where they are outputs.
F16_HD void state9(const double* st, long ld, const Origin& O, double s9[9], Att* att = nullptr) {
  const double px = st[0], py = st[ld], pz = st[2 * ld];
  const double vx = st[3 * ld], vy = st[4 * ld], vz = st[5 * ld];
  const double q0 = st[6 * ld], q1 = st[7 * ld], q2 = st[8 * ld], q3 = st[9 * ld];
  const double epa = st[F16S_EPA * ld];
  double se, ce;
  sincos(epa, &se, &ce);
  const double ex = ce * px + se * py, ey = -se * px + ce * py, ez = pz;
  const double rxy2 = ex * ex + ey * ey;
  const double radius = fm_sqrt(rxy2 + ez * ez), rxy = fm_sqrt(rxy2);
  const double ir = fm_rcp(radius), irxy = fm_rcp(rxy);
  const double sLat = ez * ir, cLat = rxy * ir, sLon = ey * irxy, cLon = ex * irxy;
  // local N/E/D axes in ECI (columns of Tl2i)
  const double n0 = -cLon * sLat, n1 = -sLon * sLat, d0 = -cLon * cLat, d1 = -sLon * cLat;
  const double N[3] = {ce * n0 - se * n1, se * n0 + ce * n1, cLat};
  const double E[2] = {ce * (-sLon) - se * cLon, se * (-sLon) + ce * cLon};
  const double Dn[3] = {ce * d0 - se * d1, se * d0 + ce * d1, -sLat};
  const double q0q0 = q0 * q0, q1q1 = q1 * q1, q2q2 = q2 * q2, q3q3 = q3 * q3;
  const double q0q1 = q0 * q1, q0q2 = q0 * q2, q0q3 = q0 * q3, q1q2 = q1 * q2, q1q3 = q1 * q3, q2q3 = q2 * q3;
  const double B[3][3] = {{q0q0 + q1q1 - q2q2 - q3q3, 2.0 * (q1q2 + q0q3), 2.0 * (q1q3 - q0q2)},
                          {2.0 * (q1q2 - q0q3), q0q0 - q1q1 + q2q2 - q3q3, 2.0 * (q2q3 + q0q1)},
                          {2.0 * (q1q3 + q0q2), 2.0 * (q2q3 - q0q1), q0q0 - q1q1 - q2q2 + q3q3}};
  const double L00 = B[0][0] * N[0] + B[0][1] * N[1] + B[0][2] * N[2];
  const double L01 = B[0][0] * E[0] + B[0][1] * E[1];
  const double L02 = B[0][0] * Dn[0] + B[0][1] * Dn[1] + B[0][2] * Dn[2];
  const double L12 = B[1][0] * Dn[0] + B[1][1] * Dn[1] + B[1][2] * Dn[2];
  const double L22 = B[2][0] * Dn[0] + B[2][1] * Dn[1] + B[2][2] * Dn[2];
  const double sp = -clampd(L02, -1.0, 1.0);
  const double theta = asin(sp);
  const double phi = atan2(L12, L22);
  double psi = atan2(L01, L00);
  psi = psi < 0.0 ? psi + 2.0 * 3.141592653589793 : psi;
  if (att) {
    att->sp = sp;
    att->cp = fm_sqrt((1.0 - sp) * (1.0 + sp));
    sc_atan2(L12, L22, att->sr, att->cr);
    sc_atan2(L01, L00, att->sy, att->cy);
    att_from_trig(*att);
  }
  const double dv[3] = {vx + kRot * py, vy - kRot * px, vz};
  double vb[3];
  mv3(B, dv, vb);
  const double alt_m = (radius - kSeaLevelRadiusFt) * kFt2M;
  // Bowring ECEF -> geodetic latitude / longitude, then back to ECEF at MSL altitude
  const double exm = ex * kFt2M, eym = ey * kFt2M, ezm = ez * kFt2M;
  const double b = O.b, ep2 = O.ep2;
  const double p = fm_sqrt(exm * exm + eym * eym);
  double sth, cth, slat, clat, slon, clon;
  sc_atan2(ezm * kWgsA, p * b, sth, cth);
  sc_atan2(ezm + ep2 * b * (sth * sth * sth), p - kWgsE2 * kWgsA * (cth * cth * cth), slat, clat);
  sc_atan2(eym, exm, slon, clon);
  const double Nr = fm_div(kWgsA, fm_sqrt(1.0 - kWgsE2 * slat * slat));
  const double dx = (Nr + alt_m) * clat * clon - O.ox, dy = (Nr + alt_m) * clat * slon - O.oy;
  const double dz = (Nr * (1.0 - kWgsE2) + alt_m) * slat - O.oz;
  s9[0] = -O.slat * O.clon * dx - O.slat * O.slon * dy + O.clat * dz;
  s9[1] = -O.slon * dx + O.clon * dy;
  s9[2] = -alt_m;
  s9[3] = phi * kR2D; s9[4] = theta * kR2D; s9[5] = psi * kR2D;
  s9[6] = vb[0] * kFt2M; s9[7] = vb[1] * kFt2M; s9[8] = vb[2] * kFt2M;
}

// ---------------------------------------------------------------- attitude helpers
F16_HD void attitude(const double s9[9], Att& A) {
  sincos(s9[3] * kD2R, &A.sr, &A.cr);
  sincos(s9[4] * kD2R, &A.sp, &A.cp);
  sincos(s9[5] * kD2R, &A.sy, &A.cy);
  att_from_trig(A);
}

F16_HD void unit_or_self(const double v[3], double o[3]) {
  const double n = norm3(v);
  if (n > 0.0) { const double in = fm_rcp(n); o[0] = v[0] * in; o[1] = v[1] * in; o[2] = v[2] * in; }
  else { o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; }
}

// 3-D antenna train angle from `own` (with NED->body R) to the point `tgt`, 0..180 deg
F16_HD double ata_deg(const double own[9], const double R[3][3], const double tgt[9]) {
  const double d[3] = {tgt[0] - own[0], tgt[1] - own[1], tgt[2] - own[2]};
  double u[3];
  unit_or_self(d, u);
  return acos(clampd(R[0][0] * u[0] + R[0][1] * u[1] + R[0][2] * u[2], -1.0, 1.0)) * kR2D;
}

// x axis along `x`, roll fixed by gravity; north, then east, when x is vertical (dir_frame);
// the identity for |x| < 1e-8.  Branch-free (both results formed, then selected), which keeps
// the frame in registers.
F16_HD void dir_frame(const double x[3], double F[3][3]) {
  const double nx = norm3(x);
  const bool ok = nx >= 1e-8;
  const double nxs = ok ? nx : 1.0;
  const double inx = fm_rcp(nxs);
  const double xn[3] = {x[0] * inx, x[1] * inx, x[2] * inx};
  // projections of down, north, east off x; the first with norm >= 1e-6 is used
  const double zd[3] = {-xn[2] * xn[0], -xn[2] * xn[1], 1.0 - xn[2] * xn[2]};
  const double zn[3] = {1.0 - xn[0] * xn[0], -xn[0] * xn[1], -xn[0] * xn[2]};
  const double ze[3] = {-xn[1] * xn[0], 1.0 - xn[1] * xn[1], -xn[1] * xn[2]};
  const bool use_d = norm3(zd) >= 1e-6, use_n = norm3(zn) >= 1e-6;
  double z[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) z[i] = use_d ? zd[i] : (use_n ? zn[i] : ze[i]);
  double n = norm3(z);
  n = fm_rcp(n > 1e-300 ? n : 1e-300);
  z[0] *= n; z[1] *= n; z[2] *= n;
  double y[3];
  cross3(z, xn, y);
  n = norm3(y);
  n = fm_rcp(n > 1e-300 ? n : 1e-300);
  y[0] *= n; y[1] *= n; y[2] *= n;
  cross3(xn, y, z);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    F[0][i] = ok ? xn[i] : (i == 0 ? 1.0 : 0.0);
    F[1][i] = ok ? y[i] : (i == 1 ? 1.0 : 0.0);
    F[2][i] = ok ? z[i] : (i == 2 ? 1.0 : 0.0);
  }
}

F16_HD double normz(double x, double lo, double hi) {
  const double mid = (hi + lo) * 0.5, inv_half = 1.0 / ((hi - lo) * 0.5);
  return (clampd(x, lo, hi) - mid) * inv_half;
}

// three-tier cone damage rate, tier 1 first (obs_reward.py:206-218)
F16_HD double damage_rate(double r_ft, double ata, double t) {
  const double a = fabs(ata);
  if (r_ft >= 500.0 && r_ft <= 3000.0 && a < 1.0) return 1.0 * (3000.0 - r_ft) * (1.0 / (3000.0 - 500.0));
  if (t >= 100.0 && r_ft >= 500.0 && r_ft <= 3500.0 && a < 2.0) return 0.3 * (3500.0 - r_ft) * (1.0 / (3500.0 - 500.0));
  if (t >= 150.0 && r_ft >= 500.0 && r_ft <= 4000.0 && a < 3.0) return 0.1 * (4000.0 - r_ft) * (1.0 / (4000.0 - 500.0));
  return 0.0;
}

F16_HD double smoothstep(double x, double e0, double e1) {
  const double z = clampd((x - e0) * (1.0 / (e1 - e0)), 0.0, 1.0);   // e0, e1: literals
  return z * z * (3.0 - 2.0 * z);
}

F16_HD void unit_fallback(const double v[3], const double fb[3], double o[3]) {
  const double n = norm3(v);
  if (n >= 1e-9) { const double in = fm_rcp(n); o[0] = v[0] * in; o[1] = v[1] * in; o[2] = v[2] * in; return; }
  double fn = norm3(fb);
  fn = fm_rcp(fn > 1e-9 ? fn : 1e-9);
  o[0] = fb[0] * fn; o[1] = fb[1] * fn; o[2] = fb[2] * fn;
}

F16_HD double align3(const double a[3], const double b[3]) {
  const double ex[3] = {1.0, 0.0, 0.0};
  double au[3], bu[3];
  unit_fallback(a, ex, au);
  unit_fallback(b, au, bu);
  const double q = (1.0 + clampd(au[0] * bu[0] + au[1] * bu[1] + au[2] * bu[2], -1.0, 1.0)) * 0.5;
  return clampd(q * q * q, 0.0, 1.0);
}

// One side's final-safe attack geometry S = 0.5 broad + 0.2 safe-lead + 0.2 control-zone +
// 0.1 fine (obs_reward.py:233-310 with MY_REWARD_CONFIG).  `ata` is own->target (0..180).
F16_HD double final_safe_side(const double own[9], const double R[3][3], const double own_v[3],
                              const double tgt[9], const double tgt_v[3], double ata, double t) {
  const double ex[3] = {1.0, 0.0, 0.0};
  const double rel[3] = {tgt[0] - own[0], tgt[1] - own[1], tgt[2] - own[2]};
  const double dist_m = norm3(rel), dist_ft = dist_m * (1.0 / kFt2M);
  double los[3];
  unit_fallback(rel, ex, los);
  const double fwd[3] = {R[0][0], R[0][1], R[0][2]};
  double spd = norm3(own_v);
  const double tau = clampd(fm_div(dist_m, spd < 30.0 ? 30.0 : spd), 0.30, 1.50);
  const double lv[3] = {tgt[0] + tgt_v[0] * tau - own[0], tgt[1] + tgt_v[1] * tau - own[1],
                        tgt[2] + tgt_v[2] * tau - own[2]};
  double lead[3], path[3];
  unit_fallback(lv, los, lead);
  unit_fallback(own_v, fwd, path);
  const double intercept = (0.40 * align3(fwd, lead) + 0.60 * align3(path, lead)) / (0.40 + 0.60);
  const double direct = align3(fwd, los);
  const double ss_ata = smoothstep(ata, 3.0, 8.0);
  const double w = smoothstep(dist_ft, 1000.0, 2500.0) * ss_ata;
  const double safe_lead = w * intercept + (1.0 - w) * direct;
  const double broad = ata <= 30.0 ? 1.0 : clampd((180.0 - ata) * (1.0 / (180.0 - 30.0)), 0.0, 1.0);
  const double range_gate = smoothstep(dist_ft, 600.0, 900.0) * (1.0 - smoothstep(dist_ft, 3200.0, 4300.0));
  const double closing = (own_v[0] - tgt_v[0]) * los[0] + (own_v[1] - tgt_v[1]) * los[1] +
                         (own_v[2] - tgt_v[2]) * los[2];
  const double mean_speed = 0.5 * (spd + norm3(tgt_v));
  const double cr = fm_div(closing, mean_speed > 100.0 ? mean_speed : 100.0);
  const double desired = 0.20 * smoothstep(dist_ft, 2000.0, 4500.0) + (-0.12) * (1.0 - smoothstep(dist_ft, 650.0, 900.0));
  const double zq = (cr - desired) * (1.0 / 0.15);
  const double control = clampd((1.0 - ss_ata) * range_gate * fm_exp(-0.5 * (zq * zq)), 0.0, 1.0);
  const double fine = damage_rate(dist_ft, ata, t);
  return clampd(0.50 * broad + 0.20 * safe_lead + 0.20 * control + 0.10 * fine, 0.0, 1.0);
}

F16_HD double altitude_log(double alt_m) {
  const double x = alt_m * (1.0 / kAltLogScale);
  return fm_log(x < kAltLogFloor ? kAltLogFloor : x);
}

// body rates from two attitudes: log_SO3(R_prev R_curr^T) / dt (obs_reward.py:169-186, 601-606)
F16_HD void so3_rates(const double Rp[3][3], const double Rc[3][3], double out[3]) {
  double M[3][3];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) M[i][j] = Rp[i][0] * Rc[j][0] + Rp[i][1] * Rc[j][1] + Rp[i][2] * Rc[j][2];
  const double tr = M[0][0] + M[1][1] + M[2][2];
  const double theta = acos(clampd((tr - 1.0) * 0.5, -1.0, 1.0));
  const double denom = 2.0 * sin(theta);
  const double scale = (theta >= 1e-8 && fabs(denom) >= 1e-8) ? fm_div(theta, denom) : 0.0;
  out[0] = (M[2][1] - M[1][2]) * scale * (1.0 / kDtStep);
  out[1] = (M[0][2] - M[2][0]) * scale * (1.0 / kDtStep);
  out[2] = (M[1][0] - M[0][1]) * scale * (1.0 / kDtStep);
}

F16_HD float obs_value(double v) {
  if (v != v) return 0.0f;
  if (v == 1.0 / 0.0) return 10.0f;
  if (v == -1.0 / 0.0) return -10.0f;
  return (float)v;
}

}  // namespace f16obs
