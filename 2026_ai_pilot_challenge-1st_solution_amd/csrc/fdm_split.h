// fdm_split.h -- the batched F-16 step with each aircraft's substep spread over two cooperating
// wavefronts of one workgroup.
//
// One lane per aircraft still, but every 64 aircraft get two wavefronts: the "flight" wave owns
// the integrator (propagation, frames, body kinematics, aero build-up, forces, accelerations)
// and the "systems" wave owns the mass, FCS, atmosphere, air data and engine.  The two run
// concurrently on different SIMDs and trade what the other needs through LDS at three
// workgroup barriers per substep:
//
//   phase 1  flight:  history pushes, propagate, frames
//            systems: mass properties, previous-frame FCS channels, pitch schedule, Earth
//                     position angle
//   -- X1: altitude, cos(theta)cos(phi)  |  mass/CG/inertia, aileron/rudder/LEF/flaperon
//   phase 2  flight:  air-relative geometry (vt, alpha, beta), load factors, alpha/beta brackets,
//                     their table values and the alpha/beta-only part of each axis sum
//            systems: atmosphere, pitch loop, sin/cos of the next substep's Earth position angle
//   -- X2: vt, alpha, beta, n_y, n_z  |  rho, speed of sound, elevator
//   phase 3  flight:  dynamic pressure, mach, mach/elevator brackets and values, the six axes,
//                     quaternion rate, gravity, vg
//            systems: mach, calibrated airspeed, engine
//   -- X3: vg, p q r  |  thrust (the next substep's sin/cos(epa), written in phase 2, are read
//          by the flight wave after this exchange)
//   phase 4  flight:  forces, moments, accelerations, state update
//            systems: fuel burn, previous-frame auxiliary values
//
// The phases are cut so that each side's share between two barriers is about equal (measured
// with per-wavefront clock stamps); values only needed for the next substep's previous-frame
// inputs travel at the last exchange.
//
// Every value is computed by the same component functions (fdm_device.h) with the same
// operands as the one-lane kernel, so the two kernels agree bit for bit; this one halves the
// instructions each wavefront issues and gives each the registers of its own half of the
// state.  At 16,384 engagements the one-lane kernel has 512 wavefronts for 1,024 SIMDs; this
// one fills them.
#pragma once
#include "fdm_device.h"

namespace f16 {

constexpr int kSplitPairs = 2;                      // wavefront pairs per workgroup
constexpr int kSplitBlock = 128 * kSplitPairs;      // threads per workgroup
constexpr int kSplitAircraft = 64 * kSplitPairs;    // aircraft per workgroup

// LDS exchange fields, [pair][field][lane].
enum SplitField : int {
  // X1, flight -> systems
  kXAlt, kXCtcp,
  // X1, systems -> flight
  kXMass, kXJ, kXJinv = kXJ + 6, kXRp = kXJinv + 6, kXCg = kXRp + 3,
  kXAil = kXCg + 3, kXRud, kXLef, kXFlap,
  // X2, flight -> systems
  kXVt, kXAlpha, kXBeta, kXNpy, kXNpz,
  // X2, systems -> flight
  kXRho, kXSound, kXElev,
  // X3, flight -> systems
  kXVg, kXP, kXQ, kXR,
  // X3, systems -> flight
  kXThrust, kXCe, kXSe,
  // the mass block again: substep t's mass properties live in block t & 1 (below)
  kXMass2, kXFin = kXMass2 + (kXAil - kXMass),
  // after the last substep, flight -> systems: every value the flight wave wrote is finite
  kSplitFields
};

// Mass properties are written by the systems wave in its first phase and read by the flight
// wave in its second (CG) and fourth (forces, accelerations) phases; the next substep's first
// phase overlaps this substep's fourth, so consecutive substeps use alternate blocks and the
// flight wave does not hold the 19 values across its aero phases.
__device__ __forceinline__ int mass_block(int t) { return (t & 1) ? kXMass2 - kXMass : 0; }

typedef double SplitX[kSplitFields][64];

// The flight wave of one pair.  `s`: the aircraft's state field 0 (fields `ld` apart); `store`:
// whether this lane's aircraft exists (lanes past the batch shadow the last aircraft and store
// nothing).  Issues exactly 3 barriers per substep, like split_systems.
// With `fin` set, the wave also reports through x[kXFin] whether every state value it wrote
// (or, for S < 3, shifted) is finite, after one more workgroup barrier that split_systems
// matches.
template <int FCS_RATE>
__device__ __forceinline__ void split_flight(double* __restrict__ s, long ld, int S, bool store,
                                             double* __restrict__ o, long obs_ld,
                                             const double* __restrict__ T, SplitX& x, int lane,
                                             bool fin) {
#define F(k) s[(long)(k) * ld]
  Aircraft a;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    a.p[j] = F(F16S_POS + j); a.v[j] = F(F16S_VEL + j); a.wi[j] = F(F16S_PQRI + j);
    a.ai[j] = F(F16S_UVWIDOT + j); a.wdi[j] = F(F16S_PQRIDOT + j);
    a.vh1[j] = F(F16S_DIVEL + j); a.vh2[j] = F(F16S_DIVEL + 3 + j); a.ah1[j] = F(F16S_DUVW + j);
    a.pba[j] = F(F16S_PBA + j); a.ppd[j] = F(F16S_PPQRIDOT + j); a.ppq[j] = F(F16S_PPQRI + j);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) { a.q[j] = F(F16S_Q + j); a.qd[j] = F(F16S_QDOT + j); }
  a.epa = F(F16S_EPA);
  // Finite flag: the history values this call writes inside the substep loop are the qd, wdi,
  // v, ai each following substep integrates by plain sums (q += dt qd, wi += dt wdi, AB2/AB3 on
  // ai and v, no clamps), so a non-finite one leaves a non-finite q, wi, v or p at the end; only
  // the older entries shifted down when S < 3 need their own test.
  unsigned hist_m = 0u;
  // fewer than three substeps keep older history entries, shifted down by S
  if (store && S > 0 && S < 3) {
    for (int k = 2; k >= S; --k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double h = F(F16S_DQ + 4 * (k - S) + j);
        hist_m = fin_acc(hist_m, h);
        F(F16S_DQ + 4 * k + j) = h;
      }
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const double h1 = F(F16S_DPQRI + 3 * (k - S) + j), h2 = F(F16S_DIVEL + 3 * (k - S) + j);
        const double h3 = F(F16S_DUVW + 3 * (k - S) + j);
        hist_m = fin_acc(fin_acc(fin_acc(hist_m, h1), h2), h3);
        F(F16S_DPQRI + 3 * k + j) = h1;
        F(F16S_DIVEL + 3 * k + j) = h2;
        F(F16S_DUVW + 3 * k + j) = h3;
      }
    }
  }
  double euler[3] = {0.0, 0.0, 0.0}, mach = 0.0, alt = 0.0;
  AuxGeo g;
  Kin k;
  for (int t = 0; t < S; ++t) {
    const int slot = S - 1 - t;
    // ---- phase 1
    if (store && slot <= 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) F(F16S_DQ + 4 * slot + j) = a.qd[j];
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        F(F16S_DPQRI + 3 * slot + j) = a.wdi[j];
        F(F16S_DIVEL + 3 * slot + j) = a.v[j];
        F(F16S_DUVW + 3 * slot + j) = a.ai[j];
      }
    }
    propagate(a);
    {   // sin/cos(epa): the systems wave evaluates them one substep ahead, off this chain
      double ce, se;
      if (t == 0) {
        sincos(a.epa, &se, &ce);
      } else {
        ce = x[kXCe][lane];
        se = x[kXSe][lane];
      }
      kinematics(a.p, a.v, a.q, a.wi, ce, se, slot == 0 && o != nullptr, k, euler);
    }
    alt = k.radius - kSemiMajor;
    x[kXAlt][lane] = alt; x[kXCtcp][lane] = k.ctcp;
    __syncthreads();
    // ---- phase 2
    const int mo = mass_block(t);
    g = aux_geometry(k.uvw);
    double npy, npz;
    {
      const double cg[3] = {x[mo + kXCg][lane], x[mo + kXCg + 1][lane], x[mo + kXCg + 2][lane]};
      load_factors(a, cg, npy, npz);
    }
    x[kXVt][lane] = g.vt; x[kXAlpha][lane] = g.alpha; x[kXBeta][lane] = g.beta;
    x[kXNpy][lane] = npy; x[kXNpz][lane] = npz;
    const double alpha = g.alpha, beta = g.beta;
    const double ail = x[kXAil][lane], rud = x[kXRud][lane];
    double early[6];      // the alpha/beta-only part of each axis, so its 18 table values die here
    {
      const double lef = x[kXLef][lane], flap = x[kXFlap][lane];
      double bi2vel, ci2vel;
      aero_rates(g.vt, bi2vel, ci2vel);
      constexpr double kclge = kCLge;
      constexpr double gear = kGearPos<FCS_RATE>;
      const double p = k.wpqr[0], q = k.wpqr[1], r = k.wpqr[2];
      F16_AERO_BRACKETS_AB;
      F16_AERO_LOOKUPS_AB;
      early[0] = F16_AERO_DRAG_EARLY; early[1] = F16_AERO_SIDE_EARLY;
      early[2] = F16_AERO_LIFT_EARLY; early[3] = F16_AERO_ROLL_EARLY;
      early[4] = F16_AERO_PITCH_EARLY; early[5] = F16_AERO_YAW_EARLY;
    }
    __syncthreads();
    // ---- phase 3
    const double rho = x[kXRho][lane], sound = x[kXSound][lane], elev = x[kXElev][lane];
    const double qbar = 0.5 * rho * g.vt2;
    mach = fm_div(g.vt, sound);
    x[kXVg][lane] = fm_sqrt(k.vn * k.vn + k.ve * k.ve);
    x[kXP][lane] = k.wpqr[0]; x[kXQ][lane] = k.wpqr[1]; x[kXR][lane] = k.wpqr[2];
    quat_rate(a);
    double gi[3];
    gravity(k, gi);
    double ax[6];
    {
      constexpr double kclge = kCLge;
      const F16Br2 b2_G9_ALPHA = F16_BR2(G9_ALPHA, alpha);   // the elevator tables' alpha bracket
      F16_AERO_BRACKETS_MACH;
      F16_AERO_BRACKETS_ELEV;
      F16_AERO_LOOKUPS_MACH;
      F16_AERO_LOOKUPS_ELEV;
      ax[0] = F16_AERO_DRAG_SCALE * (early[0] + F16_AERO_DRAG_LATE);
      ax[1] = F16_AERO_SIDE_SCALE * (early[1] + F16_AERO_SIDE_LATE);
      ax[2] = F16_AERO_LIFT_SCALE * (early[2] + F16_AERO_LIFT_LATE);
      ax[3] = F16_AERO_ROLL_SCALE * (early[3] + F16_AERO_ROLL_LATE);
      ax[4] = F16_AERO_PITCH_SCALE * (early[4] + F16_AERO_PITCH_LATE);
      ax[5] = F16_AERO_YAW_SCALE * (early[5] + F16_AERO_YAW_LATE);
    }
    __syncthreads();
    // ---- phase 4
    const double thrust = x[kXThrust][lane];
    Mass mb;
    mb.mass = x[mo + kXMass][lane];
#pragma unroll
    for (int j = 0; j < 6; ++j) { mb.J[j] = x[mo + kXJ + j][lane]; mb.Jinv[j] = x[mo + kXJinv + j][lane]; }
#pragma unroll
    for (int j = 0; j < 3; ++j) { mb.rp[j] = x[mo + kXRp + j][lane]; mb.cg[j] = x[mo + kXCg + j][lane]; }
    double Fb[3], Mb[3];
    forces_moments(ax, g, mb, thrust, Fb, Mb);
    Accel ac;
    {
      double B[3][3];   // recomputed from the quaternion rather than held since phase 1
      body_dcm(a.q, B);
      accelerations(B, k.wpqr, mb, Fb, Mb, gi, ac);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      a.ai[i] = ac.ai[i]; a.wdi[i] = ac.wdi[i]; a.pba[i] = ac.pba[i];
      a.ppd[i] = ac.wdi[i]; a.ppq[i] = ac.ppq[i];
    }
  }
  if (store && S > 0) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      F(F16S_POS + j) = a.p[j]; F(F16S_VEL + j) = a.v[j]; F(F16S_PQRI + j) = a.wi[j];
      F(F16S_UVWIDOT + j) = a.ai[j]; F(F16S_PQRIDOT + j) = a.wdi[j];
      F(F16S_PBA + j) = a.pba[j]; F(F16S_PPQRIDOT + j) = a.ppd[j]; F(F16S_PPQRI + j) = a.ppq[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) { F(F16S_Q + j) = a.q[j]; F(F16S_QDOT + j) = a.qd[j]; }
    F(F16S_EPA) = a.epa;
    if (o) {
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        o[(long)j * obs_ld] = a.p[j];
        o[(long)(3 + j) * obs_ld] = a.v[j];
        o[(long)(6 + j) * obs_ld] = euler[j];
        o[(long)(9 + j) * obs_ld] = k.uvw[j];
      }
      o[12L * obs_ld] = g.alpha; o[13L * obs_ld] = g.beta; o[14L * obs_ld] = mach;
      o[15L * obs_ld] = g.vt; o[16L * obs_ld] = alt;
    }
  }
#undef F
  if (fin) {   // every flight-side value stored above (the loop's history: see hist_m)
    unsigned m = fin_acc(hist_m, a.epa);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      m = fin_acc(fin_acc(fin_acc(fin_acc(m, a.p[j]), a.v[j]), a.wi[j]), a.ai[j]);
      m = fin_acc(fin_acc(fin_acc(fin_acc(m, a.wdi[j]), a.pba[j]), a.ppd[j]), a.ppq[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fin_acc(fin_acc(m, a.q[j]), a.qd[j]);
    x[kXFin][lane] = m < kFinInf ? 1.0 : 0.0;
    __syncthreads();
  }
}

// The systems wave of one pair: fuel, engine, FCS and previous-frame auxiliary state.
// Issues exactly 3 barriers per substep, like split_flight.
// With `fin` non-null, fin[0] <- 1 if every one of the aircraft's 101 state values after the
// call is finite, else 0 (the flight wave's share arrives through x[kXFin]).  With `keep`
// non-null, the aircraft's four actions are also written to keep[0..3].
template <int FCS_RATE>
__device__ __forceinline__ void split_systems(double* __restrict__ s, long ld,
                                              const double* __restrict__ act4, int S, bool store,
                                              const double* __restrict__ T, SplitX& x, int lane,
                                              unsigned char* __restrict__ fin,
                                              double* __restrict__ keep) {
#define F(k) s[(long)(k) * ld]
  Aircraft a;
#pragma unroll
  for (int j = 0; j < 3; ++j) { a.pid_ip[j] = F(F16S_PID + 3 * j); a.pid_io[j] = F(F16S_PID + 3 * j + 2); }
#pragma unroll
  for (int j = 0; j < 9; ++j) a.pa[j] = F(F16S_PAUX + j);
  a.fuel = F(F16S_FUEL);
  a.epa = F(F16S_EPA);   // tracked with the flight wave's increments; never stored here
  a.n1 = F(F16S_ENG); a.n2 = F(F16S_ENG + 1); a.n2n = F(F16S_ENG + 2); a.ff = F(F16S_ENG + 3);
  a.k_tef = F(F16S_KIN); a.k_ail = F(F16S_KIN + 1); a.k_ele = F(F16S_KIN + 2); a.k_lef = F(F16S_KIN + 5);
  const double c_ail = act4[0], c_ele = act4[1], c_rud = act4[2], c_thr = act4[3];
  if (keep && store) { keep[0] = c_ail; keep[1] = c_ele; keep[2] = c_rud; keep[3] = c_thr; }
  double k_rud = 0.0;
  unsigned ip2_m = 0u;   // finite-flag accumulator of the PID input_prev2 values written below
  for (int t = 0; t < S; ++t) {
    const int slot = S - 1 - t;
    // ---- phase 1
    a.epa += kRot * kDt;        // the flight wave's propagate makes the same increment
    if (store && slot == 0) {   // PID input_prev2 = input_prev before the final update
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        F(F16S_PID + 3 * j + 1) = a.pid_ip[j];
        ip2_m = fin_acc(ip2_m, a.pid_ip[j]);
      }
    }
    const Mass mb = mass_props(a.fuel);
    FcsOut fc;
    const double esch = fcs_prev_frame<FCS_RATE>(a, c_ail, c_ele, c_rud, T, fc);
    k_rud = fc.k_rud;
    const int mo = mass_block(t);
    x[mo + kXMass][lane] = mb.mass;
#pragma unroll
    for (int j = 0; j < 6; ++j) { x[mo + kXJ + j][lane] = mb.J[j]; x[mo + kXJinv + j][lane] = mb.Jinv[j]; }
#pragma unroll
    for (int j = 0; j < 3; ++j) { x[mo + kXRp + j][lane] = mb.rp[j]; x[mo + kXCg + j][lane] = mb.cg[j]; }
    x[kXAil][lane] = fc.ail; x[kXRud][lane] = fc.rud; x[kXLef][lane] = fc.lef; x[kXFlap][lane] = fc.flap;
    __syncthreads();
    // ---- phase 2
    const double alt = x[kXAlt][lane], ctcp = x[kXCtcp][lane];
    const Atmos at = isa(alt, T);
    fcs_pitch<FCS_RATE>(a, esch, ctcp, fc);
    x[kXRho][lane] = at.rho; x[kXSound][lane] = at.a;
    x[kXElev][lane] = fc.elev;
    // the next substep's sin/cos(epa): read by the flight wave in that substep's first phase,
    // after this substep's third exchange; formed here, where this wave has slack
    if (t + 1 < S) {
      double sn, cn;
      sincos(a.epa + kRot * kDt, &sn, &cn);
      x[kXCe][lane] = cn;
      x[kXSe][lane] = sn;
    }
    __syncthreads();
    // ---- phase 3
    const double vt = x[kXVt][lane], alpha = x[kXAlpha][lane];
    const double npy = x[kXNpy][lane], npz = x[kXNpz][lane];
    const double mach = fm_div(vt, at.a);
    const double vc = vc_knots(mach, at.P);   // previous-frame input of the next substep's FCS
    double burn;
    x[kXThrust][lane] = engine(a, c_thr, at, mach, T, burn);
    __syncthreads();
    // ---- phase 4
    const double vg = x[kXVg][lane];
    const double p = x[kXP][lane], q = x[kXQ][lane], r = x[kXR][lane];
    a.fuel -= burn;
    a.pa[0] = alpha; a.pa[1] = mach; a.pa[2] = vc; a.pa[3] = vg;
    a.pa[4] = npy; a.pa[5] = npz; a.pa[6] = p; a.pa[7] = q; a.pa[8] = r;
  }
  if (store && S > 0) {
#pragma unroll
    for (int j = 0; j < 3; ++j) { F(F16S_PID + 3 * j) = a.pid_ip[j]; F(F16S_PID + 3 * j + 2) = a.pid_io[j]; }
#pragma unroll
    for (int j = 0; j < 9; ++j) F(F16S_PAUX + j) = a.pa[j];
    F(F16S_FUEL) = a.fuel;
    F(F16S_ENG) = a.n1; F(F16S_ENG + 1) = a.n2; F(F16S_ENG + 2) = a.n2n; F(F16S_ENG + 3) = a.ff;
    F(F16S_KIN) = a.k_tef; F(F16S_KIN + 1) = a.k_ail; F(F16S_KIN + 2) = a.k_ele;
    F(F16S_KIN + 3) = k_rud; F(F16S_KIN + 4) = kGearPos<FCS_RATE>; F(F16S_KIN + 5) = a.k_lef;
  }
#undef F
  if (fin) {   // every systems-side value stored above, then the flight wave's share
    unsigned m = fin_acc(fin_acc(fin_acc(fin_acc(ip2_m, a.fuel), a.n1), a.n2), a.n2n);
    m = fin_acc(fin_acc(fin_acc(fin_acc(m, a.ff), a.k_tef), a.k_ail), a.k_ele);
    m = fin_acc(fin_acc(m, k_rud), a.k_lef);
#pragma unroll
    for (int j = 0; j < 3; ++j) m = fin_acc(fin_acc(m, a.pid_ip[j]), a.pid_io[j]);
#pragma unroll
    for (int j = 0; j < 9; ++j) m = fin_acc(m, a.pa[j]);
    __syncthreads();
    if (store) fin[0] = (m < kFinInf && x[kXFin][lane] != 0.0) ? 1 : 0;
  }
}

}  // namespace f16
