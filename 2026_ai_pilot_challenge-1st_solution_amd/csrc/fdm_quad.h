// fdm_quad.h -- the batched F-16 step with each aircraft's substep spread over four cooperating
// wavefronts, so that at 16,384 engagements every SIMD holds two of them.
//
// One lane per aircraft; every 64 aircraft get four wavefronts ("roles") of one 512-thread
// workgroup (two such groups):
//   kin   the integrator: propagation, frames, air-relative geometry, load factors, gravity,
//         forces, moments, accelerations;
//   aero  air-relative geometry again (the same bits) and the six axes of the aero build-up;
//   fcs   the flight control system and the previous-frame auxiliary values (with the
//         calibrated airspeed they need);
//   air   mass properties, atmosphere, sin/cos of the next substep's Earth angle, engine, fuel.
// They trade values through LDS at three workgroup barriers per substep:
//   phase A  kin: (forces, accelerations of the previous substep,) history pushes, propagate,
//                 frames;  fcs: previous-frame FCS channels, pitch schedule;  air: mass
//   -- X1: altitude, cos(theta)cos(phi), body velocity, body rates | aileron, rudder, LEF,
//          flaperon | mass/CG/inertia (in the block of the substep's parity)
//   phase B  kin: geometry, load factors;  aero: geometry, the alpha-beta terms of the six
//                 axes;  fcs: pitch loop;  air: atmosphere, next sin/cos
//   -- X2: vt, alpha, n_y, n_z | elevator | rho, speed of sound, pressure, sin/cos
//   phase C  kin: quaternion rate, gravity, ground speed;  aero: the Mach/elevator terms of the
//            six axes;  fcs: Mach, calibrated airspeed;  air: Mach, engine
//   -- X3: drag, side, lift, roll, pitch, yaw | thrust | ground speed
// Every value is formed by the component functions of fdm_device.h with the operands the
// one-lane kernel gives them, so all three kernels agree bit for bit.  An aero axis is summed
// by one role in the generated order, and values a role reads from LDS after its writer's next
// phase could overwrite them are read early and held (the mass block alternates by parity).
//
// The two groups of a workgroup map their roles to waves in opposite orders, so each SIMD
// (wave w and w + 4 of the workgroup) holds two roles that are busy in different phases: the
// SIMD pairs are (kin, air) and (fcs, aero).  Within a pair, the role on the substep's critical
// path in a phase runs at raised wave priority (s_setprio), so its instructions issue first
// whenever both waves have one ready: kin in A, C and D (its forces-to-frames chain), air in B
// and C (atmosphere, engine), aero in B and C (the build-up), fcs in A.  The same results;
// 33.4 -> 32.2 us per step at 16k engagements.  Only with two groups per workgroup: with one,
// a SIMD holds one wave and raised priorities made 4,096 engagements 5 % slower.
#pragma once
#include "fdm_image.h"
#include "fdm_split.h"

namespace f16 {
// A state value's store in the last substeps: a relaxed store at system scope, the same bytes as
// a plain store, written through the L2 as it is issued rather than left dirty there for the
// write-back that ends the kernel.  Each role stores a value in the phase of the last substep
// that makes it final (kin: position, velocity, rates, attitude and Earth angle in A, the
// quaternion rate in C, the accelerations after D; fcs: PIDs, surface positions and p, q, r in B,
// the air-data values in C; air: the engine in C, fuel after D), so most of the 27 MB of a 16k
// launch drains while the last substep still computes.  Per step (HIP-graph replay, tail-chase
// engagements): 32.2 -> 31.7 us at 16k, 124 -> 117 us at 65,536, 25.9 -> 25.7 us at 4,096; the
// one-launch env step unchanged.  Plain stores at the same places gain about a third of that,
// streaming (non-temporal) ones two thirds.
__device__ __forceinline__ void put(double* p, double v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr int kQuadGroups = 2;                   // 64-aircraft groups per workgroup
constexpr int kQuadBlock = 256 * kQuadGroups;    // threads per workgroup
constexpr int kQuadAircraft = 64 * kQuadGroups;  // aircraft per workgroup

enum QuadRole : int { kRoleKin = 0, kRoleAero = 1, kRoleFcs = 2, kRoleAir = 3 };

// role of wave w (0..3) of group g
__device__ __forceinline__ int quad_role(int g, int w) {
  // group 0: kin, fcs, aero, air; group 1: air, aero, fcs, kin -> waves w and w + 4 share a
  // SIMD, so the SIMD pairs are (kin, air) and (fcs, aero)
  constexpr int kOrder[2][4] = {{kRoleKin, kRoleFcs, kRoleAero, kRoleAir},
                                {kRoleAir, kRoleAero, kRoleFcs, kRoleKin}};
  return kOrder[g][w];
}

// LDS exchange fields, [group][field][lane].
enum QuadField : int {
  // X1
  kQAlt, kQCtcp, kQU, kQV, kQW, kQP, kQQ, kQR,          // kin
  kQAil, kQRud, kQLef, kQFlap,                           // fcs
  kQMass, kQJ, kQJinv = kQJ + 6, kQRp = kQJinv + 6, kQCg = kQRp + 3,   // air, parity block 0
  kQMassB = kQCg + 3,                                    // air, parity block 1 (19 fields)
  // X2
  kQVt = kQMassB + (kQMassB - kQMass), kQAlpha,          // aero
  kQNpy, kQNpz,                                          // kin
  kQElev,                                                // fcs
  kQRho, kQSound, kQPres, kQCe, kQSe,                    // air
  // X3
  kQAx0, kQAx1, kQAx2, kQAx3, kQAx4, kQAx5,              // aero
  kQThrust,                                              // air
  kQVg,                                                  // kin
  // after the last substep: each state-holding role's finite flag
  kQFinKin, kQFinFcs,
  // the kin role's own slots: integrator values read once per substep, kept out of registers
  // across the phases that do not use them (vh1, vh2, ah1, pba, ppd, ppq)
  kQPark, kQuadFields = kQPark + 18
};
constexpr int kQVh1 = kQPark, kQVh2 = kQPark + 3, kQAh1 = kQPark + 6, kQPba = kQPark + 9,
              kQPpd = kQPark + 12, kQPpq = kQPark + 15;
__device__ __forceinline__ int quad_mass_block(int t) { return (t & 1) ? kQMassB - kQMass : 0; }

// Wave priority N for the rest of this phase, when priorities are in use (two groups per
// workgroup: two waves per SIMD to arbitrate between).
template <int N, bool P>
__device__ __forceinline__ void quad_prio() {
  if constexpr (P) __builtin_amdgcn_s_setprio(N);
}

typedef double QuadX[kQuadFields][64];

// ---- kin: the integrator.  `fin`: report the finite flag of every state value it stores
// through x[kQFinKin] after one more barrier.
template <int FCS_RATE, bool PRIO = false>
__device__ __forceinline__ void quad_kin(double* __restrict__ s, long ld, int S, bool store,
                                         double* __restrict__ out_base, long obs_ld,
                                         const double* __restrict__ T, QuadX& x, int lane,
                                         bool fin) {
#define F(k) s[(long)(k) * ld]
  Aircraft a;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    a.p[j] = F(F16S_POS + j); a.v[j] = F(F16S_VEL + j); a.wi[j] = F(F16S_PQRI + j);
    a.ai[j] = F(F16S_UVWIDOT + j); a.wdi[j] = F(F16S_PQRIDOT + j);
    a.vh1[j] = F(F16S_DIVEL + j); a.vh2[j] = F(F16S_DIVEL + 3 + j); a.ah1[j] = F(F16S_DUVW + j);
    x[kQPba + j][lane] = F(F16S_PBA + j); x[kQPpd + j][lane] = F(F16S_PPQRIDOT + j);
    x[kQPpq + j][lane] = F(F16S_PPQRI + j);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) { a.q[j] = F(F16S_Q + j); a.qd[j] = F(F16S_QDOT + j); }
  a.epa = F(F16S_EPA);
  unsigned hist_m = 0u;   // as split_flight: only the entries shifted when S < 3 need a test
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
  const bool out = out_base != nullptr && store;   // the 17-value output, written where formed
  double uvw[3] = {0.0, 0.0, 0.0}, wpqr[3] = {0.0, 0.0, 0.0};
  AuxGeo g;
  double gi[3] = {0.0, 0.0, 0.0};
  for (int t = 0; t < S; ++t) {
    const int slot = S - 1 - t;
    const int mo = quad_mass_block(t);
    // ---- phase A
    quad_prio<3, PRIO>();
    if (store && slot <= 2) {
      double* h = s;                // the history addresses are formed here (see the stores
      asm volatile("" : "+v"(h));   // after the loop)
#define H(k) h[(long)(k) * ld]
#pragma unroll
      for (int j = 0; j < 4; ++j) put(&H(F16S_DQ + 4 * slot + j), a.qd[j]);
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        put(&H(F16S_DPQRI + 3 * slot + j), a.wdi[j]);
        put(&H(F16S_DIVEL + 3 * slot + j), a.v[j]);
        put(&H(F16S_DUVW + 3 * slot + j), a.ai[j]);
      }
#undef H
    }
    propagate(a);
    if (store && slot == 0) {
      double* h = s;
      asm volatile("" : "+v"(h));
#define H(k) h[(long)(k) * ld]
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        put(&H(F16S_POS + j), a.p[j]); put(&H(F16S_VEL + j), a.v[j]); put(&H(F16S_PQRI + j), a.wi[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) put(&H(F16S_Q + j), a.q[j]);
      put(&H(F16S_EPA), a.epa);
#undef H
    }
    Kin kg;   // only what gravity reads in phase C is carried past this phase
    double vn, ve;
    {
      Kin k;
      double ce, se;
      if (t == 0) {
        sincos(a.epa, &se, &ce);
      } else {
        ce = x[kQCe][lane];
        se = x[kQSe][lane];
      }
      double euler[3];
      kinematics(a.p, a.v, a.q, a.wi, ce, se, slot == 0 && out_base != nullptr, k, euler);
      const double alt = k.radius - kSemiMajor;
      if (slot == 0 && out) {   // p and v are final here: phase D does not change them
        // the output's addresses are formed here from a pointer the compiler cannot see
        // through, not hoisted above the loop (17 of them, 2 registers each)
        double* o = out_base;
        asm volatile("" : "+v"(o));
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          o[(long)j * obs_ld] = a.p[j];
          o[(long)(3 + j) * obs_ld] = a.v[j];
          o[(long)(6 + j) * obs_ld] = euler[j];
          o[(long)(9 + j) * obs_ld] = k.uvw[j];
        }
        o[16L * obs_ld] = alt;
      }
      x[kQAlt][lane] = alt; x[kQCtcp][lane] = k.ctcp;
#pragma unroll
      for (int j = 0; j < 3; ++j) { uvw[j] = k.uvw[j]; wpqr[j] = k.wpqr[j]; }
      x[kQU][lane] = uvw[0]; x[kQV][lane] = uvw[1]; x[kQW][lane] = uvw[2];
      x[kQP][lane] = wpqr[0]; x[kQQ][lane] = wpqr[1]; x[kQR][lane] = wpqr[2];
      kg.ce = k.ce; kg.se = k.se; kg.ex = k.ex; kg.ey = k.ey; kg.ez = k.ez;
      kg.irad = k.irad; kg.sLat = k.sLat;
      vn = k.vn; ve = k.ve;
    }
    __syncthreads();
    // ---- phase B
    quad_prio<0, PRIO>();
    g = aux_geometry(uvw);
    if (slot == 0 && out) {
      double* o = out_base;
      asm volatile("" : "+v"(o));
      o[12L * obs_ld] = g.alpha; o[13L * obs_ld] = g.beta; o[15L * obs_ld] = g.vt;
    }
    double npy, npz;
    {
      const double cg[3] = {x[mo + kQCg][lane], x[mo + kQCg + 1][lane], x[mo + kQCg + 2][lane]};
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        a.pba[j] = x[kQPba + j][lane]; a.ppd[j] = x[kQPpd + j][lane]; a.ppq[j] = x[kQPpq + j][lane];
      }
      load_factors(a, cg, npy, npz);
    }
    x[kQNpy][lane] = npy; x[kQNpz][lane] = npz;
    __syncthreads();
    // ---- phase C
    quad_prio<3, PRIO>();
    {
      if (slot == 0 && out) {
        double* o = out_base;
        asm volatile("" : "+v"(o));
        o[14L * obs_ld] = fm_div(g.vt, x[kQSound][lane]);
      }
      x[kQVg][lane] = fm_sqrt(vn * vn + ve * ve);
      quat_rate(a);
      if (store && slot == 0) {
        double* h = s;
        asm volatile("" : "+v"(h));
#pragma unroll
        for (int j = 0; j < 4; ++j) put(&h[(long)(F16S_QDOT + j) * ld], a.qd[j]);
      }
      gravity(kg, gi);
    }
    __syncthreads();
    // ---- phase D
    quad_prio<3, PRIO>();
    {
      const double ax[6] = {x[kQAx0][lane], x[kQAx1][lane], x[kQAx2][lane], x[kQAx3][lane],
                            x[kQAx4][lane], x[kQAx5][lane]};
      const double thrust = x[kQThrust][lane];
      Mass mb;
      mb.mass = x[mo + kQMass][lane];
#pragma unroll
      for (int j = 0; j < 6; ++j) { mb.J[j] = x[mo + kQJ + j][lane]; mb.Jinv[j] = x[mo + kQJinv + j][lane]; }
#pragma unroll
      for (int j = 0; j < 3; ++j) { mb.rp[j] = x[mo + kQRp + j][lane]; mb.cg[j] = x[mo + kQCg + j][lane]; }
      double Fb[3], Mb[3];
      forces_moments(ax, g, mb, thrust, Fb, Mb);
      Accel ac;
      {
        double B[3][3];
        body_dcm(a.q, B);
        accelerations(B, wpqr, mb, Fb, Mb, gi, ac);
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        a.ai[i] = ac.ai[i]; a.wdi[i] = ac.wdi[i];
        x[kQPba + i][lane] = ac.pba[i]; x[kQPpd + i][lane] = ac.wdi[i]; x[kQPpq + i][lane] = ac.ppq[i];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    a.pba[j] = x[kQPba + j][lane]; a.ppd[j] = x[kQPpd + j][lane]; a.ppq[j] = x[kQPpq + j][lane];
  }
  quad_prio<0, PRIO>();
  // the state's addresses are formed here, from a pointer the compiler cannot see through:
  // hoisted above the substep loop they would stay live across it, 2 registers each
  asm volatile("" : "+v"(s));
  if (store && S > 0) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      put(&F(F16S_UVWIDOT + j), a.ai[j]); put(&F(F16S_PQRIDOT + j), a.wdi[j]);
      put(&F(F16S_PBA + j), a.pba[j]); put(&F(F16S_PPQRIDOT + j), a.ppd[j]);
      put(&F(F16S_PPQRI + j), a.ppq[j]);
    }
  }
#undef F
  if (fin) {
    unsigned m = fin_acc(hist_m, a.epa);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      m = fin_acc(fin_acc(fin_acc(fin_acc(m, a.p[j]), a.v[j]), a.wi[j]), a.ai[j]);
      m = fin_acc(fin_acc(fin_acc(fin_acc(m, a.wdi[j]), a.pba[j]), a.ppd[j]), a.ppq[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) m = fin_acc(fin_acc(m, a.q[j]), a.qd[j]);
    x[kQFinKin][lane] = m < kFinInf ? 1.0 : 0.0;
    __syncthreads();
  }
}

// ---- aero: the six axes of the aero build-up.  Holds no state.
template <int FCS_RATE, bool PRIO = false>
__device__ __forceinline__ void quad_aero(int S, const double* __restrict__ T, QuadX& x,
                                          int lane, bool fin) {
  for (int t = 0; t < S; ++t) {
    __syncthreads();
    // ---- phase B
    quad_prio<3, PRIO>();
    const double uvw[3] = {x[kQU][lane], x[kQV][lane], x[kQW][lane]};
    const AuxGeo g = aux_geometry(uvw);
    x[kQVt][lane] = g.vt; x[kQAlpha][lane] = g.alpha;
    const double alpha = g.alpha, beta = g.beta;
    const double ail = x[kQAil][lane], rud = x[kQRud][lane];
    double e0, e1, e2, e3, e4, e5;
    {
      const double lef = x[kQLef][lane], flap = x[kQFlap][lane];
      double bi2vel, ci2vel;
      aero_rates(g.vt, bi2vel, ci2vel);
      constexpr double kclge = kCLge;
      constexpr double gear = kGearPos<FCS_RATE>;
      const double p = x[kQP][lane], q = x[kQQ][lane], r = x[kQR][lane];
      F16_AERO_BRACKETS_AB;
      F16_AERO_LOOKUPS_AB;
      e0 = F16_AERO_DRAG_EARLY; e1 = F16_AERO_SIDE_EARLY; e2 = F16_AERO_LIFT_EARLY;
      e3 = F16_AERO_ROLL_EARLY; e4 = F16_AERO_PITCH_EARLY; e5 = F16_AERO_YAW_EARLY;
    }
    __syncthreads();
    // ---- phase C
    quad_prio<3, PRIO>();
    {
      const double rho = x[kQRho][lane], sound = x[kQSound][lane], elev = x[kQElev][lane];
      const double qbar = 0.5 * rho * g.vt2;
      const double mach = fm_div(g.vt, sound);
      constexpr double kclge = kCLge;
      const F16Br2 b2_G9_ALPHA = F16_BR2(G9_ALPHA, alpha);
      F16_AERO_BRACKETS_MACH;
      F16_AERO_BRACKETS_ELEV;
      F16_AERO_LOOKUPS_MACH;
      F16_AERO_LOOKUPS_ELEV;
      x[kQAx0][lane] = F16_AERO_DRAG_SCALE * (e0 + F16_AERO_DRAG_LATE);
      x[kQAx1][lane] = F16_AERO_SIDE_SCALE * (e1 + F16_AERO_SIDE_LATE);
      x[kQAx2][lane] = F16_AERO_LIFT_SCALE * (e2 + F16_AERO_LIFT_LATE);
      x[kQAx3][lane] = F16_AERO_ROLL_SCALE * (e3 + F16_AERO_ROLL_LATE);
      x[kQAx4][lane] = F16_AERO_PITCH_SCALE * (e4 + F16_AERO_PITCH_LATE);
      x[kQAx5][lane] = F16_AERO_YAW_SCALE * (e5 + F16_AERO_YAW_LATE);
    }
    __syncthreads();
    quad_prio<0, PRIO>();
  }
  if (fin) __syncthreads();
}

// ---- fcs: the FCS channels and the previous-frame auxiliary values.
template <int FCS_RATE, bool PRIO = false>
__device__ __forceinline__ void quad_fcs(double* __restrict__ s, long ld,
                                         const double* __restrict__ act4, int S, bool store,
                                         const double* __restrict__ T, QuadX& x, int lane,
                                         bool fin, double* __restrict__ keep) {
#define F(k) s[(long)(k) * ld]
  Aircraft a;
#pragma unroll
  for (int j = 0; j < 3; ++j) { a.pid_ip[j] = F(F16S_PID + 3 * j); a.pid_io[j] = F(F16S_PID + 3 * j + 2); }
#pragma unroll
  for (int j = 0; j < 9; ++j) a.pa[j] = F(F16S_PAUX + j);
  a.k_tef = F(F16S_KIN); a.k_ail = F(F16S_KIN + 1); a.k_ele = F(F16S_KIN + 2); a.k_lef = F(F16S_KIN + 5);
  const double c_ail = act4[0], c_ele = act4[1], c_rud = act4[2];
  if (keep && store) { keep[0] = c_ail; keep[1] = c_ele; keep[2] = c_rud; keep[3] = act4[3]; }
  double k_rud = 0.0;
  unsigned ip2_m = 0u;
  for (int t = 0; t < S; ++t) {
    const int slot = S - 1 - t;
    // ---- phase A
    quad_prio<2, PRIO>();
    if (store && slot == 0) {   // PID input_prev2 = input_prev before the final update
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        F(F16S_PID + 3 * j + 1) = a.pid_ip[j];
        ip2_m = fin_acc(ip2_m, a.pid_ip[j]);
      }
    }
    FcsOut fc;
    const double esch = fcs_prev_frame<FCS_RATE>(a, c_ail, c_ele, c_rud, T, fc);
    k_rud = fc.k_rud;
    x[kQAil][lane] = fc.ail; x[kQRud][lane] = fc.rud; x[kQLef][lane] = fc.lef; x[kQFlap][lane] = fc.flap;
    __syncthreads();
    // ---- phase B
    quad_prio<0, PRIO>();
    const double p = x[kQP][lane], q = x[kQQ][lane], r = x[kQR][lane];
    fcs_pitch<FCS_RATE>(a, esch, x[kQCtcp][lane], fc);
    x[kQElev][lane] = fc.elev;
    // the previous-frame values are next read by the next substep's channels: each is stored
    // as soon as it is formed, after fcs_pitch has read the old ones
    a.pa[6] = p; a.pa[7] = q; a.pa[8] = r;
    if (store && slot == 0) {
      double* h = s;
      asm volatile("" : "+v"(h));
#define H(k) h[(long)(k) * ld]
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        put(&H(F16S_PID + 3 * j), a.pid_ip[j]); put(&H(F16S_PID + 3 * j + 2), a.pid_io[j]);
        put(&H(F16S_PAUX + 6 + j), a.pa[6 + j]);
      }
      put(&H(F16S_KIN), a.k_tef); put(&H(F16S_KIN + 1), a.k_ail); put(&H(F16S_KIN + 2), a.k_ele);
      put(&H(F16S_KIN + 3), k_rud); put(&H(F16S_KIN + 4), kGearPos<FCS_RATE>);
      put(&H(F16S_KIN + 5), a.k_lef);
#undef H
    }
    __syncthreads();
    // ---- phase C
    quad_prio<0, PRIO>();
    a.pa[4] = x[kQNpy][lane]; a.pa[5] = x[kQNpz][lane];
    a.pa[0] = x[kQAlpha][lane];
    const double mach = fm_div(x[kQVt][lane], x[kQSound][lane]);
    a.pa[1] = mach;
    a.pa[2] = vc_knots(mach, x[kQPres][lane]);
    if (store && slot == 0) {
      double* h = s;
      asm volatile("" : "+v"(h));
#define H(k) h[(long)(k) * ld]
      put(&H(F16S_PAUX), a.pa[0]); put(&H(F16S_PAUX + 1), a.pa[1]); put(&H(F16S_PAUX + 2), a.pa[2]);
      put(&H(F16S_PAUX + 4), a.pa[4]); put(&H(F16S_PAUX + 5), a.pa[5]);
#undef H
    }
    __syncthreads();
    // ---- phase D
    quad_prio<0, PRIO>();
    a.pa[3] = x[kQVg][lane];
  }
  asm volatile("" : "+v"(s));   // as in quad_kin: the store addresses are formed here
  if (store && S > 0) put(&F(F16S_PAUX + 3), a.pa[3]);   // vg, formed in phase D
#undef F
  if (fin) {
    unsigned m = fin_acc(fin_acc(fin_acc(ip2_m, a.k_tef), a.k_ail), a.k_ele);
    m = fin_acc(fin_acc(m, k_rud), a.k_lef);
#pragma unroll
    for (int j = 0; j < 3; ++j) m = fin_acc(fin_acc(m, a.pid_ip[j]), a.pid_io[j]);
#pragma unroll
    for (int j = 0; j < 9; ++j) m = fin_acc(m, a.pa[j]);
    x[kQFinFcs][lane] = m < kFinInf ? 1.0 : 0.0;
    __syncthreads();
  }
}

// ---- air: mass, atmosphere, engine and fuel.  With `fin` non-null, fin[0] <- 1 if all 101 state
// values are finite (its own, and the kin and fcs roles' flags after the last barrier).
template <int FCS_RATE, bool PRIO = false>
__device__ __forceinline__ void quad_air(double* __restrict__ s, long ld,
                                         const double* __restrict__ act4, int S, bool store,
                                         const double* __restrict__ T, QuadX& x, int lane,
                                         unsigned char* __restrict__ fin) {
#define F(k) s[(long)(k) * ld]
  Aircraft a;
  a.fuel = F(F16S_FUEL);
  a.epa = F(F16S_EPA);   // tracked with the kin role's increments; never stored here
  a.n1 = F(F16S_ENG); a.n2 = F(F16S_ENG + 1); a.n2n = F(F16S_ENG + 2); a.ff = F(F16S_ENG + 3);
  const double c_thr = act4[3];
  for (int t = 0; t < S; ++t) {
    const int mo = quad_mass_block(t);
    // ---- phase A
    quad_prio<0, PRIO>();
    a.epa += kRot * kDt;   // the kin role's propagate makes the same increment
    const Mass mb = mass_props(a.fuel);
    x[mo + kQMass][lane] = mb.mass;
#pragma unroll
    for (int j = 0; j < 6; ++j) { x[mo + kQJ + j][lane] = mb.J[j]; x[mo + kQJinv + j][lane] = mb.Jinv[j]; }
#pragma unroll
    for (int j = 0; j < 3; ++j) { x[mo + kQRp + j][lane] = mb.rp[j]; x[mo + kQCg + j][lane] = mb.cg[j]; }
    __syncthreads();
    // ---- phase B
    quad_prio<3, PRIO>();
    const Atmos at = isa(x[kQAlt][lane], T);
    x[kQRho][lane] = at.rho; x[kQSound][lane] = at.a; x[kQPres][lane] = at.P;
    if (t + 1 < S) {
      double sn, cn;
      sincos(a.epa + kRot * kDt, &sn, &cn);
      x[kQCe][lane] = cn;
      x[kQSe][lane] = sn;
    }
    __syncthreads();
    // ---- phase C
    quad_prio<3, PRIO>();
    const double mach = fm_div(x[kQVt][lane], at.a);
    double burn;
    x[kQThrust][lane] = engine(a, c_thr, at, mach, T, burn);
    if (store && t + 1 == S) {
      double* h = s;
      asm volatile("" : "+v"(h));
#define H(k) h[(long)(k) * ld]
      put(&H(F16S_ENG), a.n1); put(&H(F16S_ENG + 1), a.n2); put(&H(F16S_ENG + 2), a.n2n);
      put(&H(F16S_ENG + 3), a.ff);
#undef H
    }
    __syncthreads();
    // ---- phase D
    quad_prio<0, PRIO>();
    a.fuel -= burn;
  }
  asm volatile("" : "+v"(s));   // as in quad_kin
  if (store && S > 0) {
    put(&F(F16S_FUEL), a.fuel);
  }
#undef F
  if (fin) {
    unsigned m = fin_acc(fin_acc(fin_acc(fin_acc(0u, a.fuel), a.n1), a.n2), a.n2n);
    m = fin_acc(m, a.ff);
    __syncthreads();
    if (store)
      fin[0] = (m < kFinInf && x[kQFinKin][lane] != 0.0 && x[kQFinFcs][lane] != 0.0) ? 1 : 0;
  }
}

// ------------------------------------------------------------------ the kernel
// The four-role form: each 64 aircraft on four wavefronts, G groups per
// workgroup of 256 G threads.  G = 2: 16,384 engagements put two wavefronts on every SIMD (at
// most 256 registers each) where the two-wave kernel has one, the two groups' roles paired on
// each SIMD by quad_role.  G = 1: a batch too small to give every CU a two-group workgroup
// spreads over twice as many CUs, one wavefront per SIMD (the two group orders alternate
// between workgroups).  The same results bit for bit.  OBS: the 17-value output is written
// (its own instantiation: 255 registers with it, 225 without).
template <int FCS_RATE, bool OBS, int G>
__global__ __launch_bounds__(256 * G) void fdm_step_quad_kernel(
    double* __restrict__ st, long ld, const double* __restrict__ act, int nac, int S,
    double* __restrict__ obs, long obs_ld, unsigned char* __restrict__ fin,
    double* __restrict__ act_keep) {
  static_assert(G == 1 || G == kQuadGroups, "one or two 64-aircraft groups per workgroup");
  __shared__ double T[F16M_IMAGE_LEN];
  __shared__ QuadX X[G];
  stage_image<256 * G>(T);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int role = quad_role(G == 1 ? (int)(blockIdx.x & 1) : grp, wave & 3);
  const int i = blockIdx.x * (64 * G) + grp * 64 + lane;
  const bool store = i < nac;
  const int ia = store ? i : nac - 1;   // lanes past the batch shadow the last aircraft
  constexpr bool kPrio = G == kQuadGroups;   // two waves per SIMD to arbitrate between
  if (role == kRoleKin)
    quad_kin<FCS_RATE, kPrio>(st + ia, ld, S, store, OBS ? obs + ia : nullptr, obs_ld, T, X[grp],
                              lane, fin != nullptr);
  else if (role == kRoleAero)
    quad_aero<FCS_RATE, kPrio>(S, T, X[grp], lane, fin != nullptr);
  else if (role == kRoleFcs)
    quad_fcs<FCS_RATE, kPrio>(st + ia, ld, act + 4L * ia, S, store, T, X[grp], lane,
                              fin != nullptr, act_keep ? act_keep + 4L * ia : nullptr);
  else
    quad_air<FCS_RATE, kPrio>(st + ia, ld, act + 4L * ia, S, store, T, X[grp], lane,
                              fin ? fin + ia : nullptr);
}

}  // namespace f16
