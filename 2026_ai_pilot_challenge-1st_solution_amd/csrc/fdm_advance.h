// fdm_advance.h -- per-aircraft driver of the batched step: load the SoA state into registers,
// run S substeps with the action held, write the state (and optionally the 17-value output).
#pragma once
#include "fdm_device.h"

namespace f16 {

// Advance one aircraft: `s` points at its field 0 (fields `ld` apart), `o` at its output
// field 0 (or null).  Shared by the kernel and the CPU build of the same algorithm.
template <int FCS_RATE>
F16_HD void advance_aircraft(double* __restrict__ s, long ld, const double* __restrict__ act4,
                             int S, double* __restrict__ o, long obs_ld,
                             const double* __restrict__ T) {
#define F(k) s[(long)(k) * ld]
  Aircraft a;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    a.p[j] = F(F16S_POS + j); a.v[j] = F(F16S_VEL + j); a.wi[j] = F(F16S_PQRI + j);
    a.ai[j] = F(F16S_UVWIDOT + j); a.wdi[j] = F(F16S_PQRIDOT + j);
    a.vh1[j] = F(F16S_DIVEL + j); a.vh2[j] = F(F16S_DIVEL + 3 + j); a.ah1[j] = F(F16S_DUVW + j);
    a.pba[j] = F(F16S_PBA + j); a.ppd[j] = F(F16S_PPQRIDOT + j); a.ppq[j] = F(F16S_PPQRI + j);
    a.pid_ip[j] = F(F16S_PID + 3 * j); a.pid_io[j] = F(F16S_PID + 3 * j + 2);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) { a.q[j] = F(F16S_Q + j); a.qd[j] = F(F16S_QDOT + j); }
#pragma unroll
  for (int j = 0; j < 9; ++j) a.pa[j] = F(F16S_PAUX + j);
  a.epa = F(F16S_EPA); a.fuel = F(F16S_FUEL);
  a.n1 = F(F16S_ENG); a.n2 = F(F16S_ENG + 1); a.n2n = F(F16S_ENG + 2); a.ff = F(F16S_ENG + 3);
  a.k_tef = F(F16S_KIN); a.k_ail = F(F16S_KIN + 1); a.k_ele = F(F16S_KIN + 2); a.k_lef = F(F16S_KIN + 5);
  const double c_ail = act4[0], c_ele = act4[1], c_rud = act4[2], c_thr = act4[3];

  if (S <= 0) return;
  // History slots hold the last three pushed values, newest first.  Fewer than three substeps
  // keep older entries, shifted down by S.
  if (S < 3) {
    for (int k = 2; k >= S; --k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) F(F16S_DQ + 4 * k + j) = F(F16S_DQ + 4 * (k - S) + j);
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        F(F16S_DPQRI + 3 * k + j) = F(F16S_DPQRI + 3 * (k - S) + j);
        F(F16S_DIVEL + 3 * k + j) = F(F16S_DIVEL + 3 * (k - S) + j);
        F(F16S_DUVW + 3 * k + j) = F(F16S_DUVW + 3 * (k - S) + j);
      }
    }
  }
  SubstepOut out;
  for (int t = 0; t < S; ++t) {
    const int slot = S - 1 - t;
    if (slot <= 2) {   // values pushed onto the histories at the start of this substep
#pragma unroll
      for (int j = 0; j < 4; ++j) F(F16S_DQ + 4 * slot + j) = a.qd[j];
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        F(F16S_DPQRI + 3 * slot + j) = a.wdi[j];
        F(F16S_DIVEL + 3 * slot + j) = a.v[j];
        F(F16S_DUVW + 3 * slot + j) = a.ai[j];
      }
    }
    if (slot == 0) {   // PID input_prev2 = input_prev before the final update (trigger >= 0)
#pragma unroll
      for (int j = 0; j < 3; ++j) F(F16S_PID + 3 * j + 1) = a.pid_ip[j];
    }
    substep<FCS_RATE>(a, c_ail, c_ele, c_rud, c_thr, T, slot == 0 && o != nullptr, out);
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    F(F16S_POS + j) = a.p[j]; F(F16S_VEL + j) = a.v[j]; F(F16S_PQRI + j) = a.wi[j];
    F(F16S_UVWIDOT + j) = a.ai[j]; F(F16S_PQRIDOT + j) = a.wdi[j];
    F(F16S_PBA + j) = a.pba[j]; F(F16S_PPQRIDOT + j) = a.ppd[j]; F(F16S_PPQRI + j) = a.ppq[j];
    F(F16S_PID + 3 * j) = a.pid_ip[j]; F(F16S_PID + 3 * j + 2) = a.pid_io[j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) { F(F16S_Q + j) = a.q[j]; F(F16S_QDOT + j) = a.qd[j]; }
#pragma unroll
  for (int j = 0; j < 9; ++j) F(F16S_PAUX + j) = a.pa[j];
  F(F16S_EPA) = a.epa; F(F16S_FUEL) = a.fuel;
  F(F16S_ENG) = a.n1; F(F16S_ENG + 1) = a.n2; F(F16S_ENG + 2) = a.n2n; F(F16S_ENG + 3) = a.ff;
  F(F16S_KIN) = a.k_tef; F(F16S_KIN + 1) = a.k_ail; F(F16S_KIN + 2) = a.k_ele;
  F(F16S_KIN + 3) = out.k_rud; F(F16S_KIN + 4) = out.k_gear; F(F16S_KIN + 5) = a.k_lef;
#undef F
  if (o) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      o[(long)j * obs_ld] = a.p[j];
      o[(long)(3 + j) * obs_ld] = a.v[j];
      o[(long)(6 + j) * obs_ld] = out.euler[j];
      o[(long)(9 + j) * obs_ld] = out.uvw[j];
    }
    o[12L * obs_ld] = out.alpha; o[13L * obs_ld] = out.beta; o[14L * obs_ld] = out.mach;
    o[15L * obs_ld] = out.vt; o[16L * obs_ld] = out.alt;
  }
}

}  // namespace f16
