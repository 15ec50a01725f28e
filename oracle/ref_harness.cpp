// ref_harness.cpp -- C entry points around the reference's own host-compilable FDM
// (cuda_fdm/gen/fdm.cuh + f16_gen.cuh, compiled with g++ straight from /root/reference by
// oracle/Makefile).  TEST INFRASTRUCTURE ONLY: the result (oracle/_ref/libf16ref_*.so) is a
// second, independent checker for the C restatement in f16_oracle.c and may serve as the
// "reference" CPU baseline.  fdm.cuh's FdmState is the 101-double row of cuda_fdm/ic.py:92-114.
#include <string.h>
#include "fdm.cuh"

static_assert(sizeof(FdmState) == 101 * sizeof(double), "FdmState must be 101 doubles");

// fdm_step_batch semantics (cuda_fdm/gen/fdm_kernel.cu:32-47): S steps with the action held,
// obs row = eci_pos, eci_vel, euler, vUVW, alpha, beta, mach, Vt, alt_asl.
extern "C" void ref_fdm_step_batch(double* states, const double* actions, long nac, int substeps,
                                   double* obs17, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
  for (long a = 0; a < nac; a++) {
    FdmState s;
    memcpy(&s, states + a * 101, sizeof s);
    FdmOut o;
    memset(&o, 0, sizeof o);
    const double* ac = actions + a * 4;
    for (int i = 0; i < substeps; i++) fdm_step(&s, ac[0], ac[1], ac[2], ac[3], &o);
    memcpy(states + a * 101, &s, sizeof s);
    if (obs17) {
      double* p = obs17 + a * 17;
      for (int k = 0; k < 3; k++) {
        p[k] = o.eci_pos[k]; p[3 + k] = o.eci_vel[k]; p[6 + k] = o.euler[k]; p[9 + k] = o.vUVW[k];
      }
      p[12] = o.alpha; p[13] = o.beta; p[14] = o.mach; p[15] = o.Vt; p[16] = o.alt_asl;
    }
  }
  (void)nthreads;
}

// ndec decisions x substeps with actions (ndec, nac, 4): the C1/C2 trajectory driver.
extern "C" void ref_fdm_rollout(double* states, const double* actions, long nac, int ndec,
                                int substeps, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
  for (long a = 0; a < nac; a++) {
    FdmState s;
    memcpy(&s, states + a * 101, sizeof s);
    FdmOut o;
    for (int d = 0; d < ndec; d++) {
      const double* ac = actions + ((long)d * nac + a) * 4;
      for (int i = 0; i < substeps; i++) fdm_step(&s, ac[0], ac[1], ac[2], ac[3], &o);
    }
    memcpy(states + a * 101, &s, sizeof s);
  }
  (void)nthreads;
}

extern "C" int ref_fcs_rate(void) { return (int)(1.0 / FCS_DT + 0.5); }
