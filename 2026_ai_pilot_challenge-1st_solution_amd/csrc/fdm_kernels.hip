// fdm_kernels.hip -- gfx950 kernels for the batched F-16 step and the device-side IC seeding,
// plus their C entry points (declared in include/f16_fdm.h).
//
// Layout: states are structure-of-arrays, field k of aircraft a at states[k * ld + a]
// (f16_state.h); actions are the reference's (nac, 4) rows [aileron, elevator, rudder,
// throttle]; the optional FDM output is structure-of-arrays too, (17, obs_ld).
#include <hip/hip_runtime.h>

#include "fdm_advance.h"
#include "fdm_image.h"
#include "fdm_quad.h"
#include "fdm_split.h"
#include "f16_capi_common.h"

namespace f16 {

constexpr int kBlock = 256;

// ------------------------------------------------------------------ batched substeps
// One lane per aircraft; `S` substeps with the action held, state in registers throughout
// (fdm_step_batch semantics, cuda_fdm/gen/fdm_kernel.cu:32-47).
template <int FCS_RATE>
__global__ __launch_bounds__(kBlock) void fdm_step_kernel(double* __restrict__ st, long ld,
                                                          const double* __restrict__ act, int nac,
                                                          int S, double* __restrict__ obs,
                                                          long obs_ld) {
  __shared__ double T[F16M_IMAGE_LEN];
  stage_image<kBlock>(T);
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nac) return;
  advance_aircraft<FCS_RATE>(st + i, ld, act + 4L * i, S, obs ? obs + i : nullptr, obs_ld, T);
}

// Two wavefronts per 64 aircraft (fdm_split.h): even waves fly, odd waves run the systems.
// The role is wave-uniform (a scalar branch), so each role's loop issues its own barriers and
// the two loops' barrier counts match (3 per substep each).
// `fin` (optional, S >= 1): per aircraft, 1 if all 101 state values after the call are finite.
template <int FCS_RATE>
__global__ __launch_bounds__(kSplitBlock) void fdm_step_split_kernel(
    double* __restrict__ st, long ld, const double* __restrict__ act, int nac, int S,
    double* __restrict__ obs, long obs_ld, unsigned char* __restrict__ fin,
    double* __restrict__ act_keep) {
  __shared__ double T[F16M_IMAGE_LEN];
  __shared__ SplitX X[kSplitPairs];
  stage_image<kSplitBlock>(T);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pair = wave >> 1;
  const int i = blockIdx.x * kSplitAircraft + pair * 64 + lane;
  const bool store = i < nac;
  const int ia = store ? i : nac - 1;   // lanes past the batch shadow the last aircraft
  if ((wave & 1) == 0)
    split_flight<FCS_RATE>(st + ia, ld, S, store, obs ? obs + ia : nullptr, obs_ld, T, X[pair],
                           lane, fin != nullptr);
  else
    split_systems<FCS_RATE>(st + ia, ld, act + 4L * ia, S, store, T, X[pair], lane,
                            fin ? fin + ia : nullptr, act_keep ? act_keep + 4L * ia : nullptr);
}

// ------------------------------------------------------------------ IC seeding
// build_seed_vector (cuda_fdm/ic.py:117-138): geodetic IC -> ECI state, attitude quaternion,
// and the derivatives of one throwaway force path at throttle 0.8 (FDM.seed,
// cuda_fdm/ref/jsb_fdm.py:142-210).  Row r of `ic` seeds aircraft rows[r] (or r).
__device__ __forceinline__ void mat_to_quat_dev(const double m[3][3], double Q[4]) {
  // FGMatrix33 data[] is column-major (jsb_frames.py:110-137)
  const double d[9] = {m[0][0], m[1][0], m[2][0], m[0][1], m[1][1], m[2][1], m[0][2], m[1][2], m[2][2]};
  const double t[4] = {1.0 + d[0] + d[4] + d[8], 1.0 + d[0] - d[4] - d[8],
                       1.0 - d[0] + d[4] - d[8], 1.0 - d[0] - d[4] + d[8]};
  int idx = 0;
  for (int i = 1; i < 4; ++i) if (t[i] > t[idx]) idx = i;
  if (idx == 0) {
    Q[0] = 0.5 * sqrt(t[0]);
    Q[1] = 0.25 * (d[7] - d[5]) / Q[0]; Q[2] = 0.25 * (d[2] - d[6]) / Q[0]; Q[3] = 0.25 * (d[3] - d[1]) / Q[0];
  } else if (idx == 1) {
    Q[1] = 0.5 * sqrt(t[1]);
    Q[0] = 0.25 * (d[7] - d[5]) / Q[1]; Q[2] = 0.25 * (d[3] + d[1]) / Q[1]; Q[3] = 0.25 * (d[2] + d[6]) / Q[1];
  } else if (idx == 2) {
    Q[2] = 0.5 * sqrt(t[2]);
    Q[0] = 0.25 * (d[2] - d[6]) / Q[2]; Q[1] = 0.25 * (d[3] + d[1]) / Q[2]; Q[3] = 0.25 * (d[7] + d[5]) / Q[2];
  } else {
    Q[3] = 0.5 * sqrt(t[3]);
    Q[0] = 0.25 * (d[3] - d[1]) / Q[3]; Q[1] = 0.25 * (d[6] + d[2]) / Q[3]; Q[2] = 0.25 * (d[7] + d[5]) / Q[3];
  }
}

template <int FCS_RATE>
__global__ __launch_bounds__(kBlock) void seed_kernel(const double* __restrict__ ic, int n,
                                                      double* __restrict__ st, long ld,
                                                      const long* __restrict__ rows) {
  __shared__ double T[F16M_IMAGE_LEN];
  stage_image<kBlock>(T);
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const double* c = ic + (long)F16IC_N * r;
  constexpr double d2r = M_PI / 180.0;
  const double lat = c[0] * d2r, lon = c[1] * d2r, alt_ft = c[2], vt = c[3];
  const double phi = c[4] * d2r, tht = c[5] * d2r, psi = c[6] * d2r;
  const double alpha = c[7] * d2r, beta = c[8] * d2r, fuel = c[9];

  // geodetic_to_ecef (ic.py:18-45): point on the geodetic normal with |ecef| = a + alt
  double e[3];
  {
    constexpr double a = kSemiMajor, e2 = F16M_WGS_E2;
    double sphi, cphi, slam, clam;
    sincos(lat, &sphi, &cphi);
    sincos(lon, &slam, &clam);
    const double Nn = a / sqrt(1.0 - e2 * sphi * sphi);
    const double A = cphi * cphi, B = sphi * sphi, P = Nn, Q = Nn * (1.0 - e2);
    const double b = A * P + B * Q, cst = A * P * P + B * Q * Q, R = a + alt_ft;
    const double t = -b + sqrt(b * b - cst + R * R);
    e[0] = (Nn + t) * cphi * clam;
    e[1] = (Nn + t) * cphi * slam;
    e[2] = (Nn * (1.0 - e2) + t) * sphi;
  }
  // epa = 0: ECI = ECEF.  Local frame (location_derived, jsb_frames.py:30-51).
  const double rad = sqrt(e[0] * e[0] + e[1] * e[1] + e[2] * e[2]);
  const double rxy = sqrt(e[0] * e[0] + e[1] * e[1]);
  double sLon = 0.0, cLon = 1.0, sLat = 0.0, cLat = 1.0;
  if (rxy != 0.0) { sLon = e[1] / rxy; cLon = e[0] / rxy; }
  if (rad != 0.0) { sLat = e[2] / rad; cLat = rxy / rad; }
  const double Ti2l[3][3] = {{-cLon * sLat, -sLon * sLat, cLat}, {-sLon, cLon, 0.0},
                             {-cLon * cLat, -sLon * cLat, -sLat}};
  // attitude: Ti2b = Tl2b(euler) * Ti2l (euler_to_quat + quat_to_T, jsb_frames.py:84-107)
  double qL[4];
  {
    double St, Ct, Sp, Cp, Sf, Cf;
    sincos(0.5 * tht, &St, &Ct);
    sincos(0.5 * psi, &Sp, &Cp);
    sincos(0.5 * phi, &Sf, &Cf);
    const double CfCt = Cf * Ct, CfSt = Cf * St, SfSt = Sf * St, SfCt = Sf * Ct;
    qL[0] = CfCt * Cp + SfSt * Sp; qL[1] = SfCt * Cp - CfSt * Sp;
    qL[2] = CfSt * Cp + SfCt * Sp; qL[3] = CfCt * Sp - SfSt * Cp;
    const double mag = sqrt(qL[0] * qL[0] + qL[1] * qL[1] + qL[2] * qL[2] + qL[3] * qL[3]);
    if (mag != 0.0) { const double inv = 1.0 / mag; for (int j = 0; j < 4; ++j) qL[j] *= inv; }
  }
  double Tl2b[3][3], Ti2b[3][3];
  {
    const double q0 = qL[0], q1 = qL[1], q2 = qL[2], q3 = qL[3];
    Tl2b[0][0] = q0 * q0 + q1 * q1 - q2 * q2 - q3 * q3; Tl2b[0][1] = 2.0 * (q1 * q2 + q0 * q3); Tl2b[0][2] = 2.0 * (q1 * q3 - q0 * q2);
    Tl2b[1][0] = 2.0 * (q1 * q2 - q0 * q3); Tl2b[1][1] = q0 * q0 - q1 * q1 + q2 * q2 - q3 * q3; Tl2b[1][2] = 2.0 * (q2 * q3 + q0 * q1);
    Tl2b[2][0] = 2.0 * (q1 * q3 + q0 * q2); Tl2b[2][1] = 2.0 * (q2 * q3 - q0 * q1); Tl2b[2][2] = q0 * q0 - q1 * q1 - q2 * q2 + q3 * q3;
  }
  for (int i2 = 0; i2 < 3; ++i2)
    for (int j = 0; j < 3; ++j)
      Ti2b[i2][j] = Tl2b[i2][0] * Ti2l[0][j] + Tl2b[i2][1] * Ti2l[1][j] + Tl2b[i2][2] * Ti2l[2][j];
  double q[4];
  mat_to_quat_dev(Ti2b, q);
  // velocity: eci_vel = Tb2i * vUVW + omega x pos (ic.py:79-85)
  double sa, ca, sb, cb;
  sincos(alpha, &sa, &ca);
  sincos(beta, &sb, &cb);
  const double ub[3] = {vt * ca * cb, vt * sb, vt * sa * cb};
  double v[3], wi[3];
  for (int j = 0; j < 3; ++j) v[j] = Ti2b[0][j] * ub[0] + Ti2b[1][j] * ub[1] + Ti2b[2][j] * ub[2];
  v[0] += -kRot * e[1];
  v[1] += kRot * e[0];
  for (int j = 0; j < 3; ++j) wi[j] = 0.0 + Ti2b[j][2] * kRot;   // vPQR = 0 plus Ti2b * omega
  // prev-frame auxiliary values from the IC (ic.py:123-132)
  Aircraft s;
  {
    const Atmos at = isa(alt_ft, T);
    const double mach = vt / at.a;
    const double vc = (fabs(mach) > 0.0) ? vcal_from_mach(mach, at.P) * F16M_FPSTOKTS : 0.0;
    const double pa[9] = {alpha, mach, vc, vt, 0.0, -1.0, 0.0, 0.0, 0.0};
    for (int j = 0; j < 9; ++j) s.pa[j] = pa[j];
  }
  for (int j = 0; j < 3; ++j) {
    s.p[j] = e[j]; s.v[j] = v[j]; s.wi[j] = wi[j];
    s.pba[j] = 0.0; s.ppd[j] = 0.0; s.ppq[j] = wi[j];
    s.pid_ip[j] = 0.0; s.pid_io[j] = 0.0;
  }
  for (int j = 0; j < 4; ++j) s.q[j] = q[j];
  s.epa = 0.0; s.fuel = fuel;
  s.n1 = 100.0; s.n2 = 100.0; s.n2n = (100.0 - F16M_ENG_IDLEN2) / (F16M_ENG_MAXN2 - F16M_ENG_IDLEN2);
  s.ff = 0.0;
  s.k_tef = s.k_ail = s.k_ele = s.k_lef = 0.0;
  Kin k;
  double eul[3];
  kinematics(s.p, s.v, s.q, s.wi, 1.0, 0.0, false, k, eul);
  ForceOut f;
  force_path<FCS_RATE>(s, 0.0, 0.0, 0.0, 0.8, k, T, f);   // throwaway FCS/engine (reset below)
  double qd[4];
  {
    const double p = wi[0], qq = wi[1], rr = wi[2];
    qd[0] = -0.5 * (q[1] * p + q[2] * qq + q[3] * rr);
    qd[1] = 0.5 * (q[0] * p - q[3] * qq + q[2] * rr);
    qd[2] = 0.5 * (q[3] * p + q[0] * qq - q[1] * rr);
    qd[3] = 0.5 * (-q[2] * p + q[1] * qq + q[0] * rr);
  }
  const long a = rows ? rows[r] : r;
  if (a < 0 || a >= ld) return;            // a column outside the (101, ld) buffer: no write
  double* __restrict__ o = st + a;
#define F(kk) o[(long)(kk) * ld]
  for (int j = 0; j < 3; ++j) {
    F(F16S_POS + j) = e[j]; F(F16S_VEL + j) = v[j]; F(F16S_PQRI + j) = wi[j];
    F(F16S_UVWIDOT + j) = f.ai[j]; F(F16S_PQRIDOT + j) = f.wdi[j];
    F(F16S_PBA + j) = f.pba[j]; F(F16S_PPQRIDOT + j) = f.wdi[j]; F(F16S_PPQRI + j) = f.ppq[j];
    for (int h = 0; h < 3; ++h) {
      F(F16S_DPQRI + 3 * h + j) = f.wdi[j];
      F(F16S_DIVEL + 3 * h + j) = v[j];
      F(F16S_DUVW + 3 * h + j) = f.ai[j];
    }
  }
  for (int j = 0; j < 4; ++j) {
    F(F16S_Q + j) = q[j]; F(F16S_QDOT + j) = qd[j];
    for (int h = 0; h < 3; ++h) F(F16S_DQ + 4 * h + j) = qd[j];
  }
  F(F16S_EPA) = 0.0; F(F16S_FUEL) = fuel;
  for (int j = 0; j < 9; ++j) F(F16S_PAUX + j) = s.pa[j];
  F(F16S_ENG) = 100.0; F(F16S_ENG + 1) = 100.0;
  F(F16S_ENG + 2) = (100.0 - F16M_ENG_IDLEN2) / (F16M_ENG_MAXN2 - F16M_ENG_IDLEN2); F(F16S_ENG + 3) = 0.0;
  for (int j = 0; j < 15; ++j) F(F16S_KIN + j) = 0.0;
#undef F
}

}  // namespace f16

// ------------------------------------------------------------------ C entry points
static int fdm_step_args(double* states, long ld, const double* actions, int nac, int substeps,
                         int fcs_rate, double* obs, long obs_ld) {
  if (nac < 0 || substeps < 0 || ld < nac) return F16_EINVAL;
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  if (nac == 0) return 1;
  if (!states || !actions) return F16_EINVAL;
  if (obs && obs_ld < nac) return F16_EINVAL;
  return 0;
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

static int fdm_step_split(double* states, long ld, const double* actions, int nac, int substeps,
                          int fcs_rate, double* obs, long obs_ld, unsigned char* fin,
                          void* stream, double* keep = nullptr, bool quad = true) {
  hipStream_t s = (hipStream_t)stream;
  // The four-wave kernel (16k tail-chase engagements: 32.8 vs 36.7 us without the 17-value
  // output, 36.3 vs 37.8 us with it; 64k: 133 vs 144 us, 142 vs 147 us).  Two groups per
  // workgroup once the batch gives every CU such a workgroup, else one group per workgroup.
  if (quad) {
    const bool two = (long)nac >= (long)f16::kQuadAircraft * device_cus();
#define F16_QUAD(R, O, G)                                                                     \
  hipLaunchKernelGGL((f16::fdm_step_quad_kernel<R, O, G>), dim3((nac + 64 * G - 1) / (64 * G)), \
                     dim3(256 * G), 0, s, states, ld, actions, nac, substeps, obs, obs_ld, fin, \
                     keep)
#define F16_QUAD_G(R, O) do { if (two) F16_QUAD(R, O, 2); else F16_QUAD(R, O, 1); } while (0)
    if (fcs_rate == 120) {
      if (obs) F16_QUAD_G(120, true); else F16_QUAD_G(120, false);
    } else {
      if (obs) F16_QUAD_G(60, true); else F16_QUAD_G(60, false);
    }
#undef F16_QUAD_G
#undef F16_QUAD
    return f16_last_error();
  }
  const dim3 grid((nac + f16::kSplitAircraft - 1) / f16::kSplitAircraft), block(f16::kSplitBlock);
  if (fcs_rate == 120)
    hipLaunchKernelGGL(f16::fdm_step_split_kernel<120>, grid, block, 0, s, states, ld, actions, nac, substeps, obs, obs_ld, fin, keep);
  else
    hipLaunchKernelGGL(f16::fdm_step_split_kernel<60>, grid, block, 0, s, states, ld, actions, nac, substeps, obs, obs_ld, fin, keep);
  return f16_last_error();
}

extern "C" int f16_fdm_step_batch(double* states, long ld, const double* actions, int nac,
                                  int substeps, int fcs_rate, double* obs, long obs_ld,
                                  void* stream) {
  const int rc = fdm_step_args(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld);
  if (rc) return rc < 0 ? rc : 0;
  return fdm_step_split(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld, nullptr, stream);
}

extern "C" int f16_fdm_step_batch_finite(double* states, long ld, const double* actions, int nac,
                                         int substeps, int fcs_rate, double* obs, long obs_ld,
                                         unsigned char* finite, void* stream) {
  if (substeps < 1 || !finite) return F16_EINVAL;
  const int rc = fdm_step_args(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld);
  if (rc) return rc < 0 ? rc : 0;
  return fdm_step_split(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld, finite, stream);
}

extern "C" int f16_fdm_step_batch_keep(double* states, long ld, const double* actions,
                                       double* actions_keep, int nac, int substeps, int fcs_rate,
                                       double* obs, long obs_ld, unsigned char* finite,
                                       void* stream) {
  if (!actions_keep || (finite && substeps < 1)) return F16_EINVAL;
  const int rc = fdm_step_args(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld);
  if (rc) return rc < 0 ? rc : 0;
  // the kernel reads `actions` and writes `actions_keep` as separate arrays
  const uintptr_t a0 = (uintptr_t)actions, k0 = (uintptr_t)actions_keep;
  const uintptr_t bytes = (uintptr_t)nac * 4 * sizeof(double);
  if (a0 < k0 + bytes && k0 < a0 + bytes) return F16_EINVAL;
  return fdm_step_split(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld, finite, stream,
                        actions_keep);
}

extern "C" int f16_fdm_step_batch_split(double* states, long ld, const double* actions, int nac,
                                        int substeps, int fcs_rate, double* obs, long obs_ld,
                                        void* stream) {
  const int rc = fdm_step_args(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld);
  if (rc) return rc < 0 ? rc : 0;
  return fdm_step_split(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld, nullptr, stream,
                        nullptr, false);
}

extern "C" int f16_fdm_step_batch_onelane(double* states, long ld, const double* actions,
                                          int nac, int substeps, int fcs_rate, double* obs,
                                          long obs_ld, void* stream) {
  const int rc = fdm_step_args(states, ld, actions, nac, substeps, fcs_rate, obs, obs_ld);
  if (rc) return rc < 0 ? rc : 0;
  const dim3 grid((nac + f16::kBlock - 1) / f16::kBlock), block(f16::kBlock);
  hipStream_t s = (hipStream_t)stream;
  if (fcs_rate == 120)
    hipLaunchKernelGGL(f16::fdm_step_kernel<120>, grid, block, 0, s, states, ld, actions, nac, substeps, obs, obs_ld);
  else
    hipLaunchKernelGGL(f16::fdm_step_kernel<60>, grid, block, 0, s, states, ld, actions, nac, substeps, obs, obs_ld);
  return f16_last_error();
}

extern "C" int f16_seed_batch(const double* ic, int n, int fcs_rate, double* states, long ld,
                              const long* rows, void* stream) {
  if (n < 0 || ld < 1) return F16_EINVAL;
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  if (n == 0) return 0;
  if (!ic || !states || (!rows && ld < n)) return F16_EINVAL;
  const dim3 grid((n + f16::kBlock - 1) / f16::kBlock), block(f16::kBlock);
  hipStream_t s = (hipStream_t)stream;
  if (fcs_rate == 120)
    hipLaunchKernelGGL(f16::seed_kernel<120>, grid, block, 0, s, ic, n, states, ld, rows);
  else
    hipLaunchKernelGGL(f16::seed_kernel<60>, grid, block, 0, s, ic, n, states, ld, rows);
  return f16_last_error();
}

// Register/LDS/scratch footprint of the step kernel that f16_fdm_step_batch launches (the
// four-wave kernel without the 17-value output, two groups per workgroup, as at 16,384
// engagements; the reference's profile_kernel.py reads the same attributes from the CUDA
// driver).  out = {vgprs/regs per thread, lds bytes, scratch bytes, max threads per block}.
static int kernel_info(const void* fn, int* out4) {
  if (!out4) return F16_EINVAL;
  hipFuncAttributes at;
  hipError_t e = hipFuncGetAttributes(&at, fn);
  if (e != hipSuccess) return -(1000 + (int)e);
  out4[0] = at.numRegs;
  out4[1] = (int)at.sharedSizeBytes;
  out4[2] = (int)at.localSizeBytes;
  out4[3] = at.maxThreadsPerBlock;
  return 0;
}

extern "C" int f16_fdm_kernel_info(int fcs_rate, int* out4) {
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  return kernel_info(fcs_rate == 60 ? (const void*)f16::fdm_step_quad_kernel<60, false, 2>
                                    : (const void*)f16::fdm_step_quad_kernel<120, false, 2>, out4);
}

// The same for the one-lane kernel behind f16_fdm_step_batch_onelane.
extern "C" int f16_fdm_kernel_info_onelane(int fcs_rate, int* out4) {
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  return kernel_info(fcs_rate == 60 ? (const void*)f16::fdm_step_kernel<60>
                                    : (const void*)f16::fdm_step_kernel<120>, out4);
}
