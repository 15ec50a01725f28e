// fdm_kernels_f32.hip -- the batched F-16 step in single precision (GpuDogfight
// precision="fp32", cuda_fdm/gpu_env.py:33-58), with its C entry points (include/f16_fdm.h).
//
// The model is the fp64 one, not a second copy: build.py writes float copies of the model
// headers (fdm_quad.h, fdm_split.h, fdm_advance.h, fdm_device.h, fdm_image.h, f16_model_gen.h,
// f16_state.h, the generated tables) under _build/f32/ -- every double made float, every floating literal given an f suffix,
// the libm calls made their float forms, namespace f16 renamed f16f -- and this file includes
// those copies.  The reference derives its fp32 build from its fp64 source the same way
// (cuda_rt.to_fp32, cuda_fdm/tests/cuda_rt.py:150-160).
//
// The kernel is fdm_quad.h's four-role form, each 64 aircraft on four cooperating wavefronts
// (92-100 registers a lane in float: up to five wavefronts per SIMD).  Measured at 16,384
// tail-chase engagements, 6 substeps, HIP events around each launch: 27.9 us against 36.6 us
// for the fp64 build and 48.5 us for one lane per aircraft doing the whole substep in float
// (316 registers a lane, one wavefront per SIMD, and half the SIMDs without one: the same
// results bit for bit); at 65,536 engagements 66.5 us against 133 us in fp64.
// Layout as in fdm_kernels.hip: field k of aircraft a at states[k * ld + a], output (17, obs_ld).
#include <hip/hip_runtime.h>

#include "f32/fdm_quad.h"
#include "f16_capi_common.h"

// Compute units of the current device (cached per device).
static int f32_device_cus() {
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

// Same argument rules as f16_fdm_step_batch.
extern "C" int f16_fdm_step_batch_f32(float* states, long ld, const float* actions, int nac,
                                      int substeps, int fcs_rate, float* obs, long obs_ld,
                                      void* stream) {
  if (nac < 0 || substeps < 0 || ld < nac) return F16_EINVAL;
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  if (nac == 0) return 0;
  if (!states || !actions || (obs && obs_ld < nac)) return F16_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  // two 64-aircraft groups per workgroup once the batch gives every CU such a workgroup (as in
  // the fp64 build)
  const bool two = (long)nac >= (long)f16f::kQuadAircraft * f32_device_cus();
  float* keep = nullptr;
  unsigned char* fin = nullptr;
#define F16_QUAD(R, O, G)                                                                     \
  hipLaunchKernelGGL((f16f::fdm_step_quad_kernel<R, O, G>), dim3((nac + 64 * G - 1) / (64 * G)), \
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

// Footprint of the kernel as f16_fdm_kernel_info reports the fp64 one (no 17-value output, two
// groups per workgroup).
extern "C" int f16_fdm_kernel_info_f32(int fcs_rate, int* out4) {
  if (fcs_rate != 120 && fcs_rate != 60) return F16_ERATE;
  if (!out4) return F16_EINVAL;
  hipFuncAttributes at;
  const hipError_t e = hipFuncGetAttributes(
      &at, fcs_rate == 60 ? (const void*)f16f::fdm_step_quad_kernel<60, false, 2>
                          : (const void*)f16f::fdm_step_quad_kernel<120, false, 2>);
  if (e != hipSuccess) return -(1000 + (int)e);
  out4[0] = at.numRegs;
  out4[1] = (int)at.sharedSizeBytes;
  out4[2] = (int)at.localSizeBytes;
  out4[3] = at.maxThreadsPerBlock;
  return 0;
}
