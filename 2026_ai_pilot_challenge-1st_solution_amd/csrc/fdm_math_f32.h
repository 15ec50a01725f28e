// fdm_math_f32.h -- fm_rcp, fm_div, fm_sqrt, fm_exp, fm_log and fin_acc of the single-precision
// FDM build (precision="fp32").  build.py writes that build's model headers from the fp64 ones;
// their `#include "fdm_math.h"` becomes an include of this file.
//
// fp32 division and square root are correctly rounded by default in HIP, and the device
// library's expf and logf are within 1 ulp; the reference's fp32 build (an NVRTC compile of its
// fp64 source with every double made float, cuda_fdm/tests/cuda_rt.py:150-160) calls the same
// correctly rounded division and square root and CUDA's expf and logf.  The two builds
// therefore differ by at most a last-place rounding in exp and log, against the ~1e-7 relative
// rounding of every fp32 operation.
#pragma once

#include <hip/hip_runtime.h>

namespace f16f {

__device__ __forceinline__ float fm_rcp(float b) { return 1.0f / b; }
__device__ __forceinline__ float fm_div(float a, float b) { return a / b; }
__device__ __forceinline__ float fm_sqrt(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float fm_exp(float x) { return expf(x); }
__device__ __forceinline__ float fm_log(float x) { return logf(x); }

// Finite-flag accumulator: the largest IEEE exponent field seen; every value was finite iff the
// result is below kFinInf.
__device__ __forceinline__ unsigned fin_acc(unsigned m, float x) {
  return max(m, __float_as_uint(x) & 0x7f800000u);
}
constexpr unsigned kFinInf = 0x7f800000u;

}  // namespace f16f
