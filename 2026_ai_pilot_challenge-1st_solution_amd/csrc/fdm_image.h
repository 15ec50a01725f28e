// fdm_image.h -- the F-16 model image (the aero and engine tables and the model constants of
// f16_model_gen.h, 1,635 doubles) in constant memory, and its copy into LDS at the start of
// every kernel that runs the flight model.  Each translation unit that includes this header
// holds its own copy of the image (internal linkage).
#pragma once
#include <hip/hip_runtime.h>

#include "f16_model_gen.h"

namespace f16 {

static __constant__ double c_image[F16M_IMAGE_LEN] = F16M_IMAGE_INIT;

// Copy the model image into LDS: every load of a thread is issued before its first store, so
// the copy costs one memory latency rather than one per element.  NT = threads per block.
template <int NT>
__device__ __forceinline__ void stage_image(double* T) {
  constexpr int kPer = (F16M_IMAGE_LEN + NT - 1) / NT;
  double v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = threadIdx.x + j * NT;
    v[j] = i < F16M_IMAGE_LEN ? c_image[i] : 0.0;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < F16M_IMAGE_LEN) T[i] = v[j];
  }
  __syncthreads();
}

}  // namespace f16
