// Epilogue helper shared by the GEMM kernels.
#pragma once

#include "awq_device.h"

namespace sgl_awq {

// Round four fp32 accumulators to the output dtype, add the bias in that dtype
// (the reference adds bias to the already-rounded GEMM output, awq.py:145-146,
// marlin_utils.py:412-413) and store them (8 bytes).
template <typename DT>
__device__ __forceinline__ void store4(typename DT::elem* __restrict__ out, const typename DT::elem* __restrict__ bias,
                                       int64_t m, int64_t N, int64_t n0, f32x4 v) {
  using V4 = typename DT::vec4;
  using E = typename DT::elem;
  V4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (E)v[i];
  if (bias != nullptr) {
    const V4 b = *(const V4*)(bias + n0);
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (E)((float)r[i] + (float)b[i]);
  }
  *(V4*)(out + m * N + n0) = r;
}

}  // namespace sgl_awq
