// Epilogue helper shared by the GEMM kernels.
#pragma once

#include <math.h>

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

// Gated activations of the fused gate/up epilogue (activation.py:11-23):
// silu(g) = g / (1 + exp(-g)), gelu(g) = g / 2 * (1 + erf(g / sqrt(2))).
enum : int { kActNone = 0, kActSilu = 1, kActGelu = 2 };

__device__ __forceinline__ float gated_act(int act, float g) {
  return act == kActSilu ? g / (1.f + expf(-g)) : 0.5f * g * (1.f + erff(g * 0.70710678118654752f));
}

// Fused gate/up output of four columns o0..o0+3: the gate and up sums are each
// rounded to the output dtype with their bias added in that dtype (gate bias
// at o0, up bias nh columns further: the merged projection's two halves),
// exactly as the unfused GEMM stores them; then act(gate) * up in fp32,
// rounded once (silu_and_mul / gelu_and_mul).  Output row stride ldo.
template <typename DT>
__device__ __forceinline__ void store4_act(typename DT::elem* __restrict__ out,
                                           const typename DT::elem* __restrict__ bias, int64_t m, int64_t ldo,
                                           int64_t o0, int64_t nh, f32x4 g, f32x4 u, int act) {
  using V4 = typename DT::vec4;
  using E = typename DT::elem;
  V4 rg, ru, r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    rg[i] = (E)g[i];
    ru[i] = (E)u[i];
  }
  if (bias != nullptr) {
    const V4 bg = *(const V4*)(bias + o0);
    const V4 bu = *(const V4*)(bias + nh + o0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      rg[i] = (E)((float)rg[i] + (float)bg[i]);
      ru[i] = (E)((float)ru[i] + (float)bu[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (E)(gated_act(act, (float)rg[i]) * (float)ru[i]);
  *(V4*)(out + m * ldo + o0) = r;
}

}  // namespace sgl_awq
