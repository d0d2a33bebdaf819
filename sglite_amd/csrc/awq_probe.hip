// Streaming probe: the attainable HBM rate of a decode-sized launch.
//
// A decode GEMM reads a few MB of packed weights once.  At these sizes a
// launch's time is mostly fixed cost (dispatch, the first memory round trip,
// the final store and the end-of-kernel cache release) plus the bytes of the
// busiest CU, so the 8 TB/s peak is out of reach for reasons that have
// nothing to do with the GEMM's arithmetic.  This kernel measures what a
// launch of the same grid and block size can reach when it does nothing but
// stream the same number of bytes: every thread issues all of its 16-byte
// non-temporal loads before it consumes any, folds them into one word, and
// each workgroup stores one word (as a GEMM workgroup stores its outputs).
// The benchmark reports each decode linear against both the HBM peak and this
// ceiling.  No counterpart in the reference (measurement kernels).
#include "awq_device.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// Workgroup b streams the vectors [b * per_wg, min((b + 1) * per_wg, nvec)),
// LPT 16-byte loads per thread per round, all issued before the first is used.
template <int LPT>
__global__ __launch_bounds__(1024) void stream_probe_kernel(const u32x4* __restrict__ src, int64_t nvec,
                                                            int64_t per_wg, uint32_t* __restrict__ sink) {
  const int64_t b0 = (int64_t)blockIdx.x * per_wg;
  const int64_t b1 = min(b0 + per_wg, nvec);
  const int nt = blockDim.x;
  uint32_t acc = 0;
  for (int64_t base = b0 + threadIdx.x; base < b1; base += (int64_t)LPT * nt) {
    u32x4 v[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int64_t j = min(base + (int64_t)i * nt, b1 - 1);  // in range; duplicates fold harmlessly
      v[i] = __builtin_nontemporal_load(src + j);
    }
#pragma unroll
    for (int i = 0; i < LPT; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  }
  // One word per workgroup: every thread's fold, combined through LDS.
  __shared__ uint32_t red[16];
  for (int o = 32; o >= 1; o >>= 1) acc ^= __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int w = 0; w < (nt + 63) / 64; ++w) r ^= red[w];
    sink[blockIdx.x] = r;
  }
}

// MFMA probe: each wave runs `iters` rounds of eight independent
// v_mfma_f32_32x32x16_f16 (operands in registers, no memory traffic in the
// loop) and stores one word; the fp16 MFMA rate a launch of this grid can
// sustain on the device as clocked, the compute counterpart of the streaming
// probe.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x_acc __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_probe_kernel(int64_t iters, float* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  h8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (_Float16)(0.001f * (float)((lane + i) & 7));
    b[i] = (_Float16)(0.002f * (float)((lane * 3 + i) & 7));
  }
  f16x_acc acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
  }
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) r += acc[j][e];
  if (lane == 0) sink[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = r;
}

}  // namespace

hipError_t launch_mfma_probe(int64_t iters, int64_t grid, int block, float* sink, hipStream_t s) {
  hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)grid), dim3((unsigned)block), 0, s, iters, sink);
  return hipGetLastError();
}

hipError_t launch_stream_probe(const void* src, int64_t bytes, int64_t grid, int block, uint32_t* sink,
                               hipStream_t s) {
  const int64_t nvec = bytes / 16;
  const int64_t per_wg = (nvec + grid - 1) / grid;
  const int64_t per_thread = (per_wg + block - 1) / block;
  const dim3 g((unsigned)grid), b((unsigned)block);
  const u32x4* p = (const u32x4*)src;
  if (per_thread <= 1)
    hipLaunchKernelGGL(stream_probe_kernel<1>, g, b, 0, s, p, nvec, per_wg, sink);
  else if (per_thread <= 2)
    hipLaunchKernelGGL(stream_probe_kernel<2>, g, b, 0, s, p, nvec, per_wg, sink);
  else if (per_thread <= 4)
    hipLaunchKernelGGL(stream_probe_kernel<4>, g, b, 0, s, p, nvec, per_wg, sink);
  else if (per_thread <= 8)
    hipLaunchKernelGGL(stream_probe_kernel<8>, g, b, 0, s, p, nvec, per_wg, sink);
  else
    hipLaunchKernelGGL(stream_probe_kernel<16>, g, b, 0, s, p, nvec, per_wg, sink);
  return hipGetLastError();
}

}  // namespace sgl_awq
