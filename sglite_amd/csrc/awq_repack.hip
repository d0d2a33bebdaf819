// Post-load repack of AWQ checkpoint tensors into the CDNA4 tile layout, its
// inverse, and the two dequantisation probes.
//
// Replaces the Marlin post-load step (awq_marlin_repack, marlin_permute_scales,
// awq_to_marlin_zero_points; python/sglite/srt/model_executor/layers/
// quantization/awq_marlin.py:298-319, marlin_utils.py:168-352).  Unlike the
// Marlin zero-point path, nothing leaves the device.
#include "awq_device.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// AWQ: logical column 8j + i lives in nibble rev_order(i) = {0,4,1,5,2,6,3,7}[i]
// (awq_triton.py:53-62).  rev_order is also the inverse of awq_order.
__device__ __forceinline__ constexpr int rev_order(int i) { return (i >> 1) | ((i & 1) << 2); }
// Nibble p of an AWQ word (and of a tile word) holds {0,2,4,6,1,3,5,7}[p].
__device__ __forceinline__ constexpr int awq_order(int p) { return ((p & 3) << 1) | (p >> 2); }

__device__ __forceinline__ int64_t tile_word_index(int64_t n, int64_t k, int64_t KT) {
  const int64_t nt = n >> 4, c = n & 15;
  const int64_t kt = k >> 7, w = (k >> 5) & 3, lg = (k >> 3) & 3;
  return (nt * KT + kt) * kTileWords + (lg * 16 + c) * 4 + w;
}

// One thread per (8-row block, AWQ word column): an 8x8 nibble transpose.
__global__ void repack_weights_kernel(const uint32_t* __restrict__ qw, uint32_t* __restrict__ out, int64_t K,
                                      int64_t N, int64_t KT, int64_t NT) {
  const int64_t J = NT * 2;  // word columns incl. padding (16 columns per tile = 2 AWQ words)
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = KT * 16 * J;  // (KT*128/8) row blocks
  if (idx >= total) return;
  const int64_t j = idx % J;
  const int64_t kb8 = idx / J;
  const int64_t k0 = kb8 * 8;
  const bool valid = (k0 < K) && (j * 8 < N);
  uint32_t rows[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) rows[r] = valid ? qw[(k0 + r) * (N / 8) + j] : 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t q = (rows[awq_order(p)] >> (4 * rev_order(i))) & 0xFu;
      word |= q << (4 * p);
    }
    out[tile_word_index(j * 8 + i, k0, KT)] = word;
  }
}

template <typename T>
__global__ void repack_sz_kernel(const T* __restrict__ scales, const uint32_t* __restrict__ qz, T* __restrict__ s_out,
                                 uint64_t* __restrict__ z_out, int64_t N, int64_t NT, int64_t NG) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= NT * NG) return;
  const int64_t nt = idx / NG, g = idx % NG;
  uint64_t zw = 0;
  for (int c = 0; c < 16; ++c) {
    const int64_t n = nt * 16 + c;
    T s = (T)0.0f;
    uint64_t z = 0;
    if (n < N) {
      s = scales[g * N + n];
      z = (qz[g * (N / 8) + n / 8] >> (4 * rev_order(n & 7))) & 0xFu;
    }
    s_out[idx * 16 + c] = s;
    zw |= z << (4 * c);
  }
  z_out[idx] = zw;
}

__global__ void unrepack_weights_kernel(const uint32_t* __restrict__ wt, uint32_t* __restrict__ qw, int64_t K,
                                        int64_t N, int64_t KT) {
  const int64_t J = N / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (K / 8) * J) return;
  const int64_t j = idx % J, k0 = (idx / J) * 8;
  uint32_t cols[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cols[i] = wt[tile_word_index(j * 8 + i, k0, KT)];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int p = rev_order(r);  // row k0 + r sits in nibble rev_order(r)
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= ((cols[i] >> (4 * p)) & 0xFu) << (4 * rev_order(i));
    qw[(k0 + r) * J + j] = word;
  }
}

template <typename T>
__global__ void unrepack_sz_kernel(const T* __restrict__ s_in, const uint64_t* __restrict__ z_in,
                                   T* __restrict__ scales, uint32_t* __restrict__ qz, int64_t N, int64_t NG) {
  const int64_t J = N / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= NG * J) return;
  const int64_t g = idx / J, j = idx % J;
  uint32_t word = 0;
  for (int i = 0; i < 8; ++i) {
    const int64_t n = j * 8 + i, nt = n >> 4, c = n & 15;
    scales[g * N + n] = s_in[(nt * NG + g) * 16 + c];
    const uint32_t z = (uint32_t)(z_in[nt * NG + g] >> (4 * c)) & 0xFu;
    word |= z << (4 * rev_order(i));
  }
  qz[g * J + j] = word;
}

// Probe: plain scalar dequantisation of the AWQ tensors, one thread per word.
template <typename T>
__global__ void dequant_awq_kernel(const uint32_t* __restrict__ qw, const uint32_t* __restrict__ qz,
                                   const T* __restrict__ scales, T* __restrict__ out, int64_t K, int64_t N,
                                   int64_t G) {
  const int64_t J = N / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= K * J) return;
  const int64_t k = idx / J, j = idx % J, g = k / G;
  const uint32_t w = qw[idx], z = qz[g * J + j];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = (int)((w >> (4 * rev_order(i))) & 0xFu);
    const int zz = (int)((z >> (4 * rev_order(i))) & 0xFu);
    const float s = (float)scales[g * N + j * 8 + i];
    out[k * N + j * 8 + i] = (T)((float)(q - zz) * s);  // exact product, one rounding
  }
}

// Probe: dequantisation from the tile layout with the GEMM kernels' routine.
// One wave per tile; lane writes its 32 values.
template <typename DT>
__global__ void dequant_repacked_kernel(const u32x4* __restrict__ wt, const uint16_t* __restrict__ s_r,
                                        const uint64_t* __restrict__ z_r, typename DT::elem* __restrict__ out,
                                        int64_t K, int64_t N, int64_t KT, int64_t NG, int gshift) {
  const int64_t tile = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t nt = tile / KT, kt = tile % KT;
  const int c = lane & 15, lg = lane >> 4;
  const int64_t n = nt * 16 + c;
  const u32x4 q = wt[tile * 64 + lane];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int64_t kb = kt * 128 + 32 * w;
    if (kb >= K) continue;
    const int64_t g = kb >> gshift;
    const auto zs = Dq<DT>::make(zero_nibble(z_r[nt * NG + g], c), s_r[(nt * NG + g) * 16 + c]);
    const auto v = Dq<DT>::word(q[w], zs, dq_consts());
    if (n < N) {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[(kb + lg * 8 + e) * N + n] = v[e];
    }
  }
}

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace

Geom make_geom(int64_t M, int64_t N, int64_t K, int64_t G) {
  Geom g;
  g.M = M;
  g.N = N;
  g.K = K;
  g.G = (G == -1) ? K : G;
  g.NT = (N + 15) / 16;
  g.KT = (K + 127) / 128;
  g.NG = K / g.G;
  g.gshift = 31;
  g.cus = M > 0 ? device_cu_count() : 256;
  if (g.NG > 1) {
    int s = 0;
    while ((int64_t(1) << s) < g.G) ++s;
    g.gshift = s;  // G is a power of two whenever there is more than one group
  }
  return g;
}

hipError_t launch_repack(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype,
                         const Geom& g, void* w_out, void* s_out, void* z_out, hipStream_t s) {
  const int bs = 256;
  const int64_t nw = g.KT * 16 * g.NT * 2;
  hipLaunchKernelGGL(repack_weights_kernel, dim3(blocks_for(nw, bs)), dim3(bs), 0, s, (const uint32_t*)qweight,
                     (uint32_t*)w_out, g.K, g.N, g.KT, g.NT);
  const int64_t nsz = g.NT * g.NG;
  void* sbase = s_out;
  uint64_t* zbase = (uint64_t*)z_out;
  if (nsz == 0) return hipGetLastError();
  if (dtype == 0)
    hipLaunchKernelGGL(repack_sz_kernel<_Float16>, dim3(blocks_for(nsz, bs)), dim3(bs), 0, s,
                       (const _Float16*)scales, (const uint32_t*)qzeros, (_Float16*)sbase, zbase, g.N, g.NT, g.NG);
  else
    hipLaunchKernelGGL(repack_sz_kernel<__bf16>, dim3(blocks_for(nsz, bs)), dim3(bs), 0, s, (const __bf16*)scales,
                       (const uint32_t*)qzeros, (__bf16*)sbase, zbase, g.N, g.NT, g.NG);
  return hipGetLastError();
}

hipError_t launch_unrepack(const void* w, const void* sr, const void* zr, int dtype, const Geom& g,
                           int32_t* qweight, int32_t* qzeros, void* scales, hipStream_t s) {
  const int bs = 256;
  hipLaunchKernelGGL(unrepack_weights_kernel, dim3(blocks_for((g.K / 8) * (g.N / 8), bs)), dim3(bs), 0, s,
                     (const uint32_t*)w, (uint32_t*)qweight, g.K, g.N, g.KT);
  const void* sbase = sr;
  const uint64_t* zbase = (const uint64_t*)zr;
  const int64_t n = g.NG * (g.N / 8);
  if (dtype == 0)
    hipLaunchKernelGGL(unrepack_sz_kernel<_Float16>, dim3(blocks_for(n, bs)), dim3(bs), 0, s,
                       (const _Float16*)sbase, zbase, (_Float16*)scales, (uint32_t*)qzeros, g.N, g.NG);
  else
    hipLaunchKernelGGL(unrepack_sz_kernel<__bf16>, dim3(blocks_for(n, bs)), dim3(bs), 0, s, (const __bf16*)sbase,
                       zbase, (__bf16*)scales, (uint32_t*)qzeros, g.N, g.NG);
  return hipGetLastError();
}

hipError_t launch_dequant_awq(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype,
                              const Geom& g, void* w_out, hipStream_t s) {
  const int bs = 256;
  const int64_t n = g.K * (g.N / 8);
  if (dtype == 0)
    hipLaunchKernelGGL(dequant_awq_kernel<_Float16>, dim3(blocks_for(n, bs)), dim3(bs), 0, s,
                       (const uint32_t*)qweight, (const uint32_t*)qzeros, (const _Float16*)scales,
                       (_Float16*)w_out, g.K, g.N, g.G);
  else
    hipLaunchKernelGGL(dequant_awq_kernel<__bf16>, dim3(blocks_for(n, bs)), dim3(bs), 0, s,
                       (const uint32_t*)qweight, (const uint32_t*)qzeros, (const __bf16*)scales, (__bf16*)w_out,
                       g.K, g.N, g.G);
  return hipGetLastError();
}

hipError_t launch_dequant_repacked(const void* w, const void* sr, const void* zr, int dtype, const Geom& g,
                                   void* w_out, hipStream_t s) {
  const int64_t tiles = g.NT * g.KT;
  const uint16_t* sbase = (const uint16_t*)sr;
  const uint64_t* zbase = (const uint64_t*)zr;
  if (dtype == 0)
    hipLaunchKernelGGL(dequant_repacked_kernel<F16>, dim3((unsigned)tiles), dim3(64), 0, s, (const u32x4*)w, sbase,
                       zbase, (_Float16*)w_out, g.K, g.N, g.KT, g.NG, g.gshift);
  else
    hipLaunchKernelGGL(dequant_repacked_kernel<BF16>, dim3((unsigned)tiles), dim3(64), 0, s, (const u32x4*)w,
                       sbase, zbase, (__bf16*)w_out, g.K, g.N, g.KT, g.NG, g.gshift);
  return hipGetLastError();
}

}  // namespace sgl_awq
