// Decode GEMV-regime W4A16 kernel (M <= 16) for gfx950.
//
// Each workgroup owns NTW column tiles of 16 columns and a k-range of its
// split-K slice; its WK waves take the slice's k-tiles round robin.  A launch
// of a decode-size layer (a few MB of int4 weights) is short enough that its
// time is set by how soon the weight loads are in flight, so a wave issues
// the loads of every k-tile it owns (weights, zero words, scales) before it
// computes anything, and waits for them one k-tile at a time.
//
// The activation slice of the workgroup (M rows x its k-range) is staged once
// through LDS: XPT 16-byte loads per thread, issued ahead of the weight loads
// so that their (L2) latency hides under the weights' HBM latency.  MFMA B
// fragments are then ds_read_b128 of that slice (rows >= M read row M - 1;
// their outputs are never stored).
//
// Per k-block the weights are dequantised exactly (Dq<DT>::word, the same
// rounding as the oracle) into the MFMA A operand and accumulated in fp32;
// the WK waves' partial sums are reduced through LDS by all threads, and
// split-K slices are combined across workgroups with the same fence-free
// atomic handoff as the wider decode kernel (device-scope exchanges and an
// arrival counter, fixed reduction order).
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410) for batches of up to 16 rows.
#include <algorithm>

#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

__device__ __forceinline__ float xchg_agent(float* p, float v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NTW, int WK, int KPW, int XPT, int GPT, typename DT>
__global__ __launch_bounds__(64 * WK) void gemv_kernel(
    const typename DT::elem* __restrict__ x, const u32x4* __restrict__ wt, const uint16_t* __restrict__ s_r,
    const uint64_t* __restrict__ z_r, const typename DT::elem* __restrict__ bias, typename DT::elem* __restrict__ out,
    float* __restrict__ part, int32_t* __restrict__ counters, int M, int N, int K, int NT, int KT, int NG, int gshift,
    int ktc, int KS) {
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  constexpr int NTHREADS = 64 * WK;
  constexpr int BPG = 4 / GPT;  // 32-row k-blocks per group
  // LDS: the activation slice (M x ktc*128 halves, row stride ktc*128 + 8), then
  // (after a barrier) the WK x NTW x 256 partial sums of the reduction.
  extern __shared__ u32x4 smem[];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, lg = lane >> 4;
  const int nt0 = blockIdx.x * NTW;
  const int kt_begin = blockIdx.y * ktc;
  const int kt_end = min(kt_begin + ktc, KT);
  const int nkt = kt_end - kt_begin;                        // k-tiles of this workgroup
  const int kpw = wave < nkt ? (nkt - 1 - wave) / WK + 1 : 0;  // k-tiles of this wave (<= KPW)
  const int rs = ktc * 128 + 8;                             // LDS row stride (halves)
  const DqK dk = dq_consts();

  // ---- activation slice: XPT chunks of 8 halves per thread --------------
  // chunk q -> row q / (16 ktc), halves 8 (q % (16 ktc)) of the k-range.
  u32x4 xr[XPT];
  const int cpr = ktc * 16;  // chunks per row
#pragma unroll
  for (int r = 0; r < XPT; ++r) {
    const int q = min(threadIdx.x + r * NTHREADS, M * cpr - 1);
    const int m = q / cpr, kk = (q % cpr) * 8;
    const int k = min(kt_begin * 128 + kk, K - 8);  // halves past K are zeroed when stored
    xr[r] = ld_off<u32x4>(x, ((uint32_t)m * (uint32_t)K + (uint32_t)k) * 2u);
  }

  // ---- weights, zero words and scales of every k-tile of this wave ---------
  u32x4 q[KPW][NTW];
  uint32_t zw[KPW][NTW][GPT];
  uint16_t sb[KPW][NTW][GPT];
  uint32_t woff[NTW], goff[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const uint32_t ntc = (uint32_t)min(nt0 + j, NT - 1);  // columns past N read a valid tile, never stored
    woff[j] = (ntc * (uint32_t)KT * 64u + lane) * 16u;
    goff[j] = ntc * (uint32_t)NG;
  }
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    // k-tiles past the wave's share reload its last one (no branch around loads)
    const int kt = kt_begin + wave + WK * min(i, max(kpw - 1, 0));
    const int ktl = min(kt, KT - 1);
#pragma unroll
    for (int j = 0; j < NTW; ++j) q[i][j] = ld_off_nt<u32x4>(wt, woff[j] + (uint32_t)ktl * 1024u);
#pragma unroll
    for (int gg = 0; gg < GPT; ++gg) {
      const uint32_t g = (uint32_t)min((ktl * 128 + 32 * BPG * gg) >> gshift, NG - 1);
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        const uint32_t gi = goff[j] + g;
        zw[i][j][gg] = ld_off<uint32_t>(z_r, gi * 8u + (uint32_t)(c >> 3) * 4u);
        sb[i][j][gg] = ld_off<uint16_t>(s_r, (gi * 16u + c) * 2u);
      }
    }
  }

  // ---- publish the activation slice ----------------------------------------
  _Float16* xs = (_Float16*)smem;
#pragma unroll
  for (int r = 0; r < XPT; ++r) {
    const int qi = threadIdx.x + r * NTHREADS;
    if (qi < M * cpr) {
      const int m = qi / cpr, kk = (qi % cpr) * 8;
      const bool kval = kt_begin * 128 + kk < K;
      *(u32x4*)(xs + m * rs + kk) = kval ? xr[r] : u32x4{0u, 0u, 0u, 0u};
    }
  }
  __syncthreads();

  // ---- compute ---------------------------------------------------------------
  f32x4 acc[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int xrow = min(c, M - 1) * rs + lg * 8;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    if (i < kpw) {
      const int kl = (wave + WK * i) * 128;  // k offset inside the slice
#pragma unroll
      for (int gg = 0; gg < GPT; ++gg) {
        ZS zs[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) zs[j] = Dq<DT>::make((zw[i][j][gg] >> (4 * (c & 7))) & 0xFu, sb[i][j][gg]);
#pragma unroll
        for (int b = 0; b < BPG; ++b) {
          const int w = gg * BPG + b;
          const V8 bx = __builtin_bit_cast(V8, *(const u32x4*)(xs + xrow + kl + 32 * w));
#pragma unroll
          for (int j = 0; j < NTW; ++j) acc[j] = mfma16x16x32(Dq<DT>::word(q[i][j][w], zs[j], dk), bx, acc[j]);
        }
      }
    }
  }

  // ---- reduce the WK waves: thread t sums quad t of every wave ---------------
  // quad (j, l) = column tile j, lane l: row l % 16, columns 4 (l / 16) + r.
  constexpr int NQ = NTW * 64;
  f32x4 res[(NQ + NTHREADS - 1) / NTHREADS];
  if constexpr (WK > 1) {
    __syncthreads();  // every wave is done reading the activation slice
    f32x4* red = (f32x4*)smem;
#pragma unroll
    for (int j = 0; j < NTW; ++j) red[(wave * NTW + j) * 64 + lane] = acc[j];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < (NQ + NTHREADS - 1) / NTHREADS; ++u) {
      const int qd = min((int)threadIdx.x + u * NTHREADS, NQ - 1);
      f32x4 s4 = red[qd];
#pragma unroll
      for (int o = 1; o < WK; ++o) s4 += red[o * NQ + qd];
      res[u] = s4;
    }
  } else {
#pragma unroll
    for (int j = 0; j < NTW; ++j) res[j] = acc[j];
  }

  // Quad u of this thread: tile j = qd / 64, lane l = qd % 64.
  auto quad_pos = [&](int u, int& m, int& n0) {
    const int qd = threadIdx.x + u * NTHREADS;
    const int l = qd & 63;
    m = l & 15;
    n0 = (nt0 + qd / 64) * 16 + 4 * (l >> 4);
    return qd < NQ;
  };

  if (KS == 1) {
#pragma unroll
    for (int u = 0; u < (NQ + NTHREADS - 1) / NTHREADS; ++u) {
      int m, n0;
      if (quad_pos(u, m, n0) && m < M && n0 < N) store4<DT>(out, bias, m, N, n0, res[u]);
    }
    return;
  }

  // ---- split-K handoff ------------------------------------------------------
  const int64_t Np = (int64_t)NT * 16;
  float chk = 0.f;
#pragma unroll
  for (int u = 0; u < (NQ + NTHREADS - 1) / NTHREADS; ++u) {
    int m, n0;
    if (quad_pos(u, m, n0) && m < M && n0 < Np) {
      float* p = part + ((int64_t)blockIdx.y * M + m) * Np + n0;
#pragma unroll
      for (int r = 0; r < 4; ++r) chk += xchg_agent(p + r, res[u][r]);
    }
  }
  // Consuming the returned values makes the wave wait until every exchange
  // has been performed before it reaches the barrier.
  asm volatile("" ::"v"(chk));
  __syncthreads();
  __shared__ int s_last;
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[blockIdx.x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == KS - 1);
  }
  __syncthreads();
  if (!s_last) return;
#pragma unroll
  for (int u = 0; u < (NQ + NTHREADS - 1) / NTHREADS; ++u) {
    int m, n0;
    if (quad_pos(u, m, n0) && m < M && n0 < N) {
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < KS; ++ks) {
        float* p = part + ((int64_t)ks * M + m) * Np + n0;
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] += xchg_agent(p + r, 0.f);
      }
      store4<DT>(out, bias, m, N, n0, sum);
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename DT>
hipError_t launch_gemv_dt(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                          const void* bias, void* out, const Geom& g, void* ws, int32_t* counters, hipStream_t s) {
  using E = typename DT::elem;
  const uint16_t* sbase = (const uint16_t*)sr;
  const uint64_t* zbase = (const uint64_t*)zr;
  const int ntw = p.variant / 1000, wk = (p.variant / 10) % 100, kpw = p.variant % 10;
  const int gpt = (g.NG > 1 && g.G < 128) ? (int)(128 / g.G) : 1;
  const int xpt = p.xpt;
  dim3 grid((unsigned)p.grid_x, (unsigned)p.grid_y);
  const size_t lds = (size_t)p.lds_bytes;
#define SGL_GEMV(NTW_, WK_, KPW_, XPT_, GPT_)                                                                       \
  if (ntw == NTW_ && wk == WK_ && kpw == KPW_ && xpt == XPT_ && gpt == GPT_) {                                      \
    hipLaunchKernelGGL((gemv_kernel<NTW_, WK_, KPW_, XPT_, GPT_, DT>), grid, dim3(64 * WK_), lds, s, (const E*)x,   \
                       (const u32x4*)w, sbase, zbase, (const E*)bias, (E*)out, (float*)ws, counters, (int)g.M,     \
                       (int)g.N, (int)g.K, (int)g.NT, (int)g.KT, (int)g.NG, g.gshift, p.ktc, p.ks);               \
    return hipGetLastError();                                                                                      \
  }
#define SGL_GEMV_G(NTW_, WK_, KPW_, XPT_) \
  SGL_GEMV(NTW_, WK_, KPW_, XPT_, 1) SGL_GEMV(NTW_, WK_, KPW_, XPT_, 2) SGL_GEMV(NTW_, WK_, KPW_, XPT_, 4)
#define SGL_GEMV_X(NTW_, WK_, KPW_) SGL_GEMV_G(NTW_, WK_, KPW_, 1) SGL_GEMV_G(NTW_, WK_, KPW_, 2) \
  SGL_GEMV_G(NTW_, WK_, KPW_, 4)
  SGL_GEMV_X(1, 4, 4)
  SGL_GEMV_X(1, 4, 8)
  SGL_GEMV_X(1, 8, 4)
  SGL_GEMV_X(2, 4, 4)
  SGL_GEMV_X(2, 4, 8)
  SGL_GEMV_X(2, 2, 8)
#undef SGL_GEMV_X
#undef SGL_GEMV_G
#undef SGL_GEMV
  return hipErrorInvalidValue;
}

}  // namespace

// Variant code: ntw * 1000 + wk * 10 + kpw.
bool gemv_variant_ok(int v) {
  switch (v) {
    case 1044: case 1048: case 1084: case 2044: case 2048: case 2028:
      return true;
    default:
      return false;
  }
}

hipError_t launch_gemv(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                       hipStream_t s) {
  return dtype == 0 ? launch_gemv_dt<F16>(p, x, w, sr, zr, bias, out, g, ws, counters, s)
                    : launch_gemv_dt<BF16>(p, x, w, sr, zr, bias, out, g, ws, counters, s);
}

}  // namespace sgl_awq
