// W4A16 GEMM kernels for gfx950: out[M, N] = x[M, K] @ W (+ bias), fp32 accumulation.
//
// Two kernels share the CDNA4 tile layout (awq_device.h):
//
//  * skinny_kernel (decode, M <= 32, awq_skinny.hip): HBM-bound split-K
//    kernel, one launch per linear.
//
//  * tiled_kernel (prefill, M > 32): MFMA-bound.  A workgroup computes
//    BM x 256 outputs; the activation tile (BM x 128 per k-step) is staged
//    through double-buffered LDS in MFMA-fragment order (conflict-free 16-byte
//    reads), and each wave dequantises the weights of its own 64 columns
//    straight from global memory into MFMA operands (no LDS round trip, no
//    redundant dequantisation across waves).
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410).
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// ---------------------------------------------------------------------------
// Tiled MFMA kernel: BM x 256 per workgroup, 4 waves of BM x 64.
// ---------------------------------------------------------------------------
template <int BM, typename DT>
__global__ __launch_bounds__(256) void tiled_kernel(const typename DT::elem* __restrict__ x,
                                                    const u32x4* __restrict__ wt, const uint16_t* __restrict__ s_r,
                                                    const uint64_t* __restrict__ z_r,
                                                    const typename DT::elem* __restrict__ bias,
                                                    typename DT::elem* __restrict__ out, int M, int N, int K, int NT,
                                                    int KT, int NG, int gshift) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  constexpr int MTL = BM / 16;
  constexpr int NTW = 4;
  // [buffer][m-tile][k-block][lane] -> 16 bytes: one MFMA B operand per (mt, kb)
  __shared__ u32x4 xs[2][MTL * 4 * 64];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, lg = lane >> 4;
  const int nt0 = blockIdx.x * 16 + wave * NTW;
  const DqK dk = dq_consts();
  const int64_t m0 = (int64_t)blockIdx.y * BM;

  f32x4 acc[MTL][NTW];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Loader: thread (wave, lane) fetches fragment (mt = i, kb = wave) of the
  // activation tile for i = 0..MTL-1.
  const E* xsrc[MTL];  // row starts (rows past M clamp to M - 1 and are zeroed)
  bool xval[MTL];
#pragma unroll
  for (int i = 0; i < MTL; ++i) {
    const int64_t m = m0 + i * 16 + c;
    xval[i] = m < M;
    xsrc[i] = x + min(m, (int64_t)M - 1) * K;
  }
  int ntc[NTW];
  const u32x4* wbase[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    ntc[j] = min(nt0 + j, NT - 1);
    wbase[j] = wt + (int64_t)ntc[j] * KT * 64 + lane;
  }

  u32x4 xr[MTL];
  u32x4 q[NTW], qn[NTW];
  auto load_x = [&](int kt) {
    // k-blocks past K (K % 128 != 0) read the row's first 16 bytes and are zeroed.
    const bool kval = kt * 128 + wave * 32 < K;
    const int64_t koff = kval ? (int64_t)kt * 128 + wave * 32 + lg * 8 : 0;
#pragma unroll
    for (int i = 0; i < MTL; ++i) {
      const u32x4 v = *(const u32x4*)(xsrc[i] + koff);
      xr[i] = (xval[i] && kval) ? v : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < MTL; ++i) xs[buf][(i * 4 + wave) * 64 + lane] = xr[i];
  };

  load_x(0);
#pragma unroll
  for (int j = 0; j < NTW; ++j) q[j] = wbase[j][0];
  store_x(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      load_x(kt + 1);
#pragma unroll
      for (int j = 0; j < NTW; ++j) qn[j] = wbase[j][(int64_t)(kt + 1) * 64];
    }
    int gprev = -1;
    ZS zs[NTW];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int kb = kt * 128 + 32 * w;
      if (kb >= K) break;
      const int g = kb >> gshift;
      if (g != gprev) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const int64_t gi = (int64_t)ntc[j] * NG + g;
          zs[j] = Dq<DT>::make(zero_nibble(z_r[gi], c), s_r[gi * 16 + c]);
        }
        gprev = g;
      }
      V8 a[NTW];
#pragma unroll
      for (int j = 0; j < NTW; ++j) a[j] = Dq<DT>::word(q[j][w], zs[j], dk);
#pragma unroll
      for (int mt = 0; mt < MTL; ++mt) {
        const V8 b = __builtin_bit_cast(V8, xs[cur][(mt * 4 + w) * 64 + lane]);
#pragma unroll
        for (int j = 0; j < NTW; ++j) acc[mt][j] = mfma16x16x32(a[j], b, acc[mt][j]);
      }
    }
    if (more) {
      store_x(cur ^ 1);
#pragma unroll
      for (int j = 0; j < NTW; ++j) q[j] = qn[j];
    }
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int64_t m = m0 + mt * 16 + c;
      const int n0 = (nt0 + j) * 16 + 4 * lg;
      if (m < M && n0 < N) store4<DT>(out, bias, m, N, n0, acc[mt][j]);
    }
}

// ---------------------------------------------------------------------------
// Planning and dispatch.
// ---------------------------------------------------------------------------
constexpr int kNumCU = 256;

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}

// Decode-kernel shapes that are instantiated (ntw * 10000 + wn * 100 + wk).
bool skinny_variant_ok(int v) {
  switch (v) {
    case 10104: case 10108: case 10116: case 10202: case 10401: case 10404:
    case 20202: case 20401: case 20204:
      return true;
    default:
      return false;
  }
}

template <typename DT>
hipError_t launch_tiled_dt(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                           const void* bias, void* out, const Geom& g, hipStream_t s) {
  using E = typename DT::elem;
  const uint16_t* sbase = (const uint16_t*)sr;
  const uint64_t* zbase = (const uint64_t*)zr;
  dim3 grid((unsigned)p.grid_x, (unsigned)p.grid_y);
#define SGL_TILED(BM_)                                                                                          \
  if (p.variant == BM_) {                                                                                     \
    hipLaunchKernelGGL((tiled_kernel<BM_, DT>), grid, dim3(256), 0, s, (const E*)x, (const u32x4*)w, sbase, zbase, \
                       (const E*)bias, (E*)out, (int)g.M, (int)g.N, (int)g.K, (int)g.NT, (int)g.KT, (int)g.NG,  \
                       g.gshift);                                                                             \
    return hipGetLastError();                                                                                 \
  }
  SGL_TILED(64)
  SGL_TILED(128)
  SGL_TILED(256)
#undef SGL_TILED
  return hipErrorInvalidValue;
}

}  // namespace

// GEMV plan (small M, one quantisation group per 128-row tile): every wave
// issues the loads of all its k-tiles at once.  Variant code
// ntw * 10000 + wn * 1000 + wk * 10 + kpw.  The rules come from a sweep of the
// variants and splits over the Qwen3-4B and Llama-3-8B decode shapes on
// MI355X; the split-K is the smallest that keeps each wave within its k-tile
// budget and the workgroup's activation slice within 8 loads per thread and
// 64 KiB of LDS.
// Where the GEMV kernel wins (same sweep): M <= 4, and M <= 8 on K <= 3072;
// at larger M the per-workgroup activation slice costs more than the wider
// decode kernel's per-wave fragments.
bool gemv_preferred(const Geom& g) {
  const int forced = env_int("SGL_AWQ_GEMV_MAX_M", -1);
  if (forced >= 0) return g.M <= forced;
  return g.M <= 4 || (g.M <= 8 && g.KT <= 24);
}

// 8 waves of at most 4 k-tiles, one column tile per workgroup.
int gemv_default_variant(const Geom&) { return 11084; }

bool plan_gemv(const Geom& g, GemmPlan& p) {
  if (g.NG > 1 && g.G < 128) return false;
  int v = gemv_default_variant(g);
  const int env = env_int("SGL_AWQ_GEMV_VARIANT", 0);
  if (gemv_variant_ok(env)) v = env;
  if (!gemv_variant_ok(v)) return false;
  const int ntw = v / 10000, wn = (v / 1000) % 10, wk = (v / 10) % 100, kpw = v % 10;
  const int64_t mt = (g.M + 15) / 16, threads = 64 * wn * wk;
  const int64_t gx = (g.NT + (int64_t)wn * ntw - 1) / ((int64_t)wn * ntw);
  int64_t ks = std::max<int64_t>(1, (g.KT + (int64_t)wk * kpw - 1) / ((int64_t)wk * kpw));
  const int env_ks = env_int("SGL_AWQ_GEMV_KS", 0);
  if (env_ks > 0) ks = env_ks;
  for (;;) {
    ks = std::max<int64_t>(1, std::min<int64_t>(ks, g.KT));
    const int64_t ktc = (g.KT + ks - 1) / ks;
    const int64_t xpt = (g.M * ktc * 16 + threads - 1) / threads;
    const int64_t lds = std::max<int64_t>(g.M * (ktc * 128 + 8) * 2, (int64_t)wk * wn * mt * ntw * 1024);
    if ((ktc + wk - 1) / wk > kpw || xpt > 8 || lds > 61440) {
      if (ks >= g.KT) return false;
      ks *= 2;
      continue;
    }
    p.kind = 2;
    p.variant = v;
    p.ktc = (int)ktc;
    p.ks = (int)((g.KT + ktc - 1) / ktc);
    p.xpt = xpt <= 1 ? 1 : (xpt <= 2 ? 2 : (xpt <= 4 ? 4 : 8));
    p.grid_x = gx;
    p.grid_y = p.ks;
    p.ws_bytes = p.ks > 1 ? (int64_t)p.ks * g.M * g.NT * 16 * 4 : 0;
    p.lds_bytes = lds;
    return true;
  }
}

GemmPlan plan_gemm(const Geom& g) {
  GemmPlan p{};
  if (g.M <= 32 && gemv_preferred(g) && plan_gemv(g, p)) return p;
  if (g.M <= 32) {
    p.kind = 0;
    // Variant code: ntw * 10000 + wn * 100 + wk.  Chosen from a sweep of all
    // variants over the Qwen3-4B and Llama-3-8B decode shapes on MI355X:
    // wide layers (>= 1024 column tiles) use two column tiles per wave;
    // narrower ones put one column tile per workgroup and split K over 4-16
    // waves, more of them for short or very long K.
    int ntw = 1, wn = 1, wk = 4;
    if (g.NT >= 1024) {
      ntw = 2;
      wn = g.M <= 8 ? 2 : 4;
      wk = g.M <= 8 ? 2 : 1;
    } else if (g.M > 16 && g.NT >= 384) {
      wn = 2;
      wk = 2;
    } else if (g.KT <= 24 || g.KT >= 64) {
      wk = 16;
    } else {
      wk = g.M <= 8 ? 4 : (g.M <= 16 ? 8 : 16);
    }
    const int env = env_int("SGL_AWQ_SKINNY_VARIANT", 0);
    if (skinny_variant_ok(env)) {
      ntw = env / 10000;
      wn = (env / 100) % 100;
      wk = env % 100;
    }
    const int64_t ntg = (int64_t)wn * ntw;
    p.variant = ntw * 10000 + wn * 100 + wk;
    p.grid_x = (g.NT + ntg - 1) / ntg;
    int64_t ks = 1;
    if (p.grid_x < kNumCU / 2) {
      // Few column tiles: split K so about one workgroup per CU is busy,
      // keeping >= 4 k-tiles per wave and the partial traffic
      // (KS * M * N * 8 bytes) below a quarter of the weight stream.
      ks = (kNumCU + p.grid_x - 1) / p.grid_x;
      ks = std::min(ks, std::max<int64_t>(1, g.KT / (2 * wk)));
      ks = std::min(ks, std::max<int64_t>(1, g.K / (64 * g.M)));
    }
    const int env_ks = env_int("SGL_AWQ_SKINNY_KS", 0);
    if (env_ks > 0) ks = env_ks;
    ks = std::max<int64_t>(1, std::min<int64_t>(ks, g.KT));
    p.ktc = (int)((g.KT + ks - 1) / ks);
    p.ks = (int)((g.KT + p.ktc - 1) / p.ktc);  // every workgroup gets >= 1 k-tile
    p.grid_y = p.ks;
    p.ws_bytes = p.ks > 1 ? (int64_t)p.ks * g.M * g.NT * 16 * 4 : 0;
  } else {
    p.kind = 1;
    int bm = g.M <= 64 ? 64 : 128;
    const int env = env_int("SGL_AWQ_TILED_BM", 0);
    if (env == 64 || env == 128 || env == 256) bm = env;
    p.variant = bm;
    p.grid_x = (g.NT + 15) / 16;
    p.grid_y = (g.M + bm - 1) / bm;
    p.ks = 1;
    p.ktc = (int)g.KT;
    p.ws_bytes = 0;
  }
  return p;
}

hipError_t launch_gemm(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                       hipStream_t s) {
  if (p.kind == 0) return launch_skinny(p, x, w, sr, zr, bias, out, dtype, g, ws, counters, s);
  if (p.kind == 2) return launch_gemv(p, x, w, sr, zr, bias, out, dtype, g, ws, counters, s);
  return dtype == 0 ? launch_tiled_dt<F16>(p, x, w, sr, zr, bias, out, g, s)
                    : launch_tiled_dt<BF16>(p, x, w, sr, zr, bias, out, g, s);
}

}  // namespace sgl_awq
