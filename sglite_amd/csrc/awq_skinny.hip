// Decode-regime W4A16 kernel (M <= 32) for gfx950.  HBM-bound: one launch
// streams the int4 weights once, dequantises in registers and reduces split-K
// partials across workgroups without cache-wide fences.  Built with
// -mllvm -amdgpu-mfma-vgpr-form so MFMA results stay in VGPRs, where the fp32
// group scaling reads them.
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410) for small batches.
#include <type_traits>

#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// ---------------------------------------------------------------------------
// Skinny split-K kernel.
//
// Each wave owns NTW column tiles and the k-tiles kt_begin + wk + WK*i of its
// workgroup's k-range, processed in batches of D tiles whose loads (weights,
// scales, zero words, activation fragments) are all issued before any is
// consumed.  GPT is the number of quantisation groups one 128-row tile spans
// (1 for G >= 128, 2 for G = 64, 4 for G = 32).
//
// Arithmetic per group g (rows k of the group, column n, batch row m):
//   sum_k (q - z) s x = s * (C[n][m] - (B + z) * S[m]),
//   C = sum_k (B + q) x   (v_mfma_f32_16x16x32 on the biased operand, B = 1024
//                          for fp16, 128 for bf16, built by one v_and_or per pair)
//   S = sum_k x           (the same MFMA with an all-ones operand)
// s * C is added to the fp32 accumulator right away (v_fma_mix, scale rows of
// the output fragment); the -s (B + z) * S terms of four groups at a time are
// one v_mfma_f32_16x16x4_f32 whose A operand holds -s (B + z) (exact in fp32)
// for the lane's own column and group slot, and whose B operand holds S of
// that slot.  So per weight pair the kernel executes a single VALU op.
//
// Split-K handoff between workgroups: atomic exchanges and a device-scope
// arrival counter (xchg_agent, awq_device.h).  The reduction order is fixed
// (ks = 0, 1, ...), so results are deterministic.
// ---------------------------------------------------------------------------

template <int MT, int NTW, int WN, int WK, int GPT, typename DT>
__global__ __launch_bounds__(64 * WN * WK) void skinny_kernel(
    const typename DT::elem* __restrict__ x, const u32x4* __restrict__ wt, const uint16_t* __restrict__ s_r,
    const uint64_t* __restrict__ z_r, const typename DT::elem* __restrict__ bias, typename DT::elem* __restrict__ out,
    float* __restrict__ part, int32_t* __restrict__ counters, int M, int N, int K, int NT, int KT, int NG, int gshift,
    int ktc, int KS, int act) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using V4 = typename DT::vec4;
  constexpr int NTHREADS = 64 * WN * WK;
  constexpr int NTG = WN * NTW;
  // k-tiles per batch: two batches of weights plus one of activation
  // fragments must fit the register budget (128 VGPRs for >= 512 threads).
  constexpr int D_BASE = NTHREADS >= 1024 ? 1 : NTHREADS >= 512 ? 2 : (NTW >= 4 ? 1 : 4 / NTW);
  constexpr int D = D_BASE / MT > 0 ? D_BASE / MT : 1;
  constexpr int BPG = 4 / GPT;               // 32-row k-blocks per group
  constexpr int NGR = D * GPT;               // groups per batch
  constexpr int NFB = (NGR + 3) / 4;         // correction flushes per batch

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wn = wave % WN, wk = wave / WN;
  const int c = lane & 15, lg = lane >> 4;
  const int nt0 = blockIdx.x * NTG + wn * NTW;
  const int kt_begin = blockIdx.y * ktc;
  const int kt_end = min(kt_begin + ktc, KT);
  const int first = kt_begin + wk;
  const int niter = first < kt_end ? (kt_end - first + WK - 1) / WK : 0;
  const int nbatch = (niter + D - 1) / D;
  // Batches whose tiles all exist and lie fully inside K need no masking;
  // only the last batch of a wave can hold missing tiles or the partial
  // last k-tile of a K that is not a multiple of 128.
  const bool last_masked = niter > 0 && (niter % D != 0 || first + WK * (niter - 1) >= (K >> 7));

  f32x4 acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint32_t kMask = opaque_vgpr(0x000F000Fu), kMagic = opaque_vgpr(Raw<DT>::kMagic);
  const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
  // Slot-selecting ones: operand row n (= lane column c) is all ones iff
  // n / 4 == slot, so sum(x) of the group in slot i lands in output rows
  // 4i..4i+3, i.e. in the lanes with lg == i -- the lanes that hold slot i of
  // the correction MFMA's B operand.  No per-lane select is needed.
  constexpr int NSEL = NGR < 4 ? NGR : 4;  // slots a batch uses
  V8 sel[NSEL];
#pragma unroll
  for (int i = 0; i < NSEL; ++i) {
    const uint32_t o = (c >> 2) == i ? Raw<DT>::kOnes : 0u;
    sel[i] = __builtin_bit_cast(V8, u32x4{o, o, o, o});
  }

  // 32-bit byte offsets from uniform bases (rows past M re-read row M-1;
  // their outputs are never stored).  The host keeps every buffer below 4 GiB.
  uint32_t xoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xoff[mt] = ((uint32_t)min(mt * 16 + c, M - 1) * (uint32_t)K + lg * 8) * 2u;
  // With a fused gate/up activation (two tiles per wave) the wave's tiles
  // are gate tile t = blockIdx.x * WN + wn and its up tile t + NT / 2.
  const bool paired = NTW == 2 && act != kActNone;
  const int NTg = NT >> 1, Nh = N >> 1;
  const int tpair = blockIdx.x * WN + wn;
  uint32_t woff[NTW], srow_off[NTW], sown_off[NTW], zoff[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    // columns past N read a valid tile, never stored
    const uint32_t ntc = (uint32_t)(paired ? min(tpair, NTg - 1) + j * NTg : min(nt0 + j, NT - 1));
    woff[j] = (ntc * (uint32_t)KT * 64u + lane) * 16u;
    srow_off[j] = (ntc * (uint32_t)NG * 16u + 4u * lg) * 2u;  // scales of output rows 4lg..4lg+3
    sown_off[j] = (ntc * (uint32_t)NG * 16u + c) * 2u;        // scale of the lane's own column
    zoff[j] = ntc * (uint32_t)NG * 8u;
  }
  auto tile_kt = [&](int i) { return first + WK * min(i, niter - 1); };  // missing tiles reload the last one
  auto group_of = [&](int kt, int gg) -> uint32_t {
    return (uint32_t)min((kt * 128 + 32 * gg * BPG) >> gshift, NG - 1);
  };

  // Weight-side state of one batch (long-latency HBM loads, prefetched one
  // batch ahead).  Group p of the batch sits in correction slot p % 4 of
  // flush block p / 4.
  struct WB {
    V8 xb[D][4][MT];
    u32x4 q[D][NTW];
    V4 srow[D][NTW][GPT];
    float corrA[NFB][NTW];
  };
  auto load_w = [&](int bi, WB& w) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int kt = tile_kt(bi * D + d);
#pragma unroll
      for (int j = 0; j < NTW; ++j) w.q[d][j] = ld_off_nt<u32x4>(wt, woff[j] + (uint32_t)kt * 1024u);
#pragma unroll
      for (int gg = 0; gg < GPT; ++gg) {
        const uint32_t g = group_of(kt, gg);
#pragma unroll
        for (int j = 0; j < NTW; ++j) w.srow[d][j][gg] = ld_off<V4>(s_r, srow_off[j] + g * 32u);
      }
    }
    // Correction A operand: lane (c, lg) takes -s (B + z) of its own column
    // for the group in slot lg of each flush block.
#pragma unroll
    for (int f = 0; f < NFB; ++f) {
      const int pg = min(f * 4 + lg, NGR - 1);
      const int kt = tile_kt(bi * D + pg / GPT);
      const uint32_t g = group_of(kt, pg % GPT);
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        const E sv = ld_off<E>(s_r, sown_off[j] + g * 32u);
        const uint64_t zw = ld_off<uint64_t>(z_r, zoff[j] + g * 8u);
        w.corrA[f][j] = -(float)sv * (Raw<DT>::kBias + (float)zero_nibble(zw, c));
      }
    }
  };
  // Activation fragments of one batch (L2-resident; loaded right before use,
  // and issued before the next batch's weights so that waiting for them does
  // not wait for those HBM loads -- loads return in issue order).
  auto load_x = [&](int bi, V8 (&xb)[D][4][MT], bool masked) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = bi * D + d;
      const int kt = tile_kt(i);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int kb = kt * 128 + 32 * w;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (masked) {  // missing tiles and k-blocks past K contribute zero
            const bool ok = i < niter && kb < K;
            const V8 v = ld_off<V8>(x, xoff[mt] + (uint32_t)(ok ? kb : 0) * 2u);
            xb[d][w][mt] = ok ? v : V8{};
          } else {
            xb[d][w][mt] = ld_off<V8>(x, xoff[mt] + (uint32_t)kb * 2u);
          }
        }
      }
    }
  };
  auto compute = [&](const WB& w, const V8 (&xb)[D][4][MT]) {
    f32x4 cs[MT];
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int gg = 0; gg < GPT; ++gg) {
        const int pg = d * GPT + gg, slot = pg & 3;
        f32x4 cm[MT][NTW];
#pragma unroll
        for (int b = 0; b < BPG; ++b) {
          const int kw = gg * BPG + b;
#pragma unroll
          for (int j = 0; j < NTW; ++j) {
            const V8 a = biased_word<DT>(w.q[d][j][kw], kMask, kMagic);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) cm[mt][j] = mfma16x16x32(a, xb[d][kw][mt], b == 0 ? zero4 : cm[mt][j]);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            cs[mt] = mfma16x16x32(sel[slot], xb[d][kw][mt], (slot == 0 && b == 0) ? zero4 : cs[mt]);
        }
        // s * C onto the accumulator (output rows 4lg + r).
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sr = (float)w.srow[d][j][gg][r];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][j][r] = __builtin_fmaf(sr, cm[mt][j][r], acc[mt][j][r]);
          }
        if (slot == 3 || pg == NGR - 1) {  // fold the block's -s (B + z) * sum(x) terms
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < NTW; ++j) acc[mt][j] = mfma16x16x4f32(w.corrA[pg >> 2][j], cs[mt][0], acc[mt][j]);
        }
      }
  };
  // Everything a batch needs -- activation fragments first, then weights
  // and scales -- is loaded one batch ahead; loads return in issue order, so
  // waiting for batch b never waits for batch b + 1.
  auto prefetch = [&](int bi, WB& w) {
    if (last_masked && bi == nbatch - 1)
      load_x(bi, w.xb, true);
    else
      load_x(bi, w.xb, false);
    load_w(bi, w);
  };
  auto step = [&](int bi, const WB& cur, WB& next) {
    if (bi + 1 < nbatch) prefetch(bi + 1, next);
    // Keep the prefetch ahead of this batch's compute (the scheduler would
    // otherwise interleave loads with math to save registers).
    __builtin_amdgcn_sched_barrier(0);
    compute(cur, cur.xb);
  };

  if (nbatch > 0) {
    WB wa, wb;
    prefetch(0, wa);
    for (int bi = 0; bi < nbatch; bi += 2) {
      step(bi, wa, wb);
      if (bi + 1 < nbatch) step(bi + 1, wb, wa);
    }
  }

  // Reduce the WK waves that share columns.
  if constexpr (WK > 1) {
    __shared__ f32x4 red[(WK - 1) * WN * MT * NTW * 64];
    if (wk > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < NTW; ++j) red[((((wk - 1) * WN + wn) * MT + mt) * NTW + j) * 64 + lane] = acc[mt][j];
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int o = 0; o < WK - 1; ++o)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < NTW; ++j) acc[mt][j] += red[(((o * WN + wn) * MT + mt) * NTW + j) * 64 + lane];
    }
  }

  // Output fragment of (mt, j): row m = 16*mt + c, columns n0..n0+3.
  if (KS == 1 && paired) {
    if constexpr (NTW == 2) {
      if (wk == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + c;
          if (m < M && tpair < NTg)
            store4_act<DT>(out, bias, m, Nh, tpair * 16 + 4 * lg, Nh, acc[mt][0], acc[mt][1], act);
        }
      }
    }
    return;
  }
  if (KS == 1) {
    if (wk == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const int m = mt * 16 + c;
          const int n0 = (nt0 + j) * 16 + 4 * lg;
          if (m < M && n0 < N) store4<DT>(out, bias, m, N, n0, acc[mt][j]);
        }
    }
    return;
  }

  const int64_t Np = (int64_t)NT * 16;
  if (wk == 0) {
    float chk = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        const int m = mt * 16 + c;
        // physical column of the fragment (a fused gate/up pair keeps the up
        // tile's partials at its own column, Nh further on)
        const int n0 = (paired ? (tpair + j * NTg) : (nt0 + j)) * 16 + 4 * lg;
        const bool val = paired ? tpair < NTg : n0 < Np;
        if (m < M && val) {
          float* p = part + ((int64_t)blockIdx.y * M + m) * Np + n0;
#pragma unroll
          for (int r = 0; r < 4; ++r) chk += xchg_agent(p + r, acc[mt][j][r]);
        }
      }
    // Consuming the returned values makes the wave wait until every
    // exchange has been performed before it reaches the barrier.
    asm volatile("" ::"v"(chk));
  }
  __syncthreads();
  __shared__ int s_last;
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[blockIdx.x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == KS - 1);
  }
  __syncthreads();
  if (!s_last) return;

  if (paired) {
    // Output quads of the workgroup's WN pairs: gate partial column o0, up o0 + Nh.
    constexpr int QPP = WN * 4;
    for (int idx = threadIdx.x; idx < M * QPP; idx += NTHREADS) {
      const int m = idx / QPP, qq = idx % QPP;
      const int tq = blockIdx.x * WN + qq / 4;
      if (tq >= NTg) continue;
      const int64_t o0 = (int64_t)tq * 16 + 4 * (qq % 4);
      f32x4 g = f32x4{0.f, 0.f, 0.f, 0.f}, v = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < KS; ++ks) {
        float* p = part + ((int64_t)ks * M + m) * Np + o0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          g[r] += xchg_agent(p + r, 0.f);
          v[r] += xchg_agent(p + Nh + r, 0.f);
        }
      }
      store4_act<DT>(out, bias, m, Nh, o0, Nh, g, v, act);
    }
    if (threadIdx.x == 0) __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  constexpr int QPR = NTG * 4;  // float4 quads per row of this column group
  const int64_t nbase = (int64_t)blockIdx.x * NTG * 16;
  for (int idx = threadIdx.x; idx < M * QPR; idx += NTHREADS) {
    const int m = idx / QPR;
    const int64_t n0 = nbase + 4 * (idx % QPR);
    if (n0 >= N) continue;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < KS; ++ks) {
      float* p = part + ((int64_t)ks * M + m) * Np + n0;
#pragma unroll
      for (int r = 0; r < 4; ++r) sum[r] += xchg_agent(p + r, 0.f);
    }
    store4<DT>(out, bias, m, N, n0, sum);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename DT>
hipError_t launch_skinny_dt_impl(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                                 const void* bias, void* out, const Geom& g, void* ws, int32_t* counters, int act,
                                 hipStream_t s) {
  using E = typename DT::elem;
  const uint16_t* sbase = (const uint16_t*)sr;
  const uint64_t* zbase = (const uint64_t*)zr;
  const int mt = (g.M + 15) / 16;
  const int ntw = p.variant / 10000, wn = (p.variant / 100) % 100, wk = p.variant % 100;
  const int gpt = (g.NG > 1 && g.G < 128) ? (int)(128 / g.G) : 1;
  dim3 grid((unsigned)p.grid_x, (unsigned)p.grid_y);
#define SGL_SKINNY(MT_, NTW_, WN_, WK_, GPT_)                                                                  \
  if (mt == MT_ && ntw == NTW_ && wn == WN_ && wk == WK_ && gpt == GPT_) {                                   \
    hipLaunchKernelGGL((skinny_kernel<MT_, NTW_, WN_, WK_, GPT_, DT>), grid, dim3(64 * WN_ * WK_), 0, s,     \
                       (const E*)x, (const u32x4*)w, sbase, zbase, (const E*)bias, (E*)out, (float*)ws,       \
                       counters, (int)g.M, (int)g.N, (int)g.K, (int)g.NT, (int)g.KT, (int)g.NG, g.gshift, p.ktc, \
                       p.ks, act);                                                                           \
    return hipGetLastError();                                                                                \
  }
#define SGL_SKINNY_G(MT_, NTW_, WN_, WK_) \
  SGL_SKINNY(MT_, NTW_, WN_, WK_, 1) SGL_SKINNY(MT_, NTW_, WN_, WK_, 2) SGL_SKINNY(MT_, NTW_, WN_, WK_, 4)
#define SGL_SKINNY_MT(NTW_, WN_, WK_) SGL_SKINNY_G(1, NTW_, WN_, WK_) SGL_SKINNY_G(2, NTW_, WN_, WK_)
  SGL_SKINNY_MT(1, 1, 4)
  SGL_SKINNY_MT(1, 1, 8)
  SGL_SKINNY_MT(1, 1, 16)
  SGL_SKINNY_MT(1, 2, 2)
  SGL_SKINNY_MT(1, 4, 1)
  SGL_SKINNY_MT(1, 4, 4)
  SGL_SKINNY_MT(2, 2, 2)
  SGL_SKINNY_MT(2, 4, 1)
  SGL_SKINNY_MT(2, 2, 4)
#undef SGL_SKINNY_MT
#undef SGL_SKINNY_G
#undef SGL_SKINNY
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_skinny(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                         const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                         hipStream_t s) {
  return dtype == 0 ? launch_skinny_dt_impl<F16>(p, x, w, sr, zr, bias, out, g, ws, counters, act, s)
                    : launch_skinny_dt_impl<BF16>(p, x, w, sr, zr, bias, out, g, ws, counters, act, s);
}

}  // namespace sgl_awq
