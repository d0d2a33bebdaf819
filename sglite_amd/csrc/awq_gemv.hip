// Decode-regime W4A16 kernel for small batches (M <= 32) for gfx950.
//
// Each workgroup owns WN x NTW column tiles of 16 columns and a k-range of its
// split-K slice: wave (wn, wk) takes column tiles wn*NTW .. wn*NTW + NTW - 1
// and the slice's k-tiles wk, wk + WK, ...; MT = 1 or 2 m-tiles of 16 rows.  A launch
// of a decode-size layer (a few MB of int4 weights) is short enough that its
// time is set by how soon the weight loads are in flight, so a wave issues
// the loads of every k-tile it owns (weights, zero words, scales) before it
// computes anything, and waits for them one k-tile at a time.
//
// The activation slice of the workgroup (M rows x its k-range) is staged once
// through LDS, shared by all its waves: XPT 16-byte loads per thread, issued
// ahead of the weight loads so that their (L2) latency hides under the
// weights' HBM latency.  MFMA B fragments are then ds_read_b128 of that slice
// (rows >= M read row M - 1; their outputs are never stored).
//
// The MFMA A operand is, per k-tile (one quantisation group):
//   * plain GEMMs of up to 3 rows: the biased weight B + q (one v_and_or_b32
//     per weight pair), with the group's scale and the zero-point term
//     -s (B + z) * sum(x) applied in fp32 (the workgroup sums each row's
//     k-tile once while it stages the slice);
//   * other fp16 GEMMs: the exact integers q - z, the sum scaled in fp32;
//   * bf16: the weight dequantised to (q - z) * s with the oracle's rounding
//     (Dq<DT>::word);
// the WK waves' partial sums are reduced through LDS by all threads, and
// split-K slices are combined across workgroups with the same fence-free
// atomic handoff as the wider decode kernel (device-scope exchanges and an
// arrival counter, fixed reduction order).
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410) for batches of up to 32 rows
// whose quantisation groups span whole 128-row tiles (G = 128 or G = K).
#include <algorithm>
#include <type_traits>

#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// fp32 value of a 16-bit activation or scale element.
template <typename DT>
__device__ __forceinline__ float elem_f32(uint32_t bits);
template <>
__device__ __forceinline__ float elem_f32<F16>(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
template <>
__device__ __forceinline__ float elem_f32<BF16>(uint32_t bits) {
  return __builtin_bit_cast(float, bits << 16);
}

// Sum over each aligned 16-lane row of the wave, left in the row's lane 15
// (DPP row shifts: no LDS round trip).
__device__ __forceinline__ float row16_sum(float v) {
  auto shr = [](float x, auto ctrl, auto bank_mask) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value,
                                                                 0xf, decltype(bank_mask)::value, false));
  };
  v += shr(v, std::integral_constant<int, 0x111>{}, std::integral_constant<int, 0xf>{});  // row_shr:1
  v += shr(v, std::integral_constant<int, 0x112>{}, std::integral_constant<int, 0xf>{});  // row_shr:2
  v += shr(v, std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xe>{});  // row_shr:4
  v += shr(v, std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xc>{});  // row_shr:8
  return v;
}

// Sum of the eight 16-bit elements of a 16-byte chunk, in fp32 (fp16: four
// v_dot2_f32_f16 against (1, 1)).  The words are named one by one: hipcc
// (ROCm 7.2) miscompiles __builtin_bit_cast of v[i] inside an unrolled loop
// into four uses of the first word.
template <typename DT>
__device__ __forceinline__ float chunk_sum(u32x4 v);
template <>
__device__ __forceinline__ float chunk_sum<F16>(u32x4 v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
  const uint32_t w0 = v.x, w1 = v.y, w2 = v.z, w3 = v.w;
  float s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w0), one, 0.f, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w1), one, s, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w2), one, s, false);
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w3), one, s, false);
}
template <>
__device__ __forceinline__ float chunk_sum<BF16>(u32x4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s += elem_f32<BF16>(w[i] & 0xFFFFu) + elem_f32<BF16>(w[i] >> 16);
  return s;
}

// Epilogue of a gemv workgroup with a fused gate/up activation: wave wn
// holds gate tile t = blockIdx.x * WN + wn in slot 0 and its up tile
// t + NT / 2 in slot 1.  Pair-quad pq = (wn' * MT + mt) * 64 + l covers row
// 16 mt + l % 16 and output columns 16 t' + 4 (l / 16) .. + 3 of both tiles.
// With WK > 1 the k-waves' sums are in red (quad ((wn' * MT + mt) * 2 + slot)
// * 64 + l of k-wave o at red[o * NQ + quad]); split K publishes both tiles'
// partials at their physical columns and the last workgroup applies the
// activation to the slice sums.
template <int WN, int WK, int MT, int NTHREADS, typename DT>
__device__ __forceinline__ void gemv_paired_epilogue(const f32x4 (&acc)[MT][2], const f32x4* red,
                                                     const typename DT::elem* __restrict__ bias,
                                                     typename DT::elem* __restrict__ out, float* __restrict__ part,
                                                     int32_t* __restrict__ counters, int M, int N, int NT, int KS,
                                                     int act, int wn, int lane) {
  constexpr int NQ = WN * MT * 2 * 64;
  constexpr int NP = WN * MT * 64;
  constexpr int NU = WK > 1 ? (NP + NTHREADS - 1) / NTHREADS : MT;
  const int NTg = NT >> 1, Nh = N >> 1;
  const int64_t Np = (int64_t)NT * 16;
  auto pos = [&](int u, int& m, int& tq, int& c4) {
    const int pq = WK > 1 ? (int)threadIdx.x + u * NTHREADS : (wn * MT + u) * 64 + lane;
    const int l = pq & 63, r = pq >> 6;
    m = (r % MT) * 16 + (l & 15);
    tq = blockIdx.x * WN + r / MT;
    c4 = 4 * (l >> 4);
    return pq < NP;
  };
  auto vals = [&](int u, f32x4& g, f32x4& v) {
    if constexpr (WK > 1) {
      const int pq = min((int)threadIdx.x + u * NTHREADS, NP - 1);
      const int qg = (pq >> 6) * 128 + (pq & 63);
      g = red[qg];
      v = red[qg + 64];
#pragma unroll
      for (int o = 1; o < WK; ++o) {
        g += red[o * NQ + qg];
        v += red[o * NQ + qg + 64];
      }
    } else {
      g = acc[u][0];
      v = acc[u][1];
    }
  };
  if (KS == 1) {
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      int m, tq, c4;
      if (pos(u, m, tq, c4) && m < M && tq < NTg) {
        f32x4 g, v;
        vals(u, g, v);
        store4_act<DT>(out, bias, m, Nh, tq * 16 + c4, Nh, g, v, act);
      }
    }
    return;
  }
  float chk = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    int m, tq, c4;
    if (pos(u, m, tq, c4) && m < M && tq < NTg) {
      f32x4 g, v;
      vals(u, g, v);
      float* pg = part + ((int64_t)blockIdx.y * M + m) * Np + tq * 16 + c4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        chk += xchg_agent(pg + r, g[r]);
        chk += xchg_agent(pg + Nh + r, v[r]);
      }
    }
  }
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
  for (int u = 0; u < NU; ++u) {
    int m, tq, c4;
    if (pos(u, m, tq, c4) && m < M && tq < NTg) {
      f32x4 g = f32x4{0.f, 0.f, 0.f, 0.f}, v = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int ks = 0; ks < KS; ++ks) {
        float* pg = part + ((int64_t)ks * M + m) * Np + tq * 16 + c4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          g[r] += xchg_agent(pg + r, 0.f);
          v[r] += xchg_agent(pg + Nh + r, 0.f);
        }
      }
      store4_act<DT>(out, bias, m, Nh, tq * 16 + c4, Nh, g, v, act);
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int NTW, int WN, int WK, int KPW, int MT, int XPT, typename DT, bool BIASED>
__global__ __launch_bounds__(64 * WN * WK) void gemv_kernel(
    const typename DT::elem* __restrict__ x, const u32x4* __restrict__ wt, const uint16_t* __restrict__ s_r,
    const uint64_t* __restrict__ z_r, const typename DT::elem* __restrict__ bias, typename DT::elem* __restrict__ out,
    float* __restrict__ part, int32_t* __restrict__ counters, int M, int N, int K, int NT, int KT, int NG, int gshift,
    int ktc, int KS, int act) {
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  constexpr int NTHREADS = 64 * WN * WK;
  constexpr int NTG = WN * NTW;  // column tiles of the workgroup
  // LDS: the activation slice (M x ktc*128 halves, row stride ktc*128 + 8),
  // on the biased path its per-(row, k-tile) sums (16-byte aligned), then
  // (after a barrier, over both) the WK partial sums of every output quad.
  extern __shared__ u32x4 smem[];

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wn = wave % WN, wk = wave / WN;
  const int c = lane & 15, lg = lane >> 4;
  const int nt0 = blockIdx.x * NTG + wn * NTW;
  const int kt_begin = blockIdx.y * ktc;
  const int kt_end = min(kt_begin + ktc, KT);
  const int nkt = kt_end - kt_begin;                       // k-tiles of this workgroup
  const int kpw = wk < nkt ? (nkt - 1 - wk) / WK + 1 : 0;  // k-tiles of this wave (<= KPW)
  const int rs = ktc * 128 + 8;                            // LDS row stride (halves)
  const DqK dk = dq_consts();

  // ---- activation slice: XPT chunks of 8 halves per thread --------------
  // chunk q -> row q / (16 ktc), halves 8 (q % (16 ktc)) of the k-range.
  u32x4 xr[XPT];
  const int cpr = ktc * 16;  // chunks per row
#pragma unroll
  for (int r = 0; r < XPT; ++r) {
    const int q = min((int)threadIdx.x + r * NTHREADS, M * cpr - 1);
    const int m = q / cpr, kk = (q % cpr) * 8;
    const int k = min(kt_begin * 128 + kk, K - 8);  // halves past K are zeroed when stored
    xr[r] = ld_off<u32x4>(x, ((uint32_t)m * (uint32_t)K + (uint32_t)k) * 2u);
  }

  // ---- publish the activation slice ----------------------------------------
  // With the biased operand, also the sum of every (row, k-tile) of the
  // slice, xsum[kt * M + m]: the 16 chunks of one row's k-tile are 16
  // consecutive threads (an aligned quarter wave, as cpr and NTHREADS are
  // multiples of 16).
  _Float16* xs = (_Float16*)smem;
  float* xsum = (float*)((char*)smem + ((M * rs * 2 + 15) & ~15));
  // Published after the first k-tile's weight loads are issued and before the
  // rest: the CU issues vector-memory instructions at ~24 cycles each, so a
  // barrier after all of them (up to 512 per CU) kept every k-tile's compute
  // until after the data had arrived.  Now the k-tiles are computed as their
  // weights land (Qwen3-4B gate_up at M = 8 11.9 -> 10.3 us, qkv 7.2 -> 6.7
  // us; Llama-3-8B down at M = 1 12.2 -> 10.9 us).  Plain GEMMs of up to 3 rows
  // with at most 4 k-tiles per wave still issue every load first (their short
  // launches gain more from the weights' earlier issue: o_proj at M = 1 was
  // 3.5% slower the other way).
  constexpr int kEarlyKt = BIASED && KPW <= 4 ? KPW : 1;  // k-tiles whose loads precede the publish
  auto publish = [&]() {
#pragma unroll
    for (int r = 0; r < XPT; ++r) {
      const int qi = threadIdx.x + r * NTHREADS;
      const bool live = qi < M * cpr;
      const int m = live ? qi / cpr : 0, kk = live ? (qi % cpr) * 8 : 0;
      const u32x4 v = live && kt_begin * 128 + kk < K ? xr[r] : u32x4{0u, 0u, 0u, 0u};
      if (live) *(u32x4*)(xs + m * rs + kk) = v;
      if constexpr (BIASED) {
        const float sum = row16_sum(chunk_sum<DT>(v));
        if (live && (qi & 15) == 15) xsum[(kk >> 7) * M + m] = sum;
      }
    }
    __syncthreads();
  };

  // ---- weights, zero words and scales of every k-tile of this wave ---------
  // (one quantisation group per 128-row tile: G >= 128)
  u32x4 q[KPW][NTW];
  uint32_t zw[KPW][NTW];
  uint16_t sb[KPW][NTW];   // scale of the lane's own column c
  uint2 s4[KPW][NTW];      // scales of the lane's output columns 4 lg .. 4 lg + 3 (fp32 scaling)
  // With a fused gate/up activation (two tiles per wave) the wave's tiles
  // are gate tile t = blockIdx.x * WN + wn and its up tile t + NT / 2.
  const bool paired = NTW == 2 && act != kActNone;
  const int tpair = blockIdx.x * WN + wn;
  uint32_t woff[NTW], goff[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    // columns past N read a valid tile, never stored
    const uint32_t ntc = (uint32_t)(paired ? min(tpair, (NT >> 1) - 1) + j * (NT >> 1) : min(nt0 + j, NT - 1));
    woff[j] = (ntc * (uint32_t)KT * 64u + lane) * 16u;
    goff[j] = ntc * (uint32_t)NG;
  }
  // k-tiles past the wave's share reload its last one (no branch around loads)
  auto load_kt = [&](int i) {
    const int kt = kt_begin + wk + WK * min(i, max(kpw - 1, 0));
    const int ktl = min(kt, KT - 1);
    const uint32_t g = (uint32_t)min((ktl * 128) >> gshift, NG - 1);
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      q[i][j] = ld_off_nt<u32x4>(wt, woff[j] + (uint32_t)ktl * 1024u);
      const uint32_t gi = goff[j] + g;
      zw[i][j] = ld_off<uint32_t>(z_r, gi * 8u + (uint32_t)(c >> 3) * 4u);
      sb[i][j] = ld_off<uint16_t>(s_r, (gi * 16u + c) * 2u);
      if constexpr (BIASED || std::is_same_v<DT, F16>)
        s4[i][j] = ld_off<uint2>(s_r, (gi * 16u + 4u * (uint32_t)lg) * 2u);
    }
  };
#pragma unroll
  for (int i = 0; i < kEarlyKt; ++i) load_kt(i);
  publish();
#pragma unroll
  for (int i = kEarlyKt; i < KPW; ++i) load_kt(i);

  // ---- compute ---------------------------------------------------------------
  // bf16 (not biased): per k-block the weights are dequantised to (q - z) * s
  // with the oracle's rounding (Dq<DT>::word, 13 VALU operations per 8
  // weights) into the MFMA A operand, accumulated in fp32; fp16 takes the
  // integers q - z (9 operations) and scales each k-tile's sum in fp32.
  // Biased path (GEMMs of up to 3 rows, where the vector work of dequantising
  // weighs most against the rest of the kernel): the MFMAs take the biased weights
  // B + q straight from the nibbles (one v_and_or_b32 per pair), so
  //   sum_k (q - z) s x = s * sum_k (B + q) x - s (B + z) * sum_k x :
  // the first term is scaled into the fp32 accumulator per k-tile (the lane's
  // four output columns' scales), the second is one fp32 MFMA per four
  // k-tiles, with -s (B + z) of the lane's own column in k-tile slot lg as
  // the A operand and the row sums of slot lg as the B operand.
  f32x4 acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  int xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = min(mt * 16 + c, M - 1) * rs + lg * 8;
  if constexpr (!BIASED && std::is_same_v<DT, F16>) {
    // fp16: the exact integers q - z (two VALU operations per weight pair)
    // into the MFMAs, each k-tile's sum scaled in fp32 by the lane's four
    // output-column scales, after all the k-tiles' MFMAs are issued.
    const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 t[KPW][MT][NTW];
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i < kpw) {
        const int kl = (wk + WK * i) * 128;  // k offset inside the slice
        ZS zs[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) zs[j] = Dq<DT>::make((zw[i][j] >> (4 * (c & 7))) & 0xFu, sb[i][j]);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          V8 av[NTW];
#pragma unroll
          for (int j = 0; j < NTW; ++j) av[j] = Dq<DT>::word_q_minus_z(q[i][j][w], zs[j], dk);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const V8 bx = __builtin_bit_cast(V8, *(const u32x4*)(xs + xrow[mt] + kl + 32 * w));
#pragma unroll
            for (int j = 0; j < NTW; ++j) t[i][mt][j] = mfma16x16x32(av[j], bx, w == 0 ? zero4 : t[i][mt][j]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i < kpw) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const float sc[4] = {elem_f32<DT>(s4[i][j].x & 0xFFFFu), elem_f32<DT>(s4[i][j].x >> 16),
                               elem_f32<DT>(s4[i][j].y & 0xFFFFu), elem_f32<DT>(s4[i][j].y >> 16)};
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][j][r] = fmaf(sc[r], t[i][mt][j][r], acc[mt][j][r]);
        }
      }
    }
  } else if constexpr (!BIASED) {
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i < kpw) {
        const int kl = (wk + WK * i) * 128;  // k offset inside the slice
        ZS zs[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) zs[j] = Dq<DT>::make((zw[i][j] >> (4 * (c & 7))) & 0xFu, sb[i][j]);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          V8 av[NTW];
#pragma unroll
          for (int j = 0; j < NTW; ++j) av[j] = Dq<DT>::word(q[i][j][w], zs[j], dk);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const V8 bx = __builtin_bit_cast(V8, *(const u32x4*)(xs + xrow[mt] + kl + 32 * w));
#pragma unroll
            for (int j = 0; j < NTW; ++j) acc[mt][j] = mfma16x16x32(av[j], bx, acc[mt][j]);
          }
        }
      }
    }
  } else {
    const uint32_t kMagic = opaque_vgpr(Raw<DT>::kMagic);
    const f32x4 zero4 = f32x4{0.f, 0.f, 0.f, 0.f};
    // Every k-tile's MFMAs first (each starts as soon as its loads land), the
    // scaling after all of them, so that no VALU operation waits on the MFMA
    // result just issued.
    f32x4 t[KPW][MT][NTW];
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i < kpw) {
        const int kl = (wk + WK * i) * 128;  // k offset inside the slice
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          V8 av[NTW];
#pragma unroll
          for (int j = 0; j < NTW; ++j) av[j] = biased_word<DT>(q[i][j][w], dk.lo, kMagic);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const V8 bx = __builtin_bit_cast(V8, *(const u32x4*)(xs + xrow[mt] + kl + 32 * w));
#pragma unroll
            for (int j = 0; j < NTW; ++j) t[i][mt][j] = mfma16x16x32(av[j], bx, w == 0 ? zero4 : t[i][mt][j]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i < kpw) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const float sc[4] = {elem_f32<DT>(s4[i][j].x & 0xFFFFu), elem_f32<DT>(s4[i][j].x >> 16),
                               elem_f32<DT>(s4[i][j].y & 0xFFFFu), elem_f32<DT>(s4[i][j].y >> 16)};
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][j][r] = fmaf(sc[r], t[i][mt][j][r], acc[mt][j][r]);
        }
      }
    }
#pragma unroll
    for (int ch = 0; ch < (KPW + 3) / 4; ++ch) {
      if (4 * ch < kpw) {
        float u[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) u[j] = 0.f;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          const int i = 4 * ch + ii;
          if (i < KPW && lg == ii && i < kpw) {
#pragma unroll
            for (int j = 0; j < NTW; ++j)
              u[j] = -(elem_f32<DT>(sb[i][j]) * (Raw<DT>::kBias + (float)((zw[i][j] >> (4 * (c & 7))) & 0xFu)));
          }
        }
        const int kts = wk + WK * min(4 * ch + lg, kpw - 1);  // k-tile of slot lg in the slice
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const float sv = xsum[kts * M + min(mt * 16 + c, M - 1)];
#pragma unroll
          for (int j = 0; j < NTW; ++j) acc[mt][j] = mfma16x16x4f32(u[j], sv, acc[mt][j]);
        }
      }
    }
  }

  // ---- reduce the WK waves: thread t sums quad t of every k-wave -------------
  // quad index qd = ((wn * MT + mt) * NTW + j) * 64 + lane: m-tile mt, column
  // tile wn*NTW + j, lane l: row 16 mt + l % 16, columns 4 (l / 16) + r.
  constexpr int NQ = WN * MT * NTW * 64;
  constexpr int QPT = (NQ + NTHREADS - 1) / NTHREADS;  // quads per thread
  f32x4 res[QPT];
  if constexpr (WK > 1) {
    __syncthreads();  // every wave is done reading the activation slice
    f32x4* red = (f32x4*)smem;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NTW; ++j) red[wk * NQ + ((wn * MT + mt) * NTW + j) * 64 + lane] = acc[mt][j];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      const int qd = min((int)threadIdx.x + u * NTHREADS, NQ - 1);
      f32x4 s4 = red[qd];
#pragma unroll
      for (int o = 1; o < WK; ++o) s4 += red[o * NQ + qd];
      res[u] = s4;
    }
  }

  if constexpr (NTW == 2) {
    if (paired) {
      gemv_paired_epilogue<WN, WK, MT, NTHREADS, DT>(acc, (const f32x4*)smem, bias, out, part, counters, M, N, NT, KS,
                                                    act, wn, lane);
      return;
    }
  }

  // Output quad of this thread: with WK > 1 thread t owns quads t + u*NTHREADS;
  // with WK == 1 each lane keeps its own accumulators.
  auto quad_pos = [&](int u, int& m, int& n0) {
    int qd;
    if constexpr (WK > 1) {
      qd = threadIdx.x + u * NTHREADS;
    } else {
      const int mt = u / NTW, j = u % NTW;
      qd = ((wn * MT + mt) * NTW + j) * 64 + lane;
    }
    const int l = qd & 63, t = qd >> 6;  // t = (wn' * MT + mt') * NTW + j'
    const int j = t % NTW, mt = (t / NTW) % MT, wq = t / (NTW * MT);
    m = mt * 16 + (l & 15);
    n0 = (blockIdx.x * NTG + wq * NTW + j) * 16 + 4 * (l >> 4);
    return qd < NQ;
  };
  auto quad_val = [&](int u) -> f32x4 {
    if constexpr (WK > 1) return res[u];
    else return acc[u / NTW][u % NTW];
  };
  constexpr int NU = WK > 1 ? QPT : MT * NTW;

  if (KS == 1) {
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      int m, n0;
      if (quad_pos(u, m, n0) && m < M && n0 < N) store4<DT>(out, bias, m, N, n0, quad_val(u));
    }
    return;
  }

  // ---- split-K handoff ------------------------------------------------------
  const int64_t Np = (int64_t)NT * 16;
  float chk = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    int m, n0;
    if (quad_pos(u, m, n0) && m < M && n0 < Np) {
      float* p = part + ((int64_t)blockIdx.y * M + m) * Np + n0;
      const f32x4 v = quad_val(u);
#pragma unroll
      for (int r = 0; r < 4; ++r) chk += xchg_agent(p + r, v[r]);
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
  for (int u = 0; u < NU; ++u) {
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
                          const void* bias, void* out, const Geom& g, void* ws, int32_t* counters, int act,
                          hipStream_t s) {
  using E = typename DT::elem;
  const uint16_t* sbase = (const uint16_t*)sr;
  const uint64_t* zbase = (const uint64_t*)zr;
  const int ntw = p.variant / 10000, wn = (p.variant / 1000) % 10, wk = (p.variant / 10) % 100, kpw = p.variant % 10;
  const int mt = (int)((g.M + 15) / 16);
  const int xpt = p.xpt;
  dim3 grid((unsigned)p.grid_x, (unsigned)p.grid_y);
  const size_t lds = (size_t)p.lds_bytes;
  // Plain GEMMs of up to 3 rows on one-tile waves take the biased operand
  // (same-box sweep on MI355X: 4-12% faster at M = 1, up to 7% at M = 2-3;
  // from 4 rows on, and with a fused activation, mixed or slower).
  const bool biased = g.M <= 3 && act == kActNone && ntw == 1;
#define SGL_GEMV_B(WN_, WK_, KPW_, XPT_)                                                                            \
  if (biased && wn == WN_ && wk == WK_ && kpw == KPW_ && xpt == XPT_) {                                             \
    hipLaunchKernelGGL((gemv_kernel<1, WN_, WK_, KPW_, 1, XPT_, DT, true>), grid, dim3(64 * WN_ * WK_), lds, s,      \
                       (const E*)x, (const u32x4*)w, sbase, zbase, (const E*)bias, (E*)out, (float*)ws, counters,  \
                       (int)g.M, (int)g.N, (int)g.K, (int)g.NT, (int)g.KT, (int)g.NG, g.gshift, p.ktc, p.ks, act); \
    return hipGetLastError();                                                                                     \
  }
#define SGL_GEMV_B2(WN_, WK_, KPW_) \
  SGL_GEMV_B(WN_, WK_, KPW_, 1) SGL_GEMV_B(WN_, WK_, KPW_, 2) SGL_GEMV_B(WN_, WK_, KPW_, 4) SGL_GEMV_B(WN_, WK_, KPW_, 8)
  SGL_GEMV_B2(1, 4, 8)
  SGL_GEMV_B2(1, 8, 4)
  SGL_GEMV_B2(1, 8, 3)
  SGL_GEMV_B2(2, 8, 3)
  SGL_GEMV_B2(2, 8, 4)
  SGL_GEMV_B2(1, 8, 6)
  SGL_GEMV_B2(1, 8, 8)
  SGL_GEMV_B2(1, 16, 5)
  SGL_GEMV_B2(1, 16, 6)
  SGL_GEMV_B2(1, 16, 8)
  SGL_GEMV_B2(4, 4, 4)
  SGL_GEMV_B2(5, 3, 7)
#undef SGL_GEMV_B2
#undef SGL_GEMV_B
#define SGL_GEMV(NTW_, WN_, WK_, KPW_, MT_, XPT_)                                                                  \
  if (!biased && ntw == NTW_ && wn == WN_ && wk == WK_ && kpw == KPW_ && mt == MT_ && xpt == XPT_) {               \
    hipLaunchKernelGGL((gemv_kernel<NTW_, WN_, WK_, KPW_, MT_, XPT_, DT, false>), grid, dim3(64 * WN_ * WK_), lds, s,\
                       (const E*)x, (const u32x4*)w, sbase, zbase, (const E*)bias, (E*)out, (float*)ws, counters,  \
                       (int)g.M, (int)g.N, (int)g.K, (int)g.NT, (int)g.KT, (int)g.NG, g.gshift, p.ktc, p.ks, act); \
    return hipGetLastError();                                                                                     \
  }
#define SGL_GEMV_X(NTW_, WN_, WK_, KPW_, MT_) \
  SGL_GEMV(NTW_, WN_, WK_, KPW_, MT_, 1) SGL_GEMV(NTW_, WN_, WK_, KPW_, MT_, 2) \
  SGL_GEMV(NTW_, WN_, WK_, KPW_, MT_, 4) SGL_GEMV(NTW_, WN_, WK_, KPW_, MT_, 8)
#define SGL_GEMV_M(NTW_, WN_, WK_, KPW_) SGL_GEMV_X(NTW_, WN_, WK_, KPW_, 1) SGL_GEMV_X(NTW_, WN_, WK_, KPW_, 2)
  SGL_GEMV_M(1, 1, 4, 8)
  SGL_GEMV_M(1, 1, 8, 4)
  SGL_GEMV_M(1, 1, 8, 3)
  SGL_GEMV_M(1, 2, 8, 3)
  SGL_GEMV_M(1, 2, 8, 4)
  SGL_GEMV_M(1, 1, 8, 6)
  SGL_GEMV_M(1, 1, 8, 8)
  SGL_GEMV_M(1, 1, 16, 5)
  SGL_GEMV_M(1, 1, 16, 6)
  SGL_GEMV_M(1, 1, 16, 8)
  SGL_GEMV_M(2, 1, 4, 4)
  SGL_GEMV_M(2, 1, 8, 4)
  SGL_GEMV_M(2, 1, 8, 3)
  SGL_GEMV_M(2, 2, 2, 8)
  SGL_GEMV_M(2, 2, 4, 4)
  SGL_GEMV_M(2, 4, 2, 4)
  SGL_GEMV_M(2, 4, 4, 2)
  SGL_GEMV_M(1, 4, 4, 4)
  SGL_GEMV_M(1, 5, 3, 7)
  SGL_GEMV_M(2, 3, 5, 4)
#undef SGL_GEMV_M
#undef SGL_GEMV_X
#undef SGL_GEMV
  return hipErrorInvalidValue;
}

}  // namespace

// Variant code: ntw * 10000 + wn * 1000 + wk * 10 + kpw.
bool gemv_variant_ok(int v) {
  switch (v) {
    case 11048: case 11083: case 11084: case 11086: case 11088: case 11165: case 11166: case 11168: case 12083:
    case 12084: case 15037: case 23054: case 21044: case 21083: case 21084: case 22028: case 22044: case 24024: case 24042: case 14044:
      return true;
    default:
      return false;
  }
}

hipError_t launch_gemv(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                       hipStream_t s) {
  return dtype == 0 ? launch_gemv_dt<F16>(p, x, w, sr, zr, bias, out, g, ws, counters, act, s)
                    : launch_gemv_dt<BF16>(p, x, w, sr, zr, bias, out, g, ws, counters, act, s);
}

}  // namespace sgl_awq
