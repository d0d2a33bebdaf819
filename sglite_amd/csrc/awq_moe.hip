// Grouped W4A16 MoE path for gfx950: routing, expert alignment, two grouped
// GEMMs over expert-sorted 16-row blocks, top-k combine.
//
// Data flow (fused.py:101-202 of python/sglite/srt/model_executor/layers/fused_moe/):
//   topk_softmax_kernel   logits [T, E] fp32 -> topk weights [T, k] fp32, ids [T, k] int32
//   align_kernel          ids -> routed rows (t * k + j) sorted by expert, each
//                         expert's bucket padded to the block size with the
//                         sentinel T * k; per-block expert id; padded offsets
//   moe_gemm_kernel       per (expert, column slice): the expert's rows times its
//                         AWQ weights (CDNA4 tile layout, experts stacked), fp32
//                         accumulation; epilogue either
//                           * gate/up pairing + silu (or gelu) and multiply,
//                             writing [T * k, I]    (first GEMM), or
//                           * routed-weight multiply in fp32 before the cast,
//                             writing [T * k, H]    (second GEMM)
//   moe_sum_kernel        out[t] = sum_j y[t * k + j] in fp32, cast once
//
// The grouped GEMM stages the gathered activation rows through double-buffered
// LDS in MFMA fragment order (like the prefill kernel) so the four waves of a
// workgroup share one copy, and each wave dequantises the weights of its own
// 64 columns straight from global memory into MFMA operands.  A workgroup
// serves every block of one expert for its column slice, so each expert's
// weights are streamed from HBM once per forward; workgroups of one expert are
// placed on one XCD so the expert's activation rows are fetched into one L2.
#include <math.h>

#include <algorithm>

#include "awq_device.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// ---------------------------------------------------------------------------
// Wave-level helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint64_t lanes_below(int lane) { return lane == 0 ? 0ull : (~0ull >> (64 - lane)); }

// ---------------------------------------------------------------------------
// Routing: softmax over E experts, top-k, optional renormalisation.
// One wave per token; lane l holds experts l, l + 64, ...
// Follows fused.py:11-31 (topk_softmax, then w / (sum(w) + 1e-8)).
// ---------------------------------------------------------------------------
template <int EPL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const float* __restrict__ logits, float* __restrict__ tw,
                                                           int32_t* __restrict__ tid, int T, int E, int k,
                                                           int renorm) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const float* row = logits + (int64_t)t * E;
  float v[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? row[e] : -INFINITY;
  }
  float mx = v[0];
#pragma unroll
  for (int i = 1; i < EPL; ++i) mx = fmaxf(mx, v[i]);
  mx = wave_max(mx);
  float p[EPL], s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    p[i] = lane + 64 * i < E ? expf(v[i] - mx) : 0.f;
    s += p[i];
  }
  s = wave_sum(s);
  const float inv = 1.f / s;
#pragma unroll
  for (int i = 0; i < EPL; ++i) p[i] = lane + 64 * i < E ? p[i] * inv : -1.f;  // -1: never selected

  // k rounds of a wave-wide argmax; ties go to the lower expert index.
  float wsel = 0.f, wsum = 0.f;
  int isel = 0;
  for (int j = 0; j < k; ++j) {
    float bv = p[0];
    int bi = lane;
#pragma unroll
    for (int i = 1; i < EPL; ++i)
      if (p[i] > bv) {  // strictly greater keeps the lower index of equal values
        bv = p[i];
        bi = lane + 64 * i;
      }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    // Every lane now holds the winner; its owner retires it.
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (bi == lane + 64 * i) p[i] = -1.f;
    if (lane == j) {
      wsel = bv;
      isel = bi;
    }
    wsum += bv;
  }
  if (lane < k) {
    const float w = renorm ? wsel / (wsum + 1e-8f) : wsel;
    tw[(int64_t)t * k + lane] = w;
    tid[(int64_t)t * k + lane] = isel;
  }
}

// ---------------------------------------------------------------------------
// Alignment (moe_align_block_size, fused.py:34-61): a stable counting sort of
// the routed rows i = t * k + j by expert, each bucket padded to a multiple of
// the block size with the sentinel n = T * k.  One workgroup of 1024 threads.
//   sorted[off[e] .. off[e] + cnt[e])   rows of expert e in increasing order
//   sorted[off[e] + cnt[e] .. off[e+1]) sentinel n
//   expert_ids[b]                        expert of block b (-1 past the end)
//   offsets[0..E]                        padded bucket offsets (off[E] = total)
//   *num_post_pad                        off[E]
// Rows whose id is outside [0, E) are dropped (fused.py:28-30 marks padded
// tokens with -1).
// ---------------------------------------------------------------------------
constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kMaxExperts = 512;

__global__ __launch_bounds__(kAlignThreads) void align_kernel(const int32_t* __restrict__ ids, int n, int E, int bs,
                                                              int32_t* __restrict__ sorted, int32_t* __restrict__ expert_ids,
                                                              int blocks_cap, int32_t* __restrict__ num_post_pad,
                                                              int32_t* __restrict__ offsets) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int off[kMaxExperts + 1];
  __shared__ int cursor[kMaxExperts];
  __shared__ int wcnt[kAlignWaves][kMaxExperts];
  __shared__ int wtot[kAlignWaves];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  for (int e = tid; e < E; e += kAlignThreads) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += kAlignThreads) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();

  // Exclusive scan of the padded counts (E <= 1024: one element per thread).
  const int pc = tid < E ? (cnt[tid] + bs - 1) / bs * bs : 0;
  int incl = pc;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wtot[w];
  if (tid < E) {
    off[tid] = base + incl - pc;
    cursor[tid] = base + incl - pc;
  }
  if (tid == E - 1) off[E] = base + incl;
  __syncthreads();

  const int total = off[E];
  for (int e = tid; e <= E; e += kAlignThreads) offsets[e] = off[e];
  if (tid == 0) *num_post_pad = total;
  for (int e = tid; e < E; e += kAlignThreads) {
    for (int p = off[e] + cnt[e]; p < off[e + 1]; ++p) sorted[p] = n;
    for (int b = off[e] / bs; b < off[e + 1] / bs; ++b) expert_ids[b] = e;
  }
  for (int b = total / bs + tid; b < blocks_cap; b += kAlignThreads) expert_ids[b] = -1;

  // Stable scatter, 1024 rows at a time: rank within the wave by ballots,
  // then the counts of the lower waves, then the bucket cursor.
  for (int c0 = 0; c0 < n; c0 += kAlignThreads) {
    for (int idx = tid; idx < kAlignWaves * E; idx += kAlignThreads) wcnt[idx / E][idx % E] = 0;
    __syncthreads();
    const int i = c0 + tid;
    const int e = i < n ? ids[i] : -1;
    const bool valid = e >= 0 && e < E;
    int rank = 0;
    uint64_t todo = __ballot(valid);
    while (todo) {
      const int leader = __builtin_ctzll(todo);
      const int le = __shfl(e, leader);
      const uint64_t mask = __ballot(valid && e == le);
      if (valid && e == le) rank = __popcll(mask & lanes_below(lane));
      if (lane == leader) wcnt[wave][le] = __popcll(mask);
      todo &= ~mask;
    }
    __syncthreads();
    if (valid) {
      int pos = cursor[e] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][e];
      sorted[pos] = i;
    }
    __syncthreads();
    for (int ee = tid; ee < E; ee += kAlignThreads) {
      int s = 0;
      for (int w = 0; w < kAlignWaves; ++w) s += wcnt[w][ee];
      cursor[ee] += s;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Grouped GEMM.
// ---------------------------------------------------------------------------
enum : int { kEpiPlain = 0, kEpiSilu = 1, kEpiGelu = 2 };

template <int EPI>
__device__ __forceinline__ float gate_act(float g) {
  if constexpr (EPI == kEpiSilu) {
    return g / (1.f + expf(-g));
  } else {
    return 0.5f * g * (1.f + erff(g * 0.70710678118654752f));
  }
}

struct MoeArgs {
  const void* x;           // activation rows [rows_in, K]
  const u32x4* wt;         // expert-stacked weight tiles
  const uint16_t* s_r;     // expert-stacked scales [E][NT][NG][16]
  const uint64_t* z_r;     // expert-stacked zero words [E][NT][NG]
  const int32_t* sorted;   // sorted routed rows (sentinel >= num_routed)
  const int32_t* offsets;  // padded bucket offsets [E + 1]
  const float* topk_w;     // routed weights [num_routed]
  void* out;               // [num_routed, N] or, paired, [num_routed, N / 2]
  int a_div;               // activation row of routed row r = r / a_div
  int num_routed, sorted_cap;
  int N, K, NT, KT, NG, gshift;
  int64_t w_stride, s_stride, z_stride;  // per-expert strides in u32x4 / scale / zero-word units
  int S, total;  // column slices per expert, S * E
  int mul_rw;
};

// Routed rows per pass: kMaxMt m-tiles of 16.  Two keep the kernel within
// the register budget of three workgroups per CU (the weight stream needs that
// many loads in flight); an expert with more rows takes more passes, spread
// over grid.y so that they run side by side and share the weights through L2.
constexpr int kMaxMt = 2;
constexpr int kXsBuf = kMaxMt * 4 * 64;  // one LDS buffer: [m-tile][k-block][lane]

// One pass over K for MC m-tiles (16 routed rows each) starting at sorted row
// rb.  The wave's four column tiles are ntc[0..3] of expert-local tile index.
template <int MC, int GPT, int EPI, typename DT>
__device__ __forceinline__ void moe_pass(const MoeArgs& a, u32x4* __restrict__ xs, const u32x4* __restrict__ we,
                                         const uint16_t* __restrict__ se, const uint64_t* __restrict__ ze,
                                         const int (&ntc)[4], const int (&ncol)[4], int rb, int wave, int lane) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using V4 = typename DT::vec4;
  using ZS = typename Dq<DT>::ZS;
  constexpr int BPG = 4 / GPT;  // 32-row k-blocks per group
  const int c = lane & 15, lg = lane >> 4;
  const void* x = a.x;

  // Routed row of lane column c in m-tile i (loader and epilogue share it).
  int sid[MC];
  uint32_t xoff[MC];  // byte offset of the row (the host keeps `a` below 4 GiB)
  bool xval[MC];
#pragma unroll
  for (int i = 0; i < MC; ++i) {
    sid[i] = a.sorted[rb + i * 16 + c];
    xval[i] = sid[i] >= 0 && sid[i] < a.num_routed;
    xoff[i] = (uint32_t)(xval[i] ? sid[i] / a.a_div : 0) * (uint32_t)a.K * 2u;
  }

  f32x4 acc[MC][4];
#pragma unroll
  for (int mt = 0; mt < MC; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Per-tile byte offsets inside the expert.
  uint32_t woff[4], goff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    woff[j] = ((uint32_t)ntc[j] * (uint32_t)a.KT * 64u + lane) * 16u;
    goff[j] = (uint32_t)ntc[j] * (uint32_t)a.NG;
  }

  // Everything one k-tile needs from global memory.  Two stages alternate
  // (the loop is unrolled by two) so that no register copy waits for the
  // prefetched loads before their use.
  struct Stage {
    u32x4 q[4];           // weight words of the four column tiles
    uint32_t z[4][GPT];   // zero-point word holding the lane's nibble
    uint32_t s[4][GPT];   // scale bits
    u32x4 xr[MC];         // activation fragments bound for LDS
  };

  // Rows of padding read activation row 0 and are never stored (MFMA output
  // column m depends on activation row m only).  k-blocks past K (K % 128 != 0)
  // are zeroed when they are written to LDS, so the loads themselves carry no
  // select that would make the wave wait for them right after issue.
  auto load = [&](int kt, Stage& st) {
    const uint32_t koff = (uint32_t)min(kt * 128 + wave * 32, a.K - 32) * 2u + (uint32_t)lg * 16u;
#pragma unroll
    for (int i = 0; i < MC; ++i) st.xr[i] = ld_off<u32x4>(x, xoff[i] + koff);
#pragma unroll
    for (int j = 0; j < 4; ++j) st.q[j] = ld_off_nt<u32x4>(we, woff[j] + (uint32_t)kt * 1024u);
#pragma unroll
    for (int gg = 0; gg < GPT; ++gg) {
      const uint32_t g = (uint32_t)min((kt * 128 + 32 * BPG * gg) >> a.gshift, a.NG - 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t gi = goff[j] + g;
        st.z[j][gg] = ld_off<uint32_t>(ze, gi * 8u + (uint32_t)(c >> 3) * 4u);
        st.s[j][gg] = ld_off<uint16_t>(se, (gi * 16u + c) * 2u);
      }
    }
  };
  auto store_x = [&](const Stage& st, int kt) {
    const bool kval = kt * 128 + wave * 32 < a.K;
    const int buf = kt & 1;
#pragma unroll
    for (int i = 0; i < MC; ++i)
      xs[buf * kXsBuf + (i * 4 + wave) * 64 + lane] = kval ? st.xr[i] : u32x4{0u, 0u, 0u, 0u};
  };
  auto compute = [&](const Stage& st, int kt) {
    const int buf = kt & 1;
#pragma unroll
    for (int gg = 0; gg < GPT; ++gg) {
      ZS zs[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) zs[j] = Dq<DT>::make((st.z[j][gg] >> (4 * (c & 7))) & 0xFu, (uint16_t)st.s[j][gg]);
#pragma unroll
      for (int b = 0; b < BPG; ++b) {
        const int w = gg * BPG + b;  // k-blocks past K meet zeroed activations
        V8 av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) av[j] = Dq<DT>::word(st.q[j][w], zs[j]);
#pragma unroll
        for (int mt = 0; mt < MC; ++mt) {
          const V8 bx = __builtin_bit_cast(V8, xs[buf * kXsBuf + (mt * 4 + w) * 64 + lane]);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[mt][j] = mfma16x16x32(av[j], bx, acc[mt][j]);
        }
      }
    }
  };
  // One k-tile: prefetch the next (the last tile reloads itself, so the loads
  // are unconditional), compute this one, publish the next tile's activations.
  auto step = [&](int kt, const Stage& cur, Stage& nxt) {
    const int nk = min(kt + 1, a.KT - 1);
    load(nk, nxt);
    // Keep the prefetch ahead of this tile's math (the scheduler would
    // otherwise start the math first, waiting for this tile's loads while the
    // next tile's are not yet issued).
    __builtin_amdgcn_sched_barrier(0);
    compute(cur, kt);
    store_x(nxt, kt + 1);
    __syncthreads();
  };

  Stage sa, sb;
  load(0, sa);
  store_x(sa, 0);
  __syncthreads();
  for (int kt = 0; kt < a.KT; kt += 2) {
    step(kt, sa, sb);
    if (kt + 1 < a.KT) step(kt + 1, sb, sa);
  }

  // Epilogue: lane (c, lg) of fragment (mt, j) holds row c of m-tile mt and
  // columns 4lg..4lg+3 of tile j.
  E* out = (E*)a.out;
#pragma unroll
  for (int mt = 0; mt < MC; ++mt) {
    if (!xval[mt]) continue;
    const float rw = a.mul_rw ? a.topk_w[sid[mt]] : 1.f;
    if constexpr (EPI == kEpiPlain) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (ncol[j] < 0 || ncol[j] + 4 * lg >= a.N) continue;  // N % 16 == 8: half of the last tile
        V4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = (E)(acc[mt][j][i] * rw);
        *(V4*)(out + (int64_t)sid[mt] * a.N + ncol[j] + 4 * lg) = r;
      }
    } else {
      // Tiles 0, 1 are gate tiles and 2, 3 the matching up tiles; the first
      // GEMM's output is rounded before the activation (fused.py:175-177).
      const int I = a.N >> 1;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (ncol[j] < 0) continue;
        V4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g = (float)(E)(acc[mt][j][i] * rw);
          const float u = (float)(E)(acc[mt][j + 2][i] * rw);
          r[i] = (E)(gate_act<EPI>(g) * u);
        }
        *(V4*)(out + (int64_t)sid[mt] * I + ncol[j] + 4 * lg) = r;
      }
    }
  }
}

template <int GPT, int EPI, typename DT>
__global__ __launch_bounds__(256) void moe_gemm_kernel(MoeArgs a) {
  __shared__ u32x4 xs[2 * kXsBuf];
  // XCD-aware placement: workgroup b runs on XCD b % 8; logical index L
  // walks the column slices of one expert on one XCD.
  const int per = gridDim.x >> 3;
  const int L = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (L >= a.total) return;
  const int e = L / a.S, slice = L % a.S;
  const int r0 = min(max(a.offsets[e], 0), a.sorted_cap);
  const int r1 = min(max(a.offsets[e + 1], r0), a.sorted_cap);
  const int nblk = (r1 - r0) >> 4;
  if ((int)blockIdx.y * kMaxMt >= nblk) return;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int ntc[4], ncol[4];
  if constexpr (EPI == kEpiPlain) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nt = slice * 16 + wave * 4 + j;
      ntc[j] = min(nt, a.NT - 1);
      ncol[j] = nt < a.NT && nt * 16 < a.N ? nt * 16 : -1;
    }
  } else {
    const int NTg = a.NT >> 1;  // gate tiles; up tile of gate tile t is t + NTg
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int gt = slice * 8 + wave * 2 + j;
      ntc[j] = min(gt, NTg - 1);
      ntc[j + 2] = ntc[j] + NTg;
      ncol[j] = gt < NTg ? gt * 16 : -1;
      ncol[j + 2] = -1;
    }
  }
  const u32x4* we = a.wt + e * a.w_stride;
  const uint16_t* se = a.s_r + e * a.s_stride;
  const uint64_t* ze = a.z_r + e * a.z_stride;

  static_assert(kMaxMt == 2, "pass dispatch below covers one and two m-tiles");
  for (int p = blockIdx.y; p * kMaxMt < nblk; p += gridDim.y) {
    const int rb = r0 + p * kMaxMt * 16;
    if (nblk - p * kMaxMt >= 2)
      moe_pass<2, GPT, EPI, DT>(a, xs, we, se, ze, ntc, ncol, rb, wave, lane);
    else
      moe_pass<1, GPT, EPI, DT>(a, xs, we, se, ze, ntc, ncol, rb, wave, lane);
    __syncthreads();  // the next pass refills both LDS buffers
  }
}

// ---------------------------------------------------------------------------
// Top-k combine (moe_sum_reduce, triton/fused_moe.py:7-50): fp32 sum over the
// k rows of each token, one cast.  Eight columns per thread.
// ---------------------------------------------------------------------------
template <typename DT>
__global__ __launch_bounds__(256) void moe_sum_kernel(const typename DT::elem* __restrict__ in,
                                                      typename DT::elem* __restrict__ out, int64_t T, int k, int64_t H) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = H >> 3;
  if (idx >= T * per_row) return;
  const int64_t t = idx / per_row, n0 = (idx % per_row) * 8;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < k; ++j) {
    const V8 v = *(const V8*)(in + (t * k + j) * H + n0);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] += (float)v[i];
  }
  V8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (E)s[i];
  *(V8*)(out + t * H + n0) = r;
}

template <typename DT>
hipError_t launch_moe_gemm_dt(const MoeArgs& a, int gpt, int epi, int passes, hipStream_t s) {
  const int64_t gx = (a.total + 7) / 8 * 8;
  dim3 grid((unsigned)gx, (unsigned)passes);
#define SGL_MOE(GPT_, EPI_)                                                                 \
  if (gpt == GPT_ && epi == EPI_) {                                                         \
    hipLaunchKernelGGL((moe_gemm_kernel<GPT_, EPI_, DT>), grid, dim3(256), 0, s, a);        \
    return hipGetLastError();                                                               \
  }
#define SGL_MOE_E(GPT_) SGL_MOE(GPT_, kEpiPlain) SGL_MOE(GPT_, kEpiSilu) SGL_MOE(GPT_, kEpiGelu)
  SGL_MOE_E(1)
  SGL_MOE_E(2)
  SGL_MOE_E(4)
#undef SGL_MOE_E
#undef SGL_MOE
  return hipErrorInvalidValue;
}

}  // namespace

MoeStrides moe_expert_strides(const Geom& g) {
  auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
  return MoeStrides{up(g.NT * g.KT * 1024), up(g.NT * g.NG * 16 * 2), up(g.NT * g.NG * 8)};
}

int64_t moe_sorted_capacity(int64_t n, int64_t E, int64_t bs) { return n + E * (bs - 1); }
int64_t moe_block_capacity(int64_t n, int64_t E, int64_t bs) { return (moe_sorted_capacity(n, E, bs) + bs - 1) / bs; }

hipError_t launch_moe_topk(const float* logits, float* tw, int32_t* tid, int64_t T, int64_t E, int64_t k, int renorm,
                           hipStream_t s) {
  const dim3 grid((unsigned)((T + 3) / 4));
  if (E <= 64) hipLaunchKernelGGL((topk_softmax_kernel<1>), grid, dim3(256), 0, s, logits, tw, tid, (int)T, (int)E, (int)k, renorm);
  else if (E <= 128) hipLaunchKernelGGL((topk_softmax_kernel<2>), grid, dim3(256), 0, s, logits, tw, tid, (int)T, (int)E, (int)k, renorm);
  else if (E <= 256) hipLaunchKernelGGL((topk_softmax_kernel<4>), grid, dim3(256), 0, s, logits, tw, tid, (int)T, (int)E, (int)k, renorm);
  else hipLaunchKernelGGL((topk_softmax_kernel<8>), grid, dim3(256), 0, s, logits, tw, tid, (int)T, (int)E, (int)k, renorm);
  return hipGetLastError();
}

hipError_t launch_moe_align(const int32_t* ids, int64_t n, int64_t E, int64_t bs, int32_t* sorted, int32_t* expert_ids,
                            int32_t* num_post_pad, int32_t* offsets, hipStream_t s) {
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(kAlignThreads), 0, s, ids, (int)n, (int)E, (int)bs, sorted, expert_ids,
                     (int)moe_block_capacity(n, E, bs), num_post_pad, offsets);
  return hipGetLastError();
}

hipError_t launch_moe_gemm(const MoeGemmParams& p, hipStream_t s) {
  MoeArgs a{};
  a.x = p.x;
  a.wt = (const u32x4*)p.w;
  a.s_r = (const uint16_t*)p.s;
  a.z_r = (const uint64_t*)p.z;
  a.sorted = p.sorted;
  a.offsets = p.offsets;
  a.topk_w = p.topk_w;
  a.out = p.out;
  a.a_div = (int)p.a_div;
  a.num_routed = (int)p.num_routed;
  a.sorted_cap = (int)p.sorted_cap;
  a.N = (int)p.g.N;
  a.K = (int)p.g.K;
  a.NT = (int)p.g.NT;
  a.KT = (int)p.g.KT;
  a.NG = (int)p.g.NG;
  a.gshift = p.g.gshift;
  const MoeStrides st = moe_expert_strides(p.g);
  a.w_stride = st.w / 16;
  a.s_stride = st.s / 2;
  a.z_stride = st.z / 8;
  a.S = p.epi == kEpiPlain ? (int)((p.g.NT + 15) / 16) : (int)((p.g.NT / 2 + 7) / 8);
  a.total = a.S * (int)p.E;
  a.mul_rw = p.mul_rw;
  const int gpt = (p.g.NG > 1 && p.g.G < 128) ? (int)(128 / p.g.G) : 1;
  // Passes per expert side by side: enough for an expert with the average
  // number of routed rows plus half a block of padding.
  const int64_t avg_rows = p.num_routed / p.E + 8;
  const int passes = (int)std::min<int64_t>(std::max<int64_t>((avg_rows + 16 * kMaxMt - 1) / (16 * kMaxMt), 1), 256);
  return p.dtype == 0 ? launch_moe_gemm_dt<F16>(a, gpt, p.epi, passes, s)
                      : launch_moe_gemm_dt<BF16>(a, gpt, p.epi, passes, s);
}

hipError_t launch_moe_sum(const void* in, void* out, int64_t T, int64_t k, int64_t H, int dtype, hipStream_t s) {
  const int64_t work = T * (H / 8);
  const dim3 grid((unsigned)((work + 255) / 256));
  if (work == 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL((moe_sum_kernel<F16>), grid, dim3(256), 0, s, (const _Float16*)in, (_Float16*)out, T, (int)k, H);
  else
    hipLaunchKernelGGL((moe_sum_kernel<BF16>), grid, dim3(256), 0, s, (const __bf16*)in, (__bf16*)out, T, (int)k, H);
  return hipGetLastError();
}

}  // namespace sgl_awq
