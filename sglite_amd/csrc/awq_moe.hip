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
// The grouped GEMM streams a pass's gathered activation rows into a ring of
// LDS slots in MFMA fragment order by LDS-DMA, as many k-tiles ahead as the
// weights, so the four waves of a workgroup share one copy; each wave
// dequantises the weights of its own 32 columns straight from global memory
// into MFMA operands.  A workgroup runs several column slices of one expert
// back to back in one load pipeline, and two workgroups share a CU, paired
// heavy with light by their m-tile counts.  Each expert's weights are
// streamed from HBM once per forward; workgroups of one expert are placed on
// one XCD so the expert's activation rows are fetched into one L2.
#include <math.h>

#include <algorithm>

#include "awq_buffer.h"
#include "awq_device.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// ---------------------------------------------------------------------------
// Wave-level helpers.  Reductions use DPP row shifts and row broadcasts (an
// inclusive scan that leaves the total in lane 63) and v_readlane, not
// LDS-routed shuffles, whose latency dominates these small kernels.
// ---------------------------------------------------------------------------
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_or(float v, float identity) {
  // Lanes whose source is outside the row or masked off receive `identity`.
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, identity),
                                                               __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                               BANK_MASK, false));
}

template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v) {
  const float id = MAX ? -INFINITY : 0.f;
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = op(v, dpp_or<kRowShr1, 0xf, 0xf>(v, id));
  v = op(v, dpp_or<kRowShr2, 0xf, 0xf>(v, id));
  v = op(v, dpp_or<kRowShr4, 0xf, 0xe>(v, id));
  v = op(v, dpp_or<kRowShr8, 0xf, 0xc>(v, id));
  v = op(v, dpp_or<kRowBcast15, 0xa, 0xf>(v, id));
  v = op(v, dpp_or<kRowBcast31, 0xc, 0xf>(v, id));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ int read_lane(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
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
  mx = wave_reduce<true>(mx);
  float p[EPL], s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    p[i] = lane + 64 * i < E ? expf(v[i] - mx) : 0.f;
    s += p[i];
  }
  s = wave_reduce<false>(s);
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
    const float top = wave_reduce<true>(bv);
    uint64_t m = __ballot(bv == top);
    int widx = read_lane(bi, __builtin_ctzll(m));
    for (m &= m - 1; m; m &= m - 1) widx = min(widx, read_lane(bi, __builtin_ctzll(m)));  // exact ties only
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (widx == lane + 64 * i) p[i] = -1.f;
    if (lane == j) {
      wsel = top;
      isel = widx;
    }
    wsum += top;
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
//
// Wave w owns the contiguous rows [w * chunk, (w + 1) * chunk), so a row's
// place in its bucket is the bucket offset, plus that expert's rows in lower
// waves (a per-wave count and a prefix over waves), plus its rank inside its
// own wave.  The rank needs no workgroup barrier: a wave takes its rows 64 at
// a time in row order, the lanes of one expert find each other through a
// per-wave lane mask in LDS, and the wave's LDS operations run in issue
// order.  Sentinels are written in parallel over (expert, padding slot), block
// experts over blocks (a binary search of the offsets).
// ---------------------------------------------------------------------------
constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;
constexpr int kMaxExperts = 512;
constexpr int kAlignBatch = 4;  // 64-row groups a wave holds in registers per pass over its rows

__global__ __launch_bounds__(kAlignThreads) void align_kernel(const int32_t* __restrict__ ids, int n, int E, int bs,
                                                              int32_t* __restrict__ sorted, int32_t* __restrict__ expert_ids,
                                                              int blocks_cap, int32_t* __restrict__ num_post_pad,
                                                              int32_t* __restrict__ offsets) {
  // Per wave and expert: the wave's row count, then its first free position.
  __shared__ int wpos[kAlignWaves][kMaxExperts];
  // Per wave and expert: the lanes of the current 64-row group with that expert.
  __shared__ uint64_t wmask[kAlignWaves][kMaxExperts];
  __shared__ int cnt[kMaxExperts];
  __shared__ int off[kMaxExperts + 1];
  __shared__ int wtot[kAlignWaves];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int chunk = ((n + kAlignWaves - 1) / kAlignWaves + 63) & ~63;
  const int r0 = min(n, wave * chunk), r1 = min(n, r0 + chunk);

  for (int q = tid; q < kAlignWaves * E; q += kAlignThreads) {
    wpos[q / E][q % E] = 0;
    wmask[q / E][q % E] = 0;
  }
  // The ids of kAlignBatch 64-row groups, loaded together (one round trip).
  int er[kAlignBatch];
  auto load_batch = [&](int b0) {
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      const int i = b0 + r * 64 + lane;
      er[r] = i < r1 ? ids[i] : -1;
    }
  };
  const bool one_batch = chunk <= 64 * kAlignBatch;  // the ids stay in registers between the passes
  if (one_batch) load_batch(r0);
  __syncthreads();

  // Pass 1: rows per (wave, expert).
  for (int b0 = r0; b0 < r1; b0 += 64 * kAlignBatch) {  // wave-uniform
    if (!one_batch) load_batch(b0);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r)
      if (er[r] >= 0 && er[r] < E) atomicAdd(&wpos[wave][er[r]], 1);
  }
  __syncthreads();

  // Expert totals and each wave's offset inside its expert's rows.
  int pc = 0;
  if (tid < E) {
    int sum = 0;
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) {
      const int c = wpos[w][tid];
      wpos[w][tid] = sum;
      sum += c;
    }
    cnt[tid] = sum;
    pc = (sum + bs - 1) / bs * bs;
  }
  // Exclusive scan of the padded counts (E <= 1024: one expert per thread).
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
#pragma unroll
    for (int w = 0; w < kAlignWaves; ++w) wpos[w][tid] += base + incl - pc;
  }
  if (tid == E - 1) off[E] = base + incl;
  __syncthreads();

  // Offsets, sentinels and block experts.
  const int total = off[E];
  for (int e = tid; e <= E; e += kAlignThreads) offsets[e] = off[e];
  if (tid == 0) *num_post_pad = total;
  auto bucket_of = [&](int p) {  // the expert e with off[e] <= p < off[e + 1], for p < total
    int lo = 0, hi = E;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= p) lo = mid;
      else hi = mid;
    }
    return lo;
  };
  for (int q = tid; q < E * bs; q += kAlignThreads) {  // padding slot q % bs of expert q / bs
    const int e = q / bs, p = off[e] + cnt[e] + q % bs;
    if (p < off[e + 1]) sorted[p] = n;
  }
  for (int b = tid; b < blocks_cap; b += kAlignThreads) expert_ids[b] = b * bs < total ? bucket_of(b * bs) : -1;

  // Pass 2: stable scatter, wave by wave, 64 rows at a time.
  for (int b0 = r0; b0 < r1; b0 += 64 * kAlignBatch) {  // wave-uniform
    if (!one_batch) load_batch(b0);
#pragma unroll
    for (int r = 0; r < kAlignBatch; ++r) {
      const int e = er[r];
      const bool valid = e >= 0 && e < E;
      if (valid) atomicOr((unsigned long long*)&wmask[wave][e], 1ull << lane);
      if (valid) {
        const uint64_t m = wmask[wave][e];
        sorted[wpos[wave][e] + __popcll(m & lanes_below(lane))] = b0 + r * 64 + lane;
        if ((m & lanes_below(lane)) == 0) {  // lowest lane of the expert's group
          wpos[wave][e] += __popcll(m);
          wmask[wave][e] = 0;
        }
      }
    }
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
  uint32_t x_bytes;        // rows_in * K * 2 (below 2^31: the host checks)
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
  int S;      // column slices per expert
  int U;      // slices per workgroup, run back to back in one pipeline
  int SG;     // slice groups per expert, ceil(S / U)
  int total;  // SG * E
  int cpx;    // CUs per XCD
  int mul_rw;
};

// Workgroup shape: 4 waves (one per SIMD), each owning TW = 2 16-column
// tiles of a slice (128 columns per slice; with a gate/up activation a gate
// tile and its up tile).  Two workgroups run on a CU; with eight waves in one
// workgroup the younger wave of each SIMD finished its k loop microseconds
// after the older one, alone on the SIMD.  (Four tiles per wave halve the
// activation traffic per weight byte but need more than 256 VGPRs at four
// m-tiles, and measured no faster.)  A workgroup runs U slices of one expert
// back to back in one load pipeline (the next slice's first k-tiles are
// fetched during the current slice's last ones), so the routed-row set-up and
// the pipeline fill are paid once per workgroup; the host picks U for about
// two workgroups per CU.
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTilesPerWave = 2;
// Routed rows per pass: up to kMaxMt m-tiles of 16.  An expert with more rows
// takes more passes, spread over grid.y so that they run side by side and
// share the expert's weights through L2.
constexpr int kMaxMt = 4;
// The pass's activation rows reach LDS through a ring of k-tile slots of MC *
// 4 fragments of 1 KiB ([slot][m-tile][k-block][lane]) within 80 KiB, filled
// by LDS-DMA as many k-tiles ahead as the weights.
constexpr int kXsFrags = 80;

// Weight k-tiles held in registers per wave (NS: the one being multiplied and
// NS - 1 in flight): with one quantisation group per k-tile the host picks 4,
// or 3 where K spans a multiple of three k-tiles but not of four (the k loop
// is padded to a multiple of NS); 3 with two groups per k-tile and 2 with four
// (their zero and scale words take the registers).

// One pass over `units` slices (from slice u0) and all of K for MC m-tiles
// (16 routed rows each) starting at sorted row rb.  Tile j of the wave in
// slice u0 + u is tile0[j] + u * TSU of the expert (TSU = tiles per slice in
// each half); tiles past the expert's last read as zeros (the buffer ranges
// end there) and are never stored.
template <int MC, int TW, int GPT, int EPI, int NS, typename DT>
__device__ __forceinline__ void moe_pass(const MoeArgs& a, u32x4* __restrict__ xs, const u32x4* __restrict__ we,
                                         const uint16_t* __restrict__ se, const uint64_t* __restrict__ ze,
                                         const int (&tile0)[TW], int u0, int units, int rb, int wave, int lane) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using V4 = typename DT::vec4;
  using ZS = typename Dq<DT>::ZS;
  constexpr int BPG = 4 / GPT;      // 32-row k-blocks per group
  constexpr int FR = MC * 4;        // activation fragments per k-tile
  constexpr int R = kXsFrags / FR;  // ring slots
  static_assert(R >= NS + 1, "the slot being filled must not be the one the slowest wave still reads");
  constexpr int HT = EPI == kEpiPlain ? TW : TW / 2;  // tiles per wave in each half of a slice
  constexpr int TSU = kWaves * HT;                     // slice stride in tiles
  const int c = lane & 15, lg = lane >> 4;
  const int KT = a.KT;
  const DqK dk = dq_consts();

  // Routed row of lane column c in each m-tile (the loader and the epilogue
  // share it); padding rows read activation row 0 and are never stored (MFMA
  // output column m depends on activation row m only).
  int sid[MC];
  bool sval[MC];
  uint32_t xrow[MC];  // byte offset of the lane's activation row (below x_bytes < 2^31)
  float rw[MC];       // routed weight of the row, fetched now so the epilogue does not wait for it
#pragma unroll
  for (int i = 0; i < MC; ++i) {
    sid[i] = a.sorted[rb + i * 16 + c];
    sval[i] = sid[i] >= 0 && sid[i] < a.num_routed;
    xrow[i] = (uint32_t)(sval[i] ? sid[i] / a.a_div : 0) * (uint32_t)a.K * 2u + (uint32_t)lg * 16u;
    rw[i] = a.mul_rw && sval[i] ? a.topk_w[sid[i]] : 1.f;
  }

  // Activation k-tile kt -> ring slot by LDS-DMA: wave w brings k-block w of
  // every m-tile (fragment (m-tile, w) of 16 rows x 32 k), lane (c, lg) row
  // c's 8 elements at 8 lg, straight into slot position lane.  k-blocks past K
  // (the K tail and the padding k-tiles) read at offset x_bytes, outside the
  // buffer, which returns zeros.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  auto dma_x1 = [&](int kt, int slot, int mt) {
    const int k0 = kt * 128 + wave * 32;
    load_lds16(xr, xs + (slot * FR + mt * 4 + wave) * 64, k0 < a.K ? xrow[mt] + (uint32_t)k0 * 2u : a.x_bytes, 0);
  };
  auto dma_x = [&](int kt, int slot) {
#pragma unroll
    for (int mt = 0; mt < MC; ++mt) dma_x1(kt, slot, mt);
  };

  f32x4 acc[MC][TW];
#pragma unroll
  for (int mt = 0; mt < MC; ++mt)
#pragma unroll
    for (int j = 0; j < TW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The expert's weights, zero words and scales as buffer resources that end
  // at its last tile (explicit global loads with the slice, k-tile and group
  // offsets in scalar registers); per-lane byte offsets of the wave's tiles
  // in the first slice.
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(we, (uint32_t)a.NT * (uint32_t)KT * 1024u);
  const __amdgpu_buffer_rsrc_t zr = make_rsrc(ze, (uint32_t)a.NT * (uint32_t)a.NG * 8u);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(se, (uint32_t)a.NT * (uint32_t)a.NG * 32u);
  const uint32_t wsh = (uint32_t)TSU * (uint32_t)KT * 1024u;  // per-slice shifts
  const uint32_t zsh = (uint32_t)TSU * (uint32_t)a.NG * 8u;
  const uint32_t ssh = (uint32_t)TSU * (uint32_t)a.NG * 32u;
  uint32_t woff[TW], zoff[TW], soff[TW];
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    const uint32_t t = (uint32_t)(tile0[j] + u0 * TSU);
    woff[j] = (t * (uint32_t)KT * 64u + lane) * 16u;
    zoff[j] = t * (uint32_t)a.NG * 8u + (uint32_t)(c >> 3) * 4u;
    soff[j] = (t * (uint32_t)a.NG * 16u + (uint32_t)c) * 2u;
  }

  // A k-tile's weights, zero points and scales for the wave's tiles.
  struct Stage {
    u32x4 q[TW];          // weight words of the wave's column tiles
    uint32_t z[TW][GPT];  // zero-point word holding the lane's nibble
    uint16_t s[TW][GPT];  // scale bits (kept 16-bit: a widening would wait for the load at once)
  };
  // Load l of a k-tile's LW (in issue order: the TW weight vectors, then per
  // group each tile's zero word and scale).
  auto load_w1 = [&](int u, int kt, Stage& st, int l) {
    if (l < TW) {
      st.q[l] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff[l], u * wsh + kt * 1024, kCacheStream);
    } else {
      const int r = l - TW, gg = r / (2 * TW), j = (r % (2 * TW)) >> 1;
      const int g = min((kt * 128 + 32 * BPG * gg) >> a.gshift, a.NG - 1);
      if (r & 1) st.s[j][gg] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff[j], u * ssh + g * 32, 0);
      else st.z[j][gg] = __builtin_amdgcn_raw_buffer_load_b32(zr, zoff[j], u * zsh + g * 8, 0);
    }
  };
  auto load_w = [&](int u, int kt, Stage& st) {
#pragma unroll
    for (int l = 0; l < TW * (1 + 2 * GPT); ++l) load_w1(u, kt, st, l);
  };
  // One k-tile: the activation operands and dequantised weights of k-block
  // w + 1 are fetched while k-block w's MFMAs run (operands double-buffered),
  // so no MFMA waits for an LDS read or a dequantisation issued just before.
  auto compute = [&](const Stage& st, const u32x4* buf, auto&& hook) {
    ZS zs[TW][GPT];
#pragma unroll
    for (int gg = 0; gg < GPT; ++gg)
#pragma unroll
      for (int j = 0; j < TW; ++j) zs[j][gg] = Dq<DT>::make((st.z[j][gg] >> (4 * (c & 7))) & 0xFu, st.s[j][gg]);
    V8 av[2][TW], bx[2][MC];
#pragma unroll
    for (int mt = 0; mt < MC; ++mt) bx[0][mt] = __builtin_bit_cast(V8, buf[(mt * 4) * 64 + lane]);
#pragma unroll
    for (int j = 0; j < TW; ++j) av[0][j] = Dq<DT>::word(st.q[j][0], zs[j][0], dk);
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // k-blocks past K meet zeroed activations
      hook(w);
      const int cur = w & 1, nxt = cur ^ 1;
      if (w + 1 < 4) {
#pragma unroll
        for (int mt = 0; mt < MC; ++mt) bx[nxt][mt] = __builtin_bit_cast(V8, buf[(mt * 4 + w + 1) * 64 + lane]);
#pragma unroll
        for (int j = 0; j < TW; ++j) av[nxt][j] = Dq<DT>::word(st.q[j][w + 1], zs[j][(w + 1) / BPG], dk);
      }
#pragma unroll
      for (int mt = 0; mt < MC; ++mt)
#pragma unroll
        for (int j = 0; j < TW; ++j) acc[mt][j] = mfma16x16x32(av[cur][j], bx[cur][mt], acc[mt][j]);
      if (w + 1 < 4) {
        // MC * TW MFMAs, MC LDS reads and 13 * TW vector operations (TW
        // words' dequantisation) per k-block: spread the reads and the
        // vector work between the MFMAs.
#pragma unroll
        for (int i = 0; i < MC * TW; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
          if (i < MC) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // LDS read
          __builtin_amdgcn_sched_group_barrier(0x002, (13 * TW + MC * TW - 1) / (MC * TW), 0);  // VALU
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // Epilogue of slice u: lane (c, lg) of fragment (mt, j) holds row c of
  // m-tile mt and columns 4lg..4lg+3 of tile j.
  E* out = (E*)a.out;
  auto epilogue = [&](int u) {
#pragma unroll
    for (int mt = 0; mt < MC; ++mt) {
      if (!sval[mt]) continue;
      if constexpr (EPI == kEpiPlain) {
#pragma unroll
        for (int j = 0; j < TW; ++j) {
          const int nt = tile0[j] + (u0 + u) * TSU;
          if (nt >= a.NT || nt * 16 + 4 * lg >= a.N) continue;  // N % 16 == 8: half of the last tile
          V4 r;
#pragma unroll
          for (int i = 0; i < 4; ++i) r[i] = (E)(acc[mt][j][i] * rw[mt]);
          *(V4*)(out + (int64_t)sid[mt] * a.N + nt * 16 + 4 * lg) = r;
        }
      } else {
        // Tiles 0 .. TW/2 - 1 are gate tiles and tile j + TW/2 the up tile of
        // gate tile j; the first GEMM's output is rounded before the
        // activation (fused.py:175-177).
#pragma unroll
        for (int j = 0; j < HT; ++j) {
          const int gt = tile0[j] + (u0 + u) * TSU;
          if (gt >= (a.NT >> 1)) continue;
          V4 r;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = (float)(E)(acc[mt][j][i] * rw[mt]);
            const float v = (float)(E)(acc[mt][j + HT][i] * rw[mt]);
            r[i] = (E)(gate_act<EPI>(g) * v);
          }
          *(V4*)(out + (int64_t)sid[mt] * (a.N >> 1) + gt * 16 + 4 * lg) = r;
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MC; ++mt)
#pragma unroll
      for (int j = 0; j < TW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // The steps run over (slice, k-tile), k-tiles padded to KTp (a multiple of
  // NS); activations and weights run NS - 1 steps ahead of the multiply: each
  // step issues the activation DMA and then the weight loads of step
  // s + NS - 1 (the next slice's first k-tiles during this slice's last
  // ones), waits until its own loads of step s (and everything older) have
  // landed -- all but the NS - 1 newer steps' loads, the loads completing in
  // order -- and meets the other waves at a barrier, after which every wave's
  // DMA share of step s is in LDS.  The slot filled at step s held step
  // s + NS - 1 - R <= s - 2, which every wave finished before the previous
  // step's barrier.  The barrier is a bare s_barrier: a fence would wait for
  // all loads and drain the pipeline.  The loop runs without a branch around
  // any load or multiply, so each stage keeps its registers across iterations
  // and the compiler's waits are the exact in-order counts (a conditional step
  // makes it copy stage registers, and the copy waits for their loads):
  // padding k-tiles reload the last weight k-tile and meet zero activations,
  // and the steps past the last slice load what the buffer ranges allow and
  // are never multiplied.  A slice's epilogue runs between loop iterations
  // (its stores only make later waits stricter).
  constexpr int LW = TW * (1 + 2 * GPT);  // weight, zero and scale loads per k-tile
  // With NS >= 3 a step's loads (of step s + NS - 1) are issued spread over
  // the four k-blocks of step s's multiply instead of in one burst before it:
  // the CU accepts a vector-memory instruction every ~24 cycles, and a wave
  // whose load waits behind the other seven waves' cannot issue its MFMAs.
  // Its wait then leaves NS - 2 newer steps in flight (gate_up 69.8 -> 67.6
  // us, down 40.8 -> 39.7 us on the Qwen3-30B-A3B shape).  The slot a DMA
  // fills was last read at step s + NS - 1 - R <= s - 2, before the barrier
  // that starts step s.
  constexpr bool kSpread = NS >= 3;
  constexpr int kInFlight = (kSpread ? NS - 2 : NS - 1) * (MC + LW);  // loads of the newer steps
  static_assert(kInFlight <= 63, "vmcnt holds at most 63");
  const int KTp = (KT + NS - 1) / NS * NS;
  const int nsteps = units * KTp;
  int iu = 0, ik = 0, islot = 0;  // next step to issue: slice, k-tile, ring slot
  auto advance = [&]() {
    islot = islot + 1 == R ? 0 : islot + 1;
    ik = ik + 1 == KTp ? 0 : ik + 1;
    iu = ik == 0 ? iu + 1 : iu;
  };
  auto issue = [&](Stage& st) {
    dma_x(ik, islot);
    __builtin_amdgcn_sched_barrier(0);
    load_w(iu, min(ik, KT - 1), st);
    advance();
  };
  Stage st[NS];
  // The prologue issues in the steady-state order: activation DMAs, then the
  // weight, zero and scale loads, one step after the other.  The compiler's
  // waits in the loop are derived from both ways into it, so a prologue that
  // grouped the loads by kind (all steps' DMAs first, as the scheduler does
  // across a mere memory clobber) would make the loop's first two steps wait
  // for loads of the steps after them on every iteration.
#pragma unroll
  for (int p = 0; p + 1 < NS; ++p) {
    issue(st[p]);
    __builtin_amdgcn_sched_barrier(0);
  }
  int cu = 0, ck = 0, cslot = 0;  // step being multiplied
  // units >= 1 and KTp >= NS: the loop runs at least once, so its guard does
  // not pull the prologue's weight loads below it (past the DMAs of the
  // later steps).
  int s = 0;
  do {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      Stage& sn = st[(i + NS - 1) % NS];
      if constexpr (kSpread) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kInFlight));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int kt = min(ik, KT - 1);
        compute(st[i], xs + cslot * FR * 64, [&](int w) {
          constexpr int NL = MC + LW;
#pragma unroll
          for (int l = w * NL / 4; l < (w + 1) * NL / 4; ++l) {
            if (l < MC) dma_x1(ik, islot, l);
            else load_w1(iu, kt, sn, l - MC);
          }
          __builtin_amdgcn_sched_barrier(0);
        });
        advance();
      } else {
        issue(sn);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this tile's math
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kInFlight));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        compute(st[i], xs + cslot * FR * 64, [](int) {});
      }
      cslot = cslot + 1 == R ? 0 : cslot + 1;
    }
    ck += NS;
    if (ck == KTp) {  // workgroup-uniform; no stage registers change
      epilogue(cu);
      ck = 0;
      ++cu;
    }
    s += NS;
  } while (s < nsteps);
}

// Balanced placement of the slice groups of one XCD.  Launched on an idle
// device, workgroup b runs on XCD b % 8 as the j-th (j = b / 8) of that XCD,
// and local indices j and j + cpx share a CU.  A group's time grows with its
// pass's m-tile count (per slice ~5.6 + 1.7 * m-tiles us of a CU shared by two
// workgroups), so the XCD's groups are ranked by m-tile count, heaviest first,
// and the j-th heaviest shares a CU with the j-th lightest instead of two
// heavy groups meeting on one CU by chance.  Each wave ranks the groups
// itself (one lane per group, ballots); the result is the logical group
// index, or -1 for a local index with no group.  Placement other than assumed
// changes only the balance, never the result.  The chosen group's row range
// [r0, r1) comes back with it (the lane that ranked it has loaded it), which
// spares the workgroup a dependent load before its rows can be fetched.
__device__ __forceinline__ int balanced_group(const MoeArgs& a, int xcd, int per, int j, int lane, int& g_r0,
                                              int& g_r1) {
  const int L = xcd * per + lane;
  int key = -1;  // lanes past the XCD's groups take no rank
  int r0 = 0, r1 = 0;
  if (lane < per) {
    key = 0;
    if (L < a.total) {
      const int e = L / a.SG;
      r0 = min(max(a.offsets[e], 0), a.sorted_cap);
      r1 = min(max(a.offsets[e + 1], r0), a.sorted_cap);
      key = min((r1 - r0) >> 4, kMaxMt);
    }
  }
  int rank = 0;
#pragma unroll
  for (int v = kMaxMt; v >= 0; --v) {
    const uint64_t m = __ballot(key == v);
    if (key == v) rank += __popcll(m & lanes_below(lane));
    else if (key < v) rank += __popcll(m);
  }
  const int r = j < a.cpx ? j : per - 1 - (j - a.cpx);
  const uint64_t hit = __ballot(key >= 0 && rank == r);
  if (!hit) return -1;
  const int src = __builtin_ctzll(hit);
  g_r0 = __builtin_amdgcn_readlane(r0, src);
  g_r1 = __builtin_amdgcn_readlane(r1, src);
  return xcd * per + src;
}

template <int TW, int GPT, int EPI, int NS, typename DT>
__global__ __launch_bounds__(kThreads, 2) void moe_gemm_kernel(MoeArgs a) {
  __shared__ u32x4 xs[kXsFrags * 64];
  // XCD-aware placement: workgroup b runs on XCD b % 8; logical index L
  // walks the slice groups of one expert on one XCD.  With one pass per
  // expert and between one and two workgroups per CU the groups of an XCD are
  // paired heavy with light on its CUs.
  const int per = gridDim.x >> 3, xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int lane = threadIdx.x & 63;
  const bool balanced = gridDim.y == 1 && per > a.cpx && per <= 2 * a.cpx && per <= 64;
  int r0 = 0, r1 = 0;
  const int L = balanced ? balanced_group(a, xcd, per, j, lane, r0, r1) : xcd * per + j;
  if (L < 0 || L >= a.total) return;
  const int e = L / a.SG, grp = L % a.SG;
  const int u0 = grp * a.U, units = min(a.U, a.S - u0);
  if (!balanced) {
    r0 = min(max(a.offsets[e], 0), a.sorted_cap);
    r1 = min(max(a.offsets[e + 1], r0), a.sorted_cap);
  }
  const int nblk = (r1 - r0) >> 4;
  if ((int)blockIdx.y * kMaxMt >= nblk) return;

  const int wave = threadIdx.x >> 6;
  // Tiles of the wave in slice 0: TW consecutive tiles, or TW / 2 gate tiles
  // and their up tiles (up tile of gate tile t is t + NT / 2).
  int tile0[TW];
  if constexpr (EPI == kEpiPlain) {
#pragma unroll
    for (int j = 0; j < TW; ++j) tile0[j] = wave * TW + j;
  } else {
    constexpr int HT = TW / 2;
#pragma unroll
    for (int j = 0; j < HT; ++j) {
      tile0[j] = wave * HT + j;
      tile0[j + HT] = tile0[j] + (a.NT >> 1);
    }
  }
  const u32x4* we = a.wt + e * a.w_stride;
  const uint16_t* se = a.s_r + e * a.s_stride;
  const uint64_t* ze = a.z_r + e * a.z_stride;

  for (int p = blockIdx.y; p * kMaxMt < nblk; p += gridDim.y) {
    const int rb = r0 + p * kMaxMt * 16;
    switch (min(nblk - p * kMaxMt, kMaxMt)) {
      case 1: moe_pass<1, TW, GPT, EPI, NS, DT>(a, xs, we, se, ze, tile0, u0, units, rb, wave, lane); break;
      case 2: moe_pass<2, TW, GPT, EPI, NS, DT>(a, xs, we, se, ze, tile0, u0, units, rb, wave, lane); break;
      case 3: moe_pass<3, TW, GPT, EPI, NS, DT>(a, xs, we, se, ze, tile0, u0, units, rb, wave, lane); break;
      default: moe_pass<4, TW, GPT, EPI, NS, DT>(a, xs, we, se, ze, tile0, u0, units, rb, wave, lane); break;
    }
    // The last steps' DMAs and loads (past the last slice) land before the
    // next pass reuses the ring or the workgroup ends (the fence waits for them).
    __syncthreads();
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
hipError_t launch_moe_gemm_dt(const MoeArgs& a, int tw, int gpt, int epi, int passes, hipStream_t s) {
  const int64_t gx = (a.total + 7) / 8 * 8;
  dim3 grid((unsigned)gx, (unsigned)passes);
  const int ns = gpt >= 4 ? 2 : gpt == 2 ? 3 : (a.KT % 4 != 0 && a.KT % 3 == 0) ? 3 : 4;
#define SGL_MOE(TW_, GPT_, EPI_, NS_)                                                                \
  if (tw == TW_ && gpt == GPT_ && epi == EPI_ && ns == NS_) {                                        \
    hipLaunchKernelGGL((moe_gemm_kernel<TW_, GPT_, EPI_, NS_, DT>), grid, dim3(kThreads), 0, s, a);  \
    return hipGetLastError();                                                                        \
  }
#define SGL_MOE_E(TW_, GPT_, NS_) \
  SGL_MOE(TW_, GPT_, kEpiPlain, NS_) SGL_MOE(TW_, GPT_, kEpiSilu, NS_) SGL_MOE(TW_, GPT_, kEpiGelu, NS_)
  SGL_MOE_E(2, 1, 4)
  SGL_MOE_E(2, 1, 3)
  SGL_MOE_E(2, 2, 3)
  SGL_MOE_E(2, 4, 2)
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
  a.x_bytes = (uint32_t)((p.num_routed + p.a_div - 1) / p.a_div * p.g.K * 2);
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
  const int tw = kTilesPerWave;
  a.S = p.epi == kEpiPlain ? (int)((p.g.NT + kWaves * tw - 1) / (kWaves * tw))
                            : (int)((p.g.NT / 2 + kWaves * tw / 2 - 1) / (kWaves * tw / 2));
  a.mul_rw = p.mul_rw;
  const int gpt = (p.g.NG > 1 && p.g.G < 128) ? (int)(128 / p.g.G) : 1;
  // Passes per expert side by side: enough for an expert with the average
  // number of routed rows plus half a block of padding.
  const int64_t avg_rows = p.num_routed / p.E + 8;
  const int passes =
      (int)std::min<int64_t>(std::max<int64_t>((avg_rows + 16 * kMaxMt - 1) / (16 * kMaxMt), 1), 256);
  // Slices per workgroup: about two workgroups per CU over the grid.
  const int64_t units_total = (int64_t)a.S * p.E * passes;
  const int64_t cus = device_cu_count();
  a.U = (int)std::min<int64_t>(std::max<int64_t>((units_total + 2 * cus - 1) / (2 * cus), 1), a.S);
  a.cpx = (int)std::max<int64_t>(cus / 8, 1);
  a.SG = (a.S + a.U - 1) / a.U;
  a.total = a.SG * (int)p.E;
  return p.dtype == 0 ? launch_moe_gemm_dt<F16>(a, tw, gpt, p.epi, passes, s)
                      : launch_moe_gemm_dt<BF16>(a, tw, gpt, p.epi, passes, s);
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
