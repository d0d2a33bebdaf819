// Tiled W4A16 GEMM for gfx950: prefill batches (MFMA-bound at M >= ~256), and
// batches of 16-32 rows on wide or deep matrices (32-row block, split K).
//
// A workgroup of 4 waves computes BM x 256 outputs; wave w owns the 64 output
// columns of four 16-column weight tiles and all BM rows, so every packed
// weight word is dequantised exactly once per workgroup, straight from
// registers into MFMA operands.  The k loop runs over 128-row k-tiles with NS
// pipeline stages; stage p holds one k-tile's weights, zero points and scales
// in registers and its activation tile (BM x 128) in LDS buffer p:
//
//   * activation tiles go global -> LDS directly (buffer loads with the LDS
//     destination, no registers), stored in MFMA-fragment order so every
//     operand read is one conflict-free 16-byte LDS read.  Rows past M clamp
//     to a valid row (their outputs are never stored); k-blocks past K are
//     read through a zero-length buffer, which returns zeros without touching
//     memory;
//   * weights, zero points and scales go to registers; their offsets advance
//     in scalar registers (the buffer-load SGPR offset), so no load costs
//     vector ALU work;
//   * a k-tile's loads are issued NS - 1 steps before it is computed,
//     activations first.  The vector-memory counter retires in issue order,
//     so the end of each step waits for exactly the loads older than the
//     next k-tile's activations (a count fixed at compile time) and then
//     meets the other waves at a barrier that carries no memory fence (a
//     fenced barrier would also wait for the activation loads just issued);
//   * each k-tile's four 32-row blocks are software-pipelined: block w's MFMAs
//     run while block w + 1 is dequantised into the other operand buffer.
//
// Grids of fewer output tiles than CUs split K: each workgroup computes one
// k-slice of its tile into an fp32 partial, and a second kernel sums the
// slices in slice order (deterministic) and stores the output.
//
// Workgroups are numbered XCD-aware: the hardware deals consecutive
// workgroup ids round-robin over the 8 XCDs, and the id -> tile map makes the
// workgroups that one XCD runs together cover a compact patch of 4 row blocks
// x 8 column blocks, so that XCD's L2 serves the shared activation and weight
// tiles.
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410) for large batches.
#include "awq_buffer.h"
#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_fixup.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

struct TiledArgs {
  const void* x;
  const u32x4* w;
  const uint16_t* s;
  const uint64_t* z;
  const void* bias;
  void* out;
  float* part;  // split-K partials [ks][M][NT * 16]
  int M, N, K, NT, KT, NG, gshift;
  int gx, gy;  // column blocks (256 columns), row blocks (BM rows)
  int ks, ktc;  // k-slices and k-tiles per slice
  int act;      // fused gate/up activation (kActNone: plain GEMM)
  uint32_t* tcnt;  // split tiles' counters for the in-kernel reduction (null: a second kernel sums the slices)
  int polls;       // poll bound of a workgroup waiting for its tile's other k-slices
};

// Workgroup id -> (column block, row block).  Ids b, b + 8, b + 16, ... run
// on one XCD; they are given consecutive logical indices, and logical
// indices walk groups of up to 4 row blocks column-major.
__device__ __forceinline__ void tile_of(int b, int gx, int gy, int& bx, int& by) {
  const int total = gx * gy;
  const int per = total >> 3, rem = total & 7;
  const int xcd = b & 7, idx = b >> 3;
  const int L = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
  const int band = 4 * gx;                // logical indices per group of 4 row blocks
  const int grp = L / band;
  const int rows = min(4, gy - grp * 4);  // row blocks in this group
  const int r = L - grp * band;
  bx = r / rows;
  by = grp * 4 + r % rows;
}

// Zero points and scales of a workgroup's TPW = 4 NW column tiles, staged in
// LDS in chunks of 6 quantisation groups: zero words [tile][group][8 B] in
// the first TPW / 16 KiB, scales [tile][group][16 x 2 B] in the rest, one
// 1 KiB buffer load into LDS per wave and chunk (waves below kZD copy zero
// words -- 16-byte slot i of the region is tile i / 3, groups 2 (i % 3) and
// + 1, slots past 3 TPW repeat slot 0 -- the others scales: slot i is tile
// i / 12, bytes 16 (i % 12) of its 192).  Tile slots are the workgroup's
// tiles in order, or with a fused gate/up activation its TPW / 2 gate tiles
// then their up tiles.  A chunk's first group goes in the scalar offset;
// groups past a tile's last read the next tile's (or, past the array,
// zeros) and are never used.
template <int NW>
struct ZsChunks {
  static constexpr int TPW = 4 * NW;
  static constexpr int kZD = TPW / 16;  // zero-word loads per chunk
  static constexpr int kSlots = NW * 64;  // 16-byte slots per chunk buffer
  static_assert(kZD * 64 >= 3 * TPW && (NW - kZD) * 64 == 12 * TPW, "one load per wave");
  __amdgpu_buffer_rsrc_t src;
  uint32_t off;
  bool zero;
  __device__ void init(const TiledArgs& a, int bx, int wave, int lane) {
    zero = wave < kZD;
    src = zero ? make_rsrc(a.z, (uint32_t)a.NT * (uint32_t)a.NG * 8u)
               : make_rsrc(a.s, (uint32_t)a.NT * (uint32_t)a.NG * 32u);
    auto slot_tile = [&](int u) {
      const int NTg = a.NT >> 1;
      const int tt = a.act ? (u < TPW / 2 ? bx * (TPW / 2) + u : NTg + bx * (TPW / 2) + u - TPW / 2) : bx * TPW + u;
      return (uint32_t)min(tt, a.NT - 1);
    };
    int si = wave * 64 + lane;
    if (zero) {
      si = si < 3 * TPW ? si : 0;
      off = slot_tile(si / 3) * (uint32_t)a.NG * 8u + (uint32_t)(si % 3) * 16u;
    } else {
      si -= kZD * 64;
      off = slot_tile(si / 12) * (uint32_t)a.NG * 32u + (uint32_t)(si % 12) * 16u;
    }
  }
  // The chunk starting at group g0 into buf.
  __device__ void copy(u32x4* buf, int g0, int wave) const {
    load_lds16(src, &buf[wave * 64], off, zero ? g0 * 8 : g0 * 32);
  }
  // Byte offsets in a chunk of the zero word and the scale of column c of
  // tile slot u, group 0 of the chunk (group i: + 8 i, + 32 i).
  static __device__ uint32_t zero_at(int u, int c) { return (uint32_t)u * 48u + (uint32_t)(c >> 3) * 4u; }
  static __device__ uint32_t scale_at(int u, int c) {
    return (uint32_t)kZD * 1024u + (uint32_t)u * 192u + (uint32_t)c * 2u;
  }
};

template <int GPT>
struct WStage {
  u32x4 q[4];          // one 16-byte weight vector per column tile
  uint32_t z[4][GPT];  // the zero-point word holding this lane's nibble, per group
  uint16_t s[4][GPT];  // this lane's column scale, per group
};

template <int BM, int GPT, int NS, typename DT>
__global__ __launch_bounds__(256) void tiled_kernel(TiledArgs a) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  constexpr int MTL = BM / 16;
  constexpr int NTW = 4;
  constexpr int XS = MTL * 4 * 64;              // 16-byte slots per activation buffer
  // Zero points and scales: with at most 6 groups per NS k-tiles they reach
  // LDS in ZsChunks, one chunk per NS k-tiles, double-buffered; otherwise each
  // stage loads them (2 GPT loads per tile).
  constexpr bool kZsLds = NS * GPT <= 6;
  using ZC = ZsChunks<4>;
  constexpr int kLoadsW = kZsLds ? NTW : NTW * (1 + 2 * GPT);  // load instructions per weight stage
  // Loads issued after a k-tile's activations, up to the end of the step
  // before that k-tile: its own weights and the NS - 2 k-tiles behind it.
  constexpr int kAfterX = (NS - 1) * kLoadsW + (NS - 2) * MTL;
  static_assert(kAfterX < 64, "vector-memory counter range");
  // One activation buffer per stage, as separate objects: the compiler then
  // knows which LDS loads an outstanding LDS-destination load can affect.
  // [m-tile * 4 + k-block][lane] -> one MFMA B operand (16 bytes)
  __shared__ u32x4 xs0[XS];
  __shared__ u32x4 xs1[XS];
  __shared__ u32x4 xs2[NS > 2 ? XS : 1];
  __shared__ u32x4 xs3[NS > 3 ? XS : 1];
  __shared__ u32x4 xs4[NS > 4 ? XS : 1];
  __shared__ u32x4 zsl[kZsLds ? 2 : 1][kZsLds ? ZC::kSlots : 1];  // zero-point / scale chunks
  auto xbuf = [&](int p) -> u32x4* {
    return p == 0 ? xs0 : (p == 1 ? xs1 : (p == 2 ? xs2 : (p == 3 ? xs3 : xs4)));
  };

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, lg = lane >> 4;
  // Workgroup -> (output tile, k-slice); k-slices of a tile are launched
  // tiles apart.
  const int tiles = a.gx * a.gy;
  const int kslice = (int)blockIdx.x / tiles;
  int bx, by;
  tile_of((int)blockIdx.x - kslice * tiles, a.gx, a.gy, bx, by);
  const int kt0 = kslice * a.ktc;
  const int nsteps = min(a.KT - kt0, a.ktc);
  const int kend = kt0 + nsteps;  // k-tiles from kend on belong to other slices
  const int m0 = by * BM;
  const int rows = min(BM, a.M - m0);
  const int K = a.K, KT = a.KT, NG = a.NG;
  const DqK dk = dq_consts();

  // Activations: this workgroup's rows; thread (wave, lane) loads fragment
  // (m-tile i, k-block wave) of each k-tile.
  const E* xb = (const E*)a.x + (int64_t)m0 * K;
  const uint32_t xbytes = (uint32_t)rows * (uint32_t)K * 2u;
  uint32_t xoff[MTL];
#pragma unroll
  for (int i = 0; i < MTL; ++i)
    xoff[i] = (uint32_t)min(i * 16 + c, rows - 1) * (uint32_t)K * 2u + (uint32_t)(wave * 64 + lg * 16);

  // Weights, zeros and scales of this wave's four column tiles, as two pairs
  // of adjacent tiles: tiles nt0 .. nt0 + 3, or with a fused gate/up
  // activation gate tiles t, t + 1 and their up tiles t + NT / 2, t + 1 + NT / 2
  // (the merged projection's halves), so one lane holds a gate and its up
  // column.  Tiles past the end clamp to the last tile; their columns are never
  // stored.  Each pair has its own buffer range, ending at its last real tile.
  const int nt0 = bx * 16 + wave * NTW;
  const int NTg = a.NT >> 1;
  const int pb0 = a.act ? (nt0 >> 1) : nt0;               // first tile of pair 0
  const int pb1 = a.act ? (nt0 >> 1) + NTg : nt0 + 2;     // first tile of pair 1
  int pt[NTW];  // physical tile of slot j
  bool pv[NTW];  // slot j's columns are stored
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    pt[j] = (j < 2 ? pb0 : pb1) + (j & 1);
    pv[j] = a.act ? (nt0 >> 1) + (j & 1) < NTg : pt[j] < a.NT;
  }
  __amdgpu_buffer_rsrc_t wr[2], zr[2], sr[2];
  uint32_t woff[NTW], zoff[NTW], soff[NTW];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int base = min(q == 0 ? pb0 : pb1, a.NT - 1);
    const uint32_t ntiles = (uint32_t)min(2, a.NT - base);
    wr[q] = make_rsrc(a.w + (int64_t)base * KT * 64, ntiles * (uint32_t)KT * 1024u);
    if constexpr (!kZsLds) {
      zr[q] = make_rsrc(a.z + (int64_t)base * NG, ntiles * (uint32_t)NG * 8u);
      sr[q] = make_rsrc(a.s + (int64_t)base * NG * 16, ntiles * (uint32_t)NG * 32u);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * q + h;
      const uint32_t dt = (uint32_t)(min(pt[j], a.NT - 1) - base);
      woff[j] = dt * (uint32_t)KT * 1024u + (uint32_t)lane * 16u;
      if constexpr (kZsLds) {
        // Slot j's tile slot in a chunk, and its zero word's and scale's offsets.
        const int u = a.act ? (q == 0 ? 0 : ZC::TPW / 2) + wave * 2 + h : wave * NTW + j;
        zoff[j] = ZC::zero_at(u, c);
        soff[j] = ZC::scale_at(u, c);
      } else {
        zoff[j] = dt * (uint32_t)NG * 8u + (uint32_t)(c >> 3) * 4u;
        soff[j] = (dt * (uint32_t)NG * 16u + (uint32_t)c) * 2u;
      }
    }
  }
  ZC zc;
  if constexpr (kZsLds) zc.init(a, bx, wave, lane);
  // Chunk ci: k-tiles kt0 + ci NS .. + NS - 1.
  auto chunk_g0 = [&](int ci) { return ((kt0 + ci * NS) * 128) >> a.gshift; };
  auto dma_chunk = [&](int ci) { zc.copy(zsl[ci & 1], chunk_g0(ci), wave); };
  // Zero-length range for the prefetches past the k-slice: the loads are
  // still issued (every wait count assumes a fixed number of loads per
  // step) but return zeros without a memory access.
  const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.w, 0u);
  const uint32_t zshift = 4u * (uint32_t)(c & 7);

  f32x4 acc[MTL][NTW];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Activation k-tile kt (zeros past K or past the k-slice), m-tiles
  // [i0, i1), into LDS buffer p.
  auto load_x = [&](int p, int kt, int i0, int i1) {
    const bool kval = kt < kend && kt * 128 + wave * 32 < K;  // wave-uniform
    const __amdgpu_buffer_rsrc_t r = make_rsrc(xb, kval ? xbytes : 0u);
    u32x4* dst = xbuf(p);
#pragma unroll
    for (int i = i0; i < i1; ++i) load_lds16(r, &dst[(i * 4 + wave) * 64], xoff[i], kt * 256);
  };
  // Weights, zero words and scales of k-tile kt (zeros past the k-slice).
  auto load_w = [&](WStage<GPT>& S, int kt) {
    const bool live = kt < kend;  // wave-uniform
    kt = min(kt, KT - 1);
    const int g0 = (kt * 128) >> a.gshift;  // first group of the k-tile
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const __amdgpu_buffer_rsrc_t rw = live ? wr[j >> 1] : r0;
      S.q[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff[j], kt * 1024, 0);
      if constexpr (!kZsLds) {
        const __amdgpu_buffer_rsrc_t rz = live ? zr[j >> 1] : r0, rs = live ? sr[j >> 1] : r0;
#pragma unroll
        for (int g = 0; g < GPT; ++g)
          S.z[j][g] = __builtin_amdgcn_raw_buffer_load_b32(rz, zoff[j] + 8 * g, g0 * 8, 0);
#pragma unroll
        for (int g = 0; g < GPT; ++g)
          S.s[j][g] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff[j] + 32 * g, g0 * 32, 0);
      }
    }
  };
  // Zero words and scales of k-tile kt from its chunk (k-tiles past the
  // slice are never computed: they read the last live one's).
  auto read_zs = [&](WStage<GPT>& S, int kt) {
    kt = min(kt, kend - 1);
    const int ci = (kt - kt0) / NS;
    const int gi = ((kt * 128) >> a.gshift) - chunk_g0(ci);
    const char* buf = (const char*)zsl[ci & 1];
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int g = 0; g < GPT; ++g) {
        S.z[j][g] = *(const uint32_t*)(buf + zoff[j] + (uint32_t)(gi + g) * 8u);
        S.s[j][g] = *(const uint16_t*)(buf + soff[j] + (uint32_t)(gi + g) * 32u);
      }
  };

  WStage<GPT> st[NS];
  ZS zs[NTW][GPT];  // dequantisation constants of the k-tile being computed
  V8 av[2][NTW];    // dequantised weights of the current and the next 32-row block
  V8 bf[2][MTL];    // activation fragments of the current and the next block
  auto make_zs = [&](const WStage<GPT>& S) {
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int g = 0; g < GPT; ++g) zs[j][g] = Dq<DT>::make((S.z[j][g] >> zshift) & 0xFu, S.s[j][g]);
  };
  // Operands of block w of a k-tile into buffer slot `slot`.
  auto fetch = [&](int slot, const WStage<GPT>& S, const u32x4* xsb, int w) {
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) bf[slot][mt] = __builtin_bit_cast(V8, xsb[(mt * 4 + w) * 64 + lane]);
#pragma unroll
    for (int j = 0; j < NTW; ++j) av[slot][j] = Dq<DT>::word(S.q[j][w], zs[j][w * GPT / 4], dk);
  };
  // The MFMAs of one block, with the LDS reads and dequantisation of the
  // next block spread between them (one LDS read, then four MFMAs each
  // followed by up to two VALU operations, per m-tile).
  auto mma = [&](int slot) {
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
      for (int j = 0; j < NTW; ++j) acc[mt][j] = mfma16x16x32(av[slot][j], bf[slot][mt], acc[mt][j]);
#pragma unroll
    for (int i = 0; i < MTL; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
#pragma unroll
      for (int r = 0; r < NTW; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // Every wave's activation loads of k-tile kt + 1 have landed, and every
  // wave is done reading the buffer that the next activation load refills.
  // The wait includes the LDS reads (lgkmcnt 0): block 3's operand reads and
  // the chunk reads are issued before the barrier but consumed after it, and
  // a barrier does not wait for them, while other waves refill that buffer
  // after it.  `drain` (the steps after the counted loop) waits for every
  // load: there the prefetches past the k-slice have no use, the compiler
  // removes their weight loads, and fewer loads follow k-tile kt + 1's
  // activations than kAfterX counts (with NS = 3 the last k-tile of a slice
  // was then multiplied with activation fragments that had not all landed).
  auto sync_step = [&](bool drain) {
    if (drain) __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(0));
    else __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(kAfterX));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // One k-tile.  Stage p holds k-tile kt; k-tile kt + NS - 1 is fetched into
  // stage pa (activations during blocks 0 and 1, weights during block 2), and
  // block 3 already prepares block 0 of k-tile kt + 1 (stage pn), so no step
  // starts with dequantisation work that no MFMA overlaps.
  // Zero-point / scale chunk ci + 2 is copied at the start of the second step
  // of the loop iteration that computes chunk ci's k-tiles: after the barrier
  // that ends chunk ci's last read (the first step's weight issue), and ahead
  // of the activation loads that the wait before its own first read (the
  // next iteration's second step) covers.
  auto step = [&](int p, int kt, bool drain) {
    const int pa = (p + NS - 1) % NS, pn = (p + 1) % NS;
    const int ka = kt + NS - 1;
    if constexpr (kZsLds) {
      if (p == 1) dma_chunk((kt - 1 - kt0) / NS + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    load_x(pa, ka, 0, MTL / 2);
    __builtin_amdgcn_sched_barrier(0);
    fetch(1, st[p], xbuf(p), 1);
    mma(0);
    load_x(pa, ka, MTL / 2, MTL);
    __builtin_amdgcn_sched_barrier(0);
    fetch(0, st[p], xbuf(p), 2);
    mma(1);
    load_w(st[pa], ka);  // the wait counts rely on this issue order
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kZsLds) {
      // Complete at the next barrier (sync_step waits for the LDS reads), after
      // which a chunk buffer may be refilled.
      read_zs(st[pa], ka);
      __builtin_amdgcn_sched_barrier(0);
    }
    fetch(1, st[p], xbuf(p), 3);
    mma(0);
    sync_step(drain);
    make_zs(st[pn]);
    fetch(0, st[pn], xbuf(pn), 0);
    mma(1);
  };

  // Prologue: zero-point / scale chunks 0 and 1, k-tiles 0 .. NS - 2 in
  // flight, block 0 of k-tile 0 prepared.
  if constexpr (kZsLds) {
    dma_chunk(0);
    dma_chunk(1);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int p = 0; p + 1 < NS; ++p) {
    load_x(p, kt0 + p, 0, MTL);
    __builtin_amdgcn_sched_barrier(0);
    load_w(st[p], kt0 + p);
    __builtin_amdgcn_sched_barrier(0);
  }
  sync_step(false);
  if constexpr (kZsLds) {
#pragma unroll
    for (int p = 0; p + 1 < NS; ++p) read_zs(st[p], kt0 + p);
  }
  make_zs(st[0]);
  fetch(0, st[0], xbuf(0), 0);

  // Whole rounds of NS k-tiles, then the remaining k-tiles.  A counted loop
  // keeps every step's loads unconditional, so the compiler's wait counts
  // see the true prefetch distance.
  // (Prefetches past the k-slice return zeros that are never computed.)
  int i = 0;
  for (; i + NS <= nsteps; i += NS) {
#pragma unroll
    for (int p = 0; p < NS; ++p) step(p, kt0 + i + p, false);
  }
#pragma unroll
  for (int p = 0; p + 1 < NS; ++p)
    if (i + p < nsteps) step(p, kt0 + i + p, true);

  // The last steps prefetched past the end; no load may still be writing
  // this workgroup's LDS when it exits.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  const E* bias = (const E*)a.bias;
  E* out = (E*)a.out;
  if (a.ks == 1) {
    if (a.act == kActNone) {
#pragma unroll
      for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const int m = mt * 16 + c;
          const int n0 = pt[j] * 16 + 4 * lg;
          if (m < rows && n0 < a.N) store4<DT>(out, bias, (int64_t)m0 + m, a.N, n0, acc[mt][j]);
        }
    } else {
      const int Nh = a.N >> 1;
#pragma unroll
      for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int m = mt * 16 + c;
          if (m < rows && pv[j])
            store4_act<DT>(out, bias, (int64_t)m0 + m, Nh, pt[j] * 16 + 4 * lg, Nh, acc[mt][j], acc[mt][j + 2], a.act);
        }
    }
    return;
  }

  // Split K: this slice's partial tile, in fp32, written through to memory
  // (device-scope stores), then summed by the tile's k-slice workgroups
  // (splitk_fixup) or by the reduction kernel: no dirty L2 lines are left for
  // the end-of-kernel writeback that the reduction kernel waits for.  The
  // planner keeps ks * M * Np * 4 below 2^31, so one slice's byte offsets fit
  // the 32-bit buffer offset.
  const int Np = a.NT * 16;
  uint32_t* tc = a.tcnt != nullptr ? a.tcnt + (by * a.gx + bx) * kFixupWords : nullptr;
  uint32_t fbase = 0;
  if (tc != nullptr && threadIdx.x == 0) fbase = ld_sys_u32(tc + 1);
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part + (int64_t)kslice * a.M * Np, (uint32_t)a.M * (uint32_t)Np * 4u);
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int m = mt * 16 + c;
      const int n0 = pt[j] * 16 + 4 * lg;
      if (m < rows && pv[j])
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt][j]), pr,
                                               ((uint32_t)(m0 + m) * (uint32_t)Np + (uint32_t)n0) * 4u, 0,
                                               kCacheDevice);
    }
  if (tc != nullptr) {
    // 256 columns (16 tiles) per workgroup; with a fused activation 128 gate columns.
    const FixupTile<DT> ft{a.part, out, bias, a.M, a.N, Np, a.ks, a.act, m0, rows,
                           a.act ? bx * 128 : bx * 256, a.act ? 32 : 64};
    splitk_fixup<256, DT>(ft, tc, fbase, kslice, a.polls);
  }
}

// Sum of the k-slices' partials in slice order (deterministic), plus bias, in
// the output dtype (with a fused gate/up activation: gate and up sums, then
// act(gate) * up).  One thread per four output columns; every slice's 16-byte
// load is issued before the first is added (KSMAX >= ks loads, the slices past
// ks read as zeros through the buffer range), so the reduction costs one
// memory round trip whatever the slice count.
template <int KSMAX, typename DT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part,
                                                            const typename DT::elem* __restrict__ bias,
                                                            typename DT::elem* __restrict__ out, int M, int N,
                                                            int Np, int ks, int act) {
  const uint32_t slice = (uint32_t)M * (uint32_t)Np * 4u;  // bytes per k-slice
  const __amdgpu_buffer_rsrc_t r = make_rsrc(part, slice * (uint32_t)ks);
  // Sum of four consecutive partial columns starting at byte offset off.
  auto sum4 = [&](uint32_t off) {
    f32x4 v[KSMAX];
#pragma unroll
    for (int i = 0; i < KSMAX; ++i)
      v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, (int)((uint32_t)i * slice), 0));
    f32x4 sum = v[0];
#pragma unroll
    for (int i = 1; i < KSMAX; ++i) sum += v[i];
    return sum;
  };
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int No = act == kActNone ? N : N / 2;  // output columns
  const int64_t m = q / (No / 4);
  const int64_t n0 = 4 * (q - m * (No / 4));
  if (m >= M) return;
  const uint32_t off = ((uint32_t)m * (uint32_t)Np + (uint32_t)n0) * 4u;
  if (act == kActNone) {
    store4<DT>(out, bias, m, N, n0, sum4(off));
  } else {
    // Gate column n0 and its up column n0 + N / 2 (both in the partials).
    const f32x4 g = sum4(off), u = sum4(off + (uint32_t)(N / 2) * 4u);
    store4_act<DT>(out, bias, m, No, n0, No, g, u, act);
  }
}

template <typename DT>
hipError_t launch_splitk_reduce(const float* part, const void* bias, void* out, const Geom& g, int ks, int act,
                                hipStream_t s) {
  using E = typename DT::elem;
  const int64_t quads = g.M * ((act == kActNone ? g.N : g.N / 2) / 4);
  const dim3 grid((unsigned)((quads + 255) / 256)), block(256);
  const int M = (int)g.M, N = (int)g.N, Np = (int)(g.NT * 16);
  if (ks <= 2)
    hipLaunchKernelGGL((splitk_reduce_kernel<2, DT>), grid, block, 0, s, part, (const E*)bias, (E*)out, M, N, Np, ks, act);
  else if (ks <= 4)
    hipLaunchKernelGGL((splitk_reduce_kernel<4, DT>), grid, block, 0, s, part, (const E*)bias, (E*)out, M, N, Np, ks, act);
  else if (ks <= 8)
    hipLaunchKernelGGL((splitk_reduce_kernel<8, DT>), grid, block, 0, s, part, (const E*)bias, (E*)out, M, N, Np, ks, act);
  else if (ks <= 16)
    hipLaunchKernelGGL((splitk_reduce_kernel<16, DT>), grid, block, 0, s, part, (const E*)bias, (E*)out, M, N, Np, ks,
                       act);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// 32x32 prefill kernel (v_mfma_f32_32x32x16).
//
// Same workgroup tile (BM x 256, 4 waves of 64 columns; or BM x 512 with 8
// waves, whose columns share one activation stage), pipeline and split-K
// scheme as tiled_kernel, but every MFMA is a 32x32x16 one: twice the work of
// a 16x16x32 MFMA per issued instruction, so per k-tile a wave issues half the
// MFMAs and the same dequantisation and LDS reads, leaving more issue slots for
// the vector work between them.  A wave owns two groups of 32 columns (tiles
// 2g, 2g + 1 of its four); per 16-row k-step s the MFMA A operand of lane l is
// one packed word -- column l % 32 of the group, rows 16 s + 8 (l / 32) .. + 7
// -- which the tile layout holds in word s / 2 of the 16-byte vector of lane
// (l % 16) + 16 (l / 32) (even s) or that lane + 32 (odd s) of tile
// (l % 32) / 16: two 16-byte loads per lane and group per k-tile, from the
// layout that the other kernels read.  The activation fragments in LDS are
// [m32 tile][k-step][lane] (lane l: row l % 32, columns 8 (l / 32) .. + 7).
// Each lane's accumulators hold column m = l % 32 of its m32 tile and the
// output columns 8 j + 4 (l / 32) .. + 3 (j = 0..3) of its column group.
// With KW = 2 (8 waves, BM x 256), waves w and w + 4 share columns and take
// the even and odd k-steps of each k-tile, so a one-workgroup-per-CU grid
// still runs two waves per SIMD without a smaller row block.
// ---------------------------------------------------------------------------

template <int BM, int GPT, int NS, int OCC, int NW, typename DT, int KW = 1>
__global__ __launch_bounds__(64 * NW, OCC) void mfma32_kernel(TiledArgs a) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  constexpr int MT = BM / 32;              // m32 tiles
  constexpr int XF = MT * 8;               // activation fragments (1 KiB) per k-tile
  static_assert(XF % NW == 0, "whole activation fragments per wave");
  constexpr int XPW = XF / NW;             // ... loaded by each wave
  // Zero points and scales: with at most 6 groups per NS k-tiles they reach
  // LDS in ZsChunks, one chunk per NS k-tiles, double-buffered; otherwise each
  // stage loads them (4 GPT loads per wave).
  constexpr bool kZsLds = NS * GPT <= 6;
  // KW = 2: waves w and w + NW / 2 own the same columns and split every
  // k-tile's eight k-steps, even and odd (each loads only its half of the
  // weight vectors); their accumulators are added through LDS at the end.
  constexpr int CW = NW / KW;  // column waves
  static_assert(KW == 1 || (KW == 2 && kZsLds), "the k-wave split reads its zero points and scales from LDS");
  using ZC = ZsChunks<CW>;
  constexpr int kLoadsW = kZsLds ? 4 / KW : 4 + 4 * GPT;  // weight-stage load instructions per k-tile
  constexpr int NST = 8 / KW;  // k-steps per k-tile of one wave
  // 128-row blocks issue a step's activation DMAs and weight loads spread
  // over the k-tile's eight k-steps (same order, so the same waits), not in
  // one burst before its first MFMA: the eight waves of a CU issue ~12 such
  // loads per k-tile each, the CU accepts one every ~24 cycles, and a wave
  // whose load waits in that queue cannot issue its MFMAs.  Between k-steps
  // the wait overlaps the MFMAs in flight (Llama-3-8B gate_up at M = 2048
  // 453 -> 434 us, Qwen3-4B down at M = 8192 424 -> 389 us; 32- and 64-row
  // forms, four or more waves per SIMD's worth of loads already in flight,
  // measured no gain and keep the burst).
  constexpr bool kSpread = kZsLds && BM >= 128;
  constexpr int kNL = XPW + kLoadsW;  // loads per step when spread
  constexpr int kAfterX = (NS - 1) * kLoadsW + (NS - 2) * XPW;
  static_assert(kAfterX < 64, "vector-memory counter range");
  __shared__ u32x4 xs0[(KW == 2 ? 2 : 1) * XF * 64];  // (KW = 2: also the final exchange, MT * 16 KiB)
  __shared__ u32x4 xs1[XF * 64];
  __shared__ u32x4 xs2[NS > 2 ? XF * 64 : 1];
  __shared__ u32x4 xs3[NS > 3 ? XF * 64 : 1];
  __shared__ u32x4 zsl[kZsLds ? 2 : 1][kZsLds ? ZC::kSlots : 1];  // zero-point / scale chunks
  auto xbuf = [&](int p) -> u32x4* { return p == 0 ? xs0 : (p == 1 ? xs1 : (p == 2 ? xs2 : xs3)); };

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cw = KW == 1 ? wave : wave % CW;  // column wave
  const int kw = KW == 1 ? 0 : wave / CW;     // k-wave: even (0) or odd (1) k-steps
  const int lane = threadIdx.x & 63;
  const int c32 = lane & 31, h = lane >> 5, c = lane & 15, t = (lane >> 4) & 1;
  const int tiles = a.gx * a.gy;
  const int kslice = (int)blockIdx.x / tiles;
  int bx, by;
  tile_of((int)blockIdx.x - kslice * tiles, a.gx, a.gy, bx, by);
  const int kt0 = kslice * a.ktc;
  const int nsteps = min(a.KT - kt0, a.ktc);
  const int kend = kt0 + nsteps;
  const int m0 = by * BM;
  const int rows = min(BM, a.M - m0);
  const int K = a.K, KT = a.KT, NG = a.NG;
  const DqK dk = dq_consts();

  // Activations: fragment f = i * 8 + s (m32 tile i, k-step s) of a k-tile;
  // wave w loads fragments w * XPW .. w * XPW + XPW - 1.
  const E* xb = (const E*)a.x + (int64_t)m0 * K;
  const uint32_t xbytes = (uint32_t)rows * (uint32_t)K * 2u;
  uint32_t xoff[XPW];
#pragma unroll
  for (int j = 0; j < XPW; ++j) {
    const int f = wave * XPW + j, i = f >> 3, st = f & 7;
    xoff[j] = (uint32_t)min(i * 32 + c32, rows - 1) * (uint32_t)K * 2u + (uint32_t)(st * 32 + h * 16);
  }

  // Weights of the wave's two column groups: group g covers slots 2g, 2g + 1
  // (with a fused gate/up activation: gate tiles t, t + 1 in group 0 and their
  // up tiles in group 1).  Tiles past the end clamp to the last tile.
  const int nt0 = bx * (4 * CW) + cw * 4;
  const int NTg = a.NT >> 1;
  const int pb0 = a.act ? (nt0 >> 1) : nt0;
  const int pb1 = a.act ? (nt0 >> 1) + NTg : nt0 + 2;
  int pt[4];
  bool pv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pt[j] = (j < 2 ? pb0 : pb1) + (j & 1);
    pv[j] = a.act ? (nt0 >> 1) + (j & 1) < NTg : pt[j] < a.NT;
  }
  __amdgpu_buffer_rsrc_t wr[2], zr[2], sr[2];
  uint32_t woff[2], zoff[2], soff[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int base = min(g == 0 ? pb0 : pb1, a.NT - 1);
    const uint32_t ntiles = (uint32_t)min(2, a.NT - base);
    wr[g] = make_rsrc(a.w + (int64_t)base * KT * 64, ntiles * (uint32_t)KT * 1024u);
    const uint32_t dt = (uint32_t)(min(pt[2 * g + t], a.NT - 1) - base);  // this lane's tile in the range
    woff[g] = dt * (uint32_t)KT * 1024u + (uint32_t)(c + 16 * h) * 16u;  // + 512 for the odd-step vector
    if constexpr (kZsLds) {
      // This lane's tile slot in a chunk, and its zero word's and scale's offsets.
      const int u = a.act ? (g == 0 ? 0 : ZC::TPW / 2) + cw * 2 + t : cw * 4 + 2 * g + t;
      zoff[g] = ZC::zero_at(u, c);
      soff[g] = ZC::scale_at(u, c);
    } else {
      zr[g] = make_rsrc(a.z + (int64_t)base * NG, ntiles * (uint32_t)NG * 8u);
      sr[g] = make_rsrc(a.s + (int64_t)base * NG * 16, ntiles * (uint32_t)NG * 32u);
      zoff[g] = dt * (uint32_t)NG * 8u + (uint32_t)(c >> 3) * 4u;
      soff[g] = (dt * (uint32_t)NG * 16u + (uint32_t)c) * 2u;
    }
  }
  const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.w, 0u);
  const uint32_t zshift = 4u * (uint32_t)(c & 7);
  ZC zc;
  if constexpr (kZsLds) zc.init(a, bx, cw, lane);
  // Chunk ci: k-tiles kt0 + ci NS .. + NS - 1.
  auto chunk_g0 = [&](int ci) { return ((kt0 + ci * NS) * 128) >> a.gshift; };
  auto dma_chunk = [&](int ci) {
    if (kw == 0) zc.copy(zsl[ci & 1], chunk_g0(ci), cw);
  };
  // KW = 2: this wave's half of each weight vector pair (its k-steps' words).
  uint32_t woffk[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) woffk[g] = woff[g] + 512u * (uint32_t)kw;

  f32x16 acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][g][e] = 0.f;

  auto load_x1 = [&](int p, int kt, int j) {
    const int f = wave * XPW + j, st = f & 7;
    const bool kval = kt < kend && kt * 128 + st * 16 < K;  // wave-uniform
    const __amdgpu_buffer_rsrc_t r = make_rsrc(xb, kval ? xbytes : 0u);
    load_lds16(r, &xbuf(p)[f * 64], xoff[j], kt * 256);
  };
  auto load_x = [&](int p, int kt) {
#pragma unroll
    for (int j = 0; j < XPW; ++j) load_x1(p, kt, j);
  };
  // Weight vector i (group i / 2, odd-step half i % 2) of k-tile kt.
  auto load_w1 = [&](WStage32<GPT>& S, int kt, int i) {
    const bool live = kt < kend;
    kt = min(kt, KT - 1);
    if constexpr (KW == 1) {
      const int g = i >> 1, hf = i & 1;
      S.q[g][hf] = __builtin_amdgcn_raw_buffer_load_b128(live ? wr[g] : r0, woff[g] + 512u * hf, kt * 1024, 0);
    } else {
      S.q[i][0] = __builtin_amdgcn_raw_buffer_load_b128(live ? wr[i] : r0, woffk[i], kt * 1024, 0);
    }
  };
  auto load_w = [&](WStage32<GPT>& S, int kt) {
    const bool live = kt < kend;
    kt = min(kt, KT - 1);
    const int g0 = (kt * 128) >> a.gshift;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const __amdgpu_buffer_rsrc_t rw = live ? wr[g] : r0;
      if constexpr (KW == 1) {
        S.q[g][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff[g], kt * 1024, 0);
        S.q[g][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff[g] + 512u, kt * 1024, 0);
      } else {
        S.q[g][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, woffk[g], kt * 1024, 0);
      }
      if constexpr (!kZsLds) {
        const __amdgpu_buffer_rsrc_t rz = live ? zr[g] : r0, rs = live ? sr[g] : r0;
#pragma unroll
        for (int q = 0; q < GPT; ++q)
          S.z[g][q] = __builtin_amdgcn_raw_buffer_load_b32(rz, zoff[g] + 8 * q, g0 * 8, 0);
#pragma unroll
        for (int q = 0; q < GPT; ++q)
          S.s[g][q] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff[g] + 32 * q, g0 * 32, 0);
      }
    }
  };
  // Zero words and scales of k-tile kt from its chunk (k-tiles past the
  // slice are never computed: they read the last live one's).
  auto read_zs = [&](WStage32<GPT>& S, int kt) {
    kt = min(kt, kend - 1);
    const int ci = (kt - kt0) / NS;
    const int gi = ((kt * 128) >> a.gshift) - chunk_g0(ci);
    const char* buf = (const char*)zsl[ci & 1];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int q = 0; q < GPT; ++q) {
        S.z[g][q] = *(const uint32_t*)(buf + zoff[g] + (uint32_t)(gi + q) * 8u);
        S.s[g][q] = *(const uint16_t*)(buf + soff[g] + (uint32_t)(gi + q) * 32u);
      }
  };
  // One k-tile: 8 k-steps of MT x 2 MFMAs.  The LDS reads and the
  // dequantisation of step s + 1 are issued between step s's MFMAs (one LDS
  // read and a few vector operations after each MFMA), so no MFMA waits for
  // an operand produced just before it.
  auto compute = [&](const WStage32<GPT>& S, const u32x4* xsb, auto&& hook) {
    ZS zs[2][GPT];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int q = 0; q < GPT; ++q) zs[g][q] = Dq<DT>::make((S.z[g][q] >> zshift) & 0xFu, S.s[g][q]);
    V8 av[2][2];
    V8 bx[2][MT];
    // Step s of this wave is k-step KW s + kw of the k-tile.
    const u32x4* xk = xsb + kw * 64;
    auto word_of = [&](int g, int sn) -> uint32_t {
      if constexpr (KW == 1) return S.q[g][sn & 1][sn >> 1];
      else return S.q[g][0][sn];
    };
#pragma unroll
    for (int i = 0; i < MT; ++i) bx[0][i] = __builtin_bit_cast(V8, xk[i * 8 * 64 + lane]);
#pragma unroll
    for (int g = 0; g < 2; ++g) av[0][g] = Dq<DT>::word(word_of(g, 0), zs[g][0], dk);
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      hook(st);
      const int cur = st & 1, nxt = cur ^ 1;
      if (st + 1 < NST) {
        const int sn = st + 1;
#pragma unroll
        for (int i = 0; i < MT; ++i) bx[nxt][i] = __builtin_bit_cast(V8, xk[(i * 8 + KW * sn) * 64 + lane]);
#pragma unroll
        for (int g = 0; g < 2; ++g) av[nxt][g] = Dq<DT>::word(word_of(g, sn), zs[g][sn * GPT * KW / 8], dk);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int g = 0; g < 2; ++g) acc[i][g] = mfma32x32x16(av[cur][g], bx[cur][i], acc[i][g]);
      if (st + 1 < NST) {
        // 2 MT MFMAs, MT LDS reads and 26 vector operations (two words'
        // dequantisation) per step: after each MFMA one LDS read (while
        // there are any) and up to four vector operations.
#pragma unroll
        for (int i = 0; i < 2 * MT; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          if (i < MT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // As in tiled_kernel: the wait covers the LDS reads as well (the compiler
  // moves a k-tile's last MFMAs, and the operand reads they consume, past the
  // barrier, after which other waves refill that buffer), and the steps after
  // the counted loop, whose useless weight prefetches the compiler removes,
  // wait for every load.
  auto sync_step = [&](bool drain) {
    if (drain) __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(0));
    else __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0_imm(kAfterX));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Issue order (the wait counts rely on it): chunk DMAs, activations, weights.
  // Chunks 0 and 1 are copied first; chunk ci + 2 in the second step of the
  // loop iteration that computes chunk ci's k-tiles, after the barrier that
  // ends chunk ci's last read (the first step's issue of k-tile
  // kt0 + ci NS + NS - 1), and more than one wait ahead of its first read
  // (the second step of the next iteration).
  WStage32<GPT> stg[NS];
  if constexpr (kZsLds) {
    dma_chunk(0);
    dma_chunk(1);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int p = 0; p + 1 < NS; ++p) {
    load_x(p, kt0 + p);
    __builtin_amdgcn_sched_barrier(0);
    load_w(stg[p], kt0 + p);
    __builtin_amdgcn_sched_barrier(0);
  }
  sync_step(false);
  if constexpr (kZsLds) {
#pragma unroll
    for (int p = 0; p + 1 < NS; ++p) read_zs(stg[p], kt0 + p);
  }
  auto step = [&](int p, int kt, bool drain) {
    const int pa = (p + NS - 1) % NS;
    if constexpr (kZsLds) {
      if (p == 1) dma_chunk((kt - 1 - kt0) / NS + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kSpread) {
      read_zs(stg[pa], kt + NS - 1);
      __builtin_amdgcn_sched_barrier(0);
      compute(stg[p], xbuf(p), [&](int st) {
#pragma unroll
        for (int l = st * kNL / NST; l < (st + 1) * kNL / NST; ++l) {
          if (l < XPW) load_x1(pa, kt + NS - 1, l);
          else load_w1(stg[pa], kt + NS - 1, l - XPW);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
    } else {
      load_x(pa, kt + NS - 1);
      __builtin_amdgcn_sched_barrier(0);
      load_w(stg[pa], kt + NS - 1);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kZsLds) {
        // Complete at the next barrier (sync_step waits for the LDS reads),
        // after which a chunk buffer may be refilled.
        read_zs(stg[pa], kt + NS - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      compute(stg[p], xbuf(p), [](int) {});
    }
    sync_step(drain);
  };
  int i = 0;
  for (; i + NS <= nsteps; i += NS) {
#pragma unroll
    for (int p = 0; p < NS; ++p) step(p, kt0 + i + p, false);
  }
#pragma unroll
  for (int p = 0; p + 1 < NS; ++p)
    if (i + p < nsteps) step(p, kt0 + i + p, true);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if constexpr (KW == 2) {
    // k-wave 1 hands its accumulators to k-wave 0 one column group at a time
    // through the first stage buffer (MT * 16 KiB, [column wave][m32 tile][quad]
    // [lane]); k-wave 0 adds them and stores.
    f32x4* red = (f32x4*)xs0;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      __syncthreads();  // every wave is done with the stage buffers (or the previous group)
      if (kw == 1) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            red[((cw * MT + i) * 4 + q) * 64 + lane] =
                f32x4{acc[i][g][4 * q], acc[i][g][4 * q + 1], acc[i][g][4 * q + 2], acc[i][g][4 * q + 3]};
      }
      __syncthreads();
      if (kw == 0) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 v = red[((cw * MT + i) * 4 + q) * 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][g][4 * q + e] += v[e];
          }
      }
    }
    // k-wave 1 has nothing left to store; with the in-kernel reduction it
    // still helps to sum the tile's k-slices.
    if (kw == 1 && (a.ks == 1 || a.tcnt == nullptr)) return;
  }

  // Output element e of acc[i][g]: row m0 + 32 i + c32, column 8 (e / 4) + 4 h
  // + e % 4 of group g, i.e. tile slot 2 g + e / 8, column 8 ((e / 4) & 1) +
  // 4 h + e % 4 of that tile.
  auto quad = [&](const f32x16& v, int j) { return f32x4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]}; };
  const E* bias = (const E*)a.bias;
  E* out = (E*)a.out;
  if (a.ks == 1) {
    if (a.act == kActNone) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int m = i * 32 + c32;
            const int n0 = pt[2 * g + (j >> 1)] * 16 + 8 * (j & 1) + 4 * h;
            if (m < rows && n0 < a.N) store4<DT>(out, bias, (int64_t)m0 + m, a.N, n0, quad(acc[i][g], j));
          }
    } else {
      const int Nh = a.N >> 1;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = i * 32 + c32;
          if (m < rows && pv[j >> 1])
            store4_act<DT>(out, bias, (int64_t)m0 + m, Nh, pt[j >> 1] * 16 + 8 * (j & 1) + 4 * h, Nh,
                           quad(acc[i][0], j), quad(acc[i][1], j), a.act);
        }
    }
    return;
  }
  const int Np = a.NT * 16;
  uint32_t* tc = a.tcnt != nullptr ? a.tcnt + (by * a.gx + bx) * kFixupWords : nullptr;
  uint32_t fbase = 0;
  if (tc != nullptr && threadIdx.x == 0) fbase = ld_sys_u32(tc + 1);
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part + (int64_t)kslice * a.M * Np, (uint32_t)a.M * (uint32_t)Np * 4u);
  if (KW == 1 || kw == 0) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = i * 32 + c32;
          const int slot = 2 * g + (j >> 1);
          const int n0 = pt[slot] * 16 + 8 * (j & 1) + 4 * h;
          if (m < rows && pv[slot])
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, quad(acc[i][g], j)), pr,
                                                   ((uint32_t)(m0 + m) * (uint32_t)Np + (uint32_t)n0) * 4u, 0,
                                                   kCacheDevice);
        }
  }
  if (tc != nullptr) {
    // 64 CW columns (4 CW tiles) per workgroup; with a fused activation 32 CW gate columns.
    const FixupTile<DT> ft{a.part, out, bias, a.M, a.N, Np, a.ks, a.act, m0, rows,
                           a.act ? bx * 32 * CW : bx * 64 * CW, a.act ? 8 * CW : 16 * CW};
    splitk_fixup<64 * NW, DT>(ft, tc, fbase, kslice, a.polls);
  }
}

// OCC = workgroups per CU the register budget is cut for (2: 256 registers,
// two waves per SIMD, each workgroup's activation stages in 64 KiB of LDS);
// NW = waves per workgroup (64 * NW columns).
template <int BM, int NS, int OCC, int NW, typename DT, int KW = 1>
hipError_t launch_bm32(const TiledArgs& a, int gpt, hipStream_t s) {
  const dim3 grid((unsigned)(a.gx * a.gy * a.ks)), block(64 * NW);
  switch (gpt) {
    case 1: hipLaunchKernelGGL((mfma32_kernel<BM, 1, NS, OCC, NW, DT, KW>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((mfma32_kernel<BM, 2, NS, OCC, NW, DT, KW>), grid, block, 0, s, a); break;
    case 4:
      if constexpr (KW == 1) {
        hipLaunchKernelGGL((mfma32_kernel<BM, 4, 2, OCC, NW, DT>), grid, block, 0, s, a);
        break;
      }
      return hipErrorInvalidValue;  // four groups per k-tile keep their per-stage zero/scale loads
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int BM, typename DT>
hipError_t launch_bm(const TiledArgs& a, int gpt, hipStream_t s) {
  const dim3 grid((unsigned)(a.gx * a.gy * a.ks)), block(256);
  constexpr int NS1 = BM == 32 ? 5 : 4;
  switch (gpt) {
    case 1: hipLaunchKernelGGL((tiled_kernel<BM, 1, NS1, DT>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((tiled_kernel<BM, 2, 3, DT>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((tiled_kernel<BM, 4, 2, DT>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename DT>
hipError_t launch_dt(const GemmPlan& p, const TiledArgs& a, int gpt, hipStream_t s) {
  switch (p.variant) {
    case 32: return launch_bm<32, DT>(a, gpt, s);
    case 64: return launch_bm<64, DT>(a, gpt, s);
    case 128: return launch_bm<128, DT>(a, gpt, s);
    case 1064: return launch_bm32<64, 3, 1, 4, DT>(a, gpt, s);
    case 1128: return launch_bm32<128, 3, 1, 4, DT>(a, gpt, s);
    case 2064: return launch_bm32<64, 3, 2, 4, DT>(a, gpt, s);
    case 2128: return launch_bm32<128, 2, 2, 4, DT>(a, gpt, s);
    case 4032: return launch_bm32<32, 3, 4, 4, DT>(a, gpt, s);
    case 8064: return launch_bm32<64, 3, 1, 8, DT>(a, gpt, s);
    case 8128: return launch_bm32<128, 3, 1, 8, DT>(a, gpt, s);
    case 9064: return launch_bm32<64, 3, 1, 8, DT, 2>(a, gpt, s);
    case 9128: return launch_bm32<128, 3, 1, 8, DT, 2>(a, gpt, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// Largest K the prefill kernel takes at row block bm: its per-workgroup
// activation offsets (bm rows of K elements) stay below 2^31 bytes.
int64_t tiled_max_k(int bm) { return ((int64_t(1) << 31) - 1) / (2 * (int64_t)bm); }

// `counters`: the split tiles' counters (kFixupBytes, awq_fixup.h) for the
// in-kernel reduction, or null for the reduction kernel.
hipError_t launch_tiled(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                        const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                        int act, hipStream_t s) {
  if (p.grid_x * p.grid_y * p.ks >= (int64_t(1) << 24)) return hipErrorInvalidConfiguration;
  TiledArgs a;
  a.x = x;
  a.w = (const u32x4*)w;
  a.s = (const uint16_t*)sr;
  a.z = (const uint64_t*)zr;
  a.bias = bias;
  a.out = out;
  a.M = (int)g.M;
  a.N = (int)g.N;
  a.K = (int)g.K;
  a.NT = (int)g.NT;
  a.KT = (int)g.KT;
  a.NG = (int)g.NG;
  a.gshift = g.gshift;
  a.gx = (int)p.grid_x;
  a.gy = (int)p.grid_y;
  a.ks = p.ks;
  a.ktc = p.ktc;
  a.part = (float*)ws;
  a.act = act;
  const bool fixup = p.ks > 1 && p.fixup && counters != nullptr;
  a.tcnt = fixup ? (uint32_t*)counters : nullptr;
  a.polls = p.polls;
  // Groups per 128-row k-tile: 1 for G >= 128 (or one group), else 128 / G.
  const int gpt = (g.NG > 1 && g.G < 128) ? (int)(128 / g.G) : 1;
  hipError_t e = dtype == 0 ? launch_dt<F16>(p, a, gpt, s) : launch_dt<BF16>(p, a, gpt, s);
  if (e != hipSuccess || p.ks == 1 || fixup) return e;
  return dtype == 0 ? launch_splitk_reduce<F16>((const float*)ws, bias, out, g, p.ks, act, s)
                    : launch_splitk_reduce<BF16>((const float*)ws, bias, out, g, p.ks, act, s);
}

}  // namespace sgl_awq
