// Decode-size W4A16 GEMM (M <= 32) with the split-K reduction inside the
// kernel, on 32x32x16 MFMAs (gfx950).
//
// At up to 32 rows the int4 weights are nearly all of a GEMM's traffic, and a
// launch has to spread them over every CU: the narrow projections (o and down,
// 160 column tiles) split K across workgroups.  Summing the k-slices in a
// second kernel costs a launch, about as long as a narrow layer's whole weight
// stream; here the last workgroup of each column group to finish sums them.
// The release/acquire pair that handoff needs costs about as much as the launch
// it saves, so the planner does not choose this kernel; the planner override
// (AWQ_PLAN_KSLICE_VARIANT) does.
//
// Workgroup: 4 waves = WN column waves x WK k-waves.  A wave owns 64 output
// columns (two groups of 32 in the 32x32x16 operand order, WStage32) and KPW
// consecutive k-tiles of the workgroup's k-slice of WK * KPW k-tiles; the WK
// waves of one column range add their accumulators through LDS.  Every load
// of a workgroup is issued before any is used: each wave's weights, zero
// points and scales go to registers, then the slice's activation rows go
// global -> LDS (buffer loads with the LDS destination, whole cache lines per
// instruction, in an XOR-swizzled row-major layout that the MFMA operand reads
// without bank conflicts; shared by the WN column waves).  One wait and one
// barrier later each wave dequantises and multiplies its k-tiles.  Only the
// activation rows below M are loaded; k-chunks past K read as zeros.
//
// Split-K handoff: each workgroup writes its fp32 partial with device-scope
// (SC1, write-through) 16-byte stores and waits until they have completed;
// one thread then increments the column group's arrival counter with an
// agent-scope release (arrive_release: an L2 writeback first).  The
// workgroup that sees the count reach ks - 1 executes an agent-scope acquire
// (acquire_agent: L1/L2 invalidate), reads the ks partials back with
// system-scope loads (kCacheCoherentLoad), adds them in slice order -- the
// same order whichever workgroup finishes last, so results are deterministic
// -- stores the output (bias, fused gate/up activation) and resets the
// counter for the next launch.
//
// Workgroup ids map XCD-aware onto (column group, k-slice): the workgroups one
// XCD runs hold consecutive column groups of the same k-slice, so that XCD's
// L2 fetches the slice's activation once.
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410) for decode batches.
#include "awq_buffer.h"
#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

struct KsArgs {
  const void* x;
  const u32x4* w;
  const uint16_t* s;
  const uint64_t* z;
  const void* bias;
  void* out;
  float* part;        // split-K partials [ks][M][NT * 16]
  int32_t* counters;  // one per column group; zero between launches
  int M, N, K, NT, KT, NG, gshift;
  int gx;       // column groups (WN * 64 columns; with a fused activation WN * 32 gate columns)
  int ks, ktc;  // k-slices and k-tiles per slice
  int act;      // fused gate/up activation (kActNone: plain GEMM)
};

__device__ __forceinline__ f32x4 quad_of(const f32x16& v, int j) {
  return f32x4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
}

template <int WN, int WK, int KPW, int GPT, typename DT>
__global__ __launch_bounds__(256, 2) void kslice_kernel(KsArgs a) {
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  static_assert(WN * WK == 4, "four waves per workgroup");
  constexpr int KTC = WK * KPW;  // k-tiles of a full slice
  static_assert(KTC <= 8, "activation slice within 64 KiB of LDS");
  __shared__ u32x4 xs[KTC * 8 * 64];  // [k-tile of the slice][row / 4][16-byte slot]
  __shared__ int s_last;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wn = wave % WN, wk = wave / WN;
  const int c32 = lane & 31, h = lane >> 5, c = lane & 15, t = (lane >> 4) & 1;

  // Workgroup id -> (column group, k-slice): ids b, b + 8, ... run on one XCD
  // and get consecutive logical indices.
  int bx, kslice;
  {
    const int total = a.gx * a.ks;
    const int b = (int)blockIdx.x, per = total >> 3, rem = total & 7, xcd = b & 7;
    const int L = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + (b >> 3);
    kslice = L / a.gx;
    bx = L - kslice * a.gx;
  }
  const int M = a.M, K = a.K, KT = a.KT, NG = a.NG;
  const int kt0 = kslice * a.ktc;
  const int kend = min(kt0 + a.ktc, KT);
  const DqK dk = dq_consts();

  // ---- activation rows of the slice -> LDS (issued after the weights) -------
  // Load instruction (p, i) brings rows 4 i .. 4 i + 3 of k-tile kt0 + p into
  // the 1 KiB LDS block p * 8 + i: lane l reads row r = 4 i + l / 16, 16-byte
  // chunk j = (l % 16) ^ (r % 16) of that row's 256 bytes, so each instruction
  // covers whole 128-byte lines and the chunk a lane finds at LDS slot
  // (r % 4) * 16 + (j ^ (r % 16)) of block p * 8 + r / 4 is
  // conflict-free to read back in MFMA operand order (16 consecutive lanes
  // read 16 different rows of one chunk column: 16 distinct bank groups).
  // Only the rows below M are loaded (in groups of four); the operand rows
  // above are never initialised and only reach output rows that are not
  // stored.
  const int rl4 = (min(M, 32) + 3) >> 2;  // row groups loaded per k-tile
  auto load_x = [&]() {
    const uint32_t xbytes = (uint32_t)M * (uint32_t)K * 2u;
    const int r_in = lane >> 4, pos = lane & 15;
    for (int f = wave; f < KTC * rl4; f += 4) {
      const int p = f / rl4, i = f - p * rl4, kt = kt0 + p;
      const int r = 4 * i + r_in, j = pos ^ (r & 15);
      const bool kval = kt < kend;  // wave-uniform
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, kval ? xbytes : 0u);
      // k-chunks past K read as zeros (offset beyond the buffer)
      const uint32_t off = kt * 128 + j * 8 < K ? (uint32_t)min(r, M - 1) * (uint32_t)K * 2u + (uint32_t)j * 16u
                                                 : 0x80000000u;
      load_lds16(rs, &xs[(p * 8 + i) * 64], off, kt * 256);
    }
  };

  // ---- this wave's weights -----------------------------------------------------
  // Group 0 covers tile slots 0, 1 and group 1 slots 2, 3 (with a fused
  // gate/up activation: gate tiles in group 0, their up tiles in group 1).
  // Tiles past the end clamp to the last tile; their outputs are never stored.
  const int NTg = a.NT >> 1;
  const int gb = (bx * WN + wn) * 2;  // first gate tile (fused activation)
  const int nt0 = (bx * WN + wn) * 4;  // first tile (plain)
  const int pb0 = a.act ? gb : nt0;
  const int pb1 = a.act ? gb + NTg : nt0 + 2;
  int pt[4];
  bool pv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pt[j] = (j < 2 ? pb0 : pb1) + (j & 1);
    pv[j] = a.act ? gb + (j & 1) < NTg : pt[j] < a.NT;
  }
  __amdgpu_buffer_rsrc_t wr[2], zr[2], sr[2];
  uint32_t woff[2], zoff[2], soff[2];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int base = min(g == 0 ? pb0 : pb1, a.NT - 1);
    const uint32_t ntiles = (uint32_t)min(2, a.NT - base);
    wr[g] = make_rsrc(a.w + (int64_t)base * KT * 64, ntiles * (uint32_t)KT * 1024u);
    zr[g] = make_rsrc(a.z + (int64_t)base * NG, ntiles * (uint32_t)NG * 8u);
    sr[g] = make_rsrc(a.s + (int64_t)base * NG * 16, ntiles * (uint32_t)NG * 32u);
    const uint32_t dt = (uint32_t)(min(pt[2 * g + t], a.NT - 1) - base);  // this lane's tile in the range
    woff[g] = dt * (uint32_t)KT * 1024u + (uint32_t)(c + 16 * h) * 16u;  // + 512 for the odd-step vector
    zoff[g] = dt * (uint32_t)NG * 8u + (uint32_t)(c >> 3) * 4u;
    soff[g] = (dt * (uint32_t)NG * 16u + (uint32_t)c) * 2u;
  }
  const __amdgpu_buffer_rsrc_t r0 = make_rsrc(a.w, 0u);
  const uint32_t zshift = 4u * (uint32_t)(c & 7);
  const int ktw = kt0 + wk * KPW;  // this wave's first k-tile

  // Issue order: the slice's activation rows (LDS-DMA), the first k-tile's
  // weights, then -- once this wave's DMAs have landed (the loads complete in
  // order: everything but the first k-tile's) and every wave has met -- the
  // other k-tiles' weights, so that each k-tile is multiplied as its weights
  // land instead of after the last of them.
  WStage32<GPT> stg[KPW];
  auto load_w = [&](int p) {
    const int kt = min(ktw + p, KT - 1);
    const bool live = ktw + p < kend;
    const int g0 = (kt * 128) >> a.gshift;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const __amdgpu_buffer_rsrc_t rw = live ? wr[g] : r0, rz = live ? zr[g] : r0, rs = live ? sr[g] : r0;
      stg[p].q[g][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff[g], kt * 1024, 0);
      stg[p].q[g][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, woff[g] + 512u, kt * 1024, 0);
#pragma unroll
      for (int q = 0; q < GPT; ++q)
        stg[p].z[g][q] = __builtin_amdgcn_raw_buffer_load_b32(rz, zoff[g] + 8 * q, g0 * 8, 0);
#pragma unroll
      for (int q = 0; q < GPT; ++q)
        stg[p].s[g][q] = __builtin_amdgcn_raw_buffer_load_b16(rs, soff[g] + 32 * q, g0 * 32, 0);
    }
  };
  constexpr int kLoadsKt = 2 * (2 + 2 * GPT);  // load instructions per k-tile
  load_x();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  load_w(0);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(kLoadsKt));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
#pragma unroll
  for (int p = 1; p < KPW; ++p) load_w(p);

  // ---- multiply ---------------------------------------------------------------
  f32x16 acc[2];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[g][e] = 0.f;

  // MFMA operand of k-step s (lane l: row l % 32, k-chunk 2 s + l / 32) in a
  // k-tile's LDS blocks.
  const int xr = c32, xbase = (xr >> 2) * 64 + (xr & 3) * 16;
  auto xslot = [&](int st) { return xbase + ((2 * st + h) ^ (xr & 15)); };
  // One k-tile: all eight activation operands are read from LDS first (one
  // latency for the k-tile), then 8 k-steps of two MFMAs with step s + 1's
  // dequantisation issued between step s's MFMAs.
  auto compute = [&](const WStage32<GPT>& S, const u32x4* xsb) {
    V8 bv[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) bv[st] = __builtin_bit_cast(V8, xsb[xslot(st)]);
    ZS zs[2][GPT];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int q = 0; q < GPT; ++q) zs[g][q] = Dq<DT>::make((S.z[g][q] >> zshift) & 0xFu, S.s[g][q]);
    V8 av[2][2];
#pragma unroll
    for (int g = 0; g < 2; ++g) av[0][g] = Dq<DT>::word(S.q[g][0][0], zs[g][0], dk);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int cur = st & 1, nxt = cur ^ 1;
      if (st + 1 < 8) {
        const int sn = st + 1;
#pragma unroll
        for (int g = 0; g < 2; ++g) av[nxt][g] = Dq<DT>::word(S.q[g][sn & 1][sn >> 1], zs[g][sn * GPT / 8], dk);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g) acc[g] = mfma32x32x16(av[cur][g], bv[st], acc[g]);
      if (st + 1 < 8) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 13, 0);  // VALU
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
#pragma unroll
  for (int p = 0; p < KPW; ++p)
    if (ktw + p < kend) compute(stg[p], &xs[(wk * KPW + p) * 8 * 64]);  // k-tile block of 8 KiB

  // ---- the WK k-waves of a column range add up through LDS ---------------------
  if constexpr (WK > 1) {
    __syncthreads();  // every wave is done with the activation rows
    f32x4* red = (f32x4*)xs;
    if (wk > 0) {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) red[((((wk - 1) * WN + wn) * 2 + g) * 4 + j) * 64 + lane] = quad_of(acc[g], j);
    }
    __syncthreads();
    if (wk == 0) {
#pragma unroll
      for (int o = 0; o < WK - 1; ++o)
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x4 v = red[(((o * WN + wn) * 2 + g) * 4 + j) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[g][4 * j + r] += v[r];
          }
    }
  }

  // Element e of acc[g] (wave wk == 0): row c32, column 8 (e / 4) + 4 h + e % 4
  // of group g, i.e. tile slot 2 g + e / 8, column 8 ((e / 4) & 1) + 4 h + e % 4
  // of that tile.
  const E* bias = (const E*)a.bias;
  E* out = (E*)a.out;
  const int m = c32;
  if (a.ks == 1) {
    if (wk != 0 || m >= M) return;
    if (a.act == kActNone) {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n0 = pt[2 * g + (j >> 1)] * 16 + 8 * (j & 1) + 4 * h;
          if (n0 < a.N) store4<DT>(out, bias, m, a.N, n0, quad_of(acc[g], j));
        }
    } else {
      const int Nh = a.N >> 1;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (pv[j >> 1])
          store4_act<DT>(out, bias, m, Nh, pt[j >> 1] * 16 + 8 * (j & 1) + 4 * h, Nh, quad_of(acc[0], j),
                         quad_of(acc[1], j), a.act);
    }
    return;
  }

  // ---- split-K handoff ----------------------------------------------------------
  // Partials in output order, [k-slice][row][NT * 16 columns] (fp32).
  const int Np = a.NT * 16;
  const uint32_t slice = (uint32_t)M * (uint32_t)Np * 4u;  // bytes per k-slice
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part, slice * (uint32_t)a.ks);
  if (wk == 0 && m < M) {
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int slot = 2 * g + (j >> 1);
        const int n0 = pt[slot] * 16 + 8 * (j & 1) + 4 * h;  // physical column (up tiles keep theirs)
        if (pv[slot])
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, quad_of(acc[g], j)), pr,
                                                 (uint32_t)kslice * slice + ((uint32_t)m * (uint32_t)Np + (uint32_t)n0) * 4u,
                                                 0, kCacheDevice);
      }
  }
  // The partials are complete before the arrival is counted (a release);
  // the last arrival acquires before any of its waves loads them back.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = arrive_release(&a.counters[bx]);
    s_last = prev == a.ks - 1;
    if (prev == a.ks - 1) acquire_agent();
  }
  __syncthreads();
  if (!s_last) return;

  // Last arrival: output quads of the column group, every slice's partial
  // loaded before the first is added.
  const int ks = a.ks;
  auto sum_slices = [&](uint32_t off) {
    f32x4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (i < ks)
        v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, off + (uint32_t)i * slice, 0,
                                                                               kCacheCoherentLoad));
    f32x4 tot = v[0];
#pragma unroll
    for (int i = 1; i < 16; ++i)
      if (i < ks) tot += v[i];
    return tot;
  };
  if (a.act == kActNone) {
    constexpr int QPR = WN * 16;  // output quads per row of the column group
    const int nbase = bx * WN * 64;
    for (int idx = threadIdx.x; idx < M * QPR; idx += 256) {
      const int mm = idx / QPR, n0 = nbase + 4 * (idx % QPR);
      if (n0 < a.N) store4<DT>(out, bias, mm, a.N, n0, sum_slices(((uint32_t)mm * (uint32_t)Np + (uint32_t)n0) * 4u));
    }
  } else {
    constexpr int QPR = WN * 8;  // gate quads per row of the column group
    const int Nh = a.N >> 1, nbase = bx * WN * 32;
    for (int idx = threadIdx.x; idx < M * QPR; idx += 256) {
      const int mm = idx / QPR, o0 = nbase + 4 * (idx % QPR);
      if (o0 >= Nh) continue;
      const uint32_t off = ((uint32_t)mm * (uint32_t)Np + (uint32_t)o0) * 4u;
      const f32x4 gs = sum_slices(off), us = sum_slices(off + (uint32_t)Nh * 4u);
      store4_act<DT>(out, bias, mm, Nh, o0, Nh, gs, us, a.act);
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(&a.counters[bx], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int WN, int WK, int KPW, typename DT>
hipError_t launch_shape(const KsArgs& a, int gpt, hipStream_t s) {
  const dim3 grid((unsigned)(a.gx * a.ks)), block(256);
  switch (gpt) {
    case 1: hipLaunchKernelGGL((kslice_kernel<WN, WK, KPW, 1, DT>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((kslice_kernel<WN, WK, KPW, 2, DT>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((kslice_kernel<WN, WK, KPW, 4, DT>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename DT>
hipError_t launch_dt(int v, const KsArgs& a, int gpt, hipStream_t s) {
  switch (v) {
    case 411: return launch_shape<4, 1, 1, DT>(a, gpt, s);
    case 412: return launch_shape<4, 1, 2, DT>(a, gpt, s);
    case 413: return launch_shape<4, 1, 3, DT>(a, gpt, s);
    case 414: return launch_shape<4, 1, 4, DT>(a, gpt, s);
    case 221: return launch_shape<2, 2, 1, DT>(a, gpt, s);
    case 222: return launch_shape<2, 2, 2, DT>(a, gpt, s);
    case 223: return launch_shape<2, 2, 3, DT>(a, gpt, s);
    case 224: return launch_shape<2, 2, 4, DT>(a, gpt, s);
    case 141: return launch_shape<1, 4, 1, DT>(a, gpt, s);
    case 142: return launch_shape<1, 4, 2, DT>(a, gpt, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool kslice_variant_ok(int v) {
  switch (v) {
    case 411: case 412: case 413: case 414: case 221: case 222: case 223: case 224: case 141: case 142:
      return true;
    default:
      return false;
  }
}

hipError_t launch_kslice(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                         const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                         hipStream_t s) {
  if (g.M > 32 || p.grid_x * p.ks >= (int64_t(1) << 24)) return hipErrorInvalidConfiguration;
  KsArgs a;
  a.x = x;
  a.w = (const u32x4*)w;
  a.s = (const uint16_t*)sr;
  a.z = (const uint64_t*)zr;
  a.bias = bias;
  a.out = out;
  a.part = (float*)ws;
  a.counters = counters;
  a.M = (int)g.M;
  a.N = (int)g.N;
  a.K = (int)g.K;
  a.NT = (int)g.NT;
  a.KT = (int)g.KT;
  a.NG = (int)g.NG;
  a.gshift = g.gshift;
  a.gx = (int)p.grid_x;
  a.ks = p.ks;
  a.ktc = p.ktc;
  a.act = act;
  const int gpt = (g.NG > 1 && g.G < 128) ? (int)(128 / g.G) : 1;
  return dtype == 0 ? launch_dt<F16>(p.variant, a, gpt, s) : launch_dt<BF16>(p.variant, a, gpt, s);
}

}  // namespace sgl_awq
