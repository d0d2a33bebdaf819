// Gated MLP block in one launch for decode batches (gfx950):
//   out[M, H] = down( act(x @ W_gate) * (x @ W_up) ),
// the GatedMLP forward (python/sglite/srt/model_executor/models/blocks.py:51-57:
// gate_up_proj, act_fn = silu_and_mul / gelu_and_mul, down_proj) for
// M <= 16 rows, group size 128, no bias.
//
// A decode-size linear spends a few microseconds per launch before its first
// weight bytes arrive and after its last output is stored; the block's two
// projections in two launches pay that twice, and the down projection's
// weights only start streaming once the gate/up output exists.  Here one
// workgroup per CU (a grid no larger than what the device keeps resident,
// from its occupancy query) runs both.  The down projection is split into
// column groups g (C tiles of 16 columns) and k-slices s (at most 8 k-tiles
// of the intermediate); workgroup b = g S + s owns one (g, s) pair:
//
//   loads    it issues, in this order: its activation rows, its first gate/up
//            column pair, the down projection's zero points, scales and
//            weights of (g, s), its second gate/up pair; then one pair ahead
//            of each pair it computes -- so the down weights stream from HBM
//            under the gate/up GEMM;
//   phase A  the gate/up GEMM with the activation, for gate tiles of k-slice
//            s only: the 8 nk(s) gate tiles (16 columns each) whose columns
//            are the intermediate's k-slice s are shared out over the slice's
//            column groups (tile 8 kb0(s) + g + groups j for j = 0, 1, ...),
//            each with its up tile I / 16 tiles further; its 8 waves split the
//            k-tiles, their sums are added through LDS, each gate / up value
//            is rounded as the unfused GEMM stores it, act(gate) * up is
//            rounded once and written through to the intermediate h [M, I];
//   slice    it adds one to slice s's arrival counter and polls it until all
//            the slice's workgroups have arrived -- at most `polls` times: a
//            workgroup that gives up adds one to an error word and skips
//            phase B.  So a workgroup waits only for the few others that
//            write its slice of h, and no counter is shared by the whole grid;
//   phase B  the down GEMM of (g, s): it stages k-slice s of h in LDS
//            (system-scope loads), multiplies with the weights already in
//            registers (waves w and w + 8 one tile each), writes an fp32
//            partial through and adds one to column group g's counter; the
//            group's last arrival sums the S partials in slice order
//            (deterministic) and stores the output.  Nobody waits here.
//
// Counters (the caller's, zero before the first call, never reset; 128-byte
// slots of 32 words): word 2 of slot 0 counts workgroups that gave up waiting
// (an error the host turns into an exception); slot 1 + s is k-slice s's
// barrier, slot 1 + S + g column group g's.  Word 0 of a slot counts arrivals
// over all launches, word 1 is the count before the current launch (its
// base).  Every workgroup arrives at its slice's and its group's slot exactly
// once per launch, also after giving up, and the arrival that completes a
// slot advances its base, so the counters stay consistent from launch to
// launch, whatever the shape, and after an error.  Launches that share
// counters must be stream-ordered.
//
// Weights are dequantised to (q - z) * s with the oracle's rounding
// (Dq<DT>::word) and multiplied by 16x16x32 MFMAs with fp32 accumulation.
//
// No counterpart in the reference: a fusion of its GatedMLP calls.
#include <algorithm>

#include "awq_buffer.h"
#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_fixup.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

constexpr int kMlpWaves = 8;
constexpr int kMlpThreads = 64 * kMlpWaves;

struct MlpArgs {
  const void* x;          // [M][H]
  const void* gw;         // gate_up weights: tiles [2 NTg][KTA] (gate tiles, then up tiles)
  const void* gs;         // scales [2 NTg][KTA][16]
  const void* gz;         // zeros [2 NTg][KTA] u64
  const void* dw;         // down weights: tiles [NTD][KTD]
  const void* ds;
  const void* dz;
  void* h;                // intermediate [M][I]
  float* part;            // down partials [S][M][H]
  void* out;              // [M][H]
  uint32_t* cnt;          // counter slots
  int M, H, I;
  int KTA, NTg, KTD, NTD;  // gate_up k-tiles / gate tiles; down k-tiles / column tiles
  int P, S, C, Gc;         // grid; down k-slices; down tiles per column group; column groups
  int act, polls;
};

// Thread 0 arrives at a barrier slot (an agent-scope release of this
// workgroup's stores) and polls it until `n` arrivals since `base` (at most
// `polls` polls), then acquires; every thread gets the outcome.  The arrival
// that completes the count advances the base for the next launch.  A
// workgroup that gives up adds one to the error word.
__device__ __forceinline__ bool mlp_barrier(uint32_t* slot, uint32_t base, uint32_t n, int polls, uint32_t* err,
                                            uint32_t* s_ok) {
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this workgroup's intermediate stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    asm volatile("" ::"v"(base) : "memory");  // the base was read before this arrival
    const uint32_t prev = arrive_release(slot);
    bool ready = prev - base == n - 1u;
    if (ready) st_sys_u32(slot + 1, base + n);
    for (int i = 0; !ready && i < polls; ++i) {
      __builtin_amdgcn_s_sleep(1);
      ready = ld_sys_u32(slot) - base >= n;
    }
    if (ready)
      acquire_agent();  // the others' stores, before any wave loads them
    else
      __hip_atomic_fetch_add(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_ok = ready;
  }
  __syncthreads();
  return *s_ok != 0;
}

// Zero points and scales travel as one word per (tile, k-tile): the zero
// nibble of the lane's column << 16 | the scale bits.  A wave loads them for
// four k-tiles at once -- lane (c, i) the column-c entry of k-tile i -- and
// ds_bpermute hands k-tile i's entry to every lane that needs it.
__device__ __forceinline__ uint32_t zs_pack(uint32_t zword, uint32_t sbits, uint32_t zshift) {
  return ((zword >> zshift) & 0xFu) << 16 | (sbits & 0xFFFFu);
}
__device__ __forceinline__ uint32_t zs_take(uint32_t packed, int c, int i) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute((c + 16 * i) << 2, (int)packed);
}

// One gate/up column pair for one wave: the weights of k-tiles wave + 8 i
// (i < KA <= 4), and in lane (c, i) the zero word and scale of k-tile
// wave + 8 i for column c.
template <int KA>
struct PairStage {
  u32x4 qg[KA], qu[KA];
  uint32_t zg, zu, sg, su;
};

// NPW: gate tiles per workgroup, KA: gate_up k-tiles per wave (<= 4), XPT:
// activation chunks of 8 elements per thread (M H <= 4096 XPT), KB: down
// k-tiles per slice (<= 8; all maxima; two down tiles per wave).
template <typename DT, int NPW, int KA, int XPT, int KB>
__global__ __launch_bounds__(kMlpThreads, 1) void mlp_kernel(MlpArgs a) {
  static_assert(KA <= 4 && KB <= 8, "zero points and scales are handed out four k-tiles per load");
  using E = typename DT::elem;
  using V8 = typename DT::vec8;
  using ZS = typename Dq<DT>::ZS;
  constexpr int TB = 2;
  constexpr int RB = NPW < 3 ? NPW : 3;  // gate/up pairs in flight
  extern __shared__ u32x4 smem[];
  __shared__ uint32_t s_flag;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, lg = lane >> 4;
  const int b = blockIdx.x;
  const int M = a.M, H = a.H, I = a.I;
  const int KTA = a.KTA, KTD = a.KTD;
  const DqK dk = dq_consts();
  const uint32_t zshift = 4u * (uint32_t)(c & 7);
  const uint32_t zsel = (uint32_t)(c >> 3) * 4u;

  const int cg = b / a.S, slice = b - cg * a.S;
  const int kb0 = slice * KTD / a.S, kb1 = (slice + 1) * KTD / a.S, nk = kb1 - kb0;  // this k-slice of h
  uint32_t* slots = a.cnt + (1 + slice) * kFixupWords;
  uint32_t* slotg = a.cnt + (1 + a.S + cg) * kFixupWords;
  uint32_t bases = 0, baseg = 0;
  if (threadIdx.x == 0) {
    bases = ld_sys_u32(slots + 1);
    baseg = ld_sys_u32(slotg + 1);
  }

  // Every load below is a buffer load issued unconditionally: a tile or
  // chunk outside the workgroup's share gets an offset past the buffer's
  // range (kOob), which returns zero without a memory access.  So the number
  // of loads in flight is fixed and each wait covers exactly the loads it
  // needs (a load under a branch makes the compiler wait for all of them).
  constexpr uint32_t kOob = 0x7FFFFFF0u;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)M * (uint32_t)H * 2u);
  const uint32_t ta = 2u * (uint32_t)a.NTg * (uint32_t)KTA, td = (uint32_t)a.NTD * (uint32_t)KTD;
  const __amdgpu_buffer_rsrc_t rgw = make_rsrc(a.gw, ta * 1024u), rgz = make_rsrc(a.gz, ta * 8u),
                               rgs = make_rsrc(a.gs, ta * 32u);
  const __amdgpu_buffer_rsrc_t rdw = make_rsrc(a.dw, td * 1024u), rdz = make_rsrc(a.dz, td * 8u),
                               rds = make_rsrc(a.ds, td * 32u);

  // ---- activation rows: chunk q (8 elements) = row q / (H / 8), columns 8 (q % (H / 8))
  const int cpr = H >> 3, nchunk = M * cpr;
  const int xs_stride = H + 8;  // LDS row stride (elements)
  u32x4 xr[XPT];
#pragma unroll
  for (int r = 0; r < XPT; ++r) {
    const int q = (int)threadIdx.x + r * kMlpThreads;
    const uint32_t off = q < nchunk ? ((uint32_t)(q / cpr) * (uint32_t)H + (uint32_t)(q % cpr) * 8u) * 2u : kOob;
    xr[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
  }

  // ---- gate/up pair j: gate tile 8 kb0 + cg + Gc j (while inside the slice), up tile NTg further
  auto load_pair = [&](PairStage<KA>& st, int j) {
    const int tg = kb0 * 8 + cg + a.Gc * j;
    const bool tv = tg < kb1 * 8;
    const uint32_t up = (uint32_t)a.NTg * (uint32_t)KTA;
#pragma unroll
    for (int i = 0; i < KA; ++i) {
      const int kt = wave + kMlpWaves * i;
      const bool v = tv && kt < KTA;
      const uint32_t ug = (uint32_t)tg * (uint32_t)KTA + (uint32_t)kt;
      st.qg[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rgw, v ? (ug * 64u + lane) * 16u : kOob, 0, kCacheStream));
      st.qu[i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rgw, v ? ((ug + up) * 64u + lane) * 16u : kOob, 0,
                                                       kCacheStream));
    }
    const int ktz = wave + kMlpWaves * lg;  // lane group lg: k-tile wave + 8 lg
    const bool vz = tv && lg < KA && ktz < KTA;
    const uint32_t uz = (uint32_t)tg * (uint32_t)KTA + (uint32_t)ktz;
    st.zg = __builtin_amdgcn_raw_buffer_load_b32(rgz, vz ? uz * 8u + zsel : kOob, 0, 0);
    st.zu = __builtin_amdgcn_raw_buffer_load_b32(rgz, vz ? (uz + up) * 8u + zsel : kOob, 0, 0);
    st.sg = __builtin_amdgcn_raw_buffer_load_b16(rgs, vz ? (uz * 16u + c) * 2u : kOob, 0, 0);
    st.su = __builtin_amdgcn_raw_buffer_load_b16(rgs, vz ? ((uz + up) * 16u + c) * 2u : kOob, 0, 0);
  };
  PairStage<KA> st[RB];
#pragma unroll
  for (int j = 0; j < RB; ++j) load_pair(st[j], j);

  // ---- the activation rows to LDS
  _Float16* xs = (_Float16*)smem;
  auto publish_x = [&]() {
#pragma unroll
    for (int r = 0; r < XPT; ++r) {
      const int q = (int)threadIdx.x + r * kMlpThreads;
      if (q < nchunk) *(u32x4*)(xs + (q / cpr) * xs_stride + (q % cpr) * 8) = xr[r];
    }
  };
  // Many activation chunks per thread: publish them before the down loads
  // are issued (they would not fit in registers beside them).
  if constexpr (XPT > 4) publish_x();

  // ---- down projection of (cg, slice): tiles dt[t] = cg C + wave + 8 t, k-tiles kb0 .. kb1 - 1;
  //      lane (c, i) holds the zero word and scale of k-tiles kb0 + i (lo) and kb0 + 4 + i (hi)
  int dt[TB];
  bool dv[TB];
  u32x4 qd[TB][KB];
  uint32_t zdl[TB], zdh[TB], sdl[TB], sdh[TB];
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    const int cl = wave + kMlpWaves * t;
    dt[t] = cg * a.C + cl;
    dv[t] = cl < a.C && dt[t] < a.NTD;
    const uint32_t u0 = (uint32_t)dt[t] * (uint32_t)KTD + (uint32_t)kb0;
    const bool vl = dv[t] && lg < nk, vh = dv[t] && lg + 4 < nk;
    zdl[t] = __builtin_amdgcn_raw_buffer_load_b32(rdz, vl ? (u0 + lg) * 8u + zsel : kOob, 0, 0);
    zdh[t] = __builtin_amdgcn_raw_buffer_load_b32(rdz, vh ? (u0 + lg + 4) * 8u + zsel : kOob, 0, 0);
    sdl[t] = __builtin_amdgcn_raw_buffer_load_b16(rds, vl ? ((u0 + lg) * 16u + c) * 2u : kOob, 0, 0);
    sdh[t] = __builtin_amdgcn_raw_buffer_load_b16(rds, vh ? ((u0 + lg + 4) * 16u + c) * 2u : kOob, 0, 0);
#pragma unroll
    for (int i = 0; i < KB; ++i)
      qd[t][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rdw, dv[t] && i < nk ? ((u0 + i) * 64u + lane) * 16u : kOob,
                                                       0, kCacheStream));
  }
  if constexpr (XPT <= 4) publish_x();
  __syncthreads();

  // ---- phase A
  const int xrow = min(c, M - 1) * xs_stride + lg * 8;
  f32x4 accg[NPW], accu[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    PairStage<KA>& cur = st[j % RB];
    accg[j] = accu[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (kb0 * 8 + cg + a.Gc * j < kb1 * 8) {
      const uint32_t pg = zs_pack(cur.zg, cur.sg, zshift), pu = zs_pack(cur.zu, cur.su, zshift);
#pragma unroll
      for (int i = 0; i < KA; ++i) {
        const int kt = wave + kMlpWaves * i;
        if (kt < KTA) {
          const uint32_t eg = zs_take(pg, c, i), eu = zs_take(pu, c, i);
          const ZS zsg = Dq<DT>::make(eg >> 16, (uint16_t)eg);
          const ZS zsu = Dq<DT>::make(eu >> 16, (uint16_t)eu);
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const V8 bx = __builtin_bit_cast(V8, *(const u32x4*)(xs + xrow + kt * 128 + 32 * w));
            accg[j] = mfma16x16x32(Dq<DT>::word(cur.qg[i][w], zsg, dk), bx, accg[j]);
            accu[j] = mfma16x16x32(Dq<DT>::word(cur.qu[i][w], zsu, dk), bx, accu[j]);
          }
        }
      }
    }
    if (j + RB < NPW) load_pair(cur, j + RB);
  }
  // The waves' sums through LDS (over the activation rows, now read).
  __syncthreads();
  f32x4* red = (f32x4*)smem;  // [wave][pair][gate, up][lane]
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    red[((wave * NPW + j) * 2 + 0) * 64 + lane] = accg[j];
    red[((wave * NPW + j) * 2 + 1) * 64 + lane] = accu[j];
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.h, (uint32_t)M * (uint32_t)I * 2u);
  if (wave < NPW) {
    // wave j: pair j; lane l: row l % 16, columns 4 (l / 16) .. + 3 of the pair's tile
    const int j = wave, tg = kb0 * 8 + cg + a.Gc * j, m = c;
    if (tg < kb1 * 8 && m < M) {
      f32x4 g = red[(j * 2 + 0) * 64 + lane], u = red[(j * 2 + 1) * 64 + lane];
#pragma unroll
      for (int o = 1; o < kMlpWaves; ++o) {
        g += red[((o * NPW + j) * 2 + 0) * 64 + lane];
        u += red[((o * NPW + j) * 2 + 1) * 64 + lane];
      }
      // as the unfused gate/up GEMM stores each, then act(gate) * up rounded once
      typename DT::vec4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = (E)(gated_act(a.act, (float)(E)g[e]) * (float)(E)u[e]);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, r), hr,
                                            ((uint32_t)m * (uint32_t)I + (uint32_t)(tg * 16 + 4 * lg)) * 2u, 0,
                                            kCacheDevice);
    }
  }

  // ---- every gate/up output of this k-slice is stored
  const bool ok = mlp_barrier(slots, bases, (uint32_t)a.Gc, a.polls, a.cnt + 2, &s_flag);

  const uint32_t slice_bytes = (uint32_t)M * (uint32_t)H * 4u;
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part, slice_bytes * (uint32_t)a.S);
  if (ok) {
    // ---- phase B: this k-slice of h -> LDS
    const int hs_stride = nk * 128 + 8;
    _Float16* hs = (_Float16*)smem;
    const int hcpr = nk * 16;  // 8-element chunks per row of the slice
    for (int q = threadIdx.x; q < M * hcpr; q += kMlpThreads) {
      const int m = q / hcpr, kk = (q - m * hcpr) * 8;
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(hr, ((uint32_t)m * (uint32_t)I + (uint32_t)(kb0 * 128 + kk)) * 2u,
                                                       0, kCacheCoherentLoad));
      *(u32x4*)(hs + m * hs_stride + kk) = v;
    }
    __syncthreads();
    const int hrow = min(c, M - 1) * hs_stride + lg * 8;
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      if (dv[t]) {
        const uint32_t pl = zs_pack(zdl[t], sdl[t], zshift), ph = zs_pack(zdh[t], sdh[t], zshift);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KB; ++i) {
          if (i < nk) {
            const uint32_t e = zs_take(i < 4 ? pl : ph, c, i & 3);
            const ZS zs = Dq<DT>::make(e >> 16, (uint16_t)e);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const V8 bx = __builtin_bit_cast(V8, *(const u32x4*)(hs + hrow + i * 128 + 32 * w));
              acc = mfma16x16x32(Dq<DT>::word(qd[t][i][w], zs, dk), bx, acc);
            }
          }
        }
        if (c < M)
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, acc), pr,
              (uint32_t)slice * slice_bytes + ((uint32_t)c * (uint32_t)H + (uint32_t)(dt[t] * 16 + 4 * lg)) * 4u, 0,
              kCacheDevice);
      }
    }
  }

  // ---- arrive at the column group; its last arrival sums the slices
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  if (threadIdx.x == 0) {
    asm volatile("" ::"v"(baseg) : "memory");
    const uint32_t prev = arrive_release(slotg);
    const bool last = prev - baseg == (uint32_t)a.S - 1u;
    if (last) {
      st_sys_u32(slotg + 1, baseg + (uint32_t)a.S);
      acquire_agent();
    }
    s_flag = last && ok;
  }
  __syncthreads();
  if (!s_flag) return;
  const int n0 = cg * a.C * 16, ncols = min(a.C * 16, H - n0), q4 = ncols >> 2;
  for (int q = threadIdx.x; q < M * q4; q += kMlpThreads) {
    const int m = q / q4, n = n0 + 4 * (q - m * q4);
    const uint32_t off = ((uint32_t)m * (uint32_t)H + (uint32_t)n) * 4u;
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < a.S; s0 += 8) {
      f32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (s0 + i < a.S)
          v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               pr, off, (int)((uint32_t)(s0 + i) * slice_bytes), kCacheCoherentLoad));
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (s0 + i < a.S) tot = s0 + i == 0 ? v[i] : tot + v[i];
    }
    store4<DT>((E*)a.out, nullptr, m, H, n, tot);
  }
}

// Built forms: NPW gate tiles per workgroup and KA gate_up k-tiles per wave
// (2, 3 or 4 each, equal), XPT activation chunks per thread (1, 4 or 16),
// KB = 8 down k-tiles per slice; a plan takes the smallest that covers it.
constexpr int kMlpPairForms[] = {2, 3, 4};
constexpr int kMlpXptForms[] = {1, 4, 16};
constexpr int kMlpKb = 8;

#define SGL_MLP_FORMS(X) \
  X(0, 2, 1) X(1, 2, 4) X(2, 2, 16) X(3, 3, 1) X(4, 3, 4) X(5, 3, 16) X(6, 4, 1) X(7, 4, 4) X(8, 4, 16)

template <typename DT>
const void* mlp_kernel_ptr(int form) {
  switch (form) {
#define SGL_MLP_PTR(f, n, x) \
  case f: return (const void*)mlp_kernel<DT, n, n, x, kMlpKb>;
    SGL_MLP_FORMS(SGL_MLP_PTR)
#undef SGL_MLP_PTR
  }
  return nullptr;
}

template <typename DT>
hipError_t launch_form(int form, const MlpArgs& a, size_t lds, hipStream_t s) {
  const dim3 grid((unsigned)a.P), block(kMlpThreads);
  switch (form) {
#define SGL_MLP_LAUNCH(f, n, x) \
  case f: hipLaunchKernelGGL((mlp_kernel<DT, n, n, x, kMlpKb>), grid, block, lds, s, a); break;
    SGL_MLP_FORMS(SGL_MLP_LAUNCH)
#undef SGL_MLP_LAUNCH
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

constexpr int64_t kMlpMaxLds = 156 << 10;  // and the flag word beside it, within the 160 KiB of a CU

}  // namespace

MlpPlan plan_mlp(int64_t M, int64_t H, int64_t I, int64_t G, int dtype, bool query_device) {
  MlpPlan p{};
  if (M < 1 || M > 16 || G != 128 || H % 128 != 0 || I % 128 != 0 || M * H > 16 * 4096 ||
      (dtype != 0 && dtype != 1))
    return p;
  const int64_t cus = device_cu_count();
  const int64_t KTA = H / 128, KTD = I / 128, NTD = H / 16;
  const int64_t ka = (KTA + kMlpWaves - 1) / kMlpWaves, chunks = (M * H / 8 + kMlpThreads - 1) / kMlpThreads;
  int xf = -1;
  for (int f = 0; f < 3 && xf < 0; ++f)
    if (kMlpXptForms[f] >= chunks) xf = f;
  if (xf < 0) return p;
  int64_t best = -1;
  for (int64_t C = 8; C <= 16; ++C) {  // waves w and w + 8 take one tile each
    const int64_t Gc = (NTD + C - 1) / C;
    int64_t S = std::min<int64_t>(cus / Gc, KTD);
    if (S < 1) continue;
    const int64_t nk = (KTD + S - 1) / S;
    if (nk > kMlpKb) continue;
    S = (KTD + nk - 1) / nk;  // no empty slice
    if (1 + S + Gc > kMlpCounterBytes / 128) continue;
    // a k-slice's 8 nk gate tiles are shared out over its Gc workgroups
    const int64_t P = Gc * S, npw = (8 * nk + Gc - 1) / Gc;
    int pf = -1;
    for (int f = 0; f < 3 && pf < 0; ++f)
      if (kMlpPairForms[f] >= npw && kMlpPairForms[f] >= ka) pf = f;
    if (pf < 0) continue;
    // LDS: the activation rows, then the waves' gate/up sums, then the intermediate slice
    const int64_t lds = std::max({M * (H + 8) * 2, (int64_t)kMlpWaves * kMlpPairForms[pf] * 2 * 64 * 16,
                                  M * (nk * 128 + 8) * 2});
    if (lds > kMlpMaxLds) continue;
    // KiB of weights the busiest workgroup streams; at equal cost the larger grid
    const int64_t cost = npw * 2 * KTA + C * nk;
    if (best >= 0 && (cost > best || (cost == best && P <= p.P))) continue;
    best = cost;
    p.ok = 1;
    p.form = pf * 3 + xf;
    p.P = P;
    p.S = S;
    p.C = C;
    p.groups = Gc;
    p.npw = npw;
    p.nk = nk;
    p.lds = lds;
    p.h_bytes = (M * I * 2 + 255) / 256 * 256;
    p.ws_bytes = p.h_bytes + S * M * H * 4;
  }
  if (!p.ok || !query_device) return p;
  // never more workgroups than the device keeps resident at once
  int per_cu = 0;
  const void* fn = dtype == 0 ? mlp_kernel_ptr<F16>(p.form) : mlp_kernel_ptr<BF16>(p.form);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kMlpThreads, (size_t)p.lds) != hipSuccess ||
      per_cu < 1 || p.P > (int64_t)per_cu * cus) {
    (void)hipGetLastError();
    p.ok = 0;
  }
  return p;
}

hipError_t launch_mlp(const MlpPlan& p, const void* x, const void* gw, const void* gs, const void* gz, const void* dw,
                      const void* ds, const void* dz, void* out, int64_t M, int64_t H, int64_t I, int dtype, int act,
                      void* ws, int32_t* counters, int polls, hipStream_t s) {
  MlpArgs a;
  a.x = x;
  a.gw = gw;
  a.gs = gs;
  a.gz = gz;
  a.dw = dw;
  a.ds = ds;
  a.dz = dz;
  a.h = ws;
  a.part = (float*)((char*)ws + p.h_bytes);
  a.out = out;
  a.cnt = (uint32_t*)counters;
  a.M = (int)M;
  a.H = (int)H;
  a.I = (int)I;
  a.KTA = (int)(H / 128);
  a.NTg = (int)(I / 16);
  a.KTD = (int)(I / 128);
  a.NTD = (int)(H / 16);
  a.P = (int)p.P;
  a.S = (int)p.S;
  a.C = (int)p.C;
  a.Gc = (int)p.groups;
  a.act = act;
  a.polls = polls;
  return dtype == 0 ? launch_form<F16>(p.form, a, (size_t)p.lds, s) : launch_form<BF16>(p.form, a, (size_t)p.lds, s);
}

}  // namespace sgl_awq
