// Split-K reduction inside the tiled GEMM kernels ("fix-up").
//
// A split-K plan of the tiled kernels computes each output tile as ks
// k-slices, one workgroup each, that write fp32 partials.  Instead of a second
// kernel that sums them, the ks workgroups of a tile sum them themselves, each
// one a 1/ks portion of the tile (every portion reads all ks slices and adds
// them in slice order, so the result is the same whoever reduces it):
//
//   1. the workgroup writes its partial with device-scope (write-through)
//      stores and waits until they have completed;
//   2. one thread adds 1 to the tile's arrival counter (agent-scope release,
//      arrive_release); arrival ks - 1 of this launch is the last;
//   3. every other workgroup polls the counter until all ks have arrived
//      (bounded), executes an agent-scope acquire (acquire_agent), marks its
//      portion started and reduces it, reading the slices with system-scope
//      loads (kCacheCoherentLoad); one that gives up simply exits;
//   4. the last arrival acquires, reduces its own portion, then every portion
//      that no workgroup has marked started (a portion reduced twice is
//      stored twice with the same values), and advances the tile's base.
//
// So the result never depends on the workgroups being resident at the same
// time -- the last arrival alone can finish every portion -- and a wait ends
// after a fixed number of polls whatever happens.  The host keeps split grids
// within one workgroup per CU, so on an otherwise idle device every wait ends
// as soon as the slowest k-slice arrives.
//
// Counters (one 128-byte slot of 32 words per split tile, in the caller's
// counters buffer ahead of the per-column-tile counters of the decode
// kernels): word 0 counts arrivals over all launches, word 1 is the arrival
// count before the current launch (its base), word 2 + p is base + 1 of the
// last launch in which portion p was started.  Nothing is reset: every launch
// adds ks to words 0 and 1, so a zero-filled buffer, or one left by earlier
// launches of any shape, is always consistent.  (Word 2 + p compares equal to
// a stale value only after 2^32 / ks launches on the tile, and only matters if
// a workgroup gives up in that launch.)
//
// No counterpart in the reference: its Triton path sums the split-K slices
// with a separate torch reduction (awq_triton.py:173, :193).
#pragma once

#include "awq_buffer.h"
#include "awq_epilogue.h"

namespace sgl_awq {

constexpr int kFixupWords = 32;        // counter words per split tile (one 128-byte slot)
constexpr int kFixupMaxTiles = 512;    // split tiles a counters buffer covers
constexpr int64_t kFixupBytes = int64_t(kFixupMaxTiles) * kFixupWords * 4;  // 64 KiB, at the buffer's start
constexpr int kFixupMaxSlices = 16;    // k-slices a fix-up sums (one started word each)
constexpr int kFixupDefaultPolls = 512;

// Counter words are read and written at system scope (SC0 | SC1: past every
// cache of the reading CU and XCD; see kCacheCoherentLoad).
__device__ __forceinline__ uint32_t ld_sys_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// What a workgroup needs to reduce one portion of its output tile.
template <typename DT>
struct FixupTile {
  const float* part;  // partials [ks][M][Np]
  typename DT::elem* out;
  const typename DT::elem* bias;
  int M, N, Np, ks, act;
  int m0, rows;  // the tile's first output row and its row count
  int col0;      // first output column (a fused activation: first gate column)
  int qpr;       // output quads (4 columns) per tile row

  // Portion p of the tile's rows * qpr quads: the ks slices of each quad are
  // read with system-scope loads (kCacheCoherentLoad), up to eight issued
  // before the first is added, and summed in slice order.
  template <int NTHREADS>
  __device__ void reduce(int p) const {
    const int Q = rows * qpr;
    const int lo = (int)((int64_t)Q * p / ks), hi = (int)((int64_t)Q * (p + 1) / ks);
    const uint32_t slice = (uint32_t)M * (uint32_t)Np * 4u;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(part, slice * (uint32_t)ks);
    const int No = act == kActNone ? N : N / 2;
    // Up to eight slices' loads in flight at a time (32 registers: the
    // callers' register budgets are tight), added in slice order.
    auto sum4 = [&](uint32_t off) {
      f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < ks; s0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (s0 + i < ks)
            v[i] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, (int)((uint32_t)(s0 + i) * slice),
                                                       kCacheCoherentLoad));
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (s0 + i < ks) tot = s0 + i == 0 ? v[i] : tot + v[i];
      }
      return tot;
    };
    for (int idx = lo + (int)threadIdx.x; idx < hi; idx += NTHREADS) {
      const int m = idx / qpr;
      const int n0 = col0 + 4 * (idx - m * qpr);
      if (n0 >= No) continue;
      const int64_t row = (int64_t)m0 + m;
      const uint32_t off = ((uint32_t)row * (uint32_t)Np + (uint32_t)n0) * 4u;
      if (act == kActNone) {
        store4<DT>(out, bias, row, N, n0, sum4(off));
      } else {
        const f32x4 g = sum4(off);
        __builtin_amdgcn_sched_barrier(0);
        const f32x4 u = sum4(off + (uint32_t)(N / 2) * 4u);
        store4_act<DT>(out, bias, row, No, n0, No, g, u, act);
      }
    }
  }
};

// Steps 1-4 for the calling workgroup (every thread calls it).  `tc` is the
// tile's counter slot; `base` is word 1 as thread 0 loaded it before this
// workgroup's partial stores (any time before its own arrival is safe: the
// base only moves after the last arrival).
template <int NTHREADS, typename DT>
__device__ __forceinline__ void splitk_fixup(const FixupTile<DT>& ft, uint32_t* tc, uint32_t base, int kslice,
                                             int polls) {
  __shared__ uint32_t s_fx[4];
  // The partial stores (and thread 0's base load) have completed.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  const uint32_t ks = (uint32_t)ft.ks;
  if (threadIdx.x == 0) {
    asm volatile("" ::"v"(base) : "memory");  // the base load has returned before this arrival
    const uint32_t prev = arrive_release(tc);
    const bool last = prev - base == ks - 1u;
    bool ready = last;
    for (int i = 0; !ready && i < polls; ++i) {
      __builtin_amdgcn_s_sleep(2);
      ready = ld_sys_u32(tc) - base >= ks;
    }
    if (ready) acquire_agent();  // the other slices' partials, before any wave loads them
    if (ready && !last) st_sys_u32(tc + 2 + kslice, base + 1u);
    s_fx[0] = last;
    s_fx[1] = ready;
    s_fx[3] = base;  // (only thread 0 loaded it)
  }
  __syncthreads();
  const bool last = s_fx[0] != 0;
  base = s_fx[3];
  if (s_fx[1] == 0) return;  // the last arrival reduces this portion
  ft.template reduce<NTHREADS>(kslice);
  if (!last) return;
  // Portions no other workgroup has started.
  if (threadIdx.x < 64) {
    const int p = (int)threadIdx.x;
    const bool todo = p < ft.ks && p != kslice && ld_sys_u32(tc + 2 + p) != base + 1u;
    const uint64_t mask = __ballot(todo);
    if (threadIdx.x == 0) {
      s_fx[2] = (uint32_t)mask;
      st_sys_u32(tc + 1, base + ks);  // the next launch's base
    }
  }
  __syncthreads();
  for (uint32_t todo = s_fx[2]; todo != 0u; todo &= todo - 1u) ft.template reduce<NTHREADS>(__builtin_ctz(todo));
}

}  // namespace sgl_awq
