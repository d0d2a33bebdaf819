// Buffer-resource helpers and the 32x32x16 MFMA, shared by the MFMA GEMM
// kernels (awq_tiled.hip, awq_kslice.hip).
#pragma once

#include "awq_device.h"

namespace sgl_awq {

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, dword data format (gfx9)
// Buffer cache policy SC1 (device scope): the bits the compiler gives an
// agent-scope atomic store; the store is written through the L2, so the
// release writeback below finds little to do.
constexpr int kCacheDevice = 16;
// Buffer cache policy SC0 | SC1 | NT for loads of data that other
// workgroups (possibly on other XCDs) wrote in the same launch: the
// system-scope bits plus the streaming hint, so the partials do not displace
// reused lines.  Cache bits alone do not order such a load after the arrival
// counter: with only them (no release/acquire pair) one in-kernel split-K sum
// on MI355X read a stale partial, once in several hundred launches.
constexpr int kCacheCoherentLoad = 19;
// Buffer cache policy NT (non-temporal): a stream read once.
constexpr int kCacheStream = 2;

// s_waitcnt immediate that waits until at most n vector-memory loads are
// outstanding and leaves the other counters alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
// The same with no LDS operation outstanding either (lgkmcnt 0).
constexpr int vmcnt_lgkm0_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4); }

// Handoff of plain stores between the workgroups of one launch (possibly on
// different XCDs, whose L2s are made coherent only by explicit writeback and
// invalidate).  The cache bits above keep the data's own path short, but the
// order between the data and the arrival counter comes from the memory model:
//   writer: every wave waits for its stores (vmcnt 0), a barrier, then one
//           thread executes an agent-scope release fence (buffer_wbl2 sc1:
//           the L2 writeback), waits for it, and counts the arrival with a
//           relaxed atomic -- together a release of the count;
//   reader: the workgroup that saw the count complete executes an agent-scope
//           acquire (buffer_inv sc1: L1 and L2 lines the writers' data could
//           be stale in), waits for it, and only then releases its other
//           waves through a barrier to load.
// The explicit waits matter: the compiler drops the wait of its own release
// sequence after buffer_wbl2 when no other memory operation is outstanding.
template <typename T>
__device__ __forceinline__ T arrive_release(T* counter) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  return __hip_atomic_fetch_add(counter, T(1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void acquire_agent() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// One 16-byte buffer load per lane straight into LDS: lane l's bytes land at
// dst + 16 * l (dst is wave-uniform).
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, u32x4* dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Weights of one k-tile for a wave's two groups of 32 columns in the 32x32x16
// operand order: per 16-row k-step s the A operand of lane l is one packed
// word -- column l % 32 of the group, rows 16 s + 8 (l / 32) .. + 7 -- which
// the tile layout holds in word s / 2 of the 16-byte vector of lane
// (l % 16) + 16 (l / 32) (even s) or that lane + 32 (odd s) of tile
// (l % 32) / 16 of the group.
template <int GPT>
struct WStage32 {
  u32x4 q[2][2];       // [column group][even / odd k-step vector]
  uint32_t z[2][GPT];  // the zero-point word holding this lane's nibble, per quantisation group
  uint16_t s[2][GPT];  // this lane's column scale, per quantisation group
};

}  // namespace sgl_awq
