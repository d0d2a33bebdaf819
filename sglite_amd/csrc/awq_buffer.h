// Buffer-resource helpers and the 32x32x16 MFMA, shared by the MFMA GEMM
// kernels (awq_tiled.hip, awq_kslice.hip).
#pragma once

#include "awq_device.h"

namespace sgl_awq {

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, dword data format (gfx9)
// Buffer cache policy SC1 (device scope): the bits the compiler gives an
// agent-scope atomic store; a store with it is written through to memory
// and has reached it once the store has completed (vmcnt).
constexpr int kCacheDevice = 16;
// Buffer cache policy SC0 | SC1 | NT for loads of data that other
// workgroups (possibly on other XCDs) wrote in the same launch: the
// system-scope bits, which miss in every cache level of the reading CU and
// XCD, plus the streaming hint.  Loads with SC1 alone were measured to return
// a stale copy in that situation on MI355X (an in-kernel split-K sum read
// the previous launch's partials); SC0 | SC1 did not.
constexpr int kCacheCoherentLoad = 19;
// Buffer cache policy NT (non-temporal): a stream read once.
constexpr int kCacheStream = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// One 16-byte buffer load per lane straight into LDS: lane l's bytes land at
// dst + 16 * l (dst is wave-uniform).
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, u32x4* dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}

// s_waitcnt immediate that waits until at most n vector-memory loads are
// outstanding and leaves the other counters alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

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
