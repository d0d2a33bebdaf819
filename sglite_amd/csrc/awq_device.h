// Device helpers shared by the AWQ W4A16 kernels (gfx950 / CDNA4, wave64).
//
// Repacked tile layout (the "CDNA4 tile layout"):
//   weights: 1 KiB tiles of 16 columns x 128 rows; tile (nt, kt) at
//            (nt * KT + kt) KiB.  Lane l of a tile owns one 16-byte vector
//            (4 uint32 words); word w holds column 16*nt + (l & 15) and rows
//            k0..k0+7, k0 = 128*kt + 32*w + 8*(l >> 4); nibble p holds row
//            k0 + {0,2,4,6,1,3,5,7}[p].
//   So one 16-byte load per lane is exactly the MFMA 16x16x32 operand of four
//   consecutive 32-row k-blocks for that lane's column, and the nibble order
//   lets (word >> 4i) & 0x000F000F produce the packed pair (row 2i, row 2i+1).
//   scales:  [NT][NG][16] in the activation dtype.
//   zeros:   [NT][NG] uint64, nibble c = zero point of column 16*nt + c.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sgl_awq {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTileN = 16;
constexpr int kTileK = 128;
constexpr int kTileWords = 256;  // 1 KiB

// Activation / scale element type tags.
struct F16 {
  using elem = _Float16;
  using vec8 = f16x8;
  using vec4 = f16x4;
};
struct BF16 {
  using elem = __bf16;
  using vec8 = bf16x8;
  using vec4 = bf16x4;
};

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Group-dependent dequantisation constants of one lane's column.
struct ZS16 {
  f16x2 zb;  // (1024 + z) twice
  f16x2 zh;  // -(64 + z) twice
  f16x2 s;   // scale twice
};
struct ZSbf {
  float z;
  float s;
};

// (a & mask) | bits.  gfx9 VOP3 encodings (v_and_or_b32) take no literal
// constants, so with literal masks the compiler emits v_and_b32 + v_or_b32.
// Callers pass `mask`/`bits` through opaque_vgpr() once, outside the loops;
// the compiler then selects one v_and_or_b32 itself (and, unlike inline asm
// for the instruction, keeps tracking its hazards, e.g. before an MFMA reads
// the result).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) { return (a & mask) | bits; }

// The value v, hidden from constant folding and held in a VGPR.
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Loop-invariant dequantisation constants, held in VGPRs (see and_or).
struct DqK {
  uint32_t lo;     // 0x000F000F: nibbles 0 and 4 of a word
  uint32_t hi;     // 0x00F000F0: nibbles 1 and 5
  uint32_t magic;  // 0x64006400: the fp16 pair (1024, 1024)
};
__device__ __forceinline__ DqK dq_consts() {
  return DqK{opaque_vgpr(0x000F000Fu), opaque_vgpr(0x00F000F0u), opaque_vgpr(0x64006400u)};
}

// Typed load at a 32-bit byte offset from a uniform base pointer, so the
// compiler can use the global_load saddr form (SGPR base + VGPR offset)
// instead of per-lane 64-bit address arithmetic.
template <typename T>
__device__ __forceinline__ T ld_off(const void* base, uint32_t byte_off) {
  return *(const T*)((const char*)base + byte_off);
}
template <typename T>
__device__ __forceinline__ T ld_off_nt(const void* base, uint32_t byte_off) {
  return __builtin_nontemporal_load((const T*)((const char*)base + byte_off));
}

template <typename DT>
struct Dq;

// fp16, per 32-bit word (pairs i = rows (2i, 2i+1) = nibbles (i, i + 4)):
//   nibbles 0,4:  w & 0x000F000F | 0x64006400   = the pair (1024 + q)
//   nibbles 1,5:  w & 0x00F000F0 | 0x64006400   = the pair (1024 + 16 q)
//   nibbles 2,6 and 3,7: the same on w >> 8.
// (1024 + q) - (1024 + z) and fma(1024 + 16 q, 1/16, -(64 + z)) are both the
// exact integer q - z (fp16 integers below 2048, power-of-two scaling), and
// the one packed multiply by the scale is the single round-to-nearest-even
// of (q - z) * s that the oracle specifies: 13 VALU operations per word.
template <>
struct Dq<F16> {
  using ZS = ZS16;
  __device__ __forceinline__ static ZS make(uint32_t z, uint16_t sbits) {
    ZS r;
    const uint32_t zb = 0x6400u | z;
    const uint32_t zh = 0xD400u | (z << 4);
    r.zb = __builtin_bit_cast(f16x2, zb | (zb << 16));
    r.zh = __builtin_bit_cast(f16x2, zh | (zh << 16));
    r.s = __builtin_bit_cast(f16x2, (uint32_t)sbits | ((uint32_t)sbits << 16));
    return r;
  }
  __device__ __forceinline__ static f16x8 word(uint32_t w, const ZS& zs, const DqK& k) {
    const f16x2 inv16 = __builtin_bit_cast(f16x2, 0x2C002C00u);  // (1/16, 1/16)
    const uint32_t w8 = w >> 8;
    const f16x2 a0 = __builtin_bit_cast(f16x2, and_or(w, k.lo, k.magic));
    const f16x2 a1 = __builtin_bit_cast(f16x2, and_or(w, k.hi, k.magic));
    const f16x2 a2 = __builtin_bit_cast(f16x2, and_or(w8, k.lo, k.magic));
    const f16x2 a3 = __builtin_bit_cast(f16x2, and_or(w8, k.hi, k.magic));
    const f16x2 h0 = (a0 - zs.zb) * zs.s;
    const f16x2 h1 = __builtin_elementwise_fma(a1, inv16, zs.zh) * zs.s;
    const f16x2 h2 = (a2 - zs.zb) * zs.s;
    const f16x2 h3 = __builtin_elementwise_fma(a3, inv16, zs.zh) * zs.s;
    const u32x4 r = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                     __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3)};
    return __builtin_bit_cast(f16x8, r);
  }
  // The exact integers q - z (no scaling): 9 VALU operations per word, for
  // kernels that apply the group scale to the fp32 sums instead.
  __device__ __forceinline__ static f16x8 word_q_minus_z(uint32_t w, const ZS& zs, const DqK& k) {
    const f16x2 inv16 = __builtin_bit_cast(f16x2, 0x2C002C00u);  // (1/16, 1/16)
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = __builtin_bit_cast(f16x2, and_or(w, k.lo, k.magic)) - zs.zb;
    const f16x2 h1 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, and_or(w, k.hi, k.magic)), inv16, zs.zh);
    const f16x2 h2 = __builtin_bit_cast(f16x2, and_or(w8, k.lo, k.magic)) - zs.zb;
    const f16x2 h3 = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, and_or(w8, k.hi, k.magic)), inv16, zs.zh);
    const u32x4 r = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                     __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3)};
    return __builtin_bit_cast(f16x8, r);
  }
};

// bf16: (q - z) * s is exact in fp32 (4-bit by 8-bit significands) and the
// conversion to bf16 is the single round-to-nearest-even.
template <>
struct Dq<BF16> {
  using ZS = ZSbf;
  __device__ __forceinline__ static ZS make(uint32_t z, uint16_t sbits) {
    ZS r;
    r.z = (float)z;
    r.s = __builtin_bit_cast(float, (uint32_t)sbits << 16);
    return r;
  }
  __device__ __forceinline__ static bf16x8 word(uint32_t w, const ZS& zs, const DqK&) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = (float)((w >> (4 * i)) & 0xFu);
      const float hi = (float)((w >> (4 * i + 16)) & 0xFu);
      r[2 * i] = (__bf16)((lo - zs.z) * zs.s);
      r[2 * i + 1] = (__bf16)((hi - zs.z) * zs.s);
    }
    return r;
  }
};

// Biased operand: the fp16 pairs (1024 + q_lo, 1024 + q_hi) (bf16: 128 + q)
// straight from the nibbles, with no zero subtraction or scaling.  The GEMM
// kernels scale each group's dot product in fp32 and subtract the
// (bias + z) * sum(x) term separately, so one v_and_or_b32 per pair is all the
// per-element work.
template <typename DT>
struct Raw;
template <>
struct Raw<F16> {
  static constexpr uint32_t kMagic = 0x64006400u;  // (1024, 1024)
  static constexpr uint32_t kOnes = 0x3C003C00u;   // (1, 1)
  static constexpr float kBias = 1024.f;
};
template <>
struct Raw<BF16> {
  static constexpr uint32_t kMagic = 0x43004300u;  // (128, 128)
  static constexpr uint32_t kOnes = 0x3F803F80u;   // (1, 1)
  static constexpr float kBias = 128.f;
};

template <typename DT>
__device__ __forceinline__ typename DT::vec8 biased_word(uint32_t w, uint32_t mask, uint32_t magic) {
  const u32x4 r = {and_or(w, mask, magic), and_or(w >> 4, mask, magic), and_or(w >> 8, mask, magic),
                   and_or(w >> 12, mask, magic)};
  return __builtin_bit_cast(typename DT::vec8, r);
}

__device__ __forceinline__ f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Split-K handoff between workgroups (possibly on different XCDs, whose L2s
// are not coherent with each other) uses device-scope atomics only: partials
// are written with returning atomic exchanges (complete at the device
// coherence point before the value returns), the arrival counter is a
// device-scope fetch-add, and the last workgroup reads the partials back with
// atomic exchanges.  No agent-scope fence -- i.e. no L2 writeback/invalidate
// -- is executed.
__device__ __forceinline__ float xchg_agent(float* p, float v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t zero_nibble(uint64_t zw, int c) {
  return (uint32_t)(zw >> (4 * c)) & 0xFu;
}

// Round an fp32 accumulator to the output dtype, then add the bias in that
// dtype (the reference adds bias to the already-rounded GEMM output,
// awq.py:145-146 / marlin_utils.py:412-413).
template <typename DT>
__device__ __forceinline__ typename DT::elem finish(float acc, const typename DT::elem* bias, int n) {
  typename DT::elem r = (typename DT::elem)acc;
  if (bias != nullptr) r = (typename DT::elem)((float)r + (float)bias[n]);
  return r;
}

}  // namespace sgl_awq
