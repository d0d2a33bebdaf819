// Internal launchers behind the C ABI (arguments already validated).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sgl_awq {

struct Geom {
  int64_t M, N, K, G;  // G already resolved (-1 -> K)
  int64_t NT, KT, NG;  // column tiles, row tiles, groups
  int gshift;          // group of row k = k >> gshift (31 for one group)
  int cus;             // compute units the plan fills (device_cu_count())
};

Geom make_geom(int64_t M, int64_t N, int64_t K, int64_t G);

// Compute units of the current device (256 when none is visible).
int device_cu_count();

// Planner overrides for tests and sweeps (awq_set_plan_override in the C ABI).
enum : int {
  kPlanGemvMaxM = 0,      // largest M routed to the GEMV kernel (0 disables it)
  kPlanGemvVariant = 1,   // GEMV shape code ntw*10000 + wn*1000 + wk*10 + kpw
  kPlanGemvKs = 2,        // GEMV k-slices
  kPlanSkinnyVariant = 3, // decode-kernel shape code ntw*10000 + wn*100 + wk
  kPlanSkinnyKs = 4,      // decode-kernel k-slices
  kPlanTiledMinM = 5,     // smallest M routed to the tiled kernel
  kPlanTiledBm = 6,       // tiled row-block code (32, 64, 128; 1064 ... 8128; 9064, 9128 with G >= 64)
  kPlanTiledKs = 7,       // tiled k-slices
  kPlanKsliceVariant = 8, // in-kernel split-K decode kernel shape wn*100 + wk*10 + kpw
  kPlanTiledFixup = 9,    // 0: tiled split-K plans sum their slices in a second kernel
  kPlanFixupPolls = 10,   // poll bound of the in-kernel split-K reduction (0: only the last arrival reduces)
  kPlanKnobs = 11
};
bool set_plan_override(int knob, int value);
void clear_plan_overrides();

hipError_t launch_repack(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype,
                         const Geom& g, void* w_out, void* s_out, void* z_out, hipStream_t s);
hipError_t launch_unrepack(const void* w, const void* sr, const void* zr, int dtype, const Geom& g,
                           int32_t* qweight, int32_t* qzeros, void* scales, hipStream_t s);
hipError_t launch_dequant_awq(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype,
                              const Geom& g, void* w_out, hipStream_t s);
hipError_t launch_dequant_repacked(const void* w, const void* sr, const void* zr, int dtype, const Geom& g,
                                   void* w_out, hipStream_t s);

// GEMM plan: which kernel and how K is split.
struct GemmPlan {
  int kind;      // 0 = skinny (M <= 32), 1 = tiled MFMA GEMM, 2 = GEMV (M <= 32),
                 // 3 = k-slice kernel (M <= 32, split-K reduced in the kernel)
  int variant;   // kernel template selector
  int ks;        // k-splits across workgroups
  int ktc;       // k-tiles per workgroup
  int xpt;       // activation chunks per thread (GEMV)
  int64_t grid_x, grid_y;
  int64_t ws_bytes;
  int64_t lds_bytes;  // dynamic LDS (GEMV)
  int fixup;          // tiled split K: the k-slice workgroups sum the slices (awq_fixup.h)
  int polls;          // ... each polling at most this often for the tile's other slices
};

// act: fused gate/up activation of the output (0 none, 1 silu, 2 gelu; the
// GEMM's two column halves are gate and up, the output has N / 2 columns).
GemmPlan plan_gemm(const Geom& g, int act = 0);
hipError_t launch_skinny(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                         const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                         hipStream_t s);
bool gemv_variant_ok(int v);
hipError_t launch_gemv(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                       hipStream_t s);
bool kslice_variant_ok(int v);
hipError_t launch_kslice(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                         const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                         hipStream_t s);
int64_t tiled_max_k(int bm);
hipError_t launch_tiled(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                        const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters, int act,
                        hipStream_t s);
// `counters`: the caller's counters buffer (awq_counter_bytes: the split
// tiles' counters of the tiled kernels, then one int32 per column tile for
// the decode kernels) of `counter_bytes` bytes, or null.
hipError_t launch_gemm(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                       int64_t counter_bytes, int act, hipStream_t s);

// Grouped MoE path (awq_moe.hip).
// Byte strides between consecutive experts' repacked weights, scales, zeros.
struct MoeStrides {
  int64_t w, s, z;
};
MoeStrides moe_expert_strides(const Geom& g);
int64_t moe_sorted_capacity(int64_t n, int64_t E, int64_t bs);
int64_t moe_block_capacity(int64_t n, int64_t E, int64_t bs);
hipError_t launch_moe_topk(const float* logits, float* tw, int32_t* tid, int64_t T, int64_t E, int64_t k, int renorm,
                           hipStream_t s);
hipError_t launch_moe_align(const int32_t* ids, int64_t n, int64_t E, int64_t bs, int32_t* sorted, int32_t* expert_ids,
                            int32_t* num_post_pad, int32_t* offsets, hipStream_t s);

struct MoeGemmParams {
  const void* x;           // activation rows
  const void* w;           // expert-stacked repacked weights / scales / zeros
  const void* s;
  const void* z;
  const int32_t* sorted;   // from launch_moe_align
  const int32_t* offsets;  // padded bucket offsets [E + 1]
  const float* topk_w;     // routed weights [num_routed]
  void* out;
  int64_t E, a_div, num_routed, sorted_cap;
  Geom g;       // per-expert geometry (M unused)
  int epi;      // 0 plain, 1 silu_and_mul, 2 gelu_and_mul (gate/up pairing)
  int mul_rw;   // multiply by the routed weight before the cast
  int dtype;
};
hipError_t launch_moe_gemm(const MoeGemmParams& p, hipStream_t s);
// Streaming probe (awq_probe.hip).
hipError_t launch_stream_probe(const void* src, int64_t bytes, int64_t grid, int block, uint32_t* sink,
                               hipStream_t s);
hipError_t launch_mfma_probe(int64_t iters, int64_t grid, int block, float* sink, hipStream_t s);
// Threads per workgroup of a plan's main kernel.
int plan_threads(const GemmPlan& p);

hipError_t launch_moe_sum(const void* in, void* out, int64_t T, int64_t k, int64_t H, int dtype, hipStream_t s);

// Gated MLP block in one launch (awq_mlp.hip).  Counters: 128-byte slots of
// 32 words; word 2 of slot 0 counts workgroups that gave up waiting, slot
// 1 + s is k-slice s's barrier, slot 1 + S + g column group g's.
constexpr int64_t kMlpCounterBytes = 64 << 10;
constexpr int kMlpDefaultPolls = 1 << 15;
struct MlpPlan {
  int ok;         // 0: outside the built forms (the caller runs the two GEMMs)
  int form;       // kernel instantiation
  int64_t P;      // workgroups (one per CU at most)
  int64_t S;      // k-slices of the down projection
  int64_t C;      // down column tiles per column group
  int64_t groups; // column groups (P = groups * S)
  int64_t npw;    // gate tiles per workgroup (of its k-slice)
  int64_t nk;     // down k-tiles per slice
  int64_t lds;    // dynamic LDS bytes
  int64_t h_bytes, ws_bytes;  // intermediate, then fp32 partials
};
// query_device: also check the grid against the device's occupancy for the
// kernel (false: the shape rules alone, for a host without a GPU).
MlpPlan plan_mlp(int64_t M, int64_t H, int64_t I, int64_t G, int dtype, bool query_device = true);
hipError_t launch_mlp(const MlpPlan& p, const void* x, const void* gw, const void* gs, const void* gz, const void* dw,
                      const void* ds, const void* dz, void* out, int64_t M, int64_t H, int64_t I, int dtype, int act,
                      void* ws, int32_t* counters, int polls, hipStream_t s);

}  // namespace sgl_awq
