// Internal launchers behind the C ABI (arguments already validated).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sgl_awq {

struct Geom {
  int64_t M, N, K, G;  // G already resolved (-1 -> K)
  int64_t NT, KT, NG;  // column tiles, row tiles, groups
  int gshift;          // group of row k = k >> gshift (31 for one group)
};

Geom make_geom(int64_t M, int64_t N, int64_t K, int64_t G);

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
  int kind;      // 0 = skinny (M <= 32), 1 = tiled MFMA GEMM
  int variant;   // kernel template selector
  int ks;        // k-splits across workgroups (skinny)
  int ktc;       // k-tiles per workgroup (skinny)
  int64_t grid_x, grid_y;
  int64_t ws_bytes;
};

GemmPlan plan_gemm(const Geom& g);
hipError_t launch_skinny(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                         const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                         hipStream_t s);
hipError_t launch_gemm(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                       hipStream_t s);

}  // namespace sgl_awq
