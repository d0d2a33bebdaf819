// W4A16 GEMM planning and dispatch for gfx950: out[M, N] = x[M, K] @ W
// (+ bias), fp32 accumulation, optionally with the gated activation of a
// merged gate/up projection fused (out[M, N / 2] = act(gate) * up).  Four
// kernel kinds share the CDNA4 tile layout (awq_device.h):
//
//  * gemv_kernel (awq_gemv.hip): batches of a few rows, HBM-bound;
//  * skinny_kernel (awq_skinny.hip): decode batches up to 32 rows, HBM-bound
//    split-K;
//  * the tiled kind (awq_tiled.hip: tiled_kernel on 16x16x32 MFMAs,
//    mfma32_kernel on 32x32x16 ones): prefill (MFMA-bound), mid-size batches
//    and 5-32 rows on large or deep matrices, split K summed by a second
//    reduction kernel (or, on request, inside the GEMM kernel);
//  * kslice_kernel (awq_kslice.hip): decode batches up to 32 rows, split K
//    reduced by the last workgroup of each column group (planner override
//    only).
//
// Replaces awq_gemm_kernel / awq_gemm_triton
// (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:16-195)
// and gptq_marlin_gemm (marlin_utils.py:388-410).
#include <limits.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "awq_device.h"
#include "awq_epilogue.h"
#include "awq_fixup.h"
#include "awq_launch.h"

namespace sgl_awq {

namespace {

// ---------------------------------------------------------------------------
// Planning and dispatch.
// ---------------------------------------------------------------------------
// Planner overrides (tests and sweeps only; see awq_set_plan_override).  An
// unset knob holds kUnset and the planner's own choice stands.
constexpr int kUnset = INT_MIN;
std::atomic<int> g_override[kPlanKnobs] = {kUnset, kUnset, kUnset, kUnset, kUnset, kUnset,
                                           kUnset, kUnset, kUnset, kUnset, kUnset};

int knob(int k, int dflt) {
  const int v = g_override[k].load(std::memory_order_relaxed);
  return v == kUnset ? dflt : v;
}

// CU count of each device, queried once (0 = not yet known).
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];

// Decode-kernel shapes that are instantiated (ntw * 10000 + wn * 100 + wk).
bool skinny_variant_ok(int v) {
  switch (v) {
    case 10104: case 10108: case 10116: case 10202: case 10401: case 10404:
    case 20202: case 20401: case 20204:
      return true;
    default:
      return false;
  }
}

// LDS a GEMV workgroup may use for its activation slice: gfx950 gives one
// workgroup up to 160 KiB; 4 KiB stay free for the kernel's static LDS.
constexpr int64_t kGemvLdsMax = 156 * 1024;

// Split of K for a GEMV variant: the smallest count that keeps each wave
// within its KPW k-tiles and the workgroup's activation slice within 8 loads
// per thread and kGemvLdsMax of LDS.  0 if none fits.
struct GemvSplit {
  int64_t ks, ktc, xpt, lds;
};
GemvSplit gemv_split(const Geom& g, int v, int64_t ks) {
  const int ntw = v / 10000, wn = (v / 1000) % 10, wk = (v / 10) % 100, kpw = v % 10;
  const int64_t mt = (g.M + 15) / 16, threads = 64 * wn * wk;
  for (ks = std::max<int64_t>(1, std::min<int64_t>(ks, g.KT)); ks <= g.KT; ++ks) {
    const int64_t ktc = (g.KT + ks - 1) / ks;
    const int64_t xpt = (g.M * ktc * 16 + threads - 1) / threads;
    // activation slice (rows padded by 8 halves), up to 3 rows its per-k-tile
    // row sums (the biased-operand path), then (reusing the space) the
    // k-waves' partial sums
    const int64_t lds = std::max<int64_t>(((g.M * (ktc * 128 + 8) * 2 + 15) & ~int64_t(15)) +
                                              (g.M <= 3 ? ktc * g.M * 4 : 0),
                                          (int64_t)wk * wn * mt * ntw * 1024);
    if ((ktc + wk - 1) / wk <= kpw && xpt <= 8 && lds <= kGemvLdsMax) return {(g.KT + ktc - 1) / ktc, ktc, xpt, lds};
  }
  return {0, 0, 0, 0};
}
int64_t gemv_min_ks(const Geom& g, int v) {
  const int wk = (v / 10) % 100, kpw = v % 10;
  return (g.KT + (int64_t)wk * kpw - 1) / ((int64_t)wk * kpw);
}
}  // namespace

bool set_plan_override(int k, int value) {
  if (k < 0 || k >= kPlanKnobs) return false;
  g_override[k].store(value, std::memory_order_relaxed);
  return true;
}

void clear_plan_overrides() {
  for (auto& o : g_override) o.store(kUnset, std::memory_order_relaxed);
}

// Compute units of the current device (what the grid and split-K choices fill),
// from hipDeviceAttributeMultiprocessorCount on the first call per device; a
// partitioned MI355X (CPX/DPX modes) reports its partition's share.  256 (a
// whole MI355X) when no device is visible, so that host-only planning queries
// stay answerable.
int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 256;
  }
  if (dev < kMaxDevices) {
    const int c = g_cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  if (dev < kMaxDevices) g_cus[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// GEMV variant (code ntw * 10000 + wn * 1000 + wk * 10 + kpw): 8 waves of at
// most 3 or 4 k-tiles each, whichever splits K fewer times (3 on a tie: fewer
// load slots re-read a wave's last tile).  At 1-3 rows a K of 25-128 k-tiles
// (4 rows from 33 k-tiles: Llama-3-8B down at M = 4 13.5 -> 11.8 us; up to 6
// rows for 65-80 k-tiles) goes to the smallest of 8 waves x 4, 6 or
// 8 and 16 waves x 5, 6 or 8 k-tiles that covers it: a split costs a
// cross-workgroup handoff (~1.7 us), more than the workgroups it adds save
// (Qwen3-4B down 8.4 -> 7.5 us at M = 1, 9.9 -> 9.3 us at M = 6; Llama-3-8B
// down 12.2 -> 11.0 us and 70B-sized o 12.5 -> 10.9 us at M = 1; at 4 rows
// and more on other depths the larger activation slices lose).  One column
// tile per workgroup up to 4 rows; from 5 rows (7 on layers of >= 2048 column
// tiles, where the workgroup count matters more) two column tiles share a
// workgroup of 16 waves, which halves the activation slices staged per weight
// byte.  With a fused gate/up activation a workgroup holds one gate tile and
// its up tile, in 8 waves of 3 or 4 k-tiles by the same rule (the Qwen3-4B
// gate_up, 20 k-tiles, unsplit: 12.3 -> 9.9 us at M = 1, 13.8 -> 10.9 us at
// M = 4).  (Graph-replay sweep of the variants over the Qwen3-4B, Llama-3-8B
// and Llama-3-70B shapes.)
int gemv_default_variant(const Geom& g, int act) {
  if (act) {
    // 7+ rows on 513-768 gate/up pairs with K within 20 k-tiles (the Qwen3-4B
    // gate_up): three pairs per workgroup (3 x 5 waves of 4 k-tiles), 203
    // workgroups that each stage the activation slice once (13.4 -> 11.4 us
    // at M = 8; even at M = 6, slower at M = 4).
    if (g.M >= 7 && g.NT > 1024 && g.NT <= 1536 && g.KT <= 20) return 23054;
    const int64_t k3 = gemv_split(g, 21083, gemv_min_ks(g, 21083)).ks, k4 = gemv_split(g, 21084, gemv_min_ks(g, 21084)).ks;
    return (k3 > 0 && (k4 == 0 || k3 <= k4)) ? 21083 : 21084;
  }
  // 1025-1280 column tiles (the Qwen3-4B gate_up, 1216) and K within 21
  // k-tiles, 2+ rows: five column tiles per workgroup (5 x 3 waves of 7
  // k-tiles) put one workgroup on each CU, which then stages the activation
  // slice once instead of five times (12.2 -> 10.1 us at M = 8; at M = 1 and
  // on layers whose workgroup count misses 256 it is slower).
  // From 14 rows on 1025-1536 column tiles with K within 20 k-tiles, six
  // column tiles per workgroup (3 x 5 waves of 4 k-tiles, 203 workgroups on
  // the Qwen3-4B gate_up) beat five: 11.8 -> 11.2 us at M = 16, and up to 24
  // rows they beat the tiled kernel too (14.5 -> 13.2 us at M = 24).
  if (g.M >= 14 && g.NT > 1024 && g.NT <= 1536 && g.KT <= 20) return 23054;
  if (g.M >= 2 && g.NT > 1024 && g.NT <= 1280 && g.KT <= 21) return 15037;
  if (g.KT > 24 && g.KT <= 128 && (g.M <= 3 || (g.M == 4 && g.KT > 32) || (g.M <= 6 && g.KT > 64 && g.KT <= 80))) {
    for (int v : {11084, 11086, 11088, 11165, 11166, 11168})
      if (((v / 10) % 100) * (v % 10) >= g.KT) return v;
  }
  // Two column tiles per workgroup only where that still leaves >= 192
  // workgroups (tensor-parallel shards at M = 8: a 1280-column qkv shard, 80
  // tiles, 9.7 -> 9.1 us with one tile per workgroup), from 4 rows below 2048
  // column tiles (4096 x 14336 at M = 4: 10.8 -> 9.7 us; 4096 x 28672 at
  // M = 6: 19.0 -> 18.2 us).
  const int wn = g.M >= (g.NT >= 2048 ? 7 : 4) && g.NT >= 384 ? 2 : 1;
  const int v3 = 10083 + wn * 1000, v4 = v3 + 1;
  const int64_t k3 = gemv_split(g, v3, gemv_min_ks(g, v3)).ks, k4 = gemv_split(g, v4, gemv_min_ks(g, v4)).ks;
  return (k3 > 0 && (k4 == 0 || k3 <= k4)) ? v3 : v4;
}

// 17-32 rows with K of 17-24 k-tiles on layers of >= 384 column tiles, where
// the GEMV kernel's default plan stages the whole activation slice unsplit
// (at most 8 loads per thread): its two-tile (or six-tile) workgroups beat the
// tiled kernel there (Qwen3-4B qkv at M = 24: 11.1 -> 8.6 us, at M = 25: 11.2
// -> 8.8 us).  Beyond that the slice needs a K split and the tiled kernel wins.
bool gemv_unsplit_short_k(const Geom& g) {
  if (g.M <= 16 || g.M > 32 || g.KT <= 16 || g.KT > 24 || g.NT < 384) return false;
  const int v = gemv_default_variant(g, 0);
  return gemv_split(g, v, gemv_min_ks(g, v)).ks == 1;
}

// Where the GEMV kernel wins over the decode (skinny) kernel, from a
// graph-replay sweep of M = 1..16 over the Qwen3-4B, Llama-3-8B and
// Llama-3-70B projections on MI355X:
//  * up to 4 rows, except 3-4 rows on very wide layers (>= 2048 column
//    tiles: 5-10% slower than the skinny kernel's two-tile waves);
//  * 5-16 rows, except on wide layers (>= 1024 column tiles) with K beyond
//    24 k-tiles other than at 7-8 rows, narrow ones (< 384 column tiles) with K of 25-63
//    k-tiles, and wherever the activation slice would cut a workgroup's K
//    range to 16 k-tiles or fewer (2 per wave): there the workgroup's staged
//    activation slice costs more than the skinny kernel's per-wave fragments;
//  * 17-32 rows with short K on layers of >= 384 column tiles whose
//    activation slice it stages unsplit (gemv_unsplit_short_k).
// A fused gate/up activation keeps the GEMV kernel up to 4 rows, and up to 8
// rows when K fits in 24 k-tiles.
bool gemv_preferred(const Geom& g, int act) {
  const int forced = knob(kPlanGemvMaxM, -1);
  if (forced >= 0) return g.M <= forced;
  if (act) return g.M <= 4 || (g.M <= 8 && g.KT <= 24);
  // K of at most 8 k-tiles (tensor-parallel o_proj shards): the GEMV
  // kernel's staged activation slice costs more than the skinny kernel's
  // per-wave fragments up to 16 rows (1024 x 8192 at M = 1: 5.2 -> 4.7 us;
  // 1024 x 4096 at M = 8: 5.0 -> 4.5 us); at 17-32 rows on wide layers the
  // GEMV kernel's two-tile workgroups win (1024 x 8192 at M = 32: 7.6 -> 6.7 us).
  if (g.KT <= 8) return g.M > 16 && g.NT >= 384;
  if (g.M <= 4) return g.M <= 2 || g.NT < 2048;
  if (g.M > 16) return gemv_unsplit_short_k(g);
  // Fewer than 128 column tiles, up to 8 rows: the skinny kernel would split
  // K to fill the CUs (4096 x 1536 at M = 8: 9.0 -> 6.8 us on the GEMV
  // kernel, K unsplit); from 12 rows the skinny kernel's 16-wave workgroups
  // win (7.4 against 8.4 us at M = 12).  Narrow layers with short K (at most
  // 16 k-tiles) keep the skinny kernel (2048 x 4096 at M = 8: 5.8 -> 5.2 us).
  if (g.NT < 128) return g.M <= 8;
  if (g.KT <= 16 && g.NT <= 256) return false;
  if (g.KT <= 24) return true;
  // Wide layers with deep K: the skinny kernel's two-tile waves, except at
  // 7-8 rows below 2048 column tiles, where the GEMV kernel's two-tile
  // workgroups win (4096 x 28672
  // at M = 7: 19.5 -> 18.3 us, at M = 8: 20.4 -> 18.8 us; at 5-6 rows the two
  // are within run-to-run noise of each other).
  if ((g.NT >= 1024 && (g.M <= 6 || g.M > 8 || g.NT >= 2048)) || (g.NT < 384 && g.KT < 64)) return false;
  const int v = gemv_default_variant(g, 0);
  return gemv_split(g, v, gemv_min_ks(g, v)).ktc > 16;
}

bool plan_gemv(const Geom& g, GemmPlan& p, int act) {
  if (g.NG > 1 && g.G < 128) return false;
  int v = gemv_default_variant(g, act);
  const int env = knob(kPlanGemvVariant, 0);
  if (gemv_variant_ok(env) && (!act || env / 10000 == 2)) v = env;
  if (!gemv_variant_ok(v)) return false;
  const int ntw = v / 10000, wn = (v / 1000) % 10;
  const int env_ks = knob(kPlanGemvKs, 0);
  const GemvSplit sp = gemv_split(g, v, env_ks > 0 ? env_ks : gemv_min_ks(g, v));
  if (sp.ks == 0) return false;
  p.kind = 2;
  p.variant = v;
  p.ktc = (int)sp.ktc;
  p.ks = (int)sp.ks;
  p.xpt = sp.xpt <= 1 ? 1 : (sp.xpt <= 2 ? 2 : (sp.xpt <= 4 ? 4 : 8));
  p.grid_x = (g.NT + (int64_t)wn * ntw - 1) / ((int64_t)wn * ntw);
  p.grid_y = p.ks;
  p.ws_bytes = p.ks > 1 ? (int64_t)p.ks * g.M * g.NT * 16 * 4 : 0;
  p.lds_bytes = sp.lds;
  return true;
}

// Batches of 5..32 rows: the tiled kernel (32-row block, K split up to 16
// ways) beats both decode kernels on deep or wide matrices (graph replay of
// the Qwen3-4B, Llama-3-8B, Llama-3-70B linears and their tensor-parallel
// shards at M = 1..32 on MI355X):
//  * 17-32 rows: K * N >= 12M with N >= 6144 or K >= 8192 (at M = 32 qkv,
//    gate_up and down run 8-15% faster, e.g. 29.1 -> 24.7 us for a
//    4096 x 28672 gate_up; the o_proj shapes stay 8-15% faster on the decode
//    kernel), and the narrow deep layers below, except short K on wide
//    layers whose activation slice the GEMV kernel stages unsplit;
//  * 10-16 rows: K >= 8192 and K * N >= 40M (14336 x 4096 down: 19.4 ->
//    15.4 us at M = 16; 28672 x 8192 down: 67.7 -> 37.3 us);
//  * 5-9 rows: K >= 8192 and 4096 <= N < 32768 (the 70B qkv, o and down
//    projections: 48.7 -> 36.4 us for the down projection at M = 8; the
//    Llama-3-8B down, 14336 x 4096: 16.5 -> 13.8 us at M = 8 and 14.8 ->
//    12.7 us at M = 5 on the 32-row 32x32 kernel with 16 k-slices);
//  * 9-16 rows with >= 32 k-tiles, N >= 8192 and K * N >= 20M.
// A fused gate/up activation uses the 17-32 and 9-16 row rules only.
bool tiled_preferred(const Geom& g, int act) {
  const int forced = knob(kPlanTiledMinM, 0);
  if (forced > 0) return g.M >= forced;
  if (g.M > 32) return true;
  const int64_t kn = g.K * g.N;
  // Narrow layers with deep K (>= 48 k-tiles on <= 256 column tiles, or
  // >= 32 k-tiles on < 128) split K 14-16 ways on the 32-row kernel from 17
  // rows (Llama-3-8B down at TP2, 7168 x 4096, M = 24: 16.4 -> 12.7 us; the
  // 70B qkv shard, 8192 x 1280: 13.7 -> 11.3 us; 4096 x 1536: 10.8 -> 9.5
  // us), from 10 rows with >= 64 k-tiles (Qwen3-4B down at M = 12: 14.5 ->
  // 11.3 us), and from 28 rows with >= 32 k-tiles (o_proj-shaped 4096 x 2560
  // at M = 32: 12.1 -> 11.5 us).
  const bool narrow_deep = (g.KT >= 48 && g.NT <= 256) || (g.KT >= 32 && g.NT < 128);
  if (g.M > 16) {
    if (gemv_unsplit_short_k(g)) return false;  // the GEMV kernel's
    return (kn >= 12000000 && (g.N >= 6144 || g.K >= 8192)) || narrow_deep || (g.M >= 28 && g.KT >= 32 && g.NT <= 256);
  }
  // (9-16 rows: K of at most 31 k-tiles stays on the GEMV kernel, whose
  // workgroups stage the short activation slice once: the Qwen3-4B gate_up at
  // M = 16 13.1 -> 11.0 us, the 70B down shard, 3584 x 8192, 10.7 -> 9.2 us;
  // 32 and more k-tiles go tiled, where from 9 rows the GEMV kernel's
  // activation slice takes 8 chunks per thread: 4096 x 14336 at M = 10 15.2
  // -> 13.4 us, at M = 12 15.6 -> 13.5 us.)
  if (g.M >= 9 && g.KT >= 32 && g.N >= 8192 && kn >= 20000000) return true;
  if (act) return false;
  if (g.M >= 10)
    return (g.K >= 8192 && kn >= 40000000) || (g.KT >= 64 && g.NT <= 256 && (g.NT >= 128 || g.M >= 12));
  return g.M >= 5 && g.K >= 8192 && g.N >= 4096 && g.N < 32768;
}

// k-slice kernel plan of shape v (wn * 100 + wk * 10 + kpw): one k-slice of
// wk * kpw k-tiles per workgroup, column groups of wn * 64 columns (wn * 32
// gate columns with a fused activation).
bool plan_kslice(const Geom& g, int v, int act, GemmPlan& p) {
  if (g.M > 32 || !kslice_variant_ok(v)) return false;
  const int wn = v / 100, wk = (v / 10) % 10, kpw = v % 10;
  const int64_t ktc = (int64_t)wk * kpw;
  const int64_t ks = (g.KT + ktc - 1) / ktc;
  const int64_t gx = act ? ((g.NT >> 1) + 2 * wn - 1) / (2 * wn) : (g.NT + 4 * wn - 1) / (4 * wn);
  const int64_t ws = ks > 1 ? ks * g.M * g.NT * 16 * 4 : 0;
  if (ks > 16 || ws >= (int64_t(1) << 31)) return false;
  p.kind = 3;
  p.variant = v;
  p.ktc = (int)ktc;
  p.ks = (int)ks;
  p.grid_x = gx;
  p.grid_y = 1;
  p.ws_bytes = ws;
  return true;
}

// The k-slice kernel is not chosen by the planner (only by the override):
// its handoff of plain partial stores needs an agent-scope release (an L2
// writeback) in every workgroup and an acquire in the last one, and with
// them it loses to the other decode forms on every shape it used to win
// (graph-replay sweep on MI355X, Qwen3-4B down 9728 x 2560: 12.96 us at M = 8
// against 10.41 for the split GEMV, 15.61 at M = 32 against 13.48 for the
// 16-slice 32-row tiled kernel; o_proj 4096 x 2560 at M = 32: 12.32 against
// 11.59).

GemmPlan plan_gemm(const Geom& g, int act) {
  GemmPlan p{};
  const int ksv = knob(kPlanKsliceVariant, 0);
  if (ksv != 0 && plan_kslice(g, ksv, act, p)) return p;
  const bool tiled = tiled_preferred(g, act);
  if (!tiled && gemv_preferred(g, act) && plan_gemv(g, p, act)) return p;
  if (!tiled) {
    p.kind = 0;
    // Variant code: ntw * 10000 + wn * 100 + wk.  Chosen from a sweep of all
    // variants over the Qwen3-4B and Llama-3-8B decode shapes on MI355X:
    // wide layers (>= 1024 column tiles) use two column tiles per wave;
    // narrower ones put one column tile per workgroup and split K over 4-16
    // waves, more of them for short or very long K.
    // Short K (at most 8 k-tiles) at up to 16 rows: two column tiles per
    // workgroup in two waves each where that still gives one workgroup per
    // CU, else 16 waves on one tile; otherwise narrow layers with up to 16
    // k-tiles take 4 waves (1024 x 4096 at M = 32: 5.9 -> 5.4 us; 2048 x 4096
    // at M = 8: 5.3 -> 5.0 us).  Narrow layers with 17-31 or 48-63 k-tiles
    // take 16 waves (3584 x 4096 at M = 8: 7.5 -> 6.6 us; 7168 x 4096: 11.4 ->
    // 9.7 us), 32-47 k-tiles 4 waves up to 8 rows and 8 beyond (4096 x 2560
    // at M = 24: 10.6 -> 10.3 us), except on layers of fewer than 128 column
    // tiles, where 16 waves keep K unsplit (4096 x 1536 at M = 10: 7.4 -> 7.0
    // us).
    int ntw = 1, wn = 1, wk = 4;
    if (g.NT >= 1024) {
      ntw = 2;
      wn = g.M <= 8 ? 2 : 4;
      wk = g.M <= 8 ? 2 : 1;
    } else if (g.KT <= 8 && g.M <= 16) {
      wn = g.NT >= 2 * g.cus ? 2 : 1;
      wk = wn == 2 ? 2 : 16;
    } else if (g.M > 16 && g.NT >= 384) {
      wn = 2;
      wk = 2;
    } else if (g.KT <= 16) {
      wk = 4;
    } else if (g.NT < 128 || g.KT < 32 || g.KT >= 48) {
      wk = 16;
    } else {
      wk = g.M <= 8 ? 4 : 8;
    }
    if (act && ntw != 2) {  // a fused gate/up pair needs two tiles per wave
      ntw = 2;
      wn = 2;
      wk = g.M <= 16 ? 4 : 2;
    }
    const int env = knob(kPlanSkinnyVariant, 0);
    if (skinny_variant_ok(env) && (!act || env / 10000 == 2)) {
      ntw = env / 10000;
      wn = (env / 100) % 100;
      wk = env % 100;
    }
    const int64_t ntg = (int64_t)wn * ntw;
    p.variant = ntw * 10000 + wn * 100 + wk;
    p.grid_x = (g.NT + ntg - 1) / ntg;
    int64_t ks = 1;
    if (p.grid_x < g.cus / 2) {
      // Few column tiles: split K so about one workgroup per CU is busy,
      // keeping >= 4 k-tiles per wave and the partial traffic
      // (KS * M * N * 8 bytes) below a quarter of the weight stream.
      ks = (g.cus + p.grid_x - 1) / p.grid_x;
      ks = std::min(ks, std::max<int64_t>(1, g.KT / (2 * wk)));
      ks = std::min(ks, std::max<int64_t>(1, g.K / (64 * g.M)));
    }
    const int env_ks = knob(kPlanSkinnyKs, 0);
    if (env_ks > 0) ks = env_ks;
    ks = std::max<int64_t>(1, std::min<int64_t>(ks, g.KT));
    p.ktc = (int)((g.KT + ks - 1) / ks);
    p.ks = (int)((g.KT + p.ktc - 1) / p.ktc);  // every workgroup gets >= 1 k-tile
    p.grid_y = p.ks;
    p.ws_bytes = p.ks > 1 ? (int64_t)p.ks * g.M * g.NT * 16 * 4 : 0;
  } else {
    p.kind = 1;
    // Row block and k-slices from a cost model fitted to sweeps over the
    // Llama-3-8B and Qwen3-4B linears at M = 16 .. 2048 on MI355X (it picks
    // the measured best, or within 6%, in 71 of 72 cases): time ~ waves of
    // 256 workgroups x (k-tiles per slice + 1), a 64-row step costing 0.75
    // and a 32-row step 0.3 of a 128-row one, plus the partial traffic of the
    // split-K reduction.  The 32-row block serves batches of at most 32 rows.
    // Row-block codes: 32, 64, 128 = tiled_kernel (16x16x32 MFMAs);
    // 1064, 1128 = mfma32_kernel (32x32x16 MFMAs) at 64 and 128 rows;
    // 2064, 2128 = the same with registers for two workgroups per CU;
    // 4032 = the same at 32 rows with registers for four;
    // 8064, 8128 = 8 waves and 512 columns per workgroup, one per CU.
    // 32-row blocks beyond 32 rows, up to 160, on layers of at most 8192
    // columns and 4096 rows of K (graph-replay A/B at M = 48..160 over the
    // Llama-3-8B and Qwen3-4B linears: qkv and o 7-19% faster in the 32x32
    // kernel with four workgroups per CU; wider or deeper layers, gate_up and
    // down, 3-16% slower, so they keep 64- and 128-row blocks), and up to 112
    // rows on layers of at most 4096 columns and 12288 rows of K (Qwen3-4B
    // down at M = 40..112: 5-10% faster; even at 128, slower at 160).  With
    // K of 4097-8192 the 64-row block stays (a 70B-sized o_proj, K = N = 8192,
    // at M = 40 / 64 / 96 / 128: 21.6 -> 20.5 / 23.4 -> 22.4 / 33.9 -> 29.9 /
    // 35.9 -> 31.2 us against 32-row blocks).
    const bool bm32_ok = g.M <= 32 || (g.M <= 160 && g.N <= 8192 && g.K <= 4096) ||
                         (g.M <= 112 && g.N <= 4096 && g.K <= 12288);
    const int env_bm = knob(kPlanTiledBm, 0);
    const bool env_bm_ok = env_bm == 32 || env_bm == 64 || env_bm == 128 || env_bm == 1064 || env_bm == 1128 ||
                           env_bm == 2064 || env_bm == 2128 || env_bm == 4032 || env_bm == 8064 || env_bm == 8128 ||
                           ((env_bm == 9064 || env_bm == 9128) && g.G >= 64);
    const int env_ks = knob(kPlanTiledKs, 0);
    const int64_t Np = g.NT * 16;
    double best = 0.0;
    int best_bm = 0, best_ks = 1;
    for (int code : {32, 64, 128, 1064, 1128, 2064, 2128, 4032, 8064, 8128, 9064, 9128}) {
      const int bm = code % 1000;
      // the cost model ranks the 16x16 codes; the rules below move shapes to the 32x32 forms
      if (env_bm_ok ? code != env_bm : code >= 1000) continue;
      if (g.K > tiled_max_k(bm) || (!env_bm_ok && bm == 32 && !bm32_ok)) continue;
      const int64_t tiles = ((g.NT + 15) / 16) * ((g.M + bm - 1) / bm);
      const int64_t min_ktc = g.M <= 32 ? 2 : 4;  // k-tiles per slice at least
      for (int ks : {1, 2, 3, 4, 6, 8, 12, 16}) {
        if (env_ks > 0 ? ks != 1 : (ks > 1 && ks > g.KT / min_ktc)) continue;
        const int64_t ktc = (g.KT + ks - 1) / ks, kse = (g.KT + ktc - 1) / ktc;
        if (kse > 1 && kse * g.M * Np * 4 >= (int64_t(1) << 31)) continue;  // 32-bit partial offsets
        const int64_t waves = (tiles * kse + g.cus - 1) / g.cus;
        double t = (double)waves * (double)(ktc + 1) * (bm == 32 ? 0.3 : (bm == 64 ? 0.75 : 1.0));
        if (kse > 1) t += (double)kse * (double)g.M * (double)Np * 4.0 / 3.2e6;
        if (best_bm == 0 || t < best) {
          best = t;
          best_bm = code;
          best_ks = ks;
        }
      }
    }
    if (best_bm == 0) best_bm = 64;  // K beyond every limit is rejected by the C ABI
    int64_t ks = env_ks > 0 ? env_ks : best_ks;
    ks = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(ks, g.KT), 16));  // the reduction takes <= 16
    while (ks > 1 && ks * g.M * Np * 4 >= (int64_t(1) << 31)) --ks;
    // Grids of at least 1.5 waves of 128-row tiles, unsplit, with at most two
    // groups per k-tile: the 32x32-MFMA kernel with two workgroups per CU
    // (Llama-3-8B gate_up at M = 2048: 472 -> 432 us; every linear at
    // M = 8192: 3-8% faster).  On one wave of tiles the second workgroup has
    // nothing to overlap with and the 16x16 kernel's deeper prefetch wins.
    // 32-row blocks with one group per k-tile: the 32x32-MFMA kernel at 32
    // rows with registers for four workgroups per CU (graph-replay sweep of
    // the Qwen3-4B and Llama-3-8B linears at M = 16 and 32: 4-12% faster, e.g.
    // Qwen3-4B gate_up at M = 16 15.1 -> 13.3 us; since its zero points and
    // scales come from LDS also at 12-16 k-slices: Llama-3-8B down at M = 12,
    // 16, 32 15.6 -> 14.1, 15.7 -> 14.6, 17.2 -> 16.9 us).
    if (!env_bm_ok && best_bm == 32 && g.G >= 128) best_bm = 4032;
    // One 8-wave workgroup of 512 columns per CU instead of two of 256: the
    // CU's columns share one activation stage (half the activation loads
    // per weight byte), and a grid of at most one round, or of whole rounds,
    // of 512-column tiles keeps every CU equally loaded where 256-column
    // tiles would double up on some CUs only (Llama-3-8B qkv at M = 2048:
    // 129 -> 112 us; qkv, o and down at M = 8192: 2-3% faster; gate_up at
    // M = 2048, 3.5 rounds, stays faster with two workgroups per CU; at
    // M = 1024, whose last round is three quarters full, 232 -> 220 us).
    // Above 256 rows, an unsplit grid of at most half a round of 128 x 256
    // tiles (more goes to code 9128 below) takes the 32x32-MFMA kernel at one
    // workgroup per CU (on grids of 160-192 tiles it was 8-11% faster than
    // the 16x16 kernel: Llama-3-8B and Qwen3-4B qkv at M = 1024 65.0 -> 59.2
    // and 44.6 -> 40.8 us), and one of between one and one and a half rounds
    // the 8-wave kernel when its 512-column tiles fit one round (Qwen3-4B
    // gate_up at M = 512, 304 tiles: 86.0 -> 60.6 us).
    // Above 192 rows, a grid of more than half and at most one round of
    // 128 x 256 tiles runs the 32x32-MFMA kernel with 8 waves that split each
    // k-tile's k-steps in two (code 9128: two waves per SIMD on a one-
    // workgroup-per-CU grid, K unsplit): Qwen3-4B down at M = 2048 120.1 (3
    // k-slices) -> 110.5 us, o_proj 60.8 -> 55.2 us; Llama-3-8B o at M = 2048
    // 73.0 -> 70.0 us, qkv at M = 1024 61.4 -> 59.1 us; 70B-sized qkv at
    // M = 512 105.3 -> 98.0 us, o at M = 1024 128.0 -> 124.9 us; Llama-3-8B
    // down at M = 2048 ties; at 193-256 rows, where every row block pads to
    // 256, Llama-3-8B / Qwen3-4B gate_up at M = 256 69.0 -> 64.7 / 39.4 ->
    // 37.3 us (at 192 rows it ties the 64-row forms, which pad less below).
    // On half a round or less the split-K plans win.
    // 65-128 rows on layers the 32-row rule leaves out (wide: more than 8192
    // columns) with K up to 4096, where the cost model picks 128-row blocks
    // with split K: K unsplit in the 32-row 32x32 form when its tiles fit one
    // round (Qwen3-4B gate_up at M = 72 / 80 / 96: 24.6 -> 21.0 / 25.3 ->
    // 21.2 / 26.5 -> 21.2 us), else in the 64-row k-wave split (Llama-3-8B
    // gate_up at M = 80 / 96: 41.6 -> 39.6 / 42.8 -> 39.7 us, at 72 a tie).
    if (!env_bm_ok && best_bm == 128 && g.G >= 128 && g.M > 64 && g.M <= 128 && g.K <= 4096) {
      const int64_t cb = (g.NT + 15) / 16;
      if (cb * ((g.M + 31) / 32) <= g.cus) {
        best_bm = 4032;
        ks = 1;
      } else if (cb * ((g.M + 63) / 64) <= g.cus) {
        best_bm = 9064;
        ks = 1;
      }
    }
    // 129-192 rows where the cost model picks 128-row blocks with split K:
    // the 64-row k-wave split with the most k-slices (up to the chosen count)
    // whose grid fits one round (Llama-3-8B down at M = 160 / 192: 39.9 ->
    // 36.3 / 40.7 -> 37.7 us with 4 slices; 70B-sized o at M = 160 / 192:
    // 44.6 -> 40.9 / 45.2 -> 42.6 us and down 120.1 -> 115.1 / 121.3 -> 119.2
    // us with 2 slices).
    if (!env_bm_ok && best_bm == 128 && ks > 1 && g.G >= 128 && g.M > 128 && g.M <= 192) {
      const int64_t t64 = ((g.NT + 15) / 16) * ((g.M + 63) / 64);
      int64_t k9 = 0;
      for (int c : {2, 3, 4, 6, 8, 12, 16})
        if (c <= ks && t64 * c <= g.cus) k9 = c;
      if (k9 >= 2) {
        best_bm = 9064;
        ks = k9;
      }
    }
    const int64_t t2_128 = ((g.NT + 15) / 16) * ((g.M + 127) / 128);
    // (With K of fewer than 16 k-tiles the split leaves too few k-steps per
    // wave: a 1024 x 4096 o_proj shard at M = 2048 runs 28.8 us there and
    // 27.0 us in the two-workgroup form.)
    if (!env_bm_ok && best_bm == 128 && g.G >= 64 && g.M > 192 && g.KT >= 16 && 2 * t2_128 > g.cus &&
        t2_128 <= g.cus) {
      best_bm = 9128;
      ks = 1;
    }
    if (!env_bm_ok && best_bm == 128 && ks == 1 && g.G >= 64) {
      const int64_t t2 = t2_128;
      const int64_t t8 = ((g.NT + 31) / 32) * ((g.M + 127) / 128);
      const int64_t cus = g.cus;
      if (2 * t2 >= 3 * cus) {
        best_bm = 2128;
        if (g.G >= 128 && (t8 <= cus || t8 % cus == 0 || 4 * (t8 % cus) >= 3 * cus)) best_bm = 8128;
      } else if (g.M > 256 && (t2 < cus || (g.KT < 16 && t2 <= cus))) {
        best_bm = 2128;
      } else if (g.M > 256 && g.G >= 128 && t2 > cus && t8 <= cus) {
        best_bm = 8128;
      }
    }
    // Batches of up to 256 rows with K unsplit, one group per k-tile
    // (graph-replay sweep of the Qwen3-4B and Llama-3-8B linears at M =
    // 96..256): a 128-row block on a grid whose 64 x 512 tiles fill at most
    // three quarters of the CUs takes the 8-wave 64-row form (two waves per
    // SIMD, less row padding: Llama-3-8B gate_up at M = 160 / 192 69.8 ->
    // 61.5 / 71.1 -> 63.3 us, Qwen3-4B gate_up at M = 224 44.1 -> 39.6 us;
    // on fuller grids it was 0.5-3% slower), and a 64-row block the 32x32
    // kernel: with at most one round of 64 x 256 tiles its 8-wave k-wave
    // split (code 9064, two waves per SIMD at one workgroup per CU: Qwen3-4B
    // gate_up at M = 112 / 128 / 160 / 192 27.8 -> 23.9 / 27.7 -> 23.9 /
    // 28.4 -> 26.7 / 29.5 -> 27.5 us, Llama-3-8B gate_up at M = 112 / 128
    // 43.5 -> 41.1 / 43.6 -> 41.8 us, 70B-sized gate_up at M = 40 / 64 83.5 ->
    // 77.4 / 88.3 -> 80.6 us against the two-workgroup form), else the two-
    // workgroup form (code 2064: Qwen3-4B gate_up at M = 128 30.5 -> 28.2 us
    // against the 16x16 kernel, 1-8% faster in every case measured).
    // A 64-row block takes the 32x32 kernel at larger M too (a 4096 x 1536
    // qkv shard at M = 2048: 45.3 -> 37.6 us in the k-wave split).
    if (!env_bm_ok && ks == 1 && g.G >= 128) {
      const int64_t t8 = ((g.NT + 31) / 32) * ((g.M + 63) / 64);
      const int64_t t64 = ((g.NT + 15) / 16) * ((g.M + 63) / 64);
      if (best_bm == 128 && g.M <= 256 && 4 * t8 <= 3 * (int64_t)g.cus) best_bm = 8064;
      else if (best_bm == 64) best_bm = t64 <= g.cus ? 9064 : 2064;
    }
    p.variant = best_bm;
    p.grid_x = best_bm >= 8000 && best_bm < 9000 ? (g.NT + 31) / 32 : (g.NT + 15) / 16;
    p.grid_y = (g.M + best_bm % 1000 - 1) / (best_bm % 1000);
    p.ktc = (int)((g.KT + ks - 1) / ks);
    p.ks = (int)((g.KT + p.ktc - 1) / p.ktc);  // every slice gets >= 1 k-tile
    p.ws_bytes = p.ks > 1 ? (int64_t)p.ks * g.M * g.NT * 16 * 4 : 0;
    // On request (AWQ_PLAN_TILED_FIXUP) the k-slice workgroups sum the slices
    // themselves (awq_fixup.h) when the tiles fit the counters and the grid
    // fits one workgroup per CU, so that on an idle device every k-slice of a
    // tile is resident together.  Off by default: graph-replay A/B over the
    // Qwen3-4B and Llama-3-8B split-K shapes at M = 16..256 measured the second
    // kernel 3-14% faster at M <= 160 (Qwen3-4B gate_up at M = 32: 15.5 against
    // 17.2 us; Llama-3-8B down at M = 16: 14.0 against 16.0 us), equal at 128
    // and 6% slower only for the Llama-3-8B o_proj at M = 256.
    const int64_t tiles = p.grid_x * p.grid_y;
    p.fixup = p.ks > 1 && p.ks <= kFixupMaxSlices && tiles <= kFixupMaxTiles && tiles * p.ks <= g.cus &&
              knob(kPlanTiledFixup, 0) != 0;
    p.polls = std::max(0, knob(kPlanFixupPolls, kFixupDefaultPolls));
  }
  return p;
}

int plan_threads(const GemmPlan& p) {
  if (p.kind == 1) return p.variant >= 8000 ? 512 : 256;
  if (p.kind == 3) return 256;
  if (p.kind == 2) return 64 * ((p.variant / 1000) % 10) * ((p.variant / 10) % 100);
  return 64 * ((p.variant / 100) % 100) * (p.variant % 100);
}

hipError_t launch_gemm(const GemmPlan& p, const void* x, const void* w, const void* sr, const void* zr,
                       const void* bias, void* out, int dtype, const Geom& g, void* ws, int32_t* counters,
                       int64_t counter_bytes, int act, hipStream_t s) {
  // The decode kernels' per-column-tile counters follow the split tiles' ones.
  int32_t* col = counters != nullptr && counter_bytes >= kFixupBytes ? counters + kFixupBytes / 4 : nullptr;
  if (p.kind == 0) return launch_skinny(p, x, w, sr, zr, bias, out, dtype, g, ws, col, act, s);
  if (p.kind == 2) return launch_gemv(p, x, w, sr, zr, bias, out, dtype, g, ws, col, act, s);
  if (p.kind == 3) return launch_kslice(p, x, w, sr, zr, bias, out, dtype, g, ws, col, act, s);
  return launch_tiled(p, x, w, sr, zr, bias, out, dtype, g, ws, col != nullptr ? counters : nullptr, act, s);
}

}  // namespace sgl_awq
