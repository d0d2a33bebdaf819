/*
 * sglite_awq.h -- C ABI of the MI355X (gfx950) AWQ W4A16 linear engine.
 *
 * Plain pointers and sizes only.  Every entry point that launches work takes
 * the caller's HIP stream, enqueues asynchronously and never synchronises the
 * device, allocates no device memory and takes no host-dependent decision
 * from device data, so it may be recorded into a HIP graph.  Every function
 * returning int returns 0 on success or a negative AWQ_STATUS_* code; the
 * message of the last failure on the calling thread is awq_last_error().
 * Each entry point that launches work opens a roctx range named after itself
 * for the duration of the call (rocprofv3 --marker-trace attributes the
 * kernels to the operation; the library links librocprofiler-sdk-roctx).
 *
 * Tensor conventions (all row-major, device pointers):
 *   qweight  int32 [K, N/8]   AWQ nibble order [0,2,4,6,1,3,5,7]
 *   qzeros   int32 [K/G, N/8] same packing
 *   scales   fp16|bf16 [K/G, N]
 *   x        fp16|bf16 [M, K]   (same dtype as scales)
 *   out      fp16|bf16 [M, N]
 * G is the group size: 32, 64, 128 or K (-1 is accepted and means K).
 * Requirements: K % 32 == 0, K % G == 0, N % 8 == 0 (the AWQ linear method's
 * own checks, python/sglite/srt/model_executor/layers/quantization/awq.py:76-85).
 * Engine limits (AWQ_STATUS_UNSUPPORTED beyond them): K < 2^24, N < 2^30,
 * M < 2^24 (the kernels address one workgroup's rows with 32-bit offsets).
 */
#ifndef SGLITE_AWQ_H
#define SGLITE_AWQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* awq_stream_t; /* == hipStream_t */

enum {
  AWQ_STATUS_OK = 0,
  AWQ_STATUS_INVALID_ARGUMENT = -1, /* bad pointer, shape, dtype or group size */
  AWQ_STATUS_UNSUPPORTED = -2,      /* valid request outside what is built     */
  AWQ_STATUS_HIP_ERROR = -3,        /* a HIP runtime call failed               */
  AWQ_STATUS_WORKSPACE = -4         /* workspace missing or too small          */
};

enum { AWQ_DTYPE_FP16 = 0, AWQ_DTYPE_BF16 = 1 };

/* Message of the last failed call on this thread ("" if none). */
const char* awq_last_error(void);

/* Library version string, e.g. "sglite-awq-gfx950 0.4". */
const char* awq_version(void);

/* ABI revision of this header.  A caller checks awq_abi_version() ==
 * AWQ_ABI_VERSION (the value it was built against) before its first call:
 *   1  the first release;
 *   2  awq_w4a16_gemm / awq_w4a16_gemm_act take `int64_t counter_bytes`
 *      after `counters` (the symbol names did not change);
 *   3  awq_counter_bytes(N) covers the tiled kernels' split-tile counters
 *      too (AWQ_COUNTER_TILE_BYTES ahead of the per-column-tile counters),
 *      counters must be 128-byte aligned; awq_noalloc_init and the planner
 *      knobs AWQ_PLAN_TILED_FIXUP / AWQ_PLAN_FIXUP_POLLS are new;
 *   4  the gated MLP block (awq_gated_mlp and its plan, workspace and error
 *      calls) is new.
 * No counterpart in the reference (its kernels are Python and Triton). */
#define AWQ_ABI_VERSION 4
int awq_abi_version(void);

/* ---- post-load repack ------------------------------------------------------
 * Replaces the Marlin post-load step of
 * python/sglite/srt/model_executor/layers/quantization/awq_marlin.py:298-319
 * (marlin_make_workspace, awq_marlin_repack, marlin_permute_scales,
 * awq_to_marlin_zero_points): rewrites the AWQ checkpoint tensors into the
 * CDNA4 tile layout, on the device, with no host round trip.
 *
 * Weights w: tiles of 16 columns x 128 rows (1 KiB), tile (nt, kt) at
 * (nt*ceil(K/128) + kt) KiB; lane l of a tile owns 4 words, word w holds
 * column 16*nt + l%16, rows k0..k0+7 with k0 = 128*kt + 32*w + 8*(l/16),
 * nibble p = row k0 + [0,2,4,6,1,3,5,7][p].  Rows >= K and columns >= N
 * hold 0.
 * Scales s: [ceil(N/16)][K/G][16] in the scale dtype (0 past N).
 * Zeros  z: [ceil(N/16)][K/G] uint64, nibble c = zero point of column 16*nt+c.
 * All three buffers must be 16-byte aligned.                               */
int64_t awq_repacked_weight_bytes(int64_t K, int64_t N);
int64_t awq_repacked_scale_bytes(int64_t K, int64_t N, int64_t G);
int64_t awq_repacked_zero_bytes(int64_t K, int64_t N, int64_t G);
int awq_repack_cdna4(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype,
                     int64_t K, int64_t N, int64_t G, void* w_out, void* s_out, void* z_out,
                     awq_stream_t stream);

/* Inverse of awq_repack_cdna4 (checkpoint export and round-trip checks). */
int awq_unrepack_cdna4(const void* w, const void* s, const void* z, int dtype, int64_t K, int64_t N,
                       int64_t G, int32_t* qweight_out, int32_t* qzeros_out, void* scales_out,
                       awq_stream_t stream);

/* ---- dequantisation --------------------------------------------------------
 * W[k, n] = rnd((q - z) * s) for AWQ tensors, the arithmetic of
 * python/sglite/srt/model_executor/layers/quantization/awq_triton.py:119-122,
 * written to w_out [K, N] in the scale dtype (bit-exact probe). */
int awq_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype,
                int64_t K, int64_t N, int64_t G, void* w_out, awq_stream_t stream);

/* Same result from the repacked buffers, computed by Dq<>::word, the
 * dequantisation routine of the prefill kernels (tiled_kernel, mfma32_kernel),
 * the k-slice decode kernel, the grouped MoE kernel and the bf16 GEMV path
 * (proves their in-kernel dequantisation is bit-exact).  The fp16 decode paths feed the MFMAs the exact integers q - z
 * (GEMV, 4+ rows) or the biased nibbles 1024 + q (GEMV up to 3 rows and the
 * skinny kernel) and apply the group scale to the fp32 sums instead; their
 * outputs are checked against the oracle within the GEMM tolerance. */
int awq_dequant_repacked(const void* w, const void* s, const void* z, int dtype, int64_t K, int64_t N,
                         int64_t G, void* w_out, awq_stream_t stream);

/* ---- W4A16 GEMM ------------------------------------------------------------
 * out[M, N] = rnd(x[M, K] @ W) (+ bias[N] in the activation dtype), fp32
 * accumulation; bias (if any) must be 8-byte aligned.  Replaces awq_gemm_triton
 * (python/sglite/srt/model_executor/layers/quantization/awq_triton.py:144-195,
 * called from awq.py:141-147) and gptq_marlin_gemm + bias
 * (python/sglite/srt/model_executor/layers/quantization/marlin_utils.py:388-415).
 *
 * Split-K scratch: `ws` must hold awq_workspace_bytes(M, N, K, G) bytes (any
 * content; may be NULL when that is 0).  `counters` (int32, counter_bytes
 * long, 128-byte aligned) must hold at least awq_counter_bytes(N) bytes that
 * are zero before the first call on them; every call leaves them valid for
 * the next (the decode kernels' per-column-tile counters zero again, the
 * tiled kernels' split-tile counters advanced consistently), whatever shape
 * the next call has.  A buffer sized for the largest N may be shared by
 * every linear of a stream.  Both are checked whenever the plan splits K
 * (AWQ_STATUS_WORKSPACE if missing or short); the tiled kernels (kind 1)
 * accept NULL counters and then sum their k-slices in a second kernel
 * instead of in the GEMM kernel itself.  Calls sharing `counters` must not run
 * concurrently (use one counters buffer per stream).
 * Layout: AWQ_COUNTER_TILE_BYTES of split-tile counters (32 words per output
 * tile of a split tiled plan, at most 512 tiles), then one int32 per
 * 16-column tile. */
#define AWQ_COUNTER_TILE_BYTES (64ll << 10)
int64_t awq_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t G);
/* Which kernel awq_w4a16_gemm runs for this shape: 0 = decode split-K kernel,
 * 1 = tiled MFMA kernel, 2 = small-batch GEMV kernel, 3 = k-slice decode
 * kernel (benchmarks and diagnostics; no counterpart in the reference). */
int awq_gemm_kernel_kind(int64_t M, int64_t N, int64_t K, int64_t G);
int64_t awq_counter_bytes(int64_t N);
int awq_w4a16_gemm(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                   int64_t M, int64_t N, int64_t K, int64_t G, int dtype,
                   void* ws, int64_t ws_bytes, int32_t* counters, int64_t counter_bytes, awq_stream_t stream);

/* ---- W4A16 GEMM that allocates nothing --------------------------------------
 * Same plan, kernels and result as awq_w4a16_gemm (bit-identical output), but
 * the split-K workspace and arrival counters live in a static device array of
 * the library (AWQ_NOALLOC_WORKSPACE_BYTES of workspace plus counters for N up
 * to AWQ_NOALLOC_MAX_N columns, held on every device the library runs on
 * until the process ends).  For callers that cannot allocate device memory:
 * code being captured into a HIP graph, tight serving loops, harnesses that
 * forbid hipMalloc.  The caller passes inputs and outputs only; the call
 * makes no hipMalloc/hipFree and no allocating library call.  Shapes whose
 * workspace exceeds the scratch return AWQ_STATUS_UNSUPPORTED.  All calls on
 * one device share its scratch: calls that overlap in time on one device
 * (concurrent streams or threads) race and must be serialised by the caller.
 * No counterpart in the reference. */
#define AWQ_NOALLOC_WORKSPACE_BYTES (64ll << 20)
#define AWQ_NOALLOC_MAX_N (1ll << 20)
/* Resolve the current device's scratch and clear its counters on `stream`
 * (a fill kernel, no allocation).  Optional: the first awq_w4a16_gemm_noalloc
 * call on a device does the same, and if that call is being captured into a
 * graph the fill kernel becomes a node of the graph.  Call it once per device
 * before capturing to keep the graph free of it. */
int awq_noalloc_init(awq_stream_t stream);
int awq_w4a16_gemm_noalloc(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                           int64_t M, int64_t N, int64_t K, int64_t G, int dtype, awq_stream_t stream);

/* ---- W4A16 GEMM with the gated activation fused ----------------------------
 * out[M, N/2] = act(gate) * up, where [gate | up] = x[M, K] @ W (+ bias[N]) are
 * the two column halves of a merged gate_up projection (gate columns first,
 * MergedColumnParallelLinear of layers/linear.py:127-143).  Each half is
 * rounded to the activation dtype (bias added in that dtype) exactly as
 * awq_w4a16_gemm stores it, then act(gate) * up is computed in fp32 and
 * rounded once: GatedMLP.forward's gate_up_proj + act_fn
 * (python/sglite/srt/model_executor/models/blocks.py:51-57; silu_and_mul /
 * gelu_and_mul of layers/activation.py:11-23) without the [M, N]
 * intermediate or its second launch.  N % 32 == 0; out 8-byte aligned.
 * Workspace and counters as for awq_w4a16_gemm, sized by
 * awq_workspace_bytes_act; awq_gemm_kernel_kind_act names the kernel it runs
 * (codes as for awq_gemm_kernel_kind).  No counterpart in the reference: a
 * fusion of two of its calls. */
enum { AWQ_ACT_SILU = 1, AWQ_ACT_GELU = 2 };
int64_t awq_workspace_bytes_act(int64_t M, int64_t N, int64_t K, int64_t G);
int awq_gemm_kernel_kind_act(int64_t M, int64_t N, int64_t K, int64_t G);
int awq_w4a16_gemm_act(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                       int64_t M, int64_t N, int64_t K, int64_t G, int dtype, int activation, void* ws,
                       int64_t ws_bytes, int32_t* counters, int64_t counter_bytes, awq_stream_t stream);

/* ---- gated MLP block in one launch -------------------------------------------
 * out[M, H] = down(act(x @ W_gate) * (x @ W_up)) for decode batches: the
 * GatedMLP forward (python/sglite/srt/model_executor/models/blocks.py:51-57:
 * gate_up_proj, silu_and_mul / gelu_and_mul, down_proj) as one kernel whose
 * down-projection weight loads are issued before the gate/up outputs exist.
 *   x        [M, H], 16-byte aligned; out [M, H], 8-byte aligned
 *   gu_*     the merged gate/up projection repacked as K = H, N = 2I (gate
 *            columns first, then up: MergedColumnParallelLinear's layout)
 *   dn_*     the down projection repacked as K = I, N = H
 *   G == 128, no bias; each gate / up value is rounded to the dtype and
 *   act(gate) * up rounded once, as awq_w4a16_gemm_act stores it, and the
 *   down projection's fp32 k-slice sums are added in a fixed order.
 *   ws       awq_gated_mlp_workspace_bytes bytes, 256-byte aligned
 *   counters AWQ_MLP_COUNTER_BYTES bytes, 128-byte aligned, zero before the
 *            first call and then left alone (every call leaves them valid
 *            for the next; calls that share them must be stream-ordered)
 *   polls    how often a workgroup polls the arrival count of its k-slice of
 *            the intermediate (the workgroups that write that slice) before
 *            it gives up (negative: AWQ_MLP_DEFAULT_POLLS; 0: only each
 *            slice's last arrival proceeds).  A workgroup that gives up counts
 *            itself in word 2 of the counters and skips the down projection;
 *            every workgroup still exits and the counters stay valid, but
 *            that call's output is wrong: awq_gated_mlp_take_errors reports it.
 * The grid is one workgroup per CU at most, never more than the device's
 * occupancy query for the kernel allows at once, so on an otherwise idle
 * device no wait lasts longer than the slowest workgroup's gate/up work.
 * Shapes outside the built forms (M > 16, H > 4096, I / 16 tiles beyond four
 * per workgroup, ...) return AWQ_STATUS_UNSUPPORTED: awq_gated_mlp_plan
 * tells beforehand, and the caller runs awq_w4a16_gemm_act and
 * awq_w4a16_gemm instead.  No counterpart in the reference: a fusion of its
 * GatedMLP calls. */
#define AWQ_MLP_COUNTER_BYTES (64ll << 10)
#define AWQ_MLP_DEFAULT_POLLS (1 << 15)
/* 1 if awq_gated_mlp runs this shape on the current device, 0 if not;
 * info (8 entries, may be null): workgroups, down k-slices, down column tiles
 * per group, column groups, gate tiles per workgroup, down k-tiles per slice,
 * LDS bytes, workspace bytes. */
int awq_gated_mlp_plan(int64_t M, int64_t H, int64_t I, int64_t G, int dtype, int64_t* info);
int64_t awq_gated_mlp_workspace_bytes(int64_t M, int64_t H, int64_t I, int64_t G, int dtype);
int awq_gated_mlp(const void* x, const void* gu_w, const void* gu_s, const void* gu_z, const void* dn_w,
                  const void* dn_s, const void* dn_z, void* out, int64_t M, int64_t H, int64_t I, int64_t G, int dtype,
                  int activation, int polls, void* ws, int64_t ws_bytes, int32_t* counters, int64_t counter_bytes,
                  awq_stream_t stream);
/* Synchronizes `stream`, returns the number of workgroups that gave up
 * waiting since the last call (>= 0) and clears the count.  Not while the
 * stream is being captured. */
int64_t awq_gated_mlp_take_errors(int32_t* counters, int64_t counter_bytes, awq_stream_t stream);

/* ---- planner overrides (tests and sweeps) -----------------------------------
 * Force a kernel choice or split for every later GEMM of the process (all
 * threads), e.g. to run each kernel instantiation against the oracle.  The
 * planner's own choice is best for serving; the overrides are off by default
 * and never read from the environment.  Shape codes that are not
 * instantiated are ignored.  No counterpart in the reference.
 *   AWQ_PLAN_GEMV_MAX_M      largest M routed to the GEMV kernel (0 disables it)
 *   AWQ_PLAN_GEMV_VARIANT    GEMV shape ntw*10000 + wn*1000 + wk*10 + kpw
 *   AWQ_PLAN_GEMV_KS         GEMV k-slices across workgroups
 *   AWQ_PLAN_SKINNY_VARIANT  decode-kernel shape ntw*10000 + wn*100 + wk
 *   AWQ_PLAN_SKINNY_KS       decode-kernel k-slices
 *   AWQ_PLAN_TILED_MIN_M     smallest M routed to the tiled kernel
 *   AWQ_PLAN_TILED_BM        tiled row-block code: 32, 64, 128 (16x16x32 MFMA
 *                            kernel); 1064, 1128, 2064, 2128, 4032 (32x32x16
 *                            MFMA kernel at 64/128/32 rows with registers for
 *                            1, 2 or 4 workgroups per CU); 8064, 8128 (its
 *                            8-wave, 512-column form); 9064, 9128 (its 8-wave
 *                            k-wave-split form at 64/128 rows, only with
 *                            G >= 64)
 *   AWQ_PLAN_TILED_KS        tiled k-slices
 *   AWQ_PLAN_KSLICE_VARIANT  k-slice decode-kernel shape wn*100 + wk*10 + kpw
 *                            (M <= 32; any other value leaves the plan alone;
 *                            the planner itself does not choose this kernel)
 *   AWQ_PLAN_TILED_FIXUP     1: split-K tiled plans sum their k-slices inside
 *                            the GEMM kernel when the counters are given
 *                            (default 0: in a second kernel)
 *   AWQ_PLAN_FIXUP_POLLS     how often a k-slice workgroup polls for its
 *                            tile's other slices before it leaves the sum to
 *                            the last one (0: never waits) */
enum {
  AWQ_PLAN_GEMV_MAX_M = 0,
  AWQ_PLAN_GEMV_VARIANT = 1,
  AWQ_PLAN_GEMV_KS = 2,
  AWQ_PLAN_SKINNY_VARIANT = 3,
  AWQ_PLAN_SKINNY_KS = 4,
  AWQ_PLAN_TILED_MIN_M = 5,
  AWQ_PLAN_TILED_BM = 6,
  AWQ_PLAN_TILED_KS = 7,
  AWQ_PLAN_KSLICE_VARIANT = 8,
  AWQ_PLAN_TILED_FIXUP = 9,
  AWQ_PLAN_FIXUP_POLLS = 10
};
int awq_set_plan_override(int knob, int value);
void awq_clear_plan_overrides(void);

/* Compute units of the current device that the planner fills (queried once
 * per device; 256 when no device is visible).  No counterpart in the
 * reference. */
int awq_device_cu_count(void);

/* ---- diagnostics and measurement (no counterpart in the reference) ---------
 * awq_gemm_plan_info: the plan that awq_w4a16_gemm (activation 0) or
 * awq_w4a16_gemm_act (AWQ_ACT_SILU / AWQ_ACT_GELU) runs for this shape on the
 * current device, written to info[0..5]: kernel kind (as
 * awq_gemm_kernel_kind), shape code, k-slices across workgroups, workgroups
 * per launch, threads per workgroup, workspace bytes.
 *
 * awq_stream_probe: streams `bytes` (a multiple of 16, src 16-byte aligned)
 * with `grid` workgroups of `block` threads (64..1024, a multiple of 64),
 * every thread issuing all its 16-byte loads before consuming them, and
 * stores one word per workgroup to sink (sink_bytes >= 4 * grid).  Timed with
 * a GEMM's own grid and block size and its weight bytes, it gives the rate a
 * launch of that shape can reach at all (the decode roofline's attainable
 * ceiling). */
int awq_gemm_plan_info(int64_t M, int64_t N, int64_t K, int64_t G, int activation, int64_t* info);
/* 1 if that plan splits K on the tiled kernels and sums the k-slices inside
 * the GEMM kernel (when awq_w4a16_gemm is given counters), 0 otherwise. */
int awq_gemm_plan_fixup(int64_t M, int64_t N, int64_t K, int64_t G, int activation);
int awq_stream_probe(const void* src, int64_t bytes, int64_t grid, int block, uint32_t* sink, int64_t sink_bytes,
                     awq_stream_t stream);
/* awq_mfma_probe: `grid` workgroups of `block` threads (64..256), each wave
 * running `iters` rounds of eight independent v_mfma_f32_32x32x16_f16 on
 * register operands (8 x 32768 flops per round and wave), one float per wave
 * to sink (sink_bytes >= 4 * grid *
 * block / 64): the dense fp16 MFMA rate the device sustains as clocked, the
 * prefill roofline's attainable ceiling. */
int awq_mfma_probe(int64_t iters, int64_t grid, int block, float* sink, int64_t sink_bytes, awq_stream_t stream);

/* ---- grouped MoE -------------------------------------------------------------
 * The stages of the fused MoE backend
 * (python/sglite/srt/model_executor/layers/fused_moe/fused.py:101-202) with AWQ
 * expert weights.  Experts are stacked: expert e's repacked weights, scales
 * and zeros (awq_repack_cdna4 of that expert) start at e times the strides
 * awq_moe_expert_strides reports (each buffer's per-expert size rounded up to
 * 256 bytes).  A routed row is r = t * topk + j (token t, slot j). */

int awq_moe_expert_strides(int64_t K, int64_t N, int64_t G, int64_t* w_stride, int64_t* s_stride,
                           int64_t* z_stride);

/* softmax(gating_output[T, E]) -> top-k -> optionally w / (sum(w) + 1e-8);
 * replaces sgl_kernel.topk_softmax and the renormalisation of fused.py:11-31.
 * Ties go to the lower expert index.  E <= 512, 1 <= topk <= min(E, 64). */
int awq_moe_topk_softmax(const float* gating_output, float* topk_weights, int32_t* topk_ids, int64_t T,
                         int64_t E, int64_t topk, int renormalize, awq_stream_t stream);

/* Sorts the routed rows by expert (stable) and pads each expert's bucket to a
 * multiple of block_size with the sentinel numel; replaces
 * moe_align_block_size (fused.py:34-61, sgl_kernel's align kernel).
 *   sorted_ids[awq_moe_sorted_capacity(numel, E, block_size)]
 *   expert_ids[awq_moe_block_capacity(numel, E, block_size)]  (-1 past the end)
 *   num_tokens_post_pad[1], expert_offsets[E + 1] (padded bucket starts)
 * Ids outside [0, E) are dropped.  block_size % 16 == 0, E <= 512,
 * numel < 2^24. */
int64_t awq_moe_sorted_capacity(int64_t numel, int64_t E, int64_t block_size);
int64_t awq_moe_block_capacity(int64_t numel, int64_t E, int64_t block_size);
int awq_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t E, int64_t block_size,
                             int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_tokens_post_pad,
                             int32_t* expert_offsets, awq_stream_t stream);

enum { AWQ_MOE_ACT_NONE = 0, AWQ_MOE_ACT_SILU = 1, AWQ_MOE_ACT_GELU = 2 };

/* Grouped W4A16 GEMM over the expert buckets; replaces fused_moe_kernel
 * (python/sglite/kernels/triton/fused_moe.py:54-183, launched by
 * python/sglite/kernels/moe_triton.py:8-65) for AWQ B operands.
 *   a        [a_rows, K]; routed row r reads activation row r / top_k
 *            (top_k = topk for the first GEMM, 1 for the second, as in
 *            moe_triton.py's `top_k` argument)
 *   w/s/z    expert-stacked repacked weights of [K, N] per expert
 *   out      activation == AWQ_MOE_ACT_NONE: [num_routed, N], row r
 *            activation != NONE: N = 2I (gate columns first, then up), the
 *            gate/up outputs are rounded and combined as
 *            act(gate) * up -> [num_routed, I] (silu_and_mul / gelu_and_mul of
 *            python/sglite/srt/model_executor/layers/activation.py:11-23);
 *            needs I % 16 == 0
 *   mul_routed_weight: multiply by topk_weights[r] (fp32) before the cast
 *            (MUL_ROUTED_WEIGHT, triton/fused_moe.py:174-178)
 * Rows of padding (id >= num_routed) are skipped. */
int awq_moe_w4a16_gemm(const void* a, int64_t a_rows, const void* w, const void* s, const void* z, int64_t E,
                       int64_t N, int64_t K, int64_t G, int dtype, const int32_t* sorted_ids, int64_t sorted_cap,
                       const int32_t* expert_offsets, const float* topk_weights, int64_t num_routed, int64_t top_k,
                       int activation, int mul_routed_weight, void* out, awq_stream_t stream);

/* out[t, :] = rnd(sum_j in[t, j, :]) with an fp32 sum; replaces
 * moe_sum_reduce_triton (python/sglite/kernels/moe_triton.py:68-102).
 * H % 8 == 0; in and out 16-byte aligned. */
int awq_moe_sum_reduce(const void* in, void* out, int64_t T, int64_t topk, int64_t H, int dtype,
                       awq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SGLITE_AWQ_H */
