/*
 * sglite_awq.h -- C ABI of the MI355X (gfx950) AWQ W4A16 linear engine.
 *
 * Plain pointers and sizes only.  Every entry point that launches work takes
 * the caller's HIP stream, enqueues asynchronously and never synchronises the
 * device, allocates no device memory and takes no host-dependent decision
 * from device data, so it may be recorded into a HIP graph.  Every function
 * returning int returns 0 on success or a negative AWQ_STATUS_* code; the
 * message of the last failure on the calling thread is awq_last_error().
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

/* Library version string, e.g. "sglite-awq-gfx950 0.1". */
const char* awq_version(void);

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

/* Same result from the repacked buffers, computed by the device routine the
 * GEMM kernels use (proves the in-kernel dequantisation is bit-exact). */
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
 * content; may be NULL when that is 0).  `counters` must hold
 * awq_counter_bytes(N) bytes that are zero before the first call on them;
 * every call leaves them zero again.  Calls sharing `counters` must not run
 * concurrently (use one counters buffer per stream). */
int64_t awq_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t G);
int64_t awq_counter_bytes(int64_t N);
int awq_w4a16_gemm(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                   int64_t M, int64_t N, int64_t K, int64_t G, int dtype,
                   void* ws, int64_t ws_bytes, int32_t* counters, awq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SGLITE_AWQ_H */
