// C ABI of the AWQ W4A16 engine (declared in include/sglite_awq.h).
//
// Argument validation mirrors the reference's checks and turns each into a
// status code plus a thread-local message instead of a Python exception:
//   group size in {-1, 32, 64, 128} or == K
//     (layers/quantization/awq_triton.py:159-166, marlin_utils.py:86-88)
//   K % G == 0, N % 8 == 0 (layers/quantization/awq.py:76-85)
// The Python wrapper raises ValueError for AWQ_STATUS_INVALID_ARGUMENT and
// RuntimeError otherwise.
#include <rocprofiler-sdk-roctx/roctx.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/sglite_awq.h"
#include "awq_epilogue.h"
#include "awq_fixup.h"
#include "awq_launch.h"

using namespace sgl_awq;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return AWQ_STATUS_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(AWQ_STATUS_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// Shape rules shared by every entry point.  On success *G_out holds the
// resolved group size.
int check_shape(int64_t K, int64_t N, int64_t G, int dtype, int64_t* G_out) {
  if (dtype != AWQ_DTYPE_FP16 && dtype != AWQ_DTYPE_BF16)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "dtype must be AWQ_DTYPE_FP16 (0) or AWQ_DTYPE_BF16 (1), got %d", dtype);
  if (K <= 0 || N <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "K and N must be positive (K=%lld, N=%lld)",
                                    (long long)K, (long long)N);
  if (K >= (int64_t(1) << 24) || N >= (int64_t(1) << 30))
    return fail(AWQ_STATUS_UNSUPPORTED, "K must be below 2^24 and N below 2^30 (K=%lld, N=%lld)", (long long)K,
                (long long)N);
  const int64_t Gr = (G == -1) ? K : G;
  if (!(Gr == 32 || Gr == 64 || Gr == 128 || Gr == K))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "group size must be -1, 32, 64, 128 or K, got %lld", (long long)G);
  if (K % Gr != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "The input size is not aligned with the quantized weight shape (K=%lld, group size %lld).",
                (long long)K, (long long)Gr);
  if (K % 32 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "K must be a multiple of 32, got %lld", (long long)K);
  if (N % 8 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "The output size is not aligned with the quantized weight shape (N=%lld, pack factor 8).",
                (long long)N);
  *G_out = Gr;
  return AWQ_STATUS_OK;
}

// Split-K counters (awq_counter_bytes): the split tiles' counters of the
// tiled kernels' in-kernel reduction (kFixupBytes), then one int32 per column
// tile for the GEMV and decode kernels.  The tiled kernels take them when
// given (else a second kernel sums the k-slices); the others need them.
constexpr int64_t counter_bytes_for(int64_t N) { return kFixupBytes + ((N + 15) / 16) * 4; }
static_assert(AWQ_COUNTER_TILE_BYTES == kFixupBytes, "header and kernels agree on the tile counters");
static_assert(AWQ_MLP_COUNTER_BYTES == kMlpCounterBytes && AWQ_MLP_DEFAULT_POLLS == kMlpDefaultPolls,
              "header and kernel agree on the gated MLP counters");

int check_counters(const GemmPlan& p, int64_t N, const int32_t* counters, int64_t counter_bytes, const char* who) {
  if (p.kind == 1) {
    if (counters && !aligned(counters, 128))
      return fail(AWQ_STATUS_WORKSPACE, "%s: counters must be 128-byte aligned", who);
    return AWQ_STATUS_OK;
  }
  const int64_t need = counter_bytes_for(N);
  if (!counters) return fail(AWQ_STATUS_WORKSPACE, "%s: split-K needs the counters buffer", who);
  if (counter_bytes < need)
    return fail(AWQ_STATUS_WORKSPACE, "%s: counters of %lld bytes needed, %lld given", who, (long long)need,
                (long long)counter_bytes);
  if (!aligned(counters, 128)) return fail(AWQ_STATUS_WORKSPACE, "%s: counters must be 128-byte aligned", who);
  return AWQ_STATUS_OK;
}

// Arguments of a plain GEMM call, checked; on success (and M > 0) the
// geometry and plan.
int gemm_prepare(const void* x, const void* w, const void* s, const void* z, const void* bias, const void* out,
                 int64_t M, int64_t N, int64_t K, int64_t G, int dtype, const char* who, Geom* g, GemmPlan* p) {
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (M < 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be non-negative, got %lld", (long long)M);
  if (M == 0) return ok();
  if (M > (int64_t(1) << 24)) return fail(AWQ_STATUS_UNSUPPORTED, "M must be below 2^24, got %lld", (long long)M);
  if (!x || !w || !s || !z || !out) return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: null pointer argument", who);
  if (!aligned(x, 16)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: x must be 16-byte aligned", who);
  if (!aligned(out, 8)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: out must be 8-byte aligned", who);
  if (!aligned(w, 16) || !aligned(s, 16) || !aligned(z, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: repacked buffers must be 16-byte aligned", who);
  if (bias && !aligned(bias, 8)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: bias must be 8-byte aligned", who);
  *g = make_geom(M, N, K, Gr);
  *p = plan_gemm(*g);
  return AWQ_STATUS_OK;
}

// ---- static scratch of awq_w4a16_gemm_noalloc ------------------------------
// The split-K workspace (kScratchWsBytes) followed by the counters
// (kScratchCounterBytes: the split tiles' counters, then one int32 per column
// tile for up to AWQ_NOALLOC_MAX_N columns), in device memory that exists
// from the code object's load to the end of the process, one copy per
// device.  In host code `scratch` names a host-side stand-in, never the device
// memory: the device address comes from hipGetSymbolAddress, once per device,
// and only that address is handed to kernels.
constexpr int64_t kScratchWsBytes = AWQ_NOALLOC_WORKSPACE_BYTES;
constexpr int64_t kScratchCounterBytes = kFixupBytes + AWQ_NOALLOC_MAX_N / 16 * 4;
static_assert(kScratchWsBytes % 256 == 0, "the counters start 256-byte aligned");
static_assert(kScratchCounterBytes == counter_bytes_for(AWQ_NOALLOC_MAX_N), "scratch counters cover AWQ_NOALLOC_MAX_N columns");
static __device__ __align__(256) unsigned char scratch[kScratchWsBytes + kScratchCounterBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kScratchDevices];

__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Device address of the current device's scratch.  The first call on a device
// resolves it and clears the counters on `stream` with a fill kernel (they
// also start zeroed from the code object's zero-filled data); when `stream`
// is being captured into a graph the fill kernel becomes a node of the graph
// and runs ahead of the GEMM at every replay.  Every GEMM leaves the counters
// in a valid state for the next (awq_fixup.h; the decode kernels' are left
// zero).  awq_noalloc_init does the same ahead of any capture.
int scratch_base(hipStream_t stream, char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(AWQ_STATUS_HIP_ERROR, "hipGetDevice failed");
  if (dev < 0 || dev >= kScratchDevices)
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_w4a16_gemm_noalloc: device %d beyond the %d supported", dev,
                kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(AWQ_STATUS_HIP_ERROR, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    const int64_t n = kScratchCounterBytes / 4;
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       (uint32_t*)((char*)ptr + kScratchWsBytes), n);
    const hipError_t le = hipGetLastError();
    if (le != hipSuccess) return fail(AWQ_STATUS_HIP_ERROR, "scratch clear launch: %s", hipGetErrorString(le));
    g_scratch_ptr[dev] = (char*)ptr;
  }
  *out = g_scratch_ptr[dev];
  return AWQ_STATUS_OK;
}

// A roctx range around each compute entry point, named after it: the call
// shows in a rocprofv3 --marker-trace and encloses the kernels it launches
// (the per-op ranges the reference's nvtx_annotate gives its layers,
// utils/torch_utils.py:26-44).  Without a tool attached a push/pop pair is a
// few tens of nanoseconds.
struct TraceRange {
  explicit TraceRange(const char* name) { roctxRangePushA(name); }
  ~TraceRange() { roctxRangePop(); }
  TraceRange(const TraceRange&) = delete;
  TraceRange& operator=(const TraceRange&) = delete;
};

}  // namespace

extern "C" {

const char* awq_last_error(void) { return g_last_error.c_str(); }

const char* awq_version(void) { return "sglite-awq-gfx950 0.4"; }

int awq_abi_version(void) { return AWQ_ABI_VERSION; }

int64_t awq_repacked_weight_bytes(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "K and N must be positive");
  return ((N + 15) / 16) * ((K + 127) / 128) * 1024;
}

int64_t awq_repacked_scale_bytes(int64_t K, int64_t N, int64_t G) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  return ((N + 15) / 16) * (K / Gr) * 16 * 2;
}

int64_t awq_repacked_zero_bytes(int64_t K, int64_t N, int64_t G) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  return ((N + 15) / 16) * (K / Gr) * 8;
}

int awq_repack_cdna4(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype, int64_t K,
                     int64_t N, int64_t G, void* w_out, void* s_out, void* z_out, awq_stream_t stream) {
  const TraceRange range("awq_repack_cdna4");
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (!qweight || !qzeros || !scales || !w_out || !s_out || !z_out)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_repack_cdna4: null pointer argument");
  if (!aligned(w_out, 16) || !aligned(s_out, 16) || !aligned(z_out, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_repack_cdna4: output buffers must be 16-byte aligned");
  const Geom g = make_geom(0, N, K, Gr);
  return hip_status(launch_repack(qweight, qzeros, scales, dtype, g, w_out, s_out, z_out, (hipStream_t)stream),
                    "awq_repack_cdna4 launch");
}

int awq_unrepack_cdna4(const void* w, const void* s, const void* z, int dtype, int64_t K, int64_t N, int64_t G,
                       int32_t* qweight_out, int32_t* qzeros_out, void* scales_out, awq_stream_t stream) {
  const TraceRange range("awq_unrepack_cdna4");
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (!w || !s || !z || !qweight_out || !qzeros_out || !scales_out)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_unrepack_cdna4: null pointer argument");
  if (!aligned(w, 16) || !aligned(s, 16) || !aligned(z, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_unrepack_cdna4: repacked buffers must be 16-byte aligned");
  const Geom g = make_geom(0, N, K, Gr);
  return hip_status(
      launch_unrepack(w, s, z, dtype, g, qweight_out, qzeros_out, scales_out, (hipStream_t)stream),
      "awq_unrepack_cdna4 launch");
}

int awq_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, int dtype, int64_t K, int64_t N,
                int64_t G, void* w_out, awq_stream_t stream) {
  const TraceRange range("awq_dequant");
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (!qweight || !qzeros || !scales || !w_out)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_dequant: null pointer argument");
  const Geom g = make_geom(0, N, K, Gr);
  return hip_status(launch_dequant_awq(qweight, qzeros, scales, dtype, g, w_out, (hipStream_t)stream),
                    "awq_dequant launch");
}

int awq_dequant_repacked(const void* w, const void* s, const void* z, int dtype, int64_t K, int64_t N, int64_t G,
                         void* w_out, awq_stream_t stream) {
  const TraceRange range("awq_dequant_repacked");
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (!w || !s || !z || !w_out)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_dequant_repacked: null pointer argument");
  if (!aligned(w, 16) || !aligned(s, 16) || !aligned(z, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_dequant_repacked: repacked buffers must be 16-byte aligned");
  const Geom g = make_geom(0, N, K, Gr);
  return hip_status(launch_dequant_repacked(w, s, z, dtype, g, w_out, (hipStream_t)stream),
                    "awq_dequant_repacked launch");
}

int64_t awq_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t G) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (M < 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be non-negative");
  if (M == 0) return 0;
  return plan_gemm(make_geom(M, N, K, Gr)).ws_bytes;
}

int awq_gemm_kernel_kind(int64_t M, int64_t N, int64_t K, int64_t G) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (M <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be positive");
  return plan_gemm(make_geom(M, N, K, Gr)).kind;
}

int64_t awq_counter_bytes(int64_t N) {
  if (N <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "N must be positive");
  return counter_bytes_for(N);
}

int awq_w4a16_gemm(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                   int64_t M, int64_t N, int64_t K, int64_t G, int dtype, void* ws, int64_t ws_bytes,
                   int32_t* counters, int64_t counter_bytes, awq_stream_t stream) {
  const TraceRange range("awq_w4a16_gemm");
  Geom g;
  GemmPlan p;
  int st = gemm_prepare(x, w, s, z, bias, out, M, N, K, G, dtype, "awq_w4a16_gemm", &g, &p);
  if (st != 0 || M == 0) return st;
  if (p.ws_bytes > 0) {
    if (!ws || ws_bytes < p.ws_bytes)
      return fail(AWQ_STATUS_WORKSPACE, "awq_w4a16_gemm: workspace of %lld bytes needed, %lld given",
                  (long long)p.ws_bytes, (long long)(ws ? ws_bytes : 0));
    if (!aligned(ws, 16)) return fail(AWQ_STATUS_WORKSPACE, "awq_w4a16_gemm: workspace must be 16-byte aligned");
    st = check_counters(p, N, counters, counter_bytes, "awq_w4a16_gemm");
    if (st != 0) return st;
  }
  return hip_status(launch_gemm(p, x, w, s, z, bias, out, dtype, g, ws, counters, counters ? counter_bytes : 0,
                                kActNone, (hipStream_t)stream),
                    "awq_w4a16_gemm launch");
}

int awq_noalloc_init(awq_stream_t stream) {
  const TraceRange range("awq_noalloc_init");
  char* base = nullptr;
  const int st = scratch_base((hipStream_t)stream, &base);
  return st != 0 ? st : ok();
}

int awq_w4a16_gemm_noalloc(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                           int64_t M, int64_t N, int64_t K, int64_t G, int dtype, awq_stream_t stream) {
  const TraceRange range("awq_w4a16_gemm_noalloc");
  Geom g;
  GemmPlan p;
  int st = gemm_prepare(x, w, s, z, bias, out, M, N, K, G, dtype, "awq_w4a16_gemm_noalloc", &g, &p);
  if (st != 0 || M == 0) return st;
  void* ws = nullptr;
  int32_t* counters = nullptr;
  if (p.ws_bytes > 0) {
    if (p.ws_bytes > kScratchWsBytes)
      return fail(AWQ_STATUS_UNSUPPORTED,
                  "awq_w4a16_gemm_noalloc: this shape's split-K workspace (%lld bytes) exceeds the static scratch "
                  "of %lld bytes; use awq_w4a16_gemm with a caller workspace",
                  (long long)p.ws_bytes, (long long)kScratchWsBytes);
    if (p.kind != 1 && N > AWQ_NOALLOC_MAX_N)
      return fail(AWQ_STATUS_UNSUPPORTED, "awq_w4a16_gemm_noalloc: N = %lld exceeds the static counters' %lld columns",
                  (long long)N, (long long)AWQ_NOALLOC_MAX_N);
    char* base = nullptr;
    st = scratch_base((hipStream_t)stream, &base);
    if (st != 0) return st;
    ws = base;
    counters = (int32_t*)(base + kScratchWsBytes);
  }
  return hip_status(launch_gemm(p, x, w, s, z, bias, out, dtype, g, ws, counters,
                                counters ? kScratchCounterBytes : 0, kActNone, (hipStream_t)stream),
                    "awq_w4a16_gemm_noalloc launch");
}

int64_t awq_workspace_bytes_act(int64_t M, int64_t N, int64_t K, int64_t G) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (M < 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be non-negative");
  if (N % 32 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "a gate/up projection needs N %% 32 == 0, got %lld", (long long)N);
  if (M == 0) return 0;
  return plan_gemm(make_geom(M, N, K, Gr), kActSilu).ws_bytes;
}

int awq_gemm_kernel_kind_act(int64_t M, int64_t N, int64_t K, int64_t G) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (M <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be positive");
  if (N % 32 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "a gate/up projection needs N %% 32 == 0, got %lld", (long long)N);
  return plan_gemm(make_geom(M, N, K, Gr), kActSilu).kind;
}

int awq_w4a16_gemm_act(const void* x, const void* w, const void* s, const void* z, const void* bias, void* out,
                       int64_t M, int64_t N, int64_t K, int64_t G, int dtype, int activation, void* ws,
                       int64_t ws_bytes, int32_t* counters, int64_t counter_bytes, awq_stream_t stream) {
  const TraceRange range("awq_w4a16_gemm_act");
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (activation != AWQ_ACT_SILU && activation != AWQ_ACT_GELU)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_w4a16_gemm_act: activation must be AWQ_ACT_SILU or AWQ_ACT_GELU, got %d",
                activation);
  if (N % 32 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "awq_w4a16_gemm_act: N must be a multiple of 32 (two halves of whole 16-column tiles), got %lld",
                (long long)N);
  if (M < 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be non-negative, got %lld", (long long)M);
  if (M == 0) return ok();
  if (M > (int64_t(1) << 24)) return fail(AWQ_STATUS_UNSUPPORTED, "M must be below 2^24, got %lld", (long long)M);
  if (!x || !w || !s || !z || !out)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_w4a16_gemm_act: null pointer argument");
  if (!aligned(x, 16)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_w4a16_gemm_act: x must be 16-byte aligned");
  if (!aligned(out, 8)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_w4a16_gemm_act: out must be 8-byte aligned");
  if (!aligned(w, 16) || !aligned(s, 16) || !aligned(z, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_w4a16_gemm_act: repacked buffers must be 16-byte aligned");
  if (bias && !aligned(bias, 8))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_w4a16_gemm_act: bias must be 8-byte aligned");
  const int act = activation == AWQ_ACT_SILU ? kActSilu : kActGelu;
  const Geom g = make_geom(M, N, K, Gr);
  const GemmPlan p = plan_gemm(g, act);
  if (p.ws_bytes > 0) {
    if (!ws || ws_bytes < p.ws_bytes)
      return fail(AWQ_STATUS_WORKSPACE, "awq_w4a16_gemm_act: workspace of %lld bytes needed, %lld given",
                  (long long)p.ws_bytes, (long long)(ws ? ws_bytes : 0));
    if (!aligned(ws, 16)) return fail(AWQ_STATUS_WORKSPACE, "awq_w4a16_gemm_act: workspace must be 16-byte aligned");
    const int st2 = check_counters(p, N, counters, counter_bytes, "awq_w4a16_gemm_act");
    if (st2 != 0) return st2;
  }
  return hip_status(launch_gemm(p, x, w, s, z, bias, out, dtype, g, ws, counters, counters ? counter_bytes : 0, act,
                                (hipStream_t)stream),
                    "awq_w4a16_gemm_act launch");
}

int awq_gated_mlp_plan(int64_t M, int64_t H, int64_t I, int64_t G, int dtype, int64_t* info) {
  int64_t Gr = 0;
  int st = check_shape(H, 2 * I, G, dtype, &Gr);
  if (st == 0) st = check_shape(I, H, G, dtype, &Gr);
  if (st != 0) return st;
  if (M <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be positive, got %lld", (long long)M);
  const MlpPlan p = plan_mlp(M, H, I, G, dtype);
  if (info) {
    const int64_t v[8] = {p.P, p.S, p.C, p.groups, p.npw, p.nk, p.lds, p.ws_bytes};
    for (int i = 0; i < 8; ++i) info[i] = p.ok ? v[i] : 0;
  }
  ok();
  return p.ok;
}

int64_t awq_gated_mlp_workspace_bytes(int64_t M, int64_t H, int64_t I, int64_t G, int dtype) {
  int64_t Gr = 0;
  int st = check_shape(H, 2 * I, G, dtype, &Gr);
  if (st == 0) st = check_shape(I, H, G, dtype, &Gr);
  if (st != 0) return st;
  const MlpPlan p = plan_mlp(M, H, I, G, dtype, /*query_device=*/false);
  if (!p.ok)
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_gated_mlp: M=%lld H=%lld I=%lld G=%lld is outside the built forms",
                (long long)M, (long long)H, (long long)I, (long long)G);
  ok();
  return p.ws_bytes;
}

int awq_gated_mlp(const void* x, const void* gu_w, const void* gu_s, const void* gu_z, const void* dn_w,
                  const void* dn_s, const void* dn_z, void* out, int64_t M, int64_t H, int64_t I, int64_t G, int dtype,
                  int activation, int polls, void* ws, int64_t ws_bytes, int32_t* counters, int64_t counter_bytes,
                  awq_stream_t stream) {
  const TraceRange range("awq_gated_mlp");
  const char* who = "awq_gated_mlp";
  int64_t Gr = 0;
  int st = check_shape(H, 2 * I, G, dtype, &Gr);
  if (st == 0) st = check_shape(I, H, G, dtype, &Gr);
  if (st != 0) return st;
  if (activation != AWQ_ACT_SILU && activation != AWQ_ACT_GELU)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: activation must be AWQ_ACT_SILU or AWQ_ACT_GELU, got %d", who,
                activation);
  if (M < 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "M must be non-negative, got %lld", (long long)M);
  if (M == 0) return ok();
  if (!x || !gu_w || !gu_s || !gu_z || !dn_w || !dn_s || !dn_z || !out)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: null pointer argument", who);
  if (!aligned(x, 16)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: x must be 16-byte aligned", who);
  if (!aligned(out, 8)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: out must be 8-byte aligned", who);
  if (!aligned(gu_w, 16) || !aligned(gu_s, 16) || !aligned(gu_z, 16) || !aligned(dn_w, 16) || !aligned(dn_s, 16) ||
      !aligned(dn_z, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: repacked buffers must be 16-byte aligned", who);
  const MlpPlan shape = plan_mlp(M, H, I, G, dtype, /*query_device=*/false);
  if (!shape.ok)
    return fail(AWQ_STATUS_UNSUPPORTED, "%s: M=%lld H=%lld I=%lld G=%lld is outside the built forms", who,
                (long long)M, (long long)H, (long long)I, (long long)G);
  if (!ws || ws_bytes < shape.ws_bytes)
    return fail(AWQ_STATUS_WORKSPACE, "%s: workspace of %lld bytes needed, %lld given", who,
                (long long)shape.ws_bytes, (long long)(ws ? ws_bytes : 0));
  if (!aligned(ws, 256)) return fail(AWQ_STATUS_WORKSPACE, "%s: workspace must be 256-byte aligned", who);
  if (!counters || counter_bytes < AWQ_MLP_COUNTER_BYTES)
    return fail(AWQ_STATUS_WORKSPACE, "%s: counters of %lld bytes needed, %lld given", who,
                (long long)AWQ_MLP_COUNTER_BYTES, (long long)(counters ? counter_bytes : 0));
  if (!aligned(counters, 128)) return fail(AWQ_STATUS_WORKSPACE, "%s: counters must be 128-byte aligned", who);
  const MlpPlan p = plan_mlp(M, H, I, G, dtype);
  if (!p.ok)
    return fail(AWQ_STATUS_UNSUPPORTED, "%s: the device does not keep the %lld-workgroup grid resident", who,
                (long long)shape.P);
  const int act = activation == AWQ_ACT_SILU ? kActSilu : kActGelu;
  return hip_status(launch_mlp(p, x, gu_w, gu_s, gu_z, dn_w, dn_s, dn_z, out, M, H, I, dtype, act, ws, counters,
                               polls < 0 ? kMlpDefaultPolls : polls, (hipStream_t)stream),
                    "awq_gated_mlp launch");
}

int64_t awq_gated_mlp_take_errors(int32_t* counters, int64_t counter_bytes, awq_stream_t stream) {
  const char* who = "awq_gated_mlp_take_errors";
  if (!counters || counter_bytes < AWQ_MLP_COUNTER_BYTES || !aligned(counters, 128))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: counters of %lld bytes, 128-byte aligned, needed", who,
                (long long)AWQ_MLP_COUNTER_BYTES);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess)
    return fail(AWQ_STATUS_HIP_ERROR, "%s: hipStreamIsCapturing failed", who);
  if (cs != hipStreamCaptureStatusNone)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "%s: the stream is being captured", who);
  int32_t n = 0;
  hipError_t e = hipMemcpyAsync(&n, counters + 2, 4, hipMemcpyDeviceToHost, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e == hipSuccess && n != 0) {
    const int32_t zero = 0;
    e = hipMemcpyAsync(counters + 2, &zero, 4, hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  }
  if (e != hipSuccess) return fail(AWQ_STATUS_HIP_ERROR, "%s: %s", who, hipGetErrorString(e));
  ok();
  return (int64_t)(uint32_t)n;
}

int awq_set_plan_override(int knob, int value) {
  if (!set_plan_override(knob, value))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_set_plan_override: unknown knob %d", knob);
  return ok();
}

void awq_clear_plan_overrides(void) { clear_plan_overrides(); }

int awq_device_cu_count(void) { return device_cu_count(); }

int awq_gemm_plan_info(int64_t M, int64_t N, int64_t K, int64_t G, int activation, int64_t* info) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (M <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_gemm_plan_info: M must be positive");
  if (activation != 0 && activation != AWQ_ACT_SILU && activation != AWQ_ACT_GELU)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_gemm_plan_info: unknown activation %d", activation);
  if (activation != 0 && N % 32 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "a gate/up projection needs N %% 32 == 0, got %lld", (long long)N);
  if (!info) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_gemm_plan_info: null pointer argument");
  const GemmPlan p = plan_gemm(make_geom(M, N, K, Gr), activation == 0 ? kActNone : kActSilu);
  info[0] = p.kind;
  info[1] = p.variant;
  info[2] = p.ks;
  info[3] = p.grid_x * p.grid_y * (p.kind == 1 || p.kind == 3 ? p.ks : 1);
  info[4] = plan_threads(p);
  info[5] = p.ws_bytes;
  return ok();
}

int awq_gemm_plan_fixup(int64_t M, int64_t N, int64_t K, int64_t G, int activation) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (M <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_gemm_plan_fixup: M must be positive");
  if (activation != 0 && activation != AWQ_ACT_SILU && activation != AWQ_ACT_GELU)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_gemm_plan_fixup: unknown activation %d", activation);
  const GemmPlan p = plan_gemm(make_geom(M, N, K, Gr), activation == 0 ? kActNone : kActSilu);
  return p.kind == 1 && p.ks > 1 && p.fixup ? 1 : 0;
}

int awq_mfma_probe(int64_t iters, int64_t grid, int block, float* sink, int64_t sink_bytes, awq_stream_t stream) {
  if (iters < 1 || iters >= (int64_t(1) << 40))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_mfma_probe: iters must be in [1, 2^40)");
  if (grid <= 0 || grid >= (int64_t(1) << 24))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_mfma_probe: grid must be in [1, 2^24)");
  if (block < 64 || block > 256 || block % 64 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_mfma_probe: block must be 64, 128, 192 or 256");
  if (!sink || !aligned(sink, 4)) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_mfma_probe: sink must be 4-byte aligned");
  if (sink_bytes < 4 * grid * (block / 64))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_mfma_probe: sink of %lld bytes needed, %lld given",
                (long long)(4 * grid * (block / 64)), (long long)sink_bytes);
  return hip_status(launch_mfma_probe(iters, grid, block, sink, (hipStream_t)stream), "awq_mfma_probe launch");
}

int awq_stream_probe(const void* src, int64_t bytes, int64_t grid, int block, uint32_t* sink, int64_t sink_bytes,
                     awq_stream_t stream) {
  if (bytes <= 0 || bytes % 16 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_stream_probe: bytes must be a positive multiple of 16");
  if (grid <= 0 || grid >= (int64_t(1) << 31))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_stream_probe: grid must be in [1, 2^31)");
  if (block < 64 || block > 1024 || block % 64 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_stream_probe: block must be a multiple of 64 in [64, 1024]");
  if (!src || !sink) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_stream_probe: null pointer argument");
  if (!aligned(src, 16) || !aligned(sink, 4))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_stream_probe: src must be 16-byte and sink 4-byte aligned");
  if (sink_bytes < 4 * grid)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_stream_probe: sink of %lld bytes needed, %lld given",
                (long long)(4 * grid), (long long)sink_bytes);
  return hip_status(launch_stream_probe(src, bytes, grid, block, sink, (hipStream_t)stream),
                    "awq_stream_probe launch");
}

int64_t awq_moe_sorted_capacity(int64_t numel, int64_t E, int64_t block_size) {
  if (numel < 0 || E <= 0 || block_size <= 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_sorted_capacity: numel >= 0, E > 0, block_size > 0 required");
  return moe_sorted_capacity(numel, E, block_size);
}

int64_t awq_moe_block_capacity(int64_t numel, int64_t E, int64_t block_size) {
  if (numel < 0 || E <= 0 || block_size <= 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_block_capacity: numel >= 0, E > 0, block_size > 0 required");
  return moe_block_capacity(numel, E, block_size);
}

int awq_moe_expert_strides(int64_t K, int64_t N, int64_t G, int64_t* w_stride, int64_t* s_stride,
                           int64_t* z_stride) {
  int64_t Gr = 0;
  const int st = check_shape(K, N, G, AWQ_DTYPE_FP16, &Gr);
  if (st != 0) return st;
  if (!w_stride || !s_stride || !z_stride)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_expert_strides: null pointer argument");
  const MoeStrides m = moe_expert_strides(make_geom(0, N, K, Gr));
  *w_stride = m.w;
  *s_stride = m.s;
  *z_stride = m.z;
  return ok();
}

int awq_moe_topk_softmax(const float* gating_output, float* topk_weights, int32_t* topk_ids, int64_t T, int64_t E,
                         int64_t topk, int renormalize, awq_stream_t stream) {
  const TraceRange range("awq_moe_topk_softmax");
  if (T < 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_topk_softmax: T must be non-negative");
  if (E <= 0 || E > 512) return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_topk_softmax: E must be in [1, 512], got %lld",
                                     (long long)E);
  if (topk < 1 || topk > E || topk > 64)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_topk_softmax: topk must be in [1, min(E, 64)], got %lld",
                (long long)topk);
  if (T > (int64_t(1) << 24)) return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_topk_softmax: T must be below 2^24");
  if (T == 0) return ok();
  if (!gating_output || !topk_weights || !topk_ids)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_topk_softmax: null pointer argument");
  return hip_status(launch_moe_topk(gating_output, topk_weights, topk_ids, T, E, topk, renormalize ? 1 : 0,
                                    (hipStream_t)stream),
                    "awq_moe_topk_softmax launch");
}

int awq_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t E, int64_t block_size,
                             int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_tokens_post_pad,
                             int32_t* expert_offsets, awq_stream_t stream) {
  const TraceRange range("awq_moe_align_block_size");
  if (E <= 0 || E > 512)
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_align_block_size: E must be in [1, 512], got %lld", (long long)E);
  if (block_size <= 0 || block_size % 16 != 0 || block_size > 1024)
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "awq_moe_align_block_size: block_size must be a positive multiple of 16 up to 1024, got %lld",
                (long long)block_size);
  if (numel < 0 || numel >= (int64_t(1) << 24))
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_align_block_size: numel must be in [0, 2^24), got %lld",
                (long long)numel);
  if ((numel > 0 && !topk_ids) || !sorted_ids || !expert_ids || !num_tokens_post_pad || !expert_offsets)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_align_block_size: null pointer argument");
  return hip_status(launch_moe_align(topk_ids, numel, E, block_size, sorted_ids, expert_ids, num_tokens_post_pad,
                                     expert_offsets, (hipStream_t)stream),
                    "awq_moe_align_block_size launch");
}

int awq_moe_w4a16_gemm(const void* a, int64_t a_rows, const void* w, const void* s, const void* z, int64_t E,
                       int64_t N, int64_t K, int64_t G, int dtype, const int32_t* sorted_ids, int64_t sorted_cap,
                       const int32_t* expert_offsets, const float* topk_weights, int64_t num_routed, int64_t top_k,
                       int activation, int mul_routed_weight, void* out, awq_stream_t stream) {
  const TraceRange range("awq_moe_w4a16_gemm");
  int64_t Gr = 0;
  int st = check_shape(K, N, G, dtype, &Gr);
  if (st != 0) return st;
  if (E <= 0 || E > 512)
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_w4a16_gemm: E must be in [1, 512], got %lld", (long long)E);
  if (activation != AWQ_MOE_ACT_NONE && activation != AWQ_MOE_ACT_SILU && activation != AWQ_MOE_ACT_GELU)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_w4a16_gemm: unknown activation %d", activation);
  if (activation != AWQ_MOE_ACT_NONE && N % 32 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "awq_moe_w4a16_gemm: gate/up pairing needs N = 2I with I %% 16 == 0, got N=%lld", (long long)N);
  if (top_k <= 0) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_w4a16_gemm: top_k must be positive");
  if (num_routed < 0 || num_routed >= (int64_t(1) << 24) || sorted_cap < 0 || sorted_cap >= (int64_t(1) << 30))
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_w4a16_gemm: num_routed must be below 2^24 and sorted_cap below 2^30");
  if ((num_routed + top_k - 1) / top_k > a_rows)
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "awq_moe_w4a16_gemm: %lld routed rows with top_k %lld need %lld activation rows, a has %lld",
                (long long)num_routed, (long long)top_k, (long long)((num_routed + top_k - 1) / top_k),
                (long long)a_rows);
  if ((num_routed + top_k - 1) / top_k * K * 2 >= (int64_t(1) << 31))
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_w4a16_gemm: the routed activation rows must span below 2 GiB");
  if (num_routed == 0 || sorted_cap == 0) return ok();
  if (!a || !w || !s || !z || !sorted_ids || !expert_offsets || !out || (mul_routed_weight && !topk_weights))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_w4a16_gemm: null pointer argument");
  if (!aligned(a, 16) || !aligned(out, 8) || !aligned(w, 16) || !aligned(s, 16) || !aligned(z, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT,
                "awq_moe_w4a16_gemm: a, w, s, z must be 16-byte aligned and out 8-byte aligned");
  MoeGemmParams p{};
  p.x = a;
  p.w = w;
  p.s = s;
  p.z = z;
  p.sorted = sorted_ids;
  p.offsets = expert_offsets;
  p.topk_w = topk_weights;
  p.out = out;
  p.E = E;
  p.a_div = top_k;
  p.num_routed = num_routed;
  p.sorted_cap = sorted_cap;
  p.g = make_geom(0, N, K, Gr);
  p.epi = activation;
  p.mul_rw = mul_routed_weight ? 1 : 0;
  p.dtype = dtype;
  return hip_status(launch_moe_gemm(p, (hipStream_t)stream), "awq_moe_w4a16_gemm launch");
}

int awq_moe_sum_reduce(const void* in, void* out, int64_t T, int64_t topk, int64_t H, int dtype,
                       awq_stream_t stream) {
  const TraceRange range("awq_moe_sum_reduce");
  if (dtype != AWQ_DTYPE_FP16 && dtype != AWQ_DTYPE_BF16)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_sum_reduce: dtype must be 0 or 1, got %d", dtype);
  if (T < 0 || topk <= 0 || H <= 0 || H % 8 != 0)
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_sum_reduce: T >= 0, topk > 0 and H %% 8 == 0 required");
  if (T * H >= (int64_t(1) << 34) || topk > 1024)
    return fail(AWQ_STATUS_UNSUPPORTED, "awq_moe_sum_reduce: problem too large");
  if (T == 0) return ok();
  if (!in || !out) return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_sum_reduce: null pointer argument");
  if (!aligned(in, 16) || !aligned(out, 16))
    return fail(AWQ_STATUS_INVALID_ARGUMENT, "awq_moe_sum_reduce: in and out must be 16-byte aligned");
  return hip_status(launch_moe_sum(in, out, T, topk, H, dtype, (hipStream_t)stream), "awq_moe_sum_reduce launch");
}

}  // extern "C"
