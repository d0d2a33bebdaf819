"""Torch custom ops over the C ABI (namespace ``torch.ops.sglite_awq``).

PyTorch supplies device memory and the current HIP stream; all arithmetic runs
in the HIP kernels of libsglite_awq.so.  Every C-ABI entry point that launches
work is registered with ``torch.library.custom_op`` and a fake (meta)
implementation, so the ops are visible to ``torch.ops``, FakeTensor shape
propagation and ``torch.compile``; this replaces the reference's dispatch
through its torch ops ``sgl_kernel.gptq_marlin_gemm`` and
``sgl_kernel.awq_marlin_repack``
(python/sglite/srt/model_executor/layers/quantization/marlin_utils.py:388-410,
awq_marlin.py:300-305).

Every op launches on ``torch.cuda.current_stream()`` of its tensors' device,
never synchronises and allocates only through torch's caching allocator, so
it can be captured in a ``torch.cuda.graph``.  The plain-Python functions
below (``gemm``, ``repack`` ...) are the wrappers the linear methods call;
they validate arguments and call the registered ops.
"""

from __future__ import annotations

import contextlib
import ctypes
from typing import Dict, Iterator, List, NamedTuple, Optional, Tuple

import torch

from . import _lib

NAMESPACE = "sglite_awq"
_DTYPE_CODE = {torch.float16: _lib.AWQ_DTYPE_FP16, torch.bfloat16: _lib.AWQ_DTYPE_BF16}
SUPPORTED_GROUP_SIZES = (-1, 32, 64, 128)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"AWQ W4A16 supports float16 and bfloat16 activations/scales, got {dtype}") from None


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_cuda(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("AWQ HIP kernels need device tensors")


def _aligned(t: torch.Tensor, a: int = 16) -> torch.Tensor:
    """Contiguous and ``a``-byte aligned (a fresh allocation is 256-byte aligned)."""
    if t.is_contiguous() and t.data_ptr() % a == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


@contextlib.contextmanager
def _on_device(device: torch.device) -> Iterator[None]:
    """Make ``device`` current for the C ABI's planning (it fills that device's CUs)."""
    if device.index is None or torch.cuda.current_device() == device.index:
        yield
    else:
        with torch.cuda.device(device):
            yield


def resolve_group_size(group_size: int, K: int) -> int:
    return K if group_size == -1 else group_size


class Repacked(NamedTuple):
    """Repacked tensors of one linear in the CDNA4 tile layout."""
    w: torch.Tensor  # int32 [NT * KT * 256]
    s: torch.Tensor  # scale dtype [NT, NG, 16]
    z: torch.Tensor  # int64 [NT, NG]  (16 zero nibbles per word)


def repacked_sizes(K: int, N: int, group_size: int) -> Tuple[int, int, int]:
    lib = _lib.load()
    G = resolve_group_size(group_size, K)
    wb = _lib.check(lib.awq_repacked_weight_bytes(K, N), "awq_repacked_weight_bytes")
    sb = _lib.check(lib.awq_repacked_scale_bytes(K, N, G), "awq_repacked_scale_bytes")
    zb = _lib.check(lib.awq_repacked_zero_bytes(K, N, G), "awq_repacked_zero_bytes")
    return wb, sb, zb


def _check_awq_shapes(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> Tuple[int, int, int]:
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32:
        raise ValueError("qweight and qzeros must be int32")
    if qweight.dim() != 2 or qzeros.dim() != 2 or scales.dim() != 2:
        raise ValueError("qweight, qzeros and scales must be 2-D")
    K, N8 = qweight.shape
    N = N8 * 8
    ng = qzeros.shape[0]
    if ng == 0 or K % ng:
        raise ValueError(f"qzeros rows ({ng}) must divide K ({K})")
    G = K // ng
    if qzeros.shape[1] != N8 or tuple(scales.shape) != (ng, N):
        raise ValueError(f"inconsistent AWQ shapes: qweight {tuple(qweight.shape)}, qzeros {tuple(qzeros.shape)}, "
                         f"scales {tuple(scales.shape)}")
    return K, N, G


# ---------------------------------------------------------------------------
# Registered ops: repack / unrepack / dequantisation probes.
# ---------------------------------------------------------------------------

@torch.library.custom_op(f"{NAMESPACE}::awq_repack_cdna4", mutates_args=(), device_types="cuda")
def _repack_op(qweight: torch.Tensor, qzeros: torch.Tensor,
               scales: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    K, N, G = _check_awq_shapes(qweight, qzeros, scales)
    code = dtype_code(scales.dtype)
    wb, sb, zb = repacked_sizes(K, N, G)
    dev = qweight.device
    NT, NG = (N + 15) // 16, K // G
    w = torch.empty(wb // 4, dtype=torch.int32, device=dev)
    s = torch.empty((NT, NG, 16), dtype=scales.dtype, device=dev)
    z = torch.empty((NT, NG), dtype=torch.int64, device=dev)
    assert s.numel() * 2 == sb and z.numel() * 8 == zb
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    with _on_device(dev):
        _lib.check(_lib.load().awq_repack_cdna4(qweight.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), code, K, N,
                                                G, w.data_ptr(), s.data_ptr(), z.data_ptr(), _stream(dev)),
                   "awq_repack_cdna4")
    return w, s, z


@_repack_op.register_fake
def _(qweight, qzeros, scales):
    K, N8 = qweight.shape
    N, NG = N8 * 8, qzeros.shape[0]
    NT, KT = (N + 15) // 16, (K + 127) // 128
    return (qweight.new_empty(NT * KT * 256), scales.new_empty((NT, NG, 16)),
            qweight.new_empty((NT, NG), dtype=torch.int64))


@torch.library.custom_op(f"{NAMESPACE}::awq_unrepack_cdna4", mutates_args=(), device_types="cuda")
def _unrepack_op(w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, K: int, N: int,
                 G: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    dev = w.device
    qweight = torch.empty((K, N // 8), dtype=torch.int32, device=dev)
    qzeros = torch.empty((K // G, N // 8), dtype=torch.int32, device=dev)
    scales = torch.empty((K // G, N), dtype=s.dtype, device=dev)
    with _on_device(dev):
        _lib.check(_lib.load().awq_unrepack_cdna4(w.data_ptr(), s.data_ptr(), z.data_ptr(), dtype_code(s.dtype), K, N,
                                                  G, qweight.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                                  _stream(dev)), "awq_unrepack_cdna4")
    return qweight, qzeros, scales


@_unrepack_op.register_fake
def _(w, s, z, K, N, G):
    return (w.new_empty((K, N // 8)), w.new_empty((K // G, N // 8)), s.new_empty((K // G, N)))


@torch.library.custom_op(f"{NAMESPACE}::awq_dequant", mutates_args=(), device_types="cuda")
def _dequant_op(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    K, N, G = _check_awq_shapes(qweight, qzeros, scales)
    out = torch.empty((K, N), dtype=scales.dtype, device=qweight.device)
    with _on_device(qweight.device):
        _lib.check(_lib.load().awq_dequant(qweight.contiguous().data_ptr(), qzeros.contiguous().data_ptr(),
                                           scales.contiguous().data_ptr(), dtype_code(scales.dtype), K, N, G,
                                           out.data_ptr(), _stream(qweight.device)), "awq_dequant")
    return out


@_dequant_op.register_fake
def _(qweight, qzeros, scales):
    return scales.new_empty((qweight.shape[0], qweight.shape[1] * 8))


@torch.library.custom_op(f"{NAMESPACE}::awq_dequant_repacked", mutates_args=(), device_types="cuda")
def _dequant_repacked_op(w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, K: int, N: int, G: int) -> torch.Tensor:
    out = torch.empty((K, N), dtype=s.dtype, device=w.device)
    with _on_device(w.device):
        _lib.check(_lib.load().awq_dequant_repacked(w.data_ptr(), s.data_ptr(), z.data_ptr(), dtype_code(s.dtype), K,
                                                    N, G, out.data_ptr(), _stream(w.device)), "awq_dequant_repacked")
    return out


@_dequant_repacked_op.register_fake
def _(w, s, z, K, N, G):
    return s.new_empty((K, N))


def repack(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> Repacked:
    """AWQ checkpoint tensors -> CDNA4 tile layout (device side, no host copy)."""
    _require_cuda(qweight, qzeros, scales)
    _check_awq_shapes(qweight, qzeros, scales)
    dtype_code(scales.dtype)
    return Repacked(*torch.ops.sglite_awq.awq_repack_cdna4(qweight, qzeros, scales))


def unrepack(r: Repacked, K: int, N: int, group_size: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """CDNA4 tile layout -> AWQ (qweight, qzeros, scales)."""
    _require_cuda(r.w, r.s, r.z)
    return tuple(torch.ops.sglite_awq.awq_unrepack_cdna4(r.w, r.s, r.z, K, N, resolve_group_size(group_size, K)))


def dequant(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """W[K, N] = rnd((q - z) * s) from AWQ tensors (bit-exact probe)."""
    _require_cuda(qweight, qzeros, scales)
    _check_awq_shapes(qweight, qzeros, scales)
    return torch.ops.sglite_awq.awq_dequant(qweight, qzeros, scales)


def dequant_repacked(r: Repacked, K: int, N: int, group_size: int) -> torch.Tensor:
    """W[K, N] from the repacked tensors, via Dq<>::word (the prefill and MoE kernels' dequant routine)."""
    _require_cuda(r.w, r.s, r.z)
    return torch.ops.sglite_awq.awq_dequant_repacked(r.w, r.s, r.z, K, N, resolve_group_size(group_size, K))


# ---------------------------------------------------------------------------
# Planning queries and overrides.
# ---------------------------------------------------------------------------

def workspace_bytes(M: int, N: int, K: int, group_size: int) -> int:
    G = resolve_group_size(group_size, K)
    return _lib.check(_lib.load().awq_workspace_bytes(M, N, K, G), "awq_workspace_bytes")


def workspace_bytes_act(M: int, N: int, K: int, group_size: int) -> int:
    """Split-K workspace of ``gemm(..., activation=...)`` (its plan pairs gate and up tiles)."""
    G = resolve_group_size(group_size, K)
    return _lib.check(_lib.load().awq_workspace_bytes_act(M, N, K, G), "awq_workspace_bytes_act")


KERNEL_NAMES = {0: "skinny_kernel", 1: "tiled_kernel", 2: "gemv_kernel", 3: "kslice_kernel"}


def gemm_kernel(M: int, N: int, K: int, group_size: int, activation: Optional[str] = None) -> str:
    """Name of the kernel ``gemm`` runs for this shape (with ``activation``:
    the fused gate/up GEMM's kernel)."""
    G = resolve_group_size(group_size, K)
    lib = _lib.load()
    if activation is None:
        return KERNEL_NAMES[_lib.check(lib.awq_gemm_kernel_kind(M, N, K, G), "awq_gemm_kernel_kind")]
    return KERNEL_NAMES[_lib.check(lib.awq_gemm_kernel_kind_act(M, N, K, G), "awq_gemm_kernel_kind_act")]


class PlanInfo(NamedTuple):
    kernel: str           # kernel kind (KERNEL_NAMES): which family and planner branch
    variant: int
    k_slices: int
    workgroups: int
    threads: int
    workspace_bytes: int
    function: str = ""    # the __global__ function the GEMM launch runs
    fixup: bool = False   # split K summed inside the GEMM kernel (no second launch, given counters)


def kernel_function(kind: str, variant: int) -> str:
    """Name of the HIP kernel a plan's GEMM launch runs: the tiled kind runs
    ``tiled_kernel`` for row-block codes below 1000 (16x16x32 MFMAs) and
    ``mfma32_kernel`` for the others (32x32x16 MFMAs)."""
    if kind == "tiled_kernel" and variant >= 1000:
        return "mfma32_kernel"
    return kind


def plan_info(M: int, N: int, K: int, group_size: int, activation: Optional[str] = None) -> PlanInfo:
    """The plan ``gemm`` runs for this shape on the current device."""
    G = resolve_group_size(group_size, K)
    info = (ctypes.c_int64 * 6)()
    act = 0 if activation is None else _GATED_ACT[activation]
    lib = _lib.load()
    _lib.check(lib.awq_gemm_plan_info(M, N, K, G, act, info), "awq_gemm_plan_info")
    fixup = _lib.check(lib.awq_gemm_plan_fixup(M, N, K, G, act), "awq_gemm_plan_fixup") == 1
    kind = KERNEL_NAMES[int(info[0])]
    return PlanInfo(kind, *[int(v) for v in info[1:]], function=kernel_function(kind, int(info[1])), fixup=fixup)


PLAN_KNOBS = {"gemv_max_m": _lib.AWQ_PLAN_GEMV_MAX_M, "gemv_variant": _lib.AWQ_PLAN_GEMV_VARIANT,
              "gemv_ks": _lib.AWQ_PLAN_GEMV_KS, "skinny_variant": _lib.AWQ_PLAN_SKINNY_VARIANT,
              "skinny_ks": _lib.AWQ_PLAN_SKINNY_KS, "tiled_min_m": _lib.AWQ_PLAN_TILED_MIN_M,
              "tiled_bm": _lib.AWQ_PLAN_TILED_BM, "tiled_ks": _lib.AWQ_PLAN_TILED_KS,
              "kslice_variant": _lib.AWQ_PLAN_KSLICE_VARIANT, "tiled_fixup": _lib.AWQ_PLAN_TILED_FIXUP,
              "fixup_polls": _lib.AWQ_PLAN_FIXUP_POLLS}


def set_plan_override(knob: str, value: int) -> None:
    """Force a planner choice for every later GEMM of the process (tests and sweeps)."""
    _lib.check(_lib.load().awq_set_plan_override(PLAN_KNOBS[knob], int(value)), "awq_set_plan_override")


def clear_plan_overrides() -> None:
    _lib.load().awq_clear_plan_overrides()


@contextlib.contextmanager
def plan_overrides(**knobs: int) -> Iterator[None]:
    """``with plan_overrides(gemv_max_m=0, skinny_variant=10104): ...`` -- all overrides are cleared on exit."""
    try:
        for k, v in knobs.items():
            set_plan_override(k, v)
        yield
    finally:
        clear_plan_overrides()


def device_cu_count() -> int:
    return int(_lib.load().awq_device_cu_count())


def make_counters(N: int, device: torch.device) -> torch.Tensor:
    """Split-K counters (awq_counter_bytes): zeroed once here; every GEMM call leaves them valid for the
    next, whatever its shape (torch allocations are 512-byte aligned, as the 128 the library needs)."""
    nbytes = _lib.check(_lib.load().awq_counter_bytes(N), "awq_counter_bytes")
    return torch.zeros(nbytes // 4, dtype=torch.int32, device=device)


def counters_settled(counters: torch.Tensor) -> bool:
    """True when no GEMM is in flight on ``counters``: the decode kernels' per-column-tile counters are
    zero and every split tile of the tiled kernels has as many arrivals as its base (each launch that
    split a tile advanced both by its k-slice count)."""
    nt = _lib.AWQ_COUNTER_TILE_BYTES // 4
    tiles = counters[:nt].view(-1, 32)
    return bool(torch.equal(tiles[:, 0], tiles[:, 1])) and int(counters[nt:].abs().sum()) == 0


# ---------------------------------------------------------------------------
# Split-K workspace: one growing buffer per (device, stream) for eager calls
# (the reference sizes its Marlin workspace once at load, awq_marlin.py:298);
# a call being captured into a graph takes a fresh buffer from the graph's
# pool instead, so that replays never share eager memory.
# ---------------------------------------------------------------------------

_WS_CACHE: Dict[Tuple[int, int], torch.Tensor] = {}


def _workspace(nbytes: int, device: torch.device) -> Optional[torch.Tensor]:
    if nbytes <= 0:
        return None
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), _stream(device))
    buf = _WS_CACHE.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WS_CACHE[key] = buf
    return buf


_GATED_ACT = {"silu": _lib.AWQ_ACT_SILU, "gelu": _lib.AWQ_ACT_GELU}


def _gemm_launch(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, bias: Optional[torch.Tensor],
                 counters: Optional[torch.Tensor], out: torch.Tensor, K: int, N: int, G: int, act: int) -> None:
    M = x.shape[0]
    if M == 0:
        return
    dev = x.device
    lib = _lib.load()
    with _on_device(dev):
        if act == 0:
            wsb = _lib.check(lib.awq_workspace_bytes(M, N, K, G), "awq_workspace_bytes")
        else:
            wsb = _lib.check(lib.awq_workspace_bytes_act(M, N, K, G), "awq_workspace_bytes_act")
        ws = _workspace(wsb, dev)
        cb = 0 if counters is None else counters.numel() * 4
        if act == 0:
            _lib.check(lib.awq_w4a16_gemm(x.data_ptr(), w.data_ptr(), s.data_ptr(), z.data_ptr(), _ptr(bias),
                                          out.data_ptr(), M, N, K, G, dtype_code(x.dtype), _ptr(ws), wsb,
                                          _ptr(counters), cb, _stream(dev)), "awq_w4a16_gemm")
        else:
            _lib.check(lib.awq_w4a16_gemm_act(x.data_ptr(), w.data_ptr(), s.data_ptr(), z.data_ptr(), _ptr(bias),
                                              out.data_ptr(), M, N, K, G, dtype_code(x.dtype), act, _ptr(ws), wsb,
                                              _ptr(counters), cb, _stream(dev)), "awq_w4a16_gemm_act")


@torch.library.custom_op(f"{NAMESPACE}::awq_w4a16_gemm", mutates_args=("counters",), device_types="cuda")
def _gemm_op(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, bias: Optional[torch.Tensor],
             counters: Optional[torch.Tensor], K: int, N: int, G: int) -> torch.Tensor:
    out = torch.empty((x.shape[0], N), dtype=x.dtype, device=x.device)
    _gemm_launch(x, w, s, z, bias, counters, out, K, N, G, 0)
    return out


@_gemm_op.register_fake
def _(x, w, s, z, bias, counters, K, N, G):
    return x.new_empty((x.shape[0], N))


@torch.library.custom_op(f"{NAMESPACE}::awq_w4a16_gemm_out", mutates_args=("counters", "out"), device_types="cuda")
def _gemm_out_op(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, bias: Optional[torch.Tensor],
                 counters: Optional[torch.Tensor], out: torch.Tensor, K: int, N: int, G: int) -> None:
    _gemm_launch(x, w, s, z, bias, counters, out, K, N, G, 0)


@_gemm_out_op.register_fake
def _(x, w, s, z, bias, counters, out, K, N, G):
    return None


@torch.library.custom_op(f"{NAMESPACE}::awq_w4a16_gemm_act", mutates_args=("counters",), device_types="cuda")
def _gemm_act_op(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, bias: Optional[torch.Tensor],
                 counters: Optional[torch.Tensor], K: int, N: int, G: int, activation: str) -> torch.Tensor:
    out = torch.empty((x.shape[0], N // 2), dtype=x.dtype, device=x.device)
    _gemm_launch(x, w, s, z, bias, counters, out, K, N, G, _GATED_ACT[activation])
    return out


@_gemm_act_op.register_fake
def _(x, w, s, z, bias, counters, K, N, G, activation):
    return x.new_empty((x.shape[0], N // 2))


@torch.library.custom_op(f"{NAMESPACE}::awq_w4a16_gemm_act_out", mutates_args=("counters", "out"),
                         device_types="cuda")
def _gemm_act_out_op(x: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, bias: Optional[torch.Tensor],
                     counters: Optional[torch.Tensor], out: torch.Tensor, K: int, N: int, G: int,
                     activation: str) -> None:
    _gemm_launch(x, w, s, z, bias, counters, out, K, N, G, _GATED_ACT[activation])


@_gemm_act_out_op.register_fake
def _(x, w, s, z, bias, counters, out, K, N, G, activation):
    return None


def _check_out(out: torch.Tensor, shape: Tuple[int, ...], dtype: torch.dtype, device: torch.device,
               what: str = "out") -> None:
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"{what} must have shape {tuple(shape)}, got {tuple(out.shape)}")
    if out.dtype != dtype:
        raise ValueError(f"{what} must be {dtype}, got {out.dtype}")
    if out.device != device:
        raise ValueError(f"{what} must be on {device}, got {out.device}")
    if not out.is_contiguous() or out.data_ptr() % 8:
        raise ValueError(f"{what} must be contiguous and 8-byte aligned")


def _check_counters(counters: torch.Tensor, N: int, device: torch.device) -> None:
    if counters.dtype != torch.int32:
        raise ValueError(f"counters must be int32, got {counters.dtype}")
    if counters.device != device:
        raise ValueError(f"counters must be on {device}, got {counters.device}")
    if not counters.is_contiguous():
        raise ValueError("counters must be contiguous")
    need = _lib.check(_lib.load().awq_counter_bytes(N), "awq_counter_bytes") // 4
    if counters.numel() < need:
        raise ValueError(f"counters must hold at least {need} int32 (awq_counter_bytes({N}) bytes), "
                         f"got {counters.numel()}")
    if counters.data_ptr() % 128:
        raise ValueError("counters must be 128-byte aligned")


def gemm(x: torch.Tensor, r: Repacked, K: int, N: int, group_size: int, bias: Optional[torch.Tensor] = None,
         counters: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
         activation: Optional[str] = None) -> torch.Tensor:
    """out[M, N] = rnd(x[M, K] @ W) (+ bias), fp32 accumulation, on x's current stream.

    With ``activation`` ("silu" or "gelu") the two column halves of W are a
    merged gate/up projection and the output is ``act(gate) * up``, [M, N / 2],
    each half rounded (bias added) as the plain GEMM stores it, then the
    product in fp32, rounded once.  ``counters`` (from ``make_counters``, zero
    between calls) is needed whenever the plan splits K across workgroups."""
    _require_cuda(x, r.w, r.s, r.z)
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [M, {K}], got {tuple(x.shape)}")
    if x.dtype != r.s.dtype:
        raise ValueError(f"activation dtype {x.dtype} does not match the scale dtype {r.s.dtype}")
    if activation is not None and activation not in _GATED_ACT:
        raise ValueError(f"unsupported activation {activation!r}")
    if r.w.device != x.device or r.s.device != x.device or r.z.device != x.device:
        raise ValueError("x and the repacked weights must be on one device")
    G = resolve_group_size(group_size, K)
    M = x.shape[0]
    dev = x.device
    x = _aligned(x)
    if bias is not None:
        _require_cuda(bias)
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} elements, got {bias.numel()}")
        bias = _aligned(bias.to(x.dtype).reshape(-1), 8)
    if counters is not None:
        _check_counters(counters, N, dev)
    elif M > 0:
        wsb = workspace_bytes(M, N, K, G) if activation is None else workspace_bytes_act(M, N, K, G)
        if wsb > 0 and plan_info(M, N, K, G, activation).kernel != "tiled_kernel":
            raise ValueError("this shape splits K across workgroups: pass the layer's counters (make_counters)")
    ncols = N if activation is None else N // 2
    if out is not None:
        _check_out(out, (M, ncols), x.dtype, dev)
    if activation is None:
        if out is None:
            return torch.ops.sglite_awq.awq_w4a16_gemm(x, r.w, r.s, r.z, bias, counters, K, N, G)
        torch.ops.sglite_awq.awq_w4a16_gemm_out(x, r.w, r.s, r.z, bias, counters, out, K, N, G)
        return out
    if out is None:
        return torch.ops.sglite_awq.awq_w4a16_gemm_act(x, r.w, r.s, r.z, bias, counters, K, N, G, activation)
    torch.ops.sglite_awq.awq_w4a16_gemm_act_out(x, r.w, r.s, r.z, bias, counters, out, K, N, G, activation)
    return out


def gemm_noalloc(x: torch.Tensor, r: Repacked, K: int, N: int, group_size: int, out: torch.Tensor,
                 bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``gemm`` through awq_w4a16_gemm_noalloc: the split-K workspace and counters are the library's
    static per-device scratch, so the call allocates nothing (x, out and bias must already be
    contiguous and aligned).  Calls overlapping on one device race on that scratch."""
    _require_cuda(x, r.w, out, bias)
    M = x.shape[0]
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [M, {K}], got {tuple(x.shape)}")
    if x.dtype != r.s.dtype:
        raise ValueError(f"activation dtype {x.dtype} does not match the scale dtype {r.s.dtype}")
    _check_out(out, (M, N), x.dtype, x.device)
    if not x.is_contiguous() or (bias is not None and (not bias.is_contiguous() or bias.numel() != N
                                                       or bias.dtype != x.dtype)):
        raise ValueError("x (and bias: N elements of x's dtype) must be contiguous")
    with _on_device(x.device):
        _noalloc_ready(x.device)
        _lib.check(_lib.load().awq_w4a16_gemm_noalloc(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(),
                                                      _ptr(bias), out.data_ptr(), M, N, K,
                                                      resolve_group_size(group_size, K), dtype_code(x.dtype),
                                                      _stream(x.device)), "awq_w4a16_gemm_noalloc")
    return out


_NOALLOC_READY: set = set()


def _noalloc_ready(device: torch.device) -> None:
    """Resolve the device's static scratch ahead of the first call (awq_noalloc_init), unless that
    call is being captured: then the library's first call puts the counter clearing in the graph."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx in _NOALLOC_READY or torch.cuda.is_current_stream_capturing():
        return
    _lib.check(_lib.load().awq_noalloc_init(_stream(device)), "awq_noalloc_init")
    _NOALLOC_READY.add(idx)


# ---------------------------------------------------------------------------
# Gated MLP block in one launch (awq_gated_mlp): gate_up -> act(gate) * up ->
# down for decode batches, GatedMLP.forward (blocks.py:51-57) as one kernel.
# ---------------------------------------------------------------------------


class MlpPlan(NamedTuple):
    workgroups: int
    k_slices: int         # k-slices of the down projection
    tiles_per_group: int  # down column tiles per column group
    groups: int           # down column groups
    gate_tiles: int       # gate tiles per workgroup
    k_tiles: int          # down k-tiles per slice
    lds_bytes: int
    ws_bytes: int


def gated_mlp_plan(M: int, H: int, I: int, group_size: int, dtype: torch.dtype = torch.float16) -> Optional[MlpPlan]:
    """The one-launch plan for this block on the current device, or None when the shape is outside
    the built forms (then the block runs as its two GEMMs)."""
    info = (ctypes.c_int64 * 8)()
    r = _lib.check(_lib.load().awq_gated_mlp_plan(M, H, I, resolve_group_size(group_size, H), dtype_code(dtype),
                                                  info), "awq_gated_mlp_plan")
    return MlpPlan(*[int(v) for v in info]) if r == 1 else None


def make_mlp_counters(device: torch.device) -> torch.Tensor:
    """Counters of the one-launch gated MLP (AWQ_MLP_COUNTER_BYTES, zeroed once here; every call
    leaves them valid for the next).  Calls that share them must be ordered on one stream."""
    return torch.zeros(_lib.AWQ_MLP_COUNTER_BYTES // 4, dtype=torch.int32, device=device)


def mlp_counters_settled(counters: torch.Tensor) -> bool:
    """True when no one-launch gated MLP is in flight on ``counters``: every 128-byte slot has as many
    arrivals as its base (each launch advanced both by its arrivals)."""
    slots = counters.view(-1, 32)
    return bool(torch.equal(slots[:, 0], slots[:, 1]))


def mlp_take_errors(counters: torch.Tensor) -> int:
    """Synchronize the current stream and return (and clear) the number of workgroups that gave up
    waiting for their k-slice of the intermediate since the last check."""
    _require_cuda(counters)
    with _on_device(counters.device):
        return _lib.check(_lib.load().awq_gated_mlp_take_errors(counters.data_ptr(), counters.numel() * 4,
                                                                _stream(counters.device)), "awq_gated_mlp_take_errors")


def mlp_check(counters: torch.Tensor) -> None:
    """Raise AWQKernelError when a one-launch gated MLP on ``counters`` gave up waiting (its output
    was wrong) since the last check; the counters stay valid for further calls."""
    n = mlp_take_errors(counters)
    if n:
        raise _lib.AWQKernelError(f"awq_gated_mlp: {n} workgroup(s) gave up waiting for the intermediate; "
                                  "the outputs of those calls are invalid")


def _mlp_launch(x: torch.Tensor, gw: torch.Tensor, gs: torch.Tensor, gz: torch.Tensor, dw: torch.Tensor,
                ds: torch.Tensor, dz: torch.Tensor, counters: torch.Tensor, out: torch.Tensor, H: int, I: int,
                G: int, activation: str, polls: int) -> None:
    M = x.shape[0]
    if M == 0:
        return
    dev = x.device
    lib = _lib.load()
    with _on_device(dev):
        wsb = _lib.check(lib.awq_gated_mlp_workspace_bytes(M, H, I, G, dtype_code(x.dtype)),
                         "awq_gated_mlp_workspace_bytes")
        ws = _workspace(wsb, dev)
        _lib.check(lib.awq_gated_mlp(x.data_ptr(), gw.data_ptr(), gs.data_ptr(), gz.data_ptr(), dw.data_ptr(),
                                     ds.data_ptr(), dz.data_ptr(), out.data_ptr(), M, H, I, G, dtype_code(x.dtype),
                                     _GATED_ACT[activation], polls, _ptr(ws), wsb, counters.data_ptr(),
                                     counters.numel() * 4, _stream(dev)), "awq_gated_mlp")


@torch.library.custom_op(f"{NAMESPACE}::awq_gated_mlp_out", mutates_args=("counters", "out"), device_types="cuda")
def _mlp_out_op(x: torch.Tensor, gw: torch.Tensor, gs: torch.Tensor, gz: torch.Tensor, dw: torch.Tensor,
                ds: torch.Tensor, dz: torch.Tensor, counters: torch.Tensor, out: torch.Tensor, H: int, I: int, G: int,
                activation: str, polls: int) -> None:
    _mlp_launch(x, gw, gs, gz, dw, ds, dz, counters, out, H, I, G, activation, polls)


@_mlp_out_op.register_fake
def _(x, gw, gs, gz, dw, ds, dz, counters, out, H, I, G, activation, polls):
    return None


def gated_mlp(x: torch.Tensor, gate_up: Repacked, down: Repacked, H: int, I: int, group_size: int,
              counters: torch.Tensor, activation: str = "silu", out: Optional[torch.Tensor] = None,
              polls: Optional[int] = None) -> torch.Tensor:
    """out[M, H] = down(act(gate) * up) of a gated MLP block in one launch (awq_gated_mlp).

    ``gate_up`` is the merged projection repacked as K = H, N = 2I (gate columns first), ``down`` the
    down projection as K = I, N = H; group size 128, no bias.  The gate and up values are rounded and
    combined exactly as ``gemm(..., activation=...)`` stores them, and the down projection's k-slice
    sums are added in a fixed order.  ``counters`` from ``make_mlp_counters``.  ``polls`` bounds each
    workgroup's wait for its k-slice of the intermediate (None: the library default); a workgroup
    that gives up makes the call's output invalid and is reported by ``mlp_check``.  Raises RuntimeError when
    ``gated_mlp_plan`` has no plan for the shape."""
    _require_cuda(x, gate_up.w, down.w, counters)
    if x.dim() != 2 or x.shape[1] != H:
        raise ValueError(f"x must be [M, {H}], got {tuple(x.shape)}")
    if x.dtype != gate_up.s.dtype or x.dtype != down.s.dtype:
        raise ValueError(f"activation dtype {x.dtype} does not match the scale dtypes")
    if activation not in _GATED_ACT:
        raise ValueError(f"unsupported activation {activation!r}")
    dev = x.device
    for t in (gate_up.w, gate_up.s, gate_up.z, down.w, down.s, down.z):
        if t.device != dev:
            raise ValueError("x and the repacked weights must be on one device")
    if counters.dtype != torch.int32 or counters.device != dev or not counters.is_contiguous() \
            or counters.numel() * 4 < _lib.AWQ_MLP_COUNTER_BYTES or counters.data_ptr() % 128:
        raise ValueError("counters must be make_mlp_counters(device)")
    G = resolve_group_size(group_size, H)
    M = x.shape[0]
    x = _aligned(x)
    if out is None:
        out = torch.empty((M, H), dtype=x.dtype, device=dev)
    else:
        _check_out(out, (M, H), x.dtype, dev)
    torch.ops.sglite_awq.awq_gated_mlp_out(x, gate_up.w, gate_up.s, gate_up.z, down.w, down.s, down.z, counters,
                                           out, H, I, G, activation, -1 if polls is None else int(polls))
    return out


def stream_probe(src: torch.Tensor, nbytes: int, grid: int, block: int, sink: torch.Tensor) -> None:
    """Stream ``nbytes`` of ``src`` with ``grid`` workgroups of ``block`` threads (awq_stream_probe)."""
    _require_cuda(src, sink)
    if nbytes > src.numel() * src.element_size():
        raise ValueError("nbytes exceeds the source buffer")
    with _on_device(src.device):
        _lib.check(_lib.load().awq_stream_probe(src.data_ptr(), nbytes, grid, block, sink.data_ptr(),
                                                sink.numel() * sink.element_size(), _stream(src.device)),
                   "awq_stream_probe")


def mfma_probe(iters: int, grid: int, block: int, sink: torch.Tensor) -> None:
    """``grid`` x ``block`` threads of back-to-back 32x32x16 fp16 MFMAs (awq_mfma_probe)."""
    _require_cuda(sink)
    with _on_device(sink.device):
        _lib.check(_lib.load().awq_mfma_probe(iters, grid, block, sink.data_ptr(), sink.numel() * sink.element_size(),
                                              _stream(sink.device)), "awq_mfma_probe")


# ---------------------------------------------------------------------------
# Grouped MoE (experts stacked on dim 0).
# ---------------------------------------------------------------------------

class RepackedExperts(NamedTuple):
    """Expert-stacked repacked tensors, one row per expert (rows padded to
    256 bytes); ``expert(e)`` views expert e's linear as a ``Repacked``."""
    w: torch.Tensor  # int32 [E, w_stride / 4]
    s: torch.Tensor  # scale dtype [E, s_stride / 2]
    z: torch.Tensor  # int64 [E, z_stride / 8]
    K: int
    N: int
    G: int

    def expert(self, e: int) -> Repacked:
        NT, NG = (self.N + 15) // 16, self.K // self.G
        return Repacked(self.w[e, :NT * ((self.K + 127) // 128) * 256], self.s[e, :NT * NG * 16].view(NT, NG, 16),
                        self.z[e, :NT * NG].view(NT, NG))


def expert_strides(K: int, N: int, group_size: int) -> Tuple[int, int, int]:
    """Byte strides between consecutive experts' weights, scales and zero words."""
    G = resolve_group_size(group_size, K)
    w, s, z = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.load().awq_moe_expert_strides(K, N, G, ctypes.byref(w), ctypes.byref(s), ctypes.byref(z)),
               "awq_moe_expert_strides")
    return w.value, s.value, z.value


@torch.library.custom_op(f"{NAMESPACE}::awq_repack_experts", mutates_args=(), device_types="cuda")
def _repack_experts_op(qweight: torch.Tensor, qzeros: torch.Tensor,
                       scales: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    E = qweight.shape[0]
    K, N, G = _check_awq_shapes(qweight[0], qzeros[0], scales[0])
    code = dtype_code(scales.dtype)
    ws, ss, zs = expert_strides(K, N, G)
    dev = qweight.device
    w = torch.empty((E, ws // 4), dtype=torch.int32, device=dev)
    s = torch.zeros((E, ss // 2), dtype=scales.dtype, device=dev)
    z = torch.zeros((E, zs // 8), dtype=torch.int64, device=dev)
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    lib = _lib.load()
    with _on_device(dev):
        st = _stream(dev)
        for e in range(E):
            _lib.check(lib.awq_repack_cdna4(qweight[e].data_ptr(), qzeros[e].data_ptr(), scales[e].data_ptr(), code, K,
                                            N, G, w[e].data_ptr(), s[e].data_ptr(), z[e].data_ptr(), st),
                       "awq_repack_cdna4")
    return w, s, z


@_repack_experts_op.register_fake
def _(qweight, qzeros, scales):
    E, K, N8 = qweight.shape
    N, NG = N8 * 8, qzeros.shape[1]
    NT, KT = (N + 15) // 16, (K + 127) // 128

    def up(b):
        return (b + 255) // 256 * 256
    return (qweight.new_empty((E, up(NT * KT * 1024) // 4)), scales.new_empty((E, up(NT * NG * 32) // 2)),
            qweight.new_empty((E, up(NT * NG * 8) // 8), dtype=torch.int64))


def repack_experts(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> RepackedExperts:
    """AWQ expert stacks ``[E, K, N/8]`` / ``[E, K/G, N/8]`` / ``[E, K/G, N]`` -> stacked tile layout.

    Each expert is repacked into its own row of the stacks (the layout
    ``awq_moe_w4a16_gemm`` expects)."""
    _require_cuda(qweight, qzeros, scales)
    if qweight.dim() != 3 or qzeros.dim() != 3 or scales.dim() != 3:
        raise ValueError("expert stacks must be 3-D [E, ...]")
    E = qweight.shape[0]
    if qzeros.shape[0] != E or scales.shape[0] != E:
        raise ValueError("qweight, qzeros and scales must stack the same number of experts")
    K, N, G = _check_awq_shapes(qweight[0], qzeros[0], scales[0])
    dtype_code(scales.dtype)
    w, s, z = torch.ops.sglite_awq.awq_repack_experts(qweight, qzeros, scales)
    return RepackedExperts(w, s, z, K, N, G)


@torch.library.custom_op(f"{NAMESPACE}::awq_moe_topk_softmax", mutates_args=(), device_types="cuda")
def _topk_op(gating_output: torch.Tensor, topk: int, renormalize: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    logits = _aligned(gating_output.float(), 4)
    T, E = logits.shape
    w = torch.empty((T, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((T, topk), dtype=torch.int32, device=logits.device)
    with _on_device(logits.device):
        _lib.check(_lib.load().awq_moe_topk_softmax(logits.data_ptr(), w.data_ptr(), ids.data_ptr(), T, E, topk,
                                                    1 if renormalize else 0, _stream(logits.device)),
                   "awq_moe_topk_softmax")
    return w, ids


@_topk_op.register_fake
def _(gating_output, topk, renormalize):
    T = gating_output.shape[0]
    return (gating_output.new_empty((T, topk), dtype=torch.float32),
            gating_output.new_empty((T, topk), dtype=torch.int32))


def moe_topk_softmax(gating_output: torch.Tensor, topk: int, renormalize: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(fp32 logits) -> top-k -> optional ``w / (sum(w) + 1e-8)``; (weights fp32, ids int32)."""
    _require_cuda(gating_output)
    if gating_output.dim() != 2:
        raise ValueError("gating_output must be [T, E]")
    return tuple(torch.ops.sglite_awq.awq_moe_topk_softmax(gating_output, topk, bool(renormalize)))


class MoeAlignment(NamedTuple):
    sorted_ids: torch.Tensor          # int32 [sorted capacity]
    expert_ids: torch.Tensor          # int32 [block capacity]
    num_tokens_post_pad: torch.Tensor  # int32 [1]
    expert_offsets: torch.Tensor      # int32 [E + 1]


def _align_caps(n: int, num_experts: int, block_size: int) -> Tuple[int, int]:
    lib = _lib.load()
    cap = _lib.check(lib.awq_moe_sorted_capacity(n, num_experts, block_size), "awq_moe_sorted_capacity")
    bcap = _lib.check(lib.awq_moe_block_capacity(n, num_experts, block_size), "awq_moe_block_capacity")
    return cap, bcap


@torch.library.custom_op(f"{NAMESPACE}::awq_moe_align_block_size", mutates_args=(), device_types="cuda")
def _align_op(topk_ids: torch.Tensor, block_size: int,
              num_experts: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    ids = topk_ids.contiguous().reshape(-1)
    n = ids.numel()
    cap, bcap = _align_caps(n, num_experts, block_size)
    dev = ids.device
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(bcap, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    with _on_device(dev):
        _lib.check(_lib.load().awq_moe_align_block_size(ids.data_ptr() if n else None, n, num_experts, block_size,
                                                        sorted_ids.data_ptr(), expert_ids.data_ptr(), npp.data_ptr(),
                                                        offsets.data_ptr(), _stream(dev)), "awq_moe_align_block_size")
    return sorted_ids, expert_ids, npp, offsets


@_align_op.register_fake
def _(topk_ids, block_size, num_experts):
    cap, bcap = _align_caps(topk_ids.numel(), num_experts, block_size)
    return (topk_ids.new_empty(cap), topk_ids.new_empty(bcap), topk_ids.new_empty(1),
            topk_ids.new_empty(num_experts + 1))


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int) -> MoeAlignment:
    """Stable sort of the routed rows by expert, buckets padded to ``block_size`` (sentinel ``topk_ids.numel()``)."""
    _require_cuda(topk_ids)
    if topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32")
    return MoeAlignment(*torch.ops.sglite_awq.awq_moe_align_block_size(topk_ids, block_size, num_experts))


_ACT_CODE = {None: _lib.AWQ_MOE_ACT_NONE, "silu": _lib.AWQ_MOE_ACT_SILU, "gelu": _lib.AWQ_MOE_ACT_GELU}
_ACT_NAME = {"none": None, "silu": "silu", "gelu": "gelu"}


@torch.library.custom_op(f"{NAMESPACE}::awq_moe_w4a16_gemm", mutates_args=("out",), device_types="cuda")
def _moe_gemm_op(a: torch.Tensor, w: torch.Tensor, s: torch.Tensor, z: torch.Tensor, sorted_ids: torch.Tensor,
                 expert_offsets: torch.Tensor, topk_weights: Optional[torch.Tensor], out: torch.Tensor, K: int, N: int,
                 G: int, num_routed: int, top_k: int, activation: str, mul_routed_weight: bool) -> None:
    E = w.shape[0]
    with _on_device(a.device):
        _lib.check(_lib.load().awq_moe_w4a16_gemm(
            a.data_ptr(), a.shape[0], w.data_ptr(), s.data_ptr(), z.data_ptr(), E, N, K, G, dtype_code(a.dtype),
            sorted_ids.data_ptr(), sorted_ids.numel(), expert_offsets.data_ptr(), _ptr(topk_weights), num_routed,
            top_k, _ACT_CODE[_ACT_NAME[activation]], 1 if mul_routed_weight else 0, out.data_ptr(),
            _stream(a.device)), "awq_moe_w4a16_gemm")


@_moe_gemm_op.register_fake
def _(a, w, s, z, sorted_ids, expert_offsets, topk_weights, out, K, N, G, num_routed, top_k, activation,
      mul_routed_weight):
    return None


def moe_gemm(a: torch.Tensor, experts: RepackedExperts, K: int, N: int, group_size: int, align: MoeAlignment,
             topk_weights: Optional[torch.Tensor], num_routed: int, top_k: int, activation: Optional[str] = None,
             mul_routed_weight: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Grouped W4A16 GEMM over the expert buckets.

    Routed row r reads ``a[r // top_k]``; the output has ``num_routed`` rows of
    ``N`` columns, or ``N / 2`` with a gate/up ``activation`` ("silu"/"gelu")."""
    _require_cuda(a, experts.w)
    if a.dim() != 2 or a.shape[1] != K:
        raise ValueError(f"a must be [rows, {K}], got {tuple(a.shape)}")
    if a.dtype != experts.s.dtype:
        raise ValueError(f"activation dtype {a.dtype} does not match the scale dtype {experts.s.dtype}")
    if activation not in _ACT_CODE:
        raise ValueError(f"unsupported activation {activation!r}")
    if mul_routed_weight and topk_weights is None:
        raise ValueError("mul_routed_weight needs topk_weights")
    G = resolve_group_size(group_size, K)
    ncols = N // 2 if activation is not None else N
    a = _aligned(a)
    if out is None:
        out = torch.empty((num_routed, ncols), dtype=a.dtype, device=a.device)
    else:
        _check_out(out, (num_routed, ncols), a.dtype, a.device)
    if topk_weights is not None:
        topk_weights = _aligned(topk_weights.float().reshape(-1), 4)
        if topk_weights.numel() < num_routed:
            raise ValueError(f"topk_weights must hold {num_routed} routed weights, got {topk_weights.numel()}")
    torch.ops.sglite_awq.awq_moe_w4a16_gemm(a, experts.w, experts.s, experts.z, align.sorted_ids, align.expert_offsets,
                                            topk_weights, out, K, N, G, num_routed, top_k,
                                            "none" if activation is None else activation, bool(mul_routed_weight))
    return out


@torch.library.custom_op(f"{NAMESPACE}::awq_moe_sum_reduce", mutates_args=("out",), device_types="cuda")
def _moe_sum_op(inp: torch.Tensor, out: torch.Tensor) -> None:
    T, k, H = inp.shape
    with _on_device(inp.device):
        _lib.check(_lib.load().awq_moe_sum_reduce(inp.data_ptr(), out.data_ptr(), T, k, H, dtype_code(inp.dtype),
                                                  _stream(inp.device)), "awq_moe_sum_reduce")


@_moe_sum_op.register_fake
def _(inp, out):
    return None


def moe_sum_reduce(inp: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[t] = rnd(sum_j inp[t, j]) with an fp32 sum (inp [T, k, H], out [T, H])."""
    _require_cuda(inp, out)
    if inp.dim() != 3 or out.dim() != 2 or out.shape[0] != inp.shape[0] or out.shape[1] != inp.shape[2]:
        raise ValueError(f"shapes do not match: in {tuple(inp.shape)}, out {tuple(out.shape)}")
    if inp.dtype != out.dtype:
        raise ValueError("in and out must share a dtype")
    if not (inp.is_contiguous() and out.is_contiguous()):
        raise ValueError("in and out must be contiguous")
    torch.ops.sglite_awq.awq_moe_sum_reduce(inp, out)
    return out


REGISTERED_OPS: List[str] = [
    "awq_repack_cdna4", "awq_unrepack_cdna4", "awq_dequant", "awq_dequant_repacked", "awq_w4a16_gemm",
    "awq_w4a16_gemm_out", "awq_w4a16_gemm_act", "awq_w4a16_gemm_act_out", "awq_repack_experts",
    "awq_moe_topk_softmax", "awq_moe_align_block_size", "awq_moe_w4a16_gemm", "awq_moe_sum_reduce",
]
