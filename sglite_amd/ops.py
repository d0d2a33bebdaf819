"""Torch-facing wrappers over the C ABI.

PyTorch supplies device memory and the current HIP stream; all arithmetic runs
in the HIP kernels of libsglite_awq.so.  Every function launches on
``torch.cuda.current_stream()`` of the tensors' device, never synchronises and
allocates only through torch's caching allocator, so it can be captured in a
``torch.cuda.graph``.
"""

from __future__ import annotations

from typing import NamedTuple, Optional, Tuple

import torch

from . import _lib

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


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("AWQ HIP kernels need device tensors")


def _aligned(t: torch.Tensor, a: int = 16) -> torch.Tensor:
    """Contiguous and ``a``-byte aligned (a fresh allocation is 256-byte aligned)."""
    if t.is_contiguous() and t.data_ptr() % a == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


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


def repack(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> Repacked:
    """AWQ checkpoint tensors -> CDNA4 tile layout (device side, no host copy)."""
    _require_cuda(qweight, qzeros, scales)
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
    lib = _lib.load()
    _lib.check(lib.awq_repack_cdna4(qweight.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), code, K, N, G,
                                    w.data_ptr(), s.data_ptr(), z.data_ptr(), _stream(dev)), "awq_repack_cdna4")
    return Repacked(w, s, z)


def unrepack(r: Repacked, K: int, N: int, group_size: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """CDNA4 tile layout -> AWQ (qweight, qzeros, scales)."""
    _require_cuda(r.w, r.s, r.z)
    G = resolve_group_size(group_size, K)
    dev = r.w.device
    qweight = torch.empty((K, N // 8), dtype=torch.int32, device=dev)
    qzeros = torch.empty((K // G, N // 8), dtype=torch.int32, device=dev)
    scales = torch.empty((K // G, N), dtype=r.s.dtype, device=dev)
    lib = _lib.load()
    _lib.check(lib.awq_unrepack_cdna4(r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(), dtype_code(r.s.dtype), K, N, G,
                                      qweight.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), _stream(dev)),
               "awq_unrepack_cdna4")
    return qweight, qzeros, scales


def dequant(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """W[K, N] = rnd((q - z) * s) from AWQ tensors (bit-exact probe)."""
    _require_cuda(qweight, qzeros, scales)
    K, N, G = _check_awq_shapes(qweight, qzeros, scales)
    out = torch.empty((K, N), dtype=scales.dtype, device=qweight.device)
    lib = _lib.load()
    _lib.check(lib.awq_dequant(qweight.contiguous().data_ptr(), qzeros.contiguous().data_ptr(),
                               scales.contiguous().data_ptr(), dtype_code(scales.dtype), K, N, G, out.data_ptr(),
                               _stream(qweight.device)), "awq_dequant")
    return out


def dequant_repacked(r: Repacked, K: int, N: int, group_size: int) -> torch.Tensor:
    """W[K, N] from the repacked tensors, via the GEMM kernels' dequant routine."""
    _require_cuda(r.w, r.s, r.z)
    G = resolve_group_size(group_size, K)
    out = torch.empty((K, N), dtype=r.s.dtype, device=r.w.device)
    lib = _lib.load()
    _lib.check(lib.awq_dequant_repacked(r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(), dtype_code(r.s.dtype), K, N,
                                        G, out.data_ptr(), _stream(r.w.device)), "awq_dequant_repacked")
    return out


def workspace_bytes(M: int, N: int, K: int, group_size: int) -> int:
    G = resolve_group_size(group_size, K)
    return _lib.check(_lib.load().awq_workspace_bytes(M, N, K, G), "awq_workspace_bytes")


def make_counters(N: int, device: torch.device) -> torch.Tensor:
    """Split-K arrival counters: zeroed once here, left zeroed by every GEMM call."""
    nbytes = _lib.check(_lib.load().awq_counter_bytes(N), "awq_counter_bytes")
    return torch.zeros(nbytes // 4, dtype=torch.int32, device=device)


def gemm(x: torch.Tensor, r: Repacked, K: int, N: int, group_size: int, bias: Optional[torch.Tensor] = None,
         counters: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[M, N] = rnd(x[M, K] @ W) (+ bias), fp32 accumulation, on x's current stream."""
    _require_cuda(x, r.w)
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [M, {K}], got {tuple(x.shape)}")
    if x.dtype != r.s.dtype:
        raise ValueError(f"activation dtype {x.dtype} does not match the scale dtype {r.s.dtype}")
    G = resolve_group_size(group_size, K)
    M = x.shape[0]
    dev = x.device
    x = _aligned(x)
    if bias is not None:
        _require_cuda(bias)
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} elements, got {bias.numel()}")
        bias = _aligned(bias.to(x.dtype).reshape(-1), 8)
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=dev)
    lib = _lib.load()
    wsb = workspace_bytes(M, N, K, G) if M > 0 else 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev) if wsb > 0 else None
    if wsb > 0 and counters is None:
        raise ValueError("this shape splits K across workgroups: pass the layer's counters (make_counters)")
    _lib.check(lib.awq_w4a16_gemm(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(), _ptr(bias),
                                  out.data_ptr(), M, N, K, G, dtype_code(x.dtype), _ptr(ws), wsb, _ptr(counters),
                                  _stream(dev)), "awq_w4a16_gemm")
    return out
