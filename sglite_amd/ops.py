"""Torch-facing wrappers over the C ABI.

PyTorch supplies device memory and the current HIP stream; all arithmetic runs
in the HIP kernels of libsglite_awq.so.  Every function launches on
``torch.cuda.current_stream()`` of the tensors' device, never synchronises and
allocates only through torch's caching allocator, so it can be captured in a
``torch.cuda.graph``.
"""

from __future__ import annotations

import ctypes
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


KERNEL_NAMES = {0: "skinny_kernel", 1: "tiled_kernel", 2: "gemv_kernel"}


def gemm_kernel(M: int, N: int, K: int, group_size: int, activation: Optional[str] = None) -> str:
    """Name of the kernel ``gemm`` runs for this shape (with ``activation``:
    the fused gate/up GEMM's kernel)."""
    G = resolve_group_size(group_size, K)
    lib = _lib.load()
    if activation is None:
        return KERNEL_NAMES[_lib.check(lib.awq_gemm_kernel_kind(M, N, K, G), "awq_gemm_kernel_kind")]
    return KERNEL_NAMES[_lib.check(lib.awq_gemm_kernel_kind_act(M, N, K, G), "awq_gemm_kernel_kind_act")]


def make_counters(N: int, device: torch.device) -> torch.Tensor:
    """Split-K arrival counters: zeroed once here, left zeroed by every GEMM call."""
    nbytes = _lib.check(_lib.load().awq_counter_bytes(N), "awq_counter_bytes")
    return torch.zeros(nbytes // 4, dtype=torch.int32, device=device)


def workspace_bytes_act(M: int, N: int, K: int, group_size: int) -> int:
    """Split-K workspace of ``gemm(..., activation=...)`` (its plan pairs gate and up tiles)."""
    G = resolve_group_size(group_size, K)
    return _lib.check(_lib.load().awq_workspace_bytes_act(M, N, K, G), "awq_workspace_bytes_act")


_GATED_ACT = {"silu": _lib.AWQ_ACT_SILU, "gelu": _lib.AWQ_ACT_GELU}


def gemm(x: torch.Tensor, r: Repacked, K: int, N: int, group_size: int, bias: Optional[torch.Tensor] = None,
         counters: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
         activation: Optional[str] = None) -> torch.Tensor:
    """out[M, N] = rnd(x[M, K] @ W) (+ bias), fp32 accumulation, on x's current stream.

    With ``activation`` ("silu" or "gelu") the two column halves of W are a
    merged gate/up projection and the output is ``act(gate) * up``, [M, N / 2],
    each half rounded (bias added) as the plain GEMM stores it, then the
    product in fp32, rounded once."""
    _require_cuda(x, r.w)
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"x must be [M, {K}], got {tuple(x.shape)}")
    if x.dtype != r.s.dtype:
        raise ValueError(f"activation dtype {x.dtype} does not match the scale dtype {r.s.dtype}")
    if activation is not None and activation not in _GATED_ACT:
        raise ValueError(f"unsupported activation {activation!r}")
    G = resolve_group_size(group_size, K)
    M = x.shape[0]
    dev = x.device
    x = _aligned(x)
    if bias is not None:
        _require_cuda(bias)
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} elements, got {bias.numel()}")
        bias = _aligned(bias.to(x.dtype).reshape(-1), 8)
    ncols = N if activation is None else N // 2
    if out is None:
        out = torch.empty((M, ncols), dtype=x.dtype, device=dev)
    lib = _lib.load()
    if M > 0:
        wsb = workspace_bytes(M, N, K, G) if activation is None else workspace_bytes_act(M, N, K, G)
    else:
        wsb = 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev) if wsb > 0 else None
    if wsb > 0 and counters is None:
        raise ValueError("this shape splits K across workgroups: pass the layer's counters (make_counters)")
    if activation is None:
        _lib.check(lib.awq_w4a16_gemm(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(), _ptr(bias),
                                      out.data_ptr(), M, N, K, G, dtype_code(x.dtype), _ptr(ws), wsb, _ptr(counters),
                                      _stream(dev)), "awq_w4a16_gemm")
    else:
        _lib.check(lib.awq_w4a16_gemm_act(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(), _ptr(bias),
                                          out.data_ptr(), M, N, K, G, dtype_code(x.dtype), _GATED_ACT[activation],
                                          _ptr(ws), wsb, _ptr(counters), _stream(dev)), "awq_w4a16_gemm_act")
    return out


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
    code = dtype_code(scales.dtype)
    ws, ss, zs = expert_strides(K, N, G)
    dev = qweight.device
    w = torch.empty((E, ws // 4), dtype=torch.int32, device=dev)
    s = torch.zeros((E, ss // 2), dtype=scales.dtype, device=dev)
    z = torch.zeros((E, zs // 8), dtype=torch.int64, device=dev)
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    lib = _lib.load()
    st = _stream(dev)
    for e in range(E):
        _lib.check(lib.awq_repack_cdna4(qweight[e].data_ptr(), qzeros[e].data_ptr(), scales[e].data_ptr(), code, K, N, G,
                                        w[e].data_ptr(), s[e].data_ptr(), z[e].data_ptr(), st), "awq_repack_cdna4")
    return RepackedExperts(w, s, z, K, N, G)


def moe_topk_softmax(gating_output: torch.Tensor, topk: int, renormalize: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(fp32 logits) -> top-k -> optional ``w / (sum(w) + 1e-8)``; (weights fp32, ids int32)."""
    _require_cuda(gating_output)
    if gating_output.dim() != 2:
        raise ValueError("gating_output must be [T, E]")
    logits = _aligned(gating_output.float(), 4)
    T, E = logits.shape
    w = torch.empty((T, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((T, topk), dtype=torch.int32, device=logits.device)
    _lib.check(_lib.load().awq_moe_topk_softmax(logits.data_ptr(), w.data_ptr(), ids.data_ptr(), T, E, topk,
                                                1 if renormalize else 0, _stream(logits.device)),
               "awq_moe_topk_softmax")
    return w, ids


class MoeAlignment(NamedTuple):
    sorted_ids: torch.Tensor          # int32 [sorted capacity]
    expert_ids: torch.Tensor          # int32 [block capacity]
    num_tokens_post_pad: torch.Tensor  # int32 [1]
    expert_offsets: torch.Tensor      # int32 [E + 1]


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int) -> MoeAlignment:
    """Stable sort of the routed rows by expert, buckets padded to ``block_size`` (sentinel ``topk_ids.numel()``)."""
    _require_cuda(topk_ids)
    if topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32")
    ids = topk_ids.contiguous().reshape(-1)
    n = ids.numel()
    lib = _lib.load()
    cap = _lib.check(lib.awq_moe_sorted_capacity(n, num_experts, block_size), "awq_moe_sorted_capacity")
    bcap = _lib.check(lib.awq_moe_block_capacity(n, num_experts, block_size), "awq_moe_block_capacity")
    dev = ids.device
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(bcap, dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    _lib.check(lib.awq_moe_align_block_size(ids.data_ptr() if n else None, n, num_experts, block_size,
                                            sorted_ids.data_ptr(), expert_ids.data_ptr(), npp.data_ptr(),
                                            offsets.data_ptr(), _stream(dev)), "awq_moe_align_block_size")
    return MoeAlignment(sorted_ids, expert_ids, npp, offsets)


_ACT_CODE = {None: _lib.AWQ_MOE_ACT_NONE, "silu": _lib.AWQ_MOE_ACT_SILU, "gelu": _lib.AWQ_MOE_ACT_GELU}


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
    G = resolve_group_size(group_size, K)
    E = experts.w.shape[0]
    ncols = N // 2 if activation is not None else N
    a = _aligned(a)
    if out is None:
        out = torch.empty((num_routed, ncols), dtype=a.dtype, device=a.device)
    if topk_weights is not None:
        topk_weights = _aligned(topk_weights.float().reshape(-1), 4)
    _lib.check(_lib.load().awq_moe_w4a16_gemm(
        a.data_ptr(), a.shape[0], experts.w.data_ptr(), experts.s.data_ptr(), experts.z.data_ptr(), E, N, K, G,
        dtype_code(a.dtype), align.sorted_ids.data_ptr(), align.sorted_ids.numel(), align.expert_offsets.data_ptr(),
        _ptr(topk_weights), num_routed, top_k, _ACT_CODE[activation], 1 if mul_routed_weight else 0, out.data_ptr(),
        _stream(a.device)), "awq_moe_w4a16_gemm")
    return out


def moe_sum_reduce(inp: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[t] = rnd(sum_j inp[t, j]) with an fp32 sum (inp [T, k, H], out [T, H])."""
    _require_cuda(inp, out)
    if inp.dim() != 3 or out.dim() != 2 or out.shape[0] != inp.shape[0] or out.shape[1] != inp.shape[2]:
        raise ValueError(f"shapes do not match: in {tuple(inp.shape)}, out {tuple(out.shape)}")
    if inp.dtype != out.dtype:
        raise ValueError("in and out must share a dtype")
    if not (inp.is_contiguous() and out.is_contiguous()):
        raise ValueError("in and out must be contiguous")
    T, k, H = inp.shape
    _lib.check(_lib.load().awq_moe_sum_reduce(inp.data_ptr(), out.data_ptr(), T, k, H, dtype_code(inp.dtype),
                                              _stream(inp.device)), "awq_moe_sum_reduce")
    return out
