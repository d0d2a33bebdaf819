"""Helpers shared by the AWQ linear methods (the CDNA4 counterpart of marlin_utils).

Both reference methods -- ``awq`` (Triton) and ``awq_marlin`` -- run on the
one HIP engine here, so their create/process/apply steps share this module.
Reference helpers mirrored (python/sglite/srt/model_executor/layers/
quantization/marlin_utils.py): ``get_scalar_types`` :19-44,
``check_marlin_supported`` :58-96, ``verify_marlin_supports_shape`` :99-135,
``marlin_make_workspace`` :138-151, ``apply_awq_marlin_linear`` :355-415.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch
from torch.nn.parameter import Parameter

from .. import ops

# Shape constraints of the repacked kernels that the Marlin method also states
# (marlin_utils.py:12-15).
MIN_THREAD_N = 64
MIN_THREAD_K = 128
SUPPORTED_GROUP_SIZES = [-1, 32, 64, 128]


class ScalarType:
    """Minimal stand-in for sgl_kernel's ScalarType: a name and a bit width."""

    def __init__(self, name: str, size_bits: int):
        self.name = name
        self.size_bits = size_bits

    def __repr__(self) -> str:
        return self.name

    def __eq__(self, other: object) -> bool:
        if isinstance(other, ScalarType):
            return self.name == other.name
        return self.name == other

    def __hash__(self) -> int:
        return hash(self.name)


class _ScalarTypes:
    uint4 = ScalarType("uint4", 4)
    uint8 = ScalarType("uint8", 8)
    uint4b8 = ScalarType("uint4b8", 4)
    uint8b128 = ScalarType("uint8b128", 8)


scalar_types = _ScalarTypes()


def device_arch(device: Optional[torch.device] = None) -> str:
    """gfx architecture name of a device without initialising HIP when none is up."""
    if not (torch.cuda.is_available() and torch.cuda.is_initialized()):
        return ""
    props = torch.cuda.get_device_properties(device or torch.cuda.current_device())
    return getattr(props, "gcnArchName", "").split(":")[0]


def check_awq_supported(quant_type: ScalarType, group_size: int, has_zp: bool = False,
                        check_device: bool = True) -> bool:
    """Whether the HIP engine serves this quantization (check_marlin_supported semantics).

    Zero-point schemes support uint4 only, so 8-bit AWQ is rejected exactly as
    in the reference (marlin_utils.py:86-96).  With ``check_device`` the
    current device must be a gfx950 when HIP is initialised.
    """
    if check_device:
        arch = device_arch()
        if arch and arch != "gfx950":
            return False
    if group_size not in SUPPORTED_GROUP_SIZES:
        return False
    supported = [scalar_types.uint4] if has_zp else [scalar_types.uint4b8, scalar_types.uint8b128]
    return quant_type in supported


def verify_supports_shape(output_size_per_partition: int, input_size_per_partition: int, input_size: int,
                          group_size: int) -> None:
    """ValueError unless N % 64 == 0, K % 128 == 0 and K % G == 0 (marlin_utils.py:99-135)."""
    if output_size_per_partition % MIN_THREAD_N != 0:
        raise ValueError(
            f"output_size_per_partition={output_size_per_partition} not divisible by {MIN_THREAD_N}. "
            "Consider reducing tensor_parallel_size.")
    if input_size_per_partition % MIN_THREAD_K != 0:
        raise ValueError(
            f"input_size_per_partition={input_size_per_partition} not divisible by {MIN_THREAD_K}. "
            "Consider reducing tensor_parallel_size.")
    if group_size < input_size and input_size_per_partition % group_size != 0:
        raise ValueError(
            f"input_size_per_partition={input_size_per_partition} not divisible by group_size={group_size}. "
            "Consider reducing tensor_parallel_size.")


def make_awq_parameters(input_size: int, output_size: int, group_size: int, pack_factor: int) -> Dict[str, Any]:
    """Checkpoint-shaped AWQ tensors with the reference's loader attributes (awq.py:87-124)."""
    from .base_config import set_weight_attrs

    num_groups = input_size // group_size
    qweight = Parameter(torch.empty(input_size, output_size // pack_factor, dtype=torch.int32), requires_grad=False)
    set_weight_attrs(qweight, {"input_dim": 0, "output_dim": 1, "packed_dim": 1, "pack_factor": pack_factor})
    qzeros = Parameter(torch.empty(num_groups, output_size // pack_factor, dtype=torch.int32), requires_grad=False)
    set_weight_attrs(qzeros, {"input_dim": 0, "output_dim": 1, "packed_dim": 1, "pack_factor": pack_factor})
    scales = Parameter(torch.empty(num_groups, output_size), requires_grad=False)
    set_weight_attrs(scales, {"input_dim": 0, "output_dim": 1})
    return {"qweight": qweight, "qzeros": qzeros, "scales": scales}


def repack_awq_weights(weights: Dict[str, Any], group_size: int) -> Dict[str, Any]:
    """Post-load step: AWQ tensors -> CDNA4 tiles plus the split-K counters.

    Returns a new dict (the old AWQ tensors are dropped), like
    awq_marlin.py:325-334.  ``qweight``/``qzeros``/``scales`` keep their names
    (so linear.py:89-92 re-binds the layer attributes); ``workspace`` is a
    runtime tensor; ``_``-prefixed entries are metadata.
    """
    qweight, qzeros, scales = weights["qweight"], weights["qzeros"], weights["scales"]
    K = int(qweight.shape[0])
    N = int(qweight.shape[1]) * 8
    G = K if group_size == -1 else group_size
    if qzeros.shape[0] * G != K:
        raise ValueError(f"qzeros has {qzeros.shape[0]} group rows, expected K / group_size = {K // G}")
    r = ops.repack(qweight.data, qzeros.data, scales.data)
    return {
        "qweight": Parameter(r.w, requires_grad=False),
        "qzeros": Parameter(r.z, requires_grad=False),
        "scales": Parameter(r.s, requires_grad=False),
        "workspace": ops.make_counters(N, r.w.device),
        "_input_size": K,
        "_output_size": N,
        "_group_size": G,
        "_weights_processed": True,
        "_cdna4": True,
    }


def apply_awq_linear(weights: Dict[str, Any], x: torch.Tensor, bias: Optional[torch.Tensor],
                     group_size: int, activation: Optional[str] = None) -> torch.Tensor:
    """y = x @ W (+ bias) for repacked weights; raw AWQ weights are repacked on the fly.

    Output shape x.shape[:-1] + (N,), dtype x.dtype, bias added after the GEMM
    in the activation dtype (awq.py:133-147; marlin_utils.py:390-415).  With
    ``activation`` the output is act(gate) * up of the two column halves,
    x.shape[:-1] + (N / 2,), computed in the GEMM's epilogue.
    """
    if not weights.get("_cdna4", False):
        weights = repack_awq_weights(weights, group_size)
    K = weights["_input_size"]
    N = weights["_output_size"]
    G = weights["_group_size"]
    r = ops.Repacked(weights["qweight"], weights["scales"], weights["qzeros"])
    out_shape = x.shape[:-1] + (N if activation is None else N // 2,)
    y = ops.gemm(x.reshape(-1, x.shape[-1]), r, K, N, G, bias=bias, counters=weights["workspace"],
                 activation=activation)
    return y.reshape(out_shape)
