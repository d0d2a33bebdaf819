"""``awq_marlin`` quantization config and linear method on the HIP engine.

Interface of python/sglite/srt/model_executor/layers/quantization/
awq_marlin.py:30-364 (AWQMarlinConfig, AWQMarlinLinearMethod).  The name is
kept so checkpoints and model code that select "awq_marlin" work unchanged;
there is no Marlin here: post-load processing repacks into the CDNA4 tile
layout on the device and apply runs the gfx950 kernels.
"""

from typing import Any, Dict, List, Optional

import torch

from . import cdna4_utils
from .base_config import LinearMethodBase, QuantizationConfig
from .cdna4_utils import check_awq_supported, scalar_types, verify_supports_shape


class AWQMarlinConfig(QuantizationConfig):
    """4-bit AWQ with zero points and group size -1/32/64/128 (awq_marlin.py:30-151)."""

    # Quantized weight bit width -> scalar type (awq_marlin.py:41-44).
    TYPE_MAP = {4: scalar_types.uint4, 8: scalar_types.uint8}

    def __init__(self, weight_bits: int, group_size: int, zero_point: bool) -> None:
        self.weight_bits = weight_bits
        self.group_size = group_size
        self.zero_point = zero_point
        self.pack_factor = 32 // weight_bits
        if weight_bits not in self.TYPE_MAP:
            raise ValueError(
                f"AWQ Marlin only supports {list(self.TYPE_MAP.keys())} bits, but got {weight_bits} bits.")
        self.quant_type = self.TYPE_MAP[weight_bits]
        if not check_awq_supported(self.quant_type, group_size, zero_point, check_device=False):
            raise ValueError(
                "AWQ Marlin does not support this configuration: "
                f"bits={weight_bits}, group_size={group_size}, zero_point={zero_point}. "
                "group_size must be in [-1, 32, 64, 128].")

    def __repr__(self) -> str:
        return (f"AWQMarlinConfig(weight_bits={self.weight_bits}, group_size={self.group_size}, "
                f"zero_point={self.zero_point})")

    def get_name(self) -> str:
        return "awq_marlin"

    def get_supported_act_dtypes(self) -> List[torch.dtype]:
        return [torch.half, torch.bfloat16]

    def get_min_capability(self) -> int:
        return 80

    @staticmethod
    def get_config_filenames() -> List[str]:
        return ["quant_config.json", "quantize_config.json"]

    @classmethod
    def from_config(cls, config: Dict[str, Any]) -> "AWQMarlinConfig":
        weight_bits = cls.get_from_keys(config, ["w_bit", "bits"])
        group_size = cls.get_from_keys(config, ["q_group_size", "group_size"])
        zero_point = cls.get_from_keys(config, ["zero_point"])
        return cls(weight_bits, group_size, zero_point)

    @classmethod
    def is_awq_marlin_compatible(cls, quant_config: Dict[str, Any]) -> bool:
        """Config-only compatibility check (awq_marlin.py:112-143)."""
        quant_method = quant_config.get("quant_method", "").lower()
        num_bits = quant_config.get("w_bit") or quant_config.get("bits")
        group_size = quant_config.get("q_group_size") or quant_config.get("group_size")
        zero_point = quant_config.get("zero_point")
        if quant_method != "awq":
            return False
        if num_bits is None or group_size is None or zero_point is None:
            return False
        if num_bits not in cls.TYPE_MAP:
            return False
        return check_awq_supported(cls.TYPE_MAP[num_bits], group_size, zero_point, check_device=False)

    def get_linear_method(self) -> "AWQMarlinLinearMethod":
        return AWQMarlinLinearMethod(self)

    def get_scaled_act_names(self) -> List[str]:
        return ["gelu", "gelu_fast", "gelu_new", "gelu_pytorch_tanh"]


class AWQMarlinLinearMethod(LinearMethodBase):
    """AWQ linear method with the Marlin method's shape rules and metadata (awq_marlin.py:154-364)."""

    def __init__(self, quant_config: AWQMarlinConfig):
        self.quant_config = quant_config

    def create_weights(self, input_size: int, output_size: int) -> Dict[str, Any]:
        """AWQ checkpoint tensors plus ``_``-metadata (awq_marlin.py:169-268)."""
        group_size = self.quant_config.group_size
        if group_size == -1:
            group_size = input_size
        verify_supports_shape(output_size_per_partition=output_size, input_size_per_partition=input_size,
                              input_size=input_size, group_size=group_size)
        if input_size % group_size != 0:
            raise ValueError(
                f"input_size={input_size} is not divisible by group_size={group_size}. "
                "This can be caused by too large tensor parallel size.")
        if output_size % self.quant_config.pack_factor != 0:
            raise ValueError(
                f"output_size={output_size} is not divisible by pack_factor={self.quant_config.pack_factor}. "
                "This can be caused by too large tensor parallel size.")
        weights = cdna4_utils.make_awq_parameters(input_size, output_size, group_size, self.quant_config.pack_factor)
        weights.update({
            "_input_size": input_size,
            "_output_size": output_size,
            "_num_groups": input_size // group_size,
            "_weights_processed": False,
        })
        return weights

    def process_weights_after_loading(self, weights: Dict[str, Any]) -> Dict[str, Any]:
        """Repack AWQ -> CDNA4 tiles on the device (replaces awq_marlin.py:270-334)."""
        if weights.get("_weights_processed", False):
            return weights
        group_size = self.quant_config.group_size
        if group_size == -1:
            group_size = weights["_input_size"]
        return cdna4_utils.repack_awq_weights(weights, group_size)

    def apply_weights(self, weights: Dict[str, Any], x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        group_size = self.quant_config.group_size
        if group_size == -1:
            group_size = weights["_input_size"]
        return cdna4_utils.apply_awq_linear(weights, x, bias, group_size)

    def apply_weights_act(self, weights: Dict[str, Any], x: torch.Tensor, activation: str,
                          bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """act(gate) * up in the gate/up GEMM's epilogue (one launch, no [M, N] intermediate)."""
        group_size = self.quant_config.group_size
        if group_size == -1:
            group_size = weights["_input_size"]
        return cdna4_utils.apply_awq_linear(weights, x, bias, group_size, activation=activation)
