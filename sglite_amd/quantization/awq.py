"""``awq`` quantization config and linear method on the HIP engine.

Interface of python/sglite/srt/model_executor/layers/quantization/awq.py:11-147
(AWQConfig, AWQLinearMethod).  The reference runs its Triton fallback on the
raw AWQ tensors; here ``process_weights_after_loading`` repacks them into the
CDNA4 tile layout and ``apply_weights`` runs the gfx950 kernels.
"""

from typing import Any, Dict, List, Optional

import torch

from . import cdna4_utils
from .base_config import LinearMethodBase, QuantizationConfig


class AWQConfig(QuantizationConfig):
    """AWQ configuration: ``bits`` must be 4 (awq.py:13-24)."""

    def __init__(self, weight_bits: int, group_size: int, zero_point: bool) -> None:
        self.weight_bits = weight_bits
        self.group_size = group_size
        self.zero_point = zero_point
        if self.weight_bits != 4:
            raise ValueError(
                "Currently, only 4-bit weight quantization is supported for AWQ, "
                f"but got {self.weight_bits} bits.")
        self.pack_factor = 32 // self.weight_bits

    def __repr__(self) -> str:
        return f"AWQConfig(weight_bits={self.weight_bits}, group_size={self.group_size}, zero_point={self.zero_point})"

    def get_name(self) -> str:
        return "awq"

    def get_supported_act_dtypes(self) -> List[torch.dtype]:
        # Same declaration as awq.py:38-40 (no caller enforces it); the kernels
        # behind this method also run bf16, which the engine's dtype cast of
        # checkpoint scales can produce (engine.py:171).
        return [torch.half]

    def get_min_capability(self) -> int:
        # CUDA compute capability in the reference (awq.py:42-44); kept for
        # interface parity, the device check is the gfx950 arch name.
        return 75

    @staticmethod
    def get_config_filenames() -> List[str]:
        return ["quant_config.json", "quantize_config.json"]

    @classmethod
    def from_config(cls, config: Dict[str, Any]) -> "AWQConfig":
        weight_bits = cls.get_from_keys(config, ["w_bit", "bits"])
        group_size = cls.get_from_keys(config, ["q_group_size", "group_size"])
        zero_point = cls.get_from_keys(config, ["zero_point"])
        return cls(weight_bits, group_size, zero_point)

    def get_linear_method(self) -> "AWQLinearMethod":
        return AWQLinearMethod(self)

    def get_scaled_act_names(self) -> List[str]:
        return ["gelu", "gelu_fast", "gelu_new", "gelu_pytorch_tanh"]


class AWQLinearMethod(LinearMethodBase):
    """AWQ linear method (awq.py:68-147) on the gfx950 engine."""

    def __init__(self, quant_config: AWQConfig):
        self.quant_config = quant_config

    def _group_size(self, input_size: int) -> int:
        g = self.quant_config.group_size
        return input_size if g == -1 else g

    def create_weights(self, input_size: int, output_size: int) -> Dict[str, Any]:
        """qweight int32 [K, N/8], qzeros int32 [K/G, N/8], scales [K/G, N] (awq.py:74-124)."""
        G = self._group_size(input_size)
        if input_size % G != 0:
            raise ValueError(
                "The input size is not aligned with the quantized weight shape. "
                "This can be caused by too large tensor parallel size.")
        if output_size % self.quant_config.pack_factor != 0:
            raise ValueError(
                "The output size is not aligned with the quantized weight shape. "
                "This can be caused by too large tensor parallel size.")
        return cdna4_utils.make_awq_parameters(input_size, output_size, G, self.quant_config.pack_factor)

    def process_weights_after_loading(self, weights: Dict[str, Any]) -> Dict[str, Any]:
        if weights.get("_weights_processed", False):
            return weights
        K = int(weights["qweight"].shape[0])
        return cdna4_utils.repack_awq_weights(weights, self._group_size(K))

    def apply_weights(self, weights: Dict[str, Any], x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        K = int(weights["_input_size"]) if "_input_size" in weights else int(weights["qweight"].shape[0])
        return cdna4_utils.apply_awq_linear(weights, x, bias, self._group_size(K))

    def apply_weights_act(self, weights: Dict[str, Any], x: torch.Tensor, activation: str,
                          bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """act(gate) * up in the gate/up GEMM's epilogue (one launch, no [M, N] intermediate)."""
        K = int(weights["_input_size"]) if "_input_size" in weights else int(weights["qweight"].shape[0])
        return cdna4_utils.apply_awq_linear(weights, x, bias, self._group_size(K), activation=activation)
