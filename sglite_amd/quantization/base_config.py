"""Plugin interface of SGLite's quantized linear methods.

Same names, signatures, argument meaning and error behaviour as
python/sglite/srt/model_executor/layers/quantization/base_config.py:9-91, so a
caller written against the reference binds to this package unchanged.
"""

from abc import ABC, abstractmethod
from typing import Any, Dict, List, Optional

import torch


def set_weight_attrs(weight: torch.Tensor, weight_attrs: Optional[Dict[str, Any]]) -> None:
    """Attach loader metadata to a tensor; refuse to overwrite an attribute.

    base_config.py:9-19: RuntimeError when the attribute already exists.
    """
    if weight_attrs is None:
        return
    for key, value in weight_attrs.items():
        if hasattr(weight, key):
            raise RuntimeError(f"Overwriting existing attribute {key} on weight tensor.")
        setattr(weight, key, value)


class LinearMethodBase(ABC):
    """A linear method owns weight allocation, post-load processing and apply.

    Lifecycle (python/sglite/srt/model_executor/layers/linear.py:32-35, 80-96,
    101-103): ``create_weights`` once per layer, checkpoint tensors loaded into
    the returned dict, ``process_weights_after_loading`` once, then
    ``apply_weights`` per forward.  One instance is shared by every layer of a
    model, so implementations keep no per-layer state.
    """

    @abstractmethod
    def create_weights(self, input_size: int, output_size: int) -> Dict[str, Any]:
        raise NotImplementedError

    @abstractmethod
    def apply_weights(self, weights: Dict[str, Any], x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        raise NotImplementedError

    def process_weights_after_loading(self, weights: Dict[str, Any]) -> Dict[str, Any]:
        return weights

    def apply_weights_act(self, weights: Dict[str, Any], x: torch.Tensor, activation: str,
                          bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """act(gate) * up of a merged gate/up projection (gate columns first): the
        GEMM then silu_and_mul / gelu_and_mul in fp32, as GatedMLP.forward does
        (blocks.py:51-57, activation.py:11-23).  No counterpart in the reference
        interface; methods with a fused kernel override it."""
        y = self.apply_weights(weights, x, bias).float()
        d = y.shape[-1] // 2
        if activation == "silu":
            g = torch.nn.functional.silu(y[..., :d])
        elif activation == "gelu":
            g = torch.nn.functional.gelu(y[..., :d])
        else:
            raise ValueError(f"Unsupported activation function: {activation}")
        return (g * y[..., d:]).to(x.dtype)


class QuantizationConfig(ABC):
    """Configuration of a quantization scheme (base_config.py:45-91)."""

    @abstractmethod
    def get_name(self) -> str:
        raise NotImplementedError

    @abstractmethod
    def get_supported_act_dtypes(self) -> List[torch.dtype]:
        raise NotImplementedError

    @abstractmethod
    def get_min_capability(self) -> int:
        raise NotImplementedError

    @staticmethod
    @abstractmethod
    def get_config_filenames() -> List[str]:
        raise NotImplementedError

    @classmethod
    @abstractmethod
    def from_config(cls, config: Dict[str, Any]) -> "QuantizationConfig":
        raise NotImplementedError

    @staticmethod
    def get_from_keys(config: Dict[str, Any], keys: List[str]) -> Any:
        """First value present under any of ``keys``; ValueError if none (base_config.py:75-81)."""
        for key in keys:
            if key in config:
                return config[key]
        raise ValueError(f"Cannot find any of {keys} in the model's quantization config.")

    @abstractmethod
    def get_linear_method(self) -> LinearMethodBase:
        raise NotImplementedError

    @abstractmethod
    def get_scaled_act_names(self) -> List[str]:
        raise NotImplementedError
