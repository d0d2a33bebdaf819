"""Unquantized linear method (python/sglite/srt/model_executor/layers/quantization/unquant.py:11-39).

Part of the quantization package's exported surface: the fallback method
``_TPLinearBase`` uses when a layer has no quantization config.
"""

from typing import Any, Dict, Optional

import torch
import torch.nn.functional as F
from torch.nn.parameter import Parameter

from .base_config import LinearMethodBase, set_weight_attrs


class UnquantizedLinearMethod(LinearMethodBase):
    """Dense weight [N, K] applied with F.linear."""

    def __init__(self, separate_bias_add: bool = False):
        self.separate_bias_add = separate_bias_add

    def create_weights(self, input_size: int, output_size: int) -> Dict[str, Any]:
        weight = Parameter(torch.empty(output_size, input_size), requires_grad=False)
        set_weight_attrs(weight, {"input_dim": 1, "output_dim": 0})
        return {"weight": weight}

    def apply_weights(self, weights: Dict[str, Any], x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        weight = weights["weight"]
        if self.separate_bias_add:
            y = F.linear(x, weight)
            return y + bias if bias is not None else y
        return F.linear(x, weight, bias)
