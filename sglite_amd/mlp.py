"""Gated feed-forward block over the plugin's linear layers.

Mirror of ``GatedMLP`` (python/sglite/srt/model_executor/models/blocks.py:27-57):
gate_up_proj (MergedColumnParallelLinear of two intermediate_size halves, gate
first), act_fn (silu_and_mul / gelu_and_mul, blocks.py:38-42), down_proj
(RowParallelLinear).  The gate/up projection and the activation run as one
call, ``MergedColumnParallelLinear.forward_act``: with the AWQ methods the
activation is applied in the GEMM's epilogue, so the [M, 2I] gate/up output is
never written.  State-dict keys are ``gate_up_proj.*`` and ``down_proj.*``.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch

from .linear import MergedColumnParallelLinear, RowParallelLinear
from .quantization import LinearMethodBase


def _concat_prefix(prefix: str, name: str) -> str:
    return f"{prefix}.{name}" if prefix else name


class GatedMLP:
    """gate_up -> act(gate) * up -> down (GatedMLP, blocks.py:27-57)."""

    def __init__(self, hidden_size: int, intermediate_size: int, hidden_act: str = "silu",
                 linear_method: Optional[LinearMethodBase] = None, tp_size: int = 1, process_group=None):
        if hidden_act not in ("silu", "gelu"):
            raise ValueError(f"Unsupported activation function: {hidden_act}")
        self.hidden_act = hidden_act
        self.gate_up_proj = MergedColumnParallelLinear(hidden_size, [intermediate_size, intermediate_size], False,
                                                       linear_method, tp_size)
        self.down_proj = RowParallelLinear(intermediate_size, hidden_size, False, linear_method, tp_size,
                                           process_group)

    def state_dict_keys(self, prefix: str = "") -> List[str]:
        return (self.gate_up_proj.state_dict_keys(_concat_prefix(prefix, "gate_up_proj"))
                + self.down_proj.state_dict_keys(_concat_prefix(prefix, "down_proj")))

    def load_state_dict(self, state_dict: Dict[str, torch.Tensor], *, prefix: str = "",
                        _internal: bool = False) -> None:
        self.gate_up_proj.load_state_dict(state_dict, prefix=_concat_prefix(prefix, "gate_up_proj"), _internal=True)
        self.down_proj.load_state_dict(state_dict, prefix=_concat_prefix(prefix, "down_proj"), _internal=True)
        if not _internal and state_dict:
            raise RuntimeError(f"Unexpected keys in state_dict: {list(state_dict.keys())}")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj.forward(self.gate_up_proj.forward_act(x, self.hidden_act))

    __call__ = forward
