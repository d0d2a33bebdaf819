"""Gated feed-forward block over the plugin's linear layers.

Mirror of ``GatedMLP`` (python/sglite/srt/model_executor/models/blocks.py:27-57):
gate_up_proj (MergedColumnParallelLinear of two intermediate_size halves, gate
first), act_fn (silu_and_mul / gelu_and_mul, blocks.py:38-42), down_proj
(RowParallelLinear).  The gate/up projection and the activation run as one
call, ``MergedColumnParallelLinear.forward_act``: with the AWQ methods the
activation is applied in the GEMM's epilogue, so the [M, 2I] gate/up output is
never written.  With ``one_launch=True``, decode batches whose shape the
one-launch kernel covers (``ops.gated_mlp_plan``: M <= 16, group size 128, no
bias, both projections repacked AWQ) run the whole block -- gate/up, activation
and down projection -- as one launch (``ops.gated_mlp``).  It is off by
default: on MI355X the exchange of the intermediate between workgroups inside
that launch costs more than the second launch it saves (Qwen3-4B, M = 1:
21 us against 16.6 us per block for the two calls).  State-dict keys are
``gate_up_proj.*`` and ``down_proj.*``.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch

from . import ops
from .linear import MergedColumnParallelLinear, RowParallelLinear
from .quantization import LinearMethodBase


def _concat_prefix(prefix: str, name: str) -> str:
    return f"{prefix}.{name}" if prefix else name


class GatedMLP:
    """gate_up -> act(gate) * up -> down (GatedMLP, blocks.py:27-57)."""

    def __init__(self, hidden_size: int, intermediate_size: int, hidden_act: str = "silu",
                 linear_method: Optional[LinearMethodBase] = None, tp_size: int = 1, process_group=None,
                 one_launch: bool = False):
        if hidden_act not in ("silu", "gelu"):
            raise ValueError(f"Unsupported activation function: {hidden_act}")
        self.hidden_act = hidden_act
        self.one_launch = one_launch
        self._mlp_counters: Optional[torch.Tensor] = None
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

    def _one_launch_weights(self, x: torch.Tensor):
        """(gate_up, down, H, I, G) when the block can run as one launch for x, else None."""
        gu, dn = self.gate_up_proj._weights, self.down_proj._weights
        if not (self.one_launch and x.is_cuda and gu.get("_cdna4") and dn.get("_cdna4")):
            return None
        if self.gate_up_proj.bias is not None or self.down_proj.bias is not None:
            return None
        H, I, G = gu["_input_size"], gu["_output_size"] // 2, gu["_group_size"]
        if dn["_input_size"] != I or dn["_output_size"] != H or dn["_group_size"] != G:
            return None
        M = x.numel() // H
        if M < 1 or ops.gated_mlp_plan(M, H, I, G, x.dtype) is None:
            return None
        return (ops.Repacked(gu["qweight"], gu["scales"], gu["qzeros"]),
                ops.Repacked(dn["qweight"], dn["scales"], dn["qzeros"]), H, I, G)

    def check_errors(self) -> None:
        """Raise when a one-launch call of this block gave up waiting for its intermediate since the
        last check (synchronizes the current stream; call it at the serving loop's sync points)."""
        if self._mlp_counters is not None:
            ops.mlp_check(self._mlp_counters)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        one = self._one_launch_weights(x)
        if one is not None:
            gu, dn, H, I, G = one
            if self._mlp_counters is None or self._mlp_counters.device != x.device:
                self._mlp_counters = ops.make_mlp_counters(x.device)
            y = ops.gated_mlp(x.reshape(-1, H), gu, dn, H, I, G, self._mlp_counters, self.hidden_act)
            y = y.reshape(x.shape[:-1] + (H,))
            if self.down_proj._tp_size > 1:
                torch.distributed.all_reduce(y, group=self.down_proj._group)
            return y
        return self.down_proj.forward(self.gate_up_proj.forward_act(x, self.hidden_act))

    __call__ = forward
