"""Mixture-of-experts layer over AWQ expert stacks.

Mirror of ``MoELayer`` (python/sglite/srt/model_executor/layers/moe_layer.py:11-64)
for AWQ checkpoints:

* the constructor takes the same arguments (num_experts, top_k, hidden_size,
  intermediate_size, renormalize, activation, apply_router_weight_on_input),
  plus the AWQ group size, the activation dtype and explicit tensor-parallel
  arguments in place of the reference's process-group globals;
* intermediate_size is split over tp_size ranks (moe_layer.py:35-36), and
  each rank holds all experts' column slice of gate/up and row slice of down;
* the state dict holds the expert-stacked AWQ tensors the checkpoint loader
  yields for ``<prefix>.experts.<i>.{gate,up,down}_proj.{qweight,qzeros,scales}``
  once gate and up are merged (weight_loader.py:17-30, :80-89, :134-142):
      gate_up_proj.qweight  int32 [E, H, 2I/8]    down_proj.qweight  int32 [E, I, H/8]
      gate_up_proj.qzeros   int32 [E, H/G, 2I/8]  down_proj.qzeros   int32 [E, I/G, H/8]
      gate_up_proj.scales   dtype [E, H/G, 2I]    down_proj.scales   dtype [E, I/G, H]
  with I the per-rank intermediate size and gate columns before up columns;
* the public attributes are shape-only ("meta") tensors that state what the
  state dict must hold; ``load_state_dict`` checks all six tensors' shapes
  and dtypes first (the BaseModule contract, layers/base.py:40-62), pops them
  and repacks each stack into the CDNA4 tile layout on its device; the
  checkpoint tensors are not kept, and a later load repacks again;
* ``forward(hidden_states, router_logits)`` runs the MoE backend (routing,
  grouped GEMMs, top-k sum) and all-reduces the output when tp_size > 1
  (moe_layer.py:48-64).
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch

from ..linear import div_even
from .fused import AWQMoeWeights, process_awq_moe_weights

_AWQ_NAMES = ("qweight", "qzeros", "scales")


def _concat_prefix(prefix: str, name: str) -> str:
    return f"{prefix}.{name}" if prefix else name


class AWQExpertStack:
    """One projection's expert-stacked AWQ tensors: [E, K, N/8], [E, K/G, N/8], [E, K/G, N]."""

    def __init__(self, num_experts: int, input_size: int, output_size: int, group_size: int,
                 params_dtype: torch.dtype):
        G = input_size if group_size == -1 else group_size
        if input_size % G:
            raise ValueError(f"The input size {input_size} is not aligned with the quantized weight shape. "
                             f"This can be caused by too large tensor parallel size.")
        if output_size % 8:
            raise ValueError(f"The output size {output_size} is not aligned with the quantized weight shape. "
                             f"This can be caused by too large tensor parallel size.")
        self.input_size, self.output_size, self.group_size = input_size, output_size, G
        E = num_experts
        self.qweight = torch.empty((E, input_size, output_size // 8), dtype=torch.int32, device="meta")
        self.qzeros = torch.empty((E, input_size // G, output_size // 8), dtype=torch.int32, device="meta")
        self.scales = torch.empty((E, input_size // G, output_size), dtype=params_dtype, device="meta")
        self._weights: Optional[AWQMoeWeights] = None

    @property
    def weights(self) -> AWQMoeWeights:
        if self._weights is None:
            raise RuntimeError("expert weights are not loaded (call load_state_dict first)")
        return self._weights

    def state_dict(self, prefix: str = "", result: Optional[Dict[str, torch.Tensor]] = None):
        result = result if result is not None else {}
        for name in _AWQ_NAMES:
            result[_concat_prefix(prefix, name)] = getattr(self, name)
        return result

    def take(self, state_dict: Dict[str, torch.Tensor], prefix: str = "") -> Dict[str, torch.Tensor]:
        """This stack's three tensors from ``state_dict``, checked against the expected
        shapes and dtypes; nothing is removed from ``state_dict``."""
        items = {}
        for name in _AWQ_NAMES:
            key = _concat_prefix(prefix, name)
            if key not in state_dict:
                raise KeyError(key)
            param, item = getattr(self, name), state_dict[key]
            assert isinstance(item, torch.Tensor)
            assert param.shape == item.shape and param.dtype == item.dtype, (
                f"{key}: expected {tuple(param.shape)} {param.dtype}, got {tuple(item.shape)} {item.dtype}")
            items[name] = item
        return items

    def process(self, items: Dict[str, torch.Tensor]) -> None:
        """Post-load repack of checked tensors into the tile layout (on their device)."""
        self._weights = process_awq_moe_weights(items["qweight"], items["qzeros"], items["scales"])


class AWQMoELayer:
    """Experts of one MoE block with AWQ W4A16 weights (MoELayer, moe_layer.py:11-64)."""

    def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 renormalize: bool = True, activation: str = "silu", apply_router_weight_on_input: bool = False,
                 group_size: int = 128, params_dtype: torch.dtype = torch.float16, tp_size: int = 1,
                 process_group=None, backend: str = "awq_fused"):
        if activation not in ("silu", "gelu"):
            raise ValueError(f"unsupported activation {activation!r}")
        if not 1 <= top_k <= num_experts:
            raise ValueError(f"top_k must be in [1, {num_experts}], got {top_k}")
        self.num_experts = num_experts
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.renormalize = renormalize
        self.activation = activation
        self.apply_router_weight_on_input = apply_router_weight_on_input
        self.tp_size = tp_size
        self._group = process_group
        local = div_even(intermediate_size, tp_size)
        if local % 16:
            raise ValueError(f"the per-rank intermediate size {local} must be a multiple of 16 "
                             "(gate/up pairs are combined in 16-column tiles)")
        self.intermediate_size_per_partition = local
        self.gate_up_proj = AWQExpertStack(num_experts, hidden_size, 2 * local, group_size, params_dtype)
        self.down_proj = AWQExpertStack(num_experts, local, hidden_size, group_size, params_dtype)
        from . import create_moe_backend

        self._backend = create_moe_backend(backend)

    def state_dict(self, *, prefix: str = "", result: Optional[Dict[str, torch.Tensor]] = None):
        result = result if result is not None else {}
        self.gate_up_proj.state_dict(_concat_prefix(prefix, "gate_up_proj"), result)
        self.down_proj.state_dict(_concat_prefix(prefix, "down_proj"), result)
        return result

    def state_dict_keys(self, prefix: str = "") -> List[str]:
        return list(self.state_dict(prefix=prefix).keys())

    def load_state_dict(self, state_dict: Dict[str, torch.Tensor], *, prefix: str = "",
                        _internal: bool = False) -> None:
        stacks = ((self.gate_up_proj, _concat_prefix(prefix, "gate_up_proj")),
                  (self.down_proj, _concat_prefix(prefix, "down_proj")))
        items = [stack.take(state_dict, p) for stack, p in stacks]  # check everything before any work
        for _, p in stacks:
            for name in _AWQ_NAMES:
                state_dict.pop(_concat_prefix(p, name))
        for (stack, _), it in zip(stacks, items):
            stack.process(it)
        if not _internal and state_dict:
            raise RuntimeError(f"Unexpected keys in state_dict: {list(state_dict.keys())}")

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        """Route ``hidden_states [T, H]`` by ``router_logits [T, E]`` through the experts."""
        out = self._backend.forward(hidden_states=hidden_states, w1=self.gate_up_proj.weights,
                                    w2=self.down_proj.weights, gating_output=router_logits, topk=self.top_k,
                                    renormalize=self.renormalize, activation=self.activation,
                                    apply_router_weight_on_input=self.apply_router_weight_on_input)
        if self.tp_size > 1:
            torch.distributed.all_reduce(out, group=self._group)
        return out

    __call__ = forward
