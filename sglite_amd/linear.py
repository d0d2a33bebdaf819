"""Tensor-parallel linear layers that drive a linear method's lifecycle.

Mirror of python/sglite/srt/model_executor/layers/linear.py:15-194 (the caller
side of the plugin boundary):

* construction calls ``create_weights(local_in, local_out)`` and keeps
  ``_``-prefixed entries out of the state dict (linear.py:32-45);
* ``load_state_dict`` pops this layer's tensors with exact shape/dtype checks,
  re-points the method's weight map, restores metadata and runs
  ``process_weights_after_loading`` once, re-binding only attributes that
  already exist (linear.py:50-99);
* ``forward`` is ``apply_weights(weights, x, bias)``; a row-parallel layer
  all-reduces its partial output when tp_size > 1 (linear.py:101-103, 189-194).

Tensor-parallel sizes are explicit arguments here (tp_rank, tp_size) instead
of the reference's process-group globals.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch

from .quantization import LinearMethodBase, UnquantizedLinearMethod


def div_even(a: int, b: int, allow_replicate: bool = False) -> int:
    """a / b, which must divide evenly; with ``allow_replicate`` a < b gives 1."""
    if allow_replicate and a < b:
        if b % a:
            raise ValueError(f"{b} is not a multiple of {a}")
        return 1
    if a % b:
        raise ValueError(f"{a} is not divisible by {b}")
    return a // b


def _concat_prefix(prefix: str, name: str) -> str:
    return f"{prefix}.{name}" if prefix else name


class _TPLinearBase:
    def __init__(self, full_isize: int, full_osize: int, local_isize: int, local_osize: int, has_bias: bool,
                 linear_method: Optional[LinearMethodBase] = None, tp_size: int = 1):
        self.full_input_size = full_isize
        self.full_output_size = full_osize
        self.local_input_size = local_isize
        self.local_output_size = local_osize
        self._tp_size = tp_size
        self._linear_method = linear_method or UnquantizedLinearMethod()
        self._weights: Dict[str, Any] = self._linear_method.create_weights(local_isize, local_osize)
        self._weight_metadata: Dict[str, Any] = {}
        for name in list(self._weights.keys()):
            if name.startswith("_"):
                self._weight_metadata[name] = self._weights.pop(name)
        for name, tensor in self._weights.items():
            setattr(self, name, tensor)
        self.bias = torch.empty(local_osize) if has_bias else None
        self._weights_processed = False

    def state_dict_keys(self, prefix: str = "") -> List[str]:
        return [_concat_prefix(prefix, n) for n, v in self.__dict__.items()
                if not n.startswith("_") and isinstance(v, torch.Tensor)]

    def load_state_dict(self, state_dict: Dict[str, torch.Tensor], *, prefix: str = "", _internal: bool = False) -> None:
        for name, param in list(self.__dict__.items()):
            if name.startswith("_") or not isinstance(param, torch.Tensor):
                continue
            item = state_dict.pop(_concat_prefix(prefix, name))
            assert isinstance(item, torch.Tensor)
            assert param.shape == item.shape and param.dtype == item.dtype, (
                f"{name}: expected {tuple(param.shape)} {param.dtype}, got {tuple(item.shape)} {item.dtype}")
            setattr(self, name, item)
        for name in list(self._weights.keys()):
            if hasattr(self, name):
                self._weights[name] = getattr(self, name)
        for name, value in self._weight_metadata.items():
            self._weights[name] = value
        if not self._weights_processed:
            processed = self._linear_method.process_weights_after_loading(self._weights)
            self._weight_metadata = {}
            for name, value in processed.items():
                if name.startswith("_"):
                    self._weight_metadata[name] = value
                else:
                    self._weights[name] = value
                    if hasattr(self, name):  # runtime tensors (workspace) stay out of the state dict
                        setattr(self, name, value)
            self._weights.update(self._weight_metadata)
            self._weights_processed = True
        if not _internal and state_dict:
            raise RuntimeError(f"Unexpected keys in state_dict: {list(state_dict.keys())}")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._linear_method.apply_weights(self._weights, x, self.bias)

    __call__ = forward


class ReplicatedLinear(_TPLinearBase):
    def __init__(self, input_size: int, output_size: int, has_bias: bool,
                 linear_method: Optional[LinearMethodBase] = None):
        super().__init__(input_size, output_size, input_size, output_size, has_bias, linear_method)


class MergedColumnParallelLinear(_TPLinearBase):
    """Fused column-parallel projection (gate_up): local N = sum(size / tp) (linear.py:127-143)."""

    def __init__(self, input_size: int, output_sizes: List[int], has_bias: bool,
                 linear_method: Optional[LinearMethodBase] = None, tp_size: int = 1):
        tp_sizes = [div_even(s, tp_size) for s in output_sizes]
        super().__init__(input_size, sum(output_sizes), input_size, sum(tp_sizes), has_bias, linear_method, tp_size)

    def forward_act(self, x: torch.Tensor, activation: str) -> torch.Tensor:
        """act(gate) * up of a two-part (gate, up) projection: the layer's forward
        followed by silu_and_mul / gelu_and_mul (blocks.py:53-55), fused into the
        GEMM when the linear method has a fused kernel."""
        return self._linear_method.apply_weights_act(self._weights, x, activation, self.bias)


class QKVParallelLinear(_TPLinearBase):
    """Fused q/k/v projection: local N = (Hq/tp + 2 Hkv/tp) * d (linear.py:146-168)."""

    def __init__(self, hidden_size: int, head_dim: int, num_qo_heads: int, num_kv_heads: int, has_bias: bool,
                 linear_method: Optional[LinearMethodBase] = None, tp_size: int = 1):
        local_qo = div_even(num_qo_heads, tp_size)
        local_kv = div_even(num_kv_heads, tp_size, allow_replicate=True)
        super().__init__(hidden_size, (num_qo_heads + 2 * num_kv_heads) * head_dim, hidden_size,
                         (local_qo + 2 * local_kv) * head_dim, has_bias, linear_method, tp_size)


class RowParallelLinear(_TPLinearBase):
    """Row-parallel projection (o, down): local K = K / tp, all-reduce of the output (linear.py:171-194)."""

    def __init__(self, input_size: int, output_size: int, has_bias: bool,
                 linear_method: Optional[LinearMethodBase] = None, tp_size: int = 1, process_group=None):
        self._group = process_group
        super().__init__(input_size, output_size, div_even(input_size, tp_size), output_size, has_bias,
                         linear_method, tp_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self._linear_method.apply_weights(self._weights, x, self.bias)
        if self._tp_size > 1:
            torch.distributed.all_reduce(y, group=self._group)
        return y

    __call__ = forward
