"""Fused MoE forward with AWQ W4A16 experts.

Follows python/sglite/srt/model_executor/layers/fused_moe/fused.py:
  fused_topk            fused.py:11-31   (topk_softmax + renormalise)
  moe_align_block_size  fused.py:34-61   (sort routed rows by expert, pad buckets)
  get_default_config    fused.py:64-86
  fused_experts_impl    fused.py:101-202 (GEMM1 -> act_and_mul -> GEMM2 x routed
                                          weight -> top-k sum into hidden_states)
  FusedMoe.forward      fused.py:207-233
Every stage runs in the HIP kernels of libsglite_awq.so; the gate/up
activation is fused into the first grouped GEMM's epilogue and the routed
weight into the second's.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Dict, NamedTuple, Optional, Tuple

import torch

from .. import ops

# Routed rows per MFMA tile: the grouped GEMM works on 16-row blocks.
BLOCK_SIZE_M = 16


class AWQMoeWeights(NamedTuple):
    """One expert stack after the post-load repack."""
    experts: ops.RepackedExperts
    input_size: int    # K per expert
    output_size: int   # N per expert
    group_size: int

    @property
    def num_experts(self) -> int:
        return self.experts.w.shape[0]


def process_awq_moe_weights(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor) -> AWQMoeWeights:
    """Expert-stacked AWQ checkpoint tensors ``[E, K, N/8]`` / ``[E, K/G, N/8]`` / ``[E, K/G, N]``
    (experts stacked on dim 0 as the reference's loader does, weight_loader.py:134-142)
    -> the tile layout, on the device."""
    E, K, N8 = qweight.shape
    G = K // qzeros.shape[1]
    return AWQMoeWeights(ops.repack_experts(qweight, qzeros, scales), K, N8 * 8, G)


def fused_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor, topk: int, renormalize: bool,
               num_token_non_padded: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k routing (fused.py:11-31): fp32 weights ``[T, topk]`` and int32 expert ids."""
    assert hidden_states.shape[0] == gating_output.shape[0], "Number of tokens mismatch"
    topk_weights, topk_ids = ops.moe_topk_softmax(gating_output, topk, renormalize)
    if num_token_non_padded is not None:
        indices = torch.arange(0, topk_ids.shape[0], device=topk_ids.device)
        topk_ids[indices >= num_token_non_padded, :] = -1
    return topk_weights, topk_ids


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int,
                         num_experts: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(sorted_ids, expert_ids, num_tokens_post_pad) as fused.py:34-61 returns them, plus the
    padded bucket offsets ``[E + 1]`` the grouped GEMM reads.  Padding entries hold
    ``topk_ids.numel()``; ids outside ``[0, num_experts)`` are dropped."""
    a = ops.moe_align_block_size(topk_ids, block_size, num_experts)
    return a.sorted_ids, a.expert_ids, a.num_tokens_post_pad, a.expert_offsets


def get_default_config(M: int, E: int, N: int, K: int, topk: int) -> Dict[str, int]:
    """Kernel configuration (fused.py:64-86).  The grouped W4A16 kernel tiles the
    routed rows in 16-row MFMA blocks and chooses its column slices itself."""
    return {"BLOCK_SIZE_M": BLOCK_SIZE_M}


def fused_experts_impl(hidden_states: torch.Tensor, w1: AWQMoeWeights, w2: AWQMoeWeights, topk_weights: torch.Tensor,
                       topk_ids: torch.Tensor, activation: str = "silu",
                       apply_router_weight_on_input: bool = False) -> torch.Tensor:
    """Run alignment, both grouped GEMMs and the top-k sum; writes into ``hidden_states``
    and returns it, as fused.py:101-202 does."""
    if activation not in ("silu", "gelu"):
        raise ValueError(f"unsupported activation {activation!r}")
    assert hidden_states.shape[1] == w1.input_size, "Hidden size mismatch"
    assert topk_weights.shape == topk_ids.shape, "topk shape mismatch"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert hidden_states.dtype in (torch.float16, torch.bfloat16)
    assert w1.num_experts == w2.num_experts, "expert counts differ"
    assert w2.input_size == w1.output_size // 2, "w2's input size must be half of w1's output size"
    assert w2.output_size == hidden_states.shape[1], "w2's output size must equal the hidden size"
    T, H = hidden_states.shape
    top_k = topk_ids.shape[1]
    E = w1.num_experts
    num_routed = T * top_k
    if num_routed == 0:
        return hidden_states
    config = get_default_config(T, E, w1.output_size, w1.input_size, top_k)
    align = ops.moe_align_block_size(topk_ids.to(torch.int32), config["BLOCK_SIZE_M"], E)
    # First GEMM: gate/up, routed row r reads token r // top_k; act(gate) * up
    # fused into the epilogue (intermediate_cache1 -> intermediate_cache2).
    cache2 = ops.moe_gemm(hidden_states, w1.experts, w1.input_size, w1.output_size, w1.group_size, align, topk_weights,
                          num_routed, top_k, activation=activation, mul_routed_weight=apply_router_weight_on_input)
    # Second GEMM: down, routed row r reads cache2[r]; the routed weight is
    # applied in fp32 before the cast (MUL_ROUTED_WEIGHT = not on input).
    cache3 = ops.moe_gemm(cache2, w2.experts, w2.input_size, w2.output_size, w2.group_size, align, topk_weights,
                          num_routed, 1, activation=None, mul_routed_weight=not apply_router_weight_on_input)
    ops.moe_sum_reduce(cache3.view(T, top_k, H), hidden_states)
    return hidden_states


class BaseMoeBackend(ABC):
    """MoE backend interface (fused_moe/base.py:8-26)."""

    @abstractmethod
    def forward(self, hidden_states: torch.Tensor, w1, w2, gating_output: torch.Tensor, topk: int, renormalize: bool,
                activation: str, apply_router_weight_on_input: bool) -> torch.Tensor:
        ...


class AWQFusedMoe(BaseMoeBackend):
    """Fused MoE backend over AWQ expert stacks (FusedMoe, fused.py:205-233)."""

    def forward(self, hidden_states: torch.Tensor, w1: AWQMoeWeights, w2: AWQMoeWeights, gating_output: torch.Tensor,
                topk: int, renormalize: bool, activation: str = "silu",
                apply_router_weight_on_input: bool = False) -> torch.Tensor:
        topk_weights, topk_ids = fused_topk(hidden_states=hidden_states, gating_output=gating_output, topk=topk,
                                            renormalize=renormalize)
        return fused_experts_impl(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                                  apply_router_weight_on_input=apply_router_weight_on_input)
