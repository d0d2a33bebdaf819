"""Grouped W4A16 MoE backend (AWQ experts on the gfx950 engine).

Mirrors the fused MoE backend interface of
python/sglite/srt/model_executor/layers/fused_moe/ (registry __init__.py:22-35,
BaseMoeBackend base.py:8-26, FusedMoe fused.py:205-233) with AWQ expert stacks
in place of the dense ``[E, 2I, H]`` / ``[E, H, I]`` weights.
"""

from __future__ import annotations

from typing import Callable, Dict

from .fused import (AWQFusedMoe, AWQMoeWeights, BaseMoeBackend, fused_experts_impl, fused_topk, get_default_config,
                    moe_align_block_size, process_awq_moe_weights)

SUPPORTED_MOE_BACKENDS: Dict[str, Callable[[], BaseMoeBackend]] = {"awq_fused": AWQFusedMoe}


def create_moe_backend(backend: str) -> BaseMoeBackend:
    """Create a registered MoE backend by name (fused_moe/__init__.py:32-34)."""
    try:
        return SUPPORTED_MOE_BACKENDS[backend]()
    except KeyError:
        raise ValueError(f"unknown MoE backend {backend!r}; registered: {sorted(SUPPORTED_MOE_BACKENDS)}") from None


from .layer import AWQExpertStack, AWQMoELayer  # noqa: E402  (the layer resolves backends by name)

__all__ = [
    "AWQExpertStack",
    "AWQFusedMoe",
    "AWQMoELayer",
    "AWQMoeWeights",
    "BaseMoeBackend",
    "SUPPORTED_MOE_BACKENDS",
    "create_moe_backend",
    "fused_experts_impl",
    "fused_topk",
    "get_default_config",
    "moe_align_block_size",
    "process_awq_moe_weights",
]
