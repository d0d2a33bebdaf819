"""Quantized linear methods of SGLite, served by the gfx950 AWQ engine.

Same exports and lazy-import behaviour as
python/sglite/srt/model_executor/layers/quantization/__init__.py:10-55: the
base types import eagerly; the AWQ methods, which load the HIP library, import
on first use.  Both method names ("awq", "awq_marlin") run the same kernels.
"""

from .base_config import LinearMethodBase, QuantizationConfig, set_weight_attrs
from .unquant import UnquantizedLinearMethod


def get_quantization_config(method_name: str) -> type:
    """Config class for a method name; ValueError for unknown names (quantization/__init__.py:15-29)."""
    method_name = method_name.lower()
    if method_name == "awq":
        from .awq import AWQConfig

        return AWQConfig
    if method_name == "awq_marlin":
        from .awq_marlin import AWQMarlinConfig

        return AWQMarlinConfig
    raise ValueError(f"Unknown quantization method: {method_name!r}. Supported methods: ['awq', 'awq_marlin']")


def __getattr__(name: str):
    if name in ("AWQConfig", "AWQLinearMethod"):
        from . import awq

        return getattr(awq, name)
    if name in ("AWQMarlinConfig", "AWQMarlinLinearMethod"):
        from . import awq_marlin

        return getattr(awq_marlin, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


__all__ = [
    "AWQConfig",
    "AWQLinearMethod",
    "AWQMarlinConfig",
    "AWQMarlinLinearMethod",
    "LinearMethodBase",
    "QuantizationConfig",
    "UnquantizedLinearMethod",
    "set_weight_attrs",
    "get_quantization_config",
]
