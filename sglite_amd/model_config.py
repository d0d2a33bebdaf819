"""AWQ quantization-config detection.

Mirror of python/sglite/srt/model_executor/models/config.py:28-89
(``load_quantization_config``, ``_create_awq_config``): the AWQ config comes
from ``hf_config.quantization_config`` or, failing that, from
``quant_config.json`` / ``quantize_config.json`` in a local model directory.
AWQ is recognised by ``quant_method == "awq"`` or, with no method given, by a
``w_bit``/``bits`` key.  The reference then prefers the Marlin method and
falls back to Triton; here both methods run the same gfx950 kernels, and the
same preference decides only which config class (and so which shape rules and
metadata) the model gets.  Remote hub lookups are not performed.
"""

from __future__ import annotations

import json
import logging
import os
from typing import Any, Dict, Optional

logger = logging.getLogger(__name__)


def load_quantization_config(model_path: str, hf_config: Optional[Any] = None,
                             force_awq_triton: bool = False) -> Optional[Any]:
    config_dict = None
    if hf_config is not None:
        quant_cfg = getattr(hf_config, "quantization_config", None)
        if quant_cfg is None and isinstance(hf_config, dict):
            quant_cfg = hf_config.get("quantization_config")
        if quant_cfg is not None:
            if hasattr(quant_cfg, "to_dict"):
                config_dict = quant_cfg.to_dict()
            elif isinstance(quant_cfg, dict):
                config_dict = quant_cfg
    if config_dict is None:
        if not os.path.isdir(model_path):
            return None
        for name in ("quant_config.json", "quantize_config.json"):
            path = os.path.join(model_path, name)
            if os.path.exists(path):
                with open(path, "r") as f:
                    config_dict = json.load(f)
                break
    if config_dict is None:
        return None
    quant_method = config_dict.get("quant_method", "").lower()
    is_awq = quant_method == "awq" or (not quant_method and ("w_bit" in config_dict or "bits" in config_dict))
    if is_awq:
        return _create_awq_config(config_dict, force_awq_triton)
    return None


def _create_awq_config(config_dict: Dict[str, Any], force_awq_triton: bool = False) -> Any:
    from .quantization.awq import AWQConfig
    from .quantization.awq_marlin import AWQMarlinConfig

    if not force_awq_triton and AWQMarlinConfig.is_awq_marlin_compatible(config_dict):
        try:
            cfg = AWQMarlinConfig.from_config(config_dict)
            logger.info("Using the gfx950 AWQ engine (awq_marlin method).")
            return cfg
        except Exception as e:  # same fallback as the reference
            logger.debug("awq_marlin setup failed, using the awq method: %s", e)
    cfg = AWQConfig.from_config(config_dict)
    logger.info("Using the gfx950 AWQ engine (awq method).")
    return cfg
