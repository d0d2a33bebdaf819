"""ctypes binding of libsglite_awq.so (the C ABI in include/sglite_awq.h).

The library is built in-tree by ``__graft_entry__.build()`` (or
``make -C sglite_amd/csrc``).  There is no fallback: if the library is missing
every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsglite_awq.so")

AWQ_STATUS_OK = 0
AWQ_STATUS_INVALID_ARGUMENT = -1
AWQ_STATUS_UNSUPPORTED = -2
AWQ_STATUS_HIP_ERROR = -3
AWQ_STATUS_WORKSPACE = -4

AWQ_DTYPE_FP16 = 0
AWQ_DTYPE_BF16 = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES = {
    "awq_last_error": (ctypes.c_char_p, []),
    "awq_version": (ctypes.c_char_p, []),
    "awq_abi_version": (_int, []),
    "awq_repacked_weight_bytes": (_i64, [_i64, _i64]),
    "awq_repacked_scale_bytes": (_i64, [_i64, _i64, _i64]),
    "awq_repacked_zero_bytes": (_i64, [_i64, _i64, _i64]),
    "awq_repack_cdna4": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "awq_unrepack_cdna4": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "awq_dequant": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _vp]),
    "awq_dequant_repacked": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _vp]),
    "awq_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "awq_counter_bytes": (_i64, [_i64]),
    "awq_gemm_kernel_kind": (_int, [_i64, _i64, _i64, _i64]),
    "awq_w4a16_gemm": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _i64,
                              _vp]),
    "awq_noalloc_init": (_int, [_vp]),
    "awq_w4a16_gemm_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp]),
    "awq_workspace_bytes_act": (_i64, [_i64, _i64, _i64, _i64]),
    "awq_gemm_kernel_kind_act": (_int, [_i64, _i64, _i64, _i64]),
    "awq_w4a16_gemm_act": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _vp, _i64, _vp,
                                  _i64, _vp]),
    "awq_gated_mlp_plan": (_int, [_i64, _i64, _i64, _i64, _int, ctypes.POINTER(_i64)]),
    "awq_gated_mlp_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "awq_gated_mlp": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _int, _vp,
                             _i64, _vp, _i64, _vp]),
    "awq_gated_mlp_take_errors": (_i64, [_vp, _i64, _vp]),
    "awq_set_plan_override": (_int, [_int, _int]),
    "awq_clear_plan_overrides": (None, []),
    "awq_device_cu_count": (_int, []),
    "awq_gemm_plan_info": (_int, [_i64, _i64, _i64, _i64, _int, ctypes.POINTER(_i64)]),
    "awq_gemm_plan_fixup": (_int, [_i64, _i64, _i64, _i64, _int]),
    "awq_stream_probe": (_int, [_vp, _i64, _i64, _int, _vp, _i64, _vp]),
    "awq_mfma_probe": (_int, [_i64, _i64, _int, _vp, _i64, _vp]),
    "awq_moe_expert_strides": (_int, [_i64, _i64, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                      ctypes.POINTER(_i64)]),
    "awq_moe_topk_softmax": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "awq_moe_sorted_capacity": (_i64, [_i64, _i64, _i64]),
    "awq_moe_block_capacity": (_i64, [_i64, _i64, _i64]),
    "awq_moe_align_block_size": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "awq_moe_w4a16_gemm": (_int, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _vp, _i64,
                                  _i64, _int, _int, _vp, _vp]),
    "awq_moe_sum_reduce": (_int, [_vp, _vp, _i64, _i64, _i64, _int, _vp]),
}

AWQ_ACT_SILU = 1
AWQ_ACT_GELU = 2

AWQ_PLAN_GEMV_MAX_M = 0
AWQ_PLAN_GEMV_VARIANT = 1
AWQ_PLAN_GEMV_KS = 2
AWQ_PLAN_SKINNY_VARIANT = 3
AWQ_PLAN_SKINNY_KS = 4
AWQ_PLAN_TILED_MIN_M = 5
AWQ_PLAN_TILED_BM = 6
AWQ_PLAN_TILED_KS = 7
AWQ_PLAN_KSLICE_VARIANT = 8
AWQ_PLAN_TILED_FIXUP = 9
AWQ_PLAN_FIXUP_POLLS = 10

# The header revision this binding follows (AWQ_ABI_VERSION).
AWQ_ABI_VERSION = 4
# Split-tile counters ahead of the per-column-tile counters (AWQ_COUNTER_TILE_BYTES).
AWQ_COUNTER_TILE_BYTES = 64 << 10

# Counters of the one-launch gated MLP block (AWQ_MLP_COUNTER_BYTES) and its default poll bound.
AWQ_MLP_COUNTER_BYTES = 64 << 10
AWQ_MLP_DEFAULT_POLLS = 1 << 15

AWQ_NOALLOC_WORKSPACE_BYTES = 64 << 20
AWQ_NOALLOC_MAX_N = 1 << 20

AWQ_MOE_ACT_NONE = 0
AWQ_MOE_ACT_SILU = 1
AWQ_MOE_ACT_GELU = 2

_lib: Optional[ctypes.CDLL] = None


class AWQKernelError(RuntimeError):
    """A HIP-side failure reported by the C ABI."""


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once; raise RuntimeError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: the AWQ HIP engine is not built "
            "(run __graft_entry__.build() or `make -C sglite_amd/csrc`)."
        )
    lib = ctypes.CDLL(path)
    # A library built from another header revision would take these
    # argument lists differently: refuse it before binding anything.
    abi = getattr(lib, "awq_abi_version", None)
    found = abi() if abi is not None else 1
    if found != AWQ_ABI_VERSION:
        raise RuntimeError(f"{path} implements AWQ ABI {found}, this binding needs {AWQ_ABI_VERSION}: rebuild it")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().awq_last_error().decode()


def check(status: int, what: str) -> int:
    """Map a C-ABI status to the reference's exception types.

    Shape/config problems raise ValueError, as the reference's linear methods
    do (python/sglite/srt/model_executor/layers/quantization/awq.py:76-85);
    everything else raises RuntimeError.
    """
    if status >= 0:
        return status
    msg = f"{what}: {last_error()}"
    if status == AWQ_STATUS_INVALID_ARGUMENT:
        raise ValueError(msg)
    if status == AWQ_STATUS_HIP_ERROR:
        raise AWQKernelError(msg)
    raise RuntimeError(msg)
