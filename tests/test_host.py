"""CPU tests of the host side: the C ABI library loads and exports every
declared symbol, argument validation maps to the reference's exception types,
and the plugin API (configs, linear methods, linear plumbing, config
detection) behaves like python/sglite/srt/model_executor/layers/quantization/*
and models/config.py.  No test here launches GPU work."""

import ctypes
import json
import os
import re

import numpy as np
import pytest
import torch

from oracle import awq_oracle as oracle
from sglite_amd import _lib, ops
from sglite_amd.quantization import (LinearMethodBase, QuantizationConfig, UnquantizedLinearMethod,
                                     get_quantization_config, set_weight_attrs)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sglite_awq.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(awq_[a-z0-9_]+)\s*\(", text)))


# --------------------------------------------------------------------------
# C ABI
# --------------------------------------------------------------------------

def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert set(_lib.SIGNATURES) == set(declared)


def test_version_and_empty_error():
    lib = _lib.load()
    assert lib.awq_version().decode().startswith("sglite-awq-gfx950")


@pytest.mark.parametrize("K,N,G", [(2560, 6144, 128), (96, 24, 32), (384, 40, -1), (4096, 28672, 64)])
def test_size_queries_match_layout(K, N, G):
    lib = _lib.load()
    Gr = K if G == -1 else G
    sh = oracle.repacked_shapes(K, N, Gr)
    assert lib.awq_repacked_weight_bytes(K, N) == sh["w_bytes"]
    assert lib.awq_repacked_scale_bytes(K, N, G) == sh["s_bytes"]
    assert lib.awq_repacked_zero_bytes(K, N, G) == sh["z_bytes"]
    # the tiled kernels' split-tile counters, then one int32 per column tile
    assert lib.awq_counter_bytes(N) == _lib.AWQ_COUNTER_TILE_BYTES + 4 * ((N + 15) // 16)
    assert lib.awq_workspace_bytes(0, N, K, G) == 0


def test_workspace_query_is_bounded():
    lib = _lib.load()
    for (K, N) in [(2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560)]:
        for M in (1, 8, 32):
            ws = lib.awq_workspace_bytes(M, N, K, 128)
            assert ws >= 0
            assert ws % (4 * M * 16) == 0
            # split-K partials stay well below the int4 weight stream
            assert ws <= K * N // 2
        # prefill kernel: scratch only when it splits K (small grids), then
        # ks slices of fp32 partials, 2 <= ks <= 16
        NT = (N + 15) // 16
        for M in (64, 512, 2048):
            ws = lib.awq_workspace_bytes(M, N, K, 128)
            ks, rem = divmod(ws, M * NT * 16 * 4)
            assert rem == 0 and (ks == 0 or 2 <= ks <= 16)
    assert lib.awq_workspace_bytes(8192, 28672, 4096, 128) == 0  # full grids never split


@pytest.mark.parametrize("K,N,routes", [
    (2560, 6144, "g" * 16),                    # Qwen3-4B qkv: short K, GEMV throughout
    (4096, 2560, "g" * 4 + "s" * 12),          # Qwen3-4B o_proj: narrow, 32 k-tiles
    (2560, 19456, "g" * 16),                   # Qwen3-4B gate_up: short K stays on the GEMV kernel
    (9728, 2560, "g" * 9 + "t" * 7),           # Qwen3-4B down: 76 k-tiles on 160 column tiles, tiled from 10 rows
    (4096, 6144, "g" * 16),                    # Llama-3-8B qkv
    (4096, 28672, "g" * 4 + "ss" + "gg" + "t" * 8),  # Llama-3-8B gate_up: wide; two-tile GEMV at 7-8 rows
    (14336, 4096, "g" * 4 + "t" * 12),         # Llama-3-8B down: deep, 32-row 32x32 kernel from 5 rows
    (8192, 10240, "g" * 4 + "t" * 12),         # Llama-3-70B qkv
    (8192, 57344, "gg" + "s" * 6 + "t" * 8),   # Llama-3-70B gate_up: very wide
    (28672, 8192, "g" * 4 + "t" * 12),         # Llama-3-70B down
    (4096, 1536, "g" * 8 + "s" * 8),           # Llama-3-8B qkv at TP4: < 128 column tiles
    (8192, 1280, "g" * 8 + "sss" + "t" * 5),   # Llama-3-70B qkv at TP8: < 128 column tiles, 64 k-tiles
])
def test_decode_routing(K, N, routes):
    """Kernel choice for 1..16 rows (g = GEMV, s = skinny decode kernel, t = tiled)."""
    names = {"g": "gemv_kernel", "s": "skinny_kernel", "t": "tiled_kernel"}
    got = "".join(next(k for k, v in names.items() if v == ops.gemm_kernel(M, N, K, 128))
                  for M in range(1, len(routes) + 1))
    assert got == routes, (K, N)


def test_routing_at_17_to_32_rows():
    """17-32 rows: short K on layers of >= 384 column tiles stays on the GEMV
    kernel while its activation slice fits unsplit (25 rows on the Qwen3-4B
    qkv, 24 on its gate_up); narrow layers with deep K (>= 48 k-tiles, or >= 32
    on < 128 column tiles) split K on the 32-row tiled kernel; o_proj-shaped
    layers (32 k-tiles, <= 256 column tiles) keep the skinny kernel up to 27
    rows.  The planner never picks the k-slice kernel; the override does."""
    for M in (17, 20, 24):
        assert ops.gemm_kernel(M, 6144, 2560, 128) == "gemv_kernel"
        assert ops.gemm_kernel(M, 19456, 2560, 128) == "gemv_kernel"
        assert ops.gemm_kernel(M, 2560, 4096, 128) == "skinny_kernel"
    assert ops.gemm_kernel(25, 6144, 2560, 128) == "gemv_kernel"
    assert ops.workspace_bytes(25, 6144, 2560, 128) == 0
    assert ops.gemm_kernel(25, 19456, 2560, 128) == "tiled_kernel"
    for M in (26, 28, 32):
        assert ops.gemm_kernel(M, 6144, 2560, 128) == "tiled_kernel"
    for M in (28, 32):
        assert ops.gemm_kernel(M, 2560, 4096, 128) == "tiled_kernel"
    for M in (17, 24, 32):
        assert ops.gemm_kernel(M, 2560, 9728, 128) == "tiled_kernel"  # 76 k-tiles
        assert ops.gemm_kernel(M, 4096, 7168, 128) == "tiled_kernel"  # 56 k-tiles
        assert ops.gemm_kernel(M, 1536, 4096, 128) == "tiled_kernel"  # 96 column tiles
        assert ops.gemm_kernel(M, 4096, 3584, 128) == "skinny_kernel"  # 28 k-tiles
    for M in range(1, 33):
        for K, N in ((4096, 2560), (9728, 2560), (4096, 4096), (7168, 4096)):
            assert ops.gemm_kernel(M, N, K, 128) != "kslice_kernel"
    with ops.plan_overrides(kslice_variant=142):
        info = ops.plan_info(32, 2560, 4096, 128)
        assert info.kernel == "kslice_kernel" and info.variant == 142 and info.k_slices == 4
        assert info.workgroups == 160


def test_gemv_keeps_deep_k_unsplit_at_few_rows():
    """Up to 128 k-tiles one GEMV workgroup covers K at 1-3 rows (no split-K
    workspace), 33-128 at 4 rows, and 65-80 k-tiles up to 6 rows; beyond that
    the 8-wave plans split K again."""
    for K in (4224, 6144, 8192, 9728, 11008, 14336):
        for M in (1, 2, 3):
            assert ops.gemm_kernel(M, 4096, K, 128) == "gemv_kernel"
            assert ops.workspace_bytes(M, 4096, K, 128) == 0, (M, K)
    for M in (4, 5, 6):
        assert ops.workspace_bytes(M, 2560, 9728, 128) == 0, M
    assert ops.workspace_bytes(8, 2560, 9728, 128) > 0
    assert ops.workspace_bytes(4, 4096, 14336, 128) == 0
    assert ops.workspace_bytes(5, 4096, 14336, 128) > 0
    assert ops.workspace_bytes(1, 8192, 28672, 128) > 0  # 224 k-tiles still split


def test_tensor_parallel_shard_routing():
    """Shapes the planner was not tuned on (one GPU's share of tensor-parallel
    linears): short K goes to the skinny kernel up to 16 rows, very narrow
    layers keep K unsplit on the GEMV kernel, and the GEMV kernel's two-tile
    workgroups need at least 384 column tiles."""
    assert ops.gemm_kernel(1, 8192, 1024, 128) == "skinny_kernel"   # 70B o_proj at TP8
    assert ops.plan_info(1, 8192, 1024, 128).variant == 10202
    assert ops.plan_info(8, 4096, 1024, 128).variant == 10116       # Llama-3-8B o_proj at TP4
    assert ops.gemm_kernel(32, 8192, 1024, 128) == "gemv_kernel"
    info = ops.plan_info(8, 1536, 4096, 128)                        # Llama-3-8B qkv at TP4
    assert info.kernel == "gemv_kernel" and info.k_slices == 1
    assert ops.plan_info(8, 1280, 8192, 128).variant == 11084       # 70B qkv at TP8: one tile per workgroup
    assert ops.plan_info(8, 6144, 2560, 128).variant == 12083       # Qwen3-4B qkv keeps two
    assert ops.plan_info(2048, 1536, 4096, 128).variant == 9064     # 64-row block on the 32x32 kernel
    assert ops.plan_info(2048, 4096, 1024, 128).variant == 2128     # short K: no k-wave split


def test_fused_activation_routing():
    """The fused gate/up GEMM keeps the GEMV kernel to 8 rows on short K and the
    skinny kernel beyond, while the plain GEMM takes the GEMV kernel to 16 rows."""
    assert ops.gemm_kernel(12, 2080, 2560, 128) == "gemv_kernel"
    assert ops.gemm_kernel(12, 2080, 2560, 128, activation="silu") == "skinny_kernel"
    assert ops.gemm_kernel(8, 19456, 2560, 128, activation="silu") == "gemv_kernel"
    assert ops.gemm_kernel(300, 1056, 1024, 128, activation="gelu") == "tiled_kernel"
    with pytest.raises(ValueError, match="N % 32"):
        ops.gemm_kernel(1, 2064, 1024, 128, activation="silu")


@pytest.mark.parametrize("K,N,G,dtype,msg", [
    (100, 64, 128, 0, "group size"),
    (256, 64, 48, 0, "group size"),
    (256, 60, 128, 0, "output size"),
    (0, 64, 128, 0, "positive"),
    (256, 64, 128, 7, "dtype"),
    (96, 64, 64, 0, "input size"),
])
def test_invalid_shapes_raise_value_error(K, N, G, dtype, msg):
    lib = _lib.load()
    fake = 0x10000  # never dereferenced: validation fails first
    st = lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, 4, N, K, G, dtype, None, 0, None, 0, None)
    assert st == _lib.AWQ_STATUS_INVALID_ARGUMENT
    with pytest.raises(ValueError, match=msg):
        _lib.check(st, "awq_w4a16_gemm")


def test_null_and_misaligned_pointers_rejected():
    lib = _lib.load()
    fake = 0x10000
    assert lib.awq_w4a16_gemm(None, fake, fake, fake, None, fake, 4, 64, 256, 128, 0, None, 0, None, 0, None) == -1
    assert "null" in _lib.last_error()
    assert lib.awq_w4a16_gemm(fake + 2, fake, fake, fake, None, fake, 4, 64, 256, 128, 0, None, 0, None, 0, None) == -1
    assert "aligned" in _lib.last_error()
    assert lib.awq_repack_cdna4(fake, fake, fake, 0, 256, 64, 128, fake + 4, fake, fake, None) == -1
    assert lib.awq_dequant(None, fake, fake, 0, 256, 64, 128, fake, None) == -1


def test_missing_workspace_is_reported_before_launch():
    lib = _lib.load()
    fake = 0x10000
    K, N, M = 28672, 512, 1  # 32 column tiles, 224 k-tiles: the plan splits K across workgroups
    need = lib.awq_workspace_bytes(M, N, K, 128)
    assert need > 0
    st = lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, M, N, K, 128, 0, None, 0, None, 0, None)
    assert st == _lib.AWQ_STATUS_WORKSPACE
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.check(st, "awq_w4a16_gemm")
    st = lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, M, N, K, 128, 0, fake, need, None, 0, None)
    assert st == _lib.AWQ_STATUS_WORKSPACE and "counters" in _lib.last_error()


def test_short_counters_are_reported_before_launch():
    lib = _lib.load()
    fake = 0x10000
    K, N, M = 28672, 512, 1  # split K on the GEMV kernel: arrival counters needed
    need = lib.awq_workspace_bytes(M, N, K, 128)
    cb = lib.awq_counter_bytes(N)
    st = lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, M, N, K, 128, 0, fake, need, fake, cb - 4, None)
    assert st == _lib.AWQ_STATUS_WORKSPACE and "counters of" in _lib.last_error()
    st = lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, M, N, K, 128, 0, fake, need, fake + 64, cb, None)
    assert st == _lib.AWQ_STATUS_WORKSPACE and "aligned" in _lib.last_error()


def test_abi_version_and_counter_layout():
    lib = _lib.load()
    assert lib.awq_abi_version() == _lib.AWQ_ABI_VERSION == 4
    assert lib.awq_version().decode().endswith("0.4")
    # the constants the binding mirrors agree with the library's sizes
    assert lib.awq_counter_bytes(16) == _lib.AWQ_COUNTER_TILE_BYTES + 4
    assert lib.awq_counter_bytes(_lib.AWQ_NOALLOC_MAX_N) == _lib.AWQ_COUNTER_TILE_BYTES + _lib.AWQ_NOALLOC_MAX_N // 4
    # a library of another ABI revision is refused before any symbol is bound
    import ctypes
    saved = _lib.AWQ_ABI_VERSION
    try:
        _lib.AWQ_ABI_VERSION = 3
        with pytest.raises(RuntimeError, match="ABI"):
            _lib._lib, keep = None, _lib._lib
            try:
                _lib.load()
            finally:
                _lib._lib = keep
    finally:
        _lib.AWQ_ABI_VERSION = saved
    assert isinstance(_lib.load(), ctypes.CDLL)


def test_tiled_split_k_accepts_missing_counters():
    # the tiled kernels take the counters when given (sum in the kernel) and
    # fall back to a second kernel without them; misaligned ones are refused
    lib = _lib.load()
    fake = 0x10000
    M, N, K = 32, 6144, 2560
    from sglite_amd import ops
    info = ops.plan_info(M, N, K, 128)
    assert info.kernel == "tiled_kernel" and info.k_slices > 1 and info.function == "mfma32_kernel"
    assert not info.fixup  # opt-in
    with ops.plan_overrides(tiled_fixup=1):
        assert ops.plan_info(M, N, K, 128).fixup
    need = lib.awq_workspace_bytes(M, N, K, 128)
    st = lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, M, N, K, 128, 0, fake, need, fake + 64, 1 << 20, None)
    assert st == _lib.AWQ_STATUS_WORKSPACE and "128-byte aligned" in _lib.last_error()


def test_plan_overrides_and_plan_info():
    lib = _lib.load()
    assert lib.awq_set_plan_override(99, 1) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert "knob" in _lib.last_error()
    assert ops.gemm_kernel(1, 6144, 2560, 128) == "gemv_kernel"
    with ops.plan_overrides(gemv_max_m=0):
        assert ops.gemm_kernel(1, 6144, 2560, 128) == "skinny_kernel"
        with pytest.raises(KeyError):
            ops.set_plan_override("no_such_knob", 1)
    assert ops.gemm_kernel(1, 6144, 2560, 128) == "gemv_kernel"
    with ops.plan_overrides(tiled_min_m=1, tiled_bm=64, tiled_ks=2):
        info = ops.plan_info(8, 6144, 2560, 128)
        assert info.kernel == "tiled_kernel" and info.variant == 64 and info.k_slices == 2
        assert info.workspace_bytes == 2 * 8 * 6144 * 4 and info.threads == 256
        assert info.workgroups == (6144 // 256) * 1 * 2
    with ops.plan_overrides(kslice_variant=141):
        # o_proj 4096 x 2560 at M = 32: 64-column groups, 4 k-tiles per slice
        info = ops.plan_info(32, 2560, 4096, 128)
        assert info.kernel == "kslice_kernel" and info.variant == 141 and info.k_slices == 8
        assert info.workgroups == 40 * 8 and info.threads == 256
        assert info.workspace_bytes == 8 * 32 * 2560 * 4
        # fused gate/up: 32 gate columns per wave
        info = ops.plan_info(16, 2 * 1040, 2048, 128, "silu")
        assert info.kernel == "kslice_kernel" and info.workgroups == 33 * 4  # 65 gate tiles, two per wave
        assert ops.plan_info(33, 2560, 4096, 128).kernel != "kslice_kernel"  # one 32-row block only
        assert ops.plan_info(32, 2560, 4096 * 5, 128).kernel != "kslice_kernel"  # > 16 slices
    with ops.plan_overrides(kslice_variant=999):  # not instantiated: ignored
        assert ops.plan_info(32, 2560, 4096, 128).kernel != "kslice_kernel"
    for M, N, K in [(1, 6144, 2560), (8, 2560, 4096), (32, 19456, 2560), (2048, 28672, 4096)]:
        info = ops.plan_info(M, N, K, 128)
        assert info.kernel == ops.gemm_kernel(M, N, K, 128)
        assert info.workspace_bytes == ops.workspace_bytes(M, N, K, 128)
        assert info.workgroups >= 1 and info.threads % 64 == 0 and 64 <= info.threads <= 1024
    assert ops.device_cu_count() >= 1


@pytest.mark.parametrize("M,N,K,variant,ks,wgs", [
    (8, 4096, 14336, 4032, 16, 256),     # Llama-3-8B down: 32-row 32x32 form, 16 k-slices
    (32, 4096, 14336, 4032, 16, 256),
    (128, 28672, 4096, 9064, 1, 224),    # Llama-3-8B gate_up: 64-row 32x32 k-wave split (one round)
    (64, 57344, 8192, 9064, 1, 224),     # 70B-sized gate_up
    (96, 19456, 2560, 4032, 1, 228),     # wide, 65-128 rows, K <= 4096: K unsplit in 32-row blocks
    (96, 28672, 4096, 9064, 1, 224),     # ... or in the 64-row k-wave split when 32-row tiles overflow
    (160, 4096, 14336, 9064, 4, 192),    # 129-192 rows, split K: the 64-row k-wave split, one round
    (192, 8192, 8192, 9064, 2, 192),
    (160, 28672, 4096, 8064, 1, 168),    # 8-wave 64-row form: 168 of 256 CUs
    (256, 19456, 2560, 9128, 1, 152),    # Qwen3-4B gate_up: 193-256 rows pad to 256 in every form
    (192, 19456, 2560, 9064, 1, 228),
    (224, 28672, 4096, 9128, 1, 224),    # one round of 128 x 256 tiles: the k-wave split
    (192, 28672, 4096, 8064, 1, 168),
    (2048, 28672, 4096, 2128, 1, 1792),  # 3.5 rounds: two workgroups per CU
    (2048, 6144, 4096, 8128, 1, 192),    # at most one round of 512-column tiles
    (2048, 4096, 4096, 9128, 1, 256),    # one round of 256-column tiles: 8 waves splitting the k-steps
    (8192, 28672, 4096, 8128, 1, 3584),  # whole rounds
    (1024, 28672, 4096, 8128, 1, 448),   # last round of 512-column tiles three quarters full
    (2048, 19456, 2560, 2128, 1, 1216),  # last round a quarter full: two workgroups per CU
    (1024, 6144, 4096, 9128, 1, 192),    # over half a round, at most one: 32x32 k-wave split
    (2048, 2560, 4096, 9128, 1, 160),
    (2048, 2560, 9728, 9128, 1, 160),    # the k-wave split also replaces a 3-way K split
    (1024, 2560, 4096, 128, 3, 240),     # half a round or less (80 tiles): split K stays
    (512, 19456, 2560, 8128, 1, 152),    # 1.2 rounds of 256-column tiles, 0.6 of 512-column ones
    (64, 2560, 9728, 4032, 11, 220),     # Qwen3-4B down: 32-row blocks up to 112 rows at K <= 12288
    (112, 2560, 9728, 4032, 6, 240),
    (128, 2560, 9728, 64, 11, 220),
    (64, 4096, 14336, 64, 16, 256),      # Llama-3-8B down (K = 14336) keeps 64-row blocks
])
def test_tiled_plan_forms(M, N, K, variant, ks, wgs):
    """The planner's row-block form per batch size on a whole MI355X (256 CUs, the
    host-side planning default)."""
    if ops.device_cu_count() != 256:
        pytest.skip("the forms are pinned for a whole MI355X (256 CUs)")
    info = ops.plan_info(M, N, K, 128)
    assert (info.kernel, info.variant, info.k_slices, info.workgroups) == ("tiled_kernel", variant, ks, wgs)


def test_tiled_plan_forms_with_fused_activation():
    """The fused gate/up GEMM takes the same row-block forms as the plain one
    at prefill sizes (the gated pairs stay within a workgroup in each form)."""
    if ops.device_cu_count() != 256:
        pytest.skip("the forms are pinned for a whole MI355X (256 CUs)")
    for M, N, K, variant in [(1024, 4160, 2560, 9128), (512, 19456, 1024, 8128), (2048, 19456, 2560, 2128)]:
        assert ops.plan_info(M, N, K, 128, "silu").variant == variant, (M, N, K)
        assert ops.plan_info(M, N, K, 128).variant == variant, (M, N, K)


def test_stream_probe_validates_before_launch():
    lib = _lib.load()
    fake = 0x10000
    assert lib.awq_stream_probe(fake, 100, 4, 256, fake, 16, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert lib.awq_stream_probe(fake, 4096, 4, 96, fake, 16, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert lib.awq_stream_probe(fake, 4096, 0, 256, fake, 16, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert lib.awq_stream_probe(fake, 4096, 8, 256, fake, 16, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert "sink" in _lib.last_error()
    assert lib.awq_stream_probe(None, 4096, 4, 256, fake, 16, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT


def test_noalloc_entry_rejects_before_launch():
    lib = _lib.load()
    fake = 0x10000
    # 9728 x 2560 at M = 4096 splits K into 80 MiB of partials: beyond the static scratch
    assert lib.awq_workspace_bytes(4096, 2560, 9728, 128) > _lib.AWQ_NOALLOC_WORKSPACE_BYTES
    st = lib.awq_w4a16_gemm_noalloc(fake, fake, fake, fake, None, fake, 4096, 2560, 9728, 128, 0, None)
    assert st == _lib.AWQ_STATUS_UNSUPPORTED and "scratch" in _lib.last_error()
    assert lib.awq_w4a16_gemm_noalloc(None, fake, fake, fake, None, fake, 4, 64, 256, 128, 0, None) == -1
    assert lib.awq_w4a16_gemm_noalloc(fake, fake, fake, fake, None, fake, 4, 60, 256, 128, 0, None) == -1
    assert lib.awq_w4a16_gemm_noalloc(None, None, None, None, None, None, 0, 64, 256, 128, 0, None) == 0


def test_fused_activation_entry_validates_before_launch():
    lib = _lib.load()
    fake = 0x10000  # never dereferenced: validation fails first
    args = (fake, fake, fake, fake, None, fake)
    assert lib.awq_w4a16_gemm_act(*args, 4, 64, 256, 128, 0, 3, None, 0, None, 0, None) == -1
    assert "activation" in _lib.last_error()
    assert lib.awq_w4a16_gemm_act(*args, 4, 48, 256, 128, 0, _lib.AWQ_ACT_SILU, None, 0, None, 0, None) == -1
    assert "multiple of 32" in _lib.last_error()
    assert lib.awq_w4a16_gemm_act(None, fake, fake, fake, None, fake, 4, 64, 256, 128, 0, _lib.AWQ_ACT_GELU, None, 0,
                                  None, 0, None) == -1
    assert "null" in _lib.last_error()
    assert lib.awq_w4a16_gemm_act(*args, 0, 64, 256, 128, 0, _lib.AWQ_ACT_SILU, None, 0, None, 0, None) == 0
    assert lib.awq_workspace_bytes_act(4, 48, 256, 128) == -1
    # a gate/up projection narrow enough to split K needs the workspace and the counters
    M, N, K = 1, 512, 8192
    need = lib.awq_workspace_bytes_act(M, N, K, 128)
    assert need > 0
    st = lib.awq_w4a16_gemm_act(*args, M, N, K, 128, 0, _lib.AWQ_ACT_SILU, None, 0, None, 0, None)
    assert st == _lib.AWQ_STATUS_WORKSPACE


def test_gated_mlp_entry_validates_before_launch():
    lib = _lib.load()
    fake = 0x10000  # never dereferenced: validation fails first
    # workspace: the intermediate [M, I] (256-byte rounded), then 1..256 fp32 [M, H] partials
    for M, H, I in [(1, 2560, 9728), (8, 2560, 9728), (16, 4096, 14336), (3, 512, 768)]:
        b = lib.awq_gated_mlp_workspace_bytes(M, H, I, 128, 0)
        hb = (M * I * 2 + 255) // 256 * 256
        assert b > hb and (b - hb) % (M * H * 4) == 0 and 1 <= (b - hb) // (M * H * 4) <= 256, (M, H, I, b)
    # outside the built forms: more rows, a wider hidden size, another group size
    for M, H, I, G in [(17, 2560, 9728, 128), (1, 8192, 3584, 128), (1, 2560, 9728, 64)]:
        assert lib.awq_gated_mlp_workspace_bytes(M, H, I, G, 0) == _lib.AWQ_STATUS_UNSUPPORTED
    assert lib.awq_gated_mlp_workspace_bytes(1, 2560, 9727, 128, 0) == -1  # 2I columns not packable
    w = (fake,) * 7
    M, H, I = 4, 2560, 9728
    need = lib.awq_gated_mlp_workspace_bytes(M, H, I, 128, 0)
    cb = _lib.AWQ_MLP_COUNTER_BYTES

    def call(*, x=fake, act=_lib.AWQ_ACT_SILU, m=M, ws=fake, wsb=need, cnt=fake, cntb=cb, h=H, g=128):
        return lib.awq_gated_mlp(x, *w, m, h, I, g, 0, act, -1, ws, wsb, cnt, cntb, None)

    assert call(act=3) == -1 and "activation" in _lib.last_error()
    assert call(x=None) == -1 and "null" in _lib.last_error()
    assert call(x=fake + 8) == -1 and "aligned" in _lib.last_error()
    assert call(m=17) == _lib.AWQ_STATUS_UNSUPPORTED and "built forms" in _lib.last_error()
    assert call(g=64) == _lib.AWQ_STATUS_UNSUPPORTED
    assert call(ws=None) == _lib.AWQ_STATUS_WORKSPACE and "workspace" in _lib.last_error()
    assert call(wsb=need - 1) == _lib.AWQ_STATUS_WORKSPACE
    assert call(ws=fake + 16) == _lib.AWQ_STATUS_WORKSPACE and "256-byte" in _lib.last_error()
    assert call(cnt=None) == _lib.AWQ_STATUS_WORKSPACE and "counters" in _lib.last_error()
    assert call(cntb=cb - 4) == _lib.AWQ_STATUS_WORKSPACE
    assert call(cnt=fake + 64) == _lib.AWQ_STATUS_WORKSPACE and "128-byte" in _lib.last_error()
    assert call(m=0, x=None) == 0
    assert lib.awq_gated_mlp_take_errors(None, cb, None) == -1
    assert lib.awq_gated_mlp_take_errors(fake, cb - 4, None) == -1


def test_m_zero_is_a_noop():
    # an empty batch launches nothing, so no buffer is needed (shape checks still apply)
    lib = _lib.load()
    assert lib.awq_w4a16_gemm(None, None, None, None, None, None, 0, 64, 256, 128, 0, None, 0, None, 0, None) == 0
    assert lib.awq_w4a16_gemm(None, None, None, None, None, None, 0, 60, 256, 128, 0, None, 0, None, 0, None) == -1
    fake = 0x10000
    assert lib.awq_w4a16_gemm(fake, fake, fake, fake, None, fake, 0, 64, 256, 128, 0, None, 0, None, 0, None) == 0


# --------------------------------------------------------------------------
# configs and methods (quantization/__init__.py, base_config.py, awq.py, awq_marlin.py)
# --------------------------------------------------------------------------

def test_get_quantization_config_names():
    from sglite_amd.quantization.awq import AWQConfig
    from sglite_amd.quantization.awq_marlin import AWQMarlinConfig

    assert get_quantization_config("AWQ") is AWQConfig
    assert get_quantization_config("awq_marlin") is AWQMarlinConfig
    with pytest.raises(ValueError, match="Unknown quantization method"):
        get_quantization_config("gptq")


def test_lazy_exports():
    import sglite_amd.quantization as q

    assert q.AWQLinearMethod.__name__ == "AWQLinearMethod"
    assert q.AWQMarlinLinearMethod.__name__ == "AWQMarlinLinearMethod"
    with pytest.raises(AttributeError):
        q.NotAThing  # noqa: B018


def test_awq_config_from_config_and_errors():
    cls = get_quantization_config("awq")
    cfg = cls.from_config({"w_bit": 4, "q_group_size": 128, "zero_point": True})
    assert (cfg.weight_bits, cfg.group_size, cfg.zero_point, cfg.pack_factor) == (4, 128, True, 8)
    assert cfg.get_name() == "awq"
    assert cfg.get_supported_act_dtypes() == [torch.half]
    assert cfg.get_config_filenames() == ["quant_config.json", "quantize_config.json"]
    assert isinstance(cfg.get_linear_method(), LinearMethodBase)
    with pytest.raises(ValueError, match="only 4-bit"):
        cls(8, 128, True)
    with pytest.raises(ValueError, match="Cannot find any of"):
        cls.from_config({"bits": 4, "zero_point": True})
    assert QuantizationConfig.get_from_keys({"bits": 4, "w_bit": 8}, ["w_bit", "bits"]) == 8


def test_awq_marlin_config_rules():
    cls = get_quantization_config("awq_marlin")
    cfg = cls.from_config({"bits": 4, "group_size": 64, "zero_point": True})
    assert cfg.quant_type.size_bits == 4 and cfg.get_name() == "awq_marlin"
    assert cfg.get_supported_act_dtypes() == [torch.half, torch.bfloat16]
    with pytest.raises(ValueError, match="does not support this configuration"):
        cls(8, 128, True)  # uint8 with zero points is not served (marlin_utils.py:91-96)
    with pytest.raises(ValueError, match="does not support this configuration"):
        cls(4, 256, True)
    with pytest.raises(ValueError, match="only supports"):
        cls(3, 128, True)
    ok = {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True}
    assert cls.is_awq_marlin_compatible(ok)
    assert not cls.is_awq_marlin_compatible({**ok, "quant_method": "gptq"})
    assert not cls.is_awq_marlin_compatible({**ok, "bits": 8})
    assert not cls.is_awq_marlin_compatible({k: v for k, v in ok.items() if k != "zero_point"})
    assert not cls.is_awq_marlin_compatible({**ok, "group_size": 96})
    assert cls.is_awq_marlin_compatible({**ok, "group_size": -1})


def test_set_weight_attrs_refuses_overwrite():
    t = torch.empty(2)
    set_weight_attrs(t, {"input_dim": 0})
    set_weight_attrs(t, None)
    with pytest.raises(RuntimeError, match="Overwriting"):
        set_weight_attrs(t, {"input_dim": 1})


def test_awq_create_weights_shapes_and_errors():
    m = get_quantization_config("awq")(4, 128, True).get_linear_method()
    w = m.create_weights(2560, 6144)
    assert w["qweight"].shape == (2560, 768) and w["qweight"].dtype == torch.int32
    assert w["qzeros"].shape == (20, 768) and w["qzeros"].dtype == torch.int32
    assert w["scales"].shape == (20, 6144) and w["scales"].dtype == torch.get_default_dtype()
    assert (w["qweight"].packed_dim, w["qweight"].pack_factor, w["scales"].output_dim) == (1, 8, 1)
    assert set(w) == {"qweight", "qzeros", "scales"}
    with pytest.raises(ValueError, match="input size is not aligned"):
        m.create_weights(2500, 6144)
    with pytest.raises(ValueError, match="output size is not aligned"):
        m.create_weights(2560, 6140)


def test_awq_marlin_create_weights_metadata_and_errors():
    m = get_quantization_config("awq_marlin")(4, -1, True).get_linear_method()
    w = m.create_weights(256, 128)
    assert w["qzeros"].shape == (1, 16) and w["_num_groups"] == 1
    assert (w["_input_size"], w["_output_size"], w["_weights_processed"]) == (256, 128, False)
    m = get_quantization_config("awq_marlin")(4, 128, True).get_linear_method()
    with pytest.raises(ValueError, match="not divisible by 64"):
        m.create_weights(256, 96)
    with pytest.raises(ValueError, match="not divisible by 128"):
        m.create_weights(192, 128)


def test_scale_dtype_follows_default_dtype():
    m = get_quantization_config("awq")(4, 128, True).get_linear_method()
    old = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.bfloat16)
        assert m.create_weights(256, 64)["scales"].dtype == torch.bfloat16
    finally:
        torch.set_default_dtype(old)


# --------------------------------------------------------------------------
# linear plumbing (linear.py) with the dense method, on CPU
# --------------------------------------------------------------------------

def test_linear_plumbing_dense_roundtrip():
    from sglite_amd.linear import MergedColumnParallelLinear, QKVParallelLinear, RowParallelLinear

    lin = MergedColumnParallelLinear(32, [16, 16], has_bias=True)
    assert lin.state_dict_keys("mlp.gate_up_proj") == ["mlp.gate_up_proj.weight", "mlp.gate_up_proj.bias"]
    W = torch.randn(32, 32)
    b = torch.randn(32)
    sd = {"mlp.gate_up_proj.weight": W, "mlp.gate_up_proj.bias": b, "extra": torch.zeros(1)}
    with pytest.raises(RuntimeError, match="Unexpected keys"):
        lin.load_state_dict(dict(sd), prefix="mlp.gate_up_proj")
    lin = MergedColumnParallelLinear(32, [16, 16], has_bias=True)
    lin.load_state_dict({k: v for k, v in sd.items() if k != "extra"}, prefix="mlp.gate_up_proj")
    x = torch.randn(3, 32)
    torch.testing.assert_close(lin(x), x @ W.T + b)
    qkv = QKVParallelLinear(64, 16, 4, 2, has_bias=False, tp_size=2)
    assert qkv.local_output_size == (2 + 2 * 1) * 16
    row = RowParallelLinear(64, 32, has_bias=False, tp_size=2)
    assert row.local_input_size == 32
    with pytest.raises(AssertionError):
        RowParallelLinear(64, 32, has_bias=False).load_state_dict({"weight": torch.randn(32, 63)})


def test_linear_plumbing_processes_once_and_hides_runtime_tensors():
    from sglite_amd.linear import ReplicatedLinear

    calls = []

    class Probe(UnquantizedLinearMethod):
        def create_weights(self, i, o):
            w = super().create_weights(i, o)
            w["_meta"] = 7
            return w

        def process_weights_after_loading(self, weights):
            calls.append(dict(weights))
            return {"weight": weights["weight"] * 2, "workspace": torch.zeros(3), "_meta": weights["_meta"]}

    lin = ReplicatedLinear(8, 4, has_bias=False, linear_method=Probe())
    assert lin.state_dict_keys() == ["weight"]
    W = torch.randn(4, 8)
    lin.load_state_dict({"weight": W})
    assert len(calls) == 1 and calls[0]["_meta"] == 7
    assert lin.state_dict_keys() == ["weight"]  # workspace did not become an attribute
    assert "workspace" in lin._weights and lin._weights["_meta"] == 7
    torch.testing.assert_close(lin.weight, W * 2)


# --------------------------------------------------------------------------
# quant-config detection (models/config.py:28-89)
# --------------------------------------------------------------------------

def test_load_quantization_config_sources(tmp_path):
    from sglite_amd.model_config import load_quantization_config
    from sglite_amd.quantization.awq import AWQConfig
    from sglite_amd.quantization.awq_marlin import AWQMarlinConfig

    class HF:
        quantization_config = {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True}

    assert isinstance(load_quantization_config("nowhere", HF()), AWQMarlinConfig)
    assert isinstance(load_quantization_config("nowhere", HF(), force_awq_triton=True), AWQConfig)
    (tmp_path / "quant_config.json").write_text(json.dumps({"w_bit": 4, "q_group_size": 64, "zero_point": True}))
    cfg = load_quantization_config(str(tmp_path))
    assert isinstance(cfg, AWQConfig) and cfg.group_size == 64  # no quant_method -> not Marlin-compatible
    assert load_quantization_config(str(tmp_path / "missing")) is None

    class GPTQ:
        quantization_config = {"quant_method": "gptq", "bits": 4}

    assert load_quantization_config("nowhere", GPTQ()) is None


# --------------------------------------------------------------------------
# MoE entry points: validation happens before any GPU work
# --------------------------------------------------------------------------

def test_moe_capacity_queries():
    lib = _lib.load()
    assert lib.awq_moe_sorted_capacity(4096, 128, 16) == 4096 + 128 * 15
    assert lib.awq_moe_block_capacity(4096, 128, 16) == (4096 + 128 * 15 + 15) // 16
    assert lib.awq_moe_sorted_capacity(0, 1, 16) == 15
    assert lib.awq_moe_sorted_capacity(-1, 4, 16) == _lib.AWQ_STATUS_INVALID_ARGUMENT


def test_moe_topk_validation():
    lib = _lib.load()
    assert lib.awq_moe_topk_softmax(None, None, None, 4, 1000, 8, 1, None) == _lib.AWQ_STATUS_UNSUPPORTED
    assert lib.awq_moe_topk_softmax(None, None, None, 4, 8, 9, 1, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert "topk" in _lib.last_error()
    assert lib.awq_moe_topk_softmax(None, None, None, 4, 8, 2, 1, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert lib.awq_moe_topk_softmax(None, None, None, 0, 8, 2, 1, None) == _lib.AWQ_STATUS_OK


def test_moe_align_validation():
    lib = _lib.load()
    st = lib.awq_moe_align_block_size(None, 10, 8, 24, None, None, None, None, None)
    assert st == _lib.AWQ_STATUS_INVALID_ARGUMENT and "block_size" in _lib.last_error()
    assert lib.awq_moe_align_block_size(None, 10, 600, 16, None, None, None, None, None) == _lib.AWQ_STATUS_UNSUPPORTED
    assert lib.awq_moe_align_block_size(None, 10, 8, 16, None, None, None, None, None) == \
        _lib.AWQ_STATUS_INVALID_ARGUMENT


def _moe_gemm_status(**kw):
    a = dict(a=None, a_rows=4, w=None, s=None, z=None, E=8, N=256, K=256, G=128, dtype=0, sorted_ids=None,
             sorted_cap=64, offsets=None, tw=None, num_routed=8, top_k=2, act=1, mul=0, out=None, stream=None)
    a.update(kw)
    return _lib.load().awq_moe_w4a16_gemm(*a.values())


def test_moe_gemm_validation():
    assert _moe_gemm_status(N=48) == _lib.AWQ_STATUS_INVALID_ARGUMENT  # gate/up pairing needs I % 16 == 0
    assert "pairing" in _lib.last_error()
    assert _moe_gemm_status(act=7) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert _moe_gemm_status(a_rows=3) == _lib.AWQ_STATUS_INVALID_ARGUMENT  # 8 routed rows / top_k 2 need 4 rows
    assert "activation rows" in _lib.last_error()
    assert _moe_gemm_status(G=48) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert _moe_gemm_status(E=0) == _lib.AWQ_STATUS_UNSUPPORTED
    assert _moe_gemm_status(top_k=0) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert _moe_gemm_status() == _lib.AWQ_STATUS_INVALID_ARGUMENT  # null pointers
    assert _moe_gemm_status(num_routed=0) == _lib.AWQ_STATUS_OK       # nothing routed: no launch


def test_moe_sum_validation():
    lib = _lib.load()
    assert lib.awq_moe_sum_reduce(None, None, 4, 8, 12, 0, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert lib.awq_moe_sum_reduce(None, None, 4, 8, 16, 3, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT
    assert lib.awq_moe_sum_reduce(None, None, 0, 8, 16, 0, None) == _lib.AWQ_STATUS_OK
    assert lib.awq_moe_sum_reduce(None, None, 4, 8, 16, 0, None) == _lib.AWQ_STATUS_INVALID_ARGUMENT


def test_moe_backend_registry():
    from sglite_amd.moe import SUPPORTED_MOE_BACKENDS, AWQFusedMoe, create_moe_backend
    assert isinstance(create_moe_backend("awq_fused"), AWQFusedMoe)
    assert "awq_fused" in SUPPORTED_MOE_BACKENDS
    with pytest.raises(ValueError):
        create_moe_backend("nope")
