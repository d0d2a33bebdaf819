"""GPU parity of the GEMM with the gated activation fused (awq_w4a16_gemm_act):
out = act(gate) * up over the two column halves of a merged gate/up
projection, against the oracle's fp32-accumulated GEMM (each half rounded,
bias added in the activation dtype) followed by silu_and_mul / gelu_and_mul in
fp32, rounded once: max|err| <= 2e-2 * max|ref|.  Every kernel that can hold a
gate tile and its up tile together is driven: the small-batch GEMV (every
two-tile shape), the decode kernel (every two-tile shape), the prefill kernel
(every row block), with and without split K; fp16 and bf16, silu and gelu,
with and without bias, and an odd number of gate tiles (the last workgroup
holds half a pair set)."""

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2


def _ops():
    from sglite_amd import ops

    return ops


def _reference(x, t, G, bias, act):
    y = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], bias, G)
    return oracle._ACT[act](y).to(x.dtype)


def _check(M, K, I, G=128, dtype=torch.float16, act="silu", with_bias=False, env=None, plan=None,
           kernel=None, seed=0):
    ops = _ops()
    N = 2 * I
    t = oracle.make_awq_linear(K, N, G, seed=seed + M + K, dtype=dtype)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    bias = torch.randn(N, generator=torch.Generator().manual_seed(seed + 7)).to(dtype) if with_bias else None
    for k, v in (env or {}).items():
        plan.set(k, v)
    if kernel is not None:
        assert ops.gemm_kernel(M, N, K, G, activation=act) == kernel
    cnt = ops.make_counters(N, DEV)
    x = oracle.make_activation(M, K, seed=seed + 3, dtype=dtype)
    y = ops.gemm(x.to(DEV), r, K, N, G, bias=None if bias is None else bias.to(DEV), counters=cnt, activation=act)
    assert tuple(y.shape) == (M, I)
    ref = _reference(x, t, G, bias, act)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (M, K, I, G, dtype, act, env, err, mx)
    assert ops.counters_settled(cnt)
    return y


@pytest.mark.parametrize("M,K,I,kernel", [
    (1, 2048, 1040, "gemv_kernel"),     # one slice per workgroup
    (1, 8192, 1040, "gemv_kernel"),     # split K
    (4, 2560, 528, "gemv_kernel"),
    (12, 2048, 1040, "skinny_kernel"),  # split K
    (24, 2048, 1040, "skinny_kernel"),
    (16, 1024, 9728, "skinny_kernel"),  # wide: two-tile shapes by default
    (40, 2048, 1040, "tiled_kernel"),   # split K
    (300, 1024, 528, "tiled_kernel"),
    (1024, 2560, 2080, "tiled_kernel"),  # over half a round of 128 x 256 tiles: the 8-wave k-wave split
    (512, 1024, 9728, "tiled_kernel"),   # 1.2 rounds of them, 0.6 of 512-column tiles: the 8-wave kernel
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_silu_matches_oracle(M, K, I, kernel, dtype, plan):
    _check(M, K, I, dtype=dtype, kernel=kernel, plan=plan)


@pytest.mark.parametrize("M", [7, 8])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("with_bias", [False, True])
def test_qwen3_4b_gate_up_three_pair_plan(M, dtype, with_bias):
    """The plan that ships for the Qwen3-4B gate_up at 7-8 rows: three gate/up
    pairs per workgroup (shape 23054), K = 2560 unsplit, 608 pairs so the last
    workgroup holds two of three."""
    ops = _ops()
    assert ops.plan_info(M, 2 * 9728, 2560, 128, activation="silu").variant == 23054
    assert ops.workspace_bytes_act(M, 2 * 9728, 2560, 128) == 0
    _check(M, 2560, 9728, dtype=dtype, with_bias=with_bias, kernel="gemv_kernel")


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("M", [1, 12, 64])
def test_fused_activation_with_bias(act, M, plan):
    _check(M, 1024, 272, act=act, with_bias=True, plan=plan)


@pytest.mark.parametrize("variant", [21044, 21083, 21084, 22028, 22044, 23054, 24024, 24042])
@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("K", [4096, 2560])
def test_every_two_tile_gemv_shape(variant, M, K, plan):
    """Every two-tile GEMV shape, on a K that splits (4096) and one that most shapes take unsplit (2560)."""
    _check(M, K, 1040, env={"gemv_variant": variant, "gemv_max_m": 8}, kernel="gemv_kernel",
           plan=plan)


@pytest.mark.parametrize("variant", [20202, 20401, 20204])
@pytest.mark.parametrize("M", [3, 20])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_every_two_tile_decode_shape(variant, M, G, plan):
    _check(M, 4096, 1040, G=G, env={"skinny_variant": variant, "gemv_max_m": 0},
           kernel="skinny_kernel", plan=plan)


@pytest.mark.parametrize("bm", [32, 64, 128, 1064, 1128, 2064, 2128, 4032, 8064, 8128, 9064, 9128])
@pytest.mark.parametrize("ks", [1, 3])
@pytest.mark.parametrize("G", [32, 64, 128, -1])
def test_every_prefill_row_block(bm, ks, G, plan):
    K = 1312 if G == 32 else (1280 if G != -1 else 1152)
    _check(70, K, 1040, G=G, env={"tiled_bm": bm, "tiled_ks": ks, "tiled_min_m": 1},
           kernel="tiled_kernel", plan=plan)


def test_fused_equals_unfused_gemm_then_activation(plan):
    """Same kernel and plan with and without the activation: the fused output
    is the plain GEMM's rounded output run through silu in fp32 (prefill
    kernel, no split K), to within one fp16 ulp of the product (the device's
    exp and torch's may differ in the last fp32 bit)."""
    ops = _ops()
    M, K, I, G = 256, 2048, 2048, 128
    N = 2 * I
    t = oracle.make_awq_linear(K, N, G, seed=11)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    plan.set("tiled_ks", "1")  # one k-slice: both calls store straight from the accumulators
    assert ops.workspace_bytes(M, N, K, G) == 0 and ops.workspace_bytes_act(M, N, K, G) == 0
    x = oracle.make_activation(M, K, seed=12).to(DEV)
    y = ops.gemm(x, r, K, N, G).float()
    fused = ops.gemm(x, r, K, N, G, activation="silu").float()
    g, u = y[:, :I], y[:, I:]
    ref = (g / (1.0 + torch.exp(-g)) * u).to(torch.float16).float()
    ulp = torch.clamp(ref.abs(), min=2.0 ** -14) * 2.0 ** -10
    assert bool(((fused - ref).abs() <= ulp).all())
    assert (fused == ref).float().mean().item() > 0.99


@pytest.mark.parametrize("method_name", ["awq", "awq_marlin"])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_gated_mlp_block_against_oracle(method_name, act):
    """GatedMLP (blocks.py:27-57) on the AWQ plugin: gate_up with the activation
    fused, then down; oracle: GEMM, silu_and_mul / gelu_and_mul rounded, GEMM."""
    from sglite_amd.mlp import GatedMLP
    from sglite_amd.quantization import get_quantization_config

    torch.set_default_dtype(torch.float16)
    try:
        cfg = get_quantization_config(method_name).from_config(
            {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True})
        H, I = 512, 768
        mlp = GatedMLP(H, I, act, linear_method=cfg.get_linear_method())
        tgu = oracle.make_awq_linear(H, 2 * I, 128, seed=21)
        tdn = oracle.make_awq_linear(I, H, 128, seed=22)
        sd = {f"mlp.gate_up_proj.{k}": v.to(DEV) for k, v in tgu.items()}
        sd.update({f"mlp.down_proj.{k}": v.to(DEV) for k, v in tdn.items()})
        assert sorted(mlp.state_dict_keys("mlp")) == sorted(sd)
        mlp.load_state_dict(sd, prefix="mlp")
        for M in (1, 7, 40):
            x = oracle.make_activation(M, H, seed=30 + M)
            y = mlp(x.to(DEV))
            h = _reference(x, tgu, 128, None, act)
            ref = oracle.awq_gemm(h, tdn["qweight"], tdn["qzeros"], tdn["scales"], None, 128)
            ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
            assert ok, (method_name, act, M, err, mx)
    finally:
        torch.set_default_dtype(torch.float32)
