"""GPU parity of the k-slice decode kernel (kslice_kernel: M <= 32, K split
across workgroups and reduced by the last workgroup of each column group)
against the CPU oracle, through the C ABI.

Every instantiated shape (column waves x k-waves x k-tiles per wave) at every
groups-per-k-tile count and both dtypes, on a K with a partial last k-tile
(and, for G < 128, groups past K inside it) and an N with a half column tile
(N % 16 == 8) so that the last column group is partial; row counts 1..32;
with and without split K (K of one slice and of several); bias; the fused
gate/up activation with an odd gate-tile count; back-to-back calls that reuse
one counters buffer (the last workgroup must leave it zero).  Bar: max|err| <=
2e-2 * max|ref| of the fp32-accumulated oracle; results are deterministic
(two calls agree bit for bit whichever workgroup finishes last)."""

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2
VARIANTS = [411, 412, 413, 414, 221, 222, 223, 224, 141, 142]


def _ops():
    from sglite_amd import ops

    return ops


def _linear(K, N, G, seed, dtype=torch.float16):
    t = oracle.make_awq_linear(K, N, G, seed=seed, dtype=dtype)
    return t, {k: v.to(DEV) for k, v in t.items()}


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("G", [32, 64, 128, -1])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_every_kslice_shape(variant, G, dtype, plan):
    ops = _ops()
    K = {32: 1824, 64: 1856, 128: 1920, -1: 1120}[G]  # <= 15 k-tiles: one k-tile per slice stays within 16 slices
    N = 264
    t, d = _linear(K, N, G, seed=variant + (G if G > 0 else 5), dtype=dtype)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    plan.set("kslice_variant", variant)
    for M in (1, 7, 20, 32):
        info = ops.plan_info(M, N, K, G)
        assert info.kernel == "kslice_kernel" and info.variant == variant, info
        kt = (K + 127) // 128
        ktc = (variant // 10 % 10) * (variant % 10)
        assert info.k_slices == (kt + ktc - 1) // ktc
        x = oracle.make_activation(M, K, seed=M + variant, dtype=dtype)
        y = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
        ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
        ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
        assert ok, (variant, G, M, err, mx)
        y2 = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    assert ops.counters_settled(cnt)


@pytest.mark.parametrize("variant", [411, 222, 141])
@pytest.mark.parametrize("K", [256, 1024])
def test_kslice_single_slice_and_bias(variant, K, plan):
    """K within one slice (no handoff: the workgroup stores its output) and
    a bias added in the activation dtype."""
    ops = _ops()
    N, G = 200, 128
    t, d = _linear(K, N, G, seed=K + variant)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(variant)).to(torch.float16)
    plan.set("kslice_variant", variant)
    for M in (3, 16, 32):
        x = oracle.make_activation(M, K, seed=M + K)
        y = ops.gemm(x.to(DEV), r, K, N, G, bias=bias.to(DEV), counters=cnt)
        ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], bias, G)
        ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
        assert ok, (variant, K, M, err, mx)
    assert ops.counters_settled(cnt)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_kslice_fused_activation(variant, act, plan):
    """Gate tile and up tile in one wave (gate/up pairing), split K, an odd
    number of gate tiles (I = 1040: 65 tiles), bias on both halves."""
    ops = _ops()
    K, I, G = 2048, 1040, 128
    N = 2 * I
    t, d = _linear(K, N, G, seed=variant + 11)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(variant + 1)).to(torch.float16)
    plan.set("kslice_variant", variant)
    for M in (2, 32):
        assert ops.plan_info(M, N, K, G, act).kernel == "kslice_kernel"
        x = oracle.make_activation(M, K, seed=M + 3)
        y = ops.gemm(x.to(DEV), r, K, N, G, bias=bias.to(DEV), counters=cnt, activation=act)
        ref = oracle._ACT[act](oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], bias, G)).to(x.dtype)
        ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
        assert ok, (variant, act, M, err, mx)
    assert ops.counters_settled(cnt)


@pytest.mark.parametrize("variant", [411, 222, 141, 142])
@pytest.mark.parametrize("K,N", [(4096, 2560), (9728, 2560), (2560, 6144)])
def test_kslice_at_qwen3_4b_decode_sizes(variant, K, N, plan):
    """Full Qwen3-4B decode projections at M = 32 and 8 (up to 10 k-slices
    per column group) against the oracle."""
    ops = _ops()
    G = 128
    t, d = _linear(K, N, G, seed=K + N + variant)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    plan.set("kslice_variant", variant)
    for M in (8, 32):
        info = ops.plan_info(M, N, K, G)
        if info.kernel != "kslice_kernel":  # more than 16 slices: the planner declines
            assert (K // 128 + (variant // 10 % 10) * (variant % 10) - 1) // ((variant // 10 % 10) * (variant % 10)) > 16
            continue
        x = oracle.make_activation(M, K, seed=M)
        y = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
        ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
        ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
        assert ok, (variant, K, N, M, err, mx)
    assert ops.counters_settled(cnt)
