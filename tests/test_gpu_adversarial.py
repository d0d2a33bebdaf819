"""Decode-kernel arithmetic under adversarial activations, against the CPU oracle.

The fp16 decode paths do not dequantise to rnd((q - z) * s) per weight: the
GEMV kernel at 1-3 rows and the skinny kernel feed the MFMAs the biased
nibbles B + q (B = 1024 fp16, 128 bf16) and subtract s * (B + z) * sum(x) in
fp32; the GEMV kernel at 4-16 rows feeds the exact integers q - z and scales
the fp32 sums.  (The tiled and k-slice kernels dequantise bit-exactly into
their MFMA operands.)  Their accuracy rests on fp32 headroom that zero-mean N(0, 1)
activations never test, so every path here runs activations with a large
mean, outlier channels (x300, +-1000) and fp16-extreme channels (+-5e4), in
fp16 and bf16, and is held to the GEMM contract (max|err| <= 2e-2 * max|ref|)
and to an element-wise bound: |err| <= rtol * |ref| + atol * max|ref| with
rtol four output ulps (2^-8 fp16, 2^-5 bf16) and atol 1e-3 (fp16) / 4e-3
(bf16) of max|ref|."""

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2
RTOL = {torch.float16: 2.0 ** -8, torch.bfloat16: 2.0 ** -5}
ATOL = {torch.float16: 1e-3, torch.bfloat16: 4e-3}


def _run(M, K, N, dtype, kind, plan=None, knobs=None, kernel=None, activation=None, seed=0, x_scale=1.0):
    from sglite_amd import ops

    G = 128
    t = oracle.make_awq_linear(K, N, G, seed=seed + K + N, dtype=dtype)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    for k, v in (knobs or {}).items():
        plan.set(k, v)
    if kernel is not None:
        assert ops.gemm_kernel(M, N, K, G, activation=activation) == kernel
    x = oracle.make_adversarial_activation(M, K, kind, seed=seed + M, dtype=dtype)
    if x_scale != 1.0:
        x = (x.float() * x_scale).to(dtype)
    y = ops.gemm(x.to(DEV), r, K, N, G, counters=ops.make_counters(N, DEV), activation=activation)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
    if activation is not None:
        ref = oracle._ACT[activation](ref).to(dtype)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, ("contract", M, K, N, dtype, kind, err, mx)
    eok, ratio = oracle.elementwise_ok(y, ref, RTOL[dtype], ATOL[dtype])
    assert eok, ("element-wise", M, K, N, dtype, kind, ratio, err, mx)


KINDS = oracle.ADVERSARIAL_KINDS
DTYPES = [torch.float16, torch.bfloat16]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M", [1, 2, 3])
def test_gemv_biased_operand(M, dtype, kind):
    """GEMV at 1-3 rows: the biased operand B + q (Qwen3-4B qkv-like shape)."""
    _run(M, 2560, 1024, dtype, kind, kernel="gemv_kernel")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M", [4, 8, 16])
def test_gemv_exact_integer_operand(M, dtype, kind, plan):
    """GEMV at 4-16 rows (forced: from 9 rows this 64-column-tile layer goes to the skinny
    kernel): fp16 takes the integers q - z, bf16 the dequantised weight."""
    _run(M, 2560, 1024, dtype, kind, plan=plan, knobs={"gemv_max_m": 16}, kernel="gemv_kernel")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M", [1, 9, 32])
def test_skinny_biased_operand(M, dtype, kind, plan):
    """The skinny decode kernel (biased operand for every M), forced for every row count, split K."""
    _run(M, 4096, 1024, dtype, kind, plan=plan, knobs={"gemv_max_m": 0, "tiled_min_m": 33}, kernel="skinny_kernel")


@pytest.mark.parametrize("kind", ["mean10", "outliers"])
@pytest.mark.parametrize("M", [1, 8, 24])
def test_fused_gate_up_paths(M, kind):
    """Fused gate/up activation (GEMV pairs at 1 and 8 rows, skinny pairs at 24).  The activations
    are scaled by 1/10 (the ratio of the mean and the outliers to the bulk is kept) so that
    silu(gate) * up stays inside fp16; fp16-extreme inputs overflow the gated product itself."""
    _run(M, 2560, 2 * 1040, torch.float16, kind, activation="silu", x_scale=0.1)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_tiled_dequant_path(dtype, kind):
    """The prefill kernel (bit-exact dequantisation into the MFMAs) at 48 rows, split K."""
    _run(48, 4096, 1024, dtype, kind, kernel="tiled_kernel")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("M", [8, 32])
def test_kslice_dequant_path(M, dtype, kind, plan):
    """The k-slice decode kernel (bit-exact dequantisation into 32x32 MFMAs, the split-K
    reduction in the kernel; chosen by override only) on the Qwen3-4B down and o_proj shapes."""
    K, N = (9728, 2560) if M == 8 else (4096, 2560)
    _run(M, K, N, dtype, kind, plan=plan, knobs={"kslice_variant": 142}, kernel="kslice_kernel")
