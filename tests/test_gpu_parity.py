"""GPU parity of the HIP engine against the CPU oracle, through the C ABI.

Bar: dequantisation (probe, repack round trip, and the GEMM kernels' own
in-register routine) is bit-exact; GEMM outputs are within
max|err| <= 2e-2 * max|ref| of the fp32-accumulated oracle.  Oracle sizes stay
small enough for the CPU; at the workloads' full sizes the reference is a
torch fp32 matmul on the GPU of the dequantised weight, whose bit-exactness
is itself checked in the same test.
"""

import os

import numpy as np
import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "awq_golden.npz")
TOL = 2e-2


def _ops():
    from sglite_amd import ops

    return ops


def _linear(K, N, G, seed, dtype=torch.float16):
    t = oracle.make_awq_linear(K, N, G, seed=seed, dtype=dtype)
    return t, {k: v.to(DEV) for k, v in t.items()}


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


SHAPES = [  # (K, N, G)
    (256, 64, 128),
    (96, 24, 32),      # K % 128 != 0, N % 16 != 0
    (384, 40, -1),     # channelwise
    (512, 136, 64),
    (2560, 96, 128),
]


@pytest.mark.parametrize("K,N,G", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dequant_probe_bit_exact(K, N, G, dtype):
    ops = _ops()
    t, d = _linear(K, N, G, seed=K + N, dtype=dtype)
    W = ops.dequant(d["qweight"], d["qzeros"], d["scales"])
    ref = oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], G)
    assert torch.equal(_bits(W), _bits(ref))


@pytest.mark.parametrize("K,N,G", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_repack_matches_layout_and_roundtrips(K, N, G, dtype):
    ops = _ops()
    t, d = _linear(K, N, G, seed=K * 3 + N, dtype=dtype)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    wb, sz = oracle.repack_cdna4(t["qweight"], t["qzeros"], t["scales"], G)
    np.testing.assert_array_equal(r.w.cpu().numpy().view(np.uint8), wb)
    got_sz = np.concatenate([r.s.cpu().view(torch.int16).numpy().view(np.uint8).reshape(-1),
                             r.z.cpu().numpy().view(np.uint8).reshape(-1)])
    np.testing.assert_array_equal(got_sz, sz)
    qw, qz, s = ops.unrepack(r, K, N, G)
    assert torch.equal(qw.cpu(), t["qweight"]) and torch.equal(qz.cpu(), t["qzeros"])
    assert torch.equal(_bits(s), _bits(t["scales"]))


@pytest.mark.parametrize("K,N,G", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_in_kernel_dequant_bit_exact(K, N, G, dtype):
    ops = _ops()
    t, d = _linear(K, N, G, seed=K + 7 * N, dtype=dtype)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    W = ops.dequant_repacked(r, K, N, G)
    ref = oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], G)
    assert torch.equal(_bits(W), _bits(ref))


def _gemm_case(K, N, G, M, seed, dtype=torch.float16, bias=False):
    ops = _ops()
    t, d = _linear(K, N, G, seed=seed, dtype=dtype)
    x = oracle.make_activation(M, K, seed=seed + 1, dtype=dtype)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(seed + 2)) * 0.5).to(dtype) if bias else None
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    y = ops.gemm(x.to(DEV), r, K, N, G, bias=None if b is None else b.to(DEV), counters=cnt)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], b, G)
    return y, ref, cnt


@pytest.mark.parametrize("M", [1, 2, 3, 8, 15, 16, 17, 31, 32, 33, 64, 65, 100, 128, 129, 256, 300])
def test_gemm_parity_m_sweep(M):
    y, ref, cnt = _gemm_case(1024, 320, 128, M, seed=100 + M)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)
    assert _ops().counters_settled(cnt)  # counters left settled for the next call


@pytest.mark.parametrize("K,N,G", [(96, 24, 32), (384, 40, -1), (512, 136, 64), (4224, 72, 128), (160, 8, 32)])
@pytest.mark.parametrize("M", [1, 5, 32, 70])
def test_gemm_parity_ragged_shapes(K, N, G, M):
    y, ref, _ = _gemm_case(K, N, G, M, seed=K + N + M)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)


@pytest.mark.parametrize("M", [1, 7, 32, 48, 200])
def test_gemm_bias(M):
    y, ref, _ = _gemm_case(768, 128, 128, M, seed=300 + M, bias=True)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)


@pytest.mark.parametrize("M", [1, 16, 32, 96])
def test_gemm_bf16(M):
    y, ref, _ = _gemm_case(1024, 256, 64, M, seed=400 + M, dtype=torch.bfloat16)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)


def test_gemm_golden_fixtures():
    ops = _ops()
    g = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in g.files if "/" in k})
    for name in names:
        K, N, G = (int(v) for v in g[f"{name}/shape"])
        dt = torch.bfloat16 if "bf16" in name else torch.float16
        half = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(dt)  # noqa: E731
        qw = torch.from_numpy(g[f"{name}/qweight"]).to(DEV)
        qz = torch.from_numpy(g[f"{name}/qzeros"]).to(DEV)
        s = half(g[f"{name}/scales"]).to(DEV)
        r = ops.repack(qw, qz, s)
        W = ops.dequant_repacked(r, K, N, G)
        np.testing.assert_array_equal(_bits(W).numpy().view(np.uint16), g[f"{name}/W"])
        bias = half(g[f"{name}/bias"]).to(DEV) if f"{name}/bias" in g.files else None
        cnt = ops.make_counters(N, DEV)
        for key in g.files:
            if key.startswith(f"{name}/x"):
                M = key.split("/x")[1]
                y = ops.gemm(half(g[key]).to(DEV), r, K, N, G, bias=bias, counters=cnt)
                ref = half(g[f"{name}/y{M}"])
                ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
                assert ok, (name, M, err, mx)


def test_split_k_is_deterministic():
    ops = _ops()
    K, N, G = 28672, 512, 128  # few column tiles, 224 k-tiles: the plan splits K across workgroups
    _, d = _linear(K, N, G, seed=500)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    assert ops.workspace_bytes(1, N, K, G) > 0
    for M in (1, 8, 32):
        x = oracle.make_activation(M, K, seed=501 + M).to(DEV)
        ys = [ops.gemm(x, r, K, N, G, counters=cnt) for _ in range(4)]
        for y in ys[1:]:
            assert torch.equal(y, ys[0])
        assert ops.counters_settled(cnt)


def _gpu_reference(x, W):
    return (x.float() @ W.float()).to(x.dtype)


def _sample_rows(M):
    if M <= 320:  # every row (the first and last 128 plus 64 between need M > 320)
        return torch.arange(M)
    g = torch.Generator().manual_seed(M)
    mid = torch.randperm(M - 256, generator=g)[:64] + 128
    return torch.cat([torch.arange(128), mid.sort().values, torch.arange(M - 128, M)])


def _check_full_size(y, W, x, t, K, N, G=128):
    """A full-size GEMM output against the CPU oracle on sampled rows x three
    256-column blocks (first, middle, last), the HIP dequantisation of the same
    blocks bit-exact against the oracle's, and every output against a GPU fp32
    matmul of that (pinned) dequantised weight."""
    rows = _sample_rows(x.shape[0])
    yc = y.cpu()
    for c0 in sorted({0, (N // 2) // 256 * 256, max(0, N - 256)}):
        c1 = min(N, c0 + 256)
        qw, qz, sc = t["qweight"][:, c0 // 8:c1 // 8], t["qzeros"][:, c0 // 8:c1 // 8], t["scales"][:, c0:c1]
        assert torch.equal(_bits(W[:, c0:c1]), _bits(oracle.dequantize(qw, qz, sc, G))), c0
        ref = oracle.awq_gemm(x[rows], qw, qz, sc, None, G)
        ok, err, mx = oracle.tolerance_ok(yc[rows][:, c0:c1], ref, TOL)
        assert ok, ("oracle block", c0, err, mx)
    ok, err, mx = oracle.tolerance_ok(y, _gpu_reference(x.to(DEV), W), TOL)
    assert ok, ("full", err, mx)


QWEN3_4B = [(2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560)]
LLAMA3_8B = [(4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)]


@pytest.mark.parametrize("K,N", QWEN3_4B)
@pytest.mark.parametrize("M", [1, 8, 32])
def test_qwen3_4b_layer_decode(K, N, M):
    ops = _ops()
    t, d = _linear(K, N, 128, seed=K + N)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    W = ops.dequant_repacked(r, K, N, 128)
    W_probe = ops.dequant(d["qweight"], d["qzeros"], d["scales"])
    assert torch.equal(W, W_probe)
    x = oracle.make_activation(M, K, seed=100 + M)
    y = ops.gemm(x.to(DEV), r, K, N, 128, counters=ops.make_counters(N, DEV))
    _check_full_size(y, W, x, t, K, N)


@pytest.mark.parametrize("K,N", QWEN3_4B)
@pytest.mark.parametrize("M", [64, 96, 512, 2048])
def test_qwen3_4b_prefill_sizes(K, N, M):
    """Qwen3-4B linears at mid-size batches (the down projection in 32-row
    blocks with split K) and at prefill chunk sizes whose grids are under one
    round or between one and one and a half rounds of 128 x 256 tiles (the
    planner routes them to the one-workgroup 32x32 and the 8-wave forms)."""
    ops = _ops()
    t, d = _linear(K, N, 128, seed=K + N)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    W = ops.dequant_repacked(r, K, N, 128)
    x = oracle.make_activation(M, K, seed=300 + M)
    y = ops.gemm(x.to(DEV), r, K, N, 128, counters=ops.make_counters(N, DEV))
    _check_full_size(y, W, x, t, K, N)


@pytest.mark.parametrize("K,N", LLAMA3_8B)
@pytest.mark.parametrize("M", [1, 8, 16, 64, 96, 128, 160, 256, 1024, 2048, 8192])
def test_llama3_8b_shapes(K, N, M):
    """Llama-3-8B's linears at every M the workload names, up to the reference's largest prefill chunk
    (max_extend_tokens = 8192, scheduler/config.py:20), and the decode batches
    64-160 that graph capture covers (cuda_graph.py:76)."""
    ops = _ops()
    t, d = _linear(K, N, 128, seed=K * 2 + N)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    W = ops.dequant_repacked(r, K, N, 128)
    x = oracle.make_activation(M, K, seed=200 + M)
    y = ops.gemm(x.to(DEV), r, K, N, 128, counters=ops.make_counters(N, DEV))
    assert y.shape == (M, N)
    _check_full_size(y, W, x, t, K, N)


def test_qwen3_4b_qkv_m16_against_cpu_oracle():
    """Qwen3-4B qkv_proj K=2560, N=6144, G=128, x [16, 2560], seed 0, checked on the CPU oracle."""
    y, ref, _ = _gemm_case(2560, 6144, 128, 16, seed=0)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)


@pytest.mark.parametrize("method_name", ["awq", "awq_marlin"])
def test_linear_method_lifecycle(method_name):
    from sglite_amd.linear import MergedColumnParallelLinear, QKVParallelLinear, RowParallelLinear
    from sglite_amd.quantization import get_quantization_config

    torch.set_default_dtype(torch.float16)
    try:
        cfg = get_quantization_config(method_name).from_config(
            {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True})
        method = cfg.get_linear_method()
        layers = {
            "qkv": QKVParallelLinear(512, 64, 8, 2, has_bias=True, linear_method=method),
            "o": RowParallelLinear(512, 512, has_bias=False, linear_method=method),
            "gate_up": MergedColumnParallelLinear(512, [256, 256], has_bias=False, linear_method=method),
        }
        for i, (name, lin) in enumerate(layers.items()):
            K, N = lin.local_input_size, lin.local_output_size
            t = oracle.make_awq_linear(K, N, 128, seed=600 + i)
            sd = {f"{name}.{k}": v.to(DEV) for k, v in t.items()}
            b = None
            if lin.bias is not None:
                b = torch.randn(N, generator=torch.Generator().manual_seed(700 + i)).to(torch.float16)
                sd[f"{name}.bias"] = b.to(DEV)
            lin.load_state_dict(sd, prefix=name)
            assert lin._weights["_weights_processed"] and "workspace" in lin._weights
            assert "workspace" not in lin.state_dict_keys(name)
            for M in (1, 9, 40):
                x = oracle.make_activation(M, K, seed=800 + M).reshape(1, M, K)
                y = lin(x.to(DEV))
                assert y.shape == (1, M, N) and y.dtype == torch.float16
                ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], b, 128)
                ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
                assert ok, (name, M, err, mx)
    finally:
        torch.set_default_dtype(torch.float32)


def test_apply_without_processing_repacks_on_the_fly():
    from sglite_amd.quantization import get_quantization_config

    method = get_quantization_config("awq")(4, 64, True).get_linear_method()
    K, N = 256, 64
    t = oracle.make_awq_linear(K, N, 64, seed=900)
    x = oracle.make_activation(3, K, seed=901)
    y = method.apply_weights({k: v.to(DEV) for k, v in t.items()}, x.to(DEV))
    ok, err, mx = oracle.tolerance_ok(y, oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, 64), TOL)
    assert ok, (err, mx)


@pytest.mark.parametrize("K,N", [(4096, 2560), (8192, 512)])
@pytest.mark.parametrize("M", [1, 8, 64])
def test_hip_graph_capture_replays(M, K, N):
    ops = _ops()
    G = 128
    _, d = _linear(K, N, G, seed=1000 + M)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    x = oracle.make_activation(M, K, seed=1001).to(DEV)
    eager = ops.gemm(x, r, K, N, G, counters=cnt).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            ops.gemm(x, r, K, N, G, counters=cnt)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = ops.gemm(x, r, K, N, G, counters=cnt)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i
        # eager work between replays, sharing the counters
        z = ops.gemm(x, r, K, N, G, counters=cnt)
        torch.cuda.synchronize()
        assert torch.equal(z, eager)
    assert ops.counters_settled(cnt)


@pytest.mark.parametrize("variant", [10104, 10108, 10116, 10202, 10401, 10404, 20202, 20401, 20204])
@pytest.mark.parametrize("G", [128, 64, 32])
def test_every_decode_variant(variant, G, plan):
    """Each decode-kernel instantiation, with and without cross-workgroup
    split-K, on a K that gives every wave full batches plus a masked tail."""
    ops = _ops()
    # K % G == 0 with a partial last 128-row tile where G allows; N % 16 == 8
    K = {32: 2336, 64: 2368, 128: 2432}[G]
    N = 200
    t, d = _linear(K, N, G, seed=variant * 7 + G)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    plan.set("gemv_max_m", "0")  # M = 1 too through this kernel
    for ks in (1, 3):
        plan.set("skinny_variant", str(variant))
        plan.set("skinny_ks", str(ks))
        for M in (1, 9, 17, 32):
            x = oracle.make_activation(M, K, seed=M + ks)
            y = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
            ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
            ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
            assert ok, (variant, G, ks, M, err, mx)
        assert ops.counters_settled(cnt)


@pytest.mark.parametrize("M", [1, 20])
def test_decode_bf16_variants(M, plan):
    ops = _ops()
    K, N, G = 2304, 136, 64
    t, d = _linear(K, N, G, seed=77 + M, dtype=torch.bfloat16)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    x = oracle.make_activation(M, K, seed=78, dtype=torch.bfloat16)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
    plan.set("gemv_max_m", "0")
    for variant in (10116, 20202, 10401):
        plan.set("skinny_variant", str(variant))
        y = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
        ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
        assert ok, (variant, err, mx)


@pytest.mark.parametrize("variant", [11048, 11083, 11084, 11086, 11088, 11165, 11166, 11168, 12083, 12084, 15037,
                                     21044, 21083, 21084, 22028, 22044, 23054, 24024, 24042, 14044])
@pytest.mark.parametrize("G", [128, -1])
def test_every_gemv_variant(variant, G, plan):
    """Each small-batch GEMV instantiation, with and without cross-workgroup
    split-K, for batch sizes over both m-tile counts (1..32 rows; 1 and 3 rows
    take the biased-operand arithmetic), on a K with a partial last 128-row
    tile and N % 16 == 8."""
    ops = _ops()
    K, N = 2432, 200
    t, d = _linear(K, N, G, seed=variant % 997 + (G if G > 0 else 7))
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    plan.set("gemv_max_m", "32")
    plan.set("gemv_variant", str(variant))
    for ks in (1, 3):
        plan.set("gemv_ks", str(ks))
        for M in (1, 3, 4, 16, 17, 32):
            x = oracle.make_activation(M, K, seed=M + ks)
            y = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
            ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
            ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
            assert ok, (variant, G, ks, M, err, mx)
        assert ops.counters_settled(cnt)


@pytest.mark.parametrize("K,N", [(4224, 136), (6144, 200), (8192, 72), (9728, 160), (11008, 88), (14336, 96)])
def test_gemv_unsplit_deep_k(K, N):
    """1-3 rows over K of 33-112 k-tiles (up to 6 rows at 76 k-tiles): the
    default plan covers the whole K in one workgroup of 8 or 16 waves of up to
    8 k-tiles each."""
    ops = _ops()
    G = 128
    t, d = _linear(K, N, G, seed=K % 1009 + N)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    for M in (1, 2, 3) if K != 9728 else (1, 3, 5, 6):
        assert ops.gemm_kernel(M, N, K, G) == "gemv_kernel"
        assert ops.workspace_bytes(M, N, K, G) == 0  # no split K
        x = oracle.make_activation(M, K, seed=M + 5)
        y = ops.gemm(x.to(DEV), r, K, N, G, counters=cnt)
        ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
        ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
        assert ok, (K, N, M, err, mx)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_bf16_and_bias(M):
    ops = _ops()
    K, N, G = 4096, 136, 128
    t, d = _linear(K, N, G, seed=91 + M, dtype=torch.bfloat16)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    x = oracle.make_activation(M, K, seed=92, dtype=torch.bfloat16)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(93)).to(torch.bfloat16)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], bias, G)
    y = ops.gemm(x.to(DEV), r, K, N, G, bias=bias.to(DEV), counters=cnt)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)


@pytest.mark.parametrize("bm", [32, 64, 128, 1064, 1128, 2064, 2128, 4032, 8064, 8128, 9064, 9128])
@pytest.mark.parametrize("G", [32, 64, 128, -1])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_every_tiled_variant(bm, G, dtype, plan):
    """Each prefill-kernel instantiation (16x16 MFMA row blocks 32/64/128,
    32x32 MFMA row blocks 64/128 (codes 1064/1128, 2064/2128 and 4032 with
    registers for more workgroups per CU, 8064/8128 with 8 waves and 512
    columns per workgroup, 9128 with 8 waves splitting the k-steps of 256
    columns; with G = 32 the planner keeps its own choice) x groups per 128-row
    k-tile x dtype): K with a partial last k-tile (and, for G < 128, groups
    past K inside it), N % 256 != 0 with N % 16 == 8, and row counts that
    leave the last row block partial; whole pipeline rounds plus a
    remainder, with and without split K.  The k-slice counts give slices of
    19 (unsplit), 7, 4 and 2 k-tiles with last slices of 5, 3 and 1 (for
    G = K: 9, 3, 2 and 1): every length modulo the 2- to 5-stage pipelines,
    and slices shorter than the prologue."""
    ops = _ops()
    K = {32: 2336, 64: 2368, 128: 2432, -1: 1120}[G]
    N = 264
    t, d = _linear(K, N, G, seed=bm + (G if G > 0 else 5), dtype=dtype)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    plan.set("tiled_bm", str(bm))
    plan.set("tiled_min_m", "1")  # small batches through this kernel too
    xs = {M: oracle.make_activation(M, K, seed=M + bm, dtype=dtype) for M in (20, 33, 130, 257)}
    refs = {M: oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G) for M, x in xs.items()}
    for ks in (1, 3, 5, 10):  # whole K per workgroup, then slices of about 7, 4 and 2 k-tiles
        plan.set("tiled_ks", str(ks))
        for M, x in xs.items():
            xd = x.to(DEV)
            y = ops.gemm(xd, r, K, N, G, counters=cnt)
            ok, err, mx = oracle.tolerance_ok(y, refs[M], TOL)
            assert ok, (bm, G, ks, M, err, mx)
            assert torch.equal(ops.gemm(xd, r, K, N, G, counters=cnt), y), (bm, G, ks, M)  # a second call
    assert ops.counters_settled(cnt)
    assert ops.gemm_kernel(20, N, K, G) == "tiled_kernel"


@pytest.mark.parametrize("code", [1064, 1128, 8128])
@pytest.mark.parametrize("K,N", [(4096, 6144), (14336, 4096)])
def test_mfma32_kernel_at_llama_prefill_sizes(code, K, N, plan):
    """The 32x32-MFMA prefill kernel at M = 2048 on Llama-3-8B shapes: against the
    CPU oracle on sampled blocks and the GPU fp32 reference over the pinned
    dequantised weight, and within fp32-reordering distance of tiled_kernel."""
    ops = _ops()
    t, d = _linear(K, N, 128, seed=K + N + code)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    W = ops.dequant_repacked(r, K, N, 128)
    x = oracle.make_activation(2048, K, seed=code)
    xd = x.to(DEV)
    cnt = ops.make_counters(N, DEV)
    plan.set("tiled_bm", code)
    y = ops.gemm(xd, r, K, N, 128, counters=cnt)
    _check_full_size(y, W, x, t, K, N)
    plan.set("tiled_bm", code % 1000)
    y_old = ops.gemm(xd, r, K, N, 128, counters=cnt)
    ok, err, mx = oracle.tolerance_ok(y, y_old, 1e-3)
    assert ok, (err, mx)


@pytest.mark.parametrize("M,K,N,G", [(64, 14336, 4096, 128), (200, 4096, 2560, 64), (40, 2368, 264, 32),
                                     (24, 4096, 28672, 128), (2048, 8192, 264, 128)])
def test_tiled_split_k_parity_and_determinism(M, K, N, G):
    """Prefill-kernel grids with fewer output tiles than CUs split K across
    workgroups; a second kernel sums the slices' fp32 partials in slice
    order, so repeated calls and graph replays are bit-identical, and the
    counters are left at zero."""
    ops = _ops()
    assert ops.gemm_kernel(M, N, K, G) == "tiled_kernel"
    assert ops.workspace_bytes(M, N, K, G) > 0
    t, d = _linear(K, N, G, seed=M + K)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    cnt = ops.make_counters(N, DEV)
    x = oracle.make_activation(M, K, seed=M)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
    xd = x.to(DEV)
    ys = [ops.gemm(xd, r, K, N, G, counters=cnt) for _ in range(10)]
    ok, err, mx = oracle.tolerance_ok(ys[0], ref, TOL)
    assert ok, (err, mx)
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    assert ops.counters_settled(cnt)
    out = torch.empty_like(ys[0])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.gemm(xd, r, K, N, G, counters=cnt, out=out)
    for _ in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ys[0])
    assert ops.counters_settled(cnt)
