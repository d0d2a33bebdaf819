"""The gated MLP block in one launch (awq_gated_mlp): gate_up -> act(gate) * up
-> down (GatedMLP.forward, blocks.py:51-57) for decode batches, against the
CPU oracle's composition of the two AWQ GEMMs (oracle.gated_mlp_dequantized)
at the Qwen3-4B and Llama-3-8B MLP shapes, fp16 and bf16, within
max|err| <= 2e-2 * max|ref|; against the two-launch path; bit-identical from
call to call and under graph replay; and the bounded k-slice barriers made to
give up from the host (polls = 0): every kernel exits, the host raises, and
the next call is right."""

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2
G = 128
SHAPES = {"qwen3_4b": (2560, 9728), "llama3_8b": (4096, 14336), "small": (512, 768)}
_BLOCKS = {}


def _ops():
    from sglite_amd import ops

    return ops


def _block(name, dtype):
    """AWQ gate_up [H, 2I] and down [I, H] of one shape: repacked on the GPU, dequantized by the
    oracle on the CPU (cached: the Llama-3-8B pair takes seconds)."""
    key = (name, dtype)
    if key not in _BLOCKS:
        ops = _ops()
        H, I = SHAPES[name]
        tgu = oracle.make_awq_linear(H, 2 * I, G, seed=H + 1, dtype=dtype)
        tdn = oracle.make_awq_linear(I, H, G, seed=H + 2, dtype=dtype)
        gu = ops.repack(tgu["qweight"].to(DEV), tgu["qzeros"].to(DEV), tgu["scales"].to(DEV))
        dn = ops.repack(tdn["qweight"].to(DEV), tdn["qzeros"].to(DEV), tdn["scales"].to(DEV))
        wgu = oracle.dequantize(tgu["qweight"], tgu["qzeros"], tgu["scales"], G)
        wdn = oracle.dequantize(tdn["qweight"], tdn["qzeros"], tdn["scales"], G)
        _BLOCKS.clear()  # one shape's weights at a time
        _BLOCKS[key] = (H, I, gu, dn, wgu, wdn)
    return _BLOCKS[key]


def _two_launches(ops, x, gu, dn, H, I, act):
    h = ops.gemm(x, gu, H, 2 * I, G, counters=ops.make_counters(2 * I, DEV), activation=act)
    return ops.gemm(h, dn, I, H, G, counters=ops.make_counters(H, DEV))


CASES = ([("qwen3_4b", M, torch.float16, "silu") for M in (1, 2, 4, 8, 16)]
         + [("qwen3_4b", 3, torch.float16, "gelu"), ("qwen3_4b", 1, torch.bfloat16, "silu"),
            ("qwen3_4b", 8, torch.bfloat16, "silu")]
         + [("llama3_8b", M, torch.float16, "silu") for M in (1, 8, 16)]
         + [("llama3_8b", 4, torch.bfloat16, "silu"), ("small", 1, torch.float16, "silu"),
            ("small", 5, torch.float16, "gelu")])


@pytest.mark.parametrize("name,M,dtype,act", CASES)
def test_one_launch_block_against_oracle(name, M, dtype, act):
    ops = _ops()
    H, I, gu, dn, wgu, wdn = _block(name, dtype)
    plan = ops.gated_mlp_plan(M, H, I, G, dtype)
    print(f"case {name} M={M} {dtype} {act}: {plan}", flush=True)
    assert plan is not None and plan.workgroups <= ops.device_cu_count()
    x = oracle.make_activation(M, H, seed=M + H, dtype=dtype)
    xd = x.to(DEV)
    cnt = ops.make_mlp_counters(DEV)
    y = ops.gated_mlp(xd, gu, dn, H, I, G, cnt, act)
    y2 = ops.gated_mlp(xd, gu, dn, H, I, G, cnt, act)
    torch.cuda.synchronize()
    assert ops.mlp_take_errors(cnt) == 0
    assert ops.mlp_counters_settled(cnt)
    assert y.shape == (M, H) and y.dtype == dtype
    assert torch.equal(y, y2)  # a fixed summation order
    ref = oracle.gated_mlp_dequantized(x, wgu, wdn, act)
    ok, err, mx = oracle.tolerance_ok(y, ref, TOL)
    assert ok, (err, mx)
    ok, err, mx = oracle.tolerance_ok(y, _two_launches(ops, xd, gu, dn, H, I, act), TOL)
    assert ok, ("two launches", err, mx)


def test_give_up_is_reported_and_the_next_call_is_right():
    """polls = 0: at each k-slice's barrier every workgroup but the last to arrive gives up at once.
    The kernel still ends (the synchronize returns), the host raises, the counters stay valid and a
    following call gives the result of an undisturbed one."""
    from sglite_amd._lib import AWQKernelError

    ops = _ops()
    H, I, gu, dn, *_ = _block("qwen3_4b", torch.float16)
    M = 2
    plan = ops.gated_mlp_plan(M, H, I, G)
    x = oracle.make_activation(M, H, seed=77).to(DEV)
    cnt = ops.make_mlp_counters(DEV)
    ref = ops.gated_mlp(x, gu, dn, H, I, G, cnt)
    for _ in range(2):
        ops.gated_mlp(x, gu, dn, H, I, G, cnt, polls=0)
        torch.cuda.synchronize()
        assert ops.mlp_counters_settled(cnt)
        assert ops.mlp_take_errors(cnt) == plan.workgroups - plan.k_slices
    ops.gated_mlp(x, gu, dn, H, I, G, cnt, polls=0)
    with pytest.raises(AWQKernelError, match="gave up"):
        ops.mlp_check(cnt)
    ops.mlp_check(cnt)  # cleared
    y = ops.gated_mlp(x, gu, dn, H, I, G, cnt)
    torch.cuda.synchronize()
    assert ops.mlp_take_errors(cnt) == 0
    assert torch.equal(y, ref)


def test_graph_replays_match_eager_with_shared_counters():
    """Two blocks of different shapes share one counters buffer, captured in one graph; eager calls
    run between the replays and every replay equals the eager result bit for bit."""
    ops = _ops()
    runs = []
    for name, M in (("small", 3), ("qwen3_4b", 1)):
        H, I, gu, dn, *_ = _block(name, torch.float16)
        x = oracle.make_activation(M, H, seed=5 + M).to(DEV)
        runs.append((H, I, gu, dn, x))
    cnt = ops.make_mlp_counters(DEV)
    refs = [ops.gated_mlp(x, gu, dn, H, I, G, cnt) for H, I, gu, dn, x in runs]
    outs = [torch.empty_like(r) for r in refs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for (H, I, gu, dn, x), out in zip(runs, outs):
            ops.gated_mlp(x, gu, dn, H, I, G, cnt, out=out)
    for rep in range(3):
        for (H, I, gu, dn, x), ref in zip(runs, refs):
            assert torch.equal(ops.gated_mlp(x, gu, dn, H, I, G, cnt), ref), rep
        for out in outs:
            out.zero_()
        g.replay()
        torch.cuda.synchronize()
        for out, ref in zip(outs, refs):
            assert torch.equal(out, ref), rep
    assert ops.mlp_counters_settled(cnt) and ops.mlp_take_errors(cnt) == 0


def test_layer_takes_one_launch_for_decode_batches_only():
    """GatedMLP on the AWQ method with one_launch=True: a decode batch runs the one-launch block
    (bit-identical to ops.gated_mlp on the layer's weights), a prefill batch the two GEMMs."""
    from sglite_amd.mlp import GatedMLP
    from sglite_amd.quantization import get_quantization_config

    ops = _ops()
    H, I = 512, 768
    torch.set_default_dtype(torch.float16)
    try:
        cfg = get_quantization_config("awq_marlin").from_config(
            {"quant_method": "awq", "bits": 4, "group_size": 128, "zero_point": True})
        mlp = GatedMLP(H, I, "silu", linear_method=cfg.get_linear_method(), one_launch=True)
        tgu = oracle.make_awq_linear(H, 2 * I, G, seed=61)
        tdn = oracle.make_awq_linear(I, H, G, seed=62)
        sd = {f"gate_up_proj.{k}": v.to(DEV) for k, v in tgu.items()}
        sd.update({f"down_proj.{k}": v.to(DEV) for k, v in tdn.items()})
        mlp.load_state_dict(sd)
    finally:
        torch.set_default_dtype(torch.float32)
    gw, dw = mlp.gate_up_proj._weights, mlp.down_proj._weights
    gu = ops.Repacked(gw["qweight"], gw["scales"], gw["qzeros"])
    dn = ops.Repacked(dw["qweight"], dw["scales"], dw["qzeros"])
    x = oracle.make_activation(4, H, seed=63).to(DEV)
    y = mlp(x.view(2, 2, H))
    assert y.shape == (2, 2, H) and mlp._mlp_counters is not None
    assert torch.equal(y.view(4, H), ops.gated_mlp(x, gu, dn, H, I, G, ops.make_mlp_counters(DEV)))
    mlp.check_errors()
    xp = oracle.make_activation(40, H, seed=64).to(DEV)
    assert ops.gated_mlp_plan(40, H, I, G) is None
    assert torch.equal(mlp(xp), _two_launches(ops, xp, gu, dn, H, I, "silu"))
    with pytest.raises(RuntimeError, match="built forms"):
        ops.gated_mlp(xp, gu, dn, H, I, G, ops.make_mlp_counters(DEV))
