"""Split-K plans of the tiled kernels sum their k-slices inside the GEMM
kernel (every k-slice workgroup a portion of its tile, the last arrival any
portion nobody started).  The output must be bit-identical to the
second-kernel reduction (same slice order), whoever reduces which portion:
also when no workgroup waits for the others (polls = 0: the last arrival
sums the whole tile) and when the counters are shared by calls of other
shapes, and it must match the CPU oracle."""

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2


def _ops():
    from sglite_amd import ops

    return ops


# (M, K, N, G, activation): decode and mid-size batches that split K on the
# tiled kernels (the 32-row 32x32 form, the 64- and 128-row forms, the 8-wave
# k-wave split), group sizes 128 / 64 / 32, a fused gate/up activation.
CASES = [
    (32, 2560, 6144, 128, None),     # Qwen3-4B qkv, 32 rows
    (32, 2560, 19456, 128, None),    # Qwen3-4B gate_up
    (16, 4096, 28672, 128, None),    # Llama-3-8B gate_up, 16 rows
    (64, 14336, 4096, 128, None),    # Llama-3-8B down, 16 k-slices
    (160, 14336, 4096, 128, None),   # 129-192 rows: the 64-row k-wave split
    (200, 4096, 2560, 64, None),     # G = 64
    (40, 2368, 264, 32, None),       # G = 32, ragged N
    (32, 2560, 19456, 128, "silu"),  # fused gate/up activation
    (24, 4096, 28672, 128, "gelu"),
]


@pytest.fixture(autouse=True)
def _fixup_on():
    """The in-kernel reduction is opt-in (AWQ_PLAN_TILED_FIXUP)."""
    ops = _ops()
    ops.set_plan_override("tiled_fixup", 1)
    yield
    ops.clear_plan_overrides()


def _setup(M, K, N, G, act, dtype, seed):
    ops = _ops()
    t = oracle.make_awq_linear(K, N, G, seed=seed, dtype=dtype)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    x = oracle.make_activation(M, K, seed=seed + 1, dtype=dtype)
    return ops, t, r, x


@pytest.mark.parametrize("M,K,N,G,act", CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_in_kernel_split_k_matches_second_kernel_and_oracle(M, K, N, G, act, dtype):
    ops, t, r, x = _setup(M, K, N, G, act, dtype, seed=M + K + N)
    info = ops.plan_info(M, N, K, G, act)
    print(f"case M={M} K={K} N={N} G={G} act={act} {dtype}: {info}", flush=True)
    assert info.kernel == "tiled_kernel" and info.k_slices > 1 and info.fixup, info
    xd = x.to(DEV)
    cnt = ops.make_counters(N, DEV)
    y = ops.gemm(xd, r, K, N, G, counters=cnt, activation=act)
    torch.cuda.synchronize()
    assert ops.counters_settled(cnt)
    # the second-kernel reduction: without counters, and with the in-kernel one switched off
    y_two = ops.gemm(xd, r, K, N, G, activation=act)
    ops.set_plan_override("tiled_fixup", 0)
    y_off = ops.gemm(xd, r, K, N, G, counters=cnt, activation=act)
    ops.set_plan_override("tiled_fixup", 1)
    # no workgroup waits: the last arrival sums every portion, also right
    # after a launch in which the other k-slices summed their own portions
    ops.set_plan_override("fixup_polls", 0)
    y_last = ops.gemm(xd, r, K, N, G, counters=cnt, activation=act)
    ops.set_plan_override("fixup_polls", 512)
    y_again = ops.gemm(xd, r, K, N, G, counters=cnt, activation=act)
    x2 = oracle.make_activation(M, K, seed=M + 5, dtype=dtype).to(DEV)
    ops.set_plan_override("tiled_fixup", 0)
    y2_ref = ops.gemm(x2, r, K, N, G, activation=act)
    ops.set_plan_override("tiled_fixup", 1)
    ops.set_plan_override("fixup_polls", 0)
    y2_last = ops.gemm(x2, r, K, N, G, counters=cnt, activation=act)
    ops.set_plan_override("fixup_polls", 512)
    torch.cuda.synchronize()
    assert torch.equal(y2_last, y2_ref)  # new inputs: nothing of the previous launch is read back
    torch.cuda.synchronize()
    for other in (y_two, y_off, y_last, y_again):
        assert torch.equal(other, y)
    assert ops.counters_settled(cnt)
    # against the CPU oracle (the first and last rows, every column)
    rows = sorted(set(range(min(M, 8))) | set(range(max(0, M - 8), M)))
    xs = x[rows]
    if act is None:
        ref = oracle.awq_gemm(xs, t["qweight"], t["qzeros"], t["scales"], None, G)
    else:
        ref = oracle._ACT[act](oracle.awq_gemm(xs, t["qweight"], t["qzeros"], t["scales"], None, G)).to(dtype)
    ok, err, mx = oracle.tolerance_ok(y[rows], ref, TOL)
    assert ok, (err, mx)


def test_counters_shared_across_shapes_and_graph_replays():
    """One counters buffer (sized for the widest layer) serves every shape in
    turn, eager and captured, and each result stays bit-identical to the
    second-kernel reduction."""
    ops = _ops()
    shapes = [(32, 2560, 6144), (32, 2560, 19456), (8, 4096, 2560), (64, 14336, 4096), (32, 9728, 2560)]
    cnt = ops.make_counters(19456, DEV)
    runs = []
    for i, (M, K, N) in enumerate(shapes):
        _, t, r, x = _setup(M, K, N, 128, None, torch.float16, seed=10 * i + 3)
        xd = x.to(DEV)
        ops.set_plan_override("tiled_fixup", 0)  # the second-kernel reduction, own counters
        runs.append((M, K, N, r, xd, ops.gemm(xd, r, K, N, 128, counters=ops.make_counters(N, DEV))))
        ops.set_plan_override("tiled_fixup", 1)
    outs = [torch.empty_like(ref) for *_, ref in runs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for (M, K, N, r, xd, _), out in zip(runs, outs):
            ops.gemm(xd, r, K, N, 128, counters=cnt, out=out)
    for rep in range(3):
        for (M, K, N, r, xd, ref) in runs:  # eager calls between the replays
            assert torch.equal(ops.gemm(xd, r, K, N, 128, counters=cnt), ref), (rep, M, K, N)
        for out in outs:
            out.zero_()
        g.replay()
        torch.cuda.synchronize()
        for out, (M, K, N, *_, ref) in zip(outs, runs):
            assert torch.equal(out, ref), (rep, M, K, N)
    assert ops.counters_settled(cnt)


@pytest.mark.parametrize("case", ["fixup_last_arrival", "fixup_polls", "kslice"])
def test_split_k_handoff_reads_this_launchs_partials(case, plan):
    """Regression test of the split-K handoffs through plain stores (each arrival a release,
    the reading workgroup an acquire): consecutive launches alternate two inputs on one
    counters buffer and the shared split-K workspace, so a partial read before its store
    became visible would be the previous launch's, from the other input.  Every output must
    equal the second-kernel reduction of its own input bit for bit (the k-slice kernel: its
    own first result for that input, which the CPU oracle checks)."""
    ops = _ops()
    if case == "kslice":
        M, K, N, G, act = 32, 4096, 2560, 128, None
        plan.set("kslice_variant", 142)
    else:
        M, K, N, G, act = (200, 4096, 2560, 64, None) if case == "fixup_last_arrival" else (64, 14336, 4096, 128, None)
        plan.set("tiled_fixup", 1)
        if case == "fixup_last_arrival":
            plan.set("fixup_polls", 0)
    info = ops.plan_info(M, N, K, G, act)
    print(f"case {case} M={M} K={K} N={N} G={G}: {info}", flush=True)
    assert info.k_slices > 1
    assert info.kernel == ("kslice_kernel" if case == "kslice" else "tiled_kernel")
    if case != "kslice":
        assert info.fixup
    t = oracle.make_awq_linear(K, N, G, seed=K + N)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    xs = [oracle.make_activation(M, K, seed=s) for s in (11, 12)]
    cnt = ops.make_counters(N, DEV)
    if case == "kslice":
        refs = [ops.gemm(x.to(DEV), r, K, N, G, counters=cnt) for x in xs]
    else:
        plan.set("tiled_fixup", 0)
        refs = [ops.gemm(x.to(DEV), r, K, N, G) for x in xs]
        plan.set("tiled_fixup", 1)
    torch.cuda.synchronize()
    xd = [x.to(DEV) for x in xs]
    outs = [ops.gemm(xd[i % 2], r, K, N, G, counters=cnt) for i in range(40)]
    torch.cuda.synchronize()
    for i, y in enumerate(outs):
        assert torch.equal(y, refs[i % 2]), (case, i)
    assert ops.counters_settled(cnt)
    rows = sorted(set(range(8)) | set(range(M - 8, M)))
    for x, ref in zip(xs, refs):
        ok, err, mx = oracle.tolerance_ok(ref[rows], oracle.awq_gemm(x[rows], t["qweight"], t["qzeros"], t["scales"], None, G), TOL)
        assert ok, (case, err, mx)
