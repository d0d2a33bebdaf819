"""GPU parity of the grouped W4A16 MoE path against the CPU oracle, through the C ABI.

Bars:
  * routing ids and the alignment layout: exact (the oracle restates both);
    routing weights within 1e-6 relative (fp32 exp/sum order);
  * grouped GEMMs and the whole forward: max|err| <= 2e-2 * max|ref| against
    the fp32-accumulated oracle (per routed row or per token), at sizes the
    CPU oracle finishes in seconds; at the full Qwen3-30B-A3B expert shape
    (E=128, H=2048, I=768, top-8, T=512) the reference is the same algorithm
    in fp32 on the GPU over the bit-exact dequantised experts.
"""

import numpy as np
import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2


def _ops():
    from sglite_amd import ops

    return ops


def _experts(E, K, N, G, seed, dtype=torch.float16):
    ws = [oracle.make_awq_linear(K, N, G, seed=seed + e, dtype=dtype) for e in range(E)]
    return {key: torch.stack([w[key] for w in ws]) for key in ("qweight", "qzeros", "scales")}


def _to_dev(w):
    return {k: v.to(DEV) for k, v in w.items()}


def _routing(T, E, k, seed, drop=0.0):
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(seed))
    tw, ids = oracle.fused_topk(logits, k, renormalize=True)
    if drop:
        mask = torch.rand(ids.shape, generator=torch.Generator().manual_seed(seed + 1)) < drop
        ids = torch.where(mask, torch.full_like(ids, -1), ids)
    return logits, tw, ids


def _skewed_ids(T, E, k, seed):
    """Distinct experts per token, with expert 0 taking most tokens (several passes)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    hot = torch.rand(T, generator=g) < 0.8
    ids[hot, 0] = 0
    for t in torch.nonzero(hot).flatten().tolist():  # keep the row's experts distinct
        row = ids[t]
        dup = torch.nonzero(row[1:] == 0).flatten()
        for d in dup.tolist():
            row[d + 1] = E - 1 if row[0] != E - 1 else 1
    return ids


# --------------------------------------------------------------------------
# routing and alignment
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,E,k", [(37, 8, 2), (64, 60, 4), (512, 128, 8), (9, 200, 6), (5, 512, 8), (3, 64, 1)])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_softmax_matches_oracle(T, E, k, renorm):
    ops = _ops()
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(T * E + k))
    w, ids = ops.moe_topk_softmax(logits.to(DEV), k, renorm)
    rw, rids = oracle.fused_topk(logits, k, renormalize=renorm)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-6, atol=1e-7)


def test_topk_softmax_accepts_half_logits():
    ops = _ops()
    logits = torch.randn((16, 32), generator=torch.Generator().manual_seed(4)).half()
    w, ids = ops.moe_topk_softmax(logits.to(DEV), 4, True)
    rw, rids = oracle.fused_topk(logits.float(), 4, renormalize=True)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("n,E,bs", [(0, 4, 16), (7, 4, 16), (200, 8, 16), (4096, 128, 16), (4096, 128, 64),
                                    (333, 60, 32), (50, 512, 16), (65536, 128, 16)])
def test_align_matches_oracle(n, E, bs):
    ops = _ops()
    rng = np.random.default_rng(n + E + bs)
    ids = rng.integers(-1, E, size=n).astype(np.int32)
    a = ops.moe_align_block_size(torch.from_numpy(ids).to(DEV), bs, E)
    sorted_ids, expert_ids, npp, off = oracle.moe_align_block_size(ids, bs, E)
    total = int(npp[0])
    assert int(a.num_tokens_post_pad.item()) == total
    assert torch.equal(a.expert_offsets.cpu(), torch.from_numpy(off))
    assert torch.equal(a.sorted_ids[:total].cpu(), torch.from_numpy(sorted_ids[:total]))
    assert torch.equal(a.expert_ids.cpu(), torch.from_numpy(expert_ids))


# --------------------------------------------------------------------------
# grouped GEMM
# --------------------------------------------------------------------------

GEMM_CASES = [  # (T, E, k, K, N, G)
    (40, 8, 2, 256, 128, 128),
    (33, 16, 4, 256, 256, 64),
    (21, 6, 3, 352, 96, 32),    # K % 128 != 0
    (25, 5, 2, 384, 64, -1),    # one group
    (30, 4, 2, 128, 200, 128),  # N % 16 == 8 (plain only)
]


@pytest.mark.parametrize("T,E,k,K,N,G", GEMM_CASES)
@pytest.mark.parametrize("activation", [None, "silu", "gelu"])
@pytest.mark.parametrize("mul", [False, True])
def test_grouped_gemm_matches_oracle(T, E, k, K, N, G, activation, mul):
    if activation and N % 32:
        pytest.skip("gate/up pairing needs I % 16 == 0")
    ops = _ops()
    W = _experts(E, K, N, G, seed=K + N + E)
    _, tw, ids = _routing(T, E, k, seed=T + E, drop=0.05)
    x = oracle.make_activation(T, K, seed=T + K)
    ref = oracle.moe_grouped_gemm(x, W, tw, ids, k, G, activation, mul)
    d = _to_dev(W)
    ex = ops.repack_experts(d["qweight"], d["qzeros"], d["scales"])
    align = ops.moe_align_block_size(ids.to(DEV), 16, E)
    out = ops.moe_gemm(x.to(DEV), ex, K, N, G, align, tw.to(DEV), T * k, k, activation, mul)
    valid = (ids.reshape(-1) >= 0)
    ok, err, mx = oracle.tolerance_ok(out.cpu()[valid], ref[valid], TOL)
    assert ok, (err, mx)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_grouped_gemm_skewed_routing_multi_pass(dtype):
    """Expert 0 gets ~80% of 150 tokens (about 8 passes of 32 rows), others few or none."""
    ops = _ops()
    T, E, k, K, N, G = 150, 12, 3, 256, 192, 64
    W = _experts(E, K, N, G, seed=5, dtype=dtype)
    ids = _skewed_ids(T, E, k, seed=6)
    tw = torch.rand(ids.shape, generator=torch.Generator().manual_seed(7))
    x = oracle.make_activation(T, K, seed=8, dtype=dtype)
    d = _to_dev(W)
    ex = ops.repack_experts(d["qweight"], d["qzeros"], d["scales"])
    align = ops.moe_align_block_size(ids.to(DEV), 16, E)
    for act, mul in ((None, True), ("silu", False)):
        ref = oracle.moe_grouped_gemm(x, W, tw, ids, k, G, act, mul)
        out = ops.moe_gemm(x.to(DEV), ex, K, N, G, align, tw.to(DEV), T * k, k, act, mul)
        ok, err, mx = oracle.tolerance_ok(out.cpu(), ref, TOL)
        assert ok, (act, err, mx)


def _uneven_ids(T, E, k, seed):
    """Distinct experts per token: experts 0-3 take a fifth of the rows (about
    T / 5 each: at T = 512 more than the 64 rows of one pass), experts 4-99 the
    rest and experts 100 and above none."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.empty((T, k), dtype=torch.int32)
    for t in range(T):
        pick = torch.randperm(96, generator=g)[:k] + 4
        if torch.rand(1, generator=g).item() < 0.8:
            pick[0] = t % 4
        ids[t] = pick.to(torch.int32)
    return ids


@pytest.mark.parametrize("N,activation", [(2048, None), (1928, None), (2048, "silu"), (2016, "gelu")])
def test_grouped_gemm_balanced_placement_uneven_routing(N, activation):
    """128 experts at about two workgroups per CU (the heavy/light pairing of
    an XCD's slice groups), with experts of no rows, experts of more than one
    pass and a partial last slice; every routed row of the NaN-filled output
    is written and matches the oracle."""
    ops = _ops()
    T, E, k, K, G = 512, 128, 4, 256, 128
    W = _experts(E, K, N, G, seed=N + 3)
    ids = _uneven_ids(T, E, k, seed=N)
    tw = torch.rand(ids.shape, generator=torch.Generator().manual_seed(9))
    x = oracle.make_activation(T, K, seed=10)
    d = _to_dev(W)
    ex = ops.repack_experts(d["qweight"], d["qzeros"], d["scales"])
    align = ops.moe_align_block_size(ids.to(DEV), 16, E)
    counts = torch.bincount(ids.reshape(-1).long(), minlength=E)
    assert int(counts[:4].min()) > 64 and int(counts[100:].sum()) == 0
    ncols = N // 2 if activation else N
    out = torch.full((T * k, ncols), float("nan"), dtype=torch.float16, device=DEV)
    mul = activation is None
    ops.moe_gemm(x.to(DEV), ex, K, N, G, align, tw.to(DEV), T * k, k, activation, mul, out=out)
    ref = oracle.moe_grouped_gemm(x, W, tw, ids, k, G, activation, mul)
    got = out.cpu()
    assert not torch.isnan(got).any()
    ok, err, mx = oracle.tolerance_ok(got, ref, TOL)
    assert ok, (err, mx)


def test_grouped_gemm_block_size_32_alignment():
    """Buckets padded to 32 rows (a coarser alignment) give the same rows."""
    ops = _ops()
    T, E, k, K, N, G = 40, 8, 2, 256, 128, 128
    W = _experts(E, K, N, G, seed=11)
    _, tw, ids = _routing(T, E, k, seed=12)
    x = oracle.make_activation(T, K, seed=13)
    d = _to_dev(W)
    ex = ops.repack_experts(d["qweight"], d["qzeros"], d["scales"])
    outs = []
    for bs in (16, 32):
        align = ops.moe_align_block_size(ids.to(DEV), bs, E)
        outs.append(ops.moe_gemm(x.to(DEV), ex, K, N, G, align, tw.to(DEV), T * k, k, "silu", False))
    assert torch.equal(outs[0], outs[1])


# --------------------------------------------------------------------------
# whole forward
# --------------------------------------------------------------------------

def _moe_weights(E, H, I, G, seed, dtype=torch.float16):
    return _experts(E, H, 2 * I, G, seed, dtype), _experts(E, I, H, G, seed + 1000, dtype)


@pytest.mark.parametrize("T,E,k,H,I,G", [(33, 16, 4, 256, 128, 64), (5, 4, 2, 128, 128, 128), (64, 8, 2, 384, 96, 32),
                                         (1, 16, 4, 256, 128, 128)])
@pytest.mark.parametrize("activation", ["silu", "gelu"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_experts_matches_oracle(T, E, k, H, I, G, activation, dtype):
    from sglite_amd.moe import fused_experts_impl, process_awq_moe_weights
    W1, W2 = _moe_weights(E, H, I, G, seed=T + E, dtype=dtype)
    _, tw, ids = _routing(T, E, k, seed=T * 3)
    x = oracle.make_activation(T, H, seed=T + 1, dtype=dtype)
    ref = oracle.fused_moe_awq(x, W1, W2, tw, ids, G, activation=activation)
    d1, d2 = _to_dev(W1), _to_dev(W2)
    w1 = process_awq_moe_weights(d1["qweight"], d1["qzeros"], d1["scales"])
    w2 = process_awq_moe_weights(d2["qweight"], d2["qzeros"], d2["scales"])
    hs = x.to(DEV)
    out = fused_experts_impl(hs, w1, w2, tw.to(DEV), ids.to(DEV), activation)
    assert out.data_ptr() == hs.data_ptr()  # written in place, as the reference does
    ok, err, mx = oracle.tolerance_ok(out.cpu(), ref, TOL)
    assert ok, (err, mx)


def test_fused_experts_router_weight_on_input():
    from sglite_amd.moe import fused_experts_impl, process_awq_moe_weights
    T, E, k, H, I, G = 24, 6, 1, 256, 128, 128
    W1, W2 = _moe_weights(E, H, I, G, seed=77)
    _, _, ids = _routing(T, E, k, seed=78)
    tw = torch.rand(ids.shape, generator=torch.Generator().manual_seed(79)) * 0.5 + 0.25
    x = oracle.make_activation(T, H, seed=80)
    ref = oracle.fused_moe_awq(x, W1, W2, tw, ids, G, apply_router_weight_on_input=True)
    d1, d2 = _to_dev(W1), _to_dev(W2)
    w1 = process_awq_moe_weights(d1["qweight"], d1["qzeros"], d1["scales"])
    w2 = process_awq_moe_weights(d2["qweight"], d2["qzeros"], d2["scales"])
    out = fused_experts_impl(x.to(DEV), w1, w2, tw.to(DEV), ids.to(DEV), "silu", apply_router_weight_on_input=True)
    ok, err, mx = oracle.tolerance_ok(out.cpu(), ref, TOL)
    assert ok, (err, mx)


def test_backend_forward_with_gating_output():
    """AWQFusedMoe.forward: routing on the GPU, then the grouped experts."""
    from sglite_amd.moe import AWQFusedMoe, process_awq_moe_weights
    T, E, k, H, I, G = 48, 16, 4, 256, 128, 128
    W1, W2 = _moe_weights(E, H, I, G, seed=90)
    logits, tw, ids = _routing(T, E, k, seed=91)
    x = oracle.make_activation(T, H, seed=92)
    ref = oracle.fused_moe_awq(x, W1, W2, tw, ids, G)
    d1, d2 = _to_dev(W1), _to_dev(W2)
    w1 = process_awq_moe_weights(d1["qweight"], d1["qzeros"], d1["scales"])
    w2 = process_awq_moe_weights(d2["qweight"], d2["qzeros"], d2["scales"])
    out = AWQFusedMoe().forward(x.to(DEV), w1, w2, logits.to(DEV), k, True)
    ok, err, mx = oracle.tolerance_ok(out.cpu(), ref, TOL)
    assert ok, (err, mx)


# --------------------------------------------------------------------------
# full expert shape on the GPU
# --------------------------------------------------------------------------

def _pack_awq_dev(q):
    q = q.view(q.shape[0], q.shape[1], -1, 8)
    w = torch.zeros(q.shape[:3], dtype=torch.int32, device=q.device)
    for p, col in enumerate(oracle.AWQ_ORDER):
        w |= q[..., col] << (4 * p)
    return w


def _experts_dev(E, K, N, G, gen, dtype=torch.float16):
    q = torch.randint(0, 16, (E, K, N), generator=gen, device=DEV, dtype=torch.int32)
    z = torch.randint(0, 16, (E, K // G, N), generator=gen, device=DEV, dtype=torch.int32)
    s = (torch.rand((E, K // G, N), generator=gen, device=DEV) * 0.018 + 0.002).to(dtype)
    return {"qweight": _pack_awq_dev(q), "qzeros": _pack_awq_dev(z), "scales": s}


def _grouped_ref_gpu(ops, a, W, G, tw, ids, top_k, activation, mul):
    """The oracle's grouped GEMM in fp32 on the GPU, over bit-exact dequantised experts."""
    dt = a.dtype
    flat = ids.reshape(-1).long()
    N = W["qweight"].shape[2] * 8
    out = torch.zeros((flat.numel(), N // 2 if activation else N), dtype=dt, device=DEV)
    for e in torch.unique(flat).tolist():
        rows = torch.nonzero(flat == e).flatten()
        Wd = ops.dequant(W["qweight"][e], W["qzeros"][e], W["scales"][e]).float()
        y = a[rows // top_k].float() @ Wd
        if mul:
            y = y * tw.reshape(-1)[rows].float()[:, None]
        y = y.to(dt)
        if activation:
            y = oracle.silu_and_mul(y).to(dt)
        out[rows] = y
    return out


def test_qwen3_30b_a3b_experts_full_shape():
    """E=128, H=2048, I=768, top-8, T=512: both grouped GEMMs and the combine."""
    ops = _ops()
    from sglite_amd.moe import fused_experts_impl, fused_topk, process_awq_moe_weights
    E, H, I, k, T, G = 128, 2048, 768, 8, 512, 128
    gen = torch.Generator(device=DEV).manual_seed(0)
    W1 = _experts_dev(E, H, 2 * I, G, gen)
    W2 = _experts_dev(E, I, H, G, gen)
    x = torch.randn((T, H), generator=gen, device=DEV).half()
    logits = torch.randn((T, E), generator=gen, device=DEV)
    tw, ids = fused_topk(x, logits, k, True)
    rtw, rids = oracle.fused_topk(logits.cpu(), k, renormalize=True)
    assert torch.equal(ids.cpu(), rids)
    h_ref = _grouped_ref_gpu(ops, x, W1, G, tw, ids, k, "silu", False)
    y_ref = _grouped_ref_gpu(ops, h_ref, W2, G, tw, ids, 1, None, True)
    ref = y_ref.view(T, k, H).float().sum(1).half()
    w1 = process_awq_moe_weights(W1["qweight"], W1["qzeros"], W1["scales"])
    w2 = process_awq_moe_weights(W2["qweight"], W2["qzeros"], W2["scales"])
    align = ops.moe_align_block_size(ids, 16, E)
    h = ops.moe_gemm(x, w1.experts, H, 2 * I, G, align, tw, T * k, k, "silu", False)
    ok, err, mx = oracle.tolerance_ok(h, h_ref, TOL)
    assert ok, ("gate_up", err, mx)
    out = fused_experts_impl(x.clone(), w1, w2, tw, ids, "silu")
    ok, err, mx = oracle.tolerance_ok(out, ref, TOL)
    assert ok, ("forward", err, mx)
    again = fused_experts_impl(x.clone(), w1, w2, tw, ids, "silu")
    assert torch.equal(out, again)  # deterministic


def test_fused_experts_graph_replays():
    """Alignment, both GEMMs and the combine captured in one HIP graph; every
    replay (with eager work in between) matches the eager result."""
    from sglite_amd.moe import fused_experts_impl, process_awq_moe_weights
    T, E, k, H, I, G = 64, 32, 4, 512, 256, 128
    W1, W2 = _moe_weights(E, H, I, G, seed=123)
    _, tw, ids = _routing(T, E, k, seed=124)
    x = oracle.make_activation(T, H, seed=125).to(DEV)
    d1, d2 = _to_dev(W1), _to_dev(W2)
    w1 = process_awq_moe_weights(d1["qweight"], d1["qzeros"], d1["scales"])
    w2 = process_awq_moe_weights(d2["qweight"], d2["qzeros"], d2["scales"])
    twd, idd = tw.to(DEV), ids.to(DEV)
    eager = fused_experts_impl(x.clone(), w1, w2, twd, idd, "silu")
    buf = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused_experts_impl(buf, w1, w2, twd, idd, "silu")
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fused_experts_impl(buf, w1, w2, twd, idd, "silu")
    for i in range(4):
        buf.copy_(x)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(buf, eager), i
        _ = (x.float() @ x.float().T).sum().item()  # unrelated eager work between replays


def test_checkpoint_stream_to_fused_experts():
    """Per-expert AWQ checkpoint tensors (gate/up/down of each expert) ->
    ingest (gate/up merged on packed columns, experts stacked) -> repack ->
    fused experts, against the oracle on the logical weights."""
    from sglite_amd import checkpoint
    from sglite_amd.moe import fused_experts_impl, process_awq_moe_weights
    T, E, k, H, I, G = 20, 6, 2, 256, 128, 64
    W1, W2 = _moe_weights(E, H, I, G, seed=300)
    stream = []
    for e in range(E):
        for suffix in ("qweight", "qzeros", "scales"):
            gu = W1[suffix][e]
            half = gu.shape[1] // 2
            stream.append((f"model.layers.3.mlp.experts.{e}.gate_proj.{suffix}", gu[:, :half].contiguous()))
            stream.append((f"model.layers.3.mlp.experts.{e}.up_proj.{suffix}", gu[:, half:].contiguous()))
            stream.append((f"model.layers.3.mlp.experts.{e}.down_proj.{suffix}", W2[suffix][e]))
    out = dict(checkpoint.ingest(stream, num_experts=E, dtype=torch.float16))
    pre = "model.layers.3.mlp.experts."
    w1 = process_awq_moe_weights(*(out[pre + "gate_up_proj." + s].to(DEV) for s in ("qweight", "qzeros", "scales")))
    w2 = process_awq_moe_weights(*(out[pre + "down_proj." + s].to(DEV) for s in ("qweight", "qzeros", "scales")))
    _, tw, ids = _routing(T, E, k, seed=301)
    x = oracle.make_activation(T, H, seed=302)
    ref = oracle.fused_moe_awq(x, W1, W2, tw, ids, G)
    got = fused_experts_impl(x.to(DEV), w1, w2, tw.to(DEV), ids.to(DEV), "silu")
    ok, err, mx = oracle.tolerance_ok(got.cpu(), ref, TOL)
    assert ok, (err, mx)
