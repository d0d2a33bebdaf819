"""Pins the CPU oracle (oracle/awq_oracle.py) to the reference's semantics.

Each check is chosen so that a plausible slip in the oracle -- a wrong nibble
order, a wrong group index, a dropped zero point, double rounding, bias added
before rounding -- fails at least one of them.  No reference code is imported:
the Triton and Marlin unpack paths are re-expressed literally from their source
text (awq_triton.py:53-62, 93-96, 119-120; marlin_utils.py:249-282, 336-347).
"""

import os

import math

import numpy as np
import pytest
import torch

from oracle import awq_oracle as oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "awq_golden.npz")


# --------------------------------------------------------------------------
# nibble order
# --------------------------------------------------------------------------

def test_kat_unpack_identity_word():
    # nibble p holds value p -> logical columns read nibbles [0,4,1,5,2,6,3,7]
    q = oracle.unpack_awq(np.array([[0x76543210]], dtype=np.int64))
    assert q.tolist() == [[0, 4, 1, 5, 2, 6, 3, 7]]


def test_kat_pack_logical_ramp():
    w = oracle.pack_awq(np.arange(8)[None, :]).view(np.uint32)
    assert int(w[0, 0]) == 0x75316420


def test_single_nibble_selects_one_column():
    for p in range(8):
        word = np.array([[np.uint32(0xA) << np.uint32(4 * p)]], dtype=np.uint32).astype(np.int64)
        q = oracle.unpack_awq(word)[0]
        assert np.count_nonzero(q) == 1
        assert q[oracle.AWQ_ORDER[p]] == 0xA


def _triton_literal_unpack(packed: np.ndarray) -> np.ndarray:
    """awq_triton.py:53-62, 93-96, 119: triple interleave then (b >> shifts) & 0xF."""
    b = packed.astype(np.int64).astype(np.int32)

    def interleave(a, c):  # tl.interleave: result[..., 2i] = a[..., i], result[..., 2i+1] = c[..., i]
        r = np.empty(a.shape[:-1] + (a.shape[-1] * 2,), dtype=a.dtype)
        r[..., 0::2] = a
        r[..., 1::2] = c
        return r

    b = interleave(b, b)
    b = interleave(b, b)
    b = interleave(b, b)
    reverse_awq_order_tensor = ((np.arange(0, 2) * 4)[None, :] + np.arange(0, 4)[:, None]).reshape(8)
    shifts = reverse_awq_order_tensor * 4
    BK, BN = b.shape
    shifts = np.broadcast_to(shifts[None, :], (BK * (BN // 8), 8)).reshape(BK, BN)
    return (b >> shifts) & 0xF  # arithmetic shift, as in Triton on int32


def _marlin_literal_unpack(packed: np.ndarray) -> np.ndarray:
    """marlin_utils.py:272-281 (unpack_cols) then :340-348 (undo the AWQ interleave)."""
    size_k, n8 = packed.shape
    size_n = n8 * 8
    p = packed.astype(np.int64).astype(np.uint32)
    q_res = np.zeros((size_k, size_n), dtype=np.uint32)
    for i in range(8):
        q_res[:, i::8] = p & 0xF
        p = p >> 4
    undo = np.argsort(np.array([0, 2, 4, 6, 1, 3, 5, 7]))
    return q_res.reshape((-1, 8))[:, undo].ravel().reshape((-1, size_n)).astype(np.int32)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_unpack_matches_triton_and_marlin_readings(seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 2**32, size=(17, 9), dtype=np.uint64).astype(np.uint32).view(np.int32)
    q = oracle.unpack_awq(packed)
    np.testing.assert_array_equal(q, _triton_literal_unpack(packed))
    np.testing.assert_array_equal(q, _marlin_literal_unpack(packed))


def test_pack_unpack_roundtrip():
    rng = np.random.default_rng(5)
    q = rng.integers(0, 16, size=(33, 40))
    np.testing.assert_array_equal(oracle.unpack_awq(oracle.pack_awq(q)), q)


# --------------------------------------------------------------------------
# dequantisation
# --------------------------------------------------------------------------

def _pair_grid_weights(scales_list, dtype):
    """K = G = 32 (one group); column n: q = n % 16, z = (n // 16) % 16, s = scales_list[n // 256]."""
    S = len(scales_list)
    N = 256 * S
    K = 32
    n = np.arange(N)
    q = np.broadcast_to((n % 16)[None, :], (K, N)).copy()
    z = ((n // 16) % 16)[None, :]
    s = torch.tensor(np.repeat(np.asarray(scales_list, dtype=np.float64), 256)[None, :]).to(dtype)
    return q, z, s


def _fp16_sweep():
    # every positive normal fp16 in [2^-10, 2^10) plus their negatives, thinned
    vals = np.arange(0x1400, 0x6400, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    return np.concatenate([vals, -vals[::5], [0.0]])


def test_dequant_fp16_exhaustive_pairs_against_numpy_rounding():
    sw = _fp16_sweep()
    q, z, s = _pair_grid_weights(sw, torch.float16)
    W = oracle.dequantize(oracle.pack_awq(q), oracle.pack_awq(z), s, 32)
    expect = np.float16((q - z).astype(np.float64) * s.double().numpy())
    np.testing.assert_array_equal(W.numpy().view(np.uint16), expect.view(np.uint16))


def test_dequant_bf16_exhaustive_pairs_against_bit_rounding():
    vals = np.arange(0x3A80, 0x4480, 3, dtype=np.uint32)  # bf16 patterns ~[1e-3, 1024)
    sw = (vals << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    q, z, s = _pair_grid_weights(sw, torch.bfloat16)
    W = oracle.dequantize(oracle.pack_awq(q), oracle.pack_awq(z), s, 32)
    expect = oracle.bf16_round_bits((q - z).astype(np.float64) * s.double().numpy())
    np.testing.assert_array_equal(W.view(torch.int16).numpy().view(np.uint16), expect)


@pytest.mark.parametrize("K,N,G", [(256, 64, 128), (96, 24, 32), (384, 40, 384), (2560, 1024, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_torch_dequant_is_bit_exact_with_the_numpy_oracle(K, N, G, dtype):
    """dequantize_torch (the CPU baseline's multithreaded dequantisation) equals dequantize bit for bit."""
    t = oracle.make_awq_linear(K, N, G, seed=K + N, dtype=dtype)
    a = oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], G)
    b = oracle.dequantize_torch(t["qweight"], t["qzeros"], t["scales"], G)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_adversarial_activations_are_finite_and_shaped():
    for kind in oracle.ADVERSARIAL_KINDS:
        x = oracle.make_adversarial_activation(3, 2560, kind, seed=1)
        assert x.shape == (3, 2560) and bool(torch.isfinite(x).all())
    assert float(oracle.make_adversarial_activation(2, 512, "mean10", 0).float().mean()) > 9.0
    assert float(oracle.make_adversarial_activation(2, 512, "near_max", 0).float().abs().max()) > 4.0e4
    ok, ratio = oracle.elementwise_ok(torch.tensor([1.0, 2.0]), torch.tensor([1.0, 2.01]), 1e-2, 0.0)
    assert ok and ratio < 1.0
    ok, _ = oracle.elementwise_ok(torch.tensor([1.0, 2.2]), torch.tensor([1.0, 2.0]), 1e-2, 1e-3)
    assert not ok


def test_dequant_rounds_once_not_twice():
    # (q - z) * s with s = 1 + 2^-10 and q - z = 13 - 10: the exact product
    # 3.0029296875 is a tie between two fp16 values and rounds to even
    # (3.00390625); rounding 13*s and 10*s separately and subtracting gives
    # 3.0078125 instead.
    s = torch.tensor([[1.0 + 2.0 ** -10]], dtype=torch.float16).expand(1, 8).contiguous()
    q = np.full((32, 8), 13)
    z = np.full((1, 8), 10)
    W = oracle.dequantize(oracle.pack_awq(q), oracle.pack_awq(z), s, 32)
    assert float(W[0, 0]) == float(np.float16(3 * (1 + 2.0 ** -10)))
    sep = float(np.float16(np.float16(13 * (1 + 2.0 ** -10)) - np.float16(10 * (1 + 2.0 ** -10))))
    assert float(W[0, 0]) != sep


def test_dequant_special_cases_and_group_mapping():
    K, N, G = 512, 16, 128
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, size=(K, N))
    # q == z -> 0
    zq = q[::G][: K // G]
    same = np.repeat(zq, G, axis=0)
    s = torch.full((K // G, N), 0.013, dtype=torch.float16)
    W = oracle.dequantize(oracle.pack_awq(same), oracle.pack_awq(zq), s, G)
    assert torch.count_nonzero(W) == 0
    # z = 0, s = 1 -> q
    W = oracle.dequantize(oracle.pack_awq(q), oracle.pack_awq(np.zeros((K // G, N), int)),
                          torch.ones((K // G, N), dtype=torch.float16), G)
    np.testing.assert_array_equal(W.numpy(), q.astype(np.float16))
    # s[g] = 2^-g, q = 1, z = 0 -> W[k] = 2^-(k // G)
    sg = torch.tensor([2.0 ** -g for g in range(K // G)], dtype=torch.float16)[:, None].expand(K // G, N).contiguous()
    W = oracle.dequantize(oracle.pack_awq(np.ones((K, N), int)), oracle.pack_awq(np.zeros((K // G, N), int)), sg, G)
    expect = np.array([2.0 ** -(k // G) for k in range(K)])[:, None]
    np.testing.assert_array_equal(W.double().numpy(), np.broadcast_to(expect, (K, N)))


def test_channelwise_group_is_k():
    K, N = 256, 8
    t = oracle.make_awq_linear(K, N, -1, seed=4)
    assert t["qzeros"].shape == (1, 1) and t["scales"].shape == (1, N)
    W = oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], -1)
    q = oracle.unpack_awq(t["qweight"])
    z = oracle.unpack_awq(t["qzeros"])
    expect = np.float16((q - z[0]).astype(np.float64) * t["scales"].double().numpy()[0])
    np.testing.assert_array_equal(W.numpy(), expect)


# --------------------------------------------------------------------------
# GEMM
# --------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 3])
def test_gemm_brute_force_float64(M):
    K, N, G = 128, 8, 128
    t = oracle.make_awq_linear(K, N, G, seed=6)
    x = oracle.make_activation(M, K, seed=7)
    y = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], group_size=G)
    y64 = oracle.awq_gemm_f64(x, t["qweight"], t["qzeros"], t["scales"], G)
    # fp32 accumulation then one fp16 rounding: within one fp16 ulp of the exact value
    ulp = np.spacing(np.abs(y64).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(y.double().numpy() - y64) <= ulp + 1e-6)


def test_gemm_integer_inputs_are_exact():
    K, N, G = 256, 16, 128
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, size=(K, N))
    qw = oracle.pack_awq(q)
    qz = oracle.pack_awq(np.zeros((K // G, N), int))
    s = torch.ones((K // G, N), dtype=torch.float16)
    x = torch.tensor(rng.integers(-1, 2, size=(4, K)), dtype=torch.float16)
    y = oracle.awq_gemm(x, qw, qz, s, group_size=G)
    expect = x.double().numpy() @ q.astype(np.float64)
    assert np.all(np.abs(expect) < 2048)
    np.testing.assert_array_equal(y.double().numpy(), expect)


def test_gemm_one_hot_rows_select_weight_rows():
    K, N, G = 256, 24, 64
    t = oracle.make_awq_linear(K, N, G, seed=9)
    W = oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], G)
    rows = [0, 63, 64, 200, 255]
    x = torch.zeros((len(rows), K), dtype=torch.float16)
    for i, k in enumerate(rows):
        x[i, k] = 1.0
    y = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], group_size=G)
    assert torch.equal(y, W[rows])


def test_gemm_bias_added_after_rounding():
    K, N, G = 128, 8, 128
    t = oracle.make_awq_linear(K, N, G, seed=10)
    x = oracle.make_activation(2, K, seed=11)
    bias = torch.randn(N).to(torch.float16)
    y = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], bias, G)
    y0 = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
    assert torch.equal(y, (y0.float() + bias.float()).to(torch.float16))


def test_gemm_keeps_leading_dims():
    K, N, G = 128, 16, 128
    t = oracle.make_awq_linear(K, N, G, seed=12)
    x = oracle.make_activation(6, K, seed=13).reshape(2, 3, K)
    y = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], group_size=G)
    assert y.shape == (2, 3, N)


def test_tolerance_rule_catches_a_dropped_zero_point():
    # planted mistake: forgetting the zero point must fail the 2e-2 contract
    K, N, G = 256, 32, 128
    t = oracle.make_awq_linear(K, N, G, seed=14)
    x = oracle.make_activation(4, K, seed=15)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], group_size=G)
    zero = torch.from_numpy(oracle.pack_awq(np.zeros((K // G, N), int)))
    bad = oracle.awq_gemm(x, t["qweight"], zero, t["scales"], group_size=G)
    assert not oracle.tolerance_ok(bad, ref)[0]
    assert oracle.tolerance_ok(ref, ref)[0]


# --------------------------------------------------------------------------
# repacked layout (the engine's own format)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("K,N,G", [(256, 64, 128), (96, 24, 32), (384, 40, -1), (160, 16, 32), (4096, 48, 128)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_repack_roundtrip(K, N, G, dtype):
    t = oracle.make_awq_linear(K, N, G, seed=K + N, dtype=dtype)
    wb, sz = oracle.repack_cdna4(t["qweight"], t["qzeros"], t["scales"], G)
    sh = oracle.repacked_shapes(K, N, oracle.resolve_group_size(G, K))
    assert wb.size == sh["w_bytes"] and sz.size == sh["s_bytes"] + sh["z_bytes"]
    qw, qz, s = oracle.unrepack_cdna4(wb, sz, K, N, G, dtype)
    np.testing.assert_array_equal(qw, t["qweight"].numpy())
    np.testing.assert_array_equal(qz, t["qzeros"].numpy())
    assert torch.equal(s, t["scales"])


def test_repack_tile_word_positions():
    # a single nonzero nibble lands where the layout says
    K, N, G = 256, 32, 128
    q = np.zeros((K, N), int)
    k, n = 165, 21  # kt=1, w=1, lg=0, j=5 ; nt=1, c=5
    q[k, n] = 9
    t = {"qweight": oracle.pack_awq(q), "qzeros": oracle.pack_awq(np.zeros((K // G, N), int)),
         "scales": torch.ones((K // G, N), dtype=torch.float16)}
    wb, _ = oracle.repack_cdna4(t["qweight"], t["qzeros"], t["scales"], G)
    words = wb.view(np.uint32)
    KT = 2
    nt, kt, w, lg, c, j = 1, 1, 1, 0, 5, 5
    lane = lg * 16 + c
    idx = (nt * KT + kt) * 256 + lane * 4 + w
    p = oracle.AWQ_ORDER.index(j)
    assert words[idx] == 9 << (4 * p)
    assert np.count_nonzero(words) == 1


# --------------------------------------------------------------------------
# MoE
# --------------------------------------------------------------------------

def _moe_case(T=5, E=4, H=128, I=64, k=2, seed=20, G=64):
    w1 = [oracle.make_awq_linear(H, 2 * I, G, seed=seed + e) for e in range(E)]
    w2 = [oracle.make_awq_linear(I, H, G, seed=seed + 100 + e) for e in range(E)]
    W1 = {key: torch.stack([w[key] for w in w1]) for key in ("qweight", "qzeros", "scales")}
    W2 = {key: torch.stack([w[key] for w in w2]) for key in ("qweight", "qzeros", "scales")}
    x = oracle.make_activation(T, H, seed=seed + 7)
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(seed + 8))
    tw, ids = oracle.fused_topk(logits, k, renormalize=True)
    return x, W1, W2, tw, ids, G


def test_fused_topk_renormalises():
    logits = torch.randn((7, 16), generator=torch.Generator().manual_seed(0))
    w, ids = oracle.fused_topk(logits, 4)
    assert ids.dtype == torch.int32 and w.dtype == torch.float32
    torch.testing.assert_close(w.sum(-1), torch.ones(7), rtol=0, atol=1e-6)
    p = torch.softmax(logits, -1)
    assert torch.equal(ids.long(), torch.topk(p, 4).indices)


def test_moe_vectorised_matches_loops():
    x, W1, W2, tw, ids, G = _moe_case()
    a = oracle.fused_moe_awq(x, W1, W2, tw, ids, G)
    b = oracle.fused_moe_awq_loops(x, W1, W2, tw, ids, G)
    # same rounding points; only fp32 summation order differs
    torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("n,E,bs", [(0, 4, 16), (7, 4, 16), (200, 8, 16), (4096, 128, 16), (333, 60, 32),
                                    (50, 512, 64)])
def test_moe_align_invariants(n, E, bs):
    """Each bucket holds exactly its expert's rows in increasing order, then
    sentinels up to a multiple of the block size; ids outside [0, E) vanish."""
    rng = np.random.default_rng(n + E)
    ids = rng.integers(-1, E, size=n).astype(np.int32)
    sorted_ids, expert_ids, npp, off = oracle.moe_align_block_size(ids, bs, E)
    assert sorted_ids.size == n + E * (bs - 1)
    assert off[0] == 0 and off[E] == npp[0]
    seen = []
    for e in range(E):
        bucket = sorted_ids[off[e]:off[e + 1]]
        rows = np.nonzero(ids == e)[0]
        assert (off[e + 1] - off[e]) % bs == 0
        assert off[e + 1] - off[e] - rows.size < bs
        np.testing.assert_array_equal(bucket[:rows.size], rows)
        assert (bucket[rows.size:] == n).all()
        assert (expert_ids[off[e] // bs:off[e + 1] // bs] == e).all()
        seen.extend(rows.tolist())
    assert sorted(seen) == np.nonzero((ids >= 0) & (ids < E))[0].tolist()
    assert (expert_ids[npp[0] // bs:] == -1).all()


def test_gelu_and_mul_closed_form():
    h = torch.tensor([[-3.0, -0.5, 0.0, 2.0, 1.5, -2.0, 4.0, 0.25]])
    ref = [0.5 * g * (1 + math.erf(g / math.sqrt(2))) * u for g, u in zip(h[0, :4].tolist(), h[0, 4:].tolist())]
    # 1 + erf(x) cancels for x << 0, so the fp32 result carries an absolute error
    torch.testing.assert_close(oracle.gelu_and_mul(h)[0], torch.tensor(ref), rtol=1e-6, atol=2e-6)
    ref_s = [g / (1 + math.exp(-g)) * u for g, u in zip(h[0, :4].tolist(), h[0, 4:].tolist())]
    torch.testing.assert_close(oracle.silu_and_mul(h)[0], torch.tensor(ref_s), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("activation", [None, "silu", "gelu"])
@pytest.mark.parametrize("mul", [False, True])
def test_moe_grouped_gemm_matches_row_loops(activation, mul):
    """Per routed row: a[r // top_k] @ W[e(r)] in float64, x weight, rounded; the
    activation in float64 of the rounded halves."""
    x, W1, W2, tw, ids, G = _moe_case(T=6, E=4, k=3)
    k = ids.shape[1]
    out = oracle.moe_grouped_gemm(x, W1, tw, ids, k, G, activation, mul)
    for r in range(ids.numel()):
        e = int(ids.reshape(-1)[r])
        W = oracle.dequantize(W1["qweight"][e], W1["qzeros"][e], W1["scales"][e], G).double()
        y = x[r // k].double() @ W
        if mul:
            y = y * float(tw.reshape(-1)[r])
        y = y.half().double()
        if activation:
            d = y.shape[0] // 2
            g, u = y[:d], y[d:]
            a = g / (1 + torch.exp(-g)) if activation == "silu" else 0.5 * g * (1 + torch.erf(g / math.sqrt(2)))
            y = (a * u).half().double()
        torch.testing.assert_close(out[r].double(), y, rtol=2e-3, atol=2e-3)


def test_moe_router_weight_on_input_moves_the_multiply():
    x, W1, W2, _, ids, G = _moe_case(T=4, E=3, k=1)
    # top-1 weights without renormalisation (renormalised they would all be 1)
    tw = torch.rand(ids.shape, generator=torch.Generator().manual_seed(3)) * 0.5 + 0.25
    a = oracle.fused_moe_awq(x, W1, W2, tw, ids, G, apply_router_weight_on_input=True)
    h = oracle.moe_grouped_gemm(x, W1, tw, ids, 1, G, "silu", True)
    y = oracle.moe_grouped_gemm(h, W2, None, ids, 1, G, None, False)
    assert torch.equal(a, y.view(4, 1, -1).float().sum(1).half())
    b = oracle.fused_moe_awq(x, W1, W2, tw, ids, G)
    assert not torch.equal(a, b)


# --------------------------------------------------------------------------
# golden fixtures
# --------------------------------------------------------------------------

def _half(a, dt):
    return torch.from_numpy(a.view(np.int16).copy()).view(dt)


def test_golden_fixtures_reproduce():
    g = np.load(GOLDEN, allow_pickle=False)
    np.testing.assert_array_equal(g["kat_unpacked"][0], [0, 4, 1, 5, 2, 6, 3, 7])
    np.testing.assert_array_equal(oracle.unpack_awq(g["kat_words"].view(np.int32)[None, :]).reshape(-1, 8),
                                  g["kat_unpacked"])
    names = sorted({k.split("/")[0] for k in g.files if "/" in k})
    assert len(names) == 4
    for name in names:
        K, N, G = (int(v) for v in g[f"{name}/shape"])
        dt = torch.bfloat16 if "bf16" in name else torch.float16
        qw = torch.from_numpy(g[f"{name}/qweight"])
        qz = torch.from_numpy(g[f"{name}/qzeros"])
        s = _half(g[f"{name}/scales"], dt)
        W = oracle.dequantize(qw, qz, s, G)
        np.testing.assert_array_equal(W.view(torch.int16).numpy().view(np.uint16), g[f"{name}/W"])
        bias = _half(g[f"{name}/bias"], dt) if f"{name}/bias" in g.files else None
        for key in g.files:
            if key.startswith(f"{name}/x"):
                M = key.split("/x")[1]
                x = _half(g[key], dt)
                y = oracle.awq_gemm(x, qw, qz, s, bias, G)
                np.testing.assert_array_equal(y.view(torch.int16).numpy().view(np.uint16), g[f"{name}/y{M}"])


def _dense_gated_mlp(x, tgu, tdn, G, act):
    """The package's GatedMLP on the unquantized method with the dequantized weights."""
    from sglite_amd.mlp import GatedMLP

    H, I = x.shape[1], tdn["qweight"].shape[0]
    mlp = GatedMLP(H, I, act)
    wgu = oracle.dequantize(tgu["qweight"], tgu["qzeros"], tgu["scales"], G).float()
    wdn = oracle.dequantize(tdn["qweight"], tdn["qzeros"], tdn["scales"], G).float()
    mlp.load_state_dict({"gate_up_proj.weight": wgu.t().contiguous(), "down_proj.weight": wdn.t().contiguous()})
    return mlp(x)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_gated_mlp_oracle_matches_dense_block_in_fp32(act):
    """With fp32 activations no rounding separates the steps, so the oracle's composition must be
    the dense block (blocks.py:51-57) on the same weights: gate half first, act on the gate only,
    times up, then the down projection."""
    H, I, G, M = 256, 384, 128, 5
    tgu = oracle.make_awq_linear(H, 2 * I, G, seed=41)
    tdn = oracle.make_awq_linear(I, H, G, seed=42)
    x = oracle.make_activation(M, H, seed=43).float()
    got = oracle.gated_mlp_awq(x, tgu, tdn, G, act)
    ref = _dense_gated_mlp(x, tgu, tdn, G, act)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4 * float(ref.abs().max()))


def test_gated_mlp_oracle_is_the_two_awq_gemms():
    """At fp16 each of the oracle's GEMMs is awq_gemm itself (no bias), with the activation's
    rounding in between."""
    H, I, G, M = 256, 384, 64, 3
    tgu = oracle.make_awq_linear(H, 2 * I, G, seed=47)
    tdn = oracle.make_awq_linear(I, H, G, seed=48)
    x = oracle.make_activation(M, H, seed=49)
    y = oracle.awq_gemm(x, tgu["qweight"], tgu["qzeros"], tgu["scales"], None, G)
    h = oracle.gelu_and_mul(y).to(torch.float16)
    ref = oracle.awq_gemm(h, tdn["qweight"], tdn["qzeros"], tdn["scales"], None, G)
    assert torch.equal(oracle.gated_mlp_awq(x, tgu, tdn, G, "gelu"), ref)


def test_gated_mlp_oracle_rounds_between_steps_and_a_swapped_half_fails():
    """At fp16 the oracle rounds the gate/up output, then act(gate) * up once, and the result stays
    within fp16 error of the fp32 block; a gate/up swap (a plausible slip) is caught by the same
    tolerance rule the GPU tests use."""
    H, I, G, M = 256, 384, 128, 4
    tgu = oracle.make_awq_linear(H, 2 * I, G, seed=44)
    tdn = oracle.make_awq_linear(I, H, G, seed=45)
    x = oracle.make_activation(M, H, seed=46)
    got = oracle.gated_mlp_awq(x, tgu, tdn, G, "silu")
    assert got.dtype == torch.float16 and got.shape == (M, H)
    ref = _dense_gated_mlp(x.float(), tgu, tdn, G, "silu")
    ok, err, mx = oracle.tolerance_ok(got, ref, 2e-2)
    assert ok, (err, mx)
    y = oracle.awq_gemm(x, tgu["qweight"], tgu["qzeros"], tgu["scales"], None, G)
    swapped = torch.cat([y[:, I:], y[:, :I]], dim=1)
    h_bad = oracle.silu_and_mul(swapped).to(torch.float16)
    bad = oracle.awq_gemm(h_bad, tdn["qweight"], tdn["qzeros"], tdn["scales"], None, G)
    assert not oracle.tolerance_ok(bad, ref, 2e-2)[0]
