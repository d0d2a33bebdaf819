"""Full-size parity beyond the fp16 config shapes: bf16 at the Qwen3-4B and
Llama-3-8B shapes, the Llama-3-8B decode batches 2 and 4, one GPU's share of
tensor-parallel shards, and the Qwen3-30B-A3B expert shape against the CPU
oracle on sampled tokens.  Each GEMM output is checked against the CPU oracle
on sampled rows x three 256-column blocks (the HIP dequantisation of those
blocks bit-exact) and against a GPU fp32 matmul of the pinned weight, within
max|err| <= 2e-2 * max|ref|."""

import pytest
import torch

from oracle import awq_oracle as oracle
from test_gpu_moe import _experts_dev
from test_gpu_parity import LLAMA3_8B, QWEN3_4B, _check_full_size, _linear

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2


def _ops():
    from sglite_amd import ops

    return ops


def _full_size_case(K, N, M, seed, dtype=torch.float16):
    ops = _ops()
    t, d = _linear(K, N, 128, seed=seed, dtype=dtype)
    r = ops.repack(d["qweight"], d["qzeros"], d["scales"])
    W = ops.dequant_repacked(r, K, N, 128)
    x = oracle.make_activation(M, K, seed=seed + M, dtype=dtype)
    print(f"case K={K} N={N} M={M} {dtype}: {ops.plan_info(M, N, K, 128)}", flush=True)
    y = ops.gemm(x.to(DEV), r, K, N, 128, counters=ops.make_counters(N, DEV))
    assert y.shape == (M, N) and y.dtype == dtype
    _check_full_size(y, W, x, t, K, N)


@pytest.mark.parametrize("K,N", QWEN3_4B)
@pytest.mark.parametrize("M", [1, 8, 32])
def test_qwen3_4b_decode_bf16(K, N, M):
    _full_size_case(K, N, M, seed=K + N + 1, dtype=torch.bfloat16)


@pytest.mark.parametrize("K,N", LLAMA3_8B)
@pytest.mark.parametrize("M", [1, 16, 256, 2048])
def test_llama3_8b_bf16(K, N, M):
    _full_size_case(K, N, M, seed=K * 2 + N + 1, dtype=torch.bfloat16)


@pytest.mark.parametrize("K,N", LLAMA3_8B)
@pytest.mark.parametrize("M", [2, 4])
def test_llama3_8b_small_decode_batches(K, N, M):
    """The reference captures decode graphs at 1, 2, 4 and multiples of 8
    (cuda_graph.py:76)."""
    _full_size_case(K, N, M, seed=K * 2 + N)


# One GPU's shard of column-parallel (N / tp) and row-parallel (K / tp)
# linears (weight_loader.py:40-69, linear.py:127-194).
TP_SHARDS = [
    (8192, 1280), (1024, 8192), (8192, 7168), (3584, 8192),   # Llama-3.1-70B at TP8
    (4096, 3072), (2048, 4096), (4096, 14336), (7168, 4096),  # Llama-3-8B at TP2
    (4096, 1536), (1024, 4096), (4096, 7168), (3584, 4096),   # Llama-3-8B at TP4
]


@pytest.mark.parametrize("K,N", TP_SHARDS)
@pytest.mark.parametrize("M", [1, 8, 32, 2048])
def test_tensor_parallel_shards(K, N, M):
    _full_size_case(K, N, M, seed=K + 3 * N)


def test_qwen3_30b_a3b_experts_against_cpu_oracle():
    """E=128, H=2048, I=768, top-8, T=512: the whole forward on the GPU, six
    tokens of it against the CPU oracle's fused MoE (fused.py:101-202) on
    the experts those tokens route to."""
    from sglite_amd.moe import fused_experts_impl, fused_topk, process_awq_moe_weights
    E, H, I, k, T, G = 128, 2048, 768, 8, 512, 128
    gen = torch.Generator(device=DEV).manual_seed(7)
    W1 = _experts_dev(E, H, 2 * I, G, gen)
    W2 = _experts_dev(E, I, H, G, gen)
    x = oracle.make_activation(T, H, seed=8)
    logits = torch.randn((T, E), generator=torch.Generator().manual_seed(9))
    w1 = process_awq_moe_weights(W1["qweight"], W1["qzeros"], W1["scales"])
    w2 = process_awq_moe_weights(W2["qweight"], W2["qzeros"], W2["scales"])
    tw, ids = fused_topk(x.to(DEV), logits.to(DEV), k, True)
    out = fused_experts_impl(x.to(DEV), w1, w2, tw, ids, "silu").cpu()
    rtw, rids = oracle.fused_topk(logits, k, renormalize=True)
    assert torch.equal(ids.cpu(), rids)
    tokens = [0, 1, 255, 256, 510, 511]
    used = sorted(set(rids[tokens].reshape(-1).tolist()))
    remap = {e: i for i, e in enumerate(used)}
    sub1 = {s: W1[s][used].cpu() for s in W1}
    sub2 = {s: W2[s][used].cpu() for s in W2}
    sub_ids = torch.tensor([[remap[int(e)] for e in row] for row in rids[tokens].tolist()], dtype=torch.int64)
    ref = oracle.fused_moe_awq(x[tokens], sub1, sub2, rtw[tokens], sub_ids, G)
    ok, err, mx = oracle.tolerance_ok(out[tokens], ref, TOL)
    assert ok, (err, mx)
