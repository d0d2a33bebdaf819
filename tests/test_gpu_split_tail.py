"""Regression test for the steps after the tiled kernels' counted k loop.

Those steps prefetch k-tiles past the k-slice whose weights nobody reads, so
the compiler removes the weight loads; the loop's counted wait then let a step
pass its barrier before the next k-tile's activation fragments had landed, and
the last k-tile of a slice was multiplied with stale LDS contents.  It showed
on cold memory only: the first call after new weights and activations gave
wrong output rows (whole 16-row m-tiles) in a few tiles, the next call was
right.  Seen with G = 64 (three pipeline stages, where a slice of 3r + 2
k-tiles needs the activations of its last k-tile at such a barrier) on the
16x16 kernel at 32 and 64 rows, about once per hundred fresh shapes.

Each case here draws fresh weights and activations (on the device, so the
first call reads cold memory), makes two calls and requires them to be
bit-identical and the first to match the CPU oracle on sampled rows.  The
cases are split-K tiled plans in which some k-slice has 3r + 2 k-tiles."""

import random

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _cases(n=48, seed=77):
    from sglite_amd import ops

    rng = random.Random(seed)
    out = []
    while len(out) < n:
        G = rng.choice([64, 64, 64, 128])
        K = G * rng.randint(max(1, 512 // G), 6144 // G)
        N = 8 * rng.randint(16, 400)
        M = rng.choice([20, 32, 40, 64, 100, 200, 300, 512, 700])
        info = ops.plan_info(M, N, K, G)
        if info.kernel != "tiled_kernel" or info.k_slices == 1:
            continue
        KT = (K + 127) // 128
        ktc = -(-KT // info.k_slices)
        slices = [min(KT - s * ktc, ktc) for s in range(info.k_slices)]
        if not any(n_ > 0 and n_ % 3 == 2 for n_ in slices):
            continue
        out.append((len(out), M, K, N, G, rng.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c[0]}-M{c[1]}-K{c[2]}-N{c[3]}-G{c[4]}")
def test_split_k_tail_steps_read_landed_activations(case):
    from sglite_amd import ops

    i, M, K, N, G, dtype = case
    t = oracle.make_awq_linear(K, N, G, seed=9000 + i, dtype=dtype)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    xg = torch.Generator(device=DEV).manual_seed(9500 + i)
    x = torch.randn((M, K), generator=xg, device=DEV).to(dtype)
    cnt = ops.make_counters(N, DEV)
    y1 = ops.gemm(x, r, K, N, G, counters=cnt)
    y2 = ops.gemm(x, r, K, N, G, counters=cnt)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), (case, ops.plan_info(M, N, K, G))
    rows = sorted(set([0, M - 1] + random.Random(i).sample(range(M), min(M, 24))))
    xs = x[rows].cpu()
    ref = oracle.awq_gemm(xs, t["qweight"], t["qzeros"], t["scales"], None, G)
    ok, err, mx = oracle.tolerance_ok(y1[rows].cpu(), ref, 2e-2)
    assert ok, (case, err, mx)
