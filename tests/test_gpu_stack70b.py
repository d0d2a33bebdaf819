"""Llama-3.1-70B-shaped AWQ stack on one GPU: 80 layers x {qkv 8192->10240,
o 8192->8192, gate_up 8192->57344, down 28672->8192}, int4 group 128
(35.6 GB), run layer after layer at M = 64 and M = 4096.  Layers 0 and 79 go
through the checkpoint path (AWQ tensors -> repack) and are checked against
the CPU oracle on row x column blocks; the other layers are random repacked
tensors.  Repeated passes are bit-identical."""

import pytest
import torch

import bench
from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
G = 128
TOL = 2e-2


def _awq_linear_gpu(K, N, gen):
    q = torch.randint(0, 16, (K, N), generator=gen, device=DEV, dtype=torch.int32)
    z = torch.randint(0, 16, (K // G, N), generator=gen, device=DEV, dtype=torch.int32)
    s = (torch.rand((K // G, N), generator=gen, device=DEV) * 0.018 + 0.002).to(torch.float16)
    return bench.pack_awq_gpu(q), bench.pack_awq_gpu(z), s


def test_stack70b_checkpoint_layers_parity_and_whole_stack():
    from sglite_amd import ops
    gen = torch.Generator(device=DEV).manual_seed(0)
    awq = {}  # (layer, name) -> AWQ tensors on the CPU, for the oracle
    layers = []
    for li in range(bench.STACK70B_LAYERS):
        lay = {}
        for name, K, N in bench.STACK70B:
            if li in (0, bench.STACK70B_LAYERS - 1):
                qw, qz, sc = _awq_linear_gpu(K, N, gen)
                lay[name] = ops.repack(qw, qz, sc)
                awq[(li, name)] = (qw.cpu(), qz.cpu(), sc.cpu())
                del qw, qz, sc
            else:
                lay[name] = bench.random_repacked(ops, K, N, gen, DEV)
        layers.append(lay)
    cnts = {name: ops.make_counters(N, DEV) for name, K, N in bench.STACK70B}
    xg = torch.Generator().manual_seed(1)
    for M in (64, 4096):
        xs = {K: torch.randn((M, K), generator=xg).to(torch.float16) for _, K, _ in bench.STACK70B}
        xd = {K: v.to(DEV) for K, v in xs.items()}
        kept = {}
        for li, lay in enumerate(layers):
            for name, K, N in bench.STACK70B:
                y = ops.gemm(xd[K], lay[name], K, N, G, counters=cnts[name])
                if (li, name) in awq:
                    kept[(li, name)] = y
                assert bool(torch.isfinite(y).all()), (M, li, name)
        again = ops.gemm(xd[8192], layers[-1]["qkv_proj"], 8192, 10240, G, counters=cnts["qkv_proj"])
        assert torch.equal(again, kept[(bench.STACK70B_LAYERS - 1, "qkv_proj")])
        rows = torch.arange(M) if M <= 64 else torch.cat([torch.arange(128), torch.arange(M - 128, M)])
        for (li, name), y in kept.items():
            K, N = next((k, n) for nm, k, n in bench.STACK70B if nm == name)
            qw, qz, sc = awq[(li, name)]
            yc = y.cpu()
            for c0 in (0, (N // 2) // 256 * 256, N - 256):
                cols = slice(c0, c0 + 256)
                ref = oracle.awq_gemm(xs[K][rows], qw[:, c0 // 8:(c0 + 256) // 8], qz[:, c0 // 8:(c0 + 256) // 8],
                                      sc[:, cols], None, G)
                ok, err, mx = oracle.tolerance_ok(yc[rows][:, cols], ref, TOL)
                assert ok, (M, li, name, c0, err, mx)
        assert all(ops.counters_settled(c) for c in cnts.values())
        del xd, kept
