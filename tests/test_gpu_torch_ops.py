"""torch.ops.sglite_awq on the GPU: the registered ops give the same bytes as
the Python wrappers eagerly, inside a captured torch.cuda.graph (replayed
several times with eager work between the replays), through FakeTensor shape
propagation of real-shaped inputs, and under torch.compile (aot_eager), with
outputs checked against the CPU oracle."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2


def _setup(K, N, G=128, seed=0):
    from sglite_amd import ops

    t = oracle.make_awq_linear(K, N, G, seed=seed)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    return ops, t, r, ops.make_counters(N, DEV)


@pytest.mark.parametrize("M,K,N", [(1, 2560, 6144), (8, 4096, 2560), (32, 28672, 512), (300, 2048, 1024)])
def test_op_eager_matches_wrapper_and_oracle(M, K, N):
    ops, t, r, cnt = _setup(K, N, seed=M + K)
    x = oracle.make_activation(M, K, seed=M)
    xd = x.to(DEV)
    y_op = torch.ops.sglite_awq.awq_w4a16_gemm(xd, r.w, r.s, r.z, None, cnt, K, N, 128)
    y_py = ops.gemm(xd, r, K, N, 128, counters=cnt)
    assert torch.equal(y_op, y_py)
    out = torch.empty_like(y_op)
    torch.ops.sglite_awq.awq_w4a16_gemm_out(xd, r.w, r.s, r.z, None, cnt, out, K, N, 128)
    assert torch.equal(out, y_op)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, 128)
    ok, err, mx = oracle.tolerance_ok(y_op, ref, TOL)
    assert ok, (err, mx)
    assert ops.counters_settled(cnt)


def test_op_under_graph_capture_replays():
    ops, t, r, cnt = _setup(28672, 512, seed=3)  # split K with arrival counters
    K, N = 28672, 512
    xs = [oracle.make_activation(8, K, seed=s).to(DEV) for s in range(3)]
    x = xs[0].clone()
    eager = [torch.ops.sglite_awq.awq_w4a16_gemm(v, r.w, r.s, r.z, None, cnt, K, N, 128) for v in xs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        torch.ops.sglite_awq.awq_w4a16_gemm(x, r.w, r.s, r.z, None, cnt, K, N, 128)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = torch.ops.sglite_awq.awq_w4a16_gemm(x, r.w, r.s, r.z, None, cnt, K, N, 128)
    for i in (0, 1, 2, 1, 0):
        x.copy_(xs[i])
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between the replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager[i]), i
        del junk
    assert ops.counters_settled(cnt)


def test_fake_propagation_of_real_tensors():
    ops, t, r, cnt = _setup(4096, 6144, seed=5)
    x = oracle.make_activation(17, 4096, seed=6).to(DEV)
    with FakeTensorMode(allow_non_fake_inputs=False) as mode:
        fx = mode.from_tensor(x)
        fw, fs, fz, fc = (mode.from_tensor(v) for v in (r.w, r.s, r.z, cnt))
        fy = torch.ops.sglite_awq.awq_w4a16_gemm(fx, fw, fs, fz, None, fc, 4096, 6144, 128)
        assert fy.shape == (17, 6144) and fy.dtype == torch.float16
        fh = torch.ops.sglite_awq.awq_w4a16_gemm_act(fx, fw, fs, fz, None, fc, 4096, 6144, 128, "gelu")
        assert fh.shape == (17, 3072)


def test_torch_compile_aot_eager():
    ops, t, r, cnt = _setup(2560, 6144, seed=7)
    K, N = 2560, 6144

    def f(x):
        y = torch.ops.sglite_awq.awq_w4a16_gemm(x, r.w, r.s, r.z, None, cnt, K, N, 128)
        return y * 2.0

    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    for M in (1, 8):
        x = oracle.make_activation(M, K, seed=M).to(DEV)
        assert torch.equal(cf(x), f(x))
