"""awq_w4a16_gemm_noalloc, through the C ABI: the entry point that takes its
split-K workspace and arrival counters from the library's static per-device
scratch.  Its output must equal awq_w4a16_gemm's (same plan, same kernels) on
two calls in a row, the second with a smaller input, for every kernel family
and split-K scheme; shapes beyond the scratch are rejected before any launch."""

import ctypes

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _lib_and_ops():
    from sglite_amd import _lib, ops

    return _lib, ops


def _gemm_abi(lib, ops, x, r, K, N, G, bias=None):
    """The existing entry point, with a caller workspace and counters."""
    M = x.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=DEV)
    wsb = lib.awq_workspace_bytes(M, N, K, G)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=DEV)
    cnt = ops.make_counters(N, DEV)
    st = lib.awq_w4a16_gemm(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(),
                            None if bias is None else bias.data_ptr(), out.data_ptr(), M, N, K, G,
                            ops.dtype_code(x.dtype), ws.data_ptr(), wsb, cnt.data_ptr(), cnt.numel() * 4,
                            torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib_and_ops()[0].last_error()
    return out


def _noalloc_abi(lib, x, r, K, N, G, bias=None):
    from sglite_amd import ops

    M = x.shape[0]
    out = torch.full((M, N), float("nan"), dtype=x.dtype, device=DEV)
    st = lib.awq_w4a16_gemm_noalloc(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(),
                                    None if bias is None else bias.data_ptr(), out.data_ptr(), M, N, K, G,
                                    ops.dtype_code(x.dtype), torch.cuda.current_stream().cuda_stream)
    assert st == 0, _lib_and_ops()[0].last_error()
    return out


CASES = [  # (K, N, G, first M, second M): each pair shares weights, the second call is smaller
    (28672, 512, 128, 32, 8),    # decode kernels, split K with arrival counters in the scratch
    (28672, 512, 128, 3, 1),     # GEMV biased operand, split K
    (14336, 4096, 128, 64, 40),  # tiled kernel, split-K partials in the scratch
    (2560, 6144, 128, 16, 1),    # GEMV, no split
    (4096, 2560, 64, 300, 33),   # tiled, G = 64
]


@pytest.mark.parametrize("K,N,G,M1,M2", CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_matches_existing_entry_point(K, N, G, M1, M2, dtype):
    abi, ops = _lib_and_ops()
    lib = abi.load()
    t = oracle.make_awq_linear(K, N, G, seed=K + N + M1, dtype=dtype)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    bias = torch.randn(N, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)
    for M in (M1, M2):
        x = oracle.make_activation(M, K, seed=M, dtype=dtype).to(DEV)
        for b in (None, bias):
            want = _gemm_abi(lib, ops, x, r, K, N, G, b)
            got = _noalloc_abi(lib, x, r, K, N, G, b)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (K, N, G, M, b is None)
    # the first rows of the oracle, as a check that both are right, not only equal
    x = oracle.make_activation(M2, K, seed=M2, dtype=dtype)
    ref = oracle.awq_gemm(x, t["qweight"], t["qzeros"], t["scales"], None, G)
    ok, err, mx = oracle.tolerance_ok(_noalloc_abi(lib, x.to(DEV), r, K, N, G), ref, 2e-2)
    assert ok, (err, mx)


def test_noalloc_python_wrapper_and_limits():
    _, ops = _lib_and_ops()
    K, N = 9728, 2560
    t = oracle.make_awq_linear(K, N, 128, seed=1)
    r = ops.repack(t["qweight"].to(DEV), t["qzeros"].to(DEV), t["scales"].to(DEV))
    x = oracle.make_activation(8, K, seed=2).to(DEV)
    out = torch.empty((8, N), dtype=torch.float16, device=DEV)
    ops.gemm_noalloc(x, r, K, N, 128, out)
    assert torch.equal(out, ops.gemm(x, r, K, N, 128, counters=ops.make_counters(N, DEV)))
    big = torch.empty((4096, K), dtype=torch.float16, device=DEV)
    with pytest.raises(RuntimeError, match="scratch"):
        ops.gemm_noalloc(big, r, K, N, 128, torch.empty((4096, N), dtype=torch.float16, device=DEV))


_FIRST_CALL = r"""
import sys, torch
sys.path.insert(0, {root!r})
from oracle import awq_oracle as oracle
from sglite_amd import _lib, ops
captured = {captured!r}
dev = torch.device("cuda:0")
K, N, G = 28672, 512, 128          # split K on the decode kernels: counters in the scratch
lib = _lib.load()
t = oracle.make_awq_linear(K, N, G, seed=5)
r = ops.repack(t["qweight"].to(dev), t["qzeros"].to(dev), t["scales"].to(dev))  # loads the code object
xs = [oracle.make_activation(M, K, seed=M).to(dev) for M in (32, 8)]
outs = [torch.full((x.shape[0], N), float("nan"), dtype=torch.float16, device=dev) for x in xs]
torch.cuda.synchronize()


def calls(stream):
    for x, out in zip(xs, outs):   # the first noalloc calls of the process
        st = lib.awq_w4a16_gemm_noalloc(x.data_ptr(), r.w.data_ptr(), r.s.data_ptr(), r.z.data_ptr(), None,
                                        out.data_ptr(), x.shape[0], N, K, G, 0, stream)
        assert st == 0, _lib.last_error()


if captured:
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        calls(s.cuda_stream)
    torch.cuda.synchronize()
else:
    # The HIP runtime maps the library's static scratch (and loads kernel
    # code) on first use; awq_noalloc_init and one ordinary call of each
    # shape take that cost before the measured calls.
    want = [ops.gemm(x, r, K, N, G, counters=ops.make_counters(N, dev)) for x in xs]
    assert lib.awq_noalloc_init(torch.cuda.current_stream().cuda_stream) == 0, _lib.last_error()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    calls(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free0 == free1, ("the call allocated device memory", free0, free1)
want = [ops.gemm(x, r, K, N, G, counters=ops.make_counters(N, dev)) for x in xs]
for rep in range(3 if captured else 1):
    if captured:
        for out in outs:
            out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
    for out, w in zip(outs, want):
        assert torch.equal(out, w), rep
print("first-call ok")
"""


@pytest.mark.parametrize("captured", [True, False])
def test_noalloc_first_call_in_a_fresh_process(captured):
    """The first noalloc call of a process under graph capture (the counter
    clearing then becomes a node of the graph): every replay equals the
    existing entry point's output bit for bit.  Eager, after awq_noalloc_init:
    the calls leave the device's free memory unchanged and equal the existing
    entry point's output."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = _FIRST_CALL.format(root=root, captured=captured)
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "first-call ok" in res.stdout
