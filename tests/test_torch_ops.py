"""The C ABI's registration as torch custom ops (namespace torch.ops.sglite_awq),
on the CPU: every op is registered with a schema, and FakeTensor shape/dtype
propagation runs through the fake implementations without a GPU (the
reference's dispatch goes through its torch ops sgl_kernel.gptq_marlin_gemm and
awq_marlin_repack, marlin_utils.py:388-410, awq_marlin.py:300-305)."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from sglite_amd import ops


def test_every_op_is_registered_with_a_schema():
    for name in ops.REGISTERED_OPS:
        op = getattr(torch.ops.sglite_awq, name)
        assert str(op.default._schema).startswith(f"sglite_awq::{name}(")
    gemm = str(torch.ops.sglite_awq.awq_w4a16_gemm.default._schema)
    assert "Tensor(a5!)? counters" in gemm and gemm.endswith("-> Tensor")
    assert "Tensor(a6!) out" in str(torch.ops.sglite_awq.awq_w4a16_gemm_out.default._schema)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fake_shape_propagation(dtype):
    K, N, G, M = 4096, 6144, 128, 37
    with FakeTensorMode():
        qw = torch.empty((K, N // 8), dtype=torch.int32, device="cuda")
        qz = torch.empty((K // G, N // 8), dtype=torch.int32, device="cuda")
        sc = torch.empty((K // G, N), dtype=dtype, device="cuda")
        w, s, z = torch.ops.sglite_awq.awq_repack_cdna4(qw, qz, sc)
        assert w.shape == ((N // 16) * (K // 128) * 256,) and w.dtype == torch.int32
        assert s.shape == (N // 16, K // G, 16) and s.dtype == dtype
        assert z.shape == (N // 16, K // G) and z.dtype == torch.int64
        x = torch.empty((M, K), dtype=dtype, device="cuda")
        cnt = torch.empty(N // 16, dtype=torch.int32, device="cuda")
        y = torch.ops.sglite_awq.awq_w4a16_gemm(x, w, s, z, None, cnt, K, N, G)
        assert y.shape == (M, N) and y.dtype == dtype and y.device.type == "cuda"
        h = torch.ops.sglite_awq.awq_w4a16_gemm_act(x, w, s, z, None, cnt, K, N, G, "silu")
        assert h.shape == (M, N // 2) and h.dtype == dtype
        W = torch.ops.sglite_awq.awq_dequant_repacked(w, s, z, K, N, G)
        assert W.shape == (K, N) and W.dtype == dtype
        q2, z2, s2 = torch.ops.sglite_awq.awq_unrepack_cdna4(w, s, z, K, N, G)
        assert q2.shape == qw.shape and z2.shape == qz.shape and s2.shape == sc.shape


def test_fake_moe_ops():
    T, E, k, H, I = 64, 16, 4, 256, 128
    with FakeTensorMode():
        logits = torch.empty((T, E), dtype=torch.float32, device="cuda")
        tw, ids = torch.ops.sglite_awq.awq_moe_topk_softmax(logits, k, True)
        assert tw.shape == (T, k) and tw.dtype == torch.float32 and ids.dtype == torch.int32
        sorted_ids, expert_ids, npp, offs = torch.ops.sglite_awq.awq_moe_align_block_size(ids, 16, E)
        assert sorted_ids.shape == (T * k + E * 15,) and offs.shape == (E + 1,) and npp.shape == (1,)
        qw = torch.empty((E, H, 2 * I // 8), dtype=torch.int32, device="cuda")
        qz = torch.empty((E, H // 128, 2 * I // 8), dtype=torch.int32, device="cuda")
        sc = torch.empty((E, H // 128, 2 * I), dtype=torch.float16, device="cuda")
        w, s, z = torch.ops.sglite_awq.awq_repack_experts(qw, qz, sc)
        ws, ss, zs = ops.expert_strides(H, 2 * I, 128)
        assert w.shape == (E, ws // 4) and s.shape == (E, ss // 2) and z.shape == (E, zs // 8)
