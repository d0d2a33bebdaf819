"""CPU tests of AWQ checkpoint ingestion (shard, merge, stack, dtype) against
the oracle's dequantisation: a rule is right when the dequantised result of the
packed tensors equals the same operation applied to the logical weights."""

import pytest
import torch

from oracle import awq_oracle as oracle
from sglite_amd import checkpoint as ck


def _logical(K, N, G, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(0, 16, (K, N), generator=g, dtype=torch.int32)
    z = torch.randint(0, 16, (K // G, N), generator=g, dtype=torch.int32)
    s = (torch.rand((K // G, N), generator=g) * 0.018 + 0.002).to(torch.float16)
    return q, z, s


def _pack(q, z, s):
    return {"qweight": torch.from_numpy(oracle.pack_awq(q)), "qzeros": torch.from_numpy(oracle.pack_awq(z)),
            "scales": s}


def _deq(t, G):
    return oracle.dequantize(t["qweight"], t["qzeros"], t["scales"], G)


def test_qkv_and_gate_up_merge_on_packed_columns():
    K, G = 256, 64
    parts = {"q": 64, "k": 32, "v": 32}
    logical = {n: _logical(K, N, G, seed=i) for i, (n, N) in enumerate(parts.items())}
    stream = []
    for n in ("v", "q", "k"):  # arrival order does not matter; slot order does
        for suffix, t in _pack(*logical[n]).items():
            stream.append((f"model.layers.0.self_attn.{n}_proj.{suffix}", t))
    out = dict(ck.ingest(stream))
    fused = {k.rsplit(".", 1)[1]: v for k, v in out.items() if ".qkv_proj." in k}
    assert set(fused) == {"qweight", "qzeros", "scales"}
    assert fused["qweight"].shape == (K, 128 // 8) and fused["scales"].shape == (K // G, 128)
    ref = torch.cat([_deq(_pack(*logical[n]), G) for n in ("q", "k", "v")], dim=1)
    assert torch.equal(_deq(fused, G), ref)


def test_incomplete_merge_is_an_error():
    t = _pack(*_logical(128, 16, 128, 0))
    with pytest.raises(ValueError, match="incomplete merge"):
        list(ck.ingest([("layers.0.mlp.gate_proj.qweight", t["qweight"])]))


@pytest.mark.parametrize("world", [2, 4])
def test_column_parallel_awq_shard_is_a_column_block(world):
    K, N, G = 256, 128, 64
    t = _pack(*_logical(K, N, G, seed=5))
    full = _deq(t, G)
    for r in range(world):
        sh = {k: ck.shard_tensor(f"layers.0.mlp.up_proj.{k}", v, r, world) for k, v in t.items()}
        blk = N // world
        assert torch.equal(_deq(sh, G), full[:, r * blk:(r + 1) * blk])


@pytest.mark.parametrize("world", [2, 4])
def test_row_parallel_awq_shard_is_a_row_block(world):
    K, N, G = 512, 64, 64
    t = _pack(*_logical(K, N, G, seed=6))
    full = _deq(t, G)
    for r in range(world):
        sh = {k: ck.shard_tensor(f"layers.0.self_attn.o_proj.{k}", v, r, world) for k, v in t.items()}
        blk = K // world
        assert torch.equal(_deq(sh, G), full[r * blk:(r + 1) * blk])


def test_dense_shard_rules_and_kv_head_replication():
    w = torch.arange(8 * 6, dtype=torch.float32).view(8, 6)
    assert torch.equal(ck.shard_tensor("l.self_attn.q_proj.weight", w, 1, 2), w[4:])
    assert torch.equal(ck.shard_tensor("l.self_attn.o_proj.weight", w, 1, 2), w[:, 3:])
    # 2 kv heads of 4 rows over 4 ranks: ranks 0,1 hold head 0; ranks 2,3 head 1
    assert torch.equal(ck.shard_tensor("l.self_attn.k_proj.weight", w, 1, 4, num_kv_heads=2), w[:4])
    assert torch.equal(ck.shard_tensor("l.self_attn.k_proj.weight", w, 2, 4, num_kv_heads=2), w[4:])
    emb = torch.arange(10 * 2, dtype=torch.float32).view(10, 2)
    assert torch.equal(ck.shard_tensor("model.embed_tokens.weight", emb, 2, 3), emb[8:10])
    norm = torch.ones(6)
    assert ck.shard_tensor("model.norm.weight", norm, 1, 2) is norm


def test_expert_stacking_with_gate_up_merge_and_dtype():
    E, H, I, G = 3, 128, 64, 64
    stream, ref_gu, ref_down = [], [], []

    def cast(lg):  # the engine casts floating tensors (the scales) to its dtype
        q, z, s = lg
        return q, z, s.to(torch.bfloat16).to(torch.float16)  # bf16 values are exact in fp16 here

    for e in range(E):
        gate, up = _logical(H, I, G, seed=10 + e), _logical(H, I, G, seed=20 + e)
        down = _logical(I, H, G, seed=30 + e)
        for n, lg in (("gate_proj", gate), ("up_proj", up), ("down_proj", down)):
            for suffix, t in _pack(*lg).items():
                stream.append((f"model.layers.0.mlp.experts.{e}.{n}.{suffix}", t))
        ref_gu.append(torch.cat([_deq(_pack(*cast(gate)), G), _deq(_pack(*cast(up)), G)], dim=1))
        ref_down.append(_deq(_pack(*cast(down)), G))
    out = dict(ck.ingest(stream, num_experts=E, dtype=torch.bfloat16))
    pre = "model.layers.0.mlp.experts."
    gu = {k.rsplit(".", 1)[1]: v for k, v in out.items() if k.startswith(pre + "gate_up_proj.")}
    dn = {k.rsplit(".", 1)[1]: v for k, v in out.items() if k.startswith(pre + "down_proj.")}
    assert set(out) == {pre + n + "." + s for n in ("gate_up_proj", "down_proj") for s in ("qweight", "qzeros", "scales")}
    assert gu["qweight"].shape == (E, H, 2 * I // 8) and gu["qweight"].dtype == torch.int32
    assert gu["qzeros"].shape == (E, H // G, 2 * I // 8) and dn["scales"].shape == (E, I // G, H)
    assert gu["scales"].dtype == torch.bfloat16 and dn["scales"].dtype == torch.bfloat16
    for e in range(E):
        t = {k: (v[e].to(torch.float16) if k == "scales" else v[e]) for k, v in gu.items()}
        assert torch.equal(_deq(t, G), ref_gu[e])
        t = {k: (v[e].to(torch.float16) if k == "scales" else v[e]) for k, v in dn.items()}
        assert torch.equal(_deq(t, G), ref_down[e])


def test_incomplete_expert_stack_is_an_error():
    t = _pack(*_logical(128, 16, 128, 0))
    with pytest.raises(ValueError, match="incomplete expert"):
        list(ck.ingest([("m.experts.0.down_proj.qweight", t["qweight"])], num_experts=2))


def test_prefix_stripping_and_skips():
    x = torch.zeros(2)
    out = dict(ck.ingest([("language_model.model.norm.weight", x), ("vision_tower.a", x),
                          ("multi_modal_projector.b", x)]))
    assert list(out) == ["model.norm.weight"]


def test_safetensors_directory_round_trip(tmp_path):
    from safetensors.torch import save_file
    t = _pack(*_logical(128, 32, 64, 3))
    save_file({f"layers.0.self_attn.o_proj.{k}": v.contiguous() for k, v in t.items()},
              str(tmp_path / "model-00001.safetensors"))
    got = dict(ck.iter_safetensors(str(tmp_path)))
    for k, v in t.items():
        assert torch.equal(got[f"layers.0.self_attn.o_proj.{k}"], v)
