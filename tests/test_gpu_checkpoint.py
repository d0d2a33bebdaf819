"""End to end from an AWQ checkpoint directory on the GPU: config.json's
quantization_config -> AWQ config detection (models/config.py:28-89) -> the
streaming loader's shard / merge rules over safetensors files
(weight_loader.py:32-145) -> the plugin layers' load (device repack) ->
forward, against the CPU oracle on the checkpoint's own tensors.  The
checkpoint is synthetic (one decoder layer of per-projection AWQ tensors in
two shards); no real checkpoint is available offline.  At tp_size 2 the
column-parallel shards are the matching output columns and the row-parallel
shards' partial outputs sum to the full output."""

import json

import pytest
import torch

from oracle import awq_oracle as oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 2e-2
H, HD, NQ, NKV, I, G = 512, 64, 8, 2, 768, 128
PRE = "model.layers.0"
PROJ = {  # checkpoint projection -> (K, N)
    "self_attn.q_proj": (H, NQ * HD), "self_attn.k_proj": (H, NKV * HD), "self_attn.v_proj": (H, NKV * HD),
    "self_attn.o_proj": (NQ * HD, H), "mlp.gate_proj": (H, I), "mlp.up_proj": (H, I), "mlp.down_proj": (I, H),
}


def _write_checkpoint(path):
    from safetensors.torch import save_file

    tensors, logical = {}, {}
    for i, (name, (K, N)) in enumerate(PROJ.items()):
        t = oracle.make_awq_linear(K, N, G, seed=40 + i)
        logical[name] = t
        for k, v in t.items():
            tensors[f"{PRE}.{name}.{k}"] = v.contiguous()
    keys = sorted(tensors)
    save_file({k: tensors[k] for k in keys[: len(keys) // 2]}, str(path / "model-00001-of-00002.safetensors"))
    save_file({k: tensors[k] for k in keys[len(keys) // 2:]}, str(path / "model-00002-of-00002.safetensors"))
    cfg = {"architectures": ["Qwen2ForCausalLM"], "hidden_size": H, "num_attention_heads": NQ,
           "num_key_value_heads": NKV, "intermediate_size": I, "torch_dtype": "float16",
           "quantization_config": {"quant_method": "awq", "bits": 4, "group_size": G, "zero_point": True,
                                   "version": "gemm"}}
    (path / "config.json").write_text(json.dumps(cfg))
    return logical


def _ref(x, t, cols=None):
    qw, qz, sc = t["qweight"], t["qzeros"], t["scales"]
    if cols is not None:  # a column block: packed dim 1 of qweight/qzeros
        qw, qz, sc = qw[:, cols[0] // 8:cols[1] // 8], qz[:, cols[0] // 8:cols[1] // 8], sc[:, cols[0]:cols[1]]
    return oracle.awq_gemm(x, qw, qz, sc, None, G)


@pytest.mark.parametrize("tp", [1, 2])
def test_checkpoint_directory_to_layer_outputs(tmp_path, tp):
    from sglite_amd import checkpoint as ck
    from sglite_amd.linear import QKVParallelLinear, RowParallelLinear
    from sglite_amd.mlp import GatedMLP
    from sglite_amd.model_config import load_quantization_config
    from sglite_amd.quantization.awq_marlin import AWQMarlinConfig

    logical = _write_checkpoint(tmp_path)
    hf_config = json.loads((tmp_path / "config.json").read_text())
    cfg = load_quantization_config(str(tmp_path), hf_config)
    assert isinstance(cfg, AWQMarlinConfig)
    method = cfg.get_linear_method()
    x = oracle.make_activation(9, H, seed=5)
    torch.set_default_dtype(torch.float16)
    try:
        outs = []
        for rank in range(tp):
            qkv = QKVParallelLinear(H, HD, NQ, NKV, False, method, tp_size=tp)
            o = RowParallelLinear(NQ * HD, H, False, method, tp_size=tp)
            mlp = GatedMLP(H, I, "silu", method, tp_size=tp)
            sd = dict(ck.ingest(ck.iter_safetensors(str(tmp_path), device="cuda:0"), rank=rank, world=tp,
                                num_kv_heads=NKV))
            qkv.load_state_dict(sd, prefix=f"{PRE}.self_attn.qkv_proj", _internal=True)
            o.load_state_dict(sd, prefix=f"{PRE}.self_attn.o_proj", _internal=True)
            mlp.load_state_dict(sd, prefix=f"{PRE}.mlp", _internal=True)
            assert not sd, sorted(sd)
            xa = oracle.make_activation(9, o.local_input_size, seed=6)
            if tp == 1:
                yo, ym = o(xa.to(DEV)), mlp(x.to(DEV))
            else:  # the row-parallel all-reduce needs one process per rank: the partials are summed below
                dn = mlp.down_proj
                yo = o._linear_method.apply_weights(o._weights, xa.to(DEV), None)
                ym = dn._linear_method.apply_weights(dn._weights, mlp.gate_up_proj.forward_act(x.to(DEV), "silu"))
            outs.append((qkv(x.to(DEV)).cpu(), yo.cpu(), ym.cpu(), xa))
        # qkv: rank r holds columns [r*q/tp, ...) of q, k and v, concatenated
        for r, (yq, _, _, _) in enumerate(outs):
            parts = []
            for name, n in (("self_attn.q_proj", NQ * HD), ("self_attn.k_proj", NKV * HD),
                            ("self_attn.v_proj", NKV * HD)):
                w = n // tp
                parts.append(_ref(x, logical[name], (r * w, (r + 1) * w)))
            ok, err, mx = oracle.tolerance_ok(yq, torch.cat(parts, dim=1), TOL)
            assert ok, ("qkv", r, err, mx)
        # o: rank r multiplies its slice of the input rows; the partials sum to the full product
        t = logical["self_attn.o_proj"]
        K = NQ * HD
        full = torch.zeros(9, H)
        for r, (_, yo, _, xa) in enumerate(outs):
            k0, k1 = r * K // tp, (r + 1) * K // tp
            xs = torch.zeros(9, K, dtype=torch.float16)
            xs[:, k0:k1] = xa[:, :k1 - k0]
            full += yo.float()
            ref_part = oracle.awq_gemm(xs, t["qweight"], t["qzeros"], t["scales"], None, G)
            ok, err, mx = oracle.tolerance_ok(yo, ref_part, TOL)
            assert ok, ("o", r, err, mx)
        # mlp: gate/up column shards of I, down row shard; the rank outputs sum to the block output
        gu = torch.cat([_ref(x, logical["mlp.gate_proj"]), _ref(x, logical["mlp.up_proj"])], dim=1)
        h = oracle.silu_and_mul(gu).to(torch.float16)
        td = logical["mlp.down_proj"]
        ref = oracle.awq_gemm(h, td["qweight"], td["qzeros"], td["scales"], None, G)
        total = sum(out[2].float() for out in outs).to(torch.float16)
        ok, err, mx = oracle.tolerance_ok(total, ref, TOL)
        assert ok, ("mlp", err, mx)
    finally:
        torch.set_default_dtype(torch.float32)
