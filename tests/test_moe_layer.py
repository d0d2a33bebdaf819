"""CPU tests of the AWQ MoE layer's state-dict contract: the keys, shapes and
dtypes it expects are exactly what checkpoint ingestion yields for a per-expert
AWQ checkpoint (gate/up merged on packed columns, experts stacked on dim 0),
at tp_size 1 and 2; mismatches raise as the reference's BaseModule does; the
post-load repack refuses host tensors (no CPU path)."""

import pytest
import torch

from oracle import awq_oracle as oracle
from sglite_amd import checkpoint as ck
from sglite_amd.moe import AWQMoELayer

PRE = "model.layers.3.mlp.experts"


def _awq(K, N, G, seed):
    w = oracle.make_awq_linear(K, N, G, seed=seed)
    return {k: torch.as_tensor(v) for k, v in w.items()}


def _checkpoint(E, H, I, G):
    stream = []
    for e in range(E):
        for n, (K, N) in (("gate_proj", (H, I)), ("up_proj", (H, I)), ("down_proj", (I, H))):
            for suffix, t in _awq(K, N, G, seed=100 * e + len(n)).items():
                stream.append((f"{PRE}.{e}.{n}.{suffix}", t))
    return stream


@pytest.mark.parametrize("tp", [1, 2])
def test_layer_keys_shapes_match_ingested_checkpoint(tp):
    E, H, I, G = 4, 256, 256, 64
    for rank in range(tp):
        sd = dict(ck.ingest(_checkpoint(E, H, I, G), rank=rank, world=tp, num_experts=E))
        layer = AWQMoELayer(E, 2, H, I, group_size=G, tp_size=tp)
        want = layer.state_dict(prefix=PRE)
        assert set(want) == set(sd)
        for k, v in want.items():
            assert v.shape == sd[k].shape and v.dtype == sd[k].dtype, k
        assert want[f"{PRE}.gate_up_proj.qweight"].shape == (E, H, 2 * (I // tp) // 8)
        assert want[f"{PRE}.down_proj.scales"].shape == (E, (I // tp) // G, H)


def test_layer_rejects_bad_tensors_and_host_memory():
    E, H, I, G = 4, 256, 128, 64
    layer = AWQMoELayer(E, 2, H, I, group_size=G)
    sd = dict(ck.ingest(_checkpoint(E, H, I, G), num_experts=E))
    bad = dict(sd)
    bad[f"{PRE}.down_proj.scales"] = bad[f"{PRE}.down_proj.scales"].to(torch.bfloat16)
    with pytest.raises(AssertionError):
        layer.load_state_dict(bad, prefix=PRE)
    bad = dict(sd)
    bad[f"{PRE}.gate_up_proj.qweight"] = bad[f"{PRE}.gate_up_proj.qweight"][:, :, :-1]
    with pytest.raises(AssertionError):
        layer.load_state_dict(bad, prefix=PRE)
    missing = {k: v for k, v in sd.items() if not k.endswith("down_proj.qzeros")}
    with pytest.raises(KeyError):
        layer.load_state_dict(missing, prefix=PRE)
    with pytest.raises(ValueError, match="device tensors"):
        layer.load_state_dict(dict(sd), prefix=PRE)
    with pytest.raises(RuntimeError, match="not loaded"):
        layer.forward(torch.zeros(2, H, dtype=torch.float16), torch.zeros(2, E))


def test_layer_argument_checks():
    with pytest.raises(ValueError):
        AWQMoELayer(8, 2, 256, 200, group_size=64, tp_size=2)  # 100 % 64 != 0
    with pytest.raises(ValueError):
        AWQMoELayer(8, 2, 256, 96, group_size=32, tp_size=4)  # 24 columns per rank: not a 16-column multiple
    with pytest.raises(ValueError):
        AWQMoELayer(8, 9, 256, 128)
    with pytest.raises(ValueError):
        AWQMoELayer(8, 2, 256, 128, activation="relu")
    layer = AWQMoELayer(8, 2, 256, 128, group_size=-1)
    assert layer.gate_up_proj.group_size == 256 and layer.down_proj.group_size == 128
