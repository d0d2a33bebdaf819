"""CPU test of the gated MLP block's structure with the unquantized method:
gate_up_proj -> act(gate) * up -> down_proj, state-dict keys, and the default
(unfused) apply_weights_act of a linear method."""

import pytest
import torch

from sglite_amd.mlp import GatedMLP


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_unquantized_gated_mlp_matches_manual_block(act):
    torch.manual_seed(0)
    H, I, M = 64, 96, 5
    mlp = GatedMLP(H, I, act)
    wgu = torch.randn(2 * I, H) / 8
    wdn = torch.randn(H, I) / 8
    sd = {"gate_up_proj.weight": wgu.clone(), "down_proj.weight": wdn.clone()}
    assert sorted(mlp.state_dict_keys()) == sorted(sd)
    mlp.load_state_dict(sd)
    x = torch.randn(M, H)
    y = mlp(x)
    gu = x @ wgu.t()
    f = torch.nn.functional.silu if act == "silu" else torch.nn.functional.gelu
    ref = (f(gu[:, :I]) * gu[:, I:]) @ wdn.t()
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)


def test_gated_mlp_rejects_unknown_activation_and_extra_keys():
    with pytest.raises(ValueError):
        GatedMLP(64, 96, "relu")
    mlp = GatedMLP(8, 16)
    sd = {"gate_up_proj.weight": torch.zeros(32, 8), "down_proj.weight": torch.zeros(8, 16), "extra": torch.zeros(1)}
    with pytest.raises(RuntimeError, match="Unexpected"):
        mlp.load_state_dict(sd)
