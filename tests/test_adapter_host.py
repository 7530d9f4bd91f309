"""Host side of the residual output adapter (experiments/sva_late4_logit_distill.py:37-51,
:162-239): wrapping of socket layers, the 110k-parameter shape of the config-3
adapter, state collection and the bundle round trip (adapter_config.json +
adapter_weights.pt, read back with weights_only=True)."""

from __future__ import annotations

import json

import pytest
import torch
from torch import nn

from sva_amd import adapter


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.o_proj = nn.Linear(4, 4)


def _model(layers=4, hidden=576):
    layer_list = nn.ModuleList([nn.Module() for _ in range(layers)])
    for layer in layer_list:
        layer.self_attn = _Attn()
    model = nn.Module()
    model.model = nn.Module()
    model.model.layers = layer_list
    model.config = type("Cfg", (), {"hidden_size": hidden})()
    return model


def test_wrap_socket_layers_and_parameter_count():
    # the late-layer socket: layers 26-29 of 30, hidden 576, rank 16
    model = _model(layers=30)
    socket = [26, 27, 28, 29]
    adapter.wrap_socket_layers_with_adapters(model, socket, rank=16, scale=1.0)
    total = 0
    for i in socket:
        a = model.model.layers[i].self_attn
        assert isinstance(a, adapter.SVAResidualOutputAdapter)
        assert isinstance(a.sva_attn, _Attn)
        assert a.down.weight.shape == (16, 1152) and a.up.weight.shape == (576, 16)
        assert a.down.weight.dtype == torch.float32
        assert torch.count_nonzero(a.up.weight) == 0  # zero init: the adapter starts as the identity
        total += sum(p.numel() for p in (a.down.weight, a.up.weight))
    assert total == 110_592  # the "110k-param residual adapter"
    assert not isinstance(model.model.layers[0].self_attn, adapter.SVAResidualOutputAdapter)


def test_bundle_round_trip(tmp_path):
    model = _model()
    adapter.wrap_socket_layers_with_adapters(model, [1, 3], rank=16, scale=0.5)
    with torch.no_grad():
        for i in (1, 3):
            model.model.layers[i].self_attn.up.weight.normal_()
    adapter.save_adapter_bundle(tmp_path, model, [1, 3], {"adapter_rank": 16, "adapter_scale": 0.5})
    meta = json.loads((tmp_path / "adapter_config.json").read_text())
    assert meta["format"] == "sva_residual_output_adapter_v1" and meta["socket_layers"] == [1, 3]
    manifest, state = adapter.load_adapter_bundle(tmp_path)
    assert manifest["adapter_rank"] == 16
    assert sorted(state) == ["layers.1.down.weight", "layers.1.up.weight", "layers.3.down.weight",
                             "layers.3.up.weight"]
    other = _model()
    adapter.wrap_socket_layers_with_adapters(other, [1, 3], rank=16, scale=0.5)
    adapter.load_adapter_weights(other, [1, 3], state)
    for i in (1, 3):
        a, b = model.model.layers[i].self_attn, other.model.layers[i].self_attn
        assert torch.equal(a.down.weight, b.down.weight) and torch.equal(a.up.weight, b.up.weight)


def test_unwrapped_layer_is_rejected():
    model = _model()
    with pytest.raises(TypeError, match="not wrapped"):
        adapter.collect_adapter_state(model, [0])


def test_bundle_validation(tmp_path):
    model = _model()
    made = adapter.wrap_socket_layers_with_adapters(model, [2], rank=8, scale=1.0)
    assert made == [model.model.layers[2].self_attn]
    adapter.save_adapter_bundle(tmp_path, model, [2], {})
    _, state = adapter.load_adapter_bundle(tmp_path)
    other = _model()
    adapter.wrap_socket_layers_with_adapters(other, [2], rank=4, scale=1.0)
    with pytest.raises(ValueError, match="down.weight"):
        adapter.load_adapter_weights(other, [2], state)  # rank 8 stored, rank 4 expected
    with pytest.raises(KeyError, match="layers.2.up.weight"):
        adapter.load_adapter_weights(model, [2], {"layers.2.down.weight": state["layers.2.down.weight"]})
    cfg = json.loads((tmp_path / "adapter_config.json").read_text())
    cfg["format"] = "something_else"
    (tmp_path / "adapter_config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="format"):
        adapter.load_adapter_bundle(tmp_path)
    # a bare state dict (no "state_dict" wrapper) is accepted too
    cfg["format"] = adapter.ADAPTER_FORMAT
    (tmp_path / "adapter_config.json").write_text(json.dumps(cfg))
    torch.save(state, tmp_path / "adapter_weights.pt")
    assert sorted(adapter.load_adapter_bundle(tmp_path)[1]) == sorted(state)


def test_fresh_adapter_draws_like_the_experiment():
    """down / up are bias-free fp32 Linear layers made on the CPU: a fresh adapter's down weight is the
    default generator's N(0, 0.02^2) draw after Linear's own init (so the CPU generator advances as in the
    experiment), up is zero, and both layers are callable."""
    attn = _Attn()
    torch.manual_seed(123)
    a = adapter.SVAResidualOutputAdapter(attn, hidden_size=8, rank=3, scale=1.0)
    after = torch.rand(1)
    torch.manual_seed(123)
    down = nn.Linear(16, 3, bias=False)
    up = nn.Linear(3, 8, bias=False)
    expect = torch.empty(3, 16).normal_(0.0, 0.02)
    assert torch.equal(torch.rand(1), after), "the CPU generator advanced differently"
    assert torch.equal(a.down.weight, expect) and down.weight.shape == a.down.weight.shape
    assert torch.count_nonzero(a.up.weight) == 0 and up.weight.shape == a.up.weight.shape
    assert isinstance(a.down, nn.Linear) and a.down.bias is None and a.up.bias is None
    x = torch.randn(2, 16)
    assert torch.equal(a.up(a.down(x)), torch.zeros(2, 8))
