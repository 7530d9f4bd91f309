"""Host-side API without a GPU: artifact bundles (schema 1), statistics,
patch / unpatch / validation of the patcher, and the adapter's refusal to
run attention off the GPU (there is no CPU path)."""

from __future__ import annotations

import json
import math

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from sva_amd import (SVAArtifactBundle, SVALayerArtifacts, SVALlamaAttention, SVALlamaPatcher, SVAStats,
                     load_sva_artifact_bundle, patch_llama_attention, save_sva_artifact_bundle)


def tiny_model():
    torch.manual_seed(0)
    config = LlamaConfig(vocab_size=64, hidden_size=16, intermediate_size=32, num_hidden_layers=2,
                         num_attention_heads=2, num_key_value_heads=2, max_position_embeddings=64,
                         tie_word_embeddings=False)
    return LlamaForCausalLM(config).eval()


def tiny_bundle(layers=2, rank=4, subspaces=2, codewords=8, model_id=None):
    g = torch.Generator().manual_seed(11)
    arts = {i: SVALayerArtifacts(q_proj=torch.randn(2, 8, rank, generator=g), k_proj=torch.randn(2, 8, rank, generator=g),
                                 logit_scale=torch.zeros(2),
                                 coarse_codebooks=torch.randn(2, subspaces, codewords, rank // subspaces, generator=g),
                                 train_loss=0.5, hard_loss=0.25)
            for i in range(layers)}
    manifest = {"schema_version": 1, "rank_dim": rank, "coarse_subspaces": subspaces, "coarse_codewords": codewords,
                "default_shortlist": 4, "default_budget": 2, "layer_count": layers, "layers": list(range(layers))}
    if model_id:
        manifest["model_id"] = model_id
    return SVAArtifactBundle(manifest, arts)


def test_bundle_roundtrip(tmp_path):
    b = tiny_bundle()
    save_sva_artifact_bundle(b, tmp_path)
    manifest = json.loads((tmp_path / "sva_config.json").read_text())
    assert manifest["schema_version"] == 1 and manifest["layers"] == [0, 1]
    loaded = load_sva_artifact_bundle(tmp_path)
    assert loaded.rank_dim == 4 and loaded.coarse_subspaces == 2 and loaded.coarse_codewords == 8
    assert loaded.default_shortlist == 4 and loaded.default_budget == 2 and loaded.layer_count == 2
    for i in (0, 1):
        for name in ("q_proj", "k_proj", "logit_scale", "coarse_codebooks"):
            assert torch.equal(getattr(loaded.layers[i], name), getattr(b.layers[i], name))
        assert loaded.layers[i].train_loss == 0.5 and loaded.layers[i].route_source == "qk"
    moved = loaded.to("cpu", torch.float64)
    assert moved.layers[0].q_proj.dtype == torch.float64 and moved.layers[0].logit_scale.dtype == torch.float32


def test_bundle_validation_messages(tmp_path):
    save_sva_artifact_bundle(tiny_bundle(), tmp_path)
    manifest = json.loads((tmp_path / "sva_config.json").read_text())
    manifest["schema_version"] = 2
    (tmp_path / "sva_config.json").write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match="Unsupported SVA artifact schema"):
        load_sva_artifact_bundle(tmp_path)
    bad = tiny_bundle()
    bad.manifest["coarse_subspaces"] = 3
    with pytest.raises(ValueError, match="must be divisible by coarse_subspaces"):
        save_sva_artifact_bundle(bad, tmp_path / "x")
    bad = tiny_bundle()
    bad.manifest["coarse_codewords"] = 16
    with pytest.raises(ValueError, match="coarse_codebooks shape mismatch"):
        save_sva_artifact_bundle(bad, tmp_path / "y")
    bad = tiny_bundle()
    bad.layers[0] = SVALayerArtifacts(**{**bad.layers[0].__dict__, "route_source": "qv"})
    with pytest.raises(ValueError, match="route_source"):
        save_sva_artifact_bundle(bad, tmp_path / "z")


def test_stats_interface():
    s = SVAStats()
    s.add(0, {"queries": 2.0, "summoned": 10.0, "verified": 4.0})
    s.add_device(1, {"queries": 2.0, "summoned": torch.tensor([3, 5]), "verified": torch.tensor([1, 1])})
    assert s.totals["queries"] == 4.0 and s.totals["summoned"] == 18.0
    assert s.by_layer[1]["summoned"] == 8.0
    summary = s.summary()
    assert summary["queries"] == 4.0 and summary["avg_summoned"] == 4.5 and summary["avg_verified"] == 1.5
    assert math.isnan(summary["avg_static_total_ms"])
    s.reset()
    assert s.summary()["queries"] == 0.0


def test_patch_unpatch_and_layer_selection():
    model = tiny_model()
    originals = [layer.self_attn for layer in model.model.layers]
    handle = patch_llama_attention(model, tiny_bundle(), layers=[1])
    assert model.model.layers[0].self_attn is originals[0]
    attn = model.model.layers[1].self_attn
    assert isinstance(attn, SVALlamaAttention)
    assert attn.serving.coarse_shortlist == 4 and attn.serving.budget == 2
    assert torch.equal(attn.sva_scale, torch.ones(2))  # exp(0) clamped to [0.01, 100]
    assert handle.patch() is handle  # idempotent
    handle.reset_catalogs()
    handle.unpatch()
    assert [layer.self_attn for layer in model.model.layers] == originals
    with SVALlamaPatcher(model, tiny_bundle(), shortlist=8, budget=3) as h:
        assert h.serving.coarse_shortlist == 8 and h.serving.budget == 3
        assert all(isinstance(layer.self_attn, SVALlamaAttention) for layer in model.model.layers)
    assert [layer.self_attn for layer in model.model.layers] == originals


def test_patch_rejects_mismatches():
    model = tiny_model()
    with pytest.raises(ValueError, match="Artifact has 3 layers but model has 2"):
        patch_llama_attention(model, tiny_bundle(layers=3))
    with pytest.raises(ValueError, match="model_id"):
        model.config._name_or_path = "some/model"
        patch_llama_attention(model, tiny_bundle(model_id="other/model"))
    model.config._name_or_path = ""
    with pytest.raises(ValueError, match="outside model layer range"):
        patch_llama_attention(model, tiny_bundle(), layers=[5])
    bad = tiny_bundle()
    bad.layers[0] = SVALayerArtifacts(**{**bad.layers[0].__dict__, "q_proj": torch.zeros(3, 8, 4)})
    with pytest.raises(ValueError, match="q_proj shape"):
        patch_llama_attention(model, bad)
    with pytest.raises(ValueError, match="Unknown SVA summon_mode"):
        patch_llama_attention(model, tiny_bundle(), summon_mode="dense")


def test_attention_off_gpu_fails_loudly():
    model = tiny_model()
    patch_llama_attention(model, tiny_bundle())
    with pytest.raises(Exception, match="(?i)rocm|gpu|device|cpu"):
        with torch.no_grad():
            model(input_ids=torch.tensor([[1, 2, 3]]), use_cache=False)
    model.train()
    with pytest.raises(RuntimeError, match="inference-only"):
        model(input_ids=torch.tensor([[1, 2, 3]]), use_cache=False)
