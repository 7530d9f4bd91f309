"""GPU parity of the calibration codebook refresh (sva_amd.refresh;
experiments/export_refreshed_sva_artifact.py:73-154,
experiments/sva_codebook_refresh_benchmark.py:136-153,
experiments/sva_rotation_diagnostic.py:86-116).

sva_key_weights is bit-exact with the oracle (itself pinned to index_add_);
the top-k targets and query rows equal the oracle's; the whole driver on a
random-init Llama is checked against a torch-CPU restatement of the
reference's expressions for the catalog and the weights, and its codebooks
against the oracle's weighted k-means from the same initial centroids.  The
exported bundle loads back with the refreshed codebooks in place."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb, repeat_kv

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("boost", [4.0, 0.1, 16.0])
def test_key_weights_bit_exact(device, boost):
    from sva_amd import refresh

    rng = np.random.default_rng(5)
    H, Q, K, N = 9, 128, 16, 3000
    top_idx = rng.integers(-3, N + 3, (H, Q, K))
    top_idx[4, :, 1] = 7  # a key hit by every query
    top_valid = rng.random((H, Q, K)) < 0.9
    top_valid[4, :, 1] = True
    top_valid[6] = False
    got = refresh.topk_key_weights(torch.from_numpy(top_idx).to(device), torch.from_numpy(top_valid).to(device), N,
                                   boost).cpu().numpy()
    want = oracle.topk_key_weights(top_idx, top_valid, N, boost)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(got[6] == 1.0) and got[4, 7] > 1.0 + 0.99 * Q * boost


def test_topk_targets_and_rows(device):
    from sva_amd import refresh

    rng = np.random.default_rng(8)
    N = 700
    rows = refresh.calibration_query_positions(N, 50, 16, device)
    np.testing.assert_array_equal(rows.cpu().numpy(), oracle.query_positions(N, 50, 16))
    scores = rng.standard_normal((3, rows.numel(), N)).astype(np.float32)
    idx, valid = refresh.topk_targets(torch.from_numpy(scores).to(device), rows, 16)
    want_idx, want_valid = oracle.topk_targets(scores, rows.cpu().numpy(), 16)
    np.testing.assert_array_equal(valid.cpu().numpy(), want_valid)
    got_idx = idx.cpu().numpy()
    for h in range(3):
        for r in range(rows.numel()):
            v = want_valid[h, r]
            assert set(got_idx[h, r][v]) == set(want_idx[h, r][v])


def _tiny_llama(seed=0, hidden=256, heads=4, kv_heads=2, layers=2):
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=96, hidden_size=hidden, intermediate_size=2 * hidden, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, max_position_embeddings=1024,
                      rope_theta=10000.0, attn_implementation="eager")
    return LlamaForCausalLM(cfg).eval()


def _bundle(heads, head_dim, layers, rank=64, S=2, C=16):
    from sva_amd import SVAArtifactBundle, SVALayerArtifacts

    g = torch.Generator().manual_seed(3)
    arts = {i: SVALayerArtifacts(q_proj=torch.randn(heads, head_dim, rank, generator=g) / 8,
                                 k_proj=torch.randn(heads, head_dim, rank, generator=g) / 8,
                                 logit_scale=torch.zeros(heads),
                                 coarse_codebooks=torch.randn(heads, S, C, rank // S, generator=g),
                                 train_loss=0.0, hard_loss=0.0) for i in range(layers)}
    manifest = {"schema_version": 1, "artifact_type": "summon_verify_attention", "rank_dim": rank,
                "coarse_subspaces": S, "coarse_codewords": C, "default_shortlist": 64, "default_budget": 16,
                "layer_count": layers, "layers": list(range(layers)), "profile_name": "tiny-base"}
    return SVAArtifactBundle(manifest=manifest, layers=arts)


def _cpu_catalog(model, ids, layer_idx, bundle, samples, min_pos, topk, boost):
    # the reference's expressions (layer_qkv_from_hidden, the export driver's
    # k_low / scores lines) on the CPU, then the oracle's targets and weights
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=False, output_hidden_states=True)
        layer = model.model.layers[layer_idx]
        hidden = layer.input_layernorm(out.hidden_states[layer_idx])
        shape = (hidden.shape[0], hidden.shape[1], -1, layer.self_attn.head_dim)
        query = layer.self_attn.q_proj(hidden).view(shape).transpose(1, 2)
        key = layer.self_attn.k_proj(hidden).view(shape).transpose(1, 2)
        pos = torch.arange(ids.shape[1]).unsqueeze(0)
        cos, sin = model.model.rotary_emb(hidden, pos)
        query, key = apply_rotary_pos_emb(query, key, cos, sin)
        key = repeat_kv(key, layer.self_attn.num_key_value_groups)
        query, key = query[0].float(), key[0].float()
        k_low = torch.einsum("hkd,hdr->hkr", key, bundle.layers[layer_idx].k_proj.float())
        rows = oracle.query_positions(ids.shape[1], samples, min_pos)
        scores = torch.einsum("hqd,hkd->hqk", query[:, torch.from_numpy(rows)], key) * layer.self_attn.scaling
    idx, valid = oracle.topk_targets(scores.numpy(), rows, topk)
    return k_low.numpy(), oracle.topk_key_weights(idx, valid, ids.shape[1], boost)


def test_fit_refreshed_codebooks_matches_restatement(device, tmp_path, monkeypatch):
    from sva_amd import codebooks, load_sva_artifact_bundle, refresh

    heads, head_dim, T = 4, 64, 320
    model_cpu = _tiny_llama()
    model = copy.deepcopy(model_cpu).to(device)
    bundle = _bundle(heads, head_dim, 2)
    ids = torch.randint(0, 96, (1, T), generator=torch.Generator().manual_seed(4))
    captured = []
    real_fit = refresh.fit_weighted_product_codebooks

    def spy(k_low, weights, subspaces, codewords, iterations, seed, chunk_size=8192, initial=None):
        captured.append((k_low.clone(), weights.clone(), seed))
        return real_fit(k_low, weights, subspaces, codewords, iterations, seed, chunk_size, initial)

    monkeypatch.setattr(refresh, "fit_weighted_product_codebooks", spy)
    reports = []
    got = refresh.fit_refreshed_codebooks(
        model=model, runtime_bundle=bundle, calibration_batch={"input_ids": ids.to(device)}, layers=[0, 1],
        refresh_method="attention_weighted_strong", attention_topk=8, calibration_query_samples=40, min_query_pos=16,
        attention_boost=1.0, kmeans_iters=3, assign_chunk_size=8192, seed=29, device=device, report=reports.append)
    assert sorted(got) == [0, 1] and len(captured) == 2 and len(reports) == 2
    for layer_idx in (0, 1):
        k_low_gpu, w_gpu, seed = captured[layer_idx]
        assert seed == 29 + layer_idx * 9973
        k_low_cpu, w_cpu = _cpu_catalog(model_cpu, ids, layer_idx, bundle, 40, 16, 8, 4.0)
        np.testing.assert_allclose(k_low_gpu.cpu().numpy(), k_low_cpu, rtol=1e-4, atol=1e-4)
        np.testing.assert_array_equal(w_gpu.cpu().numpy(), w_cpu)  # boost 4x for the strong method
        # the fit from the driver's own initial draw equals the oracle's weighted k-means
        x, w = k_low_gpu, w_gpu
        S, C = 2, 16
        sub = x.shape[2] // S
        init = torch.stack([torch.stack([codebooks._initial(x[h, :, s * sub:(s + 1) * sub], w[h].clamp_min(1e-6), seed,
                                                            h, s, C) for s in range(S)]) for h in range(heads)])
        want = oracle.kmeans_fit(x.cpu().numpy(), S, 3, init.cpu().numpy(), w.cpu().numpy())
        cb = got[layer_idx].numpy()
        np.testing.assert_allclose(cb, want, rtol=1e-5, atol=1e-5)
        assert reports[layer_idx]["attention_boost"] == 4.0
        assert 0.0 < reports[layer_idx]["code_entropy"] <= 1.0
    refresh.export_refreshed_bundle(bundle, got, tmp_path / "refreshed",
                                    settings={"profile_name": "tiny-refresh", "codebook_refresh_method":
                                              "calibration_attention_weighted_strong"})
    back = load_sva_artifact_bundle(tmp_path / "refreshed")
    assert back.manifest["profile_name"] == "tiny-refresh" and back.manifest["base_profile_name"] == "tiny-base"
    for i in (0, 1):
        assert back.layers[i].coarse_codebooks.dtype == torch.bfloat16
        assert torch.equal(back.layers[i].coarse_codebooks, got[i].to(torch.bfloat16))
        assert torch.equal(back.layers[i].q_proj, bundle.layers[i].q_proj)
