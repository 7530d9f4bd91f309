"""The drop-in adapter on the GPU: the reference's adapter tests
(tests/test_sva_llama_adapter.py of the reference) run against `sva` with
the model on cuda:0, plus end-to-end equivalence: with a shortlist and a
budget that cover every key, SVA attention is exact attention, so the patched
model's logits equal the unpatched model's (eager attention, fp32) for
prefill and cached decode in every summon mode.
"""

from __future__ import annotations

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from sva import SVAArtifactBundle, SVALayerArtifacts, SVALlamaAttention, patch_llama_attention

pytestmark = pytest.mark.gpu


def make_tiny_model(device, hidden=16, heads=2, kv_heads=2, layers=2, attn="sdpa", seed=0):
    torch.manual_seed(seed)
    config = LlamaConfig(vocab_size=64, hidden_size=hidden, intermediate_size=2 * hidden, num_hidden_layers=layers,
                         num_attention_heads=heads, num_key_value_heads=kv_heads, max_position_embeddings=256,
                         rope_theta=10000.0, tie_word_embeddings=False, attn_implementation=attn)
    model = LlamaForCausalLM(config)
    model.eval()
    return model.to(device)


def make_tiny_bundle(heads=2, head_dim=8, rank=4, subspaces=2, codewords=8, layers=2, shortlist=4, budget=2):
    generator = torch.Generator().manual_seed(11)
    arts = {}
    for i in range(layers):
        arts[i] = SVALayerArtifacts(
            q_proj=torch.randn(heads, head_dim, rank, generator=generator),
            k_proj=torch.randn(heads, head_dim, rank, generator=generator),
            logit_scale=torch.zeros(heads),
            coarse_codebooks=torch.randn(heads, subspaces, codewords, rank // subspaces, generator=generator),
            train_loss=0.0, hard_loss=0.0, route_source="qk")
    manifest = {"schema_version": 1, "artifact_type": "summon_verify_attention", "rank_dim": rank,
                "coarse_subspaces": subspaces, "coarse_codewords": codewords, "default_shortlist": shortlist,
                "default_budget": budget, "layer_count": layers, "layers": list(range(layers))}
    return SVAArtifactBundle(manifest=manifest, layers=arts)


def ids(device, *tokens):
    return torch.tensor([list(tokens)], device=device)


def test_patch_prefill_unpatch(device):
    model = make_tiny_model(device)
    bundle = make_tiny_bundle()
    original = model.model.layers[0].self_attn
    handle = patch_llama_attention(model, bundle)
    assert isinstance(model.model.layers[0].self_attn, SVALlamaAttention)
    with torch.no_grad():
        output = model(input_ids=ids(device, 1, 2, 3, 4, 5, 6), use_cache=False)
    assert tuple(output.logits.shape) == (1, 6, 64)
    summary = handle.stats.summary()
    assert summary["queries"] > 0
    assert summary["avg_verified"] <= 2.0
    handle.unpatch()
    assert model.model.layers[0].self_attn is original


def test_context_manager_restores_after_cached_decode(device):
    model = make_tiny_model(device)
    original = model.model.layers[1].self_attn
    with patch_llama_attention(model, make_tiny_bundle(), shortlist=4, budget=2, summon_mode="inverted",
                               inverted_cells_per_subspace=2, adaptive_min_budget=1, adaptive_mid_budget=2) as handle:
        with torch.no_grad():
            first = model(input_ids=ids(device, 1, 2, 3, 4), use_cache=True)
            second = model(input_ids=ids(device, 5), use_cache=True, past_key_values=first.past_key_values)
        assert tuple(second.logits.shape) == (1, 1, 64)
        assert handle.stats.summary()["queries"] > 0
        assert handle.stats.summary()["avg_cell_visits"] > 0
    assert model.model.layers[1].self_attn is original


def test_static_inverted_cached_decode(device):
    model = make_tiny_model(device)
    original = model.model.layers[1].self_attn
    with patch_llama_attention(model, make_tiny_bundle(), shortlist=4, budget=2, summon_mode="inverted_static",
                               inverted_cells_per_subspace=2, profile_components=True) as handle:
        with torch.no_grad():
            first = model(input_ids=ids(device, 1, 2, 3, 4), use_cache=True)
            second = model(input_ids=ids(device, 5), use_cache=True, past_key_values=first.past_key_values)
            third = model(input_ids=ids(device, 6), use_cache=True, past_key_values=second.past_key_values)
        assert tuple(second.logits.shape) == (1, 1, 64)
        assert tuple(third.logits.shape) == (1, 1, 64)
        summary = handle.stats.summary()
        assert summary["queries"] > 0
        assert summary["avg_refill_pool"] > 0
        assert summary["avg_static_total_ms"] >= 0
        assert summary["avg_static_outer_total_ms"] >= summary["avg_static_total_ms"]
        attention = model.model.layers[1].self_attn
        assert isinstance(attention, SVALlamaAttention)
        assert attention._cached_key_len == 6
        assert attention._cached_postings_key_len == 4
        assert tuple(attention._cached_coarse_codes.shape) == (2, 4, 2)
    assert model.model.layers[1].self_attn is original


def test_static_inverted_rebuilds_after_tail_interval(device):
    model = make_tiny_model(device)
    original = model.model.layers[1].self_attn
    with patch_llama_attention(model, make_tiny_bundle(), shortlist=4, budget=2, summon_mode="inverted_static",
                               inverted_cells_per_subspace=2, static_tail_rebuild_interval=2):
        with torch.no_grad():
            first = model(input_ids=ids(device, 1, 2, 3, 4), use_cache=True)
            second = model(input_ids=ids(device, 5), use_cache=True, past_key_values=first.past_key_values)
            model(input_ids=ids(device, 6), use_cache=True, past_key_values=second.past_key_values)
        attention = model.model.layers[1].self_attn
        assert attention._cached_key_len == 6
        assert attention._cached_postings_key_len == 6
        assert tuple(attention._cached_coarse_codes.shape) == (2, 6, 2)
    assert model.model.layers[1].self_attn is original


def test_static_inverted_multitoken_cache_keeps_full_codes(device):
    model = make_tiny_model(device)
    original = model.model.layers[1].self_attn
    with patch_llama_attention(model, make_tiny_bundle(), shortlist=4, budget=2, summon_mode="inverted_static",
                               inverted_cells_per_subspace=2):
        with torch.no_grad():
            first = model(input_ids=ids(device, 1, 2, 3, 4), use_cache=True)
            second = model(input_ids=ids(device, 5, 6), use_cache=True, past_key_values=first.past_key_values)
        assert tuple(second.logits.shape) == (1, 2, 64)
        attention = model.model.layers[1].self_attn
        assert attention._cached_key_len == 6
        assert tuple(attention._cached_coarse_codes.shape) == (2, 6, 2)
    assert model.model.layers[1].self_attn is original


def test_patch_selected_layers_only(device):
    model = make_tiny_model(device)
    layer0, layer1 = model.model.layers[0].self_attn, model.model.layers[1].self_attn
    handle = patch_llama_attention(model, make_tiny_bundle(), layers=[1])
    assert model.model.layers[0].self_attn is layer0
    assert isinstance(model.model.layers[1].self_attn, SVALlamaAttention)
    with torch.no_grad():
        output = model(input_ids=ids(device, 1, 2, 3, 4), use_cache=False)
    assert tuple(output.logits.shape) == (1, 4, 64)
    assert handle.stats.summary()["queries"] > 0
    handle.unpatch()
    assert model.model.layers[0].self_attn is layer0
    assert model.model.layers[1].self_attn is layer1


@pytest.mark.parametrize("mode", ["scan", "inverted", "inverted_static"])
def test_full_budget_equals_dense_attention(device, mode):
    # GQA (4 query heads over 2 KV heads), head_dim 64, rank 64 with 2x16 codes
    heads, kv_heads, head_dim, n_tok = 4, 2, 64, 40
    model = make_tiny_model(device, hidden=heads * head_dim, heads=heads, kv_heads=kv_heads, attn="eager", seed=3)
    bundle = make_tiny_bundle(heads=heads, head_dim=head_dim, rank=64, subspaces=2, codewords=16,
                              shortlist=4096, budget=4096)
    prompt = torch.randint(0, 64, (1, n_tok), generator=torch.Generator().manual_seed(5)).to(device)
    steps = [7, 19, 33]
    with torch.no_grad():
        ref = model(input_ids=prompt, use_cache=True)
        ref_logits = [ref.logits]
        past = ref.past_key_values
        for t in steps:
            o = model(input_ids=ids(device, t), use_cache=True, past_key_values=past)
            ref_logits.append(o.logits)
            past = o.past_key_values
        with patch_llama_attention(model, bundle, summon_mode=mode, inverted_cells_per_subspace=16):
            got = model(input_ids=prompt, use_cache=True)
            got_logits = [got.logits]
            past = got.past_key_values
            for t in steps:
                o = model(input_ids=ids(device, t), use_cache=True, past_key_values=past)
                got_logits.append(o.logits)
                past = o.past_key_values
    for r, g in zip(ref_logits, got_logits):
        err = (r - g).abs().max().item() / r.abs().max().item()
        assert err < 2e-4, f"{mode}: logits differ by {err}"


@pytest.mark.parametrize("attn", ["eager", "sdpa"])
def test_batch_of_sequences_equals_each_alone(device, attn):
    # batch 3 through the packed scan path == each sequence decoded on its own
    # (a shortlist / budget well below the cache, so the selection matters)
    heads, kv_heads, head_dim, n_tok = 4, 2, 64, 48
    model = make_tiny_model(device, hidden=heads * head_dim, heads=heads, kv_heads=kv_heads, attn=attn, seed=5)
    bundle = make_tiny_bundle(heads=heads, head_dim=head_dim, rank=64, subspaces=2, codewords=16, shortlist=24,
                              budget=8)
    g = torch.Generator().manual_seed(9)
    prompts = torch.randint(0, 64, (3, n_tok), generator=g).to(device)
    steps = torch.randint(0, 64, (3, 3), generator=g).to(device)
    with torch.no_grad(), patch_llama_attention(model, bundle, summon_mode="scan") as handle:
        out = model(input_ids=prompts, use_cache=True)
        batched, past = [out.logits], out.past_key_values
        for j in range(steps.shape[1]):
            out = model(input_ids=steps[:, j:j + 1], use_cache=True, past_key_values=past)
            batched.append(out.logits)
            past = out.past_key_values
        for b in range(3):
            handle.reset_catalogs()
            out = model(input_ids=prompts[b:b + 1], use_cache=True)
            single, past = [out.logits], out.past_key_values
            for j in range(steps.shape[1]):
                out = model(input_ids=steps[b:b + 1, j:j + 1], use_cache=True, past_key_values=past)
                single.append(out.logits)
                past = out.past_key_values
            for r, s in zip(batched, single):
                err = (r[b] - s[0]).abs().max().item() / s.abs().max().item()
                assert err < 1e-4, f"sequence {b}: logits differ by {err}"


def test_batch_needs_scan_mode(device):
    model = make_tiny_model(device)
    with torch.no_grad(), patch_llama_attention(model, make_tiny_bundle(), summon_mode="inverted_static"):
        with pytest.raises(ValueError, match="summon_mode='scan'"):
            model(input_ids=torch.tensor([[1, 2, 3], [4, 5, 6]], device=device), use_cache=False)


@pytest.mark.parametrize("attn", ["eager", "sdpa"])
@pytest.mark.parametrize("batch", [1, 2])
def test_query_chunks_equal_one_pass(device, attn, batch):
    # A prefill and a multi-token extension split into chunks of 7 query
    # tokens give what one pass gives (sva/llama.py:262-328 scores every token
    # on its own); without a mask each chunk sees the first N - Q + chunk_end
    # keys, which keeps the causal rule.
    heads, kv_heads, head_dim = 4, 2, 64
    model = make_tiny_model(device, hidden=heads * head_dim, heads=heads, kv_heads=kv_heads, attn=attn, seed=7)
    bundle = make_tiny_bundle(heads=heads, head_dim=head_dim, rank=64, subspaces=2, codewords=16, shortlist=24,
                              budget=8)
    g = torch.Generator().manual_seed(13)
    prompt = torch.randint(0, 64, (batch, 45), generator=g).to(device)
    more = torch.randint(0, 64, (batch, 19), generator=g).to(device)
    results = []
    for chunk in (None, 7):
        with torch.no_grad(), patch_llama_attention(model, bundle, summon_mode="scan", query_chunk_size=chunk) as h:
            out = model(input_ids=prompt, use_cache=True)
            ext = model(input_ids=more, use_cache=True, past_key_values=out.past_key_values)
            results.append((out.logits, ext.logits, h.stats.summary()))
    (a0, a1, sa), (b0, b1, sb) = results
    for r, c in ((a0, b0), (a1, b1)):
        err = (r - c).abs().max().item() / r.abs().max().item()
        assert err < 1e-5, f"chunked logits differ by {err}"
    for key in ("queries", "avg_summoned", "avg_verified"):
        assert sa[key] == sb[key], key


def _decode_layer(device, heads=4, kv_heads=2, head_dim=64):
    model = make_tiny_model(device, hidden=heads * head_dim, heads=heads, kv_heads=kv_heads, seed=3)
    bundle = make_tiny_bundle(heads=heads, head_dim=head_dim, rank=64, subspaces=2, codewords=16, shortlist=12,
                              budget=6)
    return model, bundle


def test_padded_batch_decode_raises(device):
    # A left-padded batch gives each sequence its own mask row at every decode
    # step; the packed launch takes one mask, so it refuses rather than
    # applying sequence 0's row to all.  Equal rows decode as each sequence
    # alone.
    heads, kv_heads, head_dim, n = 4, 2, 64, 40
    model, bundle = _decode_layer(device, heads, kv_heads, head_dim)
    g = torch.Generator().manual_seed(21)
    q = torch.randn(2, heads, 1, head_dim, generator=g).to(device)
    k = torch.randn(2, kv_heads, n, head_dim, generator=g).to(device)
    v = torch.randn(2, kv_heads, n, head_dim, generator=g).to(device)
    fmin = torch.finfo(torch.float32).min
    with torch.no_grad(), patch_llama_attention(model, bundle, summon_mode="scan") as handle:
        attn = model.model.layers[0].self_attn
        padded = torch.zeros(2, 1, 1, n, device=device)
        padded[1, :, :, :5] = fmin
        with pytest.raises(ValueError, match="same attention mask"):
            attn.sva_attention(q, k, v, padded)
        shared = torch.zeros(2, 1, 1, n, device=device)
        shared[:, :, :, :5] = fmin
        handle.reset_catalogs()
        both = attn.sva_attention(q, k, v, shared)
        for b in range(2):
            handle.reset_catalogs()
            alone = attn.sva_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1], shared[b:b + 1])
            err = (both[b] - alone[0]).abs().max().item() / alone.abs().max().item()
            assert err < 1e-5, f"sequence {b}: {err}"


def test_per_head_mask(device):
    # a mask with a head dim: equal heads act as one mask, differing heads raise
    heads, kv_heads, head_dim, n = 4, 2, 64, 40
    model, bundle = _decode_layer(device, heads, kv_heads, head_dim)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(1, heads, 1, head_dim, generator=g).to(device)
    k = torch.randn(1, kv_heads, n, head_dim, generator=g).to(device)
    v = torch.randn(1, kv_heads, n, head_dim, generator=g).to(device)
    fmin = torch.finfo(torch.float32).min
    one = torch.zeros(1, 1, 1, n, device=device)
    one[..., 7:19] = fmin
    with torch.no_grad(), patch_llama_attention(model, bundle, summon_mode="scan") as handle:
        attn = model.model.layers[0].self_attn
        ref = attn.sva_attention(q, k, v, one)
        handle.reset_catalogs()
        got = attn.sva_attention(q, k, v, one.expand(1, heads, 1, n).contiguous())
        assert torch.equal(ref, got)
        differ = one.expand(1, heads, 1, n).clone()
        differ[0, 2, 0, 30] = fmin
        with pytest.raises(ValueError, match="leading"):
            attn.sva_attention(q, k, v, differ)


def test_decode_next_token_path_equals_full_checks(device):
    # after one native decode step, the next tokens take the lean path (only
    # what moves is compared again); its logits and statistics equal those of
    # the full path token by token
    heads, kv_heads, head_dim = 4, 2, 64
    model = make_tiny_model(device, hidden=heads * head_dim, heads=heads, kv_heads=kv_heads, seed=7)
    bundle = make_tiny_bundle(heads=heads, head_dim=head_dim, rank=64, subspaces=2, codewords=16, shortlist=24,
                              budget=8)
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 64, (1, 48), generator=g).to(device)
    steps = torch.randint(0, 64, (1, 6), generator=g).to(device)

    def run(lean):
        taken = []
        with torch.no_grad(), patch_llama_attention(model, bundle, summon_mode="scan") as handle:
            for layer in model.model.layers:
                attn = layer.self_attn
                if lean:
                    orig = attn._decode_next

                    def counted(q, k, v, _orig=orig):
                        out = _orig(q, k, v)
                        taken.append(out is not None)
                        return out

                    attn._decode_next = counted
                else:
                    attn._decode_next = lambda q, k, v: None
            out = model(input_ids=prompt, use_cache=True)
            logits, past = [out.logits], out.past_key_values
            for j in range(steps.shape[1]):
                out = model(input_ids=steps[:, j:j + 1], use_cache=True, past_key_values=past)
                logits.append(out.logits)
                past = out.past_key_values
            torch.cuda.synchronize()
            totals = dict(handle.stats.totals)
        return logits, totals, taken

    lean_logits, lean_totals, taken = run(True)
    full_logits, full_totals, _ = run(False)
    # two layers x six tokens; the first decode token of each layer sets the lean path up
    assert sum(taken) == 2 * (steps.shape[1] - 1), taken
    for a, b in zip(lean_logits, full_logits):
        assert torch.equal(a, b)
    assert lean_totals == full_totals and lean_totals["queries"] > 0
