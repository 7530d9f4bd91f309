"""Calibration refresh of the coarse codebooks on the GPU: re-fit each
layer's product codebooks on the key catalog of a calibration prompt,
optionally weighting the keys that real queries attend to
(experiments/export_refreshed_sva_artifact.py:73-154,
experiments/sva_codebook_refresh_benchmark.py:64-70 and :130-153,
experiments/sva_rotation_diagnostic.py:86-116 and :132-150).

Per refreshed layer, from one forward pass over the calibration batch:
  1. query / key rows of every head at every position (the layer's input
     norm, projections, rotary embedding, KV heads repeated to the query
     heads);
  2. k_low = key @ k_proj per head (the catalog the codebooks quantise);
  3. attention-weighted methods only: exact causal scores of a spread of
     query positions against every key, their top-k keys, and per-key
     weights 1 + boost per hit (``sva_key_weights``, one HIP pass);
  4. k-means (plain or weighted) with the fits of ``codebooks`` (HIP
     assignment / postings / centroid update launches);
  5. the codes of the new codebooks and two balance figures (normalised code
     entropy, mean largest-cell fraction) reported per layer.

``export_refreshed_bundle`` writes the result as a schema-1 bundle beside
the base one: the base layers with their codebooks replaced, the manifest
extended with the refresh settings.
"""

from __future__ import annotations

import math
from dataclasses import replace
from datetime import datetime, timezone
from pathlib import Path
from typing import Any, Callable

import torch

from . import kernels
from ._lib import check, lib, ptr, require_device, stream_handle
from .artifacts import SVAArtifactBundle, save_sva_artifact_bundle
from .codebooks import fit_product_codebooks, fit_weighted_product_codebooks

REFRESH_METHODS = ("identity_kmeans", "attention_weighted", "attention_weighted_strong")


def attention_boost_for(method: str, boost: float) -> float:
    """The effective boost of a refresh method: the "strong" variant weighs hits 4x."""

    if method not in REFRESH_METHODS:
        raise ValueError(f"unknown refresh method {method!r}; expected one of {REFRESH_METHODS}")
    return 4.0 * boost if method == "attention_weighted_strong" else boost


@torch.no_grad()
def topk_key_weights(top_idx: torch.Tensor, top_valid: torch.Tensor, seq_len: int, boost: float) -> torch.Tensor:
    """Per-key weights fp32 [H, seq_len]: 1, plus ``boost`` for every valid
    top-k hit of the key in that head (indices clamped into [0, seq_len)),
    each addition rounded in turn as index_add_ does.  top_idx / top_valid
    [H, ...] (any trailing shape)."""

    if top_idx.shape != top_valid.shape or top_idx.dim() < 1:
        raise ValueError(f"top_idx {tuple(top_idx.shape)} and top_valid {tuple(top_valid.shape)} must match")
    if seq_len <= 0:
        raise ValueError("seq_len must be positive")
    device = require_device(top_idx, top_valid)
    heads = int(top_idx.shape[0])
    idx = top_idx.reshape(heads, -1).to(torch.int64).contiguous()
    valid = top_valid.reshape(heads, -1).to(torch.bool).contiguous()
    weights = torch.empty(heads, seq_len, device=device, dtype=torch.float32)
    check(lib().sva_key_weights(ptr(idx), ptr(valid), heads, idx.shape[1], seq_len, float(boost), ptr(weights),
                                stream_handle(device)), "sva_key_weights")
    return weights


@torch.no_grad()
def topk_targets(scores: torch.Tensor, query_positions: torch.Tensor, topk: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k keys of each sampled query under the causal mask: scores
    [H, Qs, N] with keys after a query's position set to the fp32 minimum;
    returns (idx [H, Qs, k] int64, valid [H, Qs, k]) where rank r is valid
    iff r <= the query's position (only position + 1 keys are visible)."""

    n = scores.shape[-1]
    after = torch.arange(n, device=scores.device)[None, :] > query_positions[:, None]
    masked = scores.masked_fill(after[None], torch.finfo(scores.dtype).min)
    k = min(topk, n)
    idx = masked.topk(k, dim=-1).indices
    valid = torch.arange(k, device=scores.device)[None, :] <= query_positions[:, None]
    return idx, valid[None].expand_as(idx)


def calibration_query_positions(seq_len: int, samples: int, min_pos: int, device) -> torch.Tensor:
    """min(samples, seq_len) query rows spread evenly from clamp(min_pos) to
    the last position (rounded toward zero, duplicates dropped).  The rows
    are computed on the host, where torch's linspace rounding is fixed, and
    handed to ``device``."""

    start = max(0, min(min_pos, seq_len - 1))
    return torch.linspace(start, seq_len - 1, steps=min(samples, seq_len)).long().unique().to(device)


@torch.no_grad()
def layer_query_key(model: Any, hidden_states: tuple[torch.Tensor, ...], layer_idx: int,
                    position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, float]:
    """(query [H, T, D] fp32, key [H, T, D] fp32 with KV heads repeated, scaling)
    of sequence 0 entering layer ``layer_idx`` (hidden_states[layer_idx] is
    the layer's input)."""

    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    layer = model.model.layers[layer_idx]
    attn = layer.self_attn
    attn = getattr(attn, "sva_attn", attn)  # a socket adapter wraps the attention
    x = layer.input_layernorm(hidden_states[layer_idx])
    batch, tokens = x.shape[0], x.shape[1]
    q = attn.q_proj(x).view(batch, tokens, -1, attn.head_dim).transpose(1, 2)
    k = attn.k_proj(x).view(batch, tokens, -1, attn.head_dim).transpose(1, 2)
    cos, sin = model.model.rotary_emb(x, position_ids)
    q, k = apply_rotary_pos_emb(q, k, cos, sin)
    group = q.shape[1] // k.shape[1]
    k = k[0].repeat_interleave(group, dim=0)
    return q[0].float(), k.float(), float(attn.scaling)


@torch.no_grad()
def code_balance(codes: torch.Tensor, codewords: int) -> tuple[float, float]:
    """(mean normalised entropy, mean largest-cell fraction) of the code
    histograms of every (head, subspace); codes [H, N, S]."""

    heads, n, subspaces = codes.shape
    flat = (codes.long().permute(0, 2, 1) + torch.arange(heads * subspaces, device=codes.device).view(
        heads, subspaces, 1) * codewords).reshape(-1)
    counts = torch.bincount(flat, minlength=heads * subspaces * codewords).view(heads * subspaces, codewords).double()
    probs = counts / counts.sum(-1, keepdim=True).clamp_min(1.0)
    entropy = -(probs * probs.clamp_min(1e-12).log()).sum(-1) / math.log(max(codewords, 2))
    largest = counts.max(-1).values / counts.sum(-1).clamp_min(1.0)
    return float(entropy.mean()), float(largest.mean())


@torch.no_grad()
def fit_refreshed_codebooks(*, model, runtime_bundle: SVAArtifactBundle, calibration_batch: dict[str, torch.Tensor],
                            layers: list[int], refresh_method: str, attention_topk: int,
                            calibration_query_samples: int, min_query_pos: int, attention_boost: float,
                            kmeans_iters: int, assign_chunk_size: int, seed: int, device: torch.device,
                            report: Callable[[dict[str, Any]], None] | None = None) -> dict[int, torch.Tensor]:
    """Refreshed codebooks {layer: [H, S, C, R / S] fp32 on the host} for
    ``layers``, from one forward pass over ``calibration_batch`` (sequence 0).
    ``report`` receives one dict per layer (layer, method, boosts, code
    entropy and largest-cell fraction)."""

    boost = attention_boost_for(refresh_method, attention_boost)
    weighted = refresh_method != "identity_kmeans"
    out = model(**calibration_batch, use_cache=False, output_hidden_states=True)
    if out.hidden_states is None:
        raise ValueError("Expected calibration hidden states.")
    seq_len = int(calibration_batch["input_ids"].shape[1])
    positions = torch.arange(seq_len, device=device)[None]
    subspaces, codewords = runtime_bundle.coarse_subspaces, runtime_bundle.coarse_codewords
    refreshed: dict[int, torch.Tensor] = {}
    for layer_idx in layers:
        query, key, scaling = layer_query_key(model, out.hidden_states, layer_idx, positions)
        k_proj = runtime_bundle.layers[layer_idx].k_proj.to(device=device, dtype=torch.float32)
        k_low = torch.bmm(key, k_proj)  # [H, T, R]
        layer_seed = seed + layer_idx * 9973
        if weighted:
            rows = calibration_query_positions(seq_len, calibration_query_samples, min_query_pos, device)
            scores = torch.bmm(query[:, rows].contiguous(), key.transpose(1, 2).contiguous()) * scaling
            top_idx, top_valid = topk_targets(scores, rows, attention_topk)
            del scores
            weights = topk_key_weights(top_idx, top_valid, seq_len, boost)
            codebooks = fit_weighted_product_codebooks(k_low, weights, subspaces, codewords, kmeans_iters, layer_seed,
                                                       assign_chunk_size)
        else:
            codebooks = fit_product_codebooks(k_low, subspaces, codewords, kmeans_iters, layer_seed,
                                              assign_chunk_size)
        codes = _encode(k_low, codebooks)
        entropy, largest = code_balance(codes, codebooks.shape[2])
        if report is not None:
            report({"layer": layer_idx, "calibration_seq_len": seq_len, "refresh_method": refresh_method,
                    "attention_boost": boost if weighted else 0.0, "attention_requested_boost": attention_boost,
                    "code_entropy": entropy, "code_max_fraction": largest})
        refreshed[layer_idx] = codebooks.detach().cpu()
        del query, key, k_low, codes
    return refreshed


def _encode(k_low: torch.Tensor, codebooks: torch.Tensor) -> torch.Tensor:
    heads, n, rank = k_low.shape
    codes = torch.empty(heads, n, codebooks.shape[1], device=k_low.device,
                        dtype=torch.uint8 if codebooks.shape[2] <= 256 else torch.int16)
    eye = torch.eye(rank, device=k_low.device).expand(heads, rank, rank).contiguous()
    kernels.write_encode(k_low.contiguous(), eye, codebooks.float().contiguous(), torch.empty_like(k_low), codes)
    return codes


def export_refreshed_bundle(base: SVAArtifactBundle, refreshed: dict[int, torch.Tensor], output_dir: str | Path, *,
                            settings: dict[str, Any], artifact_dtype: torch.dtype = torch.bfloat16) -> Path:
    """Write ``base`` with the codebooks of ``refreshed`` replaced (cast to
    ``artifact_dtype``; other layers unchanged) as a schema-1 bundle; the
    manifest gains ``settings`` (profile name, method, calibration sizes ...),
    a creation time and the base profile name."""

    layers = {}
    for i, a in base.layers.items():
        layers[i] = replace(a, coarse_codebooks=refreshed[i].to(artifact_dtype)) if i in refreshed else a
    manifest = dict(base.manifest)
    manifest.update({"created_at_utc": datetime.now(timezone.utc).replace(microsecond=0).isoformat(),
                     "base_profile_name": base.manifest.get("profile_name"),
                     "codebook_refresh_layers": ",".join(str(i) for i in sorted(refreshed)),
                     "layer_count": len(layers), **settings})
    return save_sva_artifact_bundle(SVAArtifactBundle(manifest, layers), output_dir)
