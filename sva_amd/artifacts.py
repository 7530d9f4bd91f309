"""Frozen per-layer SVA artifacts: the on-disk bundle (schema version 1).

Layout of a bundle directory (sva/artifacts.py:13-15, :91-128):
  sva_config.json   manifest: schema_version, rank_dim, coarse_subspaces,
                    coarse_codewords, default_shortlist, default_budget,
                    layer_count, layers, model_id, optional weights_file
  sva_artifacts.pt  {"schema_version": 1, "layer_meta": {str(i): {...}},
                     "tensors": {"layers.{i}.q_proj" [H, D, R],
                                 "layers.{i}.k_proj" [H, D, R],
                                 "layers.{i}.logit_scale" [H],
                                 "layers.{i}.coarse_codebooks" [H, S, C, R/S]}}
Weights are read with ``torch.load(weights_only=True)`` only: a file that
needs unpickling of arbitrary objects is refused.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch

SCHEMA_VERSION = 1
WEIGHTS_NAME = "sva_artifacts.pt"
MANIFEST_NAME = "sva_config.json"


@dataclass(frozen=True)
class SVALayerArtifacts:
    """One layer's learned maps, logit scale (log space) and PQ codebooks."""

    q_proj: torch.Tensor
    k_proj: torch.Tensor
    logit_scale: torch.Tensor
    coarse_codebooks: torch.Tensor
    train_loss: float
    hard_loss: float
    route_source: str = "qk"


@dataclass(frozen=True)
class SVAArtifactBundle:
    """Manifest plus per-layer artifacts (sva/artifacts.py:30-80)."""

    manifest: dict[str, Any]
    layers: dict[int, SVALayerArtifacts]

    @property
    def model_id(self) -> str | None:
        mid = self.manifest.get("model_id")
        return None if mid is None else str(mid)

    @property
    def rank_dim(self) -> int:
        return int(self.manifest["rank_dim"])

    @property
    def coarse_subspaces(self) -> int:
        return int(self.manifest["coarse_subspaces"])

    @property
    def coarse_codewords(self) -> int:
        return int(self.manifest["coarse_codewords"])

    @property
    def default_shortlist(self) -> int:
        return int(self.manifest.get("default_shortlist", 2048))

    @property
    def default_budget(self) -> int:
        return int(self.manifest.get("default_budget", 512))

    @property
    def layer_count(self) -> int:
        return int(self.manifest.get("layer_count", len(self.layers)))

    def to(self, device: torch.device | str, dtype: torch.dtype | None = None) -> "SVAArtifactBundle":
        """Copy with tensors on `device` (and `dtype` for the maps and codebooks;
        the logit scale stays fp32)."""

        def move(t: torch.Tensor, keep_f32: bool = False) -> torch.Tensor:
            return t.to(device=device, dtype=torch.float32 if keep_f32 else (dtype or t.dtype))

        layers = {
            i: SVALayerArtifacts(
                q_proj=move(a.q_proj),
                k_proj=move(a.k_proj),
                logit_scale=move(a.logit_scale, keep_f32=True),
                coarse_codebooks=move(a.coarse_codebooks),
                train_loss=a.train_loss,
                hard_loss=a.hard_loss,
                route_source=a.route_source,
            )
            for i, a in self.layers.items()
        }
        return SVAArtifactBundle(dict(self.manifest), layers)


def _meta_float(meta: dict[str, Any], key: str) -> float:
    value = meta.get(key)
    return float("nan") if value is None else float(value)


def load_sva_artifact_bundle(artifact_dir: str | Path, map_location: str | torch.device = "cpu") -> SVAArtifactBundle:
    """Read and validate a bundle directory (sva/artifacts.py:91-128)."""

    root = Path(artifact_dir)
    manifest = json.loads((root / MANIFEST_NAME).read_text(encoding="utf-8"))
    if int(manifest.get("schema_version", -1)) != SCHEMA_VERSION:
        raise ValueError(f"Unsupported SVA artifact schema: {manifest.get('schema_version')!r}")
    payload = torch.load(root / manifest.get("weights_file", WEIGHTS_NAME), map_location=map_location,
                         weights_only=True)
    if int(payload.get("schema_version", -1)) != SCHEMA_VERSION:
        raise ValueError(f"Unsupported SVA weights schema: {payload.get('schema_version')!r}")
    tensors: dict[str, torch.Tensor] = payload["tensors"]
    metas: dict[str, dict[str, Any]] = payload.get("layer_meta", {})
    layers: dict[int, SVALayerArtifacts] = {}
    for raw in manifest["layers"]:
        i = int(raw)
        meta = metas.get(str(i), {})
        key = f"layers.{i}"
        layers[i] = SVALayerArtifacts(
            q_proj=tensors[f"{key}.q_proj"],
            k_proj=tensors[f"{key}.k_proj"],
            logit_scale=tensors[f"{key}.logit_scale"],
            coarse_codebooks=tensors[f"{key}.coarse_codebooks"],
            train_loss=_meta_float(meta, "train_loss"),
            hard_loss=_meta_float(meta, "hard_loss"),
            route_source=str(meta.get("route_source", manifest.get("route_source", "qk"))),
        )
    bundle = SVAArtifactBundle(manifest, layers)
    validate_artifact_bundle(bundle)
    return bundle


def validate_artifact_bundle(bundle: SVAArtifactBundle) -> None:
    """Shape and manifest consistency, with the reference's messages
    (sva/artifacts.py:131-167)."""

    if not bundle.layers:
        raise ValueError("SVA artifact bundle contains no layers.")
    rank, subspaces, codewords = bundle.rank_dim, bundle.coarse_subspaces, bundle.coarse_codewords
    if rank <= 0:
        raise ValueError(f"rank_dim must be positive, got {rank}.")
    if subspaces <= 0 or rank % subspaces != 0:
        raise ValueError(f"rank_dim={rank} must be divisible by coarse_subspaces={subspaces}.")
    if codewords <= 0:
        raise ValueError(f"coarse_codewords must be positive, got {codewords}.")
    for i, a in bundle.layers.items():
        if a.q_proj.shape != a.k_proj.shape:
            raise ValueError(f"Layer {i} q_proj/k_proj shape mismatch: {a.q_proj.shape} vs {a.k_proj.shape}.")
        if a.q_proj.ndim != 3:
            raise ValueError(f"Layer {i} q_proj must have shape [heads, head_dim, rank_dim].")
        if int(a.q_proj.shape[-1]) != rank:
            raise ValueError(f"Layer {i} rank_dim mismatch: {a.q_proj.shape[-1]} vs {rank}.")
        heads = int(a.q_proj.shape[0])
        if a.logit_scale.ndim != 1 or int(a.logit_scale.shape[0]) != heads:
            raise ValueError(f"Layer {i} logit_scale must have one value per attention head.")
        want = (heads, subspaces, codewords, rank // subspaces)
        if tuple(a.coarse_codebooks.shape) != want:
            raise ValueError(f"Layer {i} coarse_codebooks shape mismatch: {tuple(a.coarse_codebooks.shape)} vs {want}.")
        if a.route_source != "qk":
            raise ValueError(f"Layer {i} uses route_source={a.route_source!r}. "
                             "The production adapter currently supports qk artifacts.")


def save_sva_artifact_bundle(bundle: SVAArtifactBundle, artifact_dir: str | Path) -> Path:
    """Write a bundle in the schema-1 layout above (the layout the reference's
    exporter writes, experiments/sva_artifact_io.py:25-61)."""

    validate_artifact_bundle(bundle)
    root = Path(artifact_dir)
    root.mkdir(parents=True, exist_ok=True)
    manifest = dict(bundle.manifest)
    manifest["schema_version"] = SCHEMA_VERSION
    manifest.setdefault("layers", sorted(bundle.layers))
    manifest.setdefault("layer_count", len(bundle.layers))
    weights = manifest.get("weights_file", WEIGHTS_NAME)
    tensors: dict[str, torch.Tensor] = {}
    metas: dict[str, dict[str, Any]] = {}
    for i, a in sorted(bundle.layers.items()):
        key = f"layers.{i}"
        tensors[f"{key}.q_proj"] = a.q_proj.detach().cpu().contiguous()
        tensors[f"{key}.k_proj"] = a.k_proj.detach().cpu().contiguous()
        tensors[f"{key}.logit_scale"] = a.logit_scale.detach().float().cpu().contiguous()
        tensors[f"{key}.coarse_codebooks"] = a.coarse_codebooks.detach().cpu().contiguous()
        metas[str(i)] = {"train_loss": a.train_loss, "hard_loss": a.hard_loss, "route_source": a.route_source}
    torch.save({"schema_version": SCHEMA_VERSION, "layer_meta": metas, "tensors": tensors}, root / weights)
    (root / MANIFEST_NAME).write_text(json.dumps(manifest, indent=2, sort_keys=True), encoding="utf-8")
    return root
