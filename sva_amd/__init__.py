"""SVA summon -> verify attention on MI355X (gfx950).

Drop-in for the reference package's public API (sva/__init__.py); the lookup
runs in the HIP library built from sva_amd/csrc (``python -m sva_amd.build``).
Exports load on first use, so ``sva_amd.build`` and ``sva_amd.kernels`` do not
import transformers.
"""

from __future__ import annotations

import importlib

_EXPORTS = {
    "SVAArtifactBundle": "artifacts",
    "SVALayerArtifacts": "artifacts",
    "load_sva_artifact_bundle": "artifacts",
    "save_sva_artifact_bundle": "artifacts",
    "validate_artifact_bundle": "artifacts",
    "SVALlamaAttention": "llama",
    "SVALlamaPatcher": "llama",
    "SVALlamaServingConfig": "llama",
    "patch_llama_attention": "llama",
    "SVAStats": "stats",
}

__all__ = sorted(_EXPORTS)


def __getattr__(name: str):
    module = _EXPORTS.get(name)
    if module is None:
        raise AttributeError(f"module 'sva_amd' has no attribute {name!r}")
    value = getattr(importlib.import_module(f".{module}", __name__), name)
    globals()[name] = value
    return value
