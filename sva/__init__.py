"""Import name of the reference package (sva/__init__.py): ``import sva``,
``from sva import patch_llama_attention``, ``from sva.ops import
encode_product_keys`` and ``from sva.llama import SVALlamaAttention`` resolve
to the HIP implementation in ``sva_amd``.  The submodules are the same module
objects as sva_amd's (registered under this package's name), so state such as
the loaded library and the workspaces is shared whichever name a caller uses.
"""

from __future__ import annotations

import importlib
import sys

for _name in ("artifacts", "llama", "ops", "stats"):
    _module = importlib.import_module(f"sva_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module

from sva_amd.artifacts import SVAArtifactBundle, SVALayerArtifacts, load_sva_artifact_bundle  # noqa: E402
from sva_amd.llama import SVALlamaAttention, SVALlamaPatcher, patch_llama_attention  # noqa: E402
from sva_amd.stats import SVAStats  # noqa: E402

__all__ = [
    "SVAArtifactBundle",
    "SVALayerArtifacts",
    "SVALlamaAttention",
    "SVALlamaPatcher",
    "SVAStats",
    "load_sva_artifact_bundle",
    "patch_llama_attention",
]
