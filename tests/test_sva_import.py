"""The reference's import name on the CPU side: ``sva`` and its submodules
are sva_amd's own module objects, and the compute entry points refuse CPU
tensors (there is no CPU fallback)."""

from __future__ import annotations

import pytest
import torch


def test_sva_submodules_are_the_hip_package_modules():
    import sva
    import sva.llama
    import sva.ops
    import sva_amd.artifacts
    import sva_amd.llama
    import sva_amd.ops
    import sva_amd.stats

    assert sva.ops is sva_amd.ops and sva.llama is sva_amd.llama
    assert sva.artifacts is sva_amd.artifacts and sva.stats is sva_amd.stats
    for name in ("SVAArtifactBundle", "SVALayerArtifacts", "SVALlamaAttention", "SVALlamaPatcher", "SVAStats",
                 "load_sva_artifact_bundle", "patch_llama_attention"):
        assert name in sva.__all__ and getattr(sva, name) is not None
    assert sva.SVALlamaAttention is sva_amd.llama.SVALlamaAttention


def test_sva_ops_refuse_cpu_tensors():
    from sva.ops import assign_to_centroids, encode_product_keys, product_quantized_scores

    with pytest.raises(RuntimeError, match="no CPU fallback"):
        encode_product_keys(torch.randn(2, 10, 4), torch.randn(2, 2, 3, 2), 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        assign_to_centroids(torch.randn(10, 4), torch.randn(3, 4), 8)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        product_quantized_scores(torch.randn(2, 1, 4), torch.randn(2, 2, 3, 2), torch.zeros(2, 5, 2).long(), 4)
