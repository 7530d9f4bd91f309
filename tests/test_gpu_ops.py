"""The reference's import surface and sva.ops on the GPU.

The names a reference caller imports resolve (tests/test_sva_llama_adapter.py:8,
experiments/sva_block_elevator_benchmark.py:27-28); encode_product_keys and
assign_to_centroids give the oracle's codes (int64, first index on ties,
differences only where the two best distances are within rounding);
product_quantized_scores is bit-exact with the oracle's table and sum order
(sva/ops.py:50-71) and raises on a code outside the codebook, as the
reference's gather does.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def test_reference_caller_imports_resolve_to_the_hip_path(device):
    from sva import SVAArtifactBundle, SVALayerArtifacts, SVALlamaAttention, patch_llama_attention  # noqa: F401
    from sva import load_sva_artifact_bundle  # noqa: F401
    from sva.ops import encode_product_keys, product_quantized_scores

    import sva_amd.ops

    assert encode_product_keys is sva_amd.ops.encode_product_keys
    assert product_quantized_scores is sva_amd.ops.product_quantized_scores
    k_low = torch.randn(2, 100, 8, device=device)
    codes = encode_product_keys(k_low, torch.randn(2, 2, 8, 4, device=device), 8192)
    assert codes.device == k_low.device and codes.dtype == torch.int64 and tuple(codes.shape) == (2, 100, 2)


@pytest.mark.parametrize("S,C", [(2, 256), (4, 64), (1, 256), (8, 16)])
def test_encode_product_keys_matches_oracle(device, S, C):
    from sva.ops import encode_product_keys

    rng = np.random.default_rng(S * 100 + C)
    k_low = rng.standard_normal((9, 5000, 64)).astype(np.float32)
    cb = rng.standard_normal((9, S, C, 64 // S)).astype(np.float32)
    codes = encode_product_keys(torch.from_numpy(k_low).to(device), torch.from_numpy(cb).to(device), 8192)
    torch.cuda.synchronize()
    assert codes.dtype == torch.int64 and tuple(codes.shape) == (9, 5000, S)
    ref, gaps = oracle.encode_product_keys(k_low, cb, return_gap=True)
    diff = codes.cpu().numpy() != ref
    assert np.all(gaps[diff] <= 1e-4) and diff.sum() <= 3


def test_encode_product_keys_rejects_indivisible_rank(device):
    from sva.ops import encode_product_keys

    with pytest.raises(ValueError, match="divisible"):
        encode_product_keys(torch.randn(2, 10, 10, device=device), torch.randn(2, 3, 4, 3, device=device), 8)


def test_assign_to_centroids_matches_oracle_and_breaks_ties_low(device):
    from sva.ops import assign_to_centroids

    rng = np.random.default_rng(3)
    x = rng.standard_normal((3000, 32)).astype(np.float32)
    cents = rng.standard_normal((256, 32)).astype(np.float32)
    got = assign_to_centroids(torch.from_numpy(x).to(device), torch.from_numpy(cents).to(device), 1024)
    ref, gaps = oracle.assign_to_centroids(x, cents, return_gap=True)
    diff = got.cpu().numpy() != ref
    assert got.dtype == torch.int64 and np.all(gaps[diff] <= 1e-4) and diff.sum() <= 2
    cents[128:] = cents[:128]  # every best distance shared by two centroids: the lower index wins
    got = assign_to_centroids(torch.from_numpy(x).to(device), torch.from_numpy(cents).to(device), 1024).cpu().numpy()
    assert got.max() < 128
    np.testing.assert_array_equal(got, oracle.assign_to_centroids(x, cents))


@pytest.mark.parametrize("S,C,code_dtype", [(2, 256, torch.int64), (4, 64, torch.uint8), (1, 256, torch.int32)])
def test_product_quantized_scores_bit_exact(device, S, C, code_dtype):
    from sva.ops import product_quantized_scores

    rng = np.random.default_rng(S + C)
    H, Q, N = 9, 3, 7000
    q_low = rng.standard_normal((H, Q, 64)).astype(np.float32)
    cb = rng.standard_normal((H, S, C, 64 // S)).astype(np.float32)
    codes = rng.integers(0, C, (H, N, S))
    got = product_quantized_scores(torch.from_numpy(q_low).to(device), torch.from_numpy(cb).to(device),
                                   torch.from_numpy(codes).to(device, code_dtype), 64)
    torch.cuda.synchronize()
    assert tuple(got.shape) == (H, Q, N) and got.dtype == torch.float32
    ref = oracle.product_quantized_scores(q_low, cb, codes.astype(np.int64), 64)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_product_quantized_scores_rejects_codes_outside_the_codebook(device):
    from sva.ops import product_quantized_scores

    codes = torch.zeros(2, 50, 2, device=device, dtype=torch.int64)
    codes[1, 7, 1] = 8
    with pytest.raises(IndexError):
        product_quantized_scores(torch.randn(2, 1, 8, device=device), torch.randn(2, 2, 8, 4, device=device), codes, 8)
