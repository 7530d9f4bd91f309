"""GPU parity of the write path (sva_write_encode).

k_low bit-exact with the oracle's projection (itself bit-exact with torch's
many-row einsum, tests/test_oracle.py); codes equal to the oracle's argmin
except where the oracle's two best distances lie within a few ulp (counted
and bounded); an append in two row ranges equals one fresh encode, and so do
decode-step appends of one to four rows (their own kernel).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _case(device, N, S, C, kv_dtype, seed, H=9, G=3, D=64, R=64):
    rng = np.random.default_rng(seed)
    keys = rng.standard_normal((G, N, D)).astype(np.float32)
    k_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(np.float32)
    kt = torch.from_numpy(keys).to(device, kv_dtype)
    return kt, k_proj, cb, kt.float().cpu().numpy()


def _encode(device, kt, k_proj, cb, code_dtype, ranges):
    from sva_amd import kernels

    H, R = k_proj.shape[0], k_proj.shape[2]
    N, S = kt.shape[1], cb.shape[1]
    k_low = torch.zeros(H, N, R, device=device)
    codes = torch.zeros(H, N, S, device=device, dtype=code_dtype)
    for a, b in ranges:
        kernels.write_encode(kt, torch.from_numpy(k_proj).to(device), torch.from_numpy(cb).to(device), k_low, codes,
                             a, b - a)
    torch.cuda.synchronize()
    return k_low.cpu().numpy(), codes.cpu().numpy().astype(np.int64)


@pytest.mark.parametrize("S,C,kv_dtype,code_dtype", [(2, 256, torch.float32, torch.uint8),
                                                     (4, 64, torch.bfloat16, torch.uint8),
                                                     (1, 256, torch.float32, torch.int64),
                                                     (8, 16, torch.bfloat16, torch.int32)])
def test_write_encode_matches_oracle(device, S, C, kv_dtype, code_dtype):
    N = 5000  # not a multiple of the 64-row tile
    kt, k_proj, cb, keys = _case(device, N, S, C, kv_dtype, seed=S * 7 + C)
    k_low, codes = _encode(device, kt, k_proj, cb, code_dtype, [(0, N)])
    H, G = k_proj.shape[0], keys.shape[0]
    ref_low = np.stack([oracle.project(keys[h // (H // G)], k_proj[h]) for h in range(H)])
    np.testing.assert_array_equal(k_low.view(np.uint32), ref_low.view(np.uint32))
    ref_codes, gaps = oracle.encode_product_keys(ref_low, cb, return_gap=True)
    diff = codes != ref_codes
    # a differing code is only allowed where two centroids are equally near to
    # within rounding (the oracle's gap between its best two distances)
    assert np.all(gaps[diff] <= 1e-4), f"codes differ away from near-ties: gaps {gaps[diff][:10]}"
    assert diff.sum() <= max(3, diff.size // 100000)


@pytest.mark.parametrize("D,R,S,C", [(8, 4, 2, 8), (16, 6, 3, 5), (48, 20, 5, 33)])
def test_write_encode_any_shape(device, D, R, S, C):
    # shapes off the tiled path (rank or sub-dimension not a multiple of 4)
    N = 300
    kt, k_proj, cb, keys = _case(device, N, S, C, torch.float32, seed=D + R, H=4, G=2, D=D, R=R)
    k_low, codes = _encode(device, kt, k_proj, cb, torch.uint8, [(0, 100), (100, N)])
    ref_low = np.stack([oracle.project(keys[h // 2], k_proj[h]) for h in range(4)])
    np.testing.assert_array_equal(k_low.view(np.uint32), ref_low.view(np.uint32))
    ref_codes, gaps = oracle.encode_product_keys(ref_low, cb, return_gap=True)
    diff = codes != ref_codes
    assert np.all(gaps[diff] <= 1e-4)


def test_write_append_equals_fresh(device):
    N, S, C = 3000, 2, 256
    kt, k_proj, cb, _ = _case(device, N, S, C, torch.bfloat16, seed=5)
    fresh = _encode(device, kt, k_proj, cb, torch.uint8, [(0, N)])
    parts = _encode(device, kt, k_proj, cb, torch.uint8, [(0, 1000), (1000, 1001), (1001, 2937), (2937, N)])
    for a, b in zip(fresh, parts):
        np.testing.assert_array_equal(a, b)


def test_write_ties_take_first_centroid(device):
    # duplicated codebook rows: every row's best distance is shared by two
    # centroids; the first index wins (torch.argmin)
    N, S, C = 700, 4, 16
    kt, k_proj, cb, keys = _case(device, N, S, C, torch.float32, seed=9)
    cb[:, :, 8:] = cb[:, :, :8]
    k_low, codes = _encode(device, kt, k_proj, cb, torch.uint8, [(0, N)])
    assert codes.max() < 8
    ref_codes = oracle.encode_product_keys(k_low, cb)
    np.testing.assert_array_equal(codes, ref_codes)


@pytest.mark.parametrize("S,C,kv_dtype,code_dtype,D,R", [(2, 256, torch.bfloat16, torch.uint8, 64, 64),
                                                         (4, 64, torch.float32, torch.uint8, 64, 64),
                                                         (1, 256, torch.float32, torch.int64, 128, 64),
                                                         (3, 5, torch.float32, torch.uint8, 16, 6)])
def test_decode_appends_equal_fresh(device, S, C, kv_dtype, code_dtype, D, R):
    # appends of 1 to 4 rows (a decode step's catalog append) give the fresh encode's bits and codes
    N = 211
    kt, k_proj, cb, _ = _case(device, N, S, C, kv_dtype, seed=S + C + D, H=6, G=3, D=D, R=R)
    fresh = _encode(device, kt, k_proj, cb, code_dtype, [(0, N)])
    ranges, a, k = [(0, 100)], 100, 0
    while a < N:
        b = min(N, a + 1 + k % 4)
        ranges.append((a, b))
        a, k = b, k + 1
    steps = _encode(device, kt, k_proj, cb, code_dtype, ranges)
    np.testing.assert_array_equal(fresh[0].view(np.uint32), steps[0].view(np.uint32))
    np.testing.assert_array_equal(fresh[1], steps[1])


def test_decode_append_ties_take_first_centroid(device):
    N, S, C = 40, 2, 256
    kt, k_proj, cb, _ = _case(device, N, S, C, torch.float32, seed=13)
    cb[:, :, 128:] = cb[:, :, :128]
    k_low, codes = _encode(device, kt, k_proj, cb, torch.uint8, [(a, a + 1) for a in range(N)])
    assert codes.max() < 128
    np.testing.assert_array_equal(codes, oracle.encode_product_keys(k_low, cb))


@pytest.mark.parametrize("S,C,kv_dtype,n_rows", [
    (2, 256, torch.bfloat16, 1),    # a decode step's append: every sequence in one launch
    (4, 64, torch.float32, 3),
    (2, 256, torch.float16, 100),   # more rows: the tiled encoder, one sequence a launch
])
def test_batch_encode_equals_each_sequence(device, S, C, kv_dtype, n_rows):
    """sva_write_encode_batch over a batch of 5 caches [B, G, rows, D] equals sva_write_encode run on each
    sequence's cache and catalog slice, bit for bit, and leaves every other catalog row untouched."""
    from sva_amd import kernels

    B, G, H, D, R, rows, cap, row0 = 5, 3, 9, 64, 64, 300, 320, 150
    g = torch.Generator(device=device).manual_seed(71 + n_rows)
    keys = torch.randn(B, G, rows, D, device=device, generator=g).to(kv_dtype)
    k_proj = torch.randn(H, D, R, device=device, generator=g) / 8.0
    cb = torch.randn(H, S, C, R // S, device=device, generator=g)
    k_low = torch.full((H, B * cap, R), 7.0, device=device)
    codes = torch.full((H, B * cap, S), 9, device=device, dtype=torch.uint8)
    ref_low, ref_codes = k_low.clone(), codes.clone()
    kernels.write_encode_batch(keys, k_proj, cb, k_low, codes, cap, row0, n_rows)
    for b in range(B):
        kernels.write_encode(keys[b], k_proj, cb, ref_low[:, b * cap:(b + 1) * cap], ref_codes[:, b * cap:(b + 1) * cap],
                             row0, n_rows)
    torch.cuda.synchronize()
    assert torch.equal(k_low, ref_low), "k_low differs"
    assert torch.equal(codes, ref_codes), "codes differ"
    assert bool((k_low[:, :row0] == 7.0).all()) and bool((codes[:, cap - 1] == 9).all()), "rows outside the range written"
