"""GPU parity of the product-codebook fits (sva_amd.codebooks) with the
oracle's restatement of the reference's k-means
(experiments/sva_pq_lookup_test.py:66-106, experiments/sva_supervised_coarse_pq_test.py:88-131).

The centroid update is bit-exact with the oracle on the same labels (cell
sums in ascending row order, plain and weighted, empty cells kept).  Whole
fits from the same initial centroids match the oracle's fit; a label can
only differ where two centroids are equally near within rounding (the
assignment's own rule, tested in test_gpu_write.py), so centroids are
compared to 1e-5 and most must be bit-identical.  The seeded default
initialisation is deterministic on the device.
"""

from __future__ import annotations


import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _data(seed, H=3, N=3000, R=64):
    rng = np.random.default_rng(seed)
    return rng, rng.standard_normal((H, N, R)).astype(np.float32)


@pytest.mark.parametrize("weighted", [False, True])
def test_centroid_update_bit_exact(device, weighted):
    from sva_amd import inverted, kernels
    from sva_amd._lib import lib, ptr, stream_handle

    rng, x = _data(3 + weighted)
    H, N, R = x.shape
    S, C = 2, 64
    sub = R // S
    cent = rng.standard_normal((H, S, C, sub)).astype(np.float32)
    cent[:, :, -3:] += 50.0  # far away: empty cells, which keep their centroid
    w = (rng.random((H, N)) + 0.05).astype(np.float32) if weighted else None
    xt = torch.from_numpy(x).to(device)
    ct = torch.from_numpy(cent).to(device)
    eye = torch.eye(R, device=device).expand(H, R, R).contiguous()
    codes = torch.empty(H, N, S, device=device, dtype=torch.uint8)
    kernels.write_encode(xt, eye, ct, torch.empty_like(xt), codes)
    post = inverted.build_postings(codes, N, C)
    nxt = torch.empty_like(ct)
    wt = torch.from_numpy(w).to(device) if weighted else None
    assert lib().sva_centroid_update(ptr(xt), xt.stride(0), N, H, R, S, C, ptr(wt), ptr(post.offsets),
                                     ptr(post.ids), ptr(ct), ptr(nxt), stream_handle(device)) == 0
    got = nxt.cpu().numpy()
    labels = codes.cpu().numpy().astype(np.int64)
    for h in range(H):
        for s in range(S):
            want = oracle.kmeans_update(x[h, :, s * sub:(s + 1) * sub], labels[h, :, s], cent[h, s],
                                        None if w is None else w[h])
            np.testing.assert_array_equal(got[h, s].view(np.uint32), want.view(np.uint32), err_msg=f"{h} {s}")
    np.testing.assert_array_equal(got[:, :, -3:], cent[:, :, -3:])


@pytest.mark.parametrize("weighted,S,C", [(False, 2, 64), (True, 4, 16)])
def test_fit_matches_oracle(device, weighted, S, C):
    from sva_amd import codebooks

    rng, x = _data(11 + C)
    H, N, R = x.shape
    sub = R // S
    init = np.stack([np.stack([x[h, rng.choice(N, C, replace=False), s * sub:(s + 1) * sub] for s in range(S)])
                     for h in range(H)])
    w = (rng.random((H, N)) * 3).astype(np.float32) if weighted else None
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    if weighted:
        got = codebooks.fit_weighted_product_codebooks(t(x), t(w), S, C, 4, seed=0, initial=t(init))
    else:
        got = codebooks.fit_product_codebooks(t(x), S, C, 4, seed=0, initial=t(init))
    got = got.cpu().numpy()
    want = oracle.kmeans_fit(x, S, 4, init, w)
    assert got.shape == want.shape == (H, S, C, sub)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
    same = np.all(got.view(np.uint32) == want.view(np.uint32), axis=-1)
    assert same.mean() >= 0.95, f"only {same.mean():.3f} of the centroids are bit-identical"


def test_default_initialisation_is_seeded(device):
    from sva_amd import codebooks

    _, x = _data(5, H=2, N=600)
    xt = torch.from_numpy(x).to(device)
    a = codebooks.fit_product_codebooks(xt, 2, 256, 2, seed=7)
    b = codebooks.fit_product_codebooks(xt, 2, 256, 2, seed=7)
    assert a.shape == (2, 2, 256, 32)
    assert torch.equal(a, b)
    small = codebooks.fit_product_codebooks(xt[:, :100], 2, 256, 1, seed=7)
    assert small.shape == (2, 2, 100, 32)  # min(codewords, rows) as the reference
