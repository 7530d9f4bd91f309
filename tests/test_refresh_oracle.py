"""The oracle's codebook-refresh helpers pinned on the CPU
(experiments/sva_codebook_refresh_benchmark.py:136-153,
experiments/sva_rotation_diagnostic.py:86-116,
experiments/export_refreshed_sva_artifact.py:98-104): key weights against
their closed form and torch-CPU's index_add_, top-k targets against a brute
force per row, query positions against torch.linspace."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


def _weights_index_add(top_idx, top_valid, seq_len, boost):
    # the reference's expression, run by torch on the CPU
    idx, valid = torch.from_numpy(top_idx), torch.from_numpy(top_valid)
    w = torch.ones(idx.shape[0], seq_len, dtype=torch.float32)
    for h in range(idx.shape[0]):
        hits = idx[h][valid[h]]
        if hits.numel():
            w[h].index_add_(0, hits.long().clamp(0, seq_len - 1),
                            torch.full((hits.numel(),), float(boost), dtype=torch.float32))
    return w.numpy()


@pytest.mark.parametrize("boost", [4.0, 0.1, 16.0, 1e-3])
def test_key_weights_closed_form_and_index_add(boost):
    rng = np.random.default_rng(7)
    H, Q, K, N = 3, 40, 12, 500
    top_idx = rng.integers(-5, N + 5, (H, Q, K))  # out-of-range entries are clamped
    top_idx[1, :, 0] = 17                         # one key hit by every query
    top_valid = rng.random((H, Q, K)) < 0.8
    top_valid[1, :, 0] = True
    top_valid[2] = False                          # a head with no valid hit
    got = oracle.topk_key_weights(top_idx, top_valid, N, boost)
    np.testing.assert_array_equal(got.view(np.uint32), _weights_index_add(top_idx, top_valid, N, boost).view(np.uint32))
    # closed form: c hits give the c-fold rounded sum
    for h in range(H):
        counts = np.bincount(np.clip(top_idx[h][top_valid[h]], 0, N - 1), minlength=N)
        for n in np.flatnonzero(counts)[:50]:
            v = np.float32(1.0)
            for _ in range(counts[n]):
                v = np.float32(v + np.float32(boost))
            assert got[h, n] == v
    assert np.all(got[2] == 1.0)
    assert got[1, 17] >= 1.0 + boost * Q * 0.99


def test_key_weights_rounding_order_matters():
    # 30 rounded adds of 0.1 differ from 1 + 30 * 0.1 rounded once: a kernel
    # that multiplied the hit count would fail the GPU test
    top_idx = np.full((1, 30, 1), 3)
    top_valid = np.ones((1, 30, 1), bool)
    w = oracle.topk_key_weights(top_idx, top_valid, 8, 0.1)
    assert w[0, 3] != np.float32(1.0 + np.float32(0.1) * np.float32(30))


def test_topk_targets_brute_force():
    rng = np.random.default_rng(3)
    H, N, k = 2, 60, 8
    pos = np.array([0, 3, 7, 8, 30, 59])
    scores = rng.standard_normal((H, len(pos), N)).astype(np.float32)
    scores[0, 4, 5] = scores[0, 4, 9]  # a tie: lower key first
    idx, valid = oracle.topk_targets(scores, pos, k)
    assert idx.shape == valid.shape == (H, len(pos), k)
    for h in range(H):
        for r, p in enumerate(pos):
            visible = np.arange(p + 1)
            order = visible[np.lexsort((visible, -scores[h, r, visible].astype(np.float64)))]
            nv = min(k, p + 1)
            assert valid[h, r].sum() == nv and np.all(valid[h, r, :nv])
            np.testing.assert_array_equal(idx[h, r, :nv], order[:nv])
            assert np.all(idx[h, r, :nv] <= p)


@pytest.mark.parametrize("n", [1, 2, 7, 128, 129, 5000, 32768])
def test_query_positions_match_linspace(n):
    for samples in (1, 3, 64, 128, 4096):
        for min_pos in (-1, 0, 5, 128, 10 ** 6):
            start = max(0, min(min_pos, n - 1))
            want = torch.linspace(start, n - 1, steps=min(samples, n)).long().unique().numpy()
            np.testing.assert_array_equal(oracle.query_positions(n, samples, min_pos), want)
