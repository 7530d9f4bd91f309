"""Pins the CPU oracle (no GPU).

Each oracle function is checked against something other than itself: torch-CPU
computing the reference's own expression (sva/ops.py, sva/llama.py) on the same
inputs, float64 closed forms, brute force on small inputs, invariants, and the
reference's known-answer test.  A deliberately wrong variant (a dropped term, a
swapped operand, the wrong tie order) fails at least one of these.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle

F32 = np.float32


def _bits(a):
    return np.ascontiguousarray(a, dtype=F32).view(np.uint32)


def _wide(rng, *shape):
    # values over six decades, so that every change of summation order shows
    return (rng.standard_normal(shape) * 10.0 ** rng.integers(-3, 4, shape)).astype(F32)


# ---------------------------------------------------------------------------
# arithmetic primitives


@pytest.mark.parametrize("n", [1, 2, 3, 4, 8, 9, 15, 16, 31, 32, 33, 63, 64, 65, 127, 128, 200, 255, 256, 511, 512,
                               1000, 2048, 4096, 20000, 32768])
def test_torch_sum_matches_torch_cpu(n):
    # torch.sum over fp32 (the reductions at sva/llama.py:292 and :314);
    # lengths 5..7 take another torch kernel, and single sums beyond 32768
    # elements split across threads: neither appears on the path (rows of 64)
    rng = np.random.default_rng(n)
    for _ in range(5):
        x = _wide(rng, n)
        assert _bits(oracle.torch_sum(x)) == _bits(torch.sum(torch.from_numpy(x)).numpy())


def test_rank_scores_match_reference_expression():
    # sva/llama.py:286-292: gather k_low rows, (rows * q_low).sum(-1) / sqrt(R)
    rng = np.random.default_rng(1)
    k_low = _wide(rng, 5000, 64)
    q = _wide(rng, 64)
    idx = rng.choice(5000, 2048, replace=False)
    ref = ((torch.from_numpy(k_low)[torch.from_numpy(idx)] * torch.from_numpy(q)).sum(-1) / math.sqrt(64)).numpy()
    np.testing.assert_array_equal(_bits(oracle.rank_scores(k_low, idx, q, 64)), _bits(ref))


def test_projection_matches_many_row_einsum():
    # sva/llama.py:615: k_low = einsum("bhnd,hdr->bhnr", K, k_proj) over the cache
    rng = np.random.default_rng(2)
    keys = rng.standard_normal((1, 9, 8192, 64)).astype(F32)
    proj = (rng.standard_normal((9, 64, 64)) / 8).astype(F32)
    ref = torch.einsum("bhnd,hdr->bhnr", torch.from_numpy(keys), torch.from_numpy(proj)).numpy()[0]
    mine = np.stack([oracle.project(keys[0, h], proj[h]) for h in range(9)])
    np.testing.assert_array_equal(_bits(mine), _bits(ref))


def _fp64_bound(terms64):
    # |fl(sum) - sum| <= (k * eps) * sum|terms| for any order of k fp32 terms
    k = terms64.shape[-1]
    return k * np.finfo(F32).eps * np.abs(terms64).sum(-1)


def test_query_low_and_lut_within_fp64_bound():
    # q_low (sva/llama.py:211) and the LUT (sva/ops.py:68) for a single query row:
    # MKL's single-row kernel rounds in its own order, so the bits are held to
    # the float64 result within the order-independent bound instead
    rng = np.random.default_rng(3)
    q = rng.standard_normal((9, 1, 64)).astype(F32)
    proj = (rng.standard_normal((9, 64, 64)) / 8).astype(F32)
    scale = np.exp(rng.uniform(-1, 1, 9)).astype(F32)
    ql = oracle.query_low(q, proj, scale)
    terms = q[:, 0, :, None].astype(np.float64) * proj.astype(np.float64)  # [H, D, R]
    exact = terms.sum(1) * scale[:, None]
    bound = _fp64_bound(np.swapaxes(terms, 1, 2)) * scale[:, None] * (1 + 1e-6) + np.abs(exact) * 2 ** -23
    assert np.all(np.abs(ql[:, 0] - exact) <= bound)
    torch_ref = (torch.einsum("bhtd,hdr->bhtr", torch.from_numpy(q[None]), torch.from_numpy(proj))
                 * torch.from_numpy(scale).view(1, 9, 1, 1)).numpy()[0]
    assert np.all(np.abs(ql - torch_ref) <= 2 * bound[:, None])
    cb = rng.standard_normal((9, 2, 256, 32)).astype(F32)
    for h in range(9):
        table = oracle.lut(ql[h, 0], cb[h])
        t = cb[h].astype(np.float64) * ql[h, 0].reshape(2, 1, 32).astype(np.float64)  # [S, C, sub]
        assert np.all(np.abs(table - t.sum(-1)) <= _fp64_bound(t))
        for s in range(2):
            ref = torch.matmul(torch.from_numpy(ql[h, :, s * 32:(s + 1) * 32]), torch.from_numpy(cb[h, s]).T).numpy()[0]
            assert np.all(np.abs(table[s] - ref) <= 2 * _fp64_bound(t[s]))


def test_scan_scores_match_reference_expression():
    # sva/ops.py:64-71: scores = zeros; scores += lut[s][codes[:, s]] for s in order; / sqrt(R)
    rng = np.random.default_rng(4)
    for S, C in ((1, 256), (2, 256), (4, 64), (8, 16)):
        table = _wide(rng, S, C)
        codes = rng.integers(0, C, (10000, S))
        scores = torch.zeros(10000)
        lut_t = torch.from_numpy(table)
        codes_t = torch.from_numpy(codes)
        for s in range(S):
            scores = scores + lut_t[s][codes_t[:, s]]
        ref = (scores / math.sqrt(64)).numpy()
        got = oracle.pq_scores_from_lut(table, codes, 64)
        np.testing.assert_array_equal(_bits(got), _bits(ref))
        # invariant: keys with identical codes score identically
        dup = codes.copy()
        dup[5000:] = dup[:5000]
        g2 = oracle.pq_scores_from_lut(table, dup, 64)
        np.testing.assert_array_equal(_bits(g2[5000:]), _bits(g2[:5000]))


def test_assign_matches_reference_formula_and_brute_force():
    # sva/ops.py:10-21: ||x||^2 - 2 x.C^T + ||c||^2, argmin (first on ties)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8192, 32)).astype(F32)
    cb = rng.standard_normal((256, 32)).astype(F32)
    labels, gap = oracle.assign_to_centroids(x, cb, return_gap=True)
    xt, ct = torch.from_numpy(x), torch.from_numpy(cb)
    dist = (xt * xt).sum(-1, keepdim=True) - 2.0 * (xt @ ct.T) + (ct * ct).sum(-1).unsqueeze(0)
    ref = dist.argmin(-1).numpy()
    close = gap <= 8 * np.finfo(F32).eps * np.abs(dist.numpy()).max(-1)
    assert np.all((labels == ref) | close)
    assert (labels != ref).sum() <= 2
    # brute force in float64, away from near-ties
    d64 = ((x[:, None, :].astype(np.float64) - cb[None].astype(np.float64)) ** 2).sum(-1)
    best = d64.argmin(-1)
    srt = np.sort(d64, -1)
    clear = (srt[:, 1] - srt[:, 0]) > 1e-3
    np.testing.assert_array_equal(labels[clear], best[clear])
    # ties: the first minimum wins
    cb2 = np.concatenate([cb[:4], cb[:4]])
    lab2 = oracle.assign_to_centroids(x[:100], cb2)
    assert np.all(lab2 < 4)


def test_encode_product_keys_rejects_bad_rank():
    with pytest.raises(ValueError):
        oracle.encode_product_keys(np.zeros((1, 4, 6), F32), np.zeros((1, 4, 8, 1), F32))


# ---------------------------------------------------------------------------
# selection


def _lexsort_topk(scores, k, allowed=None):
    idx = np.arange(len(scores))
    if allowed is not None:
        idx = idx[allowed]
    order = np.lexsort((idx, -scores[idx].astype(np.float64)))
    return idx[order[:k]]


def test_topk_rule_against_lexsort_and_stable_sort():
    rng = np.random.default_rng(6)
    for n, k, distinct in ((1000, 100, 7), (5000, 2048, 50), (300, 2048, 3), (4096, 1, 2), (10000, 512, 100000)):
        scores = rng.integers(0, distinct, n).astype(F32) / 4
        got = oracle.topk(scores, k)
        np.testing.assert_array_equal(got, _lexsort_topk(scores, k))
        ref = torch.sort(torch.from_numpy(scores), descending=True, stable=True).indices[:k].numpy()
        np.testing.assert_array_equal(got, ref)
        allowed = rng.random(n) < 0.4
        np.testing.assert_array_equal(oracle.topk(scores, k, allowed=allowed), _lexsort_topk(scores, k, allowed))
    # key_index remaps the tie rule
    scores = np.array([1, 1, 1, 0], F32)
    assert oracle.topk(scores, 2, key_index=np.array([9, 3, 5, 0])).tolist() == [1, 2]


def test_top_unique_candidates_known_answer():
    # tests/test_sva_llama_adapter.py:58-73 of the reference
    sel, sc, valid, refill = oracle.top_unique_candidates([4, 4, 3, 3, 2, 1], [9.0, 8.5, 8.0, 7.5, 7.0, 6.0],
                                                          [True] * 6, budget=3, refill_factor=2)
    assert refill == 6
    assert sel[valid].tolist() == [4, 3, 2]
    assert sc[valid].tolist() == [9.0, 8.0, 7.0]


def test_top_unique_candidates_brute_force():
    rng = np.random.default_rng(7)
    for trial in range(200):
        w = int(rng.integers(1, 40))
        budget = int(rng.integers(1, 12))
        ids = rng.integers(0, 15, w)
        scores = rng.integers(0, 6, w).astype(F32)
        valid = rng.random(w) < 0.8
        sel, sc, ok, refill = oracle.top_unique_candidates(ids, scores, valid, budget)
        assert refill == min(w, max(budget, 2 * budget))
        # brute force: refill window by (masked score desc, id asc), first occurrence of each id,
        # valid ones only, then the best `budget` of those by the same rule
        masked = np.where(valid, scores, np.finfo(F32).min)
        order = np.lexsort((ids, -masked.astype(np.float64)))[:refill]
        seen, cand = set(), []
        for i in order:
            if ids[i] in seen:
                continue
            seen.add(ids[i])
            if valid[i]:
                cand.append((float(masked[i]), int(ids[i])))
        cand.sort(key=lambda t: (-t[0], t[1]))
        want = cand[:min(budget, refill)]
        assert [int(v) for v in sel[ok]] == [i for _, i in want]
        assert [float(v) for v in sc[ok]] == [s for s, _ in want]
        assert len(sel) == min(budget, refill)


# ---------------------------------------------------------------------------
# verifier and index


def test_verify_matches_float64_softmax():
    rng = np.random.default_rng(8)
    keys = rng.standard_normal((3, 4096, 64)).astype(F32)
    values = rng.standard_normal((3, 4096, 64)).astype(F32)
    q = rng.standard_normal(64).astype(F32)
    idx = rng.choice(4096, 512, replace=False)
    got = oracle.verify(q, keys[1], values[1], idx, 64 ** -0.5)
    k = torch.from_numpy(keys[1]).double()[torch.from_numpy(idx)]
    v = torch.from_numpy(values[1]).double()[torch.from_numpy(idx)]
    w = torch.softmax((k @ torch.from_numpy(q).double()) * 64 ** -0.5, 0)
    np.testing.assert_allclose(got, (w @ v).numpy(), rtol=1e-12, atol=1e-12)
    # a single key returns its value exactly
    np.testing.assert_allclose(oracle.verify(q, keys[0], values[0], np.array([7]), 0.125), values[0, 7], rtol=0)


def test_rebuild_postings_invariants():
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 16, (3, 5000, 2))
    counts, offsets, ids = oracle.rebuild_postings(codes, 16)
    for h in range(3):
        for s in range(2):
            np.testing.assert_array_equal(counts[h, s], np.bincount(codes[h, :, s], minlength=16))
            assert offsets[h, s, 0] == 0 and offsets[h, s, -1] == 5000
            np.testing.assert_array_equal(np.sort(ids[h, s]), np.arange(5000))  # a partition
            for c in range(16):
                cell = ids[h, s, offsets[h, s, c]:offsets[h, s, c + 1]]
                assert np.all(codes[h, cell, s] == c)
                assert np.all(np.diff(cell) > 0)  # ascending key id within a cell


def test_allowed_mask_rules():
    # sva/llama.py:188-198: causal with query positions [N - Q, N); additive masks > -1e4;
    # a bool mask compares True/False > -1e4, which is always true
    m = oracle.allowed_mask(3, 10)
    assert m.sum(1).tolist() == [8, 9, 10]
    add = np.zeros((1, 1, 2, 5), F32)
    add[..., 1] = np.finfo(F32).min
    assert oracle.allowed_mask(2, 5, add).sum() == 8
    assert oracle.allowed_mask(2, 5, np.zeros((1, 1, 2, 5), bool)).all()


def test_decode_in_c_matches_numpy_restatement():
    # the OpenMP C decode (the CPU baseline) against the numpy path built from the
    # pinned pieces above
    rng = np.random.default_rng(10)
    H, G, N, D, R, S, C = 9, 3, 6000, 64, 64, 2, 256
    q = rng.standard_normal((H, D)).astype(F32)
    keys = rng.standard_normal((G, N, D)).astype(F32)
    values = rng.standard_normal((G, N, D)).astype(F32)
    k_low = rng.standard_normal((H, N, R)).astype(F32)
    q_low = rng.standard_normal((H, R)).astype(F32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(F32)
    codes = rng.integers(0, C, (H, N, S)).astype(np.uint8)
    sl, fin, out, _ = oracle.decode(q, q_low, keys, values, k_low, cb, codes, 1024, 256, D ** -0.5)
    for h in range(H):
        scores = oracle.pq_scores_from_lut(oracle.lut(q_low[h], cb[h]), codes[h], R)
        short = oracle.topk(scores, 1024)
        assert set(sl[h].tolist()) == set(short.tolist())
        rank = oracle.rank_scores(k_low[h], short, q_low[h], R)
        final = short[oracle.topk(rank, 256, key_index=short)]
        assert set(fin[h].tolist()) == set(final.tolist())
        ref = oracle.verify(q[h], keys[h // 3], values[h // 3], np.sort(final), D ** -0.5)
        np.testing.assert_allclose(out[h], ref, rtol=1e-12, atol=1e-12)
    # the same cache held in arrays with spare rows (a growing cache read in place)
    cap = N + 37
    pad = lambda a: np.concatenate([a, np.full((a.shape[0], cap - N) + a.shape[2:], 7, a.dtype)], axis=1)  # noqa
    sl2, fin2, out2, _ = oracle.decode(q, q_low, pad(keys), pad(values), pad(k_low), cb, pad(codes), 1024, 256,
                                       D ** -0.5, n_keys=N)
    np.testing.assert_array_equal(sl2, sl)
    np.testing.assert_array_equal(fin2, fin)
    np.testing.assert_array_equal(out2, out)


def test_residual_adapter_matches_torch_module():
    # the reference's module (nn.Linear without bias, F.gelu) in float64 on the CPU
    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(4)
    T, H, rank = 7, 24, 4
    hidden = rng.standard_normal((T, H))
    attn = rng.standard_normal((T, H))
    down = rng.standard_normal((rank, 2 * H)) * 0.3
    up = rng.standard_normal((H, rank)) * 0.3
    got = oracle.residual_adapter(hidden, attn, down, up, 0.5)
    x = torch.cat([torch.from_numpy(hidden), torch.from_numpy(attn)], dim=-1)
    want = torch.from_numpy(attn) + F.linear(F.gelu(F.linear(x, torch.from_numpy(down))), torch.from_numpy(up)) * 0.5
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)
    # the reference initialises up to zero: the adapter starts as the identity
    np.testing.assert_array_equal(oracle.residual_adapter(hidden, attn, down, np.zeros_like(up), 1.0), attn)
    # gelu at known points: 0 -> 0, large -> identity, -large -> 0
    one = np.ones((1, 1))
    for v, expect in ((0.0, 0.0), (40.0, 40.0), (-40.0, 0.0)):
        out = oracle.residual_adapter(one, np.zeros((1, 1)), np.array([[v, 0.0]]), one, 1.0)  # pre-activation v
        assert abs(out[0, 0] - expect) < 1e-12


def test_kmeans_update_matches_torch_cpu_step():
    # the reference's update body run by torch on the CPU (index_add_ sums in row order)
    import torch

    rng = np.random.default_rng(8)
    N, C, sub = 500, 16, 8
    x = rng.standard_normal((N, sub)).astype(np.float32)
    labels = rng.integers(0, C - 2, N)  # cells C-2, C-1 empty: they keep their centroid
    cent = rng.standard_normal((C, sub)).astype(np.float32)
    w = rng.random(N).astype(np.float32) + 0.1
    xt, lt, ct, wt = map(torch.from_numpy, (x, labels, cent, w))
    sums = torch.zeros(C, sub)
    sums.index_add_(0, lt, xt)
    counts = torch.bincount(lt, minlength=C)
    want = ct.clone()
    ne = counts > 0
    want[ne] = sums[ne] / counts[ne].float()[:, None]
    got = oracle.kmeans_update(x, labels, cent)
    np.testing.assert_array_equal(got.view(np.uint32), want.numpy().view(np.uint32))
    np.testing.assert_array_equal(got[C - 2:], cent[C - 2:])
    sums = torch.zeros(C, sub)
    sums.index_add_(0, lt, xt * wt[:, None])
    counts = torch.zeros(C)
    counts.index_add_(0, lt, wt)
    want = ct.clone()
    ne = counts > 0
    want[ne] = sums[ne] / counts[ne, None]
    got = oracle.kmeans_update(x, labels, cent, w)
    np.testing.assert_array_equal(got.view(np.uint32), want.numpy().view(np.uint32))
