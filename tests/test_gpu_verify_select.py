"""GPU parity of the budget select and the GQA verifier on their own.

Budget select: exact top-B by (rank desc, key index asc) as ascending key
indices, bit-exact with the oracle, including tied ranks and counts below B.
Verifier: within 1e-5 (fp32 K/V) / 2e-2 (bf16, fp16) of the float64 oracle,
relative to the output's max magnitude, for head_dim 48 / 64 / 128, groups of
1, 3 and 8 query heads per KV head, lists that overlap inside a group (the
shared rows are read once and must still count once per head), short and
empty lists, and ragged sequences packed back to back.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _lists(rng, heads, groups, n, budget, counts, overlap):
    grp = heads // groups
    idx = np.zeros((heads, budget), np.int32)
    for g in range(groups):
        base = rng.choice(n, min(n, budget), replace=False)
        for j in range(grp):
            h = g * grp + j
            c = counts[h]
            own = rng.choice(n, c, replace=False)
            k = int(overlap * c)
            pick = np.unique(np.concatenate([base[:k], own]))[:c]
            if len(pick) < c:
                extra = np.setdiff1d(np.arange(n), pick)[: c - len(pick)]
                pick = np.concatenate([pick, extra])
            idx[h, :c] = np.sort(pick)
            idx[h, c:] = rng.integers(-5, n + 5, budget - c)  # slots past the count are never read
    return idx


@pytest.mark.parametrize("D,H,G,dtype", [(64, 9, 3, torch.float32), (64, 9, 3, torch.bfloat16),
                                         (128, 8, 1, torch.float16), (48, 8, 8, torch.float32),
                                         (128, 16, 2, torch.bfloat16), (8, 4, 2, torch.float32),
                                         (40, 6, 3, torch.bfloat16)])
def test_verify_matches_oracle(device, D, H, G, dtype):
    from sva_amd import kernels

    rng = np.random.default_rng(D + H + G)
    n, budget = 5000, 512
    counts = rng.integers(0, budget + 1, H)
    counts[0], counts[-1] = budget, 0
    fin = _lists(rng, H, G, n, budget, counts, overlap=0.6)
    q = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    keys = rng.standard_normal((G, n, D)).astype(np.float32)
    values = rng.standard_normal((G, n, D)).astype(np.float32)
    kt = torch.from_numpy(keys).to(device, dtype)
    vt = torch.from_numpy(values).to(device, dtype)
    qt = torch.from_numpy(q).to(device, dtype)
    out = kernels.verify(qt, kt, vt, torch.from_numpy(fin).to(device), torch.from_numpy(counts.astype(np.int32)).to(device),
                         n, D ** -0.5).float().cpu().numpy()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    kq, vq, qq = kt.float().cpu().numpy(), vt.float().cpu().numpy(), qt.float().cpu().numpy()
    grp = H // G
    for h in range(H):
        c = int(counts[h])
        if c == 0:
            assert np.all(out[0, h, 0] == 0)
            continue
        ref = oracle.verify(qq[0, h, 0], kq[h // grp], vq[h // grp], fin[h, :c], D ** -0.5)
        err = np.abs(out[0, h, 0] - ref).max() / np.abs(ref).max()
        assert err <= tol, f"head {h}: rel err {err}"


@pytest.mark.parametrize("budget,dtype", [(2048, torch.bfloat16), (2049, torch.bfloat16), (3000, torch.float32),
                                          (1, torch.float32), (33, torch.float16)])
def test_verify_budget_sizes(device, budget, dtype):
    # one workgroup per item up to 2048 rows (a 2048-row list is 16 rounds per wave), the slice-split form
    # beyond; a one-row list and a list shorter than a round
    from sva_amd import kernels

    rng = np.random.default_rng(budget)
    H, G, D, n = 9, 3, 64, 6000
    counts = rng.integers(0, budget + 1, H)
    counts[0], counts[1] = budget, min(budget, 7)
    fin = _lists(rng, H, G, n, budget, counts, overlap=0.3)
    q = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    keys = rng.standard_normal((G, n, D)).astype(np.float32)
    values = rng.standard_normal((G, n, D)).astype(np.float32)
    kt, vt, qt = (torch.from_numpy(a).to(device, dtype) for a in (keys, values, q))
    out = kernels.verify(qt, kt, vt, torch.from_numpy(fin).to(device), torch.from_numpy(counts.astype(np.int32)).to(device),
                         n, D ** -0.5).float().cpu().numpy()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    kq, vq, qq = kt.float().cpu().numpy(), vt.float().cpu().numpy(), qt.float().cpu().numpy()
    for h in range(H):
        c = int(counts[h])
        if c == 0:
            assert np.all(out[0, h, 0] == 0)
            continue
        ref = oracle.verify(qq[0, h, 0], kq[h // 3], vq[h // 3], fin[h, :c], D ** -0.5)
        err = np.abs(out[0, h, 0] - ref).max() / np.abs(ref).max()
        assert err <= tol, f"budget {budget} head {h} ({c} rows): rel err {err}"


@pytest.mark.parametrize("Q", [2, 400])  # 400: 3200 (sequence, KV head, token) groups, one wave per item
def test_verify_ragged_sequences(device, Q):
    from sva_amd import kernels

    rng = np.random.default_rng(3 + Q)
    lens = np.array([700, 1, 2500, 64], np.int64)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    H, G, D, budget = 6, 2, 64, 128
    rows = int(lens.sum())
    keys = rng.standard_normal((G, rows, D)).astype(np.float32)
    values = rng.standard_normal((G, rows, D)).astype(np.float32)
    q = rng.standard_normal((len(lens), H, Q, D)).astype(np.float32)
    items = len(lens) * H * Q
    fin = np.zeros((items, budget), np.int32)
    cnt = np.zeros(items, np.int32)
    for b in range(len(lens)):
        for h in range(H):
            for t in range(Q):
                it = (b * H + h) * Q + t
                c = max(0, min(budget, int(lens[b]) - t))
                cnt[it] = c
                fin[it, :c] = np.sort(rng.choice(int(lens[b]), c, replace=False))
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    out = kernels.verify(t(q), t(keys), t(values), t(fin), t(cnt), int(lens.max()), D ** -0.5,
                         seq_offsets=t(offs), seq_lens=t(lens)).cpu().numpy()
    grp = H // G
    for b in range(len(lens)):
        kb = keys[:, offs[b]:offs[b] + lens[b]]
        vb = values[:, offs[b]:offs[b] + lens[b]]
        for h in range(H):
            for tt in range(Q):
                it = (b * H + h) * Q + tt
                if cnt[it] == 0:
                    assert np.all(out[b, h, tt] == 0)
                    continue
                ref = oracle.verify(q[b, h, tt], kb[h // grp], vb[h // grp], fin[it, :cnt[it]], D ** -0.5)
                err = np.abs(out[b, h, tt] - ref).max() / np.abs(ref).max()
                assert err <= 1e-5, f"seq {b} head {h} token {tt}: rel err {err}"


@pytest.mark.parametrize("L,B,distinct", [(2048, 512, 1 << 30), (2048, 512, 40), (700, 97, 3), (300, 512, 1 << 30),
                                          (4096, 1, 5), (8192, 2048, 1 << 30), (16384, 8192, 1000),
                                          (16384, 1000, 1 << 30)])
def test_budget_select_matches_oracle(device, L, B, distinct):
    from sva_amd import kernels

    rng = np.random.default_rng(L + B)
    items = 9
    counts = np.full(items, L, np.int32)
    counts[1] = L // 3
    counts[2] = 0
    idx = np.stack([rng.permutation(10 * L)[:L] for _ in range(items)]).astype(np.int32)
    if distinct < (1 << 30):
        rank = (rng.integers(0, distinct, (items, L)) / 4).astype(np.float32)
    else:
        rank = rng.standard_normal((items, L)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    fin, fcnt = kernels.budget_select(t(idx), t(rank), t(counts), B)
    fin, fcnt = fin.cpu().numpy(), fcnt.cpu().numpy()
    for it in range(items):
        c = int(counts[it])
        keep = oracle.topk(rank[it, :c], min(B, c), key_index=idx[it, :c])
        want = np.sort(idx[it, :c][keep])
        assert fcnt[it] == len(want)
        np.testing.assert_array_equal(fin[it, :len(want)], want)


@pytest.mark.parametrize("D,H,G,Q,dtype", [(64, 9, 3, 700, torch.float32), (64, 9, 3, 700, torch.bfloat16),
                                           (128, 8, 2, 1030, torch.float32), (128, 8, 2, 1030, torch.float16),
                                           (40, 6, 3, 690, torch.float32)])
def test_verify_many_tokens_walks_slices(device, D, H, G, Q, dtype):
    # 2048 or more (KV head, token) groups: one wave per item (head_dim 64
    # and 128) or one workgroup walking all slices of its group (other head
    # dims), each with running maxima; checked against the oracle per item
    # and against the same tokens verified in calls of 16 tokens (the
    # slice-split form with its combine kernel)
    from sva_amd import kernels

    rng = np.random.default_rng(D + Q)
    n, budget = 3000, 512
    grp = H // G
    fin = np.zeros((H, Q, budget), np.int32)
    counts = np.zeros((H, Q), np.int64)
    for t in range(Q):
        c = rng.integers(0, budget + 1, H)
        c[0] = budget
        if t % 7 == 0:
            c[:] = 0 if t % 14 == 0 else c  # some tokens with no entries at all
        counts[:, t] = c
        fin[:, t] = _lists(rng, H, G, n, budget, c, overlap=0.5)
    q = rng.standard_normal((1, H, Q, D)).astype(np.float32)
    keys = rng.standard_normal((G, n, D)).astype(np.float32)
    values = rng.standard_normal((G, n, D)).astype(np.float32)
    kt, vt, qt = (torch.from_numpy(a).to(device, dtype) for a in (keys, values, q))
    fin_t = torch.from_numpy(fin.reshape(H * Q, budget)).to(device)
    cnt_t = torch.from_numpy(counts.reshape(H * Q).astype(np.int32)).to(device)
    out = kernels.verify(qt, kt, vt, fin_t, cnt_t, n, D ** -0.5).float().cpu().numpy()
    parts = []
    for t0 in range(0, Q, 16):
        t1 = min(Q, t0 + 16)
        sel = (np.arange(H)[:, None] * Q + np.arange(t0, t1)[None, :]).reshape(-1)
        sel_t = torch.from_numpy(sel).to(device)
        parts.append(kernels.verify(qt[:, :, t0:t1], kt, vt, fin_t[sel_t].contiguous(), cnt_t[sel_t].contiguous(), n,
                                    D ** -0.5).float().cpu().numpy())
    split = np.concatenate(parts, axis=2)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    kq, vq, qq = kt.float().cpu().numpy(), vt.float().cpu().numpy(), qt.float().cpu().numpy()
    scale = np.maximum(np.abs(split).max(axis=-1, keepdims=True), 1e-30)
    assert np.all(np.abs(out - split) / scale <= tol), "walking form differs from the split form"
    for h in range(H):
        for t in list(range(0, Q, 37)) + [Q - 1]:
            c = int(counts[h, t])
            if c == 0:
                assert np.all(out[0, h, t] == 0)
                continue
            ref = oracle.verify(qq[0, h, t], kq[h // grp], vq[h // grp], fin[h, t, :c], D ** -0.5)
            err = np.abs(out[0, h, t] - ref).max() / np.abs(ref).max()
            assert err <= tol, f"head {h} token {t}: rel err {err}"
