"""GPU parity of the long-context q=1 summon (many workgroups per query item).

Shortlists over caches of 64K..1M keys are compared as SETS, bit-exact, with
the oracle's top-L on the same LUT (selection rule: score desc, key index
asc); rank scores bit-exact; the wide path must also agree with the
one-workgroup-per-item path on the same inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _setup(device, N, S, C, H=9, R=64, seed=0, few=False):
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    codes = rng.integers(0, 3 if few else C, size=(H, N, S), dtype=np.uint8)
    k_low = torch.randn(H, N, R, device=device, generator=gen)
    q = rng.standard_normal((H, 1, 64)).astype(np.float32)
    q_proj = (rng.standard_normal((H, 64, R)) / 8).astype(np.float32)
    scale = np.ones(H, np.float32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(np.float32)
    return codes, k_low, q, q_proj, scale, cb


def _summon(device, codes, k_low, q, q_proj, scale, cb, L, mask=None):
    from sva_amd import kernels

    codes_t = torch.from_numpy(codes).to(device)
    q_low, lut, rng = kernels.query_lut(torch.from_numpy(q).to(device), torch.from_numpy(q_proj).to(device),
                                        torch.from_numpy(scale).to(device), torch.from_numpy(cb).to(device),
                                        codes_t, codes.shape[1], L)
    sl_idx, sl_rank, sl_count = kernels.summon(lut, rng, q_low, codes_t, k_low, codes.shape[1], L, mask=mask)
    torch.cuda.synchronize()
    return q_low[0, :, 0].cpu().numpy(), lut[0, :, 0].cpu().numpy(), sl_idx.cpu().numpy(), sl_rank.cpu().numpy(), \
        sl_count.cpu().numpy()


def _strategy(H, N, R, S, C, L, mask_type=0):
    from sva_amd import _lib

    return _lib.lib().sva_summon_strategy(1, H, 1, N, R, S, C, L, 0, mask_type)


def _check(codes, k_low, q_low, lut, sl_idx, sl_rank, sl_count, L, allowed=None):
    H, N, _ = codes.shape
    for h in range(H):
        scores = oracle.pq_scores_from_lut(lut[h], codes[h], 64)
        sl = oracle.topk(scores, L, allowed=allowed)
        cnt = int(sl_count[h])
        assert cnt == len(sl)
        got = sl_idx[h, :cnt].astype(np.int64)
        assert len(np.unique(got)) == cnt, "duplicate shortlist entries"
        assert set(got.tolist()) == set(sl.tolist()), f"head {h}: shortlist set differs"
        rows = k_low[h, torch.from_numpy(got).to(k_low.device)].cpu().numpy()
        ref = oracle.rank_scores(rows, np.arange(cnt), q_low[h], 64)
        np.testing.assert_array_equal(sl_rank[h, :cnt].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("N,S,C", [(65536, 4, 64), (200003, 2, 256), (1048576, 4, 64), (1048576, 1, 256)])
def test_wide_matches_oracle(device, N, S, C):
    assert _strategy(9, N, 64, S, C, 2048) == (2 if S == 1 else 1), "wide or code-class path not selected"
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, seed=N % 97)
    res = _summon(device, codes, k_low, q, q_proj, scale, cb, 2048)
    _check(codes, k_low, *res, 2048)


def test_wide_massive_ties_and_repeat(device):
    # 3 codewords: the threshold bin holds ~1/9 of all keys; exact resolution
    N, S, C = 120000, 2, 256
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, seed=7, few=True)
    first = _summon(device, codes, k_low, q, q_proj, scale, cb, 2048)
    _check(codes, k_low, *first, 2048)
    second = _summon(device, codes, k_low, q, q_proj, scale, cb, 2048)  # workspace reused
    for a, b in zip(first[2:], second[2:]):
        np.testing.assert_array_equal(np.sort(a, axis=-1) if a.ndim == 2 else a, np.sort(b, axis=-1) if b.ndim == 2 else b)


def test_wide_tight_budget_and_mask(device):
    N, S, C = 300000, 4, 64
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, seed=3)
    rng = np.random.default_rng(5)
    mask = np.where(rng.random(N) < 0.5, np.finfo(np.float32).min, 0.0).astype(np.float32)[None, None, None, :]
    res = _summon(device, codes, k_low, q, q_proj, scale, cb, 512, mask=torch.from_numpy(mask).to(device))
    _check(codes, k_low, *res, 512, allowed=mask[0, 0, 0] > -1e4)


def test_wide_agrees_with_item_path(device):
    from sva_amd import kernels

    N, S, C = 40000, 4, 64
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, seed=11)
    wide = _summon(device, codes, k_low, q, q_proj, scale, cb, 1024)
    # one query item per head through the per-item path: 2 tokens (q = 2) disable the wide path
    q2 = np.concatenate([q, q], axis=1)
    q_low, lut, rng = kernels.query_lut(torch.from_numpy(q2).to(device), torch.from_numpy(q_proj).to(device),
                                        torch.from_numpy(scale).to(device), torch.from_numpy(cb).to(device))
    sl_idx, sl_rank, sl_count = kernels.summon(lut, rng, q_low, torch.from_numpy(codes).to(device), k_low, N, 1024,
                                               mask=torch.zeros(1, 1, 2, N, device=device))
    sl_idx = sl_idx.view(9, 2, -1)[:, 0].cpu().numpy()
    for h in range(9):
        assert set(sl_idx[h].tolist()) == set(wide[2][h].tolist())


def test_wide_workspace_shared_across_shapes(device):
    # Regression: calls of different cache lengths and head counts share one
    # workspace, whatever earlier calls left in it.
    for N, S, C, H, few in ((150000, 2, 256, 9, True), (50000, 4, 64, 3, False), (33000, 4, 64, 9, False),
                            (150000, 2, 256, 9, True), (40000, 4, 64, 9, False)):
        codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=N % 13, few=few)
        res = _summon(device, codes, k_low, q, q_proj, scale, cb, 1024)
        _check(codes, k_low, *res, 1024)


def _sample_blocks(N, S):
    # the floor estimate's sample layout: one block of 32 keys per 256 keys,
    # at least 64 blocks, at most 32 KB of codes, block starts spread evenly
    # over the cache and rounded down to 16 keys
    return min(max(N // 256, 64), 32768 // (32 * S))


def test_wide_sampled_floor_overshoot(device):
    # Giving exactly the sampled keys the best code of every subspace puts
    # the estimate at the top of the score range, so only the rigged keys
    # reach it: with L above the sample size fewer than L keys do, and the
    # exact all-keys selection must take over; with L equal to the sample
    # size the rigged keys alone fill the shortlist.  Both the two-call path
    # and the one-call lookup are checked.
    from sva_amd import kernels

    N, S, C, H, KEYS = 40000, 4, 64, 3, 32
    blocks = _sample_blocks(N, S)
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=19)
    ql = oracle.query_low(q, q_proj, scale)[:, 0]
    for h in range(H):
        best = oracle.lut(ql[h], cb[h]).argmax(axis=1).astype(np.uint8)
        for blk in range(blocks):
            n0 = (blk * (N - KEYS) // (blocks - 1)) & ~15
            codes[h, n0:n0 + KEYS] = best
    for L in (blocks * KEYS + 1000, blocks * KEYS):
        res = _summon(device, codes, k_low, q, q_proj, scale, cb, L)
        _check(codes, k_low, *res, L)
        q_low, lut, rng, sl_idx, sl_rank, sl_count, _, _ = kernels.lookup_select(
            torch.from_numpy(q).to(device), torch.from_numpy(q_proj).to(device), torch.from_numpy(scale).to(device),
            torch.from_numpy(cb).to(device), torch.from_numpy(codes).to(device), k_low, N, L, 64)
        torch.cuda.synchronize()
        floor = np.maximum(rng[0, :, 0, 2].cpu().numpy(), rng[0, :, 0, 0].cpu().numpy())
        top = np.array([oracle.lut(ql[h], cb[h]).max(axis=1).sum() for h in range(H)], np.float32)
        assert bool((floor > 0.99 * top).all()), "the rigged samples must put the floor at the top of the range"
        _check(codes, k_low, q_low[0, :, 0].cpu().numpy(), lut[0, :, 0].cpu().numpy(), sl_idx.cpu().numpy(),
               sl_rank.cpu().numpy(), sl_count.cpu().numpy(), L)


def test_wide_candidates_beyond_lds_stage(device):
    # 3 codewords over 2 subspaces at 1M keys: the top score class holds
    # ~1/9 of the keys, far more candidates than the select kernel stages in
    # LDS; the selection runs over the per-wave lists and ties resolve by
    # key index.
    N, S, C, H = 1048576, 2, 256, 3
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=23, few=True)
    res = _summon(device, codes, k_low, q, q_proj, scale, cb, 2048)
    _check(codes, k_low, *res, 2048)


def _summon_select(device, codes, k_low, q, q_proj, scale, cb, L, B, mask=None):
    from sva_amd import kernels

    codes_t = torch.from_numpy(codes).to(device)
    q_low, lut, rng = kernels.query_lut(torch.from_numpy(q).to(device), torch.from_numpy(q_proj).to(device),
                                        torch.from_numpy(scale).to(device), torch.from_numpy(cb).to(device),
                                        codes_t, codes.shape[1], L)
    fused = kernels.summon_select(lut, rng, q_low, codes_t, k_low, codes.shape[1], L, B, mask=mask)
    sl_idx, sl_rank, sl_count = kernels.summon(lut, rng, q_low, codes_t, k_low, codes.shape[1], L, mask=mask)
    fin_idx, fin_count = kernels.budget_select(sl_idx, sl_rank, sl_count, B)
    torch.cuda.synchronize()
    return ([t.cpu().numpy() for t in fused], [t.cpu().numpy() for t in (sl_idx, sl_rank, sl_count, fin_idx, fin_count)],
            q_low[0, :, 0].cpu().numpy(), lut[0, :, 0].cpu().numpy())


def _check_fused(codes, k_low, fused, split, q_low, lut, L, B, allowed=None):
    sl_idx, sl_rank, sl_count, fin_idx, fin_count = fused
    # the shortlist and its ranks are the summon's, slot for slot
    np.testing.assert_array_equal(sl_count, split[2])
    for h in range(codes.shape[0]):
        c = int(sl_count[h])
        np.testing.assert_array_equal(sl_idx[h, :c], split[0][h, :c])
        np.testing.assert_array_equal(sl_rank[h, :c].view(np.uint32), split[1][h, :c].view(np.uint32))
    _check(codes, k_low, q_low, lut, sl_idx, sl_rank, sl_count, L, allowed=allowed)
    # the budget lists are the standalone select's, and the oracle's
    np.testing.assert_array_equal(fin_count, split[4])
    for h in range(codes.shape[0]):
        c, b = int(sl_count[h]), int(fin_count[h])
        assert b == min(B, c)
        np.testing.assert_array_equal(fin_idx[h, :b], split[3][h, :b])
        keep = oracle.topk(sl_rank[h, :c], b, key_index=sl_idx[h, :c])
        np.testing.assert_array_equal(fin_idx[h, :b], np.sort(sl_idx[h, :c][keep]))


@pytest.mark.parametrize("N,S,C,L,B,few", [(1048576, 4, 64, 2048, 512, False), (200003, 2, 256, 8192, 2048, False),
                                           (65536, 1, 256, 2048, 3000, False), (120000, 2, 256, 2048, 512, True),
                                           (1048576, 2, 256, 512, 128, False)])
def test_wide_summon_select_fused(device, N, S, C, L, B, few):
    assert _strategy(9, N, 64, S, C, L) == (2 if S == 1 else 1), "wide or code-class path not selected"
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, seed=(N + L) % 89, few=few)
    fused, split, q_low, lut = _summon_select(device, codes, k_low, q, q_proj, scale, cb, L, B)
    _check_fused(codes, k_low, fused, split, q_low, lut, L, B)


def test_summon_select_fallbacks_and_mask(device):
    # overshot floor (all-keys selection), candidates beyond the LDS stage,
    # and a float mask, each through the fused call
    N, S, C, H = 100000, 4, 64, 3
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=19)
    ql = oracle.query_low(q, q_proj, scale)[:, 0]
    for h in range(H):
        best = oracle.lut(ql[h], cb[h]).argmax(axis=1).astype(np.uint8)
        for blk in range(16):
            n0 = (blk * (N - 128) // 15) & ~15
            codes[h, n0:n0 + 128] = best
    fused, split, q_low, lut = _summon_select(device, codes, k_low, q, q_proj, scale, cb, 3000, 700)
    _check_fused(codes, k_low, fused, split, q_low, lut, 3000, 700)
    N, S, C = 1048576, 2, 256
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=23, few=True)
    fused, split, q_low, lut = _summon_select(device, codes, k_low, q, q_proj, scale, cb, 2048, 512)
    _check_fused(codes, k_low, fused, split, q_low, lut, 2048, 512)
    N, S, C = 300000, 4, 64
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=3)
    rng = np.random.default_rng(5)
    mask = np.where(rng.random(N) < 0.5, np.finfo(np.float32).min, 0.0).astype(np.float32)[None, None, None, :]
    fused, split, q_low, lut = _summon_select(device, codes, k_low, q, q_proj, scale, cb, 1024, 256,
                                              mask=torch.from_numpy(mask).to(device))
    _check_fused(codes, k_low, fused, split, q_low, lut, 1024, 256, allowed=mask[0, 0, 0] > -1e4)


@pytest.mark.parametrize("L,B", [(1024, 300), (4096, 2048), (8192, 2048)])
def test_summon_select_per_item_path(device, L, B):
    # q = 2 takes the one-workgroup-per-item summon, then the budget kernel (the item kernel's shortlists ascend,
    # so the budget is compacted in slot order; sva_budget_select sorts whatever order it is given)
    from sva_amd import kernels

    N, S, C = 40000, 4, 64
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, seed=11)
    q2 = np.concatenate([q, q[:, :, ::-1].copy()], axis=1)
    codes_t = torch.from_numpy(codes).to(device)
    q_low, lut, rng = kernels.query_lut(torch.from_numpy(q2).to(device), torch.from_numpy(q_proj).to(device),
                                        torch.from_numpy(scale).to(device), torch.from_numpy(cb).to(device))
    mask = torch.zeros(1, 1, 2, N, device=device)
    fused = kernels.summon_select(lut, rng, q_low, codes_t, k_low, N, L, B, mask=mask)
    sl_idx, sl_rank, sl_count = kernels.summon(lut, rng, q_low, codes_t, k_low, N, L, mask=mask)
    fin_idx, fin_count = kernels.budget_select(sl_idx, sl_rank, sl_count, B)
    for a, b in zip(fused, (sl_idx, sl_rank, sl_count, fin_idx, fin_count)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("case", ["many_lists", "more_lists_than_threads", "long_lists"])
def test_summon_select_staged_paths(device, case):
    # More than 512 scan lists (1.5M keys; 2.5M keys: more lists than the
    # finish kernel has threads), or lists longer than 32 candidates (a run
    # of keys with the best codes): the finish kernel stages the lists in LDS
    # instead of gathering them into registers.
    H, S, C = (1 if case == "more_lists_than_threads" else 3), 4, 64
    N = {"many_lists": 1536000, "more_lists_than_threads": 2500000, "long_lists": 300000}[case]
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=29)
    if case == "long_lists":
        ql = oracle.query_low(q, q_proj, scale)[:, 0]
        for h in range(H):
            best = oracle.lut(ql[h], cb[h]).argmax(axis=1).astype(np.uint8)
            codes[h, 50000:51000] = best
    fused, split, q_low, lut = _summon_select(device, codes, k_low, q, q_proj, scale, cb, 2048, 512)
    _check_fused(codes, k_low, fused, split, q_low, lut, 2048, 512)


@pytest.mark.parametrize("N,C,L,B,few,masked", [
    (1048576, 256, 2048, 512, False, False),   # 1M keys, ~4K keys per score class
    (300000, 100, 1024, 256, False, True),     # fewer codewords, float mask
    (120000, 256, 2048, 512, True, False),     # 3 codes: a boundary class of ~40K keys
    (70001, 256, 7168, 2048, False, False),    # the largest shortlist of the class path, partial chunk
    (1048576, 256, 512, 128, False, False),    # tight shortlist / budget
    (1048576, 256, 2048, 512, False, "sparse"),  # fewer allowed keys than L: the lowest class is the boundary
    (300000, 256, 2048, 512, True, "none"),    # every key masked: empty shortlist and budget
])
def test_class_path_single_subspace(device, N, C, L, B, few, masked):
    """One subspace of <= 256 codewords selects by code class (count, boundary class, ordered extraction,
    budget): shortlist and ranks equal the oracle's top-L (score desc, key asc) and the standalone budget
    select's lists, every head; with fewer allowed keys than L every allowed key is shortlisted, and with none
    the lists are empty."""
    assert _strategy(9, N, 64, 1, C, L) == 2, "code-class path not selected"
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, 1, C, seed=(N + C + L) % 83, few=few)
    mask = allowed = None
    if masked:
        rng = np.random.default_rng(9)
        keep = {True: rng.random(N) >= 0.4, "sparse": np.arange(N) % 1021 == 5, "none": np.zeros(N, bool)}[masked]
        m = np.where(keep, 0.0, np.finfo(np.float32).min).astype(np.float32)[None, None, None, :]
        mask, allowed = torch.from_numpy(m).to(device), m[0, 0, 0] > -1e4
    fused, split, q_low, lut = _summon_select(device, codes, k_low, q, q_proj, scale, cb, L, B, mask=mask)
    _check_fused(codes, k_low, fused, split, q_low, lut, L, B, allowed=allowed)
    if masked in ("sparse", "none"):
        assert (fused[2] == int(allowed.sum())).all(), "every allowed key is shortlisted"


def test_overshoot_at_a_million_keys_is_exact_and_reported(device):
    """The first key of every sampled block rigged to the best code of each subspace puts the sampled floor at
    the top score, so only those 256 keys reach it (fewer than L = 2048): the finish's three-pass all-keys
    select runs for every head.  The one-call decode step must still equal the oracle's shortlist, budget and
    verified output, and report the overshoot per head; the same caches unrigged report none."""
    from sva_amd import kernels

    N, S, C, H, L, B = 1 << 20, 4, 64, 9, 2048, 512
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=31)
    blocks = _sample_blocks(N, S)
    ql = oracle.query_low(q, q_proj, scale)[:, 0]
    rigged = codes.copy()
    for h in range(H):
        best = oracle.lut(ql[h], cb[h]).argmax(axis=1).astype(np.uint8)
        for blk in range(blocks):
            rigged[h, (blk * (N - 32) // (blocks - 1)) & ~15] = best
    g = torch.Generator(device=device).manual_seed(32)
    keys = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
    values = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    qb = t(q)[None].to(torch.bfloat16)
    for cds, expect in ((rigged, 1), (codes, 0)):
        plan = kernels.ScanDecodePlan(device, 1, H, 1, 64, 64, S, C, L, B)
        out = torch.empty(1, H, 1, 64, device=device, dtype=torch.float32)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        plan.run(qb, t(q_proj), t(scale), t(cb), t(cds), k_low, keys, values, N, 0.125, out=out)
        ev[0].record()
        plan.run(qb, t(q_proj), t(scale), t(cb), t(cds), k_low, keys, values, N, 0.125, out=out)
        ev[1].record()
        torch.cuda.synchronize()
        print(f"overshoot={expect}: {1e3 * ev[0].elapsed_time(ev[1]):.1f} us per step", flush=True)
        assert plan.overshoot.cpu().tolist() == [expect] * H
        _check_decode_step(plan, cds, k_low, qb, keys, values, out, L, B)


def _check_decode_step(plan, codes, k_low, qb, keys, values, out, L, B, scaling=0.125):
    """A ScanDecodePlan step against the oracle: the shortlist as a set (bit-exact ranks) over the plan's own
    table, the budget as the oracle's top-B of the shortlist's ranks (score desc, key asc) in key order, and the
    verified output within rel 1e-5 of the oracle's fp64 verifier (GQA: head h reads KV head h // (H / G))."""
    H = codes.shape[0]
    G = keys.shape[0]
    lut = plan.lut[0, :, 0].cpu().numpy()
    _check(codes, k_low, plan.q_low[0, :, 0].cpu().numpy(), lut, plan.sl_idx.cpu().numpy(),
           plan.sl_rank.cpu().numpy(), plan.sl_count.cpu().numpy(), L)
    fin_idx, fin_count = plan.fin_idx.cpu().numpy(), plan.fin_count.cpu().numpy()
    sl_idx, sl_rank, sl_count = plan.sl_idx.cpu().numpy(), plan.sl_rank.cpu().numpy(), plan.sl_count.cpu().numpy()
    qf, kf, vf = qb.float().cpu().numpy()[0, :, 0], keys.float().cpu().numpy(), values.float().cpu().numpy()
    got = out.float().cpu().numpy()[0, :, 0]
    for h in range(H):
        n = int(sl_count[h])
        keep = oracle.topk(sl_rank[h, :n], min(B, n), key_index=sl_idx[h, :n])
        want = np.sort(sl_idx[h, :n][keep])
        np.testing.assert_array_equal(fin_idx[h, :fin_count[h]], want)
        ref = oracle.verify(qf[h], kf[h // (H // G)], vf[h // (H // G)], want, scaling)
        assert np.abs(got[h] - ref).max() / np.abs(ref).max() <= 1e-5, f"head {h}"


@pytest.mark.parametrize("N,S,C,L,B", [
    (1 << 20, 4, 64, 2048, 512),   # the million-key decode workload
    (1 << 20, 4, 64, 512, 128),    # its tight budget
    (1 << 20, 2, 256, 2048, 512),  # 2x256 codes
    (1 << 20, 2, 64, 2048, 512),   # two subspaces below 64 codewords: one pair-table read per key
    (1048573, 4, 64, 2048, 512),   # a partial last 16-byte code word
    (300001, 2, 256, 1024, 256),   # a partial last word with eight keys per word
])
def test_decode_step_at_a_million_keys_matches_oracle(device, N, S, C, L, B):
    """The one-call decode step (sva_lookup_verify: the query, the scan, then the finish with the verifier) on
    caches of up to a million keys, seeded, against the oracle's shortlist, budget and fp64 verifier for every
    head."""
    from sva_amd import kernels

    H = 9
    print(f"decode step N={N} {S}x{C} L={L} B={B}", flush=True)
    codes, k_low, q, q_proj, scale, cb = _setup(device, N, S, C, H=H, seed=51 + S + L)
    g = torch.Generator(device=device).manual_seed(52)
    keys = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
    values = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    qb = t(q)[None].to(torch.bfloat16)
    # the catalog's capacity is whole 64-key blocks (16-byte aligned code rows; a partial last word when N is
    # not a multiple of 16 / S)
    padded = np.zeros((H, (N + 63) // 64 * 64, S), np.uint8)
    padded[:, :N] = codes
    plan = kernels.ScanDecodePlan(device, 1, H, 1, 64, 64, S, C, L, B)
    out = torch.empty(1, H, 1, 64, device=device, dtype=torch.float32)
    plan.run(qb, t(q_proj), t(scale), t(cb), t(padded)[:, :N], k_low, keys, values, N, 0.125, out=out)
    torch.cuda.synchronize()
    assert plan.overshoot.cpu().tolist() == [0] * H
    _check_decode_step(plan, codes, k_low, qb, keys, values, out, L, B)
