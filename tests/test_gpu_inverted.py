"""GPU parity of the inverted-index decode paths against the oracle.

Postings (CSR) equal the oracle's exactly; the unique refill selection
reproduces the reference's known-answer test and brute force; static and
adaptive decode give the oracle's chosen key sets per head (bit-exact index
sets: same LUT, same rank scores, rule score desc / key asc), its
statistics, and outputs within 1e-5 of its float64 verifier.  A ragged
batch of packed sequences (static mode, one launch per stage) gives, for
each sequence, what the oracle gives on that sequence's rows alone.  Catalog
inputs (k_low, codes) come from sva_write_encode, whose parity is tested on
its own.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _catalog(device, H=9, G=3, N=6000, D=64, R=64, S=2, C=256, seed=0):
    from sva_amd import kernels

    rng = np.random.default_rng(seed)
    keys = rng.standard_normal((G, N, D)).astype(np.float32)
    values = rng.standard_normal((G, N, D)).astype(np.float32)
    q = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    k_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    q_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    scale = np.ones(H, np.float32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    k_low = torch.empty(H, N, R, device=device)
    codes = torch.empty(H, N, S, device=device, dtype=torch.uint8)
    kernels.write_encode(t(keys), t(k_proj), t(cb), k_low, codes)
    torch.cuda.synchronize()
    return SimpleNamespace(keys=keys, values=values, q=q, q_proj=q_proj, scale=scale, cb=cb, k_low_t=k_low,
                           codes_t=codes, k_low=k_low.cpu().numpy(), codes=codes.cpu().numpy(), t=t, H=H, N=N, S=S,
                           C=C, D=D)


def _module(cat, device, mode, budget, cells, amin=None, amid=None, postings=None):
    from sva_amd.llama import SVALlamaAttention, SVALlamaServingConfig
    from sva_amd.stats import SVAStats

    serving = SVALlamaServingConfig(rank_dim=64, coarse_shortlist=4 * budget, budget=budget, summon_mode=mode,
                                    inverted_cells_per_subspace=cells, adaptive_min_budget=amin,
                                    adaptive_mid_budget=amid)
    return SimpleNamespace(serving=serving, sva_coarse_codebooks=cat.t(cat.cb), sva_q_proj=cat.t(cat.q_proj),
                           sva_scale=cat.t(cat.scale), _postings=postings, scaling=cat.D ** -0.5, stats=SVAStats(),
                           layer_idx=0, _profile_now=SVALlamaAttention._profile_now,
                           _profile_elapsed_ms=SVALlamaAttention._profile_elapsed_ms)


def test_postings_match_oracle(device):
    from sva_amd import inverted

    for C, n, skew in ((256, 5000, False), (16, 3001, True), (1024, 777, False), (64, 0, False)):
        rng = np.random.default_rng(C + n)
        codes = rng.integers(0, C, (3, max(n, 1), 2)).astype(np.int32)
        if skew:
            codes[:, : n // 2, 1] = 5
        ct = torch.from_numpy(codes.astype(np.int16 if C > 256 else np.uint8)).to(device)
        p = inverted.build_postings(ct, n, C)
        torch.cuda.synchronize()
        counts, offsets, ids = oracle.rebuild_postings(codes[:, :n], C)
        np.testing.assert_array_equal(p.offsets.cpu().numpy(), offsets)
        if n:
            np.testing.assert_array_equal(p.ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(p.max_count.cpu().numpy(), counts.max(-1))


def test_top_unique_known_answer(device):
    # tests/test_sva_llama_adapter.py:58-73 of the reference
    from sva_amd.llama import SVALlamaAttention

    idx = torch.tensor([[4, 4, 3, 3, 2, 1]], device=device)
    scores = torch.tensor([[9.0, 8.5, 8.0, 7.5, 7.0, 6.0]], device=device)
    valid = torch.ones_like(idx, dtype=torch.bool)
    sel, sc, ok, refill = SVALlamaAttention._top_unique_candidates(idx, scores, valid, budget=3, refill_factor=2)
    assert refill == 6
    assert sel[ok].tolist() == [4, 3, 2]
    assert sc[ok].tolist() == [9.0, 8.0, 7.0]


def test_top_unique_brute_force(device):
    from sva_amd import inverted

    rng = np.random.default_rng(7)
    for trial in range(40):
        rows, w = int(rng.integers(1, 5)), int(rng.integers(1, 60))
        budget = int(rng.integers(1, 14))
        ids = rng.integers(0, 20, (rows, w))
        scores = (rng.integers(0, 7, (rows, w)) / 2).astype(np.float32)
        valid = rng.random((rows, w)) < 0.8
        t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
        sel, sc, ok, refill = inverted.top_unique_candidates(t(ids), t(scores), t(valid), budget)
        sel, sc, ok = sel.cpu().numpy(), sc.cpu().numpy(), ok.cpu().numpy()
        for r in range(rows):
            e_ids, e_sc, e_ok, e_refill = oracle.top_unique_candidates(ids[r], scores[r], valid[r], budget)
            assert refill == e_refill
            assert sel.shape[1] == len(e_ids)
            np.testing.assert_array_equal(ok[r], e_ok)
            np.testing.assert_array_equal(sel[r][ok[r]], e_ids[e_ok])
            np.testing.assert_array_equal(sc[r][ok[r]], e_sc[e_ok])


def _check_decode(cat, res, ref, rtol=1e-5):
    out, fin_idx, fin_count, stats = res
    out = out[0, :, 0].float().cpu().numpy()
    fin_idx, fin_count, stats = fin_idx.cpu().numpy(), fin_count.cpu().numpy(), stats.cpu().numpy()
    for h in range(cat.H):
        want = np.sort(ref["heads"][h]["final"])
        got = fin_idx[h, : fin_count[h]]
        np.testing.assert_array_equal(got, want, err_msg=f"head {h}")
        err = np.abs(out[h] - ref["out"][h]).max() / max(np.abs(ref["out"][h]).max(), 1e-30)
        assert err <= rtol, f"head {h}: rel err {err}"
    assert float(stats[:, 0].sum()) == ref["stats"]["summoned"]
    assert float(fin_count.sum()) == ref["stats"]["verified"]
    if "refill_pool" in ref["stats"]:
        assert float(stats[:, 1].sum()) == ref["stats"]["refill_pool"]


@pytest.mark.parametrize("tail,amin,amid,masked", [(10, None, None, False), (0, 32, 64, False), (37, 16, 48, True),
                                                   (1, 1, 2, False)])
def test_static_decode_matches_oracle(device, tail, amin, amid, masked):
    from sva_amd import inverted

    cat = _catalog(device, seed=tail + 3)
    N, budget, cells = cat.N, 128, 8
    plen = N - tail
    post = inverted.build_postings(cat.codes_t, plen, cat.C)
    mod = _module(cat, device, "inverted_static", budget, cells, amin, amid, post)
    allowed = np.ones(N, bool)
    mask = None
    if masked:
        rng = np.random.default_rng(1)
        allowed = rng.random(N) < 0.7
        m = np.where(allowed, 0.0, np.finfo(np.float32).min).astype(np.float32)[None, None, None, :]
        mask = torch.from_numpy(m).to(device)
    res = inverted.static_decode(mod, cat.t(cat.q), cat.t(cat.keys), cat.t(cat.values), cat.k_low_t, cat.codes_t, N,
                                 mask, budget, return_selection=True)
    ql = oracle.query_low(cat.q[0], cat.q_proj, cat.scale)
    ref = oracle.static_decode(cat.q[0], cat.keys, cat.values, ql, cat.k_low, cat.cb,
                               oracle.rebuild_postings(cat.codes[:, :plen], cat.C), plen, budget, cells, cat.D ** -0.5,
                               adaptive_min=amin, adaptive_mid=amid, allowed=allowed)
    _check_decode(cat, res, ref)


@pytest.mark.parametrize("appended,amin,amid,masked", [(0, None, None, False), (300, 16, 48, False),
                                                       (50, 32, 64, True)])
def test_adaptive_decode_matches_oracle(device, appended, amin, amid, masked):
    from sva_amd import inverted

    cat = _catalog(device, seed=appended + 11)
    N, budget, cells = cat.N, 128, 8
    post = inverted.build_postings(cat.codes_t, N - appended, cat.C)  # rows past it: found by their codes
    mod = _module(cat, device, "inverted", budget, cells, amin, amid, post)
    allowed = np.ones(N, bool)
    mask = None
    if masked:
        rng = np.random.default_rng(2)
        allowed = rng.random(N) < 0.6
        allowed[-1] = False  # the current row disallowed: not a candidate
        m = np.where(allowed, 0.0, np.finfo(np.float32).min).astype(np.float32)[None, None, None, :]
        mask = torch.from_numpy(m).to(device)
    res = inverted.adaptive_decode(mod, cat.t(cat.q), cat.t(cat.keys), cat.t(cat.values), cat.k_low_t, cat.codes_t, N,
                                   mask, budget, return_selection=True)
    ql = oracle.query_low(cat.q[0], cat.q_proj, cat.scale)
    ref = oracle.inverted_decode(cat.q[0], cat.keys, cat.values, ql, cat.k_low, cat.cb, cat.codes, budget, cells,
                                 cat.D ** -0.5, adaptive_min=amin, adaptive_mid=amid, allowed=allowed)
    _check_decode(cat, res, ref)


def test_adaptive_decode_fallback_to_last_allowed_row(device):
    # no allowed key in the chosen cells and the current row masked: the last
    # allowed row is the only candidate (sva/llama.py:380-381)
    from sva_amd import inverted

    cat = _catalog(device, N=500, seed=5)
    N = cat.N
    post = inverted.build_postings(cat.codes_t, N, cat.C)
    mod = _module(cat, device, "inverted", 16, 2, None, None, post)
    allowed = np.zeros(N, bool)
    allowed[123] = True
    ql = oracle.query_low(cat.q[0], cat.q_proj, cat.scale)
    m = np.where(allowed, 0.0, np.finfo(np.float32).min).astype(np.float32)[None, None, None, :]
    res = inverted.adaptive_decode(mod, cat.t(cat.q), cat.t(cat.keys), cat.t(cat.values), cat.k_low_t, cat.codes_t,
                                   N, torch.from_numpy(m).to(device), 16, return_selection=True)
    ref = oracle.inverted_decode(cat.q[0], cat.keys, cat.values, ql, cat.k_low, cat.cb, cat.codes, 16, 2,
                                 cat.D ** -0.5, allowed=allowed)
    _check_decode(cat, res, ref)


# ---------------------------------------------------------------------------
# ragged static decode: packed sequences, one launch per stage, each sequence
# against the batch-1 oracle on its own rows

def _ragged_catalog(device, lens, H=9, G=3, D=64, R=64, S=2, C=256, seed=0):
    from sva_amd import kernels

    rng = np.random.default_rng(seed)
    rows = int(sum(lens))
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    keys = rng.standard_normal((G, rows, D)).astype(np.float32)
    values = rng.standard_normal((G, rows, D)).astype(np.float32)
    q = rng.standard_normal((len(lens), H, 1, D)).astype(np.float32)
    k_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    q_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    scale = np.ones(H, np.float32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    k_low = torch.empty(H, rows, R, device=device)
    codes = torch.empty(H, rows, S, device=device, dtype=torch.uint8)
    kernels.write_encode(t(keys), t(k_proj), t(cb), k_low, codes)
    torch.cuda.synchronize()
    return SimpleNamespace(keys=keys, values=values, q=q, q_proj=q_proj, scale=scale, cb=cb, k_low_t=k_low,
                           codes_t=codes, k_low=k_low.cpu().numpy(), codes=codes.cpu().numpy(), t=t, H=H, S=S, C=C,
                           D=D, offs=offs, lens=np.asarray(lens, np.int64), rows=rows)


RAGGED_LENS = [3000, 700, 5200, 1500, 130]
RAGGED_TAILS = [0, 10, 37, 1, 64]


def test_ragged_postings_match_oracle(device):
    from sva_amd import inverted

    cat = _ragged_catalog(device, RAGGED_LENS, seed=21)
    plens = cat.lens - np.asarray(RAGGED_TAILS)
    post = inverted.build_postings_ragged(cat.codes_t, cat.t(cat.offs), cat.t(plens), int(plens.max()), cat.C)
    offsets, ids, mc = post.offsets.cpu().numpy(), post.ids.cpu().numpy(), post.max_count.cpu().numpy()
    for b, (r0, pl) in enumerate(zip(cat.offs, plens)):
        counts, e_off, e_ids = oracle.rebuild_postings(cat.codes[:, r0:r0 + pl], cat.C)
        np.testing.assert_array_equal(offsets[b], e_off, err_msg=f"sequence {b}")
        np.testing.assert_array_equal(ids[:, :, r0:r0 + pl], e_ids, err_msg=f"sequence {b}")
        np.testing.assert_array_equal(mc[b], counts.max(-1), err_msg=f"sequence {b}")


@pytest.mark.parametrize("amin,amid,budget", [(None, None, 128), (16, 48, 128), (None, None, 1000)])
def test_ragged_static_decode_matches_oracle(device, amin, amid, budget):
    # budget 1000 exceeds the 130-key sequence: its budgets clamp to its length
    from sva_amd import inverted

    cat = _ragged_catalog(device, RAGGED_LENS, seed=budget + (amin or 0))
    cells = 8
    plens = cat.lens - np.asarray(RAGGED_TAILS)
    post = inverted.build_postings_ragged(cat.codes_t, cat.t(cat.offs), cat.t(plens), int(plens.max()), cat.C)
    out, fin_idx, fin_count, stats = inverted.ragged_static_decode(
        cat.t(cat.q), cat.t(cat.q_proj), cat.t(cat.scale), cat.t(cat.cb), cat.t(cat.keys), cat.t(cat.values),
        cat.k_low_t, cat.codes_t, cat.t(cat.offs), cat.t(cat.lens), post, int(max(RAGGED_TAILS)), budget, cells,
        cat.D ** -0.5, adaptive_min=amin, adaptive_mid=amid, return_selection=True)
    out = out[:, :, 0].float().cpu().numpy()
    fin_idx, fin_count, stats = fin_idx.cpu().numpy(), fin_count.cpu().numpy(), stats.cpu().numpy()
    for b, (r0, n, pl) in enumerate(zip(cat.offs, cat.lens, plens)):
        sl = slice(r0, r0 + n)
        ql = oracle.query_low(cat.q[b], cat.q_proj, cat.scale)
        ref = oracle.static_decode(cat.q[b], cat.keys[:, sl], cat.values[:, sl], ql, cat.k_low[:, sl], cat.cb,
                                   oracle.rebuild_postings(cat.codes[:, r0:r0 + pl], cat.C), int(pl), budget, cells,
                                   cat.D ** -0.5, adaptive_min=amin, adaptive_mid=amid)
        items = slice(b * cat.H, (b + 1) * cat.H)
        for h in range(cat.H):
            it = b * cat.H + h
            want = np.sort(ref["heads"][h]["final"])
            np.testing.assert_array_equal(fin_idx[it, : fin_count[it]], want, err_msg=f"sequence {b} head {h}")
            err = np.abs(out[b, h] - ref["out"][h]).max() / max(np.abs(ref["out"][h]).max(), 1e-30)
            assert err <= 1e-5, f"sequence {b} head {h}: rel err {err}"
        assert float(stats[items, 0].sum()) == ref["stats"]["summoned"], f"sequence {b}"
        assert float(fin_count[items].sum()) == ref["stats"]["verified"], f"sequence {b}"
        assert float(stats[items, 1].sum()) == ref["stats"]["refill_pool"], f"sequence {b}"


def test_config5_packed_batch_static_decode(device):
    # The ragged continuous-batch workload at its real shape: 32 sequences
    # with cache lengths log-uniform in [4096, 131072] packed contiguously,
    # bf16 K/V, 2x256 codes, static postings over all but a tail of up to 63
    # rows, 512/128 (static mode verifies min(128, 512, N) keys), cells 8.
    # The longest, the shortest and two other sequences are checked against
    # the oracle; every sequence is checked for counts and for sorted,
    # unique, in-range budget ids.
    from sva_amd import inverted, kernels

    H, G, D, R, S, C, budget, cells = 9, 3, 64, 64, 2, 256, 128, 8
    rng = np.random.default_rng(55)
    lens = np.exp(rng.uniform(np.log(4096), np.log(131072), 32)).astype(np.int64)
    tails = rng.integers(0, 64, 32).astype(np.int64)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    rows = int(lens.sum())
    print(f"config5: {rows} rows, lengths {lens.min()}..{lens.max()}", flush=True)
    g = torch.Generator(device=device).manual_seed(56)
    keys = torch.randn(G, rows, D, device=device, generator=g).to(torch.bfloat16)
    values = torch.randn(G, rows, D, device=device, generator=g).to(torch.bfloat16)
    q = rng.standard_normal((32, H, 1, D)).astype(np.float32)
    q_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    k_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    scale = np.exp(0.1 * rng.standard_normal(H)).astype(np.float32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    k_low = torch.empty(H, rows, R, device=device)
    codes = torch.empty(H, rows, S, device=device, dtype=torch.uint8)
    kernels.write_encode(keys, t(k_proj), t(cb), k_low, codes)
    plens = lens - tails
    post = inverted.build_postings_ragged(codes, t(offs), t(plens), int(plens.max()), C)
    qb = t(q).to(torch.bfloat16)
    out, fin_idx, fin_count, stats = inverted.ragged_static_decode(
        qb, t(q_proj), t(scale), t(cb), keys, values, k_low, codes, t(offs), t(lens), post, int(tails.max()), budget,
        cells, D ** -0.5, return_selection=True)
    out = out[:, :, 0].float().cpu().numpy()
    fin_idx, fin_count, stats = fin_idx.cpu().numpy(), fin_count.cpu().numpy(), stats.cpu().numpy()
    for b in range(32):
        for h in range(H):
            it = b * H + h
            ids = fin_idx[it, : fin_count[it]]
            assert 0 < fin_count[it] <= budget, f"sequence {b} head {h}: {fin_count[it]} verified"
            assert np.all(np.diff(ids) > 0) and ids[0] >= 0 and ids[-1] < lens[b], f"sequence {b} head {h}"
    order = np.argsort(lens)
    sample = sorted({int(order[-1]), int(order[0]), int(order[10]), int(order[21])})
    qf = qb.float().cpu().numpy()
    for b in sample:
        r0, n, pl = int(offs[b]), int(lens[b]), int(plens[b])
        print(f"config5: oracle on sequence {b} ({n} keys, tail {n - pl})", flush=True)
        kb = keys[:, r0:r0 + n].float().cpu().numpy()
        vb = values[:, r0:r0 + n].float().cpu().numpy()
        kl = k_low[:, r0:r0 + n].cpu().numpy()
        cd = codes[:, r0:r0 + pl].cpu().numpy()
        ql = oracle.query_low(qf[b], q_proj, scale)
        ref = oracle.static_decode(qf[b], kb, vb, ql, kl, cb, oracle.rebuild_postings(cd, C), pl, budget, cells,
                                   D ** -0.5)
        for h in range(H):
            it = b * H + h
            want = np.sort(ref["heads"][h]["final"])
            np.testing.assert_array_equal(fin_idx[it, : fin_count[it]], want, err_msg=f"sequence {b} head {h}")
            err = np.abs(out[b, h] - ref["out"][h]).max() / max(np.abs(ref["out"][h]).max(), 1e-30)
            assert err <= 1e-2, f"sequence {b} head {h}: rel err {err}"  # bf16 output
        items = slice(b * H, (b + 1) * H)
        assert float(stats[items, 0].sum()) == ref["stats"]["summoned"], f"sequence {b}"
        assert float(fin_count[items].sum()) == ref["stats"]["verified"], f"sequence {b}"
