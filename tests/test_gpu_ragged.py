"""Ragged multi-sequence decode on the GPU (no padding): sequences of
different lengths packed back to back in one cache and catalog, described by
seq_offsets / seq_lens, two query tokens per sequence with the causal rule
(key n for token t iff n <= len - Q + t).  Every sequence is checked against
the batch-1 oracle on its own rows: learned query map and table bit-exact,
shortlist and budget sets bit-exact, ranks bit-exact, verified output within
1e-5 of float64.  The reference has no ragged path (sva/llama.py:182-183 is
batch 1), so the oracle per sequence is the parity target.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,C", [(2, 256), (4, 64)])
def test_ragged_decode_end_to_end(device, S, C):
    from sva_amd import kernels

    rng = np.random.default_rng(41 + S)
    H, G, D, R, Q = 9, 3, 64, 64, 2
    lens = np.array([5000, 12003, 700, 2048], np.int64)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    total, n_seq = int(lens.sum()), len(lens)
    L, B = 1024, 256
    f32 = np.float32
    codes = rng.integers(0, C, (H, total, S), dtype=np.uint8)
    k_low = rng.standard_normal((H, total, R)).astype(f32)
    keys = rng.standard_normal((G, total, D)).astype(f32)
    values = rng.standard_normal((G, total, D)).astype(f32)
    q = rng.standard_normal((n_seq, H, Q, D)).astype(f32)
    q_proj = (rng.standard_normal((H, D, R)) / 8).astype(f32)
    scale = np.ones(H, f32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(f32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    n_keys = int(lens.max())
    q_low, lut, rg = kernels.query_lut(t(q), t(q_proj), t(scale), t(cb))
    sl_idx, sl_rank, sl_count, fin_idx, fin_count = kernels.summon_select(
        lut, rg, q_low, t(codes), t(k_low), n_keys, L, B, seq_offsets=t(offs), seq_lens=t(lens))
    out = kernels.verify(t(q), t(keys), t(values), fin_idx, fin_count, n_keys, D ** -0.5, seq_offsets=t(offs),
                         seq_lens=t(lens))
    torch.cuda.synchronize()
    q_low, lut = q_low.cpu().numpy(), lut.cpu().numpy()
    sl_idx, sl_rank, sl_count = sl_idx.cpu().numpy(), sl_rank.cpu().numpy(), sl_count.cpu().numpy()
    fin_idx, fin_count, out = fin_idx.cpu().numpy(), fin_count.cpu().numpy(), out.float().cpu().numpy()
    for b in range(n_seq):
        o, n = int(offs[b]), int(lens[b])
        ql = oracle.query_low(q[b], q_proj, scale)
        np.testing.assert_array_equal(q_low[b].view(np.uint32), ql.view(np.uint32))
        for h in range(H):
            for tok in range(Q):
                item = (b * H + h) * Q + tok
                table = oracle.lut(ql[h, tok], cb[h])
                np.testing.assert_array_equal(lut[b, h, tok].view(np.uint32), table.view(np.uint32))
                scores = oracle.pq_scores_from_lut(table, codes[h, o:o + n], R)
                allowed = np.arange(n) <= n - Q + tok
                sl = oracle.topk(scores, L, allowed=allowed)
                cnt = int(sl_count[item])
                assert cnt == len(sl), f"seq {b} head {h} token {tok}"
                got = sl_idx[item, :cnt].astype(np.int64)
                assert set(got.tolist()) == set(sl.tolist()), f"shortlist set, seq {b} head {h} token {tok}"
                rank = oracle.rank_scores(k_low[h, o:o + n], got, ql[h, tok], R)
                np.testing.assert_array_equal(sl_rank[item, :cnt].view(np.uint32), rank.view(np.uint32))
                keep = oracle.topk(rank, min(B, cnt), key_index=got)
                final = np.sort(got[keep])
                assert int(fin_count[item]) == len(final)
                np.testing.assert_array_equal(fin_idx[item, :len(final)], final)
                g = h // (H // G)
                ref = oracle.verify(q[b, h, tok], keys[g, o:o + n], values[g, o:o + n], final, D ** -0.5)
                err = np.abs(out[b, h, tok] - ref).max() / max(np.abs(ref).max(), 1e-30)
                assert err <= 1e-5, f"verifier rel err {err}, seq {b} head {h} token {tok}"
