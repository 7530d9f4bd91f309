"""GPU parity of the decode form of the query table kernel (one token of one
sequence, D = R = 64): q_low and the table bit-exact against the oracle, the
table bounds exact, and the sampled floor a valid hint.  The shapes cover
every decode form, with codeword counts that are and are not multiples of a
wavefront (per-wave and per-entry bound folds), and the 1024-thread forms
whose codebook rows are shared by two lanes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,C", [(4, 64), (4, 48), (2, 256), (2, 200), (1, 256), (1, 100)])
def test_decode_query_form_matches_oracle(device, S, C):
    from sva_amd import kernels

    H, N, L = 9, 300000, 2048
    print(f"decode query {S}x{C} N={N}", flush=True)
    rng = np.random.default_rng(S * 1000 + C)
    q = rng.standard_normal((H, 1, 64)).astype(np.float32)
    q_proj = (rng.standard_normal((H, 64, 64)) / 8).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, H).astype(np.float32)
    cb = rng.standard_normal((H, S, C, 64 // S)).astype(np.float32)
    codes = rng.integers(0, C, size=(H, N, S), dtype=np.uint8)
    q_low, lut, rg = kernels.query_lut(torch.from_numpy(q).to(device), torch.from_numpy(q_proj).to(device),
                                       torch.from_numpy(scale).to(device), torch.from_numpy(cb).to(device),
                                       torch.from_numpy(codes).to(device), N, L)
    torch.cuda.synchronize()
    q_low, lut, rg = q_low[0, :, 0].cpu().numpy(), lut[0, :, 0].cpu().numpy(), rg[0, :, 0].cpu().numpy()
    ql_ref = oracle.query_low(q, q_proj, scale)[:, 0]
    np.testing.assert_array_equal(q_low.view(np.uint32), ql_ref.view(np.uint32))
    for h in range(H):
        table = oracle.lut(ql_ref[h], cb[h])
        np.testing.assert_array_equal(lut[h].view(np.uint32), table.view(np.uint32), err_msg=f"head {h}")
        # bounds of any sum: the per-subspace minima (maxima) added in subspace order from 0
        lo = np.float32(0.0)
        hi = np.float32(0.0)
        for s in range(S):
            lo = np.float32(lo + table[s].min())
            hi = np.float32(hi + table[s].max())
        assert rg[h, 0] == lo and rg[h, 1] == hi, f"head {h}: bounds {rg[h, :2]} against {lo}, {hi}"
        floor = rg[h, 2]
        if floor == -np.inf:  # no sampled floor: every allowed key is a candidate
            continue
        # the floor is a sampled hint: inside the bounds, and (on uniform codes) below the L-th largest score
        assert lo <= floor <= hi, f"head {h}: floor {floor} outside [{lo}, {hi}]"
        scores = oracle.pq_scores_from_lut(table, codes[h], 64) * np.float32(np.sqrt(64.0))
        kth = np.sort(scores)[-L]
        assert floor <= kth, f"head {h}: floor {floor} above the {L}-th largest sum {kth}"
