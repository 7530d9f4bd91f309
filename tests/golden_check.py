"""Comparison of a full decode lookup against the reference's own outputs on
the 8192-key single-layer lookup (tests/golden/lookup8192_reference.npz, written by
tests/golden/make_golden.py).  Shared by the oracle test (CPU) and the GPU
test: each passes the pieces it computed."""

from __future__ import annotations

from pathlib import Path

import numpy as np

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "lookup8192_reference.npz"


def load():
    return dict(np.load(GOLDEN, allow_pickle=False))


def check(ref, inp, k_low, codes, q_low, lut, shortlist_sets, budget_sets, out, rtol=1e-5):
    """shortlist_sets / budget_sets: per head, 1-D arrays of key indices."""

    H = q_low.shape[0]
    # k_low: the many-row einsum, bit-exact
    np.testing.assert_array_equal(k_low[:, :16].view(np.uint32), ref["k_low_rows"].view(np.uint32))
    np.testing.assert_array_equal(k_low.astype(np.float64).sum(axis=(1, 2)), ref["k_low_head_sums"])
    # codes: equal except where two centroids tie within rounding
    _, gaps = oracle.encode_product_keys(k_low, inp["codebooks"], return_gap=True)
    diff = codes.astype(np.int64) != ref["codes"]
    assert np.all(gaps[diff] <= 1e-4) and diff.sum() <= 2
    # q_low / LUT: MKL's single-row kernel rounds in its own order; within the
    # float64 bound of the contraction
    d = inp["q"].shape[-1]
    assert np.allclose(q_low, ref["q_low"], rtol=0, atol=4 * d * np.finfo(np.float32).eps * np.abs(ref["q_low"]).max())
    assert np.allclose(lut, ref["lut"], rtol=0, atol=1e-5 * np.abs(ref["lut"]).max())
    # shortlist and budget sets.  Where the reference's L-th and (L+1)-th
    # scores are apart, the sets must equal the reference's.  Where they tie
    # (heads whose boundary keys share a code pair), torch.topk picked tie
    # members in its own order; then the keys strictly above the boundary
    # must equal the reference's, the tie members must be the lowest key
    # indices (this build's rule), and the budget and output are checked
    # against the oracle on that shortlist.
    R = q_low.shape[1]
    L = len(ref["shortlist"][0])
    G = inp["keys"].shape[0]
    for h in range(H):
        got, want = set(np.asarray(shortlist_sets[h]).tolist()), set(ref["shortlist"][h].tolist())
        got_budget, want_budget = set(np.asarray(budget_sets[h]).tolist()), set(ref["budget"][h].tolist())
        if ref["shortlist_gap"][h] > 1e-5:
            assert got == want, f"head {h}: shortlist differs from the reference"
        else:
            ref_scores = oracle.pq_scores_from_lut(ref["lut"][h], ref["codes"][h], R)
            boundary = np.sort(ref_scores)[::-1][L - 1]
            above = set(np.nonzero(ref_scores > boundary)[0].tolist())
            assert above <= want, f"head {h}: the reference's shortlist misses a key above its boundary"
            scores = oracle.pq_scores_from_lut(lut[h], codes[h], R)
            rule = set(oracle.topk(scores, L).tolist())
            assert got == rule, f"head {h}: shortlist is not the (score desc, index asc) top-{L}"
            assert above <= got, f"head {h}: shortlist misses a key above the reference's boundary"
        if got == want and ref["budget_gap"][h] > 1e-5:
            assert got_budget == want_budget, f"head {h}: budget set differs from the reference"
            err = np.abs(out[h] - ref["out"][h]).max() / np.abs(ref["out"][h]).max()
            assert err <= rtol, f"head {h}: verifier rel err {err}"
        else:
            sl = np.sort(np.fromiter(got, np.int64))
            rank = oracle.rank_scores(k_low[h], sl, q_low[h], R)
            expect = set(sl[oracle.topk(rank, len(want_budget), key_index=sl)].tolist())
            assert got_budget == expect, f"head {h}: budget set is not the top of its shortlist's rank scores"
            g = h // (H // G)
            ref_out = oracle.verify(inp["q"][h, 0], inp["keys"][g], inp["values"][g],
                                    np.sort(np.fromiter(expect, np.int64)), inp["q"].shape[-1] ** -0.5)
            err = np.abs(out[h] - ref_out).max() / np.abs(ref_out).max()
            assert err <= rtol, f"head {h}: verifier rel err {err} against the oracle"
