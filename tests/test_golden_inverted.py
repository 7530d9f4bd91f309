"""The oracle's static and adaptive inverted decode (oracle.static_decode,
oracle.inverted_decode, oracle.cell_choice) against what the reference's own
_inverted_static_decode_attention / _inverted_decode_attention chose on the
same inputs (tests/golden/inverted_reference.npz): candidate multisets
(which pin the cell choice, the postings and the tail rule), refill counts,
verified key sets, statistics, and the attention output within 1e-5."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests import golden_inverted

CASES = golden_inverted.cases()


@pytest.mark.parametrize("i", range(len(CASES)), ids=[f"{c['mode']}-{c['seed']}" for c in CASES])
def test_oracle_matches_reference_inverted_decode(i):
    c = CASES[i]
    inp = c["inputs"]
    N, C = c["N"], inp["codebooks"].shape[2]
    q_low = c["q_low"][:, None, :]
    common = dict(adaptive_min=c["amin"] or None, adaptive_mid=c["amid"] or None, low_margin=c["low"],
                  high_margin=c["high"], allowed=inp["allowed"])
    if c["mode"] == "inverted_static":
        plen = N - c["tail"]
        res = oracle.static_decode(inp["q"], inp["keys"], inp["values"], q_low, inp["k_low"], inp["codebooks"],
                                   oracle.rebuild_postings(inp["codes"][:, :plen], C), plen, c["budget"], c["cells"],
                                   64 ** -0.5, **common)
        np.testing.assert_array_equal([hd["refill"] for hd in res["heads"]], c["refill"])
    else:
        res = oracle.inverted_decode(inp["q"], inp["keys"], inp["values"], q_low, inp["k_low"], inp["codebooks"],
                                     inp["codes"], c["budget"], c["cells"], 64 ** -0.5, **common)
    for h, hd in enumerate(res["heads"]):
        np.testing.assert_array_equal(np.sort(hd["candidates"]), c["candidates"][h], err_msg=f"head {h} candidates")
    golden_inverted.check(c, [hd["final"] for hd in res["heads"]], res["out"], res["stats"])


def test_oracle_cell_choice_matches_reference_candidates():
    # the adaptive candidates of an unmasked case are exactly the keys whose
    # code lies in a chosen cell of some subspace, plus the current row
    c = next(c for c in CASES if c["mode"] == "inverted" and c["mask_frac"] == 0.0)
    inp = c["inputs"]
    for h in range(len(c["candidates"])):
        cells = oracle.cell_choice(c["q_low"][h], inp["codebooks"][h], c["cells"], 64)
        member = np.zeros(c["N"], bool)
        for s in range(cells.shape[0]):
            member |= np.isin(inp["codes"][h, :, s], cells[s])
        member[-1] = True
        np.testing.assert_array_equal(np.nonzero(member)[0], c["candidates"][h])


def test_planted_mistake_in_the_refill_rule_is_caught():
    # a refill window of budget entries instead of 2 * budget changes the
    # reference's choices on the static cases
    c = next(c for c in CASES if c["mode"] == "inverted_static" and c["tail"] == 10)
    inp = c["inputs"]
    plen = c["N"] - c["tail"]
    saved = oracle.top_unique_candidates

    def one_fold(idx, scores, valid, budget, refill_factor=2):
        return saved(idx, scores, valid, budget, 1)

    oracle.top_unique_candidates = one_fold
    try:
        res = oracle.static_decode(inp["q"], inp["keys"], inp["values"], c["q_low"][:, None, :], inp["k_low"],
                                   inp["codebooks"], oracle.rebuild_postings(inp["codes"][:, :plen], 256), plen,
                                   c["budget"], c["cells"], 64 ** -0.5)
    finally:
        oracle.top_unique_candidates = saved
    with pytest.raises(AssertionError):
        golden_inverted.check(c, [hd["final"] for hd in res["heads"]], res["out"], res["stats"])
