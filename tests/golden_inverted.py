"""The reference's own inverted-index decode choices on the seeded cases of
tests/cases.py:INVERTED_CASES (tests/golden/inverted_reference.npz, written
by tests/golden/make_inverted_golden.py from sva/llama.py:330-425 and
:427-576).  Shared by the oracle test (CPU) and the GPU test."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from tests.cases import INVERTED_CASES, inverted_inputs

GOLDEN = Path(__file__).resolve().parent / "golden" / "inverted_reference.npz"


def _split(flat, counts):
    out, pos = [], 0
    for c in counts:
        out.append(flat[pos:pos + c])
        pos += c
    return out


def cases():
    """One dict per recorded case: its parameters, its regenerated inputs
    and what the reference chose and returned."""

    z = np.load(GOLDEN, allow_pickle=False)
    result = []
    for i in range(len(INVERTED_CASES)):
        p = json.loads(str(z[f"c{i}_params"]))
        inp = inverted_inputs(p["seed"], p["N"], p["mask_frac"], p["current_masked"])
        result.append({
            **p,
            "inputs": inp,
            "q_low": z[f"c{i}_q_low"],
            "candidates": _split(z[f"c{i}_cand"], z[f"c{i}_cand_count"]),
            "final": _split(z[f"c{i}_final"], z[f"c{i}_final_count"]),
            "refill": z[f"c{i}_refill"],
            "out": z[f"c{i}_out"],
        })
    return result


def check(case, final_sets, out, stats, rtol=1e-5):
    """final_sets: per head, the verified key ids (any order); out [H, D];
    stats: the reference's stat names -> totals."""

    H = len(case["final"])
    for h in range(H):
        np.testing.assert_array_equal(np.sort(np.asarray(final_sets[h])), case["final"][h],
                                      err_msg=f"{case['mode']} seed {case['seed']} head {h}: verified keys")
        ref = case["out"][h].astype(np.float64)
        err = np.abs(np.asarray(out[h], np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err <= rtol, f"{case['mode']} seed {case['seed']} head {h}: rel err {err}"
    for name, value in stats.items():
        assert value == case["stats"][name], f"{case['mode']} seed {case['seed']}: stat {name} {value} " \
                                             f"!= {case['stats'][name]}"
