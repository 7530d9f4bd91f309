"""The CPU oracle against the reference's own outputs on the 8192-key lookup
(tests/golden/lookup8192_reference.npz)."""

from __future__ import annotations

import numpy as np

import oracle
from tests import golden_check
from tests.cases import lookup8192_inputs


def test_oracle_matches_reference_outputs():
    ref = golden_check.load()
    inp = lookup8192_inputs()
    H, G = inp["q"].shape[0], inp["keys"].shape[0]
    scale = np.exp(inp["logit_scale"]).clip(0.01, 100.0).astype(np.float32)
    q_low = oracle.query_low(inp["q"], inp["q_proj"], scale)[:, 0]
    k_low = np.stack([oracle.project(inp["keys"][h // (H // G)], inp["k_proj"][h]) for h in range(H)])
    codes = oracle.encode_product_keys(k_low, inp["codebooks"])
    lut = np.stack([oracle.lut(q_low[h], inp["codebooks"][h]) for h in range(H)])
    sl, fin, out, _ = oracle.decode(inp["q"][:, 0], q_low, inp["keys"], inp["values"], k_low, inp["codebooks"],
                                    codes.astype(np.uint8), inp["shortlist"], inp["budget"], 64 ** -0.5)
    golden_check.check(ref, inp, k_low, codes, q_low, lut, list(sl), list(fin), out)
