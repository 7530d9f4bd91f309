"""The HIP static and adaptive inverted decode against what the reference's
own _inverted_static_decode_attention / _inverted_decode_attention chose on
the same inputs (tests/golden/inverted_reference.npz): verified key sets
bit-exact, statistics equal, output within 1e-5 (fp32).  The GPU computes
its own q_low and table from q; the fixture's cases keep every decision away
from ties, so last-bit differences there cannot move a set."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from tests import golden_inverted

pytestmark = pytest.mark.gpu

CASES = golden_inverted.cases()


@pytest.mark.parametrize("i", range(len(CASES)), ids=[f"{c['mode']}-{c['seed']}" for c in CASES])
def test_gpu_inverted_decode_matches_reference(device, i):
    from sva_amd import inverted
    from sva_amd.llama import SVALlamaAttention, SVALlamaServingConfig
    from sva_amd.stats import SVAStats

    c = CASES[i]
    inp = c["inputs"]
    N, C = c["N"], inp["codebooks"].shape[2]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    serving = SVALlamaServingConfig(rank_dim=64, coarse_shortlist=4 * c["budget"], budget=c["budget"],
                                    summon_mode=c["mode"], inverted_cells_per_subspace=c["cells"],
                                    adaptive_min_budget=c["amin"] or None, adaptive_mid_budget=c["amid"] or None,
                                    adaptive_low_margin=c["low"], adaptive_high_margin=c["high"])
    codes = t(inp["codes"])
    plen = N - c["tail"]
    stats = SVAStats()
    mod = SimpleNamespace(serving=serving, sva_coarse_codebooks=t(inp["codebooks"]), sva_q_proj=t(inp["q_proj"]),
                          sva_scale=t(np.exp(inp["logit_scale"]).clip(0.01, 100.0).astype(np.float32)),
                          _postings=inverted.build_postings(codes, plen, C), scaling=64 ** -0.5, stats=stats,
                          layer_idx=0, _profile_now=SVALlamaAttention._profile_now,
                          _profile_elapsed_ms=SVALlamaAttention._profile_elapsed_ms)
    mask = None
    if not inp["allowed"].all():
        m = np.where(inp["allowed"], 0.0, np.finfo(np.float32).min).astype(np.float32)
        mask = t(m[None, None, None, :])
    budget = min(c["budget"], N)
    decode = inverted.static_decode if c["mode"] == "inverted_static" else inverted.adaptive_decode
    out, fin_idx, fin_count, _ = decode(mod, t(inp["q"])[None], t(inp["keys"]), t(inp["values"]), t(inp["k_low"]),
                                        codes, N, mask, budget, return_selection=True)
    torch.cuda.synchronize()
    fin_idx, fin_count = fin_idx.cpu().numpy(), fin_count.cpu().numpy()
    finals = [fin_idx[h, : fin_count[h]] for h in range(fin_idx.shape[0])]
    golden_inverted.check(c, finals, out[0, :, 0].float().cpu().numpy(),
                          {k: float(v) for k, v in stats.totals.items()})
