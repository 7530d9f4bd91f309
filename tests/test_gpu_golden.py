"""The whole GPU path (write encode -> query LUT -> summon -> budget ->
verify) against the reference's own outputs on the 8192-key lookup
(tests/golden/lookup8192_reference.npz)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import golden_check
from tests.cases import lookup8192_inputs

pytestmark = pytest.mark.gpu


def test_gpu_path_matches_reference_outputs(device):
    from sva_amd import kernels

    ref = golden_check.load()
    inp = lookup8192_inputs()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    H, N = inp["q"].shape[0], inp["keys"].shape[1]
    S = inp["codebooks"].shape[1]
    L, B = inp["shortlist"], inp["budget"]
    keys, values = t(inp["keys"]), t(inp["values"])
    k_low = torch.empty(H, N, 64, device=device)
    codes = torch.empty(H, N, S, device=device, dtype=torch.uint8)
    kernels.write_encode(keys, t(inp["k_proj"]), t(inp["codebooks"]), k_low, codes)
    scale = t(np.exp(inp["logit_scale"]).clip(0.01, 100.0).astype(np.float32))
    q = t(inp["q"])
    q_low, lut, rng = kernels.query_lut(q, t(inp["q_proj"]), scale, t(inp["codebooks"]), codes, N, L)
    sl_idx, sl_rank, sl_count = kernels.summon(lut, rng, q_low, codes, k_low, N, L)
    fin_idx, fin_count = kernels.budget_select(sl_idx, sl_rank, sl_count, B)
    out = kernels.verify(q, keys, values, fin_idx, fin_count, N, 64 ** -0.5)
    torch.cuda.synchronize()
    sl, sl_count = sl_idx.cpu().numpy(), sl_count.cpu().numpy()
    fin, fin_count = fin_idx.cpu().numpy(), fin_count.cpu().numpy()
    golden_check.check(ref, inp, k_low.cpu().numpy(), codes.cpu().numpy(), q_low[0, :, 0].cpu().numpy(),
                       lut[0, :, 0].cpu().numpy(), [sl[h, : sl_count[h]] for h in range(H)],
                       [fin[h, : fin_count[h]] for h in range(H)], out[0, :, 0].cpu().numpy())
    # the fused summon + budget call gives the same lists
    fused = kernels.summon_select(lut, rng, q_low, codes, k_low, N, L, B)
    torch.cuda.synchronize()
    f_sl, f_cnt, f_fin, f_fcnt = (fused[0].cpu().numpy(), fused[2].cpu().numpy(), fused[3].cpu().numpy(),
                                  fused[4].cpu().numpy())
    np.testing.assert_array_equal(f_cnt, sl_count)
    np.testing.assert_array_equal(f_fcnt, fin_count)
    for h in range(H):
        np.testing.assert_array_equal(f_sl[h, : sl_count[h]], sl[h, : sl_count[h]])
        np.testing.assert_array_equal(f_fin[h, : fin_count[h]], fin[h, : fin_count[h]])
