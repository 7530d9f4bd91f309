"""GPU parity of the scan-mode decode path against the oracle.

Stage by stage on the same inputs: the learned query map and the LUT
bit-exact, scan scores bit-exact, shortlist and budget index SETS bit-exact
(selection rule: score desc, key index asc), rank scores bit-exact, verifier
output within 1e-5 (fp32) / 2e-2 (bf16) of the float64 oracle, relative to the
output's max magnitude.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.cases import make_case

pytestmark = pytest.mark.gpu


def _kernels():
    from sva_amd import kernels

    return kernels


def _run_scan(case, device, shortlist, budget, mask=None, q_len=1):
    k = _kernels()
    q = case.t("q", device, case.dtype)
    q_low, lut, rng = k.query_lut(q, case.t("q_proj", device), case.t("scale", device), case.t("codebooks", device))
    codes = case.t("codes", device)
    k_low = case.t("k_low", device)
    sl_idx, sl_rank, sl_count = k.summon(lut, rng, q_low, codes, k_low, case.N, shortlist, mask=mask)
    fin_idx, fin_count = k.budget_select(sl_idx, sl_rank, sl_count, budget)
    keys = case.t("keys", device, case.dtype)
    values = case.t("values", device, case.dtype)
    out = k.verify(q, keys, values, fin_idx, fin_count, case.N, case.D ** -0.5)
    torch.cuda.synchronize()
    return {
        "q_low": q_low[0].cpu().numpy(), "lut": lut[0].cpu().numpy(), "range": rng[0].cpu().numpy(),
        "sl_idx": sl_idx.cpu().numpy(), "sl_rank": sl_rank.cpu().numpy(), "sl_count": sl_count.cpu().numpy(),
        "fin_idx": fin_idx.cpu().numpy(), "fin_count": fin_count.cpu().numpy(), "out": out[0].float().cpu().numpy(),
    }


def _check_case(case, res, shortlist, budget, allowed=None, tol=1e-5):
    H, Q = case.q.shape[0], case.q.shape[1]
    group = case.H // case.G
    # learned query map, bit-exact
    q_low = oracle.query_low(case.q, case.q_proj, case.scale)
    np.testing.assert_array_equal(res["q_low"].view(np.uint32), q_low.view(np.uint32))
    for h in range(H):
        for t in range(Q):
            item = h * Q + t
            table = oracle.lut(q_low[h, t], case.codebooks[h])
            np.testing.assert_array_equal(res["lut"][h, t].view(np.uint32), table.view(np.uint32))
            scores = oracle.pq_scores_from_lut(table, case.codes[h], case.R)
            sums = oracle.pq_scores_from_lut(table, case.codes[h], 1)  # before the 1/sqrt(R) scale
            lo, hi = res["range"][h, t, :2]
            al = np.ones(case.N, bool) if allowed is None else allowed[t]
            assert sums.min() >= lo and sums.max() <= hi
            sl = oracle.topk(scores, shortlist, allowed=al)
            count = int(res["sl_count"][item])
            assert count == len(sl)
            gpu_sl = res["sl_idx"][item, :count].astype(np.int64)
            assert set(gpu_sl.tolist()) == set(sl.tolist()), f"shortlist set differs (h={h}, t={t})"
            rank = oracle.rank_scores(case.k_low[h], gpu_sl, q_low[h, t], case.R)
            np.testing.assert_array_equal(res["sl_rank"][item, :count].view(np.uint32), rank.view(np.uint32))
            keep = oracle.topk(rank, min(budget, count), key_index=gpu_sl)
            final = np.sort(gpu_sl[keep])
            fcount = int(res["fin_count"][item])
            assert fcount == len(final)
            np.testing.assert_array_equal(res["fin_idx"][item, :fcount], final)
            g = h // group
            ref = oracle.verify(case.q[h, t], case.keys[g], case.values[g], final, case.D ** -0.5)
            err = np.abs(res["out"][h, t] - ref).max() / max(np.abs(ref).max(), 1e-30)
            assert err <= tol, f"verifier rel err {err} > {tol} (h={h}, t={t})"


@pytest.mark.parametrize("S,C", [(2, 256), (4, 64), (1, 256)])
def test_scan_decode_fp32_8192_keys(device, S, C):
    case = make_case(N=8192, S=S, C=C, seed=11 + S)
    res = _run_scan(case, device, 2048, 512)
    _check_case(case, res, 2048, 512)


def test_scan_decode_bf16(device):
    case = make_case(N=8192, S=4, C=64, seed=5, dtype=torch.bfloat16)
    res = _run_scan(case, device, 2048, 512)
    _check_case(case, res, 2048, 512, tol=2e-2)


def test_scan_decode_massive_ties(device):
    # 3 codewords per subspace: thousands of exactly equal scores straddle the
    # shortlist boundary; duplicated k_low rows tie the budget boundary too
    case = make_case(N=6000, S=2, C=16, seed=3, code_mode="few", ties=True)
    res = _run_scan(case, device, 700, 97)
    _check_case(case, res, 700, 97)


def test_scan_decode_small_cache_and_tight_budget(device):
    case = make_case(N=300, S=2, C=256, seed=9)
    res = _run_scan(case, device, 2048, 512)  # shortlist > keys: everything is summoned
    _check_case(case, res, 2048, 512)
    case = make_case(N=5000, S=4, C=64, seed=10)
    res = _run_scan(case, device, 512, 128)
    _check_case(case, res, 512, 128)


def test_scan_prefill_causal(device):
    # q_len > 1 with the causal rule of sva/llama.py:192-198
    q_len, n = 24, 700
    case = make_case(N=n, S=2, C=32, Q=q_len, seed=21)
    res = _run_scan(case, device, 64, 16)
    allowed = oracle.allowed_mask(q_len, n)
    _check_case(case, res, 64, 16, allowed=allowed)


@pytest.mark.parametrize("N,L,B", [(33000, 8192, 2048), (70000, 2048, 512)])
def test_scan_two_tokens_long_cache(device, N, L, B):
    # q_len 2 keeps long caches on the one-workgroup-per-item summon: 33000 keys stay in LDS beside uint16
    # shortlist slots (the batch-8 socket shape's 8192 / 2048), 70000 keys are recomputed per pass with int32 slots
    case = make_case(N=N, S=2, C=256, Q=2, seed=23 + N % 7)
    res = _run_scan(case, device, L, B)
    _check_case(case, res, L, B, allowed=oracle.allowed_mask(2, N))


def test_scan_additive_mask(device):
    q_len, n = 4, 900
    case = make_case(N=n, S=2, C=32, Q=q_len, seed=22)
    rng = np.random.default_rng(1)
    mask = np.where(rng.random((1, 1, q_len, n)) < 0.3, np.finfo(np.float32).min, 0.0).astype(np.float32)
    res = _run_scan(case, device, 128, 32, mask=torch.from_numpy(mask).to(device))
    _check_case(case, res, 128, 32, allowed=oracle.allowed_mask(q_len, n, mask))


def test_pq_scores_all_keys(device):
    k = _kernels()
    case = make_case(N=3001, S=4, C=64, seed=4)
    q_low, lut, _ = k.query_lut(case.t("q", device), case.t("q_proj", device), case.t("scale", device),
                                case.t("codebooks", device))
    scores = k.pq_scores(lut, case.t("codes", device), case.N, case.R)[0, :, 0].cpu().numpy()
    ql = oracle.query_low(case.q, case.q_proj, case.scale)
    for h in range(case.H):
        ref = oracle.pq_scores_from_lut(oracle.lut(ql[h, 0], case.codebooks[h]), case.codes[h], case.R)
        np.testing.assert_array_equal(scores[h].view(np.uint32), ref.view(np.uint32))
