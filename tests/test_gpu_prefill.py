"""GPU parity of the fused per-item summon (shortlist, rescore and budget in
one workgroup per query item, caches of up to 16K keys): the prefill shape of
sva/llama.py:262-302, many query tokens over a causal cache.

Every case is compared bit-exact with the separate per-item summon followed by
the standalone budget select (shortlist slot for slot, rank bits, budget
lists), and the small cases with the oracle (sets by score desc / key index
asc under the causal rule key n for token t of Q iff n <= N - Q + t).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _inputs(device, N, S, C, Q, H=3, seed=0, few=False, n_seq=1):
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    codes = rng.integers(0, 3 if few else C, size=(H, N, S), dtype=np.uint8)
    k_low = torch.randn(H, N, 64, device=device, generator=gen)
    q = rng.standard_normal((n_seq, H, Q, 64)).astype(np.float32)
    q_proj = (rng.standard_normal((H, 64, 64)) / 8).astype(np.float32)
    cb = rng.standard_normal((H, S, C, 64 // S)).astype(np.float32)
    return codes, k_low, q, q_proj, np.ones(H, np.float32), cb


def _run(device, codes, k_low, q, q_proj, scale, cb, n_keys, L, B, mask=None, offs=None, lens=None):
    from sva_amd import kernels

    codes_t = torch.from_numpy(codes).to(device)
    q_low, lut, rng = kernels.query_lut(torch.from_numpy(q).to(device), torch.from_numpy(q_proj).to(device),
                                        torch.from_numpy(scale).to(device), torch.from_numpy(cb).to(device))
    kw = dict(mask=mask, seq_offsets=offs, seq_lens=lens)
    fused = kernels.summon_select(lut, rng, q_low, codes_t, k_low, n_keys, L, B, **kw)
    # the prefill form: the shortlist stays in the kernel, the rest is the same
    lean = kernels.summon_select(lut, rng, q_low, codes_t, k_low, n_keys, L, B, keep_shortlist=False, **kw)
    sl_idx, sl_rank, sl_count = kernels.summon(lut, rng, q_low, codes_t, k_low, n_keys, L, **kw)
    fin_idx, fin_count = kernels.budget_select(sl_idx, sl_rank, sl_count, B)
    torch.cuda.synchronize()
    assert lean[0] is None and lean[1] is None, "the fused per-item path returned a shortlist it was not asked for"
    assert torch.equal(lean[2], fused[2]) and torch.equal(lean[4], fused[4]), "counts differ without shortlist outputs"
    lean_idx, lean_count = lean[3].cpu().numpy(), lean[4].cpu().numpy()
    for i, b in enumerate(lean_count.tolist()):
        np.testing.assert_array_equal(lean_idx[i, :b], fused[3][i, :b].cpu().numpy())
    split = (sl_idx, sl_rank, sl_count, fin_idx, fin_count)
    fused = [t.cpu().numpy() for t in fused]
    split = [t.cpu().numpy() for t in split]
    assert np.array_equal(fused[2], split[2]), "shortlist counts differ"
    assert np.array_equal(fused[4], split[4]), "budget counts differ"
    for i in range(fused[2].shape[0]):
        c, b = int(fused[2][i]), int(fused[4][i])
        assert b == min(B, c)
        np.testing.assert_array_equal(fused[0][i, :c], split[0][i, :c])
        np.testing.assert_array_equal(fused[1][i, :c].view(np.uint32), split[1][i, :c].view(np.uint32))
        np.testing.assert_array_equal(fused[3][i, :b], split[3][i, :b])
    return fused, q_low.cpu().numpy(), lut.cpu().numpy()


def _oracle_check(codes, k_low, fused, q_low, lut, L, B, n_keys):
    sl_idx, sl_rank, sl_count, fin_idx, fin_count = fused
    H, Q = q_low.shape[1], q_low.shape[2]
    for h in range(H):
        scores = None
        for t in range(Q):
            item = h * Q + t
            scores = oracle.pq_scores_from_lut(lut[0, h, t], codes[h, :n_keys], 64)
            allowed = np.arange(n_keys) <= n_keys - Q + t
            sl = oracle.topk(scores, L, allowed=allowed)
            c = int(sl_count[item])
            assert c == len(sl)
            got = sl_idx[item, :c].astype(np.int64)
            assert np.all(np.diff(got) > 0), "shortlist not in ascending key order"
            assert set(got.tolist()) == set(sl.tolist()), f"item {item}: shortlist set differs"
            rows = k_low[h, torch.from_numpy(got).to(k_low.device)].cpu().numpy()
            ref = oracle.rank_scores(rows, np.arange(c), q_low[0, h, t], 64)
            np.testing.assert_array_equal(sl_rank[item, :c].view(np.uint32), ref.view(np.uint32))
            b = int(fin_count[item])
            keep = oracle.topk(ref, b, key_index=got)
            np.testing.assert_array_equal(fin_idx[item, :b], np.sort(got[keep]))


@pytest.mark.parametrize("N,S,C,Q,L,B,few", [
    (3000, 2, 256, 6, 2048, 512, False),   # 4 keys per thread, select of L from ~3000
    (1500, 4, 64, 3, 2048, 512, False),    # fewer keys than L: the whole cache is the shortlist
    (10, 2, 256, 10, 16, 4, False),        # a prefill from scratch: token t sees t + 1 keys
    (777, 2, 256, 4, 256, 256, True),      # budget = shortlist, ties
])
def test_fused_item_matches_oracle(device, N, S, C, Q, L, B, few):
    codes, k_low, q, q_proj, scale, cb = _inputs(device, N, S, C, Q, seed=N % 31, few=few)
    fused, q_low, lut = _run(device, codes, k_low, q, q_proj, scale, cb, N, L, B)
    _oracle_check(codes, k_low, fused, q_low, lut, L, B, N)


@pytest.mark.parametrize("N,S,C,Q,L,B,few", [
    (8192, 2, 256, 4, 2048, 512, True),     # 8 keys per thread, massive ties
    (16384, 1, 256, 2, 1024, 300, False),   # 16 keys per thread, 256 distinct scores
    (12000, 4, 64, 3, 2048, 2048, False),
    (4097, 2, 256, 5, 64, 16, False),
])
def test_fused_item_matches_split_calls(device, N, S, C, Q, L, B, few):
    codes, k_low, q, q_proj, scale, cb = _inputs(device, N, S, C, Q, seed=N % 37, few=few)
    _run(device, codes, k_low, q, q_proj, scale, cb, N, L, B)


def test_fused_item_masks(device):
    # a float mask with different rows per token, and a bool mask
    N, S, C, Q = 5000, 2, 256, 3
    codes, k_low, q, q_proj, scale, cb = _inputs(device, N, S, C, Q, seed=41)
    rng = np.random.default_rng(6)
    m = np.where(rng.random((Q, N)) < 0.6, np.finfo(np.float32).min, 0.0).astype(np.float32)
    _run(device, codes, k_low, q, q_proj, scale, cb, N, 512, 128, mask=torch.from_numpy(m[None, None]).to(device))
    mb = torch.from_numpy(rng.random((Q, N)) < 0.5)[None, None].to(device)
    _run(device, codes, k_low, q, q_proj, scale, cb, N, 512, 128, mask=mb)


def test_fused_item_packed_sequences(device):
    # two packed sequences of 4000 and 2500 keys (rows 0..3999 and 4000..6499)
    lens_list = [4000, 2500]
    rows, Q, S, C = sum(lens_list), 2, 2, 256
    codes, k_low, q, q_proj, scale, cb = _inputs(device, rows, S, C, Q, seed=43, n_seq=2)
    offs = torch.tensor([0, 4000], device=device, dtype=torch.int64)
    lens = torch.tensor(lens_list, device=device, dtype=torch.int64)
    _run(device, codes, k_low, q, q_proj, scale, cb, max(lens_list), 2048, 512, offs=offs, lens=lens)


@pytest.mark.parametrize("S,C,Q,dtype", [(2, 256, 75, torch.bfloat16), (4, 64, 40, torch.float32),
                                         (1, 256, 9, torch.float16), (4, 48, 33, torch.float32),
                                         (2, 40, 20, torch.float32)])
def test_query_lut_many_tokens_matches_per_token(device, S, C, Q, dtype):
    # 8 or more tokens per head take the multi-token table kernel (weights
    # staged once per 32 tokens; fp32 MFMA where C is a multiple of 16);
    # every output equals the per-token kernel's fma chains bit for bit
    from sva_amd import kernels

    H, D, R = 3, 64, 64
    rng = np.random.default_rng(S * C + Q)
    q = torch.from_numpy(rng.standard_normal((2, H, Q, D)).astype(np.float32)).to(device, dtype)
    q_proj = torch.from_numpy((rng.standard_normal((H, D, R)) / 8).astype(np.float32)).to(device)
    scale = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).to(device)
    cb = torch.from_numpy(rng.standard_normal((H, S, C, R // S)).astype(np.float32)).to(device)
    q_low, lut, rng_out = kernels.query_lut(q, q_proj, scale, cb)
    for t in range(Q):
        ql1, lut1, rg1 = kernels.query_lut(q[:, :, t:t + 1], q_proj, scale, cb)
        assert torch.equal(q_low[:, :, t:t + 1].view(torch.int32), ql1.view(torch.int32)), f"q_low token {t}"
        assert torch.equal(lut[:, :, t:t + 1].view(torch.int32), lut1.view(torch.int32)), f"table token {t}"
        assert torch.equal(rng_out[:, :, t:t + 1, :2].view(torch.int32), rg1[..., :2].view(torch.int32)), f"bounds {t}"
        assert torch.all(rng_out[:, :, t, 2] == float("-inf"))
