"""GPU parity of the one-token lookup on the per-item register path (caches of
up to 16K keys, sva_summon_strategy 3).

There sva_lookup_verify runs the decode query, the summon and the verifier in
one launch.  Its q_low, table, bounds, shortlist and budget must equal, bit for
bit, those of the separate calls (sva_query_lut, then sva_summon_select) on
the same inputs, and its output must lie within rel 1e-5 of the oracle's fp64
verifier over the budget it chose and of the separate verifier (sva_verify).
Covered: every keys-per-thread form (4, 8 and 16 keys a thread), the 4x64,
2x256 and 1x256 layouts, bf16 / f16 / f32 K and V, a mask, a cache shorter
than the shortlist, and head_dim 128 (which takes the separate launches).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32

CASES = [
    # N, S, C, D, kv dtype, q dtype, L, B, masked
    (3000, 2, 256, 64, BF16, BF16, 2048, 512, False),    # 4 keys a thread
    (8192, 2, 256, 64, BF16, BF16, 2048, 512, False),    # the 8192-token model's cache, 8 keys a thread
    (12001, 2, 256, 64, BF16, BF16, 2048, 512, False),   # 16 keys a thread, a partial last block
    (16384, 4, 64, 64, F16, F32, 2048, 512, False),      # 4x64, the register path's largest cache
    (5000, 1, 256, 64, F32, BF16, 1024, 256, False),     # 1x256
    (8192, 2, 256, 64, BF16, BF16, 2048, 512, True),     # a mask allowing every 37th key
    (100, 2, 256, 64, BF16, F16, 2048, 512, False),      # fewer keys than the shortlist
    (1, 4, 64, 64, BF16, BF16, 2048, 512, False),        # a single key
    (16384, 2, 256, 64, BF16, BF16, 512, 512, False),    # the largest cache, budget equal to the shortlist
    (8192, 2, 256, 128, BF16, BF16, 2048, 512, False),   # head_dim 128: the separate launches
]


@pytest.mark.parametrize("N,S,C,D,kv_dtype,q_dtype,L,B,masked", CASES)
def test_one_launch_lookup_equals_separate_calls(N, S, C, D, kv_dtype, q_dtype, L, B, masked):
    from sva_amd import kernels

    device = torch.device("cuda:0")
    H, G, R = 9, 3, 64
    print(f"case N={N} S={S} C={C} D={D} kv={kv_dtype} q={q_dtype} L={L} B={B} masked={masked}", flush=True)
    g = torch.Generator(device=device).manual_seed(N * 7 + S * 3 + D)
    q = torch.randn(1, H, 1, D, device=device, generator=g).to(q_dtype)
    q_proj = torch.randn(H, D, R, device=device, generator=g) / 8.0
    scale = torch.rand(H, device=device, generator=g) + 0.5
    cb = torch.randn(H, S, C, R // S, device=device, generator=g)
    cap = (N + 63) // 64 * 64
    codes = torch.zeros(H, cap, S, device=device, dtype=torch.uint8)
    codes[:, :N] = torch.randint(0, C, (H, N, S), device=device, generator=g, dtype=torch.int32).to(torch.uint8)
    codes = codes[:, :N]
    k_low = torch.randn(H, N, R, device=device, generator=g)
    keys = torch.randn(G, N, D, device=device, generator=g).to(kv_dtype)
    values = torch.randn(G, N, D, device=device, generator=g).to(kv_dtype)
    mask = None
    if masked:
        mask = torch.full((1, 1, 1, N), -1e9, device=device)
        mask[..., ::37] = 0.0
    scaling = D ** -0.5

    plan = kernels.ScanDecodePlan(device, 1, H, 1, D, R, S, C, L, B)
    out = torch.empty(1, H, 1, D, device=device, dtype=torch.float32)
    plan.run(q, q_proj, scale, cb, codes, k_low, keys, values, N, scaling, out=out, mask=mask)

    q_low, lut, rng = kernels.query_lut(q, q_proj, scale, cb, codes, N, L)
    sl_idx, sl_rank, sl_count, fin_idx, fin_count = kernels.summon_select(lut, rng, q_low, codes, k_low, N, L, B,
                                                                          mask=mask)
    ref_out = kernels.verify(q, keys, values, fin_idx, fin_count, N, scaling, out_dtype=torch.float32)
    torch.cuda.synchronize()

    assert torch.equal(plan.q_low.reshape(H, R).cpu(), q_low.reshape(H, R).cpu()), "q_low differs"
    assert torch.equal(plan.lut.reshape(H, -1).cpu(), lut.reshape(H, -1).cpu()), "table differs"
    assert torch.equal(plan.rng.reshape(H, 4).cpu(), rng.reshape(H, 4).cpu()), "score bounds / floor differ"
    cnt, fcnt = plan.sl_count.cpu(), plan.fin_count.cpu()
    assert torch.equal(cnt, sl_count.cpu()), "shortlist counts differ"
    assert torch.equal(fcnt, fin_count.cpu()), "budget counts differ"
    a_idx, a_rank, a_fin = plan.sl_idx.cpu(), plan.sl_rank.cpu(), plan.fin_idx.cpu()
    b_idx, b_rank, b_fin = sl_idx.cpu(), sl_rank.cpu(), fin_idx.cpu()
    for h in range(H):
        c, f = int(cnt[h]), int(fcnt[h])
        assert c == min(L, N if mask is None else len(range(0, N, 37))), f"head {h}: shortlist of {c}"
        assert torch.equal(a_idx[h, :c], b_idx[h, :c]), f"head {h}: shortlist differs"
        assert torch.equal(a_rank[h, :c], b_rank[h, :c]), f"head {h}: rank scores differ"
        assert torch.equal(a_fin[h, :f], b_fin[h, :f]), f"head {h}: budget differs"

    got = out.cpu().numpy()[0, :, 0]
    sep = ref_out.cpu().numpy()[0, :, 0]
    qf, kf, vf = q.float().cpu().numpy()[0, :, 0], keys.float().cpu().numpy(), values.float().cpu().numpy()
    fin = a_fin.numpy()
    for h in range(H):
        sel = fin[h, : int(fcnt[h])]
        ref = oracle.verify(qf[h], kf[h // (H // G)], vf[h // (H // G)], np.sort(sel), scaling)
        den = max(np.abs(ref).max(), 1e-30)
        err = np.abs(got[h] - ref).max() / den
        assert err <= 1e-5, f"head {h}: rel err {err} against the oracle"
        err = np.abs(got[h] - sep[h]).max() / den
        assert err <= 1e-5, f"head {h}: rel err {err} against sva_verify"


def test_one_launch_lookup_repeats_and_graph_replays():
    """The one-launch lookup repeated on one plan gives the same outputs bit for bit, also captured in a HIP
    graph for two layers and replayed several times with eager lookups on the same plan between replays."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    H, G, D, R, S, C, L, B, N = 9, 3, 64, 64, 2, 256, 2048, 512, 8192
    layers = []
    for seed in (5, 6):
        g = torch.Generator(device=device).manual_seed(seed)
        q = torch.randn(1, H, 1, D, device=device, generator=g).to(BF16)
        q_proj = torch.randn(H, D, R, device=device, generator=g) / 8.0
        scale = torch.rand(H, device=device, generator=g) + 0.5
        cb = torch.randn(H, S, C, R // S, device=device, generator=g)
        codes = torch.randint(0, C, (H, N, S), device=device, generator=g, dtype=torch.int32).to(torch.uint8)
        k_low = torch.randn(H, N, R, device=device, generator=g)
        keys = torch.randn(G, N, D, device=device, generator=g).to(BF16)
        values = torch.randn(G, N, D, device=device, generator=g).to(BF16)
        layers.append((q, q_proj, scale, cb, codes, k_low, keys, values))
    plan = kernels.ScanDecodePlan(device, 1, H, 1, D, R, S, C, L, B)
    scaling = D ** -0.5
    eager = [plan.run(*lay, N, scaling).clone() for lay in layers]
    for rep in range(3):
        again = plan.run(*layers[rep % 2], N, scaling).clone()
        torch.cuda.synchronize()
        assert torch.equal(again, eager[rep % 2]), f"repeat {rep} differs"
    outs = [torch.empty_like(e) for e in eager]
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for lay, o in zip(layers, outs):
            plan.run(*lay, N, scaling, out=o)
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for lay, o in zip(layers, outs):
            plan.run(*lay, N, scaling, out=o)
    for rep in range(3):
        between = plan.run(*layers[rep % 2], N, scaling).clone()
        torch.cuda.synchronize()
        assert torch.equal(between, eager[rep % 2])
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {rep}, layer {i}"
