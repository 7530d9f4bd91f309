"""GPU parity of the one-call decode lookup (sva_lookup_select).

The one-call lookup (query table with the sampled floor, scan, finish) must
give sva_query_lut + sva_summon_select's q_low, table, bounds, floor,
shortlist and budget bit for bit on the same inputs, for every layout and
cache length; its shortlists are also checked as sets against the oracle's
top-L on the table, and the sampled floor must leave a full shortlist.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _inputs(device, N, S, C, q_dtype, seed, H=9, R=64, D=64):
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(1, H, 1, D, device=device, generator=g).to(q_dtype)
    q_proj = torch.randn(H, D, R, device=device, generator=g) / 8.0
    scale = torch.rand(H, device=device, generator=g) + 0.5
    cb = torch.randn(H, S, C, R // S, device=device, generator=g)
    codes = torch.randint(0, C, (H, N, S), device=device, generator=g, dtype=torch.int32).to(torch.uint8)
    # a catalog's capacity: whole 64-key blocks per head, so that the code rows stay 16-byte aligned when
    # N is not a multiple of 16 / S (the last 16-byte word of a head is then partial)
    cap = (N + 63) // 64 * 64
    padded = torch.zeros(H, cap, S, device=device, dtype=torch.uint8)
    padded[:, :N] = codes
    k_low = torch.randn(H, N, R, device=device, generator=g)
    return q, q_proj, scale, cb, padded[:, :N], k_low


def _two_calls(q, q_proj, scale, cb, codes, k_low, N, L, B, mask=None):
    from sva_amd import kernels

    q_low, lut, rng = kernels.query_lut(q, q_proj, scale, cb, codes, N, L)
    out = kernels.summon_select(lut, rng, q_low, codes, k_low, N, L, B, mask=mask)
    return (q_low, lut, rng) + tuple(out)


def _assert_same(fused, ref):
    names = ("q_low", "lut", "score_range", "sl_idx", "sl_rank", "sl_count", "fin_idx", "fin_count")
    f_cnt, r_cnt = fused[5].cpu(), ref[5].cpu()
    assert torch.equal(f_cnt, r_cnt), "shortlist counts differ"
    b_cnt = fused[7].cpu()
    assert torch.equal(b_cnt, ref[7].cpu()), "budget counts differ"
    for name, a, b in zip(names, fused, ref):
        a, b = a.cpu(), b.cpu()
        if name in ("sl_idx", "sl_rank"):
            for h in range(a.shape[0]):
                c = int(f_cnt[h])
                assert torch.equal(a[h, :c], b[h, :c]), f"{name} differs in head {h}"
        elif name == "fin_idx":
            for h in range(a.shape[0]):
                c = int(b_cnt[h])
                assert torch.equal(a[h, :c], b[h, :c]), f"{name} differs in head {h}"
        elif name not in ("sl_count", "fin_count"):
            assert torch.equal(a, b), f"{name} differs"


@pytest.mark.parametrize("N,S,C,q_dtype,L,B", [
    (1 << 20, 4, 64, torch.bfloat16, 2048, 512),   # the million-key decode workload
    (1 << 20, 4, 64, torch.float32, 512, 128),     # tight budget
    (40000, 4, 64, torch.bfloat16, 2048, 512),     # partial last chunk
    (32768, 4, 64, torch.float16, 1024, 256),      # smallest wide-scan cache
    (1 << 18, 2, 256, torch.bfloat16, 2048, 512),  # 2x256 codes
    (500003, 2, 64, torch.bfloat16, 2048, 512),    # 2x64 codes (pair table), a partial last code word
    (1048573, 4, 64, torch.float32, 2048, 512),    # a partial last code word of four-byte keys
    (20000, 4, 64, torch.bfloat16, 2048, 512),     # too short for the wide scan: two calls
])
def test_lookup_select_equals_two_calls(N, S, C, q_dtype, L, B):
    from sva_amd import kernels

    device = torch.device("cuda:0")
    print(f"lookup_select N={N} {S}x{C} {q_dtype} L={L} B={B}", flush=True)
    q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, q_dtype, seed=N + S)
    ref = _two_calls(q, q_proj, scale, cb, codes, k_low, N, L, B)
    fused = kernels.lookup_select(q, q_proj, scale, cb, codes, k_low, N, L, B)
    torch.cuda.synchronize()
    _assert_same(fused, ref)


def test_lookup_select_shortlist_matches_oracle():
    from sva_amd import kernels

    device = torch.device("cuda:0")
    N, S, C, L, B = 65536 + 4096, 4, 64, 2048, 512
    q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, torch.bfloat16, seed=5)
    q_low, lut, _, sl_idx, sl_rank, sl_count, fin_idx, fin_count = kernels.lookup_select(
        q, q_proj, scale, cb, codes, k_low, N, L, B)
    torch.cuda.synchronize()
    lut_np, codes_np = lut[0, :, 0].cpu().numpy(), codes.cpu().numpy()
    q_low_np, k_low_np = q_low[0, :, 0].cpu().numpy(), k_low.cpu().numpy()
    for h in range(q.shape[1]):
        scores = oracle.pq_scores_from_lut(lut_np[h], codes_np[h], 64)
        sl = oracle.topk(scores, L)
        cnt = int(sl_count[h])
        got = sl_idx[h, :cnt].cpu().numpy().astype(np.int64)
        assert set(got.tolist()) == set(sl.tolist()), f"head {h}: shortlist set differs"
        ranks = oracle.rank_scores(k_low_np[h], got, q_low_np[h], 64)
        assert np.array_equal(sl_rank[h, :cnt].cpu().numpy(), ranks), f"head {h}: rank scores differ"
        fin = oracle.topk(ranks, B, key_index=got)
        want = np.sort(got[fin])
        assert np.array_equal(fin_idx[h, :int(fin_count[h])].cpu().numpy(), want), f"head {h}: budget differs"


def test_lookup_select_decode_plan_uses_one_call():
    """The decode plan's one-token step equals the three-call lookup (query table, summon + budget, verify)."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    N, S, C, L, B = 1 << 19, 4, 64, 2048, 512
    q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, torch.bfloat16, seed=11)
    g = torch.Generator(device=device).manual_seed(12)
    keys = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
    values = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
    plan = kernels.ScanDecodePlan(device, 1, 9, 1, 64, 64, S, C, L, B)
    outs = []
    for _ in range(2):
        o = torch.empty(1, 9, 1, 64, device=device, dtype=torch.float32)
        plan.run(q, q_proj, scale, cb, codes, k_low, keys, values, N, 0.125, out=o)
        outs.append((o, plan.fin_idx.clone(), plan.fin_count.clone()))
    _, _, _, _, _, _, fin_idx, fin_count = _two_calls(q, q_proj, scale, cb, codes, k_low, N, L, B)
    ref = kernels.verify(q, keys, values, fin_idx, fin_count, N, 0.125, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])  # deterministic
    for o, fi, fc in outs:
        assert torch.equal(fc, fin_count) and torch.equal(fi, fin_idx)
        # the verifier inside the finish kernel sums the softmax in another order than sva_verify
        err = ((o - ref).abs().max() / ref.abs().max()).item()
        assert err <= 1e-5, f"fused verifier differs from sva_verify by {err}"


@pytest.mark.parametrize("L,B", [(2048, 512), (512, 128), (256, 64)])
def test_sampled_floor_leaves_a_full_shortlist(L, B):
    """The sampled floor is a performance hint: an overshoot (fewer than L keys at or above it) sends the
    finish kernel to its all-keys select (slower, same result).  On seeded million-key caches the floor must
    leave at least L keys for every head, small shortlists included (the floor aims at max(2 L, 4096) keys),
    and the lookup must still equal the two-call path."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    N, S, C = 1 << 20, 4, 64
    for seed in range(3):
        print(f"floor L={L} seed={seed}", flush=True)
        q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, torch.bfloat16, seed=100 + seed)
        fused = kernels.lookup_select(q, q_proj, scale, cb, codes, k_low, N, L, B)
        lut, rng = fused[1][0, :, 0], fused[2][0, :, 0]
        idx = codes.long() + torch.arange(S, device=device).view(1, 1, S) * C
        sums = torch.zeros(codes.shape[0], N, device=device)
        for s in range(S):  # the scan's order: ((0 + T0) + T1) + ...
            sums = sums + torch.gather(lut.reshape(codes.shape[0], S * C), 1, idx[:, :, s])
        floor = torch.maximum(rng[:, 2], rng[:, 0])
        above = (sums >= floor[:, None]).sum(1)
        assert bool((above >= L).all()), f"floor overshoots: {above.tolist()} keys at or above it, L={L}"
        assert bool((above <= 4 * max(2 * L, 4096)).all()), f"floor far too low: {above.tolist()}"
        _assert_same(fused, _two_calls(q, q_proj, scale, cb, codes, k_low, N, L, B))


def test_decode_plan_rejects_bad_inputs():
    """The plan hands raw pointers to the kernels, so it checks dtypes, shapes and strides first."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    N, S, C, L, B = 8192, 4, 64, 256, 64
    q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, torch.bfloat16, seed=5)
    keys = torch.randn(3, N, 64, device=device).to(torch.bfloat16)
    values = torch.randn(3, N, 64, device=device).to(torch.bfloat16)
    plan = kernels.ScanDecodePlan(device, 1, 9, 1, 64, 64, S, C, L, B)
    good = plan.run(q, q_proj, scale, cb, codes, k_low, keys, values, N, 0.125).clone()
    with pytest.raises(ValueError, match="q_proj"):
        plan.summon(q, q_proj.double(), scale, cb, codes, k_low, N)
    with pytest.raises(ValueError, match="codebooks"):
        plan.summon(q, q_proj, scale, cb.transpose(2, 3), codes, k_low, N)
    with pytest.raises(ValueError, match="k_low"):
        plan.summon(q, q_proj, scale, cb, codes, k_low.half(), N)
    with pytest.raises(ValueError, match="catalog"):
        plan.summon(q, q_proj, scale, cb, codes, k_low, N + 1)
    with pytest.raises(ValueError, match="query"):
        plan.summon(q[:, :3], q_proj, scale, cb, codes, k_low, N)
    plan.summon(q, q_proj, scale, cb, codes, k_low, N)
    strided = torch.empty(3, N, 128, device=device, dtype=torch.bfloat16)[:, :, :64]
    strided.copy_(values)
    with pytest.raises(ValueError, match="values"):
        plan.verify(q, keys, strided, N, 0.125)
    assert torch.equal(plan.verify(q, keys, values, N, 0.125), good)


def test_decode_plan_graph_replays_equal_eager():
    """The q=1 lookup (sva_lookup_select + sva_verify through the plan's static buffers) captured in one HIP
    graph for two layers: every replay, with eager lookups on the same plan between replays, gives the eager
    outputs bit for bit."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    N, S, C, L, B = 1 << 18, 4, 64, 2048, 512
    layers = []
    for seed in (31, 32):
        q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, torch.bfloat16, seed=seed)
        g = torch.Generator(device=device).manual_seed(seed + 100)
        keys = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
        values = torch.randn(3, N, 64, device=device, generator=g).to(torch.bfloat16)
        layers.append((q, q_proj, scale, cb, codes, k_low, keys, values))
    plan = kernels.ScanDecodePlan(device, 1, 9, 1, 64, 64, S, C, L, B)
    eager = [plan.run(*lay, N, 0.125).clone() for lay in layers]
    outs = [torch.empty_like(e) for e in eager]
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for lay, o in zip(layers, outs):
            plan.run(*lay, N, 0.125, out=o)
    torch.cuda.current_stream(device).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for lay, o in zip(layers, outs):
            plan.run(*lay, N, 0.125, out=o)
    for rep in range(3):
        between = plan.run(*layers[rep % 2], N, 0.125).clone()
        torch.cuda.synchronize()
        assert torch.equal(between, eager[rep % 2])
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {rep}, layer {i}"


@pytest.mark.parametrize("G,D,kv_dtype,L,B,masked", [
    (3, 64, torch.bfloat16, 2048, 512, False),
    (3, 64, torch.float32, 512, 128, False),
    (9, 64, torch.float16, 8192, 2048, False),
    (1, 128, torch.bfloat16, 1024, 256, False),
    (3, 64, torch.bfloat16, 2048, 512, True),
    (3, 64, torch.bfloat16, 2048, 512, "1x256"),
])
def test_lookup_verify_matches_oracle(G, D, kv_dtype, L, B, masked):
    """sva_lookup_verify (the verifier inside the finish kernel on the wide path) against the oracle's fp64
    verifier over the budget lists the call selected: every head, fp32 output, rel 1e-5; a mask allowing only a
    few hundred keys, and one allowing none (empty lists give zeros)."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    N, S, C, H = 40000, 4, 64, 9
    if masked == "1x256":  # the code-class path, verifier inside its budget kernel
        S, C, masked = 1, 256, False
    q, q_proj, scale, cb, codes, k_low = _inputs(device, N, S, C, torch.bfloat16, seed=41 + G + D, D=D)
    g = torch.Generator(device=device).manual_seed(42)
    keys = torch.randn(G, N, D, device=device, generator=g).to(kv_dtype)
    values = torch.randn(G, N, D, device=device, generator=g).to(kv_dtype)
    masks = [None]
    if masked:
        few = torch.full((1, 1, 1, N), -1e9, device=device)
        few[..., ::97] = 0.0
        masks = [few, torch.full((1, 1, 1, N), -1e9, device=device)]
    plan = kernels.ScanDecodePlan(device, 1, H, 1, D, 64, S, C, L, B)
    scaling = D ** -0.5
    for mask in masks:
        out = torch.empty(1, H, 1, D, device=device, dtype=torch.float32)
        plan.run(q, q_proj, scale, cb, codes, k_low, keys, values, N, scaling, out=out, mask=mask)
        torch.cuda.synchronize()
        fin_idx, fin_count = plan.fin_idx.cpu().numpy(), plan.fin_count.cpu().numpy()
        qf, kf, vf = q.float().cpu().numpy()[0, :, 0], keys.float().cpu().numpy(), values.float().cpu().numpy()
        got = out.cpu().numpy()[0, :, 0]
        for h in range(H):
            sel = fin_idx[h, : fin_count[h]]
            if len(sel) == 0:
                assert np.all(got[h] == 0.0), f"head {h}: empty list must give zeros"
                continue
            ref = oracle.verify(qf[h], kf[h // (H // G)], vf[h // (H // G)], np.sort(sel), scaling)
            err = np.abs(got[h] - ref).max() / max(np.abs(ref).max(), 1e-30)
            assert err <= 1e-5, f"head {h}: rel err {err}"


@pytest.mark.parametrize("N0,S,C,kv_dtype", [
    (40000, 2, 256, torch.bfloat16),  # the wide scan: the append on its own, then the lookup
    (8000, 2, 256, torch.bfloat16),   # the per-item path: the append inside the one-launch lookup
    (12000, 4, 64, torch.float16),    # 4x64, 16 keys a thread
    (3000, 1, 256, torch.bfloat16),   # 1x256: the append reads codeword rows in place
    (8000, 2, 256, torch.float32),    # fp32 K / V: the per-item path with the append on its own
])
def test_decode_layer_steps_equal_plan(N0, S, C, kv_dtype):
    """The native decode step (sva_decode_layer_step) over appends of one and two rows and one rebuild equals,
    bit for bit, the catalog encoded whole by sva_write_encode followed by the plan's sva_lookup_verify; its
    device statistics count every head's shortlist and budget sizes and the queries."""
    from sva_amd import kernels

    device = torch.device("cuda:0")
    H, G, D, R, L, B = 9, 3, 64, 64, 2048, 512
    print(f"case N0={N0} S={S} C={C} kv={kv_dtype}", flush=True)
    g = torch.Generator(device=device).manual_seed(61)
    q_proj = torch.randn(H, D, R, device=device, generator=g) / 8.0
    k_proj = torch.randn(H, D, R, device=device, generator=g) / 8.0
    scale = torch.rand(H, device=device, generator=g) + 0.5
    cb = torch.randn(H, S, C, R // S, device=device, generator=g)
    cap = 65536
    keys = torch.randn(G, cap, D, device=device, generator=g).to(kv_dtype)
    values = torch.randn(G, cap, D, device=device, generator=g).to(kv_dtype)
    k_low = torch.empty(H, cap, R, device=device)
    codes = torch.empty(H, cap, S, device=device, dtype=torch.uint8)
    kernels.write_encode(keys, k_proj, cb, k_low, codes, 0, N0)
    plan = kernels.ScanDecodePlan(device, 1, H, 1, D, R, S, C, L, B)
    layer = kernels.DecodeLayer(kernels.ScanDecodePlan(device, 1, H, 1, D, R, S, C, L, B), q_proj, scale, cb, k_proj,
                                D ** -0.5)
    ref_low = torch.empty_like(k_low)
    ref_codes = torch.empty_like(codes)
    summoned = verified = 0
    for step, (row_begin, n) in enumerate([(N0, N0 + 1), (N0 + 1, N0 + 3), (N0 + 3, N0 + 4), (0, N0 + 4)]):
        q = torch.randn(1, H, 1, D, device=device, generator=g).to(torch.bfloat16)
        out = torch.empty(1, H, 1, D, device=device, dtype=torch.bfloat16)
        layer.step(q, keys, values, k_low, codes, row_begin, n, out)
        kernels.write_encode(keys, k_proj, cb, ref_low, ref_codes, 0, n)
        ref = plan.run(q, q_proj, scale, cb, ref_codes, ref_low, keys, values, n, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(k_low[:, :n], ref_low[:, :n]) and torch.equal(codes[:, :n], ref_codes[:, :n])
        lp = layer.plan
        assert torch.equal(lp.counts, plan.counts), f"step {step}: counts differ"
        for h in range(H):
            c, b = int(plan.sl_count[h]), int(plan.fin_count[h])
            assert torch.equal(lp.sl_idx[h, :c], plan.sl_idx[h, :c]) and torch.equal(lp.fin_idx[h, :b],
                                                                                       plan.fin_idx[h, :b])
        assert torch.equal(out, ref), f"step {step}: outputs differ"
        summoned += int(plan.sl_count.sum())
        verified += int(plan.fin_count.sum())
    assert layer.stats.tolist() == [summoned, verified, 0, 4 * H]
    with pytest.raises(Exception, match="catalog"):
        layer.step(q, keys, values, k_low[:, :100], codes[:, :100], 0, 200, out)
