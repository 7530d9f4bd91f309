"""sva_verify_noalloc (the verifier with its slice partials in the library's
static device scratch) against sva_verify with a caller workspace, through
the C ABI: equal outputs on two calls in a row, the second with a smaller
input, and a clear refusal of a call whose partials exceed the scratch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(device, n_seq, H, G, N, D, B, kv_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_seq, H, 1, D, generator=g).to(device, kv_dtype)
    keys = torch.randn(G, n_seq * N, D, generator=g).to(device, kv_dtype)
    values = torch.randn(G, n_seq * N, D, generator=g).to(device, kv_dtype)
    items = n_seq * H
    fin_idx = torch.full((items, B), -1, dtype=torch.int32)
    fin_count = torch.empty(items, dtype=torch.int32)
    rng = np.random.default_rng(seed)
    for i in range(items):
        c = int(rng.integers(1, B + 1))
        fin_idx[i, :c] = torch.from_numpy(np.sort(rng.choice(N, c, replace=False)).astype(np.int32))
        fin_count[i] = c
    offs = torch.arange(n_seq, dtype=torch.int64) * N
    lens = torch.full((n_seq,), N, dtype=torch.int64)
    return q, keys, values, fin_idx.to(device), fin_count.to(device), offs.to(device), lens.to(device)


def _args(q, keys, values, fin_idx, fin_count, offs, lens, out, N, H, G, D, B):
    from sva_amd._lib import dtype_code

    n_seq = q.shape[0]
    return [q.data_ptr(), dtype_code(q), q.stride(0), q.stride(1), q.stride(2), keys.data_ptr(), values.data_ptr(),
            dtype_code(keys), keys.stride(0), keys.stride(1), offs.data_ptr(), lens.data_ptr(), n_seq * N,
            fin_idx.data_ptr(), fin_count.data_ptr(), n_seq, H, G, 1, D, B, D ** -0.5, out.data_ptr(),
            dtype_code(out), out.stride(0), out.stride(1), out.stride(2)]


def test_verify_noalloc_equals_verify(device):
    from sva_amd._lib import check, lib

    L = lib()
    stream = torch.cuda.current_stream(device).cuda_stream
    for n_seq, H, G, N, D, B, dt, seed in ((3, 9, 3, 40000, 64, 512, torch.bfloat16, 1),
                                          (1, 8, 2, 3000, 128, 96, torch.float32, 2)):
        q, keys, values, fin_idx, fin_count, offs, lens = _case(device, n_seq, H, G, N, D, B, dt, seed)
        want = torch.empty(n_seq, H, 1, D, device=device, dtype=dt)
        got = torch.full_like(want, float("nan"))
        need = int(L.sva_verify_workspace_bytes(n_seq, H, G, 1, D, B))
        ws = torch.empty(need, device=device, dtype=torch.uint8)
        check(L.sva_verify(*_args(q, keys, values, fin_idx, fin_count, offs, lens, want, N, H, G, D, B), ws.data_ptr(),
                           need, stream), "sva_verify")
        check(L.sva_verify_noalloc(*_args(q, keys, values, fin_idx, fin_count, offs, lens, got, N, H, G, D, B),
                                   stream), "sva_verify_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"n_seq={n_seq} H={H} B={B}: outputs differ"


def test_verify_noalloc_refuses_partials_beyond_the_scratch(device):
    from sva_amd._lib import lib

    L = lib()
    n_seq, H, G, D, B = 512, 8, 1, 256, 4096
    assert L.sva_verify_workspace_bytes(n_seq, H, G, 1, D, B) > (4 << 20)
    rc = L.sva_verify_noalloc(1, 0, 0, 0, 0, 1, 1, 0, 0, 0, None, None, 1 << 20, 1, 1, n_seq, H, G, 1, D, B, 0.1, 1, 0,
                              0, 0, 0, torch.cuda.current_stream(device).cuda_stream)
    assert rc == 3
    assert b"static scratch" in L.sva_last_error()
