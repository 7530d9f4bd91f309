"""The torch-CPU restatement of the reference's decode lookup (the CPU
baseline bench.py times) against the C oracle on the same inputs: the same
attention output on a tie-free cache (selection ties are where torch.topk
and the oracle's lowest-index rule may part)."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from oracle.torch_restatement import decode_lookup


def test_torch_restatement_matches_the_oracle():
    rng = np.random.default_rng(11)
    H, G, D, R, S, C, N, L, B = 9, 3, 64, 64, 4, 64, 3000, 512, 128
    q = rng.standard_normal((H, D)).astype(np.float32)
    q_proj = (rng.standard_normal((H, D, R)) / 8).astype(np.float32)
    scale = np.ones(H, np.float32)
    cb = rng.standard_normal((H, S, C, R // S)).astype(np.float32)
    k_low = rng.standard_normal((H, N, R)).astype(np.float32)
    codes = rng.integers(0, C, (H, N, S)).astype(np.uint8)
    keys = rng.standard_normal((G, N, D)).astype(np.float32)
    values = rng.standard_normal((G, N, D)).astype(np.float32)
    t = torch.from_numpy
    got = decode_lookup(t(q), t(q_proj), t(scale), t(cb), t(codes.astype(np.int64)), t(k_low), t(keys), t(values),
                        L, B, D ** -0.5).numpy()
    q_low = torch.einsum("hd,hdr->hr", t(q), t(q_proj)).mul_(t(scale)[:, None]).numpy()
    _, _, ref, _ = oracle.decode(q, q_low, keys, values, k_low, cb, codes, L, B, D ** -0.5)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= 1e-5, err
