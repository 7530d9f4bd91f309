"""Seeded synthetic inputs shared by the tests (numpy on the host)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class Case:
    H: int
    G: int
    N: int
    D: int
    R: int
    S: int
    C: int
    q: np.ndarray          # [H, Q, D] fp32 (values representable in the kv dtype)
    keys: np.ndarray       # [G, N, D]
    values: np.ndarray     # [G, N, D]
    k_low: np.ndarray      # [H, N, R] fp32
    q_proj: np.ndarray     # [H, D, R]
    k_proj: np.ndarray     # [H, D, R]
    scale: np.ndarray      # [H]
    codebooks: np.ndarray  # [H, S, C, R/S]
    codes: np.ndarray      # [H, N, S] uint8 / int16
    dtype: torch.dtype

    def t(self, name: str, device, dtype=None):
        a = getattr(self, name)
        t = torch.from_numpy(np.ascontiguousarray(a))
        if dtype is not None:
            t = t.to(dtype)
        return t.to(device)


def round_to(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype).float().numpy()


def make_case(H=9, G=3, N=8192, D=64, R=64, S=2, C=256, Q=1, dtype=torch.float32, seed=0,
              code_mode="random", ties=False) -> Case:
    """Random GQA cache.  code_mode='random' draws uniform codes; 'few' draws
    from 3 codewords per subspace (massive exact ties)."""

    rng = np.random.default_rng(seed)
    f = np.float32
    q = round_to(rng.standard_normal((H, Q, D)).astype(f), dtype)
    keys = round_to(rng.standard_normal((G, N, D)).astype(f), dtype)
    values = round_to(rng.standard_normal((G, N, D)).astype(f), dtype)
    k_low = rng.standard_normal((H, N, R)).astype(f)
    q_proj = (rng.standard_normal((H, D, R)) / 8.0).astype(f)
    k_proj = (rng.standard_normal((H, D, R)) / 8.0).astype(f)
    scale = np.exp(rng.standard_normal(H).astype(f) * 0.1).astype(f)
    codebooks = rng.standard_normal((H, S, C, R // S)).astype(f)
    code_dtype = np.uint8 if C <= 256 else np.int16
    if code_mode == "few":
        codes = rng.integers(0, min(3, C), size=(H, N, S)).astype(code_dtype)
    else:
        codes = rng.integers(0, C, size=(H, N, S)).astype(code_dtype)
    if ties:
        # duplicate k_low rows so rank scores tie exactly
        k_low[:, 1::2] = k_low[:, 0::2][:, : k_low[:, 1::2].shape[1]]
    return Case(H, G, N, D, R, S, C, q, keys, values, k_low, q_proj, k_proj, scale, codebooks, codes, dtype)


def lookup8192_inputs(seed: int = 20260514):
    """The single-layer decode lookup of the reference's CPU-runnable case:
    8192 cached keys, head_dim 64, 9 query heads over 3 KV heads, K/V/q iid
    N(0, 1) fp32, learned maps N(0, 1/64) of rank 64, 2 x 256 PQ codebooks of
    width 32 drawn N(0, 1), logit scale field 0 (multiplier 1.0), shortlist
    2048, budget 512, one query token.  numpy only, so the GPU tests and the
    fixture writer draw identical inputs."""

    rng = np.random.default_rng(seed)
    H, G, N, D, R, S, C = 9, 3, 8192, 64, 64, 2, 256
    return {
        "q": rng.standard_normal((H, 1, D)).astype(np.float32),
        "keys": rng.standard_normal((G, N, D)).astype(np.float32),
        "values": rng.standard_normal((G, N, D)).astype(np.float32),
        "q_proj": (rng.standard_normal((H, D, R)) / 8).astype(np.float32),
        "k_proj": (rng.standard_normal((H, D, R)) / 8).astype(np.float32),
        "logit_scale": np.zeros(H, np.float32),
        "codebooks": rng.standard_normal((H, S, C, R // S)).astype(np.float32),
        "shortlist": 2048,
        "budget": 512,
    }


# Inverted-index decode cases recorded from the reference's own
# _inverted_static_decode_attention / _inverted_decode_attention
# (tests/golden/make_inverted_golden.py writes inverted_reference.npz).
# mode, N, tail (static: rows behind the postings), budget, cells, adaptive
# min / mid budgets (0 = the reference's default), low / high margins,
# fraction of keys masked out (0: no mask), current row masked, seed.
INVERTED_CASES = [
    ("inverted_static", 6000, 10, 128, 8, 0, 0, 0.35, 0.70, 0.0, False, 101),
    ("inverted_static", 6000, 0, 128, 8, 32, 64, 0.35, 0.70, 0.0, False, 102),
    ("inverted_static", 6000, 37, 512, 8, 16, 48, 0.35, 0.70, 0.3, False, 103),
    ("inverted_static", 6000, 63, 64, 8, 1, 2, 0.20, 1.20, 0.0, False, 104),
    ("inverted_static", 6000, 0, 256, 4, 0, 0, 0.35, 0.70, 0.4, True, 105),
    ("inverted_static", 6000, 5, 128, 8, 8, 32, 0.60, 1.00, 0.0, False, 106),
    ("inverted", 6000, 0, 128, 8, 0, 0, 0.35, 0.70, 0.0, False, 201),
    ("inverted", 6000, 0, 128, 8, 16, 48, 0.35, 0.70, 0.0, False, 202),
    ("inverted", 6000, 0, 64, 8, 32, 48, 0.20, 1.20, 0.4, True, 203),
    ("inverted", 6000, 0, 512, 8, 0, 0, 0.35, 0.70, 0.0, False, 204),
    ("inverted", 6000, 0, 128, 8, 8, 32, 0.60, 1.00, 0.1, False, 207),
    # almost every key masked: heads whose chosen cells hold no allowed key
    # fall back to the last allowed row
    ("inverted", 500, 0, 16, 2, 0, 0, 0.35, 0.70, 0.995, True, 205),
]


def inverted_inputs(seed: int, N: int, mask_frac: float = 0.0, current_masked: bool = False,
                    H: int = 9, G: int = 3, D: int = 64, R: int = 64, S: int = 2, C: int = 256):
    """Seeded decode inputs of one token over an N-key catalog (numpy only):
    q [H, 1, D], keys / values [G, N, D] N(0, 1); q_proj [H, D, R] N(0, 1/64),
    logit scale field 0.1 * N(0, 1); codebooks [H, S, C, R/S] N(0, 1); the
    catalog itself drawn directly: k_low [H, N, R] N(0, 1) and codes uniform
    in [0, C); allowed [N] (mask_frac of the keys masked out, the current
    row too when current_masked)."""

    rng = np.random.default_rng(seed)
    f = np.float32
    out = {
        "q": rng.standard_normal((H, 1, D)).astype(f),
        "keys": rng.standard_normal((G, N, D)).astype(f),
        "values": rng.standard_normal((G, N, D)).astype(f),
        "q_proj": (rng.standard_normal((H, D, R)) / 8).astype(f),
        "logit_scale": (0.1 * rng.standard_normal(H)).astype(f),
        "codebooks": rng.standard_normal((H, S, C, R // S)).astype(f),
        "k_low": rng.standard_normal((H, N, R)).astype(f),
        "codes": rng.integers(0, C, (H, N, S)).astype(np.uint8),
    }
    allowed = rng.random(N) >= mask_frac
    if current_masked:
        allowed[N - 1] = False
    out["allowed"] = allowed
    return out
