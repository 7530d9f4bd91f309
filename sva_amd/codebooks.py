"""Product-codebook fits on the GPU (experiments/sva_pq_lookup_test.py:66-106,
experiments/sva_supervised_coarse_pq_test.py:88-131): k-means per (head,
subspace) over k_low rows, plain or weighted, in the reference's steps and
argument order.

Each iteration is three launches for every head and subspace at once:
assignment (sva_write_encode with an identity map: the nearest centroid of
each row, first index on ties), the cells as CSR (sva_postings_build, keys
ascending) and the centroid update (sva_centroid_update: cell means summed in
ascending key order, as index_add_ sums on the CPU; empty cells keep their
centroid).  The initial centroids are drawn with the reference's own seeded
torch calls on the fit's device (torch.randperm / torch.multinomial), so they
follow that device's generator; ``initial`` overrides them.
"""

from __future__ import annotations

import torch

from . import inverted, kernels
from ._lib import check, lib, ptr, require_device, stream_handle


def _initial(x: torch.Tensor, head_weights: torch.Tensor | None, seed: int, head: int, subspace: int,
             codewords: int) -> torch.Tensor:
    generator = torch.Generator(device=x.device)
    generator.manual_seed(seed + head * 9973 + subspace * 131 + codewords)
    if head_weights is None:
        pick = torch.randperm(x.shape[0], generator=generator, device=x.device)[:codewords]
    else:
        probs = head_weights / head_weights.sum().clamp_min(1e-6)
        pick = torch.multinomial(probs, codewords, replacement=False, generator=generator)
    return x[pick].clone()


@torch.no_grad()
def _fit(k_low: torch.Tensor, weights: torch.Tensor | None, subspaces: int, codewords: int, iterations: int,
         seed: int, initial: torch.Tensor | None) -> torch.Tensor:
    heads, seq_len, rank = k_low.shape
    if rank % subspaces != 0:
        raise ValueError(f"rank_dim={rank} must be divisible by subspaces={subspaces}")
    if weights is not None and tuple(weights.shape) != (heads, seq_len):
        raise ValueError("Weight shape must match key heads and sequence length.")
    sub = rank // subspaces
    c_eff = min(codewords, seq_len)
    device = require_device(k_low, weights, initial)
    x = k_low.float().contiguous()
    w = None
    if weights is not None:
        w = weights.float().clamp_min(1e-6).contiguous()
    if initial is not None:
        cent = initial.float().contiguous().clone()
        if tuple(cent.shape) != (heads, subspaces, c_eff, sub):
            raise ValueError(f"initial centroids must be [{heads}, {subspaces}, {c_eff}, {sub}]")
    else:
        cent = torch.stack([torch.stack([_initial(x[h, :, s * sub:(s + 1) * sub], None if w is None else w[h], seed,
                                                  h, s, c_eff) for s in range(subspaces)]) for h in range(heads)])
    eye = torch.eye(rank, device=device).expand(heads, rank, rank).contiguous()
    scratch = torch.empty_like(x)
    codes = torch.empty(heads, seq_len, subspaces, device=device,
                        dtype=torch.uint8 if c_eff <= 256 else torch.int16)
    nxt = torch.empty_like(cent)
    stream = stream_handle(device)
    for _ in range(iterations):
        kernels.write_encode(x, eye, cent, scratch, codes)  # labels: nearest centroid per (row, subspace)
        post = inverted.build_postings(codes, seq_len, c_eff)
        check(lib().sva_centroid_update(ptr(x), x.stride(0), seq_len, heads, rank, subspaces, c_eff, ptr(w),
                                        ptr(post.offsets), ptr(post.ids), ptr(cent), ptr(nxt), stream),
              "sva_centroid_update")
        cent, nxt = nxt, cent
    return cent.to(k_low.dtype)


def fit_product_codebooks(k_low: torch.Tensor, subspaces: int, codewords: int, iterations: int, seed: int,
                          chunk_size: int = 8192, initial: torch.Tensor | None = None) -> torch.Tensor:
    """experiments/sva_pq_lookup_test.py:66-106: codebooks [H, S, min(C, N), R / S].
    chunk_size (the reference's assignment chunking) does not change the result."""

    return _fit(k_low, None, subspaces, codewords, iterations, seed, initial)


def fit_weighted_product_codebooks(k_low: torch.Tensor, weights: torch.Tensor, subspaces: int, codewords: int,
                                   iterations: int, seed: int, chunk_size: int = 8192,
                                   initial: torch.Tensor | None = None) -> torch.Tensor:
    """experiments/sva_supervised_coarse_pq_test.py:88-131 (weights clamped at 1e-6)."""

    return _fit(k_low, weights, subspaces, codewords, iterations, seed, initial)
