"""The reference's core tensor operations (sva/ops.py:10-71) on the GPU, with
the reference's names, signatures and results.

Each call is one or two HIP launches over every head and subspace at once:
``encode_product_keys`` and ``assign_to_centroids`` run ``sva_write_encode``
with an identity map (the map's fma chain reproduces the rows exactly) so the
nearest codeword of every (row, subspace) comes from the write path's
distance arithmetic, first index on ties; ``product_quantized_scores`` runs
``sva_query_lut`` with an identity map and unit scale (the table
``q_part @ codebook.T``) and ``sva_pq_scores`` (the sum over subspaces in
ascending order, then ``/ sqrt(rank_dim)``).  ``chunk_size`` is the
reference's CPU memory bound; it does not change a result here.

Tensors must live on a ROCm device: these functions have no CPU path.
"""

from __future__ import annotations

import torch

from . import kernels
from ._lib import require_device


def _eye(heads: int, dim: int, device: torch.device) -> torch.Tensor:
    return torch.eye(dim, device=device, dtype=torch.float32).expand(heads, dim, dim).contiguous()


@torch.no_grad()
def encode_product_keys(k_low: torch.Tensor, codebooks: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """Product-quantization codes int64 [H, N, S] of k_low [H, N, R] against
    codebooks [H, S, C, R / S] (sva/ops.py:24-47)."""

    if k_low.dim() != 3 or codebooks.dim() != 4 or codebooks.shape[0] != k_low.shape[0]:
        raise ValueError(f"k_low [H, N, R] and codebooks [H, S, C, R/S] expected, got {tuple(k_low.shape)} and "
                         f"{tuple(codebooks.shape)}")
    n_heads, seq_len, rank_dim = k_low.shape
    subspaces = codebooks.shape[1]
    if rank_dim % subspaces != 0:
        raise ValueError(f"rank_dim={rank_dim} must be divisible by subspaces={subspaces}.")
    if codebooks.shape[3] != rank_dim // subspaces:
        raise ValueError(f"codebook width {codebooks.shape[3]} != rank_dim / subspaces = {rank_dim // subspaces}")
    device = require_device(k_low, codebooks)
    codes = torch.empty(n_heads, seq_len, subspaces, device=device, dtype=torch.int64)
    if seq_len == 0:
        return codes
    x = k_low.float().contiguous()
    copy = torch.empty_like(x)  # the identity map's output, discarded
    kernels.write_encode(x, _eye(n_heads, rank_dim, device), codebooks, copy, codes)
    return codes


@torch.no_grad()
def assign_to_centroids(x: torch.Tensor, centroids: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """Nearest centroid int64 [N] of each row of x [N, d] by squared L2
    distance, lowest index on ties (sva/ops.py:10-21)."""

    if x.dim() != 2 or centroids.dim() != 2 or x.shape[1] != centroids.shape[1]:
        raise ValueError(f"x [N, d] and centroids [C, d] expected, got {tuple(x.shape)} and {tuple(centroids.shape)}")
    return encode_product_keys(x[None], centroids[None, None], chunk_size)[0, :, 0]


@torch.no_grad()
def product_quantized_scores(q_low: torch.Tensor, codebooks: torch.Tensor, codes: torch.Tensor,
                             rank_dim: int) -> torch.Tensor:
    """Approximate low-rank scores fp32 [H, Q, N] of q_low [H, Q, R] against
    the codes [H, N, S] of the cached keys (sva/ops.py:50-71).  A code
    outside [0, C) raises IndexError, as the reference's gather does."""

    if q_low.dim() != 3 or codes.dim() != 3 or codebooks.dim() != 4:
        raise ValueError(f"q_low [H, Q, R], codebooks [H, S, C, R/S] and codes [H, N, S] expected, got "
                         f"{tuple(q_low.shape)}, {tuple(codebooks.shape)}, {tuple(codes.shape)}")
    n_heads, n_queries, width = q_low.shape
    subspaces, codewords = codebooks.shape[1], codebooks.shape[2]
    if width != rank_dim or rank_dim % subspaces != 0 or codebooks.shape[3] != rank_dim // subspaces:
        raise ValueError(f"q_low width {width}, rank_dim {rank_dim} and codebooks {tuple(codebooks.shape)} disagree")
    if codes.shape[0] != n_heads or codes.shape[2] != subspaces or codebooks.shape[0] != n_heads:
        raise ValueError(f"codes {tuple(codes.shape)} do not match {n_heads} heads x {subspaces} subspaces")
    device = require_device(q_low, codebooks, codes)
    seq_len = codes.shape[1]
    if seq_len == 0 or n_queries == 0:
        return torch.zeros(n_heads, n_queries, seq_len, device=device, dtype=torch.float32)
    if bool(((codes < 0) | (codes >= codewords)).any()):
        raise IndexError(f"product_quantized_scores: a code lies outside [0, {codewords})")
    if codes.dtype not in (torch.uint8, torch.int16, torch.int32, torch.int64):
        codes = codes.long()
    codes = codes.contiguous()
    ones = torch.ones(n_heads, device=device, dtype=torch.float32)
    _, lut, _ = kernels.query_lut(q_low.float()[None], _eye(n_heads, rank_dim, device), ones, codebooks)
    return kernels.pq_scores(lut, codes, seq_len, rank_dim)[0]
