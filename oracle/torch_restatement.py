"""Torch-CPU restatement of the reference's q = 1 decode lookup, for timing.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: the ``cpu_baseline``
leg of ``bench.py`` times it on the host's cores, and ``tests/`` check it
against the C oracle.  It runs the reference's own torch operations in their
order on the CPU (the reference is pure torch), so its time is the
reference's arithmetic on this host; selection ties follow ``torch.topk``,
as the reference's do.

Follows ``sva/llama.py:211`` (q_low), ``sva/ops.py:50-71`` (table, gather-sum,
/ sqrt(R)), ``sva/llama.py:276-302`` (topk(L), k_low gather, rank, topk(B)),
``sva/llama.py:304-317`` with the fp32 scores of ``:532-553`` and
``experiments/sva_million_cached_decode_benchmark.py:203-221`` (verifier).
"""

from __future__ import annotations

import math

import torch


def decode_lookup(q: torch.Tensor, q_proj: torch.Tensor, scale: torch.Tensor, codebooks: torch.Tensor,
                  codes: torch.Tensor, k_low: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                  shortlist: int, budget: int, scaling: float) -> torch.Tensor:
    """One decode token: q [H, D] fp32, q_proj [H, D, R], scale [H], codebooks
    [H, S, C, R/S], codes [H, N, S] int64, k_low [H, N, R] fp32, keys / values
    [G, N, D] fp32.  Returns the attention output [H, D] fp32."""

    heads, n, subspaces = codes.shape
    rank = q_proj.shape[-1]
    q_low = torch.einsum("hd,hdr->hr", q, q_proj) * scale[:, None]                    # sva/llama.py:211
    parts = q_low.view(heads, subspaces, rank // subspaces)
    lut = torch.einsum("hsd,hscd->hsc", parts, codebooks)                             # sva/ops.py:66-68
    scores = torch.zeros(heads, n)                                                    # sva/ops.py:64
    for s in range(subspaces):
        scores += torch.gather(lut[:, s], 1, codes[:, :, s])                          # sva/ops.py:69
    scores = scores / math.sqrt(rank)                                                 # sva/ops.py:71
    top = scores.topk(min(shortlist, n), dim=-1).indices                              # sva/llama.py:276-284
    rows = torch.gather(k_low, 1, top[..., None].expand(-1, -1, rank))                # sva/llama.py:286-291
    ranks = (rows * q_low[:, None, :]).sum(-1) / math.sqrt(rank)                      # sva/llama.py:292
    chosen = ranks.topk(min(budget, top.shape[1]), dim=-1).indices                    # sva/llama.py:295
    final = top.gather(1, chosen)                                                     # sva/llama.py:296
    group = heads // keys.shape[0]
    kv = torch.arange(heads) // group                                                 # repeat_kv's head map
    k_rows = keys[kv[:, None], final]                                                 # sva/llama.py:304-313
    v_rows = values[kv[:, None], final]
    att = (k_rows * q[:, None, :]).sum(-1) * scaling                                  # fp32 scores, :545
    weights = torch.softmax(att, dim=-1)                                              # :546-553
    return (weights[..., None] * v_rows).sum(1)
