"""Inverted-index decode paths on the GPU (sva/llama.py:330-576, :626-693).

``static_decode`` is ``_inverted_static_decode_attention``: postings built at
the last rebuild, every row behind them as a tail, unique refill selection,
margin-adaptive budget, fp32 exact verification.  ``adaptive_decode`` is
``_inverted_decode_attention``: every key whose code falls in a chosen cell
(postings plus the rows appended since their build), distinct candidates,
margin-adaptive budget.  Both run as three HIP launches (candidates, select,
verify) after the query LUT; nothing here runs on the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels
from ._lib import check, code_type, lib, ptr, require_device, stream_handle

# rows appended after a postings build that the adaptive path scans by code
# before rebuilding the postings
ADAPTIVE_TAIL_REBUILD = 256


@dataclass
class Postings:
    """CSR postings of the first ``key_len`` catalog rows."""

    offsets: torch.Tensor    # [H, S, C + 1] int32
    ids: torch.Tensor        # [H, S, key_len] int32, ascending within a cell
    max_count: torch.Tensor  # [H, S] int32, largest cell per (head, subspace)
    key_len: int


def build_postings(codes: torch.Tensor, key_len: int, codewords: int) -> Postings:
    """sva/llama.py:626-657 over rows [0, key_len) of codes [H, rows, S]."""

    heads, _, subspaces = codes.shape
    device = require_device(codes)
    offsets = torch.empty(heads, subspaces, codewords + 1, device=device, dtype=torch.int32)
    ids = torch.empty(heads, subspaces, max(key_len, 1), device=device, dtype=torch.int32)
    max_count = torch.empty(heads, subspaces, device=device, dtype=torch.int32)
    check(lib().sva_postings_build(ptr(codes), code_type(codes), codes.stride(0), heads, key_len, subspaces, codewords,
                                   ptr(offsets), ptr(ids), ptr(max_count), stream_handle(device)),
          "sva_postings_build")
    return Postings(offsets, ids, max_count, key_len)


def append_postings(postings: Postings | None, codes: torch.Tensor, k_len: int, codewords: int) -> Postings:
    """sva/llama.py:659-693.  Rows past the postings are found by the
    candidate kernel from their codes, which gives the same candidate set as
    appending them to the lists; the lists are rebuilt once that tail reaches
    ADAPTIVE_TAIL_REBUILD rows."""

    if postings is None or k_len - postings.key_len >= ADAPTIVE_TAIL_REBUILD or k_len < postings.key_len:
        return build_postings(codes, k_len, codewords)
    return postings


def _budgets(serving, max_budget: int, k_len: int) -> tuple[int, int, int]:
    """(min, mid, max) budgets (sva/llama.py:346-349, :443-445)."""

    min_b = min(serving.adaptive_min_budget or max_budget, max_budget, k_len)
    mid_b = min(serving.adaptive_mid_budget or max(min_b, max_budget // 2), max_budget, k_len)
    return min_b, mid_b, min(max_budget, k_len)


def top_unique_candidates(candidate_idx: torch.Tensor, candidate_scores: torch.Tensor, candidate_valid: torch.Tensor,
                          budget: int, refill_factor: int = 2):
    """sva/llama.py:83-116 on the GPU: returns (idx [H, k] int64, scores [H, k],
    valid [H, k], refill_count) with k = min(budget, refill_count); ties are
    broken by (score desc, key index asc)."""

    width = int(candidate_idx.shape[1])
    if width == 0 or budget <= 0:
        return candidate_idx[:, :0], candidate_scores[:, :0], candidate_valid[:, :0], 0
    device = require_device(candidate_idx, candidate_scores, candidate_valid)
    rows = candidate_idx.shape[0]
    refill = min(width, max(budget, budget * refill_factor))
    cap = min(budget, refill)
    idx = candidate_idx.to(torch.int64).contiguous()
    scores = candidate_scores.float().contiguous()
    valid = candidate_valid.to(torch.uint8).contiguous()
    sel_idx = torch.empty(rows, cap, device=device, dtype=torch.int32)
    sel_scores = torch.empty(rows, cap, device=device, dtype=torch.float32)
    sel_valid = torch.empty(rows, cap, device=device, dtype=torch.uint8)
    ws = kernels.workspace(device, int(lib().sva_top_unique_workspace_bytes(rows, width, budget, refill_factor)),
                           "top_unique")
    check(lib().sva_top_unique(ptr(idx), ptr(scores), ptr(valid), rows, width, budget, refill_factor, ptr(sel_idx),
                               ptr(sel_scores), ptr(sel_valid), ptr(ws), ws.numel(), stream_handle(device)),
          "sva_top_unique")
    return sel_idx.to(torch.int64), sel_scores.to(candidate_scores.dtype), sel_valid.bool(), refill


def _mask_row(mask: torch.Tensor | None, k_len: int):
    """The token's mask row for the candidate kernel: (tensor, mask type)."""

    m, mtype, _ = kernels.mask_args(mask, 1, k_len)
    return m, mtype


def _decode(module, query, keys, values, k_low, codes, k_len: int, mask, budget: int, adaptive: bool,
            return_selection: bool = False):
    serving = module.serving
    heads = query.shape[1]
    cb = module.sva_coarse_codebooks
    subspaces, codewords = int(cb.shape[1]), int(cb.shape[2])
    rank = serving.rank_dim
    cells = min(serving.inverted_cells_per_subspace, codewords)
    postings: Postings = module._postings
    device = query.device
    profile = serving.profile_components and not adaptive
    timings: dict[str, float] = {}
    t0 = module._profile_now(device) if profile else 0.0
    q_low, lut, _ = kernels.query_lut(query, module.sva_q_proj, module.sva_scale, cb)
    tail_start = min(max(postings.key_len, 0), k_len)
    slots = int(lib().sva_inverted_slots(subspaces, postings.key_len, k_len, tail_start))
    comp = torch.empty(heads, slots, device=device, dtype=torch.int64)
    flag = torch.empty(heads, slots, device=device, dtype=torch.uint8)
    m, mtype = _mask_row(mask, k_len)
    check(lib().sva_inverted_candidates(
        ptr(lut), ptr(q_low), ptr(k_low), k_low.stride(0), ptr(codes), code_type(codes), codes.stride(0),
        ptr(postings.offsets), ptr(postings.ids), postings.key_len, tail_start, k_len, heads, subspaces, codewords,
        rank, cells, ptr(m), mtype, 1 if adaptive else 0, ptr(comp), ptr(flag), slots, stream_handle(device)),
        "sva_inverted_candidates")
    if profile:
        timings["static_catalog_ms"] = module._profile_elapsed_ms(device, t0)
        t1 = module._profile_now(device)
    min_b, mid_b, max_b = _budgets(serving, budget, k_len)
    fin_idx = torch.empty(heads, max_b, device=device, dtype=torch.int32)
    fin_count = torch.empty(heads, device=device, dtype=torch.int32)
    stats = torch.empty(heads, 4, device=device, dtype=torch.float32)
    ws = kernels.workspace(device, int(lib().sva_unique_select_workspace_bytes(heads, max_b, 2, slots)), "inverted")
    tail_len = k_len - tail_start
    check(lib().sva_unique_refill_select(
        ptr(comp), ptr(flag), slots, heads, 1 if adaptive else 0, max_b, min_b, mid_b,
        float(serving.adaptive_low_margin), float(serving.adaptive_high_margin), 2, ptr(postings.max_count),
        subspaces, cells, tail_len, ptr(fin_idx), ptr(fin_count), ptr(stats), ptr(ws), ws.numel(),
        stream_handle(device)), "sva_unique_refill_select")
    if profile:
        timings["static_refill_ms"] = module._profile_elapsed_ms(device, t1)  # includes the budget choice
        t2 = module._profile_now(device)
    out = kernels.verify(query, keys, values, fin_idx, fin_count, k_len, module.scaling, out_dtype=query.dtype)
    if profile:
        timings["static_aggregate_ms"] = module._profile_elapsed_ms(device, t2)  # gather, exact score, softmax
        timings["static_total_ms"] = module._profile_elapsed_ms(device, t0)
    if module.stats is not None:
        values_ = {"summoned": stats[:, 0], "exact_scored": fin_count, "verified": fin_count,
                   "queries": float(heads), "cell_visits": float(heads * subspaces * cells)}
        if not adaptive:
            values_["refill_pool"] = stats[:, 1]
        if profile:
            values_["profile_calls"] = 1.0
            values_.update(timings)
        module.stats.add_device(int(module.layer_idx or 0), values_)
    if return_selection:
        return out, fin_idx, fin_count, stats
    return out


def static_decode(module, query, keys, values, k_low, codes, k_len: int, mask, budget: int,
                  return_selection: bool = False):
    """_inverted_static_decode_attention (sva/llama.py:427-576).  With
    return_selection: (out, fin_idx, fin_count, per-head stats)."""

    return _decode(module, query, keys, values, k_low, codes, k_len, mask, budget, False, return_selection)


def adaptive_decode(module, query, keys, values, k_low, codes, k_len: int, mask, budget: int,
                    return_selection: bool = False):
    """_inverted_decode_attention (sva/llama.py:330-425)."""

    return _decode(module, query, keys, values, k_low, codes, k_len, mask, budget, True, return_selection)

