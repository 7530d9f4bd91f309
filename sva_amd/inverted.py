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



@dataclass
class RaggedPostings:
    """CSR postings of every sequence of a packed batch: sequence b's first
    ``postings_lens[b]`` keys."""

    offsets: torch.Tensor        # [n_seq, H, S, C + 1] int32
    ids: torch.Tensor            # [H, S, rows] int32: sequence b's local ids at its packed rows
    max_count: torch.Tensor      # [n_seq, H, S] int32
    postings_lens: torch.Tensor  # [n_seq] int64
    max_len: int                 # the largest postings length


def build_postings_ragged(codes: torch.Tensor, seq_offsets: torch.Tensor, postings_lens: torch.Tensor,
                          max_len: int, codewords: int) -> RaggedPostings:
    """sva/llama.py:626-657 for every sequence of a packed batch at once:
    codes [H, rows, S] packed; seq_offsets / postings_lens int64 [n_seq] on
    the device; max_len the largest of postings_lens."""

    heads, rows, subspaces = codes.shape
    n_seq = int(seq_offsets.numel())
    device = require_device(codes, seq_offsets, postings_lens)
    offsets = torch.empty(n_seq, heads, subspaces, codewords + 1, device=device, dtype=torch.int32)
    ids = torch.empty(heads, subspaces, rows, device=device, dtype=torch.int32)
    max_count = torch.empty(n_seq, heads, subspaces, device=device, dtype=torch.int32)
    check(lib().sva_postings_build_ragged(ptr(codes), code_type(codes), codes.stride(0), ptr(seq_offsets),
                                          ptr(postings_lens), n_seq, heads, rows, subspaces, codewords, ptr(offsets),
                                          ptr(ids), ptr(max_count), stream_handle(device)),
          "sva_postings_build_ragged")
    return RaggedPostings(offsets, ids, max_count, postings_lens, int(max_len))


def ragged_static_decode(query, q_proj, scale, codebooks, keys, values, k_low, codes, seq_offsets, k_lens,
                         postings: RaggedPostings, max_tail: int, budget: int, cells: int, scaling: float,
                         adaptive_min: int | None = None, adaptive_mid: int | None = None, low_margin: float = 0.35,
                         high_margin: float = 0.70, return_selection: bool = False):
    """_inverted_static_decode_attention (sva/llama.py:427-576) for one decode
    token of every sequence of a packed batch, in four launches (query LUT,
    candidates, selection, verifier) whatever the batch size.

    query [n_seq, H, 1, D]; keys / values [G, rows, D], k_low [H, rows, R] and
    codes [H, rows, S] packed, sequence b at rows [seq_offsets[b],
    seq_offsets[b] + k_lens[b]); max_tail >= every k_lens[b] -
    postings_lens[b].  Returns out [n_seq, H, 1, D] (and, with
    return_selection, fin_idx / fin_count / stats per item b * H + h, keys
    local to their sequence)."""

    n_seq, heads, q_len, head_dim = query.shape
    if q_len != 1:
        raise ValueError("ragged static decode takes one token per sequence")
    subspaces, codewords = int(codebooks.shape[1]), int(codebooks.shape[2])
    rank = int(q_proj.shape[-1])
    rows = int(codes.shape[1])
    device = require_device(query, keys, values, k_low, codes, seq_offsets, k_lens)
    cells = min(cells, codewords)
    q_low, lut, _ = kernels.query_lut(query, q_proj, scale, codebooks)
    L = lib()
    slots = int(L.sva_inverted_slots_ragged(subspaces, postings.max_len, max_tail))
    items = n_seq * heads
    comp = torch.empty(items, slots, device=device, dtype=torch.int64)
    flag = torch.empty(items, slots, device=device, dtype=torch.uint8)
    list_counts = torch.empty(items, device=device, dtype=torch.int32)
    stream = stream_handle(device)
    check(L.sva_inverted_candidates_ragged(
        ptr(lut), ptr(q_low), ptr(k_low), k_low.stride(0), ptr(codes), code_type(codes), codes.stride(0),
        ptr(postings.offsets), ptr(postings.ids), rows, ptr(seq_offsets), ptr(postings.postings_lens), ptr(k_lens),
        n_seq, postings.max_len, max_tail, heads, subspaces, codewords, rank, cells, ptr(comp), ptr(flag),
        ptr(list_counts), slots, stream), "sva_inverted_candidates_ragged")
    fin_idx = torch.empty(items, budget, device=device, dtype=torch.int32)
    fin_count = torch.empty(items, device=device, dtype=torch.int32)
    stats = torch.empty(items, 4, device=device, dtype=torch.float32)
    ws = kernels.workspace(device, int(L.sva_unique_select_workspace_bytes(items, budget, 2, slots)), "inverted")
    check(L.sva_unique_refill_select_ragged(
        ptr(comp), ptr(flag), slots, n_seq, heads, budget, adaptive_min or 0, adaptive_mid or 0, float(low_margin),
        float(high_margin), 2, ptr(postings.max_count), subspaces, cells, ptr(postings.postings_lens), ptr(k_lens),
        ptr(list_counts), postings.max_len, ptr(fin_idx), ptr(fin_count), ptr(stats), ptr(ws), ws.numel(), stream),
        "sva_unique_refill_select_ragged")
    out = kernels.verify(query, keys, values, fin_idx, fin_count, rows, scaling, out_dtype=query.dtype,
                         seq_offsets=seq_offsets, seq_lens=k_lens)
    if return_selection:
        return out, fin_idx, fin_count, stats
    return out
