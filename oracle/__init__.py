"""CPU oracle for the SVA summon -> verify decode path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker.  The shipped ``sva_amd`` package never imports it and has no CPU
fallback.

Arithmetic lives in ``sva_oracle.c`` (built by ``oracle/Makefile`` into
``libsva_oracle.so``); this module restates the index / selection / catalog
logic of the reference on top of it with numpy.  Each function names the
reference lines it follows.

Selection rule used everywhere: top-k by (score descending, key index
ascending).  torch.topk leaves ties unspecified; the rule fixes them.

Pinning (what checks each function; see tests/test_oracle.py):
  torch_sum, project, assign_to_centroids, encode_product_keys
      bit-exact against torch-CPU's own sum / many-row einsum / matmul on the
      same inputs, brute force fp64 argmin away from near-ties.
  lut, product_quantized_scores
      LUT: within 2 ulp of torch's matmul and of fp64; scan score: closed form
      given the LUT (sequential sum, exact division by sqrt(R)), invariant
      "equal codes give equal scores".
  topk
      against numpy lexsort on (score desc, idx asc) including tie-heavy input.
  top_unique_candidates
      the reference's known-answer test (tests/test_sva_llama_adapter.py:58-73)
      and brute force.
  verify
      fp64 closed form (softmax-weighted sum) against a float64 torch softmax.
  rebuild_postings
      partition and bincount invariants, brute-force membership.
  static_decode / inverted_decode / cell_choice
      the reference's own _inverted_static_decode_attention and
      _inverted_decode_attention recorded on seeded tie-free cases
      (tests/golden/inverted_reference.npz): candidate, refill and final
      sets, stats and outputs; a planted wrong cell rule is caught.
  residual_adapter
      torch-CPU's own nn.Linear / F.gelu module of the reference on the same
      inputs (float64), the zero-initialised up projection (output = input),
      and gelu at known points.
  kmeans_update / kmeans_fit
      bit-exact against the reference's update step run by torch-CPU
      (index_add_, bincount, division) on the same labels, plain and weighted;
      empty cells keep their centroid.
  topk_key_weights
      closed form (a key with c hits weighs the c-fold rounded sum
      1 + boost + ... + boost) and torch-CPU's index_add_ on the same hits,
      invalid and out-of-range entries included.
  topk_targets
      brute force per row (sort of the allowed keys), causal counts
      (valid entries = min(k, position + 1)), every valid key at or before
      its query's position.
  query_positions
      torch.linspace(...).long().unique() on the CPU for a sweep of lengths,
      sample counts and start rows.
  golden fixtures (tests/golden/) written from the reference's own functions.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libsva_oracle.so"
_lib: ctypes.CDLL | None = None

F32 = np.float32
FMIN = np.finfo(np.float32).min


def build() -> Path:
    """Compile libsva_oracle.so with the committed Makefile."""

    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        c_p = ctypes.c_void_p
        i64 = ctypes.c_int64
        _lib.sva_oracle_torch_sum.restype = ctypes.c_float
        _lib.sva_oracle_torch_sum.argtypes = [c_p, i64]
        _lib.sva_oracle_torch_dot.restype = ctypes.c_float
        _lib.sva_oracle_torch_dot.argtypes = [c_p, c_p, i64]
        _lib.sva_oracle_float_key.restype = ctypes.c_uint32
        _lib.sva_oracle_float_key.argtypes = [ctypes.c_float]
        _lib.sva_oracle_project.argtypes = [c_p, i64, i64, c_p, i64, i64, c_p]
        _lib.sva_oracle_assign.argtypes = [c_p, i64, i64, i64, c_p, i64, c_p, c_p]
        _lib.sva_oracle_lut.argtypes = [c_p, i64, i64, i64, c_p, c_p]
        _lib.sva_oracle_pq_scores.argtypes = [c_p, i64, i64, c_p, ctypes.c_int, i64, i64, ctypes.c_float, c_p]
        _lib.sva_oracle_rank_scores.argtypes = [c_p, i64, c_p, i64, c_p, ctypes.c_float, c_p]
        _lib.sva_oracle_topk.restype = i64
        _lib.sva_oracle_topk.argtypes = [c_p, c_p, c_p, i64, i64, c_p]
        _lib.sva_oracle_verify.argtypes = [c_p, c_p, c_p, i64, c_p, i64, ctypes.c_double, c_p]
        _lib.sva_oracle_decode.restype = ctypes.c_int
        _lib.sva_oracle_decode.argtypes = [i64] * 8 + [c_p] * 7 + [ctypes.c_int, i64, i64, ctypes.c_double, c_p, c_p, c_p]
    return _lib


def _ptr(a: np.ndarray | None) -> ctypes.c_void_p | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=F32))


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def sqrt_f32(r: int) -> float:
    """fp32 value of math.sqrt(r) as torch uses it when dividing an fp32 tensor."""

    return float(F32(math.sqrt(r)))


def float_key(x: float) -> int:
    return int(lib().sva_oracle_float_key(float(x)))


# --------------------------------------------------------------------------
# arithmetic primitives


def torch_sum(x) -> np.ndarray:
    """torch.sum(dim=-1) of an fp32 array, bit-exact with torch's CPU kernel."""

    x = _f32(x)
    k = x.shape[-1]
    flat = x.reshape(-1, k)
    out = np.empty(flat.shape[0], F32)
    for i in range(flat.shape[0]):
        row = np.ascontiguousarray(flat[i])
        out[i] = lib().sva_oracle_torch_sum(_ptr(row), k)
    return out.reshape(x.shape[:-1])


def project(x, w) -> np.ndarray:
    """x [..., D] @ w [D, R] with a sequential fmaf chain over D
    (sva/llama.py:211 and :598/:615 einsums)."""

    x = _f32(x)
    w = _f32(w)
    d, r = w.shape
    flat = x.reshape(-1, d)
    out = np.empty((flat.shape[0], r), F32)
    lib().sva_oracle_project(_ptr(flat), flat.shape[0], d, _ptr(w), d, r, _ptr(out))
    return out.reshape(*x.shape[:-1], r)


def assign_to_centroids(x, centroids, return_gap: bool = False):
    """sva/ops.py:10-21 (chunking does not change per-row arithmetic)."""

    x = _f32(x)
    cb = _f32(centroids)
    n, sub = x.shape
    labels = np.empty(n, np.int64)
    gap = np.empty(n, F32)
    lib().sva_oracle_assign(_ptr(x), n, sub, sub, _ptr(cb), cb.shape[0], _ptr(labels), _ptr(gap))
    return (labels, gap) if return_gap else labels


def encode_product_keys(k_low, codebooks, return_gap: bool = False):
    """sva/ops.py:24-47: codes [H, N, S] int64 (plus per-code top-2 distance gap)."""

    k_low = _f32(k_low)
    codebooks = _f32(codebooks)
    h_count, n, rank = k_low.shape
    subspaces = codebooks.shape[1]
    if rank % subspaces != 0:
        raise ValueError(f"rank_dim={rank} must be divisible by subspaces={subspaces}.")
    sub = rank // subspaces
    codes = np.empty((h_count, n, subspaces), np.int64)
    gaps = np.empty((h_count, n, subspaces), F32)
    for h in range(h_count):
        for s in range(subspaces):
            part = np.ascontiguousarray(k_low[h, :, s * sub : (s + 1) * sub])
            codes[h, :, s], gaps[h, :, s] = assign_to_centroids(part, codebooks[h, s], return_gap=True)
    return (codes, gaps) if return_gap else codes


def lut(q_low_h, codebooks_h) -> np.ndarray:
    """Per-query table [S, C] for one head (sva/ops.py:68)."""

    q = _f32(q_low_h)
    cb = _f32(codebooks_h)
    s_count, c_count, sub = cb.shape
    out = np.empty((s_count, c_count), F32)
    lib().sva_oracle_lut(_ptr(q), s_count, c_count, sub, _ptr(cb), _ptr(out))
    return out


def pq_scores_from_lut(table, codes_h, rank_dim: int) -> np.ndarray:
    """Scores [N] for one head and one query given its table (sva/ops.py:64-71)."""

    table = _f32(table)
    codes_h = np.ascontiguousarray(codes_h)
    n, s_count = codes_h.shape
    width = codes_h.dtype.itemsize
    if width not in (1, 2, 4, 8):
        raise ValueError("codes must be 1, 2, 4 or 8 bytes wide")
    out = np.empty(n, F32)
    lib().sva_oracle_pq_scores(
        _ptr(table), s_count, table.shape[1], _ptr(codes_h), width, n, s_count, sqrt_f32(rank_dim), _ptr(out)
    )
    return out


def product_quantized_scores(q_low, codebooks, codes, rank_dim: int) -> np.ndarray:
    """sva/ops.py:50-71: q_low [H, Q, R], codes [H, N, S] -> scores [H, Q, N]."""

    q_low = _f32(q_low)
    h_count, q_count, _ = q_low.shape
    n = codes.shape[1]
    out = np.empty((h_count, q_count, n), F32)
    for h in range(h_count):
        for t in range(q_count):
            out[h, t] = pq_scores_from_lut(lut(q_low[h, t], codebooks[h]), codes[h], rank_dim)
    return out


def rank_scores(k_low_h, idx, q_low_ht, rank_dim: int) -> np.ndarray:
    """sum(k_low[idx] * q_low) / sqrt(R) in torch's sum order (sva/llama.py:292, :495)."""

    k_low_h = _f32(k_low_h)
    idx = _i64(idx)
    q = _f32(q_low_ht)
    out = np.empty(idx.shape[0], F32)
    lib().sva_oracle_rank_scores(_ptr(k_low_h), k_low_h.shape[1], _ptr(idx), idx.shape[0], _ptr(q), sqrt_f32(rank_dim), _ptr(out))
    return out


def topk(scores, k: int, allowed=None, key_index=None) -> np.ndarray:
    """Positions of the top-k allowed entries by (score desc, key index asc).

    ``key_index`` maps position -> key index for the tie rule (defaults to the
    position).  Returns min(k, #allowed) positions in selection order."""

    scores = _f32(scores)
    n = scores.shape[0]
    allowed_arr = None if allowed is None else np.ascontiguousarray(np.asarray(allowed, dtype=np.uint8))
    key_arr = None if key_index is None else _i64(key_index)
    out = np.empty(max(min(k, n), 1), np.int64)
    got = lib().sva_oracle_topk(_ptr(scores), _ptr(allowed_arr), _ptr(key_arr), n, k, _ptr(out))
    return out[:got].copy()


def verify(q_ht, keys, values, idx, scaling: float) -> np.ndarray:
    """Float64 softmax(scaling * K[idx].q) @ V[idx] (sva/llama.py:304-317)."""

    q = _f32(q_ht)
    keys = _f32(keys)
    values = _f32(values)
    idx = _i64(idx)
    out = np.empty(keys.shape[1], np.float64)
    lib().sva_oracle_verify(_ptr(q), _ptr(keys), _ptr(values), keys.shape[1], _ptr(idx), idx.shape[0], float(scaling), _ptr(out))
    return out


# --------------------------------------------------------------------------
# attention paths of sva/llama.py, one layer call at a time.  Tensors are numpy:
# query [H, Q, D]; keys/values [G, N, D]; k_low [H, N, R]; codes [H, N, S].


def allowed_mask(q_len: int, k_len: int, attention_mask=None) -> np.ndarray:
    """sva/llama.py:188-198 for batch 1: bool [Q, N] (same for every head)."""

    if attention_mask is not None:
        m = np.asarray(attention_mask)
        m = m.reshape(-1, *m.shape[-2:])[0][:q_len, :k_len]
        if m.dtype == np.bool_:
            # bool > -1e4 is True for True and False alike (the reference's rule)
            return np.ones((q_len, k_len), bool)
        return m.astype(np.float64) > -1e4
    key_pos = np.arange(k_len)
    query_pos = np.arange(q_len) if q_len == k_len else np.arange(k_len - q_len, k_len)
    return key_pos[None, :] <= query_pos[:, None]


def query_low(query, q_proj, sva_scale) -> np.ndarray:
    """q_low = einsum(q, q_proj) * scale (sva/llama.py:211).  query [H, Q, D]."""

    query = _f32(query)
    q_proj = _f32(q_proj)
    scale = _f32(sva_scale)
    out = np.empty((query.shape[0], query.shape[1], q_proj.shape[2]), F32)
    for h in range(query.shape[0]):
        out[h] = project(query[h], q_proj[h]) * scale[h]
    return out


def scan_attention(query, keys, values, q_low, k_low, codebooks, codes, shortlist: int, budget: int,
                   scaling: float, attention_mask=None):
    """Scan summon path of sva_attention (sva/llama.py:219-328) for batch 1.

    Returns dict with per (h, t): 'shortlist' (key ids, selection order, valid
    only), 'final' (valid budget ids in selection order), 'out' [H, Q, D]
    float64, and the stats counts."""

    h_count, q_count, head_dim = query.shape
    g_count, k_len, _ = keys.shape
    group = h_count // g_count
    rank_dim = k_low.shape[-1]
    actual_shortlist = min(shortlist, k_len)
    actual_budget = min(budget, actual_shortlist)
    allowed = allowed_mask(q_count, k_len, attention_mask)
    shortlists, finals = {}, {}
    out = np.zeros((h_count, q_count, head_dim), np.float64)
    summoned = verified = 0
    for h in range(h_count):
        g = h // group
        for t in range(q_count):
            table = lut(q_low[h, t], codebooks[h])
            scores = pq_scores_from_lut(table, codes[h], rank_dim)
            sl = topk(scores, actual_shortlist, allowed=allowed[t])
            rank = rank_scores(k_low[h], sl, q_low[h, t], rank_dim)
            keep = topk(rank, actual_budget, key_index=sl)
            final = sl[keep]
            shortlists[h, t] = sl
            finals[h, t] = final
            out[h, t] = verify(query[h, t], keys[g], values[g], final, scaling)
            summoned += len(sl)
            verified += len(final)
    return {
        "shortlist": shortlists,
        "final": finals,
        "out": out,
        "stats": {"summoned": float(summoned), "exact_scored": float(verified), "verified": float(verified),
                  "queries": float(h_count * q_count)},
    }


def top_unique_candidates(candidate_idx, candidate_scores, candidate_valid, budget: int, refill_factor: int = 2):
    """sva/llama.py:83-116 for one row, with the (score desc, index asc) rule.

    Returns (selected ids, selected scores, selected valid, refill_count);
    the selected arrays have min(budget, refill_count) slots like the
    reference, valid slots first in selection order."""

    idx = _i64(candidate_idx)
    scores = _f32(candidate_scores)
    valid = np.asarray(candidate_valid, bool)
    width = idx.shape[0]
    if width == 0 or budget <= 0:
        return idx[:0], scores[:0], valid[:0], 0
    refill = min(width, max(budget, budget * refill_factor))
    masked = np.where(valid, scores, FMIN).astype(F32)
    # refill entries: top `refill` of all entries (valid or not) by (masked score desc, id asc)
    order = topk(masked, refill, key_index=idx)
    refill_ids = idx[order]
    refill_valid = valid[order]
    refill_scores = masked[order]
    seen = set()
    unique_ids, unique_scores = [], []
    for i in range(refill):
        kid = int(refill_ids[i])
        if kid in seen:
            continue
        seen.add(kid)
        if refill_valid[i]:
            unique_ids.append(kid)
            unique_scores.append(refill_scores[i])
    selected_count = min(budget, refill)
    u_ids = np.asarray(unique_ids, np.int64)
    u_scores = np.asarray(unique_scores, F32)
    pick = topk(u_scores, selected_count, key_index=u_ids) if len(u_ids) else np.zeros(0, np.int64)
    sel_ids = np.zeros(selected_count, np.int64)
    sel_scores = np.full(selected_count, FMIN, F32)
    sel_valid = np.zeros(selected_count, bool)
    sel_ids[: len(pick)] = u_ids[pick]
    sel_scores[: len(pick)] = u_scores[pick]
    sel_valid[: len(pick)] = True
    return sel_ids, sel_scores, sel_valid, refill


def rebuild_postings(codes, codewords: int):
    """sva/llama.py:626-657 as CSR: counts [H, S, C], offsets [H, S, C+1],
    ids [H, S, N] (ascending key id within each cell).  The reference's dense
    layout has width max(1, counts.max())."""

    codes = np.asarray(codes)
    h_count, n, s_count = codes.shape
    counts = np.zeros((h_count, s_count, codewords), np.int64)
    offsets = np.zeros((h_count, s_count, codewords + 1), np.int64)
    ids = np.zeros((h_count, s_count, n), np.int64)
    for h in range(h_count):
        for s in range(s_count):
            labels = codes[h, :, s].astype(np.int64)
            counts[h, s] = np.bincount(labels, minlength=codewords)
            offsets[h, s, 1:] = np.cumsum(counts[h, s])
            ids[h, s] = np.argsort(labels, kind="stable")
    return counts, offsets, ids


def _adaptive_budgets(max_budget: int, k_len: int, adaptive_min, adaptive_mid):
    min_budget = min(adaptive_min or max_budget, max_budget, k_len)
    mid_budget = min(adaptive_mid or max(min_budget, max_budget // 2), max_budget, k_len)
    return min_budget, mid_budget, min(max_budget, k_len)


def cell_choice(q_low_h, codebooks_h, cells: int, rank_dim: int) -> np.ndarray:
    """Top cells per subspace by LUT / sqrt(R) (sva/llama.py:460-463, :366-369)."""

    table = lut(q_low_h, codebooks_h) / F32(sqrt_f32(rank_dim))
    table = table.astype(F32)
    s_count, c_count = table.shape
    cells = min(cells, c_count)
    return np.stack([topk(table[s], cells) for s in range(s_count)])


def static_decode(query, keys, values, q_low, k_low, codebooks, postings, postings_key_len: int, budget: int,
                  cells: int, scaling: float, adaptive_min=None, adaptive_mid=None, low_margin=0.35,
                  high_margin=0.70, allowed=None):
    """_inverted_static_decode_attention (sva/llama.py:427-576), batch 1, q_len 1.

    postings = (counts, offsets, ids) from rebuild_postings over the first
    postings_key_len keys."""

    h_count, _, head_dim = query.shape
    g_count, k_len, _ = keys.shape
    group = h_count // g_count
    rank_dim = k_low.shape[-1]
    counts, offsets, ids = postings
    s_count = counts.shape[1]
    if allowed is None:
        allowed = np.ones(k_len, bool)
    min_budget, mid_budget, max_budget = _adaptive_budgets(min(budget, k_len), k_len, adaptive_min, adaptive_mid)
    cells = min(cells, codebooks.shape[2])
    max_bucket = max(1, int(counts.max()))
    tail_start = min(max(int(postings_key_len), 0), k_len)
    tail = list(range(tail_start, k_len)) if tail_start < k_len else [k_len - 1]
    width = s_count * cells * max_bucket + len(tail)
    results = []
    summoned = refill_pool = verified = 0.0
    out = np.zeros((h_count, head_dim), np.float64)
    for h in range(h_count):
        g = h // group
        top_cells = cell_choice(q_low[h, 0], codebooks[h], cells, rank_dim)
        cand, cand_valid = [], []
        for s in range(s_count):
            for c in top_cells[s]:
                lo, hi = offsets[h, s, c], offsets[h, s, c + 1]
                members = ids[h, s, lo:hi]
                cand.extend(int(m) for m in members)
                cand_valid.extend(bool(allowed[m]) for m in members)
        cand.extend(tail)
        cand_valid.extend(bool(allowed[t]) for t in tail)
        cand = np.asarray(cand, np.int64)
        cand_valid = np.asarray(cand_valid, bool)
        scores = rank_scores(k_low[h], cand, q_low[h, 0], rank_dim) if len(cand) else np.zeros(0, F32)
        # padding slots of the dense layout are invalid entries with id 0
        pad = width - len(cand)
        cand_full = np.concatenate([cand, np.zeros(pad, np.int64)])
        valid_full = np.concatenate([cand_valid, np.zeros(pad, bool)])
        pad_score = rank_scores(k_low[h], np.zeros(1, np.int64), q_low[h, 0], rank_dim) if pad else np.zeros(0, F32)
        scores_full = np.concatenate([scores, np.repeat(pad_score, pad)]).astype(F32)
        sel_ids, sel_scores, sel_valid, refill = top_unique_candidates(cand_full, scores_full, valid_full, max_budget)
        rank_count = len(sel_ids)
        if rank_count > 1:
            margin_ref = min(min_budget, rank_count) - 1
            margin = F32(sel_scores[0]) - F32(sel_scores[margin_ref])
            if margin >= high_margin:
                b = min_budget
            elif margin >= low_margin:
                b = mid_budget
            else:
                b = max_budget
            b = min(b, rank_count)
        else:
            b = 1
        keep = sel_valid & (np.arange(rank_count) < b)
        final = sel_ids[keep]
        out[h] = verify(query[h, 0], keys[g], values[g], final, scaling)
        results.append({"candidates": cand[cand_valid], "final": final, "refill": refill})
        summoned += float(cand_valid.sum())
        refill_pool += float(refill)
        verified += float(keep.sum())
    stats = {"summoned": summoned, "refill_pool": refill_pool, "exact_scored": verified, "verified": verified,
             "queries": float(h_count), "cell_visits": float(h_count * s_count * cells)}
    return {"heads": results, "out": out, "stats": stats}


def inverted_decode(query, keys, values, q_low, k_low, codebooks, codes, budget: int, cells: int, scaling: float,
                    adaptive_min=None, adaptive_mid=None, low_margin=0.35, high_margin=0.70, allowed=None):
    """_inverted_decode_attention (sva/llama.py:330-425), batch 1, q_len 1, with
    postings covering every key (the reference appends each new key)."""

    h_count, _, head_dim = query.shape
    g_count, k_len, _ = keys.shape
    group = h_count // g_count
    rank_dim = k_low.shape[-1]
    s_count = codebooks.shape[1]
    if allowed is None:
        allowed = np.ones(k_len, bool)
    min_budget, mid_budget, max_budget = _adaptive_budgets(min(budget, k_len), k_len, adaptive_min, adaptive_mid)
    cells = min(cells, codebooks.shape[2])
    out = np.zeros((h_count, head_dim), np.float64)
    results = []
    summoned = verified = 0.0
    for h in range(h_count):
        g = h // group
        top_cells = cell_choice(q_low[h, 0], codebooks[h], cells, rank_dim)
        member = np.zeros(k_len, bool)
        for s in range(s_count):
            member |= np.isin(codes[h, :k_len, s], top_cells[s])
        member &= allowed
        if allowed[k_len - 1]:
            member[k_len - 1] = True
        cand = np.nonzero(member)[0].astype(np.int64)
        if len(cand) == 0:
            cand = np.nonzero(allowed)[0][-1:].astype(np.int64)
        scores = rank_scores(k_low[h], cand, q_low[h, 0], rank_dim)
        rank_count = min(max_budget, len(cand))
        order = topk(scores, rank_count, key_index=cand)
        if rank_count > 1:
            margin_ref = min(min_budget, rank_count) - 1
            margin = float(F32(scores[order[0]]) - F32(scores[order[margin_ref]]))
        else:
            margin = float("inf")
        if margin >= high_margin:
            b = min(min_budget, rank_count)
        elif margin >= low_margin:
            b = min(mid_budget, rank_count)
        else:
            b = rank_count
        final = cand[order[:b]]
        out[h] = verify(query[h, 0], keys[g], values[g], final, scaling)
        results.append({"candidates": cand, "final": final})
        summoned += float(len(cand))
        verified += float(b)
    stats = {"summoned": summoned, "exact_scored": verified, "verified": verified, "queries": float(h_count),
             "cell_visits": float(h_count * s_count * cells)}
    return {"heads": results, "out": out, "stats": stats}


def decode(q, q_low, keys, values, k_low, codebooks, codes, shortlist: int, budget: int, scaling: float,
           n_keys: int | None = None):
    """Whole q=1 decode lookup in C (OpenMP over heads): returns
    (shortlist [H, L], final [H, B], out [H, D] float64, threads used).
    keys / values [G, cap, D], k_low [H, cap, R], codes [H, cap, S]: the
    first n_keys (default cap) rows are the cache, so a growing cache held
    in preallocated arrays is read in place."""

    q = _f32(q)
    q_low = _f32(q_low)
    keys = _f32(keys)
    values = _f32(values)
    k_low = _f32(k_low)
    codebooks = _f32(codebooks)
    codes = np.ascontiguousarray(codes)
    h_count, head_dim = q.shape
    g_count, cap, _ = keys.shape
    n = cap if n_keys is None else int(n_keys)
    if not (0 < n <= cap and values.shape == keys.shape and k_low.shape[1] == cap and codes.shape[1] == cap):
        raise ValueError("decode: cache arrays must share their row capacity, and 0 < n_keys <= capacity")
    rank_dim = q_low.shape[1]
    s_count, c_count = codebooks.shape[1], codebooks.shape[2]
    sl = np.full((h_count, shortlist), -1, np.int64)
    fin = np.full((h_count, budget), -1, np.int64)
    out = np.zeros((h_count, head_dim), np.float64)
    threads = lib().sva_oracle_decode(
        h_count, g_count, n, cap, head_dim, rank_dim, s_count, c_count,
        _ptr(q), _ptr(q_low), _ptr(keys), _ptr(values), _ptr(k_low), _ptr(codebooks), _ptr(codes),
        codes.dtype.itemsize, shortlist, budget, float(scaling), _ptr(sl), _ptr(fin), _ptr(out),
    )
    return sl, fin, out, threads


def residual_adapter(hidden, attn, down_w, up_w, scale: float) -> np.ndarray:
    """SVAResidualOutputAdapter.forward after the attention
    (experiments/sva_late4_logit_distill.py:47-51) in float64:
    attn + up(gelu(down([hidden, attn]))) * scale, gelu the erf form.
    hidden / attn [T, H]; down [rank, 2H]; up [H, rank]."""

    x = np.concatenate([np.asarray(hidden, np.float64), np.asarray(attn, np.float64)], axis=-1)
    pre = x @ np.asarray(down_w, np.float64).T
    erf = np.vectorize(math.erf)
    z = 0.5 * pre * (1.0 + erf(pre / math.sqrt(2.0)))
    corr = (z @ np.asarray(up_w, np.float64).T) * scale
    return np.asarray(attn, np.float64) + corr


def kmeans_update(x, labels, centroids, weights=None) -> np.ndarray:
    """One centroid update of the reference's codebook fits
    (experiments/sva_pq_lookup_test.py:92-100; weighted:
    experiments/sva_supervised_coarse_pq_test.py:117-126) in float32, sums in
    ascending row order.  x [N, sub], labels [N], centroids [C, sub], weights [N]."""

    x = _f32(x)
    labels = np.asarray(labels, np.int64)
    cent = _f32(centroids)
    sums = np.zeros_like(cent)
    if weights is None:
        np.add.at(sums, labels, x)
        counts = np.bincount(labels, minlength=cent.shape[0]).astype(F32)
    else:
        w = _f32(weights)
        np.add.at(sums, labels, x * w[:, None])
        counts = np.zeros(cent.shape[0], F32)
        np.add.at(counts, labels, w)
    out = cent.copy()
    nonempty = counts > 0
    out[nonempty] = sums[nonempty] / counts[nonempty][:, None]
    return out


def kmeans_fit(k_low, subspaces: int, iterations: int, initial, weights=None) -> np.ndarray:
    """The reference's fit loop (experiments/sva_pq_lookup_test.py:66-106,
    experiments/sva_supervised_coarse_pq_test.py:88-131) from given initial
    centroids [H, S, C, sub]: assign_to_centroids, then kmeans_update."""

    k_low = _f32(k_low)
    cent = _f32(initial).copy()
    heads, _, rank = k_low.shape
    sub = rank // subspaces
    for h in range(heads):
        w = None if weights is None else np.maximum(_f32(weights)[h], F32(1e-6))
        for s in range(subspaces):
            x = k_low[h, :, s * sub:(s + 1) * sub]
            for _ in range(iterations):
                labels = assign_to_centroids(x, cent[h, s])
                cent[h, s] = kmeans_update(x, labels, cent[h, s], w)
    return cent


def topk_key_weights(top_idx, top_valid, seq_len: int, boost: float) -> np.ndarray:
    """experiments/sva_codebook_refresh_benchmark.py:136-153: weights [H,
    seq_len] fp32 = 1, plus `boost` added (rounded to fp32 each time) once per
    valid top-k hit of the key in that head, indices clamped into
    [0, seq_len).  top_idx / top_valid [H, ...]."""

    top_idx = np.asarray(top_idx, np.int64)
    top_valid = np.asarray(top_valid, bool)
    heads = top_idx.shape[0]
    w = np.ones((heads, seq_len), F32)
    for h in range(heads):
        hits = np.clip(top_idx[h][top_valid[h]], 0, seq_len - 1)
        if hits.size:
            np.add.at(w[h], hits, F32(boost))  # unbuffered: one rounded add per hit, in order
    return w


def topk_targets(scores, query_positions, topk: int):
    """experiments/sva_rotation_diagnostic.py:86-116: per (head, sampled
    query) the top-k keys of the causally masked scores (keys after the
    query's position set to the fp32 minimum), and valid[rank] = rank <=
    position (a query at position p has p + 1 keys).  scores [H, Qs, N];
    returns (idx [H, Qs, k] int64, valid [H, Qs, k] bool), ties by the lower
    key (torch.topk leaves them unspecified)."""

    scores = _f32(scores)
    pos = np.asarray(query_positions, np.int64)
    n = scores.shape[-1]
    allowed = np.arange(n)[None, None, :] <= pos[None, :, None]
    masked = np.where(allowed, scores, FMIN)
    k = min(topk, n)
    keys = np.broadcast_to(np.arange(n), masked.shape)
    order = np.lexsort((keys, -masked.astype(np.float64)), axis=-1)[..., :k]
    valid = np.broadcast_to(np.arange(k)[None, None, :] <= pos[None, :, None], order.shape)
    return order.astype(np.int64), valid.copy()


def query_positions(seq_len: int, samples: int, min_pos: int) -> np.ndarray:
    """The calibration query rows of experiments/export_refreshed_sva_artifact.py:98-104:
    round toward zero of linspace(start, seq_len - 1, min(samples, seq_len))
    in fp32, start = clamp(min_pos, 0, seq_len - 1), then unique."""

    start = max(0, min(min_pos, seq_len - 1))
    steps = min(samples, seq_len)
    if steps == 1:
        pts = np.array([start], np.float64)
    else:
        # torch.linspace on the CPU in fp32: start + i * step for the first
        # half, end - (steps - 1 - i) * step after, each one fused
        # multiply-add (the exact product in fp64, one rounding to fp32)
        step = np.float64(F32((seq_len - 1 - start) / (steps - 1)))
        i = np.arange(steps, dtype=np.float64)
        half = steps // 2
        pts = np.where(i < half, (start + i * step).astype(F32),
                       ((seq_len - 1) - (steps - 1 - i) * step).astype(F32))
    return np.unique(np.trunc(pts).astype(np.int64))


def set_threads(n: int) -> None:
    os.environ["OMP_NUM_THREADS"] = str(n)
