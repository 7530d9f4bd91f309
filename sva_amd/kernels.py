"""Tensor-level wrappers of the C-ABI entry points (one function per stage).

Every function takes device tensors, allocates its outputs with torch's
caching allocator and enqueues the kernel on torch's current stream.  Shapes
follow include/sva_hip.h: query items are [n_seq, H, Q], per-head catalogs are
[H, rows, X] with the last dim contiguous.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._lib import DTYPE_CODES, check, code_type, dtype_code, lib, ptr, require_device, stream_handle


_workspaces: dict[tuple[torch.device, str, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int, kind: str = "summon") -> torch.Tensor:
    """Scratch buffers, one per (device, kind, stream), grown on demand.  The
    kernels carry no state in them between calls, so one buffer serves every
    call made on one stream in turn; calls on another stream get their own,
    so concurrent streams never share one."""

    key = (device, kind, stream_handle(device))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 256), device=device, dtype=torch.uint8)
        _workspaces[key] = ws
    return ws


def _as_query(q: torch.Tensor) -> torch.Tensor:
    if q.dim() == 3:
        q = q.unsqueeze(0)
    if q.dim() != 4:
        raise ValueError(f"query must be [n_seq, H, Q, D] or [H, Q, D], got {tuple(q.shape)}")
    if q.stride(-1) != 1:
        q = q.contiguous()
    return q


def _f32c(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.float32 or not t.is_contiguous():
        t = t.float().contiguous()
    return t


def write_encode(keys: torch.Tensor, k_proj: torch.Tensor, codebooks: torch.Tensor, k_low: torch.Tensor,
                 codes: torch.Tensor | None, row_begin: int = 0, n_rows: int | None = None) -> None:
    """Fill k_low [H, rows, R] and codes [H, rows, S] for cache rows
    [row_begin, row_begin + n_rows) from keys [G, rows, D] (sva/llama.py:597-616,
    sva/ops.py:10-47).  k_low and codes are written in place; codes=None
    projects only."""

    if keys.dim() != 3 or keys.stride(-1) != 1:
        raise ValueError("keys must be [G, rows, D] with contiguous rows")
    heads, dim, rank = k_proj.shape
    subspaces, codewords = codebooks.shape[1], codebooks.shape[2]
    if rank % subspaces != 0:
        raise ValueError(f"rank_dim={rank} must be divisible by subspaces={subspaces}.")
    if k_low.dim() != 3 or k_low.shape[0] != heads or k_low.shape[2] != rank or k_low.stride(1) != rank \
            or k_low.stride(2) != 1 or k_low.dtype != torch.float32:
        raise ValueError("k_low must be fp32 [H, rows, R] with contiguous rows")
    if codes is not None and (codes.dim() != 3 or codes.shape[0] != heads or codes.shape[2] != subspaces
                              or codes.stride(1) != subspaces or codes.stride(2) != 1):
        raise ValueError("codes must be [H, rows, S] with contiguous rows")
    rows = keys.shape[1]
    n_rows = rows - row_begin if n_rows is None else n_rows
    limit = min(rows, k_low.shape[1], codes.shape[1] if codes is not None else rows)
    if row_begin < 0 or n_rows < 0 or row_begin + n_rows > limit:
        raise ValueError("row range outside the catalog")
    device = require_device(keys, k_proj, codebooks, k_low, codes)
    k_proj = _f32c(k_proj)
    codebooks = _f32c(codebooks)
    check(
        lib().sva_write_encode(
            ptr(keys), dtype_code(keys), keys.stride(0), keys.stride(1), row_begin, n_rows, heads, keys.shape[0], dim,
            rank, subspaces, codewords, ptr(k_proj), ptr(codebooks), ptr(k_low), k_low.stride(0), ptr(codes),
            code_type(codes) if codes is not None else 0, codes.stride(0) if codes is not None else 0,
            stream_handle(device),
        ),
        "sva_write_encode",
    )


def write_encode_batch(keys: torch.Tensor, k_proj: torch.Tensor, codebooks: torch.Tensor, k_low: torch.Tensor,
                       codes: torch.Tensor, seq_rows: int, row_begin: int, n_rows: int) -> None:
    """write_encode for every sequence of a batch of caches keys [B, G, rows, D]
    (sva/llama.py:597-616 per sequence): sequence b's catalog rows are
    [b * seq_rows, (b + 1) * seq_rows) of k_low [H, B * seq_rows, R] and codes
    [H, B * seq_rows, S]; cache rows [row_begin, row_begin + n_rows) of each
    sequence are encoded, an append of a few rows in one launch for the batch."""

    if keys.dim() != 4 or keys.stride(-1) != 1:
        raise ValueError("keys must be [B, G, rows, D] with contiguous rows")
    batch, kv_heads, rows, dim = keys.shape
    heads, _, rank = k_proj.shape
    subspaces, codewords = codebooks.shape[1], codebooks.shape[2]
    if k_low.dim() != 3 or k_low.shape[0] != heads or k_low.shape[2] != rank or k_low.stride(1) != rank \
            or k_low.stride(2) != 1 or k_low.dtype != torch.float32 or k_low.shape[1] < batch * seq_rows:
        raise ValueError("k_low must be fp32 [H, B * seq_rows, R] with contiguous rows")
    if codes.dim() != 3 or codes.shape[0] != heads or codes.shape[2] != subspaces or codes.stride(1) != subspaces \
            or codes.stride(2) != 1 or codes.shape[1] < batch * seq_rows:
        raise ValueError("codes must be [H, B * seq_rows, S] with contiguous rows")
    if row_begin < 0 or n_rows < 0 or row_begin + n_rows > min(rows, seq_rows):
        raise ValueError("row range outside the catalog")
    device = require_device(keys, k_proj, codebooks, k_low, codes)
    check(
        lib().sva_write_encode_batch(
            ptr(keys), dtype_code(keys), keys.stride(0), keys.stride(1), keys.stride(2), batch, row_begin, n_rows,
            heads, kv_heads, dim, rank, subspaces, codewords, ptr(_f32c(k_proj)), ptr(_f32c(codebooks)), ptr(k_low),
            k_low.stride(0), seq_rows, ptr(codes), code_type(codes), codes.stride(0), stream_handle(device),
        ),
        "sva_write_encode_batch",
    )


def query_lut(q: torch.Tensor, q_proj: torch.Tensor, scale: torch.Tensor, codebooks: torch.Tensor,
              codes: torch.Tensor | None = None, n_keys: int = 0, shortlist: int = 0):
    """q_low [n_seq,H,Q,R], lut [n_seq,H,Q,S,C], score_range [n_seq,H,Q,4] (sva/llama.py:211, sva/ops.py:66-68).

    With `codes`, the summon threshold estimate is sampled from the cache."""

    q = _as_query(q)
    q_proj, scale, codebooks = _f32c(q_proj), _f32c(scale), _f32c(codebooks)
    device = require_device(q, q_proj, scale, codebooks)
    n_seq, heads, q_len, head_dim = q.shape
    rank = q_proj.shape[-1]
    subspaces, codewords = codebooks.shape[1], codebooks.shape[2]
    if tuple(q_proj.shape) != (heads, head_dim, rank):
        raise ValueError(f"q_proj shape {tuple(q_proj.shape)} != {(heads, head_dim, rank)}")
    q_low = torch.empty(n_seq, heads, q_len, rank, device=device, dtype=torch.float32)
    lut = torch.empty(n_seq, heads, q_len, subspaces, codewords, device=device, dtype=torch.float32)
    rng = torch.empty(n_seq, heads, q_len, 4, device=device, dtype=torch.float32)
    ctype = code_type(codes) if codes is not None else 0
    chs = codes.stride(0) if codes is not None else 0
    check(
        lib().sva_query_lut(
            ptr(q), dtype_code(q), q.stride(0), q.stride(1), q.stride(2), n_seq, heads, q_len, head_dim, rank,
            subspaces, codewords, ptr(q_proj), ptr(scale), ptr(codebooks), ptr(codes), ctype, chs, n_keys,
            max(shortlist, 1), ptr(q_low), ptr(lut), ptr(rng), stream_handle(device),
        ),
        "sva_query_lut",
    )
    return q_low, lut, rng


def _check_catalog(name: str, t: torch.Tensor, heads: int, width: int) -> None:
    if t.dim() != 3 or t.shape[0] != heads or t.shape[2] != width or t.stride(2) != 1 or t.stride(1) != width:
        raise ValueError(f"{name} must be [H={heads}, rows, {width}] with contiguous rows, got {tuple(t.shape)} "
                         f"strides {t.stride()}")


def pq_scores(lut: torch.Tensor, codes: torch.Tensor, n_keys: int, rank: int,
              seq_offsets: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None) -> torch.Tensor:
    """All scan scores [n_seq, H, Q, n_keys] (sva/ops.py:50-71)."""

    n_seq, heads, q_len, subspaces, codewords = lut.shape
    _check_catalog("codes", codes, heads, subspaces)
    device = require_device(lut, codes, seq_offsets, seq_lens)
    scores = torch.empty(n_seq, heads, q_len, n_keys, device=device, dtype=torch.float32)
    check(
        lib().sva_pq_scores(
            ptr(lut), ptr(codes), code_type(codes), codes.stride(0), ptr(seq_offsets), ptr(seq_lens), n_seq, heads,
            q_len, n_keys, rank, subspaces, codewords, ptr(scores), stream_handle(device),
        ),
        "sva_pq_scores",
    )
    return scores


_uniform_masks: dict[tuple, bool] = {}


def mask_is_uniform(lead: torch.Tensor) -> bool:
    """Whether every slice lead[i] equals lead[0] (lead: [n, Q, N]).  The
    answer is kept per mask storage and version (data pointer, version
    counter, shape, strides), so a mask reused across layers and steps costs
    one device comparison, and one host sync, rather than one per call."""

    if lead.shape[0] <= 1:
        return True
    key = (lead.data_ptr(), lead._version, tuple(lead.shape), tuple(lead.stride()), lead.dtype, lead.device)
    hit = _uniform_masks.get(key)
    if hit is None:
        hit = bool(torch.equal(lead[1:], lead[:1].expand_as(lead[1:])))
        if len(_uniform_masks) >= 4096:
            _uniform_masks.clear()
        _uniform_masks[key] = hit
    return hit


def mask_args(mask: torch.Tensor | None, q_len: int, n_keys: int):
    """(tensor, mask type, token stride) for an HF attention mask [..., Q, >=N].

    The kernels take one [Q, N] mask for every head and sequence, so a mask
    whose leading dims (batch, heads) hold more than one slice must repeat
    the same slice; a mask that differs per head or per sequence raises
    ValueError rather than being cut to its first slice."""

    if mask is None:
        return None, 0, 0
    lead = mask.reshape(-1, *mask.shape[-2:])[:, :q_len, :n_keys]
    if not mask_is_uniform(lead):
        raise ValueError(f"attention mask {tuple(mask.shape)} differs across its leading (batch / head) dims; the "
                         f"kernels take one mask for every sequence and head")
    m = lead[0]
    if m.dtype not in _lib.MASK_TYPES:
        m = m.float()
    if m.stride(-1) != 1:
        m = m.contiguous()
    return m, _lib.MASK_TYPES[m.dtype], m.stride(0)


def summon(lut, score_range, q_low, codes, k_low, n_keys: int, shortlist: int, mask: torch.Tensor | None = None,
           seq_offsets: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None):
    """Shortlist (idx, rank score, count) per query item (sva/llama.py:270-292)."""

    n_seq, heads, q_len, subspaces, codewords = lut.shape
    rank = q_low.shape[-1]
    _check_catalog("codes", codes, heads, subspaces)
    _check_catalog("k_low", k_low, heads, rank)
    device = require_device(lut, score_range, q_low, codes, k_low, seq_offsets, seq_lens, mask)
    items = n_seq * heads * q_len
    sl_idx = torch.empty(items, shortlist, device=device, dtype=torch.int32)
    sl_rank = torch.empty(items, shortlist, device=device, dtype=torch.float32)
    sl_count = torch.empty(items, device=device, dtype=torch.int32)
    m, mtype, mstride = mask_args(mask, q_len, n_keys)
    ws_bytes = int(lib().sva_summon_workspace_bytes(n_seq, heads, q_len, n_keys, shortlist))
    ws = workspace(device, ws_bytes)
    check(
        lib().sva_summon(
            ptr(lut), ptr(score_range), ptr(q_low), ptr(codes), code_type(codes), codes.stride(0), ptr(k_low),
            k_low.stride(0), ptr(seq_offsets), ptr(seq_lens), n_seq, heads, q_len, n_keys, rank, subspaces,
            codewords, shortlist, ptr(m), mtype, mstride, ptr(sl_idx), ptr(sl_rank), ptr(sl_count), ptr(ws),
            ws.numel(), stream_handle(device),
        ),
        "sva_summon",
    )
    return sl_idx, sl_rank, sl_count


def budget_select(sl_idx: torch.Tensor, sl_rank: torch.Tensor, sl_count: torch.Tensor, budget: int):
    """Budget lists (ascending key indices) and counts (sva/llama.py:293-302)."""

    items, shortlist = sl_idx.shape
    device = require_device(sl_idx, sl_rank, sl_count)
    fin_idx = torch.empty(items, budget, device=device, dtype=torch.int32)
    fin_count = torch.empty(items, device=device, dtype=torch.int32)
    check(
        lib().sva_budget_select(ptr(sl_idx), ptr(sl_rank), ptr(sl_count), items, shortlist, budget, ptr(fin_idx),
                                ptr(fin_count), stream_handle(device)),
        "sva_budget_select",
    )
    return fin_idx, fin_count


def summon_select(lut, score_range, q_low, codes, k_low, n_keys: int, shortlist: int, budget: int,
                  mask: torch.Tensor | None = None, seq_offsets: torch.Tensor | None = None,
                  seq_lens: torch.Tensor | None = None, keep_shortlist: bool = True):
    """Shortlist and budget in one call (sva/llama.py:262-302):
    (sl_idx, sl_rank, sl_count, fin_idx, fin_count).

    keep_shortlist=False: where the shapes take the fused per-item path
    (sva_summon_strategy 3) the shortlist stays inside the kernel and
    sl_idx / sl_rank come back as None, as the reference's attention keeps
    only the budget; elsewhere they are returned as usual."""

    n_seq, heads, q_len, subspaces, codewords = lut.shape
    rank = q_low.shape[-1]
    _check_catalog("codes", codes, heads, subspaces)
    _check_catalog("k_low", k_low, heads, rank)
    device = require_device(lut, score_range, q_low, codes, k_low, seq_offsets, seq_lens, mask)
    items = n_seq * heads * q_len
    m, mtype, mstride = mask_args(mask, q_len, n_keys)
    if not keep_shortlist:
        keep_shortlist = lib().sva_summon_strategy(n_seq, heads, q_len, n_keys, rank, subspaces, codewords,
                                                   shortlist, code_type(codes), mtype) != 3
    sl_idx = sl_rank = None
    if keep_shortlist:
        sl_idx = torch.empty(items, shortlist, device=device, dtype=torch.int32)
        sl_rank = torch.empty(items, shortlist, device=device, dtype=torch.float32)
    sl_count = torch.empty(items, device=device, dtype=torch.int32)
    fin_idx = torch.empty(items, budget, device=device, dtype=torch.int32)
    fin_count = torch.empty(items, device=device, dtype=torch.int32)
    ws_bytes = int(lib().sva_summon_workspace_bytes(n_seq, heads, q_len, n_keys, shortlist))
    ws = workspace(device, ws_bytes)
    check(
        lib().sva_summon_select(
            ptr(lut), ptr(score_range), ptr(q_low), ptr(codes), code_type(codes), codes.stride(0), ptr(k_low),
            k_low.stride(0), ptr(seq_offsets), ptr(seq_lens), n_seq, heads, q_len, n_keys, rank, subspaces,
            codewords, shortlist, ptr(m), mtype, mstride, ptr(sl_idx), ptr(sl_rank), ptr(sl_count), budget,
            ptr(fin_idx), ptr(fin_count), ptr(ws), ws.numel(), stream_handle(device),
        ),
        "sva_summon_select",
    )
    return sl_idx, sl_rank, sl_count, fin_idx, fin_count


def lookup_select(q, q_proj, scale, codebooks, codes, k_low, n_keys: int, shortlist: int, budget: int,
                  mask: torch.Tensor | None = None):
    """Query side and summon of one decode token in one call (sva/llama.py:211, sva/ops.py:50-71,
    sva/llama.py:276-302): (q_low, lut, score_range, sl_idx, sl_rank, sl_count, fin_idx, fin_count), equal to
    query_lut followed by summon_select.  q: [1, H, 1, D] or [H, 1, D]."""

    q = _as_query(q)
    q_proj, scale, codebooks = _f32c(q_proj), _f32c(scale), _f32c(codebooks)
    n_seq, heads, q_len, head_dim = q.shape
    if n_seq != 1 or q_len != 1:
        raise ValueError("lookup_select takes one token of one sequence")
    rank = q_proj.shape[-1]
    subspaces, codewords = codebooks.shape[1], codebooks.shape[2]
    if tuple(q_proj.shape) != (heads, head_dim, rank):
        raise ValueError(f"q_proj shape {tuple(q_proj.shape)} != {(heads, head_dim, rank)}")
    _check_catalog("codes", codes, heads, subspaces)
    _check_catalog("k_low", k_low, heads, rank)
    device = require_device(q, q_proj, scale, codebooks, codes, k_low, mask)
    f32, i32 = torch.float32, torch.int32
    q_low = torch.empty(1, heads, 1, rank, device=device, dtype=f32)
    lut = torch.empty(1, heads, 1, subspaces, codewords, device=device, dtype=f32)
    rng = torch.empty(1, heads, 1, 4, device=device, dtype=f32)
    sl_idx = torch.empty(heads, shortlist, device=device, dtype=i32)
    sl_rank = torch.empty(heads, shortlist, device=device, dtype=f32)
    sl_count = torch.empty(heads, device=device, dtype=i32)
    fin_idx = torch.empty(heads, budget, device=device, dtype=i32)
    fin_count = torch.empty(heads, device=device, dtype=i32)
    m, mtype, mstride = mask_args(mask, 1, n_keys)
    ws = workspace(device, int(lib().sva_summon_workspace_bytes(1, heads, 1, n_keys, shortlist)))
    check(
        lib().sva_lookup_select(
            ptr(q), dtype_code(q), q.stride(1), heads, head_dim, rank, subspaces, codewords, ptr(q_proj), ptr(scale),
            ptr(codebooks), ptr(codes), code_type(codes), codes.stride(0), ptr(k_low), k_low.stride(0), n_keys,
            shortlist, ptr(m), mtype, mstride, ptr(q_low), ptr(lut), ptr(rng), ptr(sl_idx), ptr(sl_rank),
            ptr(sl_count), budget, ptr(fin_idx), ptr(fin_count), ptr(ws), ws.numel(), stream_handle(device),
        ),
        "sva_lookup_select",
    )
    return q_low, lut, rng, sl_idx, sl_rank, sl_count, fin_idx, fin_count


def verify(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, fin_idx: torch.Tensor,
           fin_count: torch.Tensor, n_keys: int, scaling: float, out_dtype: torch.dtype | None = None,
           seq_offsets: torch.Tensor | None = None, seq_lens: torch.Tensor | None = None) -> torch.Tensor:
    """Verified attention output [n_seq, H, Q, D] (sva/llama.py:304-317)."""

    q = _as_query(q)
    n_seq, heads, q_len, head_dim = q.shape
    if keys.dim() != 3 or keys.stride(-1) != 1 or values.stride() != keys.stride() or keys.shape != values.shape:
        raise ValueError("keys/values must be [G, rows, D] views with identical strides and contiguous rows")
    if keys.dtype != values.dtype:
        raise TypeError("keys and values must share a dtype")
    kv_heads = keys.shape[0]
    budget = fin_idx.shape[1]
    device = require_device(q, keys, values, fin_idx, fin_count, seq_offsets, seq_lens)
    out = torch.empty(n_seq, heads, q_len, head_dim, device=device, dtype=out_dtype or q.dtype)
    ws = workspace(device, int(lib().sva_verify_workspace_bytes(n_seq, heads, kv_heads, q_len, head_dim, budget)),
                   "verify")
    check(
        lib().sva_verify(
            ptr(q), dtype_code(q), q.stride(0), q.stride(1), q.stride(2), ptr(keys), ptr(values), dtype_code(keys),
            keys.stride(0), keys.stride(1), ptr(seq_offsets), ptr(seq_lens), n_keys, ptr(fin_idx), ptr(fin_count),
            n_seq, heads, kv_heads, q_len, head_dim, budget, float(scaling), ptr(out), dtype_code(out), out.stride(0),
            out.stride(1), out.stride(2), ptr(ws), ws.numel(), stream_handle(device),
        ),
        "sva_verify",
    )
    return out


def scan_decode(q, q_proj, scale, codebooks, codes, k_low, keys, values, n_keys: int, shortlist: int, budget: int,
                scaling: float, mask=None, seq_offsets=None, seq_lens=None, out_dtype=None):
    """The whole scan-mode lookup for one layer call: LUT -> summon -> budget -> verify.

    shortlist/budget are the reference's actual_shortlist / actual_budget.
    Returns (out, sl_count, fin_count)."""

    q = _as_query(q)
    q_low, lut, rng = query_lut(q, q_proj, scale, codebooks, codes, n_keys, shortlist)
    _, _, sl_count, fin_idx, fin_count = summon_select(lut, rng, q_low, codes, k_low, n_keys, shortlist, budget, mask,
                                                       seq_offsets, seq_lens)
    out = verify(q, keys, values, fin_idx, fin_count, n_keys, scaling, out_dtype, seq_offsets, seq_lens)
    return out, sl_count, fin_count


def sqrt_rank(rank: int) -> float:
    return math.sqrt(rank)


class ScanDecodePlan:
    """Preallocated scan-mode decode lookup for a fixed query shape.

    Holds every intermediate buffer (q_low, LUT, shortlist, budget lists) so a
    decode step issues its three calls (query_lut, summon with the budget
    select, verify) with no allocation and one ctypes call each."""

    def __init__(self, device, n_seq: int, heads: int, q_len: int, head_dim: int, rank: int, subspaces: int,
                 codewords: int, shortlist: int, budget: int):
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.shape = (n_seq, heads, q_len, head_dim, rank, subspaces, codewords, shortlist, budget)
        items = n_seq * heads * q_len
        f32, i32 = torch.float32, torch.int32
        self.q_low = torch.empty(n_seq, heads, q_len, rank, device=self.device, dtype=f32)
        self.lut = torch.empty(n_seq, heads, q_len, subspaces, codewords, device=self.device, dtype=f32)
        self.rng = torch.empty(n_seq, heads, q_len, 4, device=self.device, dtype=f32)
        self.sl_idx = torch.empty(items, shortlist, device=self.device, dtype=i32)
        self.sl_rank = torch.empty(items, shortlist, device=self.device, dtype=f32)
        # shortlist and budget sizes, and 1 where the sampled floor overshot (one-call step only)
        self.counts = torch.zeros(3, items, device=self.device, dtype=i32)
        self.sl_count = self.counts[0]
        self.overshoot = self.counts[2]
        self.fin_idx = torch.empty(items, budget, device=self.device, dtype=i32)
        self.fin_count = self.counts[1]
        self._lib = lib()
        # the plan's own buffers, as the one-call step passes them
        self._bufs = (self.q_low.data_ptr(), self.lut.data_ptr(), self.rng.data_ptr(), self.sl_idx.data_ptr(),
                      self.sl_rank.data_ptr(), self.sl_count.data_ptr(), self.fin_idx.data_ptr(),
                      self.fin_count.data_ptr(), self.overshoot.data_ptr())
        # per stream: (summon workspace, keys it is sized for) and (verify workspace, KV heads), so that one
        # plan driven from two streams never shares a scratch buffer between them
        self._ws: dict[int, tuple[torch.Tensor, int]] = {}
        self._vws: dict[int, tuple[torch.Tensor, int]] = {}
        self._checked_weights = set()  # (data_ptr, version, dtype, shape, strides) of weights that passed

    def _check_weights(self, q_proj, scale, codebooks) -> None:
        """fp32, contiguous, on the plan's device and of the plan's shape; the
        result is kept per weight storage (one entry per layer that shares the
        plan), so a decode loop pays it once per layer."""
        key = tuple((t.data_ptr(), t._version, t.dtype, t.shape, t.stride()) for t in (q_proj, scale, codebooks))
        if key in self._checked_weights:
            return
        _, heads, _, head_dim, rank, subspaces, codewords, _, _ = self.shape
        want = {"q_proj": (q_proj, (heads, head_dim, rank)), "scale": (scale, (heads,)),
                "codebooks": (codebooks, (heads, subspaces, codewords, rank // subspaces))}
        for name, (t, shape) in want.items():
            if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shape or t.device != self.device:
                raise ValueError(f"ScanDecodePlan: {name} must be contiguous fp32 {shape} on {self.device}, got "
                                 f"{t.dtype} {tuple(t.shape)} strides {t.stride()} on {t.device}")
        if len(self._checked_weights) >= 1024:
            self._checked_weights.clear()
        self._checked_weights.add(key)

    def _check_catalog(self, codes, k_low, n_keys: int) -> None:
        _, heads, _, _, rank, subspaces, _, _, _ = self.shape
        _check_catalog("codes", codes, heads, subspaces)
        _check_catalog("k_low", k_low, heads, rank)
        if k_low.dtype != torch.float32:
            raise ValueError(f"ScanDecodePlan: k_low must be fp32, got {k_low.dtype}")
        if codes.dtype not in (torch.uint8, torch.int16, torch.int32, torch.int64):
            raise ValueError(f"ScanDecodePlan: codes must be an integer tensor, got {codes.dtype}")
        if codes.shape[1] < n_keys or k_low.shape[1] < n_keys or codes.device != self.device or \
                k_low.device != self.device:
            raise ValueError(f"ScanDecodePlan: a catalog of {codes.shape[1]} / {k_low.shape[1]} rows on "
                             f"{codes.device} / {k_low.device} for {n_keys} keys on {self.device}")

    def _check_query(self, q) -> None:
        n_seq, heads, q_len, head_dim = self.shape[:4]
        if tuple(q.shape) != (n_seq, heads, q_len, head_dim) or q.device != self.device:
            raise ValueError(f"ScanDecodePlan: query {tuple(q.shape)} on {q.device}, planned "
                             f"{(n_seq, heads, q_len, head_dim)} on {self.device}")

    def run(self, q, q_proj, scale, codebooks, codes, k_low, keys, values, n_keys: int, scaling: float, out=None,
            mask=None):
        """The whole lookup; returns the verified output.  One token of one
        sequence is one C-ABI call (sva_lookup_verify: on the wide path the
        verifier runs inside the finish kernel); otherwise summon() then
        verify()."""
        n_seq, heads, q_len, head_dim, rank, subspaces, codewords, shortlist, budget = self.shape
        if n_seq != 1 or q_len != 1:
            self.summon(q, q_proj, scale, codebooks, codes, k_low, n_keys, mask=mask)
            return self.verify(q, keys, values, n_keys, scaling, out=out)
        q = _as_query(q)
        self._check_query(q)
        self._check_weights(q_proj, scale, codebooks)
        self._check_catalog(codes, k_low, n_keys)
        self._check_kv(keys, values, n_keys)
        L = self._lib
        stream = stream_handle(self.device)
        m, mtype, mstride = mask_args(mask, q_len, n_keys)
        ws = self._summon_ws(n_keys, stream)
        vws = self._verify_ws(keys, stream)
        if out is None:
            out = torch.empty(n_seq, heads, q_len, head_dim, device=self.device, dtype=q.dtype)
        if out.stride(-1) != 1 or tuple(out.shape) != (1, heads, 1, head_dim):
            raise ValueError(f"ScanDecodePlan: out must be [1, {heads}, 1, {head_dim}] with contiguous rows")
        b_qlow, b_lut, b_rng, b_slidx, b_slrank, b_slcount, b_finidx, b_fincount, b_over = self._bufs
        check(L.sva_lookup_verify(q.data_ptr(), dtype_code(q), q.stride(1), heads, head_dim, rank, subspaces, codewords,
                                  q_proj.data_ptr(), scale.data_ptr(), codebooks.data_ptr(), codes.data_ptr(),
                                  code_type(codes), codes.stride(0), k_low.data_ptr(), k_low.stride(0), n_keys,
                                  shortlist, ptr(m), mtype, mstride, b_qlow, b_lut, b_rng, b_slidx, b_slrank,
                                  b_slcount, budget, b_finidx, b_fincount, ws.data_ptr(), ws.numel(),
                                  keys.data_ptr(), values.data_ptr(), dtype_code(keys), keys.stride(0),
                                  keys.stride(1), keys.shape[0], float(scaling), out.data_ptr(), dtype_code(out),
                                  out.stride(1), vws.data_ptr(), vws.numel(), b_over, stream),
              "sva_lookup_verify")
        return out

    def _summon_ws(self, n_keys: int, stream: int | None = None) -> torch.Tensor:
        n_seq, heads, q_len, _, _, _, _, shortlist, _ = self.shape
        stream = stream_handle(self.device) if stream is None else stream
        ws, cap = self._ws.get(stream, (None, -1))
        if n_keys > cap:
            # the summon workspace grows with the key count: sized for the next
            # multiple of 64K keys, so a decode loop re-queries it rarely
            cap = (n_keys + 65535) // 65536 * 65536
            ws = workspace(self.device, int(self._lib.sva_summon_workspace_bytes(
                n_seq, heads, q_len, cap, shortlist)), "plan")
            self._ws[stream] = (ws, cap)
        return ws

    def _verify_ws(self, keys, stream: int | None = None, kv_heads: int | None = None) -> torch.Tensor:
        n_seq, heads, q_len, head_dim, _, _, _, _, budget = self.shape
        stream = stream_handle(self.device) if stream is None else stream
        kv_heads = keys.shape[0] if kv_heads is None else kv_heads
        vws, kv = self._vws.get(stream, (None, -1))
        if vws is None or kv != kv_heads:
            vws = workspace(self.device, int(self._lib.sva_verify_workspace_bytes(
                n_seq, heads, kv_heads, q_len, head_dim, budget)), "verify")
            self._vws[stream] = (vws, kv_heads)
        return vws

    def _check_kv(self, keys, values, n_keys: int) -> None:
        _, heads, _, head_dim = self.shape[:4]
        if keys.dim() != 3 or keys.shape[1] < n_keys or keys.shape[2] != head_dim or keys.stride(-1) != 1 or \
                heads % keys.shape[0] != 0 or keys.device != self.device:
            raise ValueError(f"ScanDecodePlan: keys must be [G, >={n_keys}, {head_dim}] with contiguous rows on "
                             f"{self.device}, got {tuple(keys.shape)} strides {keys.stride()} on {keys.device}")
        if values.shape != keys.shape or values.stride() != keys.stride() or values.dtype != keys.dtype or \
                values.device != keys.device:
            raise ValueError(f"ScanDecodePlan: values {tuple(values.shape)} {values.dtype} strides {values.stride()} "
                             f"must match keys {tuple(keys.shape)} {keys.dtype} strides {keys.stride()}")

    def summon(self, q, q_proj, scale, codebooks, codes, k_low, n_keys: int, mask=None) -> None:
        """Query side, shortlist and budget into the plan's buffers (one C-ABI call for one token of one
        sequence, sva_lookup_select; otherwise sva_query_lut and sva_summon_select)."""
        n_seq, heads, q_len, head_dim, rank, subspaces, codewords, shortlist, budget = self.shape
        q = _as_query(q)
        self._check_query(q)
        self._check_weights(q_proj, scale, codebooks)
        self._check_catalog(codes, k_low, n_keys)
        L = self._lib
        stream = stream_handle(self.device)
        m, mtype, mstride = mask_args(mask, q_len, n_keys)
        ws = self._summon_ws(n_keys)
        if n_seq == 1 and q_len == 1:
            # one token: query side and summon in one call (fused where the shapes allow)
            check(L.sva_lookup_select(q.data_ptr(), dtype_code(q), q.stride(1), heads, head_dim, rank, subspaces,
                                      codewords, q_proj.data_ptr(), scale.data_ptr(), codebooks.data_ptr(),
                                      codes.data_ptr(), code_type(codes), codes.stride(0), k_low.data_ptr(),
                                      k_low.stride(0), n_keys, shortlist, ptr(m), mtype, mstride,
                                      self.q_low.data_ptr(), self.lut.data_ptr(), self.rng.data_ptr(),
                                      self.sl_idx.data_ptr(), self.sl_rank.data_ptr(), self.sl_count.data_ptr(),
                                      budget, self.fin_idx.data_ptr(), self.fin_count.data_ptr(), ws.data_ptr(),
                                      ws.numel(), stream), "sva_lookup_select")
        else:
            check(L.sva_query_lut(q.data_ptr(), dtype_code(q), q.stride(0), q.stride(1), q.stride(2), n_seq, heads,
                                  q_len, head_dim, rank, subspaces, codewords, q_proj.data_ptr(), scale.data_ptr(),
                                  codebooks.data_ptr(), codes.data_ptr(), code_type(codes), codes.stride(0), n_keys,
                                  shortlist, self.q_low.data_ptr(), self.lut.data_ptr(), self.rng.data_ptr(), stream),
                  "sva_query_lut")
            check(L.sva_summon_select(self.lut.data_ptr(), self.rng.data_ptr(), self.q_low.data_ptr(),
                                      codes.data_ptr(), code_type(codes), codes.stride(0), k_low.data_ptr(),
                                      k_low.stride(0), None, None, n_seq, heads, q_len, n_keys, rank, subspaces,
                                      codewords, shortlist, ptr(m), mtype, mstride, self.sl_idx.data_ptr(),
                                      self.sl_rank.data_ptr(), self.sl_count.data_ptr(), budget,
                                      self.fin_idx.data_ptr(), self.fin_count.data_ptr(), ws.data_ptr(), ws.numel(),
                                      stream), "sva_summon_select")

    def verify(self, q, keys, values, n_keys: int, scaling: float, out=None):
        """Exact verifier over the budget lists of the last summon()."""
        n_seq, heads, q_len, head_dim, rank, subspaces, codewords, shortlist, budget = self.shape
        q = _as_query(q)
        self._check_query(q)
        self._check_kv(keys, values, n_keys)
        L = self._lib
        stream = stream_handle(self.device)
        if out is None:
            out = torch.empty(n_seq, heads, q_len, head_dim, device=self.device, dtype=q.dtype)
        vws = self._verify_ws(keys)
        check(L.sva_verify(q.data_ptr(), dtype_code(q), q.stride(0), q.stride(1), q.stride(2), keys.data_ptr(),
                           values.data_ptr(), dtype_code(keys), keys.stride(0), keys.stride(1), None, None, n_keys,
                           self.fin_idx.data_ptr(), self.fin_count.data_ptr(), n_seq, heads, keys.shape[0], q_len,
                           head_dim, budget, float(scaling), out.data_ptr(), dtype_code(out), out.stride(0),
                           out.stride(1), out.stride(2), vws.data_ptr(), vws.numel(), stream), "sva_verify")
        return out


class DecodeLayer:
    """The native decode step of one patched layer (sva_decode_layer_*):
    catalog append, lookup with verifier and statistics in one C-ABI call per
    token (sva/llama.py:597-616, :211-317, :319-326).  Uses a ScanDecodePlan's
    buffers (one token of one sequence); `stats` is the int64 [4] device
    counter the steps add to (summoned, verified, floor overshoots, queries)."""

    STAT_ROWS = (("summoned",), ("exact_scored", "verified"), ("floor_overshoots",), ("queries",))

    def __init__(self, plan: ScanDecodePlan, q_proj: torch.Tensor, scale: torch.Tensor, codebooks: torch.Tensor,
                 k_proj: torch.Tensor, scaling: float):
        n_seq, heads, q_len, head_dim, rank, subspaces, codewords, shortlist, budget = plan.shape
        if n_seq != 1 or q_len != 1:
            raise ValueError("DecodeLayer runs one token of one sequence")
        plan._check_weights(q_proj, scale, codebooks)
        if k_proj.dtype != torch.float32 or not k_proj.is_contiguous() or tuple(k_proj.shape) != (heads, head_dim,
                                                                                                    rank):
            raise ValueError(f"DecodeLayer: k_proj must be contiguous fp32 {(heads, head_dim, rank)}")
        self.plan = plan
        self.device = plan.device
        self._weights = (q_proj, scale, codebooks, k_proj)  # kept alive: the handle points at them
        self.stats = torch.zeros(4, device=self.device, dtype=torch.int64)
        self._lib = plan._lib
        self._handle = None  # created at the first step, when the KV head count is known
        self._scaling = float(scaling)
        self._kv_heads = -1
        self._bound: tuple | None = None
        self._out: torch.Tensor | None = None  # the output buffer a step writes when none is given

    def _create(self, kv_heads: int) -> None:
        _, heads, _, head_dim, rank, subspaces, codewords, shortlist, budget = self.plan.shape
        q_proj, scale, codebooks, k_proj = self._weights
        handle = ctypes.c_void_p()
        check(self._lib.sva_decode_layer_create(heads, kv_heads, head_dim, rank, subspaces, codewords, shortlist,
                                                budget, q_proj.data_ptr(), scale.data_ptr(), codebooks.data_ptr(),
                                                k_proj.data_ptr(), self._scaling, ctypes.byref(handle)),
              "sva_decode_layer_create")
        self.close()
        self._handle = handle.value
        self._kv_heads = kv_heads
        self._bound = None

    def close(self) -> None:
        if self._handle is not None:
            self._lib.sva_decode_layer_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001  (interpreter shutdown)
            pass

    def step(self, q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, k_low: torch.Tensor,
             codes: torch.Tensor, row_begin: int, n_keys: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """Encode cache rows [row_begin, n_keys) into the catalog (k_low,
        codes), look up and verify q [1, H, 1, D] against the first n_keys
        rows of keys / values ([G, rows, D], or the cache [1, G, rows, D]),
        and return the output [1, H, 1, D] in q's dtype (written to `out`
        when given, else to the layer's own buffer, which the next step
        overwrites)."""
        plan = self.plan
        heads, head_dim = plan.shape[1], plan.shape[3]
        if q.shape != (1, heads, 1, head_dim) or q.stride(-1) != 1:
            raise ValueError(f"DecodeLayer: q must be [1, {heads}, 1, {head_dim}] with contiguous rows")
        if keys.dim() == 4:
            if keys.shape[0] != 1:
                raise ValueError("DecodeLayer: the cache must hold one sequence")
        elif keys.dim() != 3:
            raise ValueError("DecodeLayer: keys / values must be [G, rows, D] or [1, G, rows, D]")
        if keys.shape[-2] < n_keys or keys.shape[-1] != head_dim or keys.stride(-1) != 1 or \
                values.stride() != keys.stride() or values.shape != keys.shape or values.dtype != keys.dtype:
            raise ValueError("DecodeLayer: keys / values must be equal caches with contiguous rows")
        kv_heads = keys.shape[-3]
        if kv_heads != self._kv_heads:
            if heads % kv_heads != 0:
                raise ValueError(f"DecodeLayer: {heads} query heads over {kv_heads} KV heads")
            self._create(kv_heads)
        if out is None:
            out = self._out
            if out is None or out.dtype != q.dtype:
                out = self._out = torch.empty(1, heads, 1, head_dim, device=self.device, dtype=q.dtype)
        elif out.shape != q.shape or out.stride(-1) != 1:
            raise ValueError(f"DecodeLayer: out must be [1, {heads}, 1, {head_dim}] with contiguous rows")
        stream = stream_handle(self.device)
        ws = plan._summon_ws(n_keys, stream)
        vws = plan._verify_ws(None, stream, kv_heads)
        b = self._bound
        if b is None or b[0] is not k_low or b[1] is not codes or b[2] is not ws or b[3] is not vws:
            plan._check_catalog(codes, k_low, n_keys)
            if k_low.device != self.device or codes.device != self.device or keys.device != self.device:
                raise ValueError("DecodeLayer: catalog and cache must be on the plan's device")
            check(self._lib.sva_decode_layer_bind(
                self._handle, k_low.data_ptr(), k_low.stride(0), codes.data_ptr(), code_type(codes),
                codes.stride(0), min(codes.shape[1], k_low.shape[1]), plan.q_low.data_ptr(), plan.lut.data_ptr(),
                plan.rng.data_ptr(), plan.sl_idx.data_ptr(), plan.sl_rank.data_ptr(), plan.counts.data_ptr(),
                plan.fin_idx.data_ptr(), ws.data_ptr(), ws.numel(), vws.data_ptr(), vws.numel(),
                self.stats.data_ptr()), "sva_decode_layer_bind")
            self._bound = (k_low, codes, ws, vws)
        check(self._lib.sva_decode_layer_step(self._handle, q.data_ptr(), dtype_code(q), q.stride(1), keys.data_ptr(),
                                              values.data_ptr(), dtype_code(keys), keys.stride(-3), keys.stride(-2),
                                              row_begin, n_keys, out.data_ptr(), dtype_code(out), out.stride(1),
                                              stream), "sva_decode_layer_step")
        return out


    def step_next(self, q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, kst: tuple, k_low: torch.Tensor,
                  codes: torch.Tensor, row_begin: int, n_keys: int) -> torch.Tensor | None:
        """step() for the next token of a caller that compared q [1, H, 1, D]
        and the cache [1, G, rows, D] (strides `kst`, contiguous rows, K and V
        alike, one dtype, this device) with the ones a step() call accepted:
        those checks are not repeated.  None when the layer must bind its
        buffers again or its output buffer does not fit (take step())."""
        plan = self.plan
        stream = stream_handle(self.device)
        ws = plan._summon_ws(n_keys, stream)
        vws, kv = plan._vws.get(stream, (None, -1))
        b = self._bound
        out = self._out
        if (b is None or b[0] is not k_low or b[1] is not codes or b[2] is not ws or b[3] is not vws
                or kv != self._kv_heads or keys.shape[1] != self._kv_heads or out is None or out.dtype is not q.dtype):
            return None
        codes_ = DTYPE_CODES
        check(self._lib.sva_decode_layer_step(self._handle, q.data_ptr(), codes_[q.dtype], q.stride(1), keys.data_ptr(),
                                              values.data_ptr(), codes_[keys.dtype], kst[1], kst[2], row_begin,
                                              n_keys, out.data_ptr(), codes_[out.dtype], out.stride(1), stream),
              "sva_decode_layer_step")
        return out


def residual_adapter(hidden_states: torch.Tensor, attn_output: torch.Tensor, down_w: torch.Tensor,
                     up_w: torch.Tensor, scale: float) -> torch.Tensor:
    """attn_output + (up(gelu(down([hidden_states, attn_output]))) * scale).to(attn dtype)
    for every token (experiments/sva_late4_logit_distill.py:47-51), one launch."""

    if hidden_states.shape != attn_output.shape:
        raise ValueError("hidden_states and attn_output must have the same shape")
    hidden = int(attn_output.shape[-1])
    rank = int(down_w.shape[0])
    if tuple(down_w.shape) != (rank, 2 * hidden) or tuple(up_w.shape) != (hidden, rank):
        raise ValueError(f"adapter weights down {tuple(down_w.shape)} / up {tuple(up_w.shape)} do not match "
                         f"hidden size {hidden}")
    h = hidden_states.reshape(-1, hidden)
    a = attn_output.reshape(-1, hidden)
    if h.stride(-1) != 1:
        h = h.contiguous()
    if a.stride(-1) != 1:
        a = a.contiguous()
    device = require_device(h, a, down_w, up_w)
    down_w, up_w = _f32c(down_w), _f32c(up_w)
    out = torch.empty_like(a)
    check(lib().sva_residual_adapter(ptr(h), dtype_code(h), h.stride(0), ptr(a), dtype_code(a), a.stride(0),
                                     ptr(down_w), ptr(up_w), float(scale), h.shape[0], hidden, rank, ptr(out),
                                     dtype_code(out), out.stride(0), stream_handle(device)), "sva_residual_adapter")
    return out.reshape(attn_output.shape)


def stream_read(buf: torch.Tensor, sink: torch.Tensor | None = None) -> torch.Tensor:
    """A plain streaming read of `buf` (contiguous, 16-byte aligned, a
    multiple of 16 bytes) by sva_stream_read: the time a read of the same
    bytes takes on its own.  Returns the uint32 sink whose XOR is the XOR of
    every 32-bit word of `buf` (pass `sink` to reuse one)."""
    if not buf.is_contiguous():
        raise ValueError("stream_read: the buffer must be contiguous")
    device = require_device(buf)
    nbytes = buf.numel() * buf.element_size()
    words = int(lib().sva_stream_read_sink_words(nbytes))
    if sink is None:
        sink = torch.empty(max(words, 1), device=device, dtype=torch.int32)
    elif sink.dtype != torch.int32 or sink.numel() < words or sink.device != device:
        raise ValueError(f"stream_read: the sink must hold {words} int32 words on {device}")
    check(lib().sva_stream_read(ptr(buf), nbytes, ptr(sink), sink.numel(), stream_handle(device)), "sva_stream_read")
    return sink
