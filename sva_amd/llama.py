"""Llama-family drop-in attention with the SVA summon -> verify lookup on
MI355X (sva/llama.py).

The public surface mirrors the reference: ``patch_llama_attention`` with the
same keyword arguments, ``SVALlamaPatcher`` (patch / unpatch / reset_stats /
reset_catalogs / context manager / stats / bundle / serving) and
``SVALlamaAttention`` (forward returns ``(o_proj(out), None)``).  Every
lookup stage runs in the HIP library (sva_amd/csrc); torch supplies the
model's own projections, RoPE, the KV cache and device memory.  There is no
CPU path: patched layers raise on tensors that are not on a ROCm device.

Per layer the module keeps its key catalog on the GPU: low-rank keys
``k_low [H, capacity, R]`` fp32 and PQ codes ``[H, capacity, S]`` (uint8 for
up to 256 codewords), grown geometrically and appended row by row as the KV
cache grows (sva/llama.py:578-624).  The KV cache itself is read in place,
per KV head (GQA is resolved inside the kernels; nothing is expanded with
repeat_kv).
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import torch
from torch import nn
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from . import inverted, kernels
from .artifacts import SVAArtifactBundle, SVALayerArtifacts, load_sva_artifact_bundle
from .stats import SVAStats

SUMMON_MODES = ("scan", "inverted", "inverted_static")


@dataclass(frozen=True)
class SVALlamaServingConfig:
    """Serving settings of a patched attention module (sva/llama.py:22-38)."""

    rank_dim: int
    coarse_shortlist: int
    budget: int
    assign_chunk_size: int = 8192
    query_chunk_size: int | None = None
    summon_mode: str = "scan"
    inverted_cells_per_subspace: int = 8
    adaptive_min_budget: int | None = None
    adaptive_mid_budget: int | None = None
    adaptive_low_margin: float = 0.35
    adaptive_high_margin: float = 0.70
    profile_components: bool = False
    static_tail_rebuild_interval: int = 64


def _code_dtype(codewords: int) -> torch.dtype:
    if codewords <= 256:
        return torch.uint8
    if codewords <= 32768:
        return torch.int16
    return torch.int32


class SVALlamaAttention(nn.Module):
    """Replacement for one Llama attention layer (sva/llama.py:41-169)."""

    def __init__(self, original: nn.Module, layer_artifacts: SVALayerArtifacts, serving: SVALlamaServingConfig,
                 stats: SVAStats | None = None) -> None:
        super().__init__()
        if serving.summon_mode not in SUMMON_MODES:
            raise ValueError(f"Unknown SVA summon_mode: {serving.summon_mode!r}")
        self.original = original
        self.config = original.config
        self.layer_idx = original.layer_idx
        self.head_dim = original.head_dim
        self.num_key_value_groups = original.num_key_value_groups
        self.scaling = original.scaling
        self.attention_dropout = original.attention_dropout
        self.q_proj = original.q_proj
        self.k_proj = original.k_proj
        self.v_proj = original.v_proj
        self.o_proj = original.o_proj
        self.serving = serving
        self.stats = stats
        a = layer_artifacts
        self.register_buffer("sva_q_proj", a.q_proj.detach().float().clone(), persistent=False)
        self.register_buffer("sva_k_proj", a.k_proj.detach().float().clone(), persistent=False)
        self.register_buffer("sva_logit_scale", a.logit_scale.detach().float().clone(), persistent=False)
        self.register_buffer("sva_scale", a.logit_scale.detach().float().exp().clamp(0.01, 100.0).clone(),
                             persistent=False)
        self.register_buffer("sva_coarse_codebooks", a.coarse_codebooks.detach().float().clone(), persistent=False)
        # the artifact's sizes (fixed for the module's life)
        self._heads, _, self._rank = (int(x) for x in a.q_proj.shape)
        self._subspaces, self._codewords = int(a.coarse_codebooks.shape[1]), int(a.coarse_codebooks.shape[2])
        self.reset_catalog()

    # ------------------------------------------------------------------
    @staticmethod
    def _top_unique_candidates(candidate_idx: torch.Tensor, candidate_scores: torch.Tensor,
                               candidate_valid: torch.Tensor, budget: int, refill_factor: int = 2):
        """Refill window, first occurrence per key, best `budget` of those
        (sva/llama.py:83-116), on the GPU; ties by (score desc, key asc)."""

        return inverted.top_unique_candidates(candidate_idx, candidate_scores, candidate_valid, budget, refill_factor)

    @staticmethod
    def _profile_now(device: torch.device) -> float:
        if device.type == "cuda":
            torch.cuda.synchronize(device)
        return time.perf_counter()

    @staticmethod
    def _profile_elapsed_ms(device: torch.device, start: float) -> float:
        if device.type == "cuda":
            torch.cuda.synchronize(device)
        return (time.perf_counter() - start) * 1000.0

    def reset_catalog(self) -> None:
        self._k_low: torch.Tensor | None = None      # [H, capacity, R] fp32
        self._codes: torch.Tensor | None = None      # [H, capacity, S]
        self._key_len = 0                            # rows with k_low (and, unless lazy, codes)
        self._codes_len = 0                          # rows with codes
        self._signature: tuple | None = None
        self._postings: inverted.Postings | None = None
        self._decode_plan: kernels.ScanDecodePlan | None = None  # q = 1 buffers, kept across steps
        self._decode_layer: kernels.DecodeLayer | None = None    # the native decode step over those buffers
        self._fast: tuple | None = None  # what the last native step checked, for the next token's lean path

    # ------------------------------------------------------------------
    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple[torch.Tensor, torch.Tensor] | None = None,
                attention_mask: torch.Tensor | None = None, past_key_values: Any = None,
                **kwargs: Any) -> tuple[torch.Tensor, None]:
        if self.training:
            raise RuntimeError("SVA Llama adapter is inference-only. Call model.eval() before running it.")
        if kwargs.get("output_attentions"):
            raise RuntimeError("SVA Llama adapter does not materialize dense attention weights.")
        if position_embeddings is None:
            raise ValueError("SVA Llama adapter requires model-provided RoPE position embeddings.")
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        if past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx)
        out = self.sva_attention(q, k, v, attention_mask)
        out = out.transpose(1, 2).contiguous().reshape(*input_shape, -1)
        return self.o_proj(out), None

    # ------------------------------------------------------------------
    def sva_attention(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                      attention_mask: torch.Tensor | None) -> torch.Tensor:
        """query [1, H, Q, D]; key/value [1, G, N, D] (not expanded)."""

        # one scan-mode decode token of one sequence with no mask (the token
        # sees every key): the native step, behind checks kept lean because
        # they run for every layer and token
        if attention_mask is None and self._fast is not None:
            out = self._decode_next(query, key, value)
            if out is not None:
                return out
        if attention_mask is None and query.shape[2] == 1 and query.shape[0] == 1 and \
                self.serving.summon_mode == "scan" and query.is_cuda and key.is_cuda and value.is_cuda and \
                key.stride(-1) == 1 and value.stride() == key.stride() and value.shape == key.shape:
            return self._native_decode(query, key, value)
        batch, n_heads, q_len, head_dim = query.shape
        k_len = key.shape[2]
        kernels.require_device(query, key, value)
        mode = self.serving.summon_mode
        if batch != 1:
            if mode != "scan":
                raise ValueError("SVA Llama adapter runs batches larger than 1 in summon_mode='scan' only.")
            return self._scan_attention_batched(query, key, value, attention_mask)
        static_decode = mode == "inverted_static" and q_len == 1
        profile = self.serving.profile_components and static_decode
        outer = {}
        t0 = self._profile_now(query.device) if profile else 0.0
        keys = key[0]
        values = value[0]
        if keys.stride(-1) != 1:
            keys = keys.contiguous()
        if values.stride() != keys.stride():
            values = values.contiguous()
            keys = keys.contiguous()
        mask = None if attention_mask is None else attention_mask[..., :q_len, :k_len]
        if profile:
            t1 = self._profile_now(query.device)
        k_low, codes = self._key_catalog(keys, q_len)
        if profile:
            outer["static_key_catalog_ms"] = self._profile_elapsed_ms(query.device, t1)
        shortlist = min(self.serving.coarse_shortlist, k_len)
        budget = min(self.serving.budget, shortlist)
        if static_decode:
            out = inverted.static_decode(self, query, keys, values, k_low, codes, k_len, mask, budget)
            if profile and self.stats is not None:
                outer["static_outer_total_ms"] = self._profile_elapsed_ms(query.device, t0)
                self.stats.add(int(self.layer_idx or 0), {"profile_outer_calls": 1.0, **outer})
            return out
        if mode == "inverted" and q_len == 1:
            return inverted.adaptive_decode(self, query, keys, values, k_low, codes, k_len, mask, budget)
        return self._scan_attention(query, keys, values, k_low, codes, k_len, mask, shortlist, budget)

    def _native_decode(self, query, key, value):
        """One scan-mode decode token (q = 1, no mask: the token sees every
        key) in one native call, sva_decode_layer_step: the catalog append of
        the cache's new rows (the append rule of _key_catalog,
        sva/llama.py:578-624), the lookup with its verifier (:211-317) and the
        step's statistics (:319-326), summed on the device.  key / value: the
        cache [1, G, N, D], read in place."""

        k_len = key.shape[2]
        sig = (key.device, key.dtype, self._heads, key.shape[3], self.serving.rank_dim)
        can_append = (self._signature == sig and self._k_low is not None and self._key_len > 0
                      and self._key_len < k_len <= self._key_len + 1)
        self._ensure_capacity(k_len, key.device)
        row_begin = min(self._key_len, self._codes_len) if can_append else 0
        shortlist = min(self.serving.coarse_shortlist, k_len)
        budget = min(self.serving.budget, shortlist)
        layer = self._decode_layer
        if layer is None or layer.plan.shape[-2:] != (shortlist, budget) or layer.device != query.device or \
                layer.plan.shape[3] != query.shape[3]:
            shape = (1, self._heads, 1, query.shape[3], self._rank, self._subspaces, self._codewords, shortlist,
                     budget)
            plan = self._decode_plan
            if plan is None or plan.shape != shape or plan.device != query.device:
                plan = self._decode_plan = kernels.ScanDecodePlan(query.device, *shape)
            layer = self._decode_layer = kernels.DecodeLayer(plan, self.sva_q_proj, self.sva_scale,
                                                             self.sva_coarse_codebooks, self.sva_k_proj, self.scaling)
            if self.stats is not None:
                self.stats.attach_device_counter(int(self.layer_idx or 0), kernels.DecodeLayer.STAT_ROWS,
                                                 layer.stats)
        out = layer.step(query, key, value, self._k_low, self._codes, row_begin, k_len)
        self._key_len = self._codes_len = k_len
        self._postings = None
        self._signature = sig
        # the next token takes _decode_next while nothing but the key count
        # moves on (the plan's shortlist and budget are final from L keys on)
        self._fast = None
        if k_len >= self.serving.coarse_shortlist:
            self._fast = (layer, sig, query.shape, key.shape[1], key.shape[3], key.dtype, query.dtype,
                          key.get_device(), self.serving.coarse_shortlist, self.serving.budget)
        return out

    def _decode_next(self, query, key, value):
        """The native decode step for the token after one _native_decode set
        up: the cache grew by one row and its shapes, strides pattern, dtypes
        and device, the query's shape and the catalog are as checked then, so
        only those are compared again (a few attribute reads instead of the
        full checks).  None when anything differs: the caller takes the full
        path."""
        layer, sig, qshape, kv_heads, head_dim, kv_dtype, q_dtype, dev, shortlist, budget = self._fast
        serving = self.serving
        ks = key.shape
        n = ks[2]
        if (n != self._key_len + 1 or self._codes_len != self._key_len or self._signature is not sig
                or self._k_low is None or n > self._k_low.shape[1] or query.shape != qshape
                or ks[0] != 1 or ks[1] != kv_heads or ks[3] != head_dim or key.dtype is not kv_dtype
                or value.dtype is not kv_dtype or query.dtype is not q_dtype or serving.summon_mode != "scan"
                or serving.coarse_shortlist != shortlist or serving.budget != budget):
            return None
        kst = key.stride()
        if (kst[3] != 1 or value.shape != ks or value.stride() != kst or query.stride(3) != 1
                or key.get_device() != dev or value.get_device() != dev or query.get_device() != dev):
            return None
        out = layer.step_next(query, key, value, kst, self._k_low, self._codes, n - 1, n)
        if out is not None:
            self._key_len = self._codes_len = n
        return out

    def _scan_attention(self, query, keys, values, k_low, codes, k_len, mask, shortlist, budget):
        """sva/llama.py:226-328 on the HIP path, chunked over query tokens."""

        outs = []
        for qs, qe, m, n in self._query_chunks(query, k_len, mask, shortlist, budget, codes):
            qc = query[:, :, qs:qe, :]
            q_low, lut, rng = kernels.query_lut(qc, self.sva_q_proj, self.sva_scale, self.sva_coarse_codebooks,
                                                codes, n, shortlist)
            _, _, sl_count, fin_idx, fin_count = kernels.summon_select(lut, rng, q_low, codes, k_low, n, shortlist,
                                                                       budget, mask=m, keep_shortlist=False)
            outs.append(kernels.verify(qc, keys, values, fin_idx, fin_count, n, self.scaling,
                                       out_dtype=query.dtype))
            if self.stats is not None:
                self.stats.add_device(int(self.layer_idx or 0), {
                    "summoned": sl_count, "exact_scored": fin_count, "verified": fin_count,
                    "queries": float(sl_count.numel())})
        return outs[0] if len(outs) == 1 else torch.cat(outs, dim=2)

    def _query_chunks(self, query, k_len, mask, shortlist, budget, codes):
        """(qs, qe, mask, n_keys) per chunk of query tokens (sva/llama.py:221-223,
        262-268).  Every token's result is independent of the chunking, so the
        default chunk bounds the per-launch buffers (about 512 MiB) rather
        than following the reference's 128: the shortlist buffers, or, where
        the fused per-item summon keeps the shortlist inside the kernel
        (sva_summon_strategy 3), the tables and budget lists.  Without a mask
        the kernels' causal rule (key n for token t of Q iff n <= N - Q + t)
        is kept by handing chunk [qs, qe) the first N - Q + qe keys: token
        qs + t then keeps n <= N - Q + qs + t, as over the whole prompt.
        There, chunks also end where the key count crosses 4096 and 8192, the
        fused kernel's register tiers, so early tokens take the smaller one."""

        n_seq, heads, q_len = query.shape[0], query.shape[1], query.shape[2]
        fused = kernels.lib().sva_summon_strategy(
            n_seq, heads, q_len, k_len, self._rank, self._subspaces, self._codewords, shortlist,
            kernels.code_type(codes), 0) == 3
        chunk = self.serving.query_chunk_size
        if chunk is None:
            if fused:
                per_token = n_seq * heads * 4 * (budget + self._rank + self._subspaces * self._codewords + 8)
            else:
                per_token = n_seq * heads * max(shortlist, 1) * 8
            chunk = q_len if q_len * per_token <= (512 << 20) else max(128, ((512 << 20) // per_token) // 128 * 128)
        chunk = max(1, int(chunk))
        edges = set(range(chunk, q_len, chunk))
        if mask is None and fused:
            edges |= {e - (k_len - q_len) for e in (4096, 8192) if 0 < e - (k_len - q_len) < q_len}
        bounds = [0, *sorted(edges), q_len]
        for qs, qe in zip(bounds[:-1], bounds[1:]):
            if mask is not None:
                yield qs, qe, mask[..., qs:qe, :], k_len
            else:
                yield qs, qe, None, k_len - q_len + qe

    def _scan_attention_batched(self, query, key, value, attention_mask):
        """Scan mode for a batch of B equal-length sequences (the reference
        decodes batch 1): one packed launch per stage for the whole batch.
        The catalog holds sequence b at rows [b * cap, b * cap + N); K and V
        are read in place from the cache [B, G, N, D] (row offsets b * G * N
        for a contiguous cache).  Every sequence must share the attention
        mask (no padding)."""

        batch, heads, q_len, head_dim = query.shape
        k_len = key.shape[2]
        device = query.device
        k_low, codes, cap = self._key_catalog_batched(key, q_len)
        shortlist = min(self.serving.coarse_shortlist, k_len)
        budget = min(self.serving.budget, shortlist)
        mask = None
        if attention_mask is not None:
            m = attention_mask[..., :q_len, :k_len]
            # decode steps included: a left-padded batch gives each sequence
            # its own mask row, which the packed launch cannot take
            if m.shape[0] > 1 and not kernels.mask_is_uniform(m.reshape(m.shape[0], -1, m.shape[-1])):
                raise ValueError("Batched SVA attention needs the same attention mask for every sequence (no padding).")
            mask = m[:1]
        if key.stride(0) % key.stride(2) != 0 or value.stride() != key.stride() or key.stride(-1) != 1:
            key, value = key.contiguous(), value.contiguous()
        rows_per_seq = key.stride(0) // key.stride(2)
        rows = (batch - 1) * rows_per_seq + k_len
        keys = torch.as_strided(key, (key.shape[1], rows, head_dim), (key.stride(1), key.stride(2), 1),
                                key.storage_offset())
        values = torch.as_strided(value, (value.shape[1], rows, head_dim), (value.stride(1), value.stride(2), 1),
                                  value.storage_offset())
        seq = torch.arange(batch, device=device, dtype=torch.int64)
        cat_off, kv_off = seq * cap, seq * rows_per_seq
        outs = []
        for qs, qe, m, n in self._query_chunks(query, k_len, mask, shortlist, budget, codes):
            lens = torch.full((batch,), n, device=device, dtype=torch.int64)
            qc = query[:, :, qs:qe, :]
            q_low, lut, rng = kernels.query_lut(qc, self.sva_q_proj, self.sva_scale, self.sva_coarse_codebooks)
            _, _, sl_count, fin_idx, fin_count = kernels.summon_select(lut, rng, q_low, codes, k_low, n, shortlist,
                                                                       budget, mask=m, seq_offsets=cat_off,
                                                                       seq_lens=lens, keep_shortlist=False)
            outs.append(kernels.verify(qc, keys, values, fin_idx, fin_count, rows, self.scaling, out_dtype=query.dtype,
                                       seq_offsets=kv_off, seq_lens=lens))
            if self.stats is not None:
                self.stats.add_device(int(self.layer_idx or 0), {
                    "summoned": sl_count, "exact_scored": fin_count, "verified": fin_count,
                    "queries": float(sl_count.numel())})
        return outs[0] if len(outs) == 1 else torch.cat(outs, dim=2)

    def _key_catalog_batched(self, key: torch.Tensor, q_len: int):
        """The catalog of a batch of equal-length sequences (sva/llama.py:578-624
        per sequence): appended when every cache grew by at most q_len rows,
        rebuilt otherwise.  Returns (k_low, codes, cap)."""

        batch, _, k_len, head_dim = key.shape
        heads, rank = self.sva_q_proj.shape[0], self.sva_q_proj.shape[2]
        subspaces, codewords = self.sva_coarse_codebooks.shape[1], self.sva_coarse_codebooks.shape[2]
        sig = ("batch", batch, key.device, key.dtype, heads, head_dim, rank)
        same = self._signature == sig and self._k_low is not None
        can_append = (same and self._key_len > 0 and k_len > self._key_len and k_len - self._key_len <= max(q_len, 1)
                      and q_len < k_len)
        cap = self._k_low.shape[1] // batch if same else 0
        if k_len > cap:
            new_cap = max(k_len, 2 * cap, 256)
            k_low = torch.empty(heads, batch * new_cap, rank, device=key.device, dtype=torch.float32)
            codes = torch.empty(heads, batch * new_cap, subspaces, device=key.device, dtype=_code_dtype(codewords))
            if can_append:
                for b in range(batch):
                    k_low[:, b * new_cap:b * new_cap + self._key_len].copy_(
                        self._k_low[:, b * cap:b * cap + self._key_len])
                    codes[:, b * new_cap:b * new_cap + self._key_len].copy_(
                        self._codes[:, b * cap:b * cap + self._key_len])
            self._k_low, self._codes, cap = k_low, codes, new_cap
        start = self._key_len if can_append else 0
        if key.stride(-1) == 1:  # every sequence in one call (one launch for a decode step's rows)
            kernels.write_encode_batch(key, self.sva_k_proj, self.sva_coarse_codebooks, self._k_low, self._codes, cap,
                                       start, k_len - start)
        else:
            for b in range(batch):
                kernels.write_encode(key[b], self.sva_k_proj, self.sva_coarse_codebooks,
                                     self._k_low[:, b * cap:(b + 1) * cap], self._codes[:, b * cap:(b + 1) * cap],
                                     start, k_len - start)
        self._key_len = self._codes_len = k_len
        self._postings = None
        self._signature = sig
        return self._k_low, self._codes, cap

    # ------------------------------------------------------------------
    def _ensure_capacity(self, rows: int, device: torch.device) -> None:
        heads, rank = self.sva_q_proj.shape[0], self.sva_q_proj.shape[2]
        subspaces, codewords = self.sva_coarse_codebooks.shape[1], self.sva_coarse_codebooks.shape[2]
        cap = 0 if self._k_low is None else self._k_low.shape[1]
        if rows <= cap:
            return
        new_cap = max(rows, 2 * cap, 256)
        k_low = torch.empty(heads, new_cap, rank, device=device, dtype=torch.float32)
        codes = torch.empty(heads, new_cap, subspaces, device=device, dtype=_code_dtype(codewords))
        if self._k_low is not None and self._key_len:
            k_low[:, :self._key_len].copy_(self._k_low[:, :self._key_len])
            codes[:, :self._codes_len].copy_(self._codes[:, :self._codes_len])
        self._k_low, self._codes = k_low, codes

    def _encode(self, keys: torch.Tensor, row0: int, row1: int, with_codes: bool = True) -> None:
        if row1 > row0:
            kernels.write_encode(keys, self.sva_k_proj, self.sva_coarse_codebooks, self._k_low,
                                 self._codes if with_codes else None, row0, row1 - row0)

    def _key_catalog(self, keys: torch.Tensor, q_len: int):
        """Bring the catalog up to the cache's length (sva/llama.py:578-624):
        append the new rows when the cache grew by at most q_len rows since
        the last call, rebuild otherwise.  In inverted_static decode new rows
        get k_low only; their codes and the postings are made once the tail
        behind the postings reaches static_tail_rebuild_interval rows (the
        reference's lazy tail, :604-610)."""

        k_len = keys.shape[1]
        sig = (keys.device, keys.dtype, int(self.sva_q_proj.shape[0]), int(keys.shape[2]), self.serving.rank_dim)
        can_append = (self._signature == sig and self._k_low is not None and self._key_len > 0
                      and k_len > self._key_len and k_len - self._key_len <= max(q_len, 1) and q_len < k_len)
        mode = self.serving.summon_mode
        codewords = int(self.sva_coarse_codebooks.shape[2])
        self._ensure_capacity(k_len, keys.device)
        if can_append:
            start = self._key_len
            if mode == "inverted_static" and q_len == 1:
                interval = max(1, int(self.serving.static_tail_rebuild_interval))
                if self._postings is None or k_len - self._postings.key_len >= interval:
                    self._encode(keys, start, k_len, with_codes=False)
                    self._encode(keys, self._codes_len, k_len)  # codes of every row not yet coded
                    self._codes_len = k_len
                    self._postings = inverted.build_postings(self._codes, k_len, codewords)
                else:
                    self._encode(keys, start, k_len, with_codes=False)
            else:
                self._encode(keys, min(start, self._codes_len), k_len)
                self._codes_len = k_len
                if mode == "inverted":
                    self._postings = inverted.append_postings(self._postings, self._codes, k_len, codewords)
        else:
            self._encode(keys, 0, k_len)
            self._codes_len = k_len
            self._postings = None
            if mode in ("inverted", "inverted_static"):
                self._postings = inverted.build_postings(self._codes, k_len, codewords)
        self._key_len = k_len
        self._signature = sig
        return self._k_low, self._codes

    # views with the reference module's attribute names (sva/llama.py:75-81)
    @property
    def _cached_key_len(self) -> int:
        return self._key_len

    @property
    def _cached_postings_key_len(self) -> int:
        return 0 if self._postings is None else self._postings.key_len

    @property
    def _cached_coarse_codes(self) -> torch.Tensor | None:
        return None if self._codes is None else self._codes[:, :self._codes_len]

    @property
    def _cached_k_low(self) -> torch.Tensor | None:
        return None if self._k_low is None else self._k_low[None, :, :self._key_len]


class SVALlamaPatcher:
    """Reversible patch handle (sva/llama.py:695-806)."""

    def __init__(self, model: nn.Module, bundle: SVAArtifactBundle, shortlist: int | None = None,
                 budget: int | None = None, assign_chunk_size: int = 8192, query_chunk_size: int | None = None,
                 summon_mode: str = "scan", inverted_cells_per_subspace: int = 8,
                 adaptive_min_budget: int | None = None, adaptive_mid_budget: int | None = None,
                 adaptive_low_margin: float = 0.35, adaptive_high_margin: float = 0.70,
                 profile_components: bool = False, static_tail_rebuild_interval: int = 64,
                 layers: list[int] | None = None) -> None:
        if summon_mode not in SUMMON_MODES:
            raise ValueError(f"Unknown SVA summon_mode: {summon_mode!r}")
        self.model = model
        self.bundle = bundle
        self.stats = SVAStats()
        self.originals: dict[int, nn.Module] = {}
        self.layers = None if layers is None else list(dict.fromkeys(int(i) for i in layers))
        self.serving = SVALlamaServingConfig(
            rank_dim=bundle.rank_dim,
            coarse_shortlist=bundle.default_shortlist if shortlist is None else int(shortlist),
            budget=bundle.default_budget if budget is None else int(budget),
            assign_chunk_size=assign_chunk_size,
            query_chunk_size=query_chunk_size,
            summon_mode=summon_mode,
            inverted_cells_per_subspace=inverted_cells_per_subspace,
            adaptive_min_budget=adaptive_min_budget,
            adaptive_mid_budget=adaptive_mid_budget,
            adaptive_low_margin=adaptive_low_margin,
            adaptive_high_margin=adaptive_high_margin,
            profile_components=profile_components,
            static_tail_rebuild_interval=static_tail_rebuild_interval,
        )

    def patch(self) -> "SVALlamaPatcher":
        model_layers = getattr(getattr(self.model, "model", None), "layers", None)
        if model_layers is None:
            raise ValueError("Expected a Hugging Face Llama-style model with model.layers.")
        if self.originals:
            return self
        if self.bundle.layer_count != len(model_layers):
            raise ValueError(f"Artifact has {self.bundle.layer_count} layers but model has {len(model_layers)}.")
        model_id = self.bundle.model_id
        model_name = getattr(getattr(self.model, "config", None), "_name_or_path", None)
        if model_id and model_name and str(model_name) not in {"", model_id}:
            raise ValueError(f"Artifact model_id={model_id!r} does not match loaded model {model_name!r}.")
        targets = self.layers if self.layers is not None else list(range(len(model_layers)))
        for i in targets:
            if i < 0 or i >= len(model_layers):
                raise ValueError(f"Patch layer index {i} is outside model layer range 0..{len(model_layers) - 1}.")
            layer = model_layers[i]
            artifacts = self.bundle.layers.get(i)
            if artifacts is None:
                raise ValueError(f"Missing SVA artifacts for layer {i}.")
            self._validate_layer_shapes(i, layer.self_attn, artifacts)
            self.originals[i] = layer.self_attn
            replacement = SVALlamaAttention(layer.self_attn, artifacts, self.serving, self.stats)
            try:
                device = next(layer.self_attn.parameters()).device
            except StopIteration:
                device = artifacts.q_proj.device
            replacement.to(device=device)
            replacement.train(layer.self_attn.training)
            layer.self_attn = replacement
        return self

    def unpatch(self) -> None:
        layers = self.model.model.layers
        for i, original in self.originals.items():
            layers[i].self_attn = original
        self.originals.clear()

    def reset_stats(self) -> None:
        self.stats.reset()

    def reset_catalogs(self) -> None:
        for layer in self.model.model.layers:
            attention = self._unwrap_sva_attention(layer.self_attn)
            if isinstance(attention, SVALlamaAttention):
                attention.reset_catalog()

    @staticmethod
    def _unwrap_sva_attention(attention: nn.Module) -> nn.Module:
        while hasattr(attention, "sva_attn"):
            attention = getattr(attention, "sva_attn")
        return attention

    def __enter__(self) -> "SVALlamaPatcher":
        return self.patch()

    def __exit__(self, exc_type: object, exc: object, traceback: object) -> None:
        self.unpatch()

    def _validate_layer_shapes(self, i: int, attention: nn.Module, artifacts: SVALayerArtifacts) -> None:
        expected = (int(attention.config.num_attention_heads), int(attention.head_dim), self.bundle.rank_dim)
        if tuple(artifacts.q_proj.shape) != expected:
            raise ValueError(f"Layer {i} artifact q_proj shape {tuple(artifacts.q_proj.shape)} != {expected}.")
        if tuple(artifacts.k_proj.shape) != expected:
            raise ValueError(f"Layer {i} artifact k_proj shape {tuple(artifacts.k_proj.shape)} != {expected}.")


def patch_llama_attention(model: nn.Module, artifact_dir_or_bundle: str | Path | SVAArtifactBundle,
                          shortlist: int | None = None, budget: int | None = None, assign_chunk_size: int = 8192,
                          query_chunk_size: int | None = None, summon_mode: str = "scan",
                          inverted_cells_per_subspace: int = 8, adaptive_min_budget: int | None = None,
                          adaptive_mid_budget: int | None = None, adaptive_low_margin: float = 0.35,
                          adaptive_high_margin: float = 0.70, profile_components: bool = False,
                          static_tail_rebuild_interval: int = 64, layers: list[int] | None = None) -> SVALlamaPatcher:
    """Patch a Llama-family model with SVA attention; returns the (already
    applied) reversible handle (sva/llama.py:808-848)."""

    bundle = (artifact_dir_or_bundle if isinstance(artifact_dir_or_bundle, SVAArtifactBundle)
              else load_sva_artifact_bundle(artifact_dir_or_bundle))
    return SVALlamaPatcher(model, bundle, shortlist=shortlist, budget=budget, assign_chunk_size=assign_chunk_size,
                           query_chunk_size=query_chunk_size, summon_mode=summon_mode,
                           inverted_cells_per_subspace=inverted_cells_per_subspace,
                           adaptive_min_budget=adaptive_min_budget, adaptive_mid_budget=adaptive_mid_budget,
                           adaptive_low_margin=adaptive_low_margin, adaptive_high_margin=adaptive_high_margin,
                           profile_components=profile_components,
                           static_tail_rebuild_interval=static_tail_rebuild_interval, layers=layers).patch()

