"""Writes tests/golden/inverted_reference.npz: what the reference's own
SVALlamaAttention._inverted_static_decode_attention (sva/llama.py:427-576)
and ._inverted_decode_attention (sva/llama.py:330-425) choose and return on
the seeded cases of tests/cases.py:INVERTED_CASES.

Run in a container that holds the reference at /root/reference
(``python tests/golden/make_inverted_golden.py``); nothing on the GPU side runs
this file, the tests read only the .npz.  The reference's methods are called
on a real transformers LlamaAttention wrapped by the reference's
SVALlamaAttention; q_low is the reference's expression (sva/llama.py:211),
the postings its own _rebuild_postings over the first N - tail rows.  The
decode methods return only the attention output, so a TorchFunctionMode
records what they pass to torch:
  static:   the arguments and results of _top_unique_candidates (candidates
            with their validity, refill count, selected ids) and the softmax
            input (slots outside the budget hold finfo.min);
  adaptive: per head, the k_low rows gathered (the candidates) and the
            key rows gathered (the verified keys).
Before saving, every decision the cases rest on is checked to sit well away
from a tie (cell choice, refill and budget boundaries, adaptive margins), so
a last-bit difference in q_low cannot change the recorded sets.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch
from torch.overrides import TorchFunctionMode

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, "/root/reference")
sys.path.insert(1, str(ROOT))

import torch.nn.functional as F  # noqa: E402
from sva.artifacts import SVALayerArtifacts  # noqa: E402
from sva.llama import SVALlamaAttention, SVALlamaServingConfig  # noqa: E402
from sva.stats import SVAStats  # noqa: E402
from transformers import LlamaConfig  # noqa: E402
from transformers.models.llama.modeling_llama import LlamaAttention  # noqa: E402

from tests.cases import INVERTED_CASES, inverted_inputs  # noqa: E402

FMIN = torch.finfo(torch.float32).min
MIN_GAP = 1e-4  # smallest distance kept between a decision value and its neighbour


class Recorder(TorchFunctionMode):
    def __init__(self, key_states, k_low):
        super().__init__()
        self.key_states, self.k_low = key_states, k_low
        self.softmax_in, self.key_rows, self.low_rows = [], [], []

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is F.softmax:
            self.softmax_in.append(args[0].detach().clone())
        elif func is torch.Tensor.__getitem__ and isinstance(args[1], tuple) and len(args[1]) == 3:
            index = args[1][2]
            if isinstance(index, torch.Tensor):
                if args[0] is self.key_states:
                    self.key_rows.append(index.detach().clone())
                elif args[0] is self.k_low:
                    self.low_rows.append(index.detach().clone())
        return func(*args, **kwargs)


def _rank(k_low_h, idx, q):
    return ((k_low_h[idx].double() * q.double()).sum(-1) / 8.0).numpy()


def _check_gaps(name, values, boundary):
    """values sorted descending (distinct keys); no near-tie across `boundary`."""

    if 0 < boundary < len(values):
        gap = values[boundary - 1] - values[boundary]
        assert gap > MIN_GAP, f"{name}: near-tie at boundary {boundary} (gap {gap})"


def run_case(case):
    mode, N, tail, budget, cells, amin, amid, low, high, mask_frac, cur_masked, seed = case
    inp = inverted_inputs(seed, N, mask_frac, cur_masked)
    H, _, D = inp["q"].shape
    G = inp["keys"].shape[0]
    R = inp["q_proj"].shape[2]
    S, C = inp["codebooks"].shape[1], inp["codebooks"].shape[2]
    assert inp["allowed"].any(), "every key masked"
    cfg = LlamaConfig(hidden_size=H * D, num_attention_heads=H, num_key_value_heads=G, head_dim=D,
                      intermediate_size=4 * D, num_hidden_layers=1, vocab_size=32)
    original = LlamaAttention(cfg, layer_idx=0).eval()
    art = SVALayerArtifacts(q_proj=torch.from_numpy(inp["q_proj"]), k_proj=torch.from_numpy(inp["q_proj"]),
                            logit_scale=torch.from_numpy(inp["logit_scale"]),
                            coarse_codebooks=torch.from_numpy(inp["codebooks"]), train_loss=0.0, hard_loss=0.0,
                            route_source="qk")
    serving = SVALlamaServingConfig(rank_dim=R, coarse_shortlist=4 * budget, budget=budget, summon_mode=mode,
                                    inverted_cells_per_subspace=cells, adaptive_min_budget=amin or None,
                                    adaptive_mid_budget=amid or None, adaptive_low_margin=low,
                                    adaptive_high_margin=high)
    stats = SVAStats()
    attn = SVALlamaAttention(original, art, serving, stats).eval()

    query = torch.from_numpy(inp["q"])[None]                                        # [1, H, 1, D]
    key_states = torch.from_numpy(inp["keys"])[None].repeat_interleave(H // G, dim=1)   # repeat_kv
    value_states = torch.from_numpy(inp["values"])[None].repeat_interleave(H // G, dim=1)
    k_low = torch.from_numpy(inp["k_low"])[None]
    codes = torch.from_numpy(inp["codes"]).long()
    codebooks = attn.sva_coarse_codebooks
    allowed = torch.from_numpy(inp["allowed"])[None, None, None, :].expand(1, H, 1, N)
    actual_budget = min(budget, min(4 * budget, N))

    recorded = {}
    top_unique = SVALlamaAttention._top_unique_candidates

    def spy(candidate_idx, candidate_scores, candidate_valid, budget, refill_factor=2):
        res = top_unique(candidate_idx, candidate_scores, candidate_valid, budget, refill_factor)
        recorded.update(idx=candidate_idx.clone(), scores=candidate_scores.clone(), valid=candidate_valid.clone(),
                        sel=res[0].clone(), sel_scores=res[1].clone(), sel_valid=res[2].clone(), refill=res[3])
        return res

    with torch.no_grad():
        q_low = torch.einsum("bhtd,hdr->bhtr", query.float(), attn.sva_q_proj) * attn.sva_scale[None, :, None, None]
        attn._rebuild_postings(codes[:, : N - tail], C)
        rec = Recorder(key_states, k_low)
        SVALlamaAttention._top_unique_candidates = staticmethod(spy)
        try:
            with rec:
                if mode == "inverted_static":
                    out = attn._inverted_static_decode_attention(query, key_states, value_states, q_low, k_low,
                                                                 codes, codebooks, allowed, actual_budget)
                else:
                    out = attn._inverted_decode_attention(query, key_states, value_states, q_low, k_low, codes,
                                                          codebooks, allowed, actual_budget)
        finally:
            SVALlamaAttention._top_unique_candidates = staticmethod(top_unique)

    # cell choice: the cells-th and next LUT entries apart
    lut = torch.einsum("hsd,hscd->hsc", q_low[0, :, 0].reshape(H, S, R // S).double(), codebooks.double())
    for h in range(H):
        for s in range(S):
            _check_gaps(f"head {h} subspace {s} cells", np.sort(lut[h, s].numpy())[::-1] / 8.0, cells)

    cands, finals, refills = [], [], []
    if mode == "inverted_static":
        idx, valid = recorded["idx"], recorded["valid"]
        sm = rec.softmax_in[0]
        for h in range(H):
            cands.append(np.sort(idx[h][valid[h]].numpy()))
            keep = sm[h] > FMIN
            finals.append(np.sort(recorded["sel"][h][keep].numpy()))
            # refill window (entries counted with multiplicity), budget and
            # final boundaries over distinct valid keys
            ids_h = idx[h][valid[h]].numpy()
            sc = _rank(k_low[0, h], torch.from_numpy(ids_h), q_low[0, h, 0])
            order = np.lexsort((ids_h, -sc))
            r = recorded["refill"]
            if 0 < r < len(order) and ids_h[order[r - 1]] != ids_h[order[r]]:
                assert sc[order[r - 1]] - sc[order[r]] > MIN_GAP, f"head {h}: near-tie at the refill boundary"
            scores = np.sort(_rank(k_low[0, h], torch.from_numpy(np.unique(ids_h)), q_low[0, h, 0]))[::-1]
            _check_gaps(f"head {h} budget", scores, min(actual_budget, len(scores)))
            _check_gaps(f"head {h} final", scores, int(keep.sum()))
            refills.append(r)
        width = int(idx.shape[1])
    else:
        assert len(rec.low_rows) == H and len(rec.key_rows) == H
        for h in range(H):
            cands.append(np.sort(rec.low_rows[h].numpy()))
            finals.append(np.sort(rec.key_rows[h].numpy()))
            scores = np.sort(_rank(k_low[0, h], rec.low_rows[h], q_low[0, h, 0]))[::-1]
            _check_gaps(f"head {h} budget", scores, min(actual_budget, len(scores)))
            _check_gaps(f"head {h} final", scores, len(finals[-1]))
            refills.append(0)
        width = 0
    # adaptive margins: away from both thresholds
    min_b = min(amin or actual_budget, actual_budget, N)
    for h in range(H):
        if mode == "inverted_static":
            sel = recorded["sel_scores"][h].double().numpy()
            rank_count = len(sel)
            margin = sel[0] - sel[min(min_b, rank_count) - 1] if rank_count > 1 else None
        else:
            scores = np.sort(_rank(k_low[0, h], torch.from_numpy(np.unique(cands[h])), q_low[0, h, 0]))[::-1]
            rank_count = min(actual_budget, len(scores))
            margin = scores[0] - scores[min(min_b, rank_count) - 1] if rank_count > 1 else None
        if margin is not None:
            for thr in (low, high):
                assert abs(margin - thr) > MIN_GAP, f"head {h}: margin {margin} near {thr}"

    totals = {k: float(v) for k, v in stats.totals.items()}
    return {
        "params": json.dumps({"mode": mode, "N": N, "tail": tail, "budget": budget, "cells": cells, "amin": amin,
                              "amid": amid, "low": low, "high": high, "mask_frac": mask_frac,
                              "current_masked": cur_masked, "seed": seed, "width": width,
                              "stats": totals}),
        "q_low": q_low[0, :, 0].numpy(),
        "cand": np.concatenate(cands).astype(np.int32),
        "cand_count": np.array([len(c) for c in cands], np.int32),
        "final": np.concatenate(finals).astype(np.int32),
        "final_count": np.array([len(f) for f in finals], np.int32),
        "refill": np.array(refills, np.int32),
        "out": out[0, :, 0].numpy(),
    }


def main() -> None:
    torch.set_num_threads(1)
    arrays = {"torch_version": np.array(torch.__version__)}
    for i, case in enumerate(INVERTED_CASES):
        res = run_case(case)
        for k, v in res.items():
            arrays[f"c{i}_{k}"] = np.asarray(v)
        p = json.loads(res["params"])
        print(f"case {i}: {case[0]} N={case[1]} tail={case[2]} B={case[3]} finals={res['final_count'].tolist()} "
              f"stats={p['stats']}")
    path = Path(__file__).with_name("inverted_reference.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path)


if __name__ == "__main__":
    main()
