"""Runtime accounting of patched attention layers (sva/stats.py:13-54).

Same interface as the reference (``totals``, ``by_layer``, ``reset``, ``add``,
``ratio``, ``summary``), with the same keys.  Counts that live on the GPU
(shortlist and budget sizes of a decode step) are recorded with
``add_device`` / ``add_device_rows`` or kept in a device counter that the
native decode step adds to (``attach_device_counter``); they are brought to
the host only when the statistics are read, so a decode step never waits on
a device-to-host copy for its bookkeeping.  Decode heads whose sampled
shortlist floor overshot (a count the reference does not keep) are read
with ``floor_overshoots()`` and appear in no reference key.
"""

from __future__ import annotations

from collections import defaultdict

import torch


def _float_stats() -> defaultdict[str, float]:
    return defaultdict(float)


class SVAStats:
    """Aggregate statistics recorded by patched attention layers."""

    def __init__(self) -> None:
        self._totals: defaultdict[str, float] = _float_stats()
        self._by_layer: defaultdict[int, defaultdict[str, float]] = defaultdict(_float_stats)
        # (layer, name) -> float64 device accumulator not yet folded in
        self._pending: dict[tuple[int, str], torch.Tensor] = {}
        # (layer, row names) -> float64 device vector of row sums not yet folded in
        self._pending_rows: dict[tuple[int, tuple[tuple[str, ...], ...]], torch.Tensor] = {}
        # persistent int64 device counters [rows] a native step adds to: (layer, row names, counter)
        self._counters: list[tuple[int, tuple[tuple[str, ...], ...], torch.Tensor]] = []
        # counts kept beside the reference's keys (not in totals / by_layer / summary)
        self._extra: defaultdict[str, float] = _float_stats()

    # -- recording --------------------------------------------------------
    def add(self, layer_idx: int, values: dict[str, float]) -> None:
        layer = self._by_layer[layer_idx]
        for key, value in values.items():
            self._totals[key] += float(value)
            layer[key] += float(value)

    def add_device(self, layer_idx: int, values: dict[str, torch.Tensor | float]) -> None:
        """Accumulate device tensors (summed) or host floats without a sync."""

        host = {}
        for key, value in values.items():
            if isinstance(value, torch.Tensor):
                total = value.sum(dtype=torch.float64)
                slot = self._pending.get((layer_idx, key))
                self._pending[(layer_idx, key)] = total if slot is None else slot + total
            else:
                host[key] = value
        if host:
            self.add(layer_idx, host)

    def add_device_rows(self, layer_idx: int, names: tuple[tuple[str, ...], ...], counts: torch.Tensor,
                        host: dict[str, float] | None = None) -> None:
        """Accumulate the row sums of a device count matrix `counts` [rows,
        n]: row i adds to every statistic named in names[i].  One small
        device kernel per call (an int64 running matrix), no sync."""

        key = (layer_idx, names)
        slot = self._pending_rows.get(key)
        if slot is None or slot.shape != counts.shape:
            if slot is not None:
                self._fold_rows(key, slot)
            self._pending_rows[key] = counts.to(torch.int64)
        else:
            slot.add_(counts)  # one launch; the rows are summed when the statistics are read
        if host:
            self.add(layer_idx, host)

    def attach_device_counter(self, layer_idx: int, names: tuple[tuple[str, ...], ...], counter: torch.Tensor) -> None:
        """Register a persistent int64 device vector [len(names)] that decode
        steps add to on the device (row i adds to every statistic named in
        names[i]); it is folded in and zeroed when the statistics are read.
        Registering the same tensor again does nothing."""

        if counter.dtype != torch.int64 or counter.dim() != 1 or counter.numel() != len(names):
            raise ValueError(f"a device counter is int64 [{len(names)}], got {counter.dtype} {tuple(counter.shape)}")
        if not any(c is counter for _, _, c in self._counters):
            self._counters.append((layer_idx, names, counter))

    def floor_overshoots(self) -> float:
        """Decode heads whose sampled shortlist floor overshot (the exact all-keys select ran)."""

        self._flush()
        return self._extra.get("floor_overshoots", 0.0)

    def _add_named(self, layer_idx: int, name: str, v: float) -> None:
        if name == "floor_overshoots":
            self._extra[name] += v
            return
        self._totals[name] += v
        self._by_layer[layer_idx][name] += v

    def _fold_rows(self, key: tuple[int, tuple[tuple[str, ...], ...]], mat: torch.Tensor) -> None:
        layer_idx, names = key
        for row_names, v in zip(names, mat.sum(dim=1).tolist()):
            for name in row_names:
                self._add_named(layer_idx, name, float(v))

    def _flush(self) -> None:
        for layer_idx, names, counter in self._counters:
            values = counter.tolist()  # synchronizes with the steps that added to it
            counter.zero_()
            for row_names, v in zip(names, values):
                for name in row_names:
                    self._add_named(layer_idx, name, float(v))
        if self._pending_rows:
            rows, self._pending_rows = self._pending_rows, {}
            for key, mat in rows.items():
                self._fold_rows(key, mat)
        if not self._pending:
            return
        pending, self._pending = self._pending, {}
        for (layer_idx, key), value in pending.items():
            v = float(value.item())
            self._totals[key] += v
            self._by_layer[layer_idx][key] += v

    # -- reading ----------------------------------------------------------
    @property
    def totals(self) -> defaultdict[str, float]:
        self._flush()
        return self._totals

    @property
    def by_layer(self) -> defaultdict[int, defaultdict[str, float]]:
        self._flush()
        return self._by_layer

    def reset(self) -> None:
        for _, _, counter in self._counters:
            counter.zero_()
        self._pending.clear()
        self._pending_rows.clear()
        self._totals.clear()
        self._by_layer.clear()
        self._extra.clear()

    def ratio(self, numerator: str, denominator: str = "queries") -> float:
        totals = self.totals
        den = totals.get(denominator, 0.0)
        if den <= 0:
            return float("nan")
        return totals.get(numerator, 0.0) / den

    def summary(self) -> dict[str, float]:
        per_query = ("summoned", "refill_pool", "exact_scored", "verified", "cell_visits")
        out = {"queries": self.totals.get("queries", 0.0)}
        out.update({f"avg_{k}": self.ratio(k) for k in per_query})
        for k in ("catalog", "refill", "budget", "gather", "exact_score", "aggregate", "total"):
            out[f"avg_static_{k}_ms"] = self.ratio(f"static_{k}_ms", "profile_calls")
        for k in ("projection", "key_catalog", "outer_total"):
            out[f"avg_static_{k}_ms"] = self.ratio(f"static_{k}_ms", "profile_outer_calls")
        return out
