"""Residual output adapter for the late-layer socket, behind the interface of
experiments/sva_late4_logit_distill.py:37-51 and :162-239 (behaviour only).

An adapter wraps one layer's attention module (normally an SVA-patched one)
and adds a low-rank correction computed from the layer input and the
attention output::

    out = attn + (up @ gelu(down @ [hidden, attn]) * scale).to(attn.dtype)

with ``down`` [rank, 2 * hidden] and ``up`` [hidden, rank] the weights of two
bias-free fp32 ``nn.Linear`` layers (so ``adapter.down(x)`` and
``adapter.up(x)`` work as in the experiment).  They are made and initialised
on the CPU as the experiment makes them (``down`` N(0, 0.02^2) from the
default generator, ``up`` zero, so a fresh adapter is the identity on the
attention output) and then moved to the wrapped module's device.  The
forward is one HIP launch (``sva_residual_adapter``) reading the two weights;
the adapter serves inference only (the distillation that trains it is
outside this package).

On disk an adapter set is the experiment's bundle: ``adapter_config.json``
(``format`` = "sva_residual_output_adapter_v1", ``socket_layers`` and any
caller fields) beside ``adapter_weights.pt`` = ``{"state_dict": {...}}`` with
one ``layers.{i}.down.weight`` / ``layers.{i}.up.weight`` pair per socket
layer.  Weights are read back with ``weights_only=True``.
"""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Any, Iterator

import torch
from torch import nn

from . import kernels

ADAPTER_FORMAT = "sva_residual_output_adapter_v1"
_WEIGHTS = ("down.weight", "up.weight")  # per-layer entries of a bundle, in this order


def _module_device(module: nn.Module) -> torch.device:
    for t in module.parameters():
        return t.device
    for t in module.buffers():
        return t.device
    return torch.device("cpu")


class SVAResidualOutputAdapter(nn.Module):
    """The socket adapter around ``sva_attn``; returns ``(corrected attention output, attn weights)``."""

    def __init__(self, sva_attn: nn.Module, hidden_size: int, rank: int, scale: float) -> None:
        super().__init__()
        if hidden_size <= 0 or rank <= 0:
            raise ValueError(f"adapter needs hidden_size > 0 and rank > 0, got {hidden_size} and {rank}")
        device = _module_device(sva_attn)
        self.sva_attn = sva_attn
        self.scale = float(scale)
        # made and initialised on the CPU (the experiment's draw order), then moved
        down = nn.Linear(2 * hidden_size, rank, bias=False, dtype=torch.float32)
        up = nn.Linear(rank, hidden_size, bias=False, dtype=torch.float32)
        nn.init.normal_(down.weight, mean=0.0, std=0.02)
        nn.init.zeros_(up.weight)
        self.down = down.to(device)
        self.up = up.to(device)

    def forward(self, hidden_states: torch.Tensor, *args, **kwargs) -> tuple[torch.Tensor, Any]:
        attn_output, attn_weights = self.sva_attn(hidden_states, *args, **kwargs)
        if torch.is_grad_enabled() and (self.down.weight.requires_grad or self.up.weight.requires_grad):
            raise RuntimeError("SVAResidualOutputAdapter runs inference only: call it under torch.no_grad()")
        out = kernels.residual_adapter(hidden_states, attn_output, self.down.weight, self.up.weight, self.scale)
        return out, attn_weights

    def socket_state(self) -> dict[str, torch.Tensor]:
        """The adapter's own weights (not the wrapped attention's), detached host copies."""
        return {"down.weight": self.down.weight.detach().cpu(), "up.weight": self.up.weight.detach().cpu()}

    @torch.no_grad()
    def load_socket_state(self, state: dict[str, torch.Tensor]) -> None:
        for name, dst in zip(_WEIGHTS, (self.down.weight, self.up.weight)):
            src = state[name]
            if tuple(src.shape) != tuple(dst.shape):
                raise ValueError(f"adapter {name}: stored {tuple(src.shape)}, module expects {tuple(dst.shape)}")
            dst.copy_(src.to(device=dst.device, dtype=dst.dtype))


def _socket_adapters(model: nn.Module, socket_layers: list[int]) -> Iterator[tuple[int, SVAResidualOutputAdapter]]:
    layers = model.model.layers
    for i in socket_layers:
        module = layers[i].self_attn
        if not isinstance(module, SVAResidualOutputAdapter):
            raise TypeError(f"Layer {i} is not wrapped with SVAResidualOutputAdapter.")
        yield i, module


def wrap_socket_layers_with_adapters(model: nn.Module, socket_layers: list[int], rank: int,
                                     scale: float) -> list[SVAResidualOutputAdapter]:
    """Replace each socket layer's ``self_attn`` by an adapter around it (on its device); returns them."""

    hidden = int(model.config.hidden_size)
    made = []
    for i in socket_layers:
        layer = model.model.layers[i]
        layer.self_attn = SVAResidualOutputAdapter(layer.self_attn, hidden, rank, scale)
        made.append(layer.self_attn)
    return made


def collect_adapter_state(model: nn.Module, socket_layers: list[int]) -> dict[str, torch.Tensor]:
    """``layers.{i}.down.weight`` / ``layers.{i}.up.weight`` for every socket layer, on the host."""

    return {f"layers.{i}.{name}": t for i, a in _socket_adapters(model, socket_layers)
            for name, t in a.socket_state().items()}


def load_adapter_weights(model: nn.Module, socket_layers: list[int], state_dict: dict[str, torch.Tensor]) -> None:
    """Copy a bundle's weights into the wrapped socket layers (KeyError names a missing entry)."""

    for i, a in _socket_adapters(model, socket_layers):
        keys = {name: f"layers.{i}.{name}" for name in _WEIGHTS}
        missing = [k for k in keys.values() if k not in state_dict]
        if missing:
            raise KeyError(f"adapter weights lack {missing}")
        a.load_socket_state({name: state_dict[k] for name, k in keys.items()})


def save_adapter_bundle(output_dir: Path | str, model: nn.Module, socket_layers: list[int],
                        manifest: dict[str, Any]) -> None:
    """Write ``adapter_config.json`` (format, socket layers, then the caller's
    fields) and ``adapter_weights.pt``; each file is written to a temporary
    name first and renamed, so a reader never sees half a bundle file."""

    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    config = {"format": ADAPTER_FORMAT, "socket_layers": [int(i) for i in socket_layers], **manifest}
    state = collect_adapter_state(model, socket_layers)
    tmp = out / "adapter_config.json.tmp"
    tmp.write_text(json.dumps(config, indent=2) + "\n", encoding="utf-8")
    os.replace(tmp, out / "adapter_config.json")
    tmp = out / "adapter_weights.pt.tmp"
    torch.save({"state_dict": state}, tmp)
    os.replace(tmp, out / "adapter_weights.pt")


def load_adapter_bundle(adapter_dir: Path | str) -> tuple[dict[str, Any], dict[str, torch.Tensor]]:
    """(manifest, state dict) of a bundle.  The weights file may hold the
    state dict under ``state_dict`` or be the state dict itself; it is read
    with weights_only=True, so nothing in it executes."""

    d = Path(adapter_dir)
    manifest = json.loads((d / "adapter_config.json").read_text(encoding="utf-8"))
    fmt = manifest.get("format")
    if fmt is not None and fmt != ADAPTER_FORMAT:
        raise ValueError(f"{d}: adapter format {fmt!r}, expected {ADAPTER_FORMAT!r}")
    payload = torch.load(d / "adapter_weights.pt", map_location="cpu", weights_only=True)
    state = payload.get("state_dict", payload) if isinstance(payload, dict) else None
    if not isinstance(state, dict) or not all(isinstance(v, torch.Tensor) for v in state.values()):
        raise TypeError(f"Unexpected adapter weights payload in {d}.")
    return manifest, state
