"""Residual output adapter of the late-layer socket
(experiments/sva_late4_logit_distill.py:37-51, :162-239).

``SVAResidualOutputAdapter`` wraps an attention module (normally an SVA-patched
one) and adds a low-rank correction computed from the layer input and the
attention output: ``out = attn + up(gelu(down([hidden, attn]))) * scale``, the
projections in fp32.  The forward is one HIP launch (``sva_residual_adapter``);
the adapter is inference-only here (the reference trains it by distillation,
which this package does not reproduce).  The bundle format is the reference's:
``adapter_config.json`` ("sva_residual_output_adapter_v1") and
``adapter_weights.pt`` = ``{"state_dict": {"layers.{i}.down.weight",
"layers.{i}.up.weight"}}``.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any

import torch
from torch import nn

from . import kernels

ADAPTER_FORMAT = "sva_residual_output_adapter_v1"


class SVAResidualOutputAdapter(nn.Module):
    """experiments/sva_late4_logit_distill.py:37-51."""

    def __init__(self, sva_attn: nn.Module, hidden_size: int, rank: int, scale: float) -> None:
        super().__init__()
        self.sva_attn = sva_attn
        self.scale = scale
        self.down = nn.Linear(hidden_size * 2, rank, bias=False, dtype=torch.float32)
        self.up = nn.Linear(rank, hidden_size, bias=False, dtype=torch.float32)
        nn.init.normal_(self.down.weight, mean=0.0, std=0.02)
        nn.init.zeros_(self.up.weight)

    def forward(self, hidden_states: torch.Tensor, *args, **kwargs) -> tuple[torch.Tensor, None]:
        attn_output, attn_weights = self.sva_attn(hidden_states, *args, **kwargs)
        if torch.is_grad_enabled() and (self.down.weight.requires_grad or self.up.weight.requires_grad):
            raise RuntimeError("SVAResidualOutputAdapter runs inference only: call it under torch.no_grad()")
        out = kernels.residual_adapter(hidden_states, attn_output, self.down.weight, self.up.weight, self.scale)
        return out, attn_weights


def wrap_socket_layers_with_adapters(model: nn.Module, socket_layers: list[int], rank: int, scale: float) -> None:
    """experiments/sva_late4_logit_distill.py:162-174."""

    hidden_size = int(model.config.hidden_size)
    for layer_idx in socket_layers:
        layer = model.model.layers[layer_idx]
        device = next(layer.self_attn.parameters()).device
        layer.self_attn = SVAResidualOutputAdapter(layer.self_attn, hidden_size, rank, scale).to(device)


def _adapter(model: nn.Module, layer_idx: int) -> SVAResidualOutputAdapter:
    attention = model.model.layers[layer_idx].self_attn
    if not isinstance(attention, SVAResidualOutputAdapter):
        raise TypeError(f"Layer {layer_idx} is not wrapped with SVAResidualOutputAdapter.")
    return attention


def collect_adapter_state(model: nn.Module, socket_layers: list[int]) -> dict[str, torch.Tensor]:
    """experiments/sva_late4_logit_distill.py:177-185."""

    state: dict[str, torch.Tensor] = {}
    for layer_idx in socket_layers:
        attention = _adapter(model, layer_idx)
        state[f"layers.{layer_idx}.down.weight"] = attention.down.weight.detach().cpu()
        state[f"layers.{layer_idx}.up.weight"] = attention.up.weight.detach().cpu()
    return state


def save_adapter_bundle(output_dir: Path | str, model: nn.Module, socket_layers: list[int],
                        manifest: dict[str, Any]) -> None:
    """The reference's bundle layout (experiments/sva_late4_logit_distill.py:188-221):
    adapter_config.json (``format``, ``socket_layers`` and the caller's
    fields) and adapter_weights.pt."""

    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    meta = {"format": ADAPTER_FORMAT, "socket_layers": list(socket_layers), **manifest}
    (output_dir / "adapter_config.json").write_text(json.dumps(meta, indent=2) + "\n", encoding="utf-8")
    torch.save({"state_dict": collect_adapter_state(model, socket_layers)}, output_dir / "adapter_weights.pt")


def load_adapter_bundle(adapter_dir: Path | str) -> tuple[dict[str, Any], dict[str, torch.Tensor]]:
    """experiments/sva_late4_logit_distill.py:224-230; the weights are read
    with weights_only=True (tensors only, nothing executed)."""

    adapter_dir = Path(adapter_dir)
    manifest = json.loads((adapter_dir / "adapter_config.json").read_text(encoding="utf-8"))
    payload = torch.load(adapter_dir / "adapter_weights.pt", map_location="cpu", weights_only=True)
    state_dict = payload.get("state_dict", payload) if isinstance(payload, dict) else payload
    if not isinstance(state_dict, dict):
        raise TypeError(f"Unexpected adapter weights payload in {adapter_dir}.")
    return manifest, state_dict


def load_adapter_weights(model: nn.Module, socket_layers: list[int], state_dict: dict[str, torch.Tensor]) -> None:
    """experiments/sva_late4_logit_distill.py:233-239."""

    with torch.no_grad():
        for layer_idx in socket_layers:
            attention = _adapter(model, layer_idx)
            attention.down.weight.copy_(state_dict[f"layers.{layer_idx}.down.weight"].to(attention.down.weight.device))
            attention.up.weight.copy_(state_dict[f"layers.{layer_idx}.up.weight"].to(attention.up.weight.device))
