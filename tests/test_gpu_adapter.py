"""GPU parity of the fused residual output adapter (sva_residual_adapter)
against the float64 oracle of experiments/sva_late4_logit_distill.py:47-51:
within 1e-5 of the output's magnitude for fp32 activations, 2e-2 for bf16
(the correction is cast to the attention dtype before the residual add, as
the reference does); token counts that do not fill a workgroup; the module
wrapper end to end; inference only."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H,rank,dtype", [(1, 576, 16, torch.float32), (37, 576, 16, torch.float32),
                                            (8, 576, 16, torch.bfloat16), (1000, 64, 5, torch.bfloat16),
                                            (3, 2048, 64, torch.float32)])
def test_residual_adapter_matches_oracle(device, T, H, rank, dtype):
    from sva_amd import kernels

    rng = np.random.default_rng(T + H + rank)
    hidden = rng.standard_normal((T, H)).astype(np.float32)
    attn = rng.standard_normal((T, H)).astype(np.float32)
    down = (rng.standard_normal((rank, 2 * H)) * 0.02).astype(np.float32)
    up = (rng.standard_normal((H, rank)) * 0.5).astype(np.float32)
    h = torch.from_numpy(hidden).to(device, dtype)
    a = torch.from_numpy(attn).to(device, dtype)
    out = kernels.residual_adapter(h, a, torch.from_numpy(down).to(device), torch.from_numpy(up).to(device), 0.75)
    assert out.dtype == dtype and out.shape == a.shape
    ref = oracle.residual_adapter(h.float().cpu().numpy(), a.float().cpu().numpy(), down, up, 0.75)
    got = out.float().cpu().numpy()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= tol, f"rel err {err}"


class _Fixed(nn.Module):
    def __init__(self, out):
        super().__init__()
        self.out = out

    def forward(self, hidden_states, *args, **kwargs):
        return self.out, None


def test_adapter_module_wraps_attention(device):
    from sva_amd.adapter import SVAResidualOutputAdapter

    rng = np.random.default_rng(2)
    hidden = torch.from_numpy(rng.standard_normal((1, 5, 576)).astype(np.float32)).to(device, torch.bfloat16)
    attn = torch.from_numpy(rng.standard_normal((1, 5, 576)).astype(np.float32)).to(device, torch.bfloat16)
    mod = SVAResidualOutputAdapter(_Fixed(attn), 576, 16, 1.0).to(device)
    with torch.no_grad():
        out, weights = mod(hidden)
        assert weights is None
        assert torch.equal(out, attn)  # zero-initialised up projection
        mod.up.weight.normal_(std=0.5)
        out, _ = mod(hidden)
    ref = oracle.residual_adapter(hidden[0].float().cpu().numpy(), attn[0].float().cpu().numpy(),
                                  mod.down.weight.detach().cpu().numpy(), mod.up.weight.detach().cpu().numpy(), 1.0)
    err = np.abs(out[0].float().cpu().numpy() - ref).max() / np.abs(ref).max()
    assert err <= 2e-2
    with pytest.raises(RuntimeError, match="inference only"):
        mod(hidden)  # gradients enabled and trainable weights
