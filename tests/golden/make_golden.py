"""Writes tests/golden/lookup8192_reference.npz: outputs of the reference
package's own functions on tests/cases.py:lookup8192_inputs().

Run once, in a container that holds the reference at /root/reference
(``python tests/golden/make_golden.py``).  Nothing on the GPU side runs this
file; the tests read only the .npz it writes.  The steps follow
sva/llama.py:211 (q_low), :615 (k_low on repeat_kv-expanded keys), sva/ops.py
(encode_product_keys, product_quantized_scores), sva/llama.py:276-317
(shortlist, rescore, budget, verifier) for one query token.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, "/root/reference")
sys.path.insert(1, str(ROOT))

from sva.ops import encode_product_keys, product_quantized_scores  # noqa: E402

from tests.cases import lookup8192_inputs  # noqa: E402


def main() -> None:
    torch.set_num_threads(1)
    inp = lookup8192_inputs()
    H, _, D = inp["q"].shape
    G = inp["keys"].shape[0]
    R = inp["q_proj"].shape[2]
    L, B = inp["shortlist"], inp["budget"]
    q = torch.from_numpy(inp["q"])[None]                                   # [1, H, 1, D]
    keys = torch.from_numpy(inp["keys"])[None].repeat_interleave(H // G, dim=1)    # repeat_kv
    values = torch.from_numpy(inp["values"])[None].repeat_interleave(H // G, dim=1)
    q_proj, k_proj = torch.from_numpy(inp["q_proj"]), torch.from_numpy(inp["k_proj"])
    scale = torch.from_numpy(inp["logit_scale"]).exp().clamp(0.01, 100.0)
    codebooks = torch.from_numpy(inp["codebooks"])
    S, C = codebooks.shape[1], codebooks.shape[2]
    sub = R // S
    with torch.no_grad():
        q_low = torch.einsum("bhtd,hdr->bhtr", q.float(), q_proj) * scale[None, :, None, None]
        k_low = torch.einsum("bhsd,hdr->bhsr", keys.float(), k_proj)
        codes = encode_product_keys(k_low[0], codebooks, 8192)
        lut = torch.stack([torch.stack([q_low[0, h, :, s * sub:(s + 1) * sub] @ codebooks[h, s].float().T
                                        for s in range(S)]) for h in range(H)])[:, :, 0]
        scores = product_quantized_scores(q_low[0], codebooks, codes, R)[None]   # [1, H, 1, N]
        top = scores.topk(L + 1, dim=-1)
        coarse_idx = top.indices[..., :L]
        low = torch.gather(k_low[:, :, None].expand(1, H, 1, -1, R), 3,
                           coarse_idx[..., None].expand(1, H, 1, L, R))
        rank = (low * q_low[..., None, :]).sum(dim=-1) / math.sqrt(R)
        rtop = rank.topk(B + 1, dim=-1)
        final = coarse_idx.gather(-1, rtop.indices[..., :B])
        sel_k = torch.gather(keys[:, :, None].expand(1, H, 1, -1, D), 3, final[..., None].expand(1, H, 1, B, D))
        sel_v = torch.gather(values[:, :, None].expand(1, H, 1, -1, D), 3, final[..., None].expand(1, H, 1, B, D))
        att = (sel_k * q[..., None, :]).sum(-1) * D ** -0.5
        w = torch.softmax(att, dim=-1, dtype=torch.float32)
        out = (w[..., None] * sel_v).sum(-2)
    np.savez_compressed(
        Path(__file__).with_name("lookup8192_reference.npz"),
        q_low=q_low[0, :, 0].numpy(),
        lut=lut.numpy(),
        k_low_head_sums=k_low[0].double().sum(dim=(1, 2)).numpy(),
        k_low_rows=k_low[0, :, :16].numpy(),
        codes=codes.numpy().astype(np.uint8),
        shortlist=np.sort(coarse_idx[0, :, 0].numpy(), axis=-1).astype(np.int16),
        shortlist_gap=(top.values[0, :, 0, L - 1] - top.values[0, :, 0, L]).numpy(),
        budget=np.sort(final[0, :, 0].numpy(), axis=-1).astype(np.int16),
        budget_gap=(rtop.values[0, :, 0, B - 1] - rtop.values[0, :, 0, B]).numpy(),
        out=out[0, :, 0].numpy(),
        torch_version=np.array(torch.__version__),
    )
    print("wrote", Path(__file__).with_name("lookup8192_reference.npz"))


if __name__ == "__main__":
    main()
