"""sva_stream_read, the plain read the scan is priced against: every word of
the buffer is read once (the XOR of the sink is the XOR of the buffer's
32-bit words) for sizes that end inside a wave's span and inside a load, and
bad arguments raise."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096, 8192 * 4 + 48, 37748736])
def test_stream_read_folds_every_word(device, nbytes):
    from sva_amd import kernels

    g = torch.Generator(device=device).manual_seed(nbytes)
    buf = torch.randint(0, 256, (nbytes,), device=device, dtype=torch.uint8, generator=g)
    sink = kernels.stream_read(buf)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(buf.cpu().numpy().view(np.uint32))
    assert got == want


def test_stream_read_rejects_bad_buffers(device):
    from sva_amd import kernels

    with pytest.raises(RuntimeError):
        kernels.stream_read(torch.zeros(24, device=device, dtype=torch.uint8))  # not a multiple of 16
    buf = torch.zeros(64, device=device, dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        kernels.stream_read(buf[4:36])  # not 16-byte aligned
    with pytest.raises(ValueError):
        kernels.stream_read(buf, torch.zeros(1, device=device, dtype=torch.float32))
