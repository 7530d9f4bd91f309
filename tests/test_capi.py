"""The C-ABI library without a GPU: it loads, exports every entry point that
include/sva_hip.h declares, its host-only queries answer, and argument
validation fails with a message before any device work."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (the library binds to the HIP runtime torch maps)

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> list[str]:
    text = (ROOT / "include" / "sva_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sva_[a-z0-9_]+)\s*\(", text)))


def _lib():
    from sva_amd import _lib

    return _lib.lib()


def test_library_exports_every_declared_symbol():
    names = _declared()
    assert len(names) >= 10
    lib = _lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    from sva_amd import _lib as binding

    assert set(binding.exported_symbols()) == set(names), "ctypes signatures out of step with the header"


def test_abi_version_and_workspace_queries():
    lib = _lib()
    assert lib.sva_abi_version() == 1
    # the long-context q=1 path needs candidate lists; short caches need none
    big = lib.sva_summon_workspace_bytes(1, 9, 1, 1 << 20, 2048)
    assert big >= 9 * (1 << 20) * 8
    assert lib.sva_summon_workspace_bytes(1, 9, 1, 8192, 2048) <= 4096
    assert lib.sva_verify_workspace_bytes(1, 9, 3, 1, 64, 512) > 0


def test_summon_strategy_selection():
    lib = _lib()
    # 1M keys, q = 1, 4x64 codes: many workgroups per item
    assert lib.sva_summon_strategy(1, 9, 1, 1 << 20, 64, 4, 64, 2048, 0, 0) == 1
    # one subspace of <= 256 codewords: the shortlist by code class
    assert lib.sva_summon_strategy(1, 9, 1, 1 << 20, 64, 1, 256, 2048, 0, 0) == 2
    # short caches and prefill up to 16384 keys: one workgroup per item, shortlist in registers
    assert lib.sva_summon_strategy(1, 9, 1, 8192, 64, 2, 256, 2048, 0, 0) == 3
    assert lib.sva_summon_strategy(1, 9, 4096, 8192, 64, 2, 256, 2048, 0, 0) == 3
    # longer prefill, q = 1 between the two, wide codes, a long shortlist: one workgroup per item
    assert lib.sva_summon_strategy(1, 9, 16, 1 << 20, 64, 4, 64, 2048, 0, 0) == 0
    assert lib.sva_summon_strategy(1, 9, 1, 20000, 64, 2, 256, 2048, 0, 0) == 0
    assert lib.sva_summon_strategy(1, 9, 1, 1 << 20, 64, 4, 64, 2048, 3, 0) == 0  # int64 codes
    assert lib.sva_summon_strategy(1, 9, 1, 8192, 64, 2, 256, 4096, 0, 0) == 0


def test_summon_select_without_shortlist_outside_the_fused_path():
    lib = _lib()
    p = ctypes.c_void_p(256)  # never dereferenced: the arguments are refused first
    # 1M keys, q = 1: the wide path keeps the shortlist in memory
    rc = lib.sva_summon_select(p, p, p, p, 0, 0, p, 0, None, None, 1, 9, 1, 1 << 20, 64, 4, 64, 2048, None, 0, 0,
                               None, None, p, 512, p, p, p, 1 << 30, None)
    assert rc == 3  # SVA_ERR_UNSUPPORTED
    assert "shortlist" in lib.sva_last_error().decode()
    # one of the pair
    rc = lib.sva_summon_select(p, p, p, p, 0, 0, p, 0, None, None, 1, 9, 4, 8192, 64, 2, 256, 2048, None, 0, 0,
                               p, None, p, 512, p, p, p, 1 << 30, None)
    assert rc == 1


@pytest.mark.parametrize("call", ["query_lut", "summon", "summon_select", "budget", "verify"])
def test_null_pointers_are_rejected_with_a_message(call):
    lib = _lib()
    if call == "query_lut":
        rc = lib.sva_query_lut(None, 0, 0, 0, 0, 1, 9, 1, 64, 64, 2, 256, None, None, None, None, 0, 0, 0, 0, None,
                               None, None, None)
    elif call == "summon":
        rc = lib.sva_summon(None, None, None, None, 0, 0, None, 0, None, None, 1, 9, 1, 100, 64, 2, 256, 16, None, 0,
                            0, None, None, None, None, 0, None)
    elif call == "summon_select":
        rc = lib.sva_summon_select(None, None, None, None, 0, 0, None, 0, None, None, 1, 9, 1, 100, 64, 2, 256, 16,
                                   None, 0, 0, None, None, None, 4, None, None, None, 0, None)
    elif call == "budget":
        rc = lib.sva_budget_select(None, None, None, 9, 16, 4, None, None, None)
    else:
        rc = lib.sva_verify(None, 0, 0, 0, 0, None, None, 0, 0, 0, None, None, 100, None, None, 1, 9, 3, 1, 64, 4,
                            ctypes.c_float(0.125), None, 0, 0, 0, 0, None, 0, None)
    assert rc == 1  # SVA_INVALID_ARGUMENT
    msg = lib.sva_last_error().decode()
    assert "null" in msg or "pointer" in msg, msg


def test_summon_select_rejects_bad_budget():
    lib = _lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the arguments are refused first
    for B in (0, 8193):
        rc = lib.sva_summon_select(p, p, p, p, 0, 0, p, 0, None, None, 1, 9, 1, 100, 64, 2, 256, 16, None, 0, 0, p, p,
                                   p, B, p, p, p, 1 << 20, None)
        assert rc == 1
        assert "budget" in lib.sva_last_error().decode()


def test_device_tensors_are_required():
    from sva_amd import kernels

    with pytest.raises(Exception, match="(?i)cpu|device|rocm|gpu"):
        kernels.query_lut(torch.zeros(1, 9, 1, 64), torch.zeros(9, 64, 64), torch.ones(9), torch.zeros(9, 2, 256, 32))
