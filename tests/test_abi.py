"""The C ABI library loads on the host, exports every symbol that
include/drama_moe.h declares, and rejects bad geometry before any GPU work
(CPU only: no kernel is launched)."""
import ctypes
import re
from pathlib import Path

import pytest

from drama_moe import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "drama_moe.h").read_text()
    return sorted(set(re.findall(r"DMOE_API\s+[\w\s\*]+?\b(dmoe_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(names) == _lib.exported_symbols()


def test_abi_version_and_error_channel():
    lib = _lib.library()
    assert lib.dmoe_abi_version() == _lib.ABI_VERSION
    assert lib.dmoe_last_error() == b""


def _fake(ptr=0x100000):
    return ctypes.c_void_p(ptr)


@pytest.mark.parametrize("cols,group,message", [
    (100, 128, "whole 128-value groups"),
    (256, 64, "group must be 128"),
])
def test_quantize_validates_before_launch(cols, group, message):
    lib = _lib.library()
    status = lib.dmoe_fp8_quantize(_fake(), _lib.BF16, cols, 4, cols, group, _fake(), _fake(), None, None)
    assert status == -1
    assert message in lib.dmoe_last_error().decode()


def _bank(n13=256, k=256, n2=256, k2=128, scale_rows=None):
    p13 = _lib.Fp8Proj(0x10000, 0x20000, n13 * k, k, (n13 // 128) * (k // 128), k // 128, 1,
                       scale_rows or n13 // 128, k // 128, n13, k)
    p2 = _lib.Fp8Proj(0x30000, 0x40000, n2 * k2, k2, (n2 // 128) * (k2 // 128), k2 // 128, 1,
                      n2 // 128, k2 // 128, n2, k2)
    return _lib.Fp8Bank(p13, p2, 4)


def _forward(bank, tokens=1, top_k=2, ws_bytes=1 << 30):
    lib = _lib.library()
    return lib.dmoe_fp8_moe_forward(ctypes.byref(bank), _fake(), _lib.BF16, bank.w13.k, tokens, _fake(),
                                    _lib.I64, _fake(), _lib.F32, top_k, 128, _lib.BF16, _fake(),
                                    _lib.BF16, bank.w13.k, _fake(0x1000000), ws_bytes, None, None)


@pytest.mark.parametrize("bank,message", [
    (_bank(k=200), "multiple of 128"),
    (_bank(n2=384), "w2 must be"),
    (_bank(scale_rows=3), "scale rows"),
])
def test_forward_rejects_bad_bank_geometry(bank, message):
    assert _forward(bank) == -1
    assert message in _lib.library().dmoe_last_error().decode()


def test_forward_rejects_small_workspace_and_oversized_calls():
    assert _forward(_bank(), ws_bytes=16) == -1
    assert "workspace too small" in _lib.library().dmoe_last_error().decode()
    assert _forward(_bank(), tokens=200, top_k=2, ws_bytes=16) == -1  # grouped path: its own workspace
    assert "workspace too small" in _lib.library().dmoe_last_error().decode()
    assert _forward(_bank(), tokens=600000, top_k=2) == -1
    assert "1048576 route pairs" in _lib.library().dmoe_last_error().decode()
    # tokens * top_k = 2^32 + 64 would wrap to 64 pairs in 32-bit arithmetic
    wide = _bank()
    wide.experts = 64
    assert _forward(wide, tokens=(1 << 26) + 1, top_k=64) == -1
    assert "1048576 route pairs" in _lib.library().dmoe_last_error().decode()


def test_workspace_query_grows_with_pairs():
    lib = _lib.library()
    bank = _bank()
    small = lib.dmoe_fp8_workspace_bytes(ctypes.byref(bank), 8)
    large = lib.dmoe_fp8_workspace_bytes(ctypes.byref(bank), 64)
    grouped = lib.dmoe_fp8_workspace_bytes(ctypes.byref(bank), 4096)
    assert 0 < small < large < grouped
    # the grouped workspace holds at least the fp32 partials of every pair
    assert grouped >= 4096 * bank.w13.k * 4
    assert lib.dmoe_fp8_workspace_bytes(ctypes.byref(bank), (1 << 20) + 1) == 0


def test_route_and_permute_validate_geometry():
    lib = _lib.library()
    assert lib.dmoe_route_topk(_fake(), 128, 4, 128, 0, 1, _fake(), _fake(), _lib.BF16, None) == -1
    assert "top_k" in lib.dmoe_last_error().decode()
    assert lib.dmoe_permute(_fake(), _lib.I64, 2_000_000, 128, _fake(), _fake(), _fake(), _fake(), 1 << 30,
                            None, None) == -1
    assert "pair count" in lib.dmoe_last_error().decode()
    need = lib.dmoe_permute_workspace_bytes(20000, 128)
    assert need >= 20000 * 4 + 79 * 128 * 4
    assert lib.dmoe_permute(_fake(), _lib.I64, 20000, 128, _fake(), _fake(), _fake(), _fake(), need - 4,
                            None, None) == -1
    assert "workspace too small" in lib.dmoe_last_error().decode()


def test_stream_read_validates_before_launch():
    lib = _lib.library()
    assert lib.dmoe_stream_read(_fake(), 100, _fake(), None) == -1
    assert "multiple of 16" in lib.dmoe_last_error().decode()
    assert lib.dmoe_stream_read(_fake(0x100008), 1024, _fake(), None) == -1
    assert "aligned" in lib.dmoe_last_error().decode()
    assert lib.dmoe_stream_read(_fake(), 1024, None, None) == -1
