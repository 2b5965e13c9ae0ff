"""The C-ABI library loads and exports every symbol include/*.h declares;
argument validation runs on the host (no GPU needed)."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"^\s*(?:int|size_t|void)\s+(ds4hip_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "ds4hip_flash_attn_decode_fp8" in syms
    assert "ds4hip_fp8_kv_quantize_round_trip_f32" in syms


def test_library_exports_every_declared_symbol():
    from ds4cuda_amd import lib
    from ds4cuda_amd._lib import SIGNATURES
    l = lib()
    for name in declared_symbols():
        assert hasattr(l, name), name
        assert name in SIGNATURES, f"{name} missing from the ctypes signature table"


def test_shape_validation_returns_einval():
    from ds4cuda_amd import lib
    l = lib()
    assert l.ds4hip_fp8_kv_quantize_round_trip_f32(None, None, 1, 500, 64, None) == -22
    assert l.ds4hip_fp8_kv_quantize_round_trip_f32(None, None, 1, 512, 60, None) == -22
    assert l.ds4hip_fp8_kv_quantize_round_trip_f32(None, None, 0, 512, 64, None) == 0
    assert l.ds4hip_flash_attn_decode_raw_f32(None, None, None, None, None, 32, 4, 512, None) == -22
    assert l.ds4hip_flash_attn_decode_raw_f32(None, None, None, None, None, 64, 4, 256, None) == -22
    assert l.ds4hip_flash_attn_decode_mixed_f32(None, None, None, None, None, None, 64, -1, 0, 512,
                                                None) == -22
    assert l.ds4hip_get_last_error() == -22


def test_workspace_size_is_positive():
    from ds4cuda_amd.ops import decode_fp8_workspace_bytes
    assert decode_fp8_workspace_bytes([32768] * 43) > 0
    assert decode_fp8_workspace_bytes([0, 5, 0]) > 0
