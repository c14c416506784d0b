"""The C-ABI library loads and exports every entry point include/focr_hip.h
declares (CPU only: no compute calls without a GPU)."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared() -> list[str]:
    text = (ROOT / "include" / "focr_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(focr_hip_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared()
    for must in ("focr_hip_igemm_s8s8", "focr_hip_igemm_u8s8", "focr_hip_igemm_s4s8_packed",
                 "focr_hip_lm_head_i8", "focr_hip_moe_decode", "focr_hip_rswa_decode_attention",
                 "focr_hip_selftest", "focr_hip_tier"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from franken_ocr_amd import _abi

    lib = _abi.lib()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    from franken_ocr_amd import _abi

    assert sorted(_abi.exported_symbols()) == _declared()


def test_tier_reflection_without_device():
    from franken_ocr_amd import simd

    t = simd.detected_tier()
    assert t.tag == "gfx950" and t.feature == "gfx950+mfma-i8"
    assert simd.tier_string() == "gfx950+mfma-i8"


def test_no_device_fails_loudly(monkeypatch):
    """Without a GPU the product path raises; there is no CPU fallback."""
    from franken_ocr_amd import _abi
    from franken_ocr_amd.device import device_count, Context

    if device_count() > 0:
        pytest.skip("a device is visible here")
    with pytest.raises(_abi.NoDevice):
        Context(0)


def test_null_context_is_bad_handle():
    from franken_ocr_amd import _abi

    lib = _abi.lib()
    st = lib.focr_hip_igemm_s8s8(None, None, 0, None, 0, 0, 0, 0, None, 0)
    assert st == _abi.E_BAD_HANDLE
    assert "null focr_hip_ctx" in _abi.last_error()


def test_version_string():
    from franken_ocr_amd import _abi

    assert b"gfx950" in _abi.lib().focr_hip_version()
