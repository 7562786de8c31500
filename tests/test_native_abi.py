"""The C-ABI library loads (no GPU needed) and exports every entry point
include/gm_hip.h declares; the shim's signatures cover exactly those."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared() -> set[str]:
    text = (ROOT / "include" / "gm_hip.h").read_text()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(gm_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_entry_points():
    names = declared()
    assert {"gm_last_error", "gm_abi_version", "gm_softmax_forward_f32", "gm_softmax_backward_f64",
            "gm_conv_forward_f32", "gm_conv_backward_f64"} <= names


def test_library_exports_every_declared_symbol():
    from gm_attention_amd import _native

    if not _native.LIB_PATH.exists():
        pytest.fail("libgmhip.so is not built (run gm-attention_amd/build.py)")
    lib = _native.library()
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.gm_abi_version() == 1
    for stem in _native.SIGNATURES:
        assert stem + "_f32" in declared() and stem + "_f64" in declared()
    undeclared = sorted(set(_native.SIGNATURES_F32) - declared())
    assert not undeclared, undeclared


def test_errors_are_reported_not_raised_through_the_abi():
    """A bad descriptor is rejected before any launch (no GPU touched)."""
    import ctypes

    from gm_attention_amd import _native

    lib = _native.library()
    desc = (ctypes.c_int64 * 5)(3, 1, 0, 0, 2)  # frequency 3 with a 2-order table
    status = lib.gm_softmax_forward_f32(None, None, None, None, None, ctypes.cast(desc, ctypes.c_void_p), None, None,
                                        4, 0, 2, 2, 1, 1, 1.0, 1, None, None)
    assert status == 1
    assert b"exceeds the phase tables" in lib.gm_last_error()
