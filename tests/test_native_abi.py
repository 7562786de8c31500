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
    assert lib.gm_abi_version() == 3
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


def _xcd_map(nb, kind, ptr=None, per=1):
    import ctypes

    import torch

    from gm_attention_amd import _native

    lib = _native.library()
    out = (ctypes.c_int64 * nb)()
    if ptr is not None:
        ptr = ptr.contiguous()
        status = lib.gm_xcd_block_map(ctypes.c_int64(nb), kind, ctypes.c_void_p(ptr.data_ptr()),
                                      ctypes.c_int64(ptr.shape[0] - 1), per, out)
    else:
        status = lib.gm_xcd_block_map(ctypes.c_int64(nb), kind, None, ctypes.c_int64(0), per, out)
    assert status == 0, lib.gm_last_error()
    return torch.tensor(list(out), dtype=torch.int64)


@pytest.mark.parametrize("kind", [0, 1])
def test_xcd_assignments_are_permutations_of_the_blocks(kind):
    """Every hardware block runs exactly one logical block, for every grid size."""
    import torch

    for nb in range(1, 3001):
        m = _xcd_map(nb, kind)
        assert torch.equal(torch.sort(m).values, torch.arange(nb)), (kind, nb)


def test_spread_assignment_gives_every_xcd_every_band():
    """Chunks dealt round-robin: with 2 * 256 blocks each XCD (b % 8) runs two
    32-block chunks 256 apart; below 256 blocks the chunks shrink (96 blocks:
    chunks of 3) and every XCD still gets one chunk from each quarter."""
    m = _xcd_map(512, 1)
    for x in range(8):
        mine = sorted(int(v) for v in m[x::8])
        assert mine == list(range(32 * x, 32 * x + 32)) + list(range(256 + 32 * x, 256 + 32 * x + 32))
    m = _xcd_map(96, 1)
    for x in range(8):
        mine = sorted(int(v) for v in m[x::8])
        assert mine == [3 * x + j + 24 * r for r in range(4) for j in range(3)]


def test_balanced_assignment_picks_chunks_only_for_uneven_eighths():
    """Two 24x48 samples: the contiguous eighths hold 36000 and 9600 edges
    (polar and equatorial quarters), so the softmax's map (one target per
    wave, four a block) deals chunks; four samples put a pole and an equator
    in each eighth (hemispheres), so it keeps the contiguous ranges."""
    import torch

    import problems

    disc = problems.discretization(24, 48)
    for batch, spread in ((2, True), (4, False)):
        ptr = disc.edge_geometry.tile(batch, n_sources=disc.n_nodes).row_ptr
        n = ptr.shape[0] - 1
        nb = (n + 3) // 4
        got = _xcd_map(nb, 2, ptr, 4)
        want = _xcd_map(nb, 1 if spread else 0)
        assert torch.equal(got, want), batch
        assert torch.equal(torch.sort(got).values, torch.arange(nb))
