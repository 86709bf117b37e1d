"""The C-ABI library loads on the CPU host and exports exactly what include/splat_render.h declares."""

import ctypes
import os
import re

import pytest

from gaussian_splat_encoder import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "splat_render.h")


def declared():
    txt = open(HEADER).read()
    return set(re.findall(r"^(?:int|size_t|const char \*)\s*(splat_\w+)\(", txt, re.M))


def test_header_matches_binding_table():
    assert declared() == set(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.splat_abi_version() == 3


def test_workspace_queries_without_gpu():
    lib = _lib.load()
    assert lib.splat_bin_count_workspace_bytes(92160, 768, 768, 8, None) >= 8 * (92160 // 256)
    # the row plan (96 tile rows): three unit arrays, at most one unit per pair
    assert lib.splat_bin_pairs_workspace_bytes(92160, 768, 768, 8, None, 1_836_494) >= 3 * 4 * 1_836_494
    # and its histogram of 96 rows x 360 decode blocks in the count workspace
    assert lib.splat_bin_count_workspace_bytes(92160, 768, 768, 8, None) >= 8 * 96 * 360
    assert lib.splat_pair_sums_bytes(1_836_494) == 40 * 1_836_494


def test_invalid_arguments_are_reported_not_launched():
    lib = _lib.load()
    rc = lib.splat_render_fwd(None, None, None, 3, 64, 64, 8, 0, None, 0, 1, 1, None, None, None, None, None, None,
                              None, None, None)
    assert rc == 1
    assert b"null" in lib.splat_last_error()
    with pytest.raises(_lib.SplatError, match="invalid argument"):
        _lib.check(rc, "splat_render_fwd")
    assert lib.splat_bin_count(None, None, None, None, None, 9, 10, 8, 8, 8, 3.0, None, 0, None, None, None, None,
                               None, 0, None) == 1
    oct6 = ctypes.byref(_lib.SplatLevels(1, 6, 8.0, 0, 0, 0))
    # the composite renders level 0 only; FIELDS and UPS exclude each other; level range inside the table
    assert lib.splat_render_fwd(None, None, None, 3, 64, 64, 8, 0, oct6, 1, 2, 3, *[None] * 9) == 1
    assert b"level 0" in lib.splat_last_error()
    assert lib.splat_render_fwd(None, None, None, 3, 64, 64, 8, 5, oct6, 0, 1, 3, *[None] * 9) == 1
    assert b"exclude" in lib.splat_last_error()
    assert lib.splat_render_bwd(None, None, None, None, 0, 3, 64, 64, 8, 1, oct6, 1, 9, 3, *[None] * 11) == 1
    assert b"outside" in lib.splat_last_error()
    # octave 0 must be the native canvas
    assert lib.splat_levels_geometry(4, 64, 8, oct6, None, 0) < 0


def geometry(H, W, TILE, lv):
    from gaussian_splat_encoder.render_hip import levels_geometry
    return levels_geometry(H, W, TILE, lv)


def test_octave_levels_geometry():
    """Level o of an octave render is (max(8, H >> o), max(8, W >> o)) (render_triton.py:957), tiled by
    TILE; tile ids and packed pixel slots are concatenated level by level."""
    for H, W, TILE, mo in [(768, 768, 8, 6), (100, 37, 8, 3), (64, 512, 16, 6), (2048, 2048, 8, 6)]:
        geom, nt, npix = geometry(H, W, TILE, _lib.SplatLevels(1, mo, 8.0, 0, 0, 0))
        tb = pb = 0
        assert len(geom) == mo + 1
        for o, (h, w, ntx, tbase, pbase) in enumerate(geom):
            assert (h, w) == (max(8, H >> o), max(8, W >> o))
            assert ntx == -(-w // TILE) and tbase == tb and pbase == pb
            tb += ntx * -(-h // TILE)
            pb += h * w
        assert (nt, npix) == (tb, pb)


def test_octave_levels_merge_clamped_canvases():
    """Octaves past the first (8, 8) canvas render on the same canvas; they collapse into one level."""
    geom, _, _ = geometry(64, 64, 8, _lib.SplatLevels(1, 10, 8.0, 0, 0, 0))
    assert [g[:2] for g in geom] == [(64, 64), (32, 32), (16, 16), (8, 8)]
    geom, _, _ = geometry(8, 8, 8, _lib.SplatLevels(1, 6, 8.0, 0, 0, 0))
    assert [g[:2] for g in geom] == [(8, 8)]


def test_split_and_single_levels_geometry():
    geom, nt, npix = geometry(96, 80, 8, _lib.SplatLevels(2, 0, 0.0, 10, 12, 10))
    assert [g[:2] for g in geom] == [(96, 80), (12, 10)]
    assert nt == 12 * 10 + 2 * 2 and npix == 96 * 80 + 120
    geom, nt, npix = geometry(33, 17, 8, None)
    assert geom == [(33, 17, 3, 0, 0)] and nt == 15 and npix == 33 * 17


def test_upsample_adjoint_workspace():
    lib = _lib.load()
    lv = _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)
    # (2 + C) terms x H0 rows x the coarse levels' columns
    cols = sum(max(8, 768 >> o) for o in range(1, 7))
    assert lib.splat_upsample_adjoint_workspace_bytes(3, 768, 768, 8, ctypes.byref(lv)) >= 4 * 5 * 768 * cols


def test_host_rejects_cpu_tensors():
    import torch
    from gaussian_splat_encoder.render_hip import render_alpha_octave
    z = torch.zeros
    with pytest.raises(RuntimeError, match="device tensors"):
        render_alpha_octave(z(1, 4, 2), z(1, 4, 2), z(1, 4, 3), z(1, 4), z(1, 3), 16, 16)


def test_bin_rejects_unknown_flags():
    """splat_bin_count accepts only SPLAT_FLAG_LOG_SCALE, splat_bin also SPLAT_FLAG_DEFER; the check precedes any
    device work."""
    lib = _lib.load()
    for bad in (1, 8, 32, 16 | 2):
        assert lib.splat_bin_count(None, None, None, None, None, 3, 4, 16, 16, 8, 3.0, None, bad, None, None, None,
                                   None, None, 0, None) == 1
        assert b"unknown flags" in lib.splat_last_error()
    for bad in (1, 8, 64, 32 | 2):
        assert lib.splat_bin(None, None, None, None, None, 3, 4, 16, 16, 8, 3.0, None, bad, -1, None, None, None,
                             None, None, None, 0, 0, None, None, None, None, None, 0, None) == 1
        assert b"unknown flags" in lib.splat_last_error()


def test_deferred_read_needs_pair_buffers():
    """SPLAT_FLAG_DEFER without buffers for pair_cap > 0 pairs is refused before any device work (the pointers
    below are never dereferenced), and splat_bin_finish checks its arguments."""
    lib = _lib.load()
    fake = 256
    N, H, W = 4, 16, 16
    ws = lib.splat_bin_count_workspace_bytes(N, H, W, 8, None)
    assert lib.splat_bin(fake, fake, None, fake, fake, 3, N, H, W, 8, 3.0, None, _lib.FLAG_DEFER, -1, fake, fake,
                         fake, fake, fake, fake, ws, 0, None, None, None, None, None, 0, None) == 1
    assert b"deferred read" in lib.splat_last_error()
    for nlev, cap in ((0, 1), (_lib.MAX_LEVELS + 1, 1), (1, -1)):
        assert lib.splat_bin_finish(fake, fake, nlev, -1, cap, None) == 1
        assert b"splat_bin_finish" in lib.splat_last_error()


@pytest.mark.parametrize("H,W", [(1, 1), (7, 64), (64, 3)])
def test_octave_render_refuses_canvases_below_8(H, W):
    """render_alpha_octave refuses a canvas under 8 pixels a side before any device work (the reference's octave 0
    renders on a max(8, H) x max(8, W) canvas and fails adding it to the H x W field)."""
    import torch
    from gaussian_splat_encoder import render_hip as RH
    n = 4
    args = (torch.rand(1, n, 2), torch.zeros(1, n, 2), torch.rand(1, n, 3), torch.rand(1, n), torch.rand(1, 3))
    with pytest.raises(RuntimeError, match="H, W >= 8"):
        RH.render_alpha_octave(*args, H, W)
    # the level table itself is refused by the library too
    lv = _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)
    assert _lib.load().splat_levels_geometry(H, W, 8, ctypes.byref(lv), None, 0) < 0
