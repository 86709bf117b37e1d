"""The C-ABI library loads on the CPU host and exports exactly what include/splat_render.h declares."""

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
    assert lib.splat_abi_version() == 1


def test_workspace_queries_without_gpu():
    lib = _lib.load()
    assert lib.splat_bin_count_workspace_bytes(92160) >= 8 * (92160 // 256)
    # three pair-sized int32 arrays for C1's pair count plus histograms
    assert lib.splat_bin_pairs_workspace_bytes(92160, 9216, 1_836_494) >= 3 * 4 * 1_836_494
    assert lib.splat_pair_sums_bytes(1_836_494) == 48 * 1_836_494
    assert lib.splat_reduce_workspace_bytes(1_836_494) >= 2 * 40 * (1_836_494 // 64)


def test_invalid_arguments_are_reported_not_launched():
    lib = _lib.load()
    rc = lib.splat_render_fwd(None, None, None, 3, 64, 64, 8, 0, None, None, None, None, None, None, None, None, None)
    assert rc == 1
    assert b"null" in lib.splat_last_error()
    with pytest.raises(_lib.SplatError, match="invalid argument"):
        _lib.check(rc, "splat_render_fwd")
    assert lib.splat_bin_count(None, None, None, None, None, 9, 10, 8, 8, 8, 3.0, None, None, None, None, None, 0,
                               None) == 1


def test_host_rejects_cpu_tensors():
    import torch
    from gaussian_splat_encoder.render_hip import render_alpha_octave
    z = torch.zeros
    with pytest.raises(RuntimeError, match="device tensors"):
        render_alpha_octave(z(1, 4, 2), z(1, 4, 2), z(1, 4, 3), z(1, 4), z(1, 3), 16, 16)
