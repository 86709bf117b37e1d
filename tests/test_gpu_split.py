"""Split launches of the coarse levels (splat_render_fields_split / _bwd): every tile of a coarse level is split
into chunks of its pair list, one workgroup each, and the forward's partial fields are added in chunk order.

* against the unsplit FIELDS kernels (splat_render_fwd / splat_render_bwd with FLAG_FIELDS) on the same pair
  list (sums of up to a few thousand fp32 terms in another grouping): fields and per-pair sums within 1e-5 of
  their largest magnitude (per field, per record column);
* splits of 1, uneven and larger than the pair lists (empty chunks), TILE 4 / 8 / 16;
* argument checks (splits outside [1, 1024], workspace too small).
The end-to-end octave parity of the split path is covered by test_gpu_levels.py (composed oracle).
"""

import ctypes

import numpy as np
import pytest
import torch

from _gpu_util import RH, activate_scale, random_scene
from gaussian_splat_encoder import _lib

pytestmark = pytest.mark.gpu


def octave_lv():
    return _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)


def scene_bins(dev, H, W, TILE, n=2500, px=24.0, seed=31):
    mu, ls, col, op, bg, th = random_scene(n, H, W, seed=seed, dev=dev, ls_mean_px=px, ls_std=0.3, op_max=0.7)
    sc = activate_scale(ls)
    bins = RH._bin(mu, sc, col, op, th, H, W, TILE, 3.0, lv=octave_lv())
    return bins, col.shape[-1]


def splits_of(L, pattern):
    arr = (ctypes.c_int * L)()
    for l in range(L):
        arr[l] = pattern(l)
    return arr


def run_split_fwd(lib, bins, C, flags, mask, sp, dev):
    npix = bins.npix
    fl = (torch.zeros(npix, device=dev), torch.zeros(npix, device=dev), torch.zeros(npix, C, device=dev))
    L = bins.n_levels
    lvr = ctypes.byref(bins.lv)
    nb = lib.splat_fields_split_workspace_bytes(C, bins.H, bins.W, bins.TILE, lvr, 1, L, mask, sp)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
    _lib.check(lib.splat_render_fields_split(bins.p(0, "rec"), bins.p(0, "gid"), bins.p(0, "starts"), C, bins.H,
                                             bins.W, bins.TILE, flags, lvr, 1, L, mask, sp, *[t.data_ptr() for t in fl],
                                             ws.data_ptr(), nb, _lib.stream_ptr(dev)), "splat_render_fields_split")
    return fl


def run_plain_fwd(lib, bins, C, flags, mask, dev):
    npix = bins.npix
    fl = (torch.zeros(npix, device=dev), torch.zeros(npix, device=dev), torch.zeros(npix, C, device=dev))
    RH._render_fwd(lib, bins, 0, C, RH.FLAG_FIELDS | flags, (1, bins.n_levels), mask, (None,) * 5, fl,
                   _lib.stream_ptr(dev))
    return fl


def upstream(bins, C, dev, seed):
    g = torch.Generator().manual_seed(seed)
    npix = bins.npix
    return (torch.randn(npix, generator=g).to(dev), torch.randn(npix, generator=g).to(dev),
            torch.randn(npix, C, generator=g).to(dev))


def pair_sums(lib, bins, C, dev, fill):
    n = lib.splat_pair_sums_bytes(bins.tot_b[0]) // 4
    return torch.full((n,), fill, device=dev)


def close(a, b, tol):
    a, b = a.double().cpu(), b.double().cpu()
    return (a - b).abs().max().item() <= tol * max(b.abs().max().item(), 1e-30)


@pytest.mark.parametrize("TILE", [4, 8, 16])
@pytest.mark.parametrize("odds", [False, True])
def test_split_matches_unsplit(dev, TILE, odds):
    H = W = 192
    bins, C = scene_bins(dev, H, W, TILE)
    lib = _lib.load()
    L = bins.n_levels
    mask = bins.level_mask(0) & ~1
    assert mask, "the scene must hold coarse levels"
    flags = RH.FLAG_ODDS if odds else 0
    ref = run_plain_fwd(lib, bins, C, flags, mask, dev)
    dS = upstream(bins, C, dev, seed=TILE)
    lvr = ctypes.byref(bins.lv)
    R = 6 + C
    ps_ref = pair_sums(lib, bins, C, dev, float("nan"))
    RH._render_bwd(lib, bins, 0, C, RH.FLAG_FIELDS | flags, (1, L), mask, (None,) * 5 + dS, ps_ref, None,
                   _lib.stream_ptr(dev))
    patterns = [lambda l: 1, lambda l: 3, lambda l: 1 + (5 * l) % 9, lambda l: 1024]
    for pat in patterns:
        sp = splits_of(L, pat)
        got = run_split_fwd(lib, bins, C, flags, mask, sp, dev)
        torch.cuda.synchronize()
        for a, b in zip(got, ref):
            assert close(a, b, 1e-5), f"fields differ (splits {list(sp)})"
        ps = pair_sums(lib, bins, C, dev, float("nan"))
        _lib.check(lib.splat_render_fields_split_bwd(bins.p(0, "rec"), bins.p(0, "gid"), bins.p(0, "starts"),
                                                     bins.p(0, "pq"), bins.tot_b[0], C, H, W, TILE, flags, lvr, 1, L,
                                                     mask, sp, *[t.data_ptr() for t in dS], ps.data_ptr(),
                                                     _lib.stream_ptr(dev)), "splat_render_fields_split_bwd")
        torch.cuda.synchronize()
        # every pair of the coarse levels gets a record (level-0 pairs are not part of these launches)
        lev = bins.rect_b[0][:, 3].long()
        off = bins.off_b[0].long()
        cnt = off[1:] - off[:-1]
        coarse_q = torch.repeat_interleave(lev > 0, cnt)
        a = ps[:bins.tot_b[0] * R].view(-1, R)[coarse_q]
        b = ps_ref[:bins.tot_b[0] * R].view(-1, R)[coarse_q]
        assert not torch.isnan(a).any(), "a coarse pair has no record"
        for k in range(R):
            assert close(a[:, k], b[:, k], 1e-5), f"pair sums column {k} differ (splits {list(sp)})"


def test_split_argument_checks(dev):
    bins, C = scene_bins(dev, 128, 128, 8, n=600)
    lib = _lib.load()
    L = bins.n_levels
    mask = bins.level_mask(0) & ~1
    lvr = ctypes.byref(bins.lv)
    fl = [torch.zeros(bins.npix * k, device=dev) for k in (1, 1, C)]
    for bad in (0, 1025):
        sp = splits_of(L, lambda l: bad)
        assert lib.splat_fields_split_workspace_bytes(C, 128, 128, 8, lvr, 1, L, mask, sp) == 0
        rc = lib.splat_render_fields_split(bins.p(0, "rec"), bins.p(0, "gid"), bins.p(0, "starts"), C, 128, 128, 8,
                                           0, lvr, 1, L, mask, sp, *[t.data_ptr() for t in fl], None, 0,
                                           _lib.stream_ptr(dev))
        assert rc == 1 and b"splits" in lib.splat_last_error()
    sp = splits_of(L, lambda l: 4)
    nb = lib.splat_fields_split_workspace_bytes(C, 128, 128, 8, lvr, 1, L, mask, sp)
    assert nb > 0
    rc = lib.splat_render_fields_split(bins.p(0, "rec"), bins.p(0, "gid"), bins.p(0, "starts"), C, 128, 128, 8, 0,
                                       lvr, 1, L, mask, sp, *[t.data_ptr() for t in fl], None, nb - 1,
                                       _lib.stream_ptr(dev))
    assert rc == _lib.STATUS_WORKSPACE
    sp1 = splits_of(L, lambda l: 1)
    assert lib.splat_fields_split_workspace_bytes(C, 128, 128, 8, lvr, 1, L, mask, sp1) == 0
    assert lib.splat_render_fields_split(bins.p(0, "rec"), bins.p(0, "gid"), bins.p(0, "starts"), C, 128, 128, 8,
                                         RH.FLAG_FIELDS, lvr, 1, L, mask, sp1, *[t.data_ptr() for t in fl], None, 0,
                                         _lib.stream_ptr(dev)) == 1
