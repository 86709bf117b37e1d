"""Bit-exact binning on the GPU: the device pair list and tile starts equal the oracle's
(render_triton.py:351-409) for the benchmark configurations and for edge cases."""

import numpy as np
import pytest
import torch

from _gpu_util import RH, activate_scale, device_bins, np_, random_scene
from gaussian_splat_encoder import synth
from oracle import c_oracle

pytestmark = pytest.mark.gpu


def check_equal(mu, sc, H, W, TILE, cutoff):
    gid_d, st_d = device_bins(mu, sc, H, W, TILE, cutoff)
    for b in range(mu.shape[0]):
        gid_o, st_o = c_oracle.build_tiles(np_(mu[b]), np_(sc[b]), H, W, TILE, cutoff)
        assert np.array_equal(st_d[b], st_o), f"tile_starts differ (batch {b})"
        assert np.array_equal(gid_d[b], gid_o), f"gid_sorted differs (batch {b}, tot {st_o[-1]})"


@pytest.mark.parametrize("name,TILE", [("c0", 8), ("c1", 8), ("c1", 4), ("c1", 16), ("c4", 8)])
def test_configs_bit_exact(dev, name, TILE):
    s = synth.config(name)
    mu = s.mu.to(dev)
    sc = activate_scale(s.log_scale.to(dev))
    check_equal(mu, sc, s.H, s.W, TILE, 3.0)


@pytest.mark.parametrize("H,W,TILE,cutoff,n,margin", [
    (37, 51, 8, 3.0, 300, 0.3),        # ragged canvas, splats off canvas (clamped to edge tiles)
    (37, 51, 4, 5.0, 300, 0.0),
    (100, 60, 16, 3.0, 2000, 0.1),
    (8, 8, 8, 3.0, 50, 0.5),           # a single tile: no radix pass
    (2100, 2100, 8, 3.0, 20000, 0.0),  # 69,169 tiles: 17-bit keys, two 9-bit radix passes
    (1000, 700, 8, 3.0, 20000, 0.05),  # 11,000 tiles: two-phase sort on a ragged super-tile range
    (6000, 100, 8, 3.0, 20000, 0.0),   # 9,750 tiles: two-phase sort, super-tiles spanning several tile rows
    (8400, 40, 8, 3.0, 6000, 0.0),     # 1,050 tile rows: past the row plan's 1,024, the pair-sort plans
    (4200, 24, 4, 3.0, 6000, 0.1),     # 1,050 tile rows of 6 tiles
])
def test_edge_cases_bit_exact(dev, H, W, TILE, cutoff, n, margin):
    mu, ls, *_ = random_scene(n, H, W, seed=H + W + n, dev=dev, margin=margin, B=2)
    check_equal(mu, activate_scale(ls), H, W, TILE, cutoff)


@pytest.mark.parametrize("H,W,TILE,n,spread", [
    (256, 256, 8, 12000, 0.02),    # 1,024 tiles (super-tiles of 2): ~12k pairs per super-tile, two rounds
    (1024, 1024, 8, 8000, 0.01),   # 16,384 tiles (super-tiles of 32): a few dense super-tiles
    (64, 64, 2, 9000, 0.0),        # 1,024 tiles and ~9.2M pairs: past the two-phase limit, LSD passes
])
def test_dense_super_tiles_bit_exact(dev, H, W, TILE, n, spread):
    """Two-phase sort with super-tiles of more than one round (8,192 pairs) of the local sort, and the
    fallback to LSD passes when super-tiles would average more than 16,384 pairs."""
    g = torch.Generator().manual_seed(H + n)
    mu = (0.5 + spread * torch.randn(1, n, 2, generator=g)).clamp(0.0, 1.0)
    big = TILE == 2   # splats that cover the whole canvas
    ls = torch.full((1, n, 2), float(np.log(0.4 if big else 3.0 / H))) + 0.1 * torch.randn(1, n, 2, generator=g)
    check_equal(mu.to(dev), activate_scale(ls.to(dev)), H, W, TILE, 3.0)


def test_near_tile_edges_not_fma_contracted(dev):
    """Centres placed within one ulp of `tile edge + radius`, where a fused multiply-subtract floors
    differently from the reference's separately rounded ops."""
    rng = np.random.default_rng(3)
    H = W = 768
    n = 20000
    tx = rng.integers(1, 95, n)
    sx = rng.uniform(0.001, 0.01, n).astype(np.float32)
    rx = (np.float32(3.0) * sx).astype(np.float32) * np.float32(W)
    mx = ((tx * 8 + rx) / W).astype(np.float32)
    mx = np.nextafter(mx, np.where(rng.random(n) < 0.5, -np.inf, np.inf).astype(np.float32))
    my = rng.random(n).astype(np.float32)
    mu = torch.from_numpy(np.stack([my, mx], -1))[None].to(dev)
    sc = torch.from_numpy(np.stack([sx * np.float32(0.7), sx], -1))[None].to(dev)
    check_equal(mu, sc, H, W, 8, 3.0)


def test_empty_and_single(dev):
    z = torch.zeros(1, 0, 2, device=dev)
    gid_b, st_b, ntx, nt = RH._build_tiles(z, z, 32, 32, 8, 3.0)
    assert gid_b[0].tolist() == [0] and st_b[0].tolist() == [0] * 17 and (ntx, nt) == (4, 16)
    mu = torch.tensor([[[0.5, 0.5]]], device=dev)
    sc = torch.tensor([[[0.01, 0.02]]], device=dev)
    check_equal(mu, sc, 32, 32, 8, 3.0)


def test_pair_budget_raises_before_allocation(dev):
    s = synth.config("c0")
    mu = s.mu.to(dev)
    sc = activate_scale(s.log_scale.to(dev))
    with pytest.raises(RH.PairBudgetExceeded):
        RH._build_tiles(mu, sc, s.H, s.W, 8, 3.0, max_pairs=100)


# Once a binning configuration has been seen, the pair phase is queued with the remembered capacity before
# the host reads the pair count (kernels take the count from device memory). These cases run that path.
def test_speculative_pair_phase_bit_exact(dev):
    """The second and later binnings of a configuration (the speculative path) equal the oracle, over a
    batch whose images have different pair counts."""
    mu, ls, *_ = random_scene(3000, 200, 160, seed=11, dev=dev, B=3)
    sc = activate_scale(ls)
    for _ in range(3):
        check_equal(mu, sc, 200, 160, 8, 3.0)


def test_pageable_count_buffer(dev, monkeypatch):
    """The pair totals reach the host both ways: written by the offsets kernel into the pinned landing buffer,
    and copied into pageable memory (hipHostGetDevicePointer refuses it). Same lists either way."""
    mu, ls, *_ = random_scene(3000, 200, 160, seed=14, dev=dev, B=2)
    sc = activate_scale(ls)
    check_equal(mu, sc, 200, 160, 8, 3.0)
    t = torch.empty(2 + RH._lib.MAX_LEVELS, dtype=torch.int64)
    assert not t.is_pinned()
    monkeypatch.setattr(RH, "_info_host", lambda: (t, t.numpy()))
    check_equal(mu, sc, 200, 160, 8, 3.0)
    check_equal(mu, sc, 200, 160, 8, 3.0)


def test_speculative_capacity_exceeded(dev):
    """A scene with many more pairs than the remembered capacity: the speculative launch leaves an empty
    list, the host sees the count and redoes the pair phase with buffers of the right size."""
    H, W, n = 256, 256, 4000
    mu, ls, *_ = random_scene(n, H, W, seed=12, dev=dev, ls_mean_px=1.0, ls_std=0.2)
    check_equal(mu, activate_scale(ls), H, W, 8, 3.0)            # few pairs: sets the capacity
    mu2, ls2, *_ = random_scene(n, H, W, seed=13, dev=dev, ls_mean_px=12.0, ls_std=0.2)
    check_equal(mu2, activate_scale(ls2), H, W, 8, 3.0)          # many more pairs than the capacity
    check_equal(mu, activate_scale(ls), H, W, 8, 3.0)            # and back


def test_speculative_budget_and_errors(dev):
    """After a binning has set a capacity, the pair budget still raises PairBudgetExceeded, and an empty
    rect (negative scale) still raises, with the speculative launch already queued."""
    s = synth.config("c0")
    mu = s.mu.to(dev)
    sc = activate_scale(s.log_scale.to(dev))
    check_equal(mu, sc, s.H, s.W, 8, 3.0)
    with pytest.raises(RH.PairBudgetExceeded):
        RH._build_tiles(mu, sc, s.H, s.W, 8, 3.0, max_pairs=100)
    with pytest.raises(ValueError, match="empty tile rect"):
        RH._build_tiles(mu, -sc, s.H, s.W, 8, 3.0)
    check_equal(mu, sc, s.H, s.W, 8, 3.0)


def splat_bin_maps(mu, sc, H, W, TILE, lv=None):
    """splat_bin through the C-ABI with both pair maps requested (the renderer asks for pair_q only).
    Returns tot, offsets, gid_sorted, tile_starts, pair_splat, pair_q as numpy arrays."""
    lib = RH._lib.load()
    dev = mu.device
    N = mu.shape[1]
    lvr = None if lv is None else RH._lib.ctypes.byref(lv)
    geom, nt, _ = RH.levels_geometry(H, W, TILE, lv)
    col = torch.zeros(N, 1, device=dev)
    op = torch.zeros(N, device=dev)
    rec = torch.empty(N, 16, device=dev)
    rect = torch.empty(N, 4, dtype=torch.int32, device=dev)
    off = torch.empty(N + 1, dtype=torch.int32, device=dev)
    info = torch.empty(2 + len(geom), dtype=torch.int64, device=dev)
    info_h = torch.zeros(2 + RH._lib.MAX_LEVELS, dtype=torch.int64, pin_memory=True)
    ws1 = torch.empty(lib.splat_bin_count_workspace_bytes(N, H, W, TILE, lvr), dtype=torch.uint8, device=dev)
    s = RH._lib.stream_ptr(dev)
    p = RH._lib.ptr
    rc = lib.splat_bin(p(mu[0]), p(sc[0]), None, p(op), p(col), 1, N, H, W, TILE, 3.0, lvr, 0, -1, p(rec), p(rect),
                       p(off), p(info), info_h.data_ptr(), p(ws1), ws1.numel(), 0, None, None, None, None, None, 0, s)
    tot = int(info_h[0])
    assert rc == RH._lib.STATUS_CAPACITY or (rc == 0 and tot == 0)
    i32 = lambda n: torch.full((max(n, 1),), -1, dtype=torch.int32, device=dev)
    gid, starts, psplat, pq = i32(tot), i32(nt + 1), i32(tot), i32(tot)
    ws2 = torch.empty(lib.splat_bin_pairs_workspace_bytes(N, H, W, TILE, lvr, tot), dtype=torch.uint8, device=dev)
    RH._lib.check(lib.splat_bin_pairs(p(rect), p(off), p(ws1), N, H, W, TILE, lvr, tot, p(gid), p(starts), p(psplat),
                                      p(pq), p(ws2), ws2.numel(), s), "splat_bin_pairs")
    torch.cuda.synchronize()
    return tot, off.cpu().numpy(), gid.cpu().numpy(), starts.cpu().numpy(), psplat.cpu().numpy(), pq.cpu().numpy()


@pytest.mark.parametrize("H,W,TILE,n,ls_px", [(768, 768, 8, 20000, 3.0), (200, 120, 4, 3000, 6.0),
                                              (2100, 2100, 8, 20000, 3.0), (64, 64, 2, 5000, 20.0)])
def test_pair_maps(dev, H, W, TILE, n, ls_px):
    """The backward's maps between sorted and splat-major pair order: pair_splat lists each splat's pairs in
    splat order, pair_q is a permutation with pair_splat[pair_q[i]] = gid_sorted[i], and splat-major pair q of
    splat g (k = q - offsets[g] walks the rect row by row, render_triton.py:396-404) lies in the tile of its
    sorted position. Checked against the oracle's rects; the last case is a wide rect per row (list overflow
    of the row expansion's LDS stash)."""
    mu, ls, *_ = random_scene(n, H, W, seed=H + n, dev=dev, ls_mean_px=ls_px, margin=0.1)
    sc = activate_scale(ls)
    tot, off, gid, st, psplat, pq = splat_bin_maps(mu, sc, H, W, TILE)
    gid_o, st_o = c_oracle.build_tiles(np_(mu[0]), np_(sc[0]), H, W, TILE, 3.0)
    assert np.array_equal(st, st_o) and np.array_equal(gid[:tot], gid_o[:tot])
    assert np.array_equal(psplat[:tot], np.repeat(np.arange(n), np.diff(off)))
    assert np.array_equal(np.sort(pq[:tot]), np.arange(tot))
    assert np.array_equal(psplat[pq[:tot]], gid[:tot])
    tx0, tx1, ty0, ty1, _ = c_oracle.rects(np_(mu[0]), np_(sc[0]), H, W, TILE, 3.0)
    ntx = (W + TILE - 1) // TILE
    q = pq[:tot].astype(np.int64)
    g = gid[:tot]
    w = (tx1 - tx0 + 1)[g]
    k = q - off[g]
    tile_q = (ty0[g] + k // w) * ntx + tx0[g] + k % w
    tile_i = np.repeat(np.arange(len(st) - 1), np.diff(st))
    assert np.array_equal(tile_q, tile_i)


def test_many_splats_separate_scan_launches(dev):
    """1.2M splats (4,688 decode blocks): the offsets take the two-launch scan and the row histogram its own
    scan launch; pair list and starts against the oracle."""
    H = W = 1024
    mu, ls, *_ = random_scene(1_200_000, H, W, seed=71, dev=dev, ls_mean_px=0.8, ls_std=0.3)
    check_equal(mu, activate_scale(ls), H, W, 8, 3.0)
