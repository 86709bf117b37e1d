"""The deferred read of the pair count: once a binning configuration (splat count, canvas, tile, cutoff, levels)
has been seen, a forward queues its pair phase and its render launches on the speculative pair list and level
totals of the previous call before it reads the count, and repeats them when the count exceeds the capacity or
a level it did not render now holds pairs. Every case is checked against the oracle (composed per level for
octave renders)."""

import numpy as np
import pytest
import torch

from _gpu_util import IMG_TOL, RH, activate_scale, np_, random_scene
from gaussian_splat_encoder import _lib
from test_gpu_levels import run_levels
from test_gpu_render import run_case

pytestmark = pytest.mark.gpu


def octave_lv():
    return _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)


def test_octave_repeat_and_misses(dev):
    H = W = 192
    n = 2000
    small = random_scene(n, H, W, seed=81, dev=dev, ls_mean_px=1.5, ls_std=0.2)
    for _ in range(2):   # the second call is deferred on the first call's capacity and levels
        run_levels(*small, H, W, 8, octave_lv(), odds=True, seed=82)
    # many more pairs and coarser octaves than the remembered capacity and level mask: both are redone
    big = random_scene(n, H, W, seed=83, dev=dev, ls_mean_px=14.0, ls_std=0.5)
    bins = run_levels(*big, H, W, 8, octave_lv(), odds=True, seed=84)
    assert sum(1 for x in bins.level_tot_b[0] if x) >= 3
    # back to the small scene: fewer pairs and levels than speculated (empty levels render zeros)
    run_levels(*small, H, W, 8, octave_lv(), odds=False, seed=85)


def test_cull_repeat_and_capacity_miss(dev):
    H = W = 128
    n = 1500
    a = random_scene(n, H, W, seed=86, dev=dev, ls_mean_px=1.5, ls_std=0.2)
    b = random_scene(n, H, W, seed=87, dev=dev, ls_mean_px=9.0, ls_std=0.3)
    for scene in (a, a, b, a):
        run_case(*scene, H, W, 8, odds=False, fields=False, seed=88)


def test_deferred_entry_points_and_budget(dev):
    """Through the public entry points and autograd: repeated calls give identical images and gradients, and the
    pair budget still raises when the count is read after the launches were queued."""
    H = W = 96
    mu, ls, col, op, bg, th = random_scene(800, H, W, seed=89, dev=dev, ls_mean_px=3.0)
    res = []
    for _ in range(3):
        leaves = [t.clone().requires_grad_(True) for t in (mu, ls, col, op, bg, th)]
        img = RH.render_alpha_octave(*leaves[:5], H, W, theta=leaves[5], odds=True)
        img.sum().backward()
        res.append([img.detach()] + [t.grad.clone() for t in leaves])
    for r in res[1:]:
        for x, y in zip(res[0], r):
            assert torch.equal(x, y)
    sc = activate_scale(ls)
    bins = RH._bin(mu, sc, col, op, th, H, W, 8, 3.0, lv=octave_lv())
    worst = max(bins.level_tot_b[0])
    with pytest.raises(RH.PairBudgetExceeded):
        RH.render_alpha_octave(mu, ls, col, op, bg, H, W, theta=th, max_pairs=worst - 1)
    out = RH.render_alpha_octave(mu, ls, col, op, bg, H, W, theta=th, odds=True)
    assert torch.equal(out, res[0][0])
