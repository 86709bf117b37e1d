"""Backward parity for near-transparent splats (render_triton.py:697-698: g_op = sum da * falloff carries no
opacity factor). The released checkpoint's coarse layer emits opacities of 1e-11 to 1e-4 with sizes of tens of
pixels; here 5 % of the splats are drawn at opacities {0, 1e-10, 1e-8, 1e-6, 1e-4} with sigma 5-40 px per axis
and another 5 % at log-uniform opacities in [1e-12, 1]. Every gradient tensor is held to 1e-4 of its largest
reference magnitude and the opacity gradient also per splat, to 1e-4 of the summed magnitudes of that splat's
own terms (the oracle's op_scale), against the float64 C oracle: single-res (composite and fields) and
octave, alpha and odds."""

import numpy as np
import pytest
import torch

from _gpu_util import GRAD_REL_TOL, np_
from _scenes import low_opacity_scene, per_splat_op_err
from gaussian_splat_encoder import _lib
from test_gpu_levels import run_levels
from test_gpu_render import run_case

pytestmark = pytest.mark.gpu

PER_SPLAT_TOL = 1e-4


def scene_on(dev, n, H, W, seed):
    (mu, ls, col, op, bg, th), low, logu = low_opacity_scene(n, H, W, seed)
    return [t.to(dev) for t in (mu, ls, col, op, bg, th)], low, logu


def check_per_splat(g_op, gref, low):
    e, i = per_splat_op_err(np_(g_op[0]), gref["op"], gref["op_scale"])
    assert e <= PER_SPLAT_TOL, f"g_op of splat {i}: {e:.2e} of its scale"
    # the near-transparent subset has opacity gradients of the size of everyone else's
    assert np.abs(gref["op"][low]).max() > 1e-3 * np.abs(gref["op"]).max()


@pytest.mark.parametrize("odds,fields", [(False, False), (True, False), (True, True)])
def test_single_res(dev, odds, fields):
    H = W = 256
    scene, low, _ = scene_on(dev, 3000, H, W, seed=51)
    got, gref = run_case(*scene, H, W, 8, odds, fields, seed=52)
    check_per_splat(got["op"], gref, low)


@pytest.mark.parametrize("odds", [False, True])
def test_octave(dev, odds):
    H = W = 256
    scene, low, _ = scene_on(dev, 3000, H, W, seed=53)
    lv = _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)
    bins, got, gref = run_levels(*scene, H, W, 8, lv, odds, seed=54, want_grads=True)
    assert sum(1 for n in bins.level_tot_b[0] if n) >= 2
    check_per_splat(got["op"], gref, low)


def test_full_size_c2_low_opacity(dev):
    """The benchmark frame (768 x 768, 92,160 splats) with 5 % of its splats made near-transparent and large."""
    from gaussian_splat_encoder import synth
    s = synth.config("c2")
    (_, ls_l, _, op_l, _, _), low, logu = low_opacity_scene(s.n, s.H, s.W, seed=55)
    ls, op = s.log_scale.clone(), s.opacity.clone()
    ls[0, low], op[0, low], op[0, logu] = ls_l[0, low], op_l[0, low], op_l[0, logu]
    scene = [t.to(dev) for t in (s.mu, ls, s.color, op, s.bg, s.theta)]
    got, gref = run_case(*scene, s.H, s.W, 8, False, False, seed=56)
    check_per_splat(got["op"], gref, low)
