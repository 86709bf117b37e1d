"""Per-splat parity of every backward gradient where the per-tile backward takes its numerical shortcut.

The backward sums each pair's moments around the pair's own centre (the splat centre clamped to the tile) and
maps them onto sum q u, ..., sum q u v once per pair; sum q u^2 then comes out as up^2 sum q + 2 up sum q du +
sum q du^2, whose terms cancel where q sits away from that centre, more so the larger the pair's whitened span
over the tile. Pairs whose span exceeds the kernel's limit (8) take the direct form instead. Every component of
every splat is held to 1e-4 of that splat's own scale for the component (the float64 C oracle's summed term
magnitudes, render_triton.py:688-710), beside the tensor-wide bar, on scenes built around that limit:
* splats whose smaller axis puts their spans over an 8 x 8 tile at 5 to 11 (sigma about 0.3 to 0.7 px);
* splats far smaller than a pixel (direct form);
* the benchmark frame through the octave render (alpha and odds);
* a thin rotated splat (0.06 x 0.67 px), against the oracle with the float32 rotation the reference and the device
  hold, and the size of the float32 rotation's own effect against a float64 rotation.
Every run_case / run_levels call of the other GPU tests applies the same per-splat check.
"""

import numpy as np
import pytest
import torch

from _gpu_util import RH, activate_scale, np_
from _scenes import span_scene, spans
from gaussian_splat_encoder import _lib, synth
from test_gpu_levels import run_levels
from test_gpu_render import run_case

pytestmark = pytest.mark.gpu

MOMENT_SPAN = 8.0


def on(dev, scene):
    return [t.to(dev) for t in scene]


@pytest.mark.parametrize("odds,fields", [(False, False), (True, False), (True, True)])
def test_moment_span_boundary(dev, odds, fields):
    H = W = 256
    scene = span_scene(6000, H, W, seed=71)
    sp = spans(np_(scene[0][0]), np_(activate_scale(scene[1])[0]), np_(scene[5][0]), H, W)
    # the scene straddles the limit: many splats on either side of it within the window
    assert np.mean((sp > 6) & (sp <= MOMENT_SPAN)) > 0.15 and np.mean((sp > MOMENT_SPAN) & (sp < 10)) > 0.15
    run_case(*on(dev, scene), H, W, 8, odds, fields, seed=72)


@pytest.mark.parametrize("odds", [False, True])
def test_moment_span_boundary_octave(dev, odds):
    H = W = 256
    scene = span_scene(6000, H, W, seed=73)
    lv = _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)
    run_levels(*on(dev, scene), H, W, 8, lv, odds, seed=74)


@pytest.mark.parametrize("odds,fields", [(False, False), (True, True)])
def test_subpixel_splats(dev, odds, fields):
    """Splats of 0.05 to 0.35 px (spans of 8.5 to 80 over a tile: the direct form), mixed with ordinary ones."""
    H = W = 128
    scene = span_scene(3000, H, W, seed=75, lo=8.5, hi=80.0, frac=0.7)
    run_case(*on(dev, scene), H, W, 8, odds, fields, seed=76)


@pytest.mark.parametrize("TILE", [4, 16])
def test_moment_span_other_tiles(dev, TILE):
    """The span limit over 4 x 4 and 16 x 16 tiles (the same scenes give other spans there)."""
    H = W = 256
    scene = span_scene(5000, H, W, seed=77 + TILE, lo=5.0 * 7 / (TILE - 1), hi=11.0 * 7 / (TILE - 1))
    run_case(*on(dev, scene), H, W, TILE, False, False, seed=78)
    run_case(*on(dev, scene), H, W, TILE, True, True, seed=79)


@pytest.mark.parametrize("odds", [False, True])
def test_c2_octave_per_splat(dev, odds):
    """The benchmark frame (768 x 768, 92,160 splats) through the octave render, every splat's gradients."""
    s = synth.config("c2").to(dev)
    run_levels(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.theta, s.H, s.W, 8, _lib.SplatLevels(1, 6, 8.0, 0, 0, 0),
               odds, seed=80)


def test_float32_rotation_of_a_thin_splat(dev):
    """A random scene (seed 50039; FIELDS, odds) holding splat 617, 0.06 x 0.67 px rotated by 2.23 rad: an aspect of
    11.5 and far thinner than a pixel, so its pairs take the direct form. The device holds every splat's cos and
    sin as the nearest float32 values (render_triton.py:95-96 holds them in float32 as well). Against the oracle
    with the same float32 rotation every component of every splat meets the per-splat bar with a wide margin.
    Against the float64 rotation the float32 rounding of that splat's cos and sin alone moves its theta gradient by
    about 1e-4 of its scale: the oracle's own float32 and float64 rotations differ by as much, and the device's
    difference from the float64-rotation oracle stays within that."""
    from _scenes import per_splat_errors
    from _gpu_util import random_scene
    H, W = 186, 44
    scene = random_scene(626, H, W, seed=50039, dev=dev, ls_mean_px=0.3713114842386114,
                         ls_std=1.2326931862574066, op_max=0.5, theta=True)
    got, ref32 = run_case(*scene, H, W, 8, True, True, seed=39, rot32=True)   # per-splat bar inside
    got_np = {k: None if v is None else np_(v[0]) for k, v in got.items()}
    e32 = per_splat_errors(got_np, ref32)
    assert max(e for e, _ in e32.values()) < 1e-5, e32
    _, ref64 = run_case(*scene, H, W, 8, True, True, seed=39, per_splat=False, rot32=False)
    dev_th, at_dev = per_splat_errors(got_np, ref64)["theta"]
    rot_th, at_rot = per_splat_errors({"theta": ref32["theta"]}, ref64)["theta"]
    print(f"theta per-splat: device vs float64 rotation {dev_th:.2e} (splat {at_dev}), float32 vs float64 rotation "
          f"in the oracle {rot_th:.2e} (splat {at_rot})", flush=True)
    assert rot_th > 3e-5            # the scene exercises the rounding of a thin splat's rotation
    assert dev_th <= rot_th + 1e-5  # and the device's difference from the float64 rotation is that rounding


def test_thin_splat_on_a_tile_edge(dev):
    """A random scene (seed 90296; FIELDS, alpha, no rotation) holding splat 2008, 1.06 x 0.15 px, its centre on the
    pixel column at a tile edge (x = 8.5 px). Its moment across the thin axis, sum q v^2 (its x-scale gradient), comes
    from the pixel columns one pixel to either side, whose falloff is 2^-31 of the centre column's; the column to the
    left lies in the neighbouring tile. The backward keeps that tile (a negligible pair's falloff is measured against
    the 3 x 3 pixel centres around the splat's nearest one), and every component of every splat meets the per-splat
    bar; measured against the nearest centre alone the tile was dropped, half of that moment with it."""
    from _gpu_util import random_scene
    H, W = 176, 42
    scene = random_scene(2259, H, W, seed=90296, dev=dev, ls_mean_px=1.2930040205251416, ls_std=0.8795019694762315,
                         op_max=0.99, theta=False)
    sc = np_(activate_scale(scene[1])[0])
    assert abs(sc[2008, 1] * W - 0.152) < 1e-3 and abs(np_(scene[0][0])[2008, 1] * W - 8.5) < 1e-3
    run_case(*scene, H, W, 8, False, True, seed=296)
