"""Randomized parity: seeded random scenes through the culled single-res render (composite alpha and odds, fields),
the octave render and the coarse/fine split, against the float64 C oracle.

Each case draws its canvas (1 to 199 pixels a side; 8 and more for the level renders), tile size (4, 8, 16), splat
count, log-normal splat sizes from a fifth of a pixel to 30 pixels with spreads up to 1.5, opacities up to 0.02,
0.5, 0.99 or 1, rotation or none, splats spilling past the canvas or not, and the level options. Per case:
* the device pair list equals the oracle's bit for bit (culled renders);
* the image (and T) within IMG_TOL of the oracle's own forward;
* every gradient tensor within GRAD_REL_TOL and every gradient component of every splat within PER_SPLAT_TOL of
  its own scale, against the oracle's backward started from the device forward's T, asum and fg: float32 forward
  rounding decides gradients in pixels whose 1 - T is below float32 resolution or whose S_a sits at the 1e-8
  clamp, in the reference's float32 as here, so the backward is held to the bar on the quantities it receives.
  The per-splat scale sums the magnitudes of every term along the chain (composite channels, upsample adjoint).
"""

import numpy as np
import pytest
import torch

from _gpu_util import activate_scale, device_bins, random_scene
from test_gpu_levels import octave_lv, run_levels, split_lv
from test_gpu_render import oracle_pairs, run_case

pytestmark = pytest.mark.gpu

SEED0 = 1000
N_CASES = 48


def draw(k):
    rng = np.random.default_rng(SEED0 + k)
    kind = str(rng.choice(["cull", "cull", "octave", "multires"]))
    TILE = int(rng.choice([4, 8, 8, 16]))
    lo = 8 if kind != "cull" else 1
    H, W = int(rng.integers(lo, 200)), int(rng.integers(lo, 200))
    N = int(rng.integers(1, 2500))
    ls_mean = float(np.exp(rng.uniform(np.log(0.2), np.log(30.0))))
    ls_std = float(rng.uniform(0.0, 1.5))
    op_max = float(rng.choice([0.02, 0.5, 0.99, 1.0]))
    theta = bool(rng.integers(0, 2))
    odds = bool(rng.integers(0, 2))
    fields = bool(rng.integers(0, 2)) if kind == "cull" else False
    margin = float(rng.choice([0.0, 0.0, 0.3]))
    extra = {}
    if kind == "octave":
        extra = {"max_octaves": int(rng.integers(0, 8)), "base": float(rng.choice([4.0, 8.0, 16.0]))}
    elif kind == "multires":
        extra = {"cf": int(rng.choice([2, 4, 8])), "n_coarse": int(rng.integers(0, N + 1))}
    return dict(kind=kind, TILE=TILE, H=H, W=W, N=N, ls_mean=ls_mean, ls_std=ls_std, op_max=op_max, theta=theta,
                odds=odds, fields=fields, margin=margin, **extra)


@pytest.mark.parametrize("k", range(N_CASES))
def test_random_scene(dev, k):
    c = draw(k)
    print(f"random case {k}: {c}", flush=True)
    H, W, TILE = c["H"], c["W"], c["TILE"]
    scene = random_scene(c["N"], H, W, seed=SEED0 + k, dev=dev, ls_mean_px=c["ls_mean"], ls_std=c["ls_std"],
                         op_max=c["op_max"], theta=c["theta"], margin=c["margin"])
    if c["kind"] == "cull":
        mu, ls = scene[0], scene[1]
        sc = activate_scale(ls)
        gid_d, st_d = device_bins(mu, sc, H, W, TILE)
        gid_o, st_o = oracle_pairs(mu, sc, H, W, TILE)
        tot = int(st_o[-1])
        assert np.array_equal(st_d[0], np.asarray(st_o)) and np.array_equal(gid_d[0][:tot], np.asarray(gid_o)[:tot])
        run_case(*scene, H, W, TILE, c["odds"], c["fields"], seed=k, bwd_on_device_fwd=True)
    elif c["kind"] == "octave":
        run_levels(*scene, H, W, TILE, octave_lv(c["max_octaves"], c["base"]), c["odds"], seed=k,
                   bwd_on_device_fwd=True)
    else:
        run_levels(*scene, H, W, TILE, split_lv(H, W, c["n_coarse"], c["cf"]), c["odds"], seed=k,
                   bwd_on_device_fwd=True)
