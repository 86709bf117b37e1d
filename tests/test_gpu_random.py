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

A second set draws calls of the entry points themselves (render_alpha_full_triton culled and exact,
render_alpha_octave, render_alpha_multires) with batches of 1 to 3 images, 1 to 7 colour channels (more than four
render as chunks), a background of shape [B, C] or [1, C], rotation or none, and tile sizes and cutoffs, in
well-conditioned scenes (opacities 0.45 to 0.95, splats of 1 to 12 pixels): every image of a batch equals its own
single-image call bit for bit, image and gradients included, and the first image and its gradients meet the image
and gradient bars against the float64 oracle through autograd (log-scales included).
"""

import numpy as np
import pytest
import torch

from _gpu_util import GRAD_REL_TOL, IMG_TOL, RH, activate_scale, device_bins, np_, random_scene, rel_err
from test_gpu_api import NAMES, oracle_run
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


API_SEED0 = 100
N_API_CASES = 24


def draw_api(k, dev):
    rng = np.random.default_rng(API_SEED0 + k)
    kind = str(rng.choice(["cull", "cull", "exact", "octave", "multires"]))
    B, C = int(rng.integers(1, 4)), int(rng.choice([1, 2, 3, 4, 5, 7]))
    H, W = int(rng.integers(8, 100)), int(rng.integers(8, 100))
    N = int(rng.integers(1, 1200)) if kind != "exact" else int(rng.integers(1, 300))
    theta, odds = bool(rng.integers(0, 2)), bool(rng.integers(0, 2)) if kind != "exact" else False
    bg1 = bool(rng.integers(0, 2))
    TILE, cutoff = int(rng.choice([4, 8, 16])), float(rng.choice([2.0, 3.0, 4.0]))
    ls_mean = float(np.exp(rng.uniform(np.log(1.0), np.log(12.0))))
    g = torch.Generator().manual_seed(API_SEED0 + k)
    mu = torch.rand(B, N, 2, generator=g) * 1.2 - 0.1
    ls = np.log(ls_mean / max(H, W)) + 0.5 * torch.randn(B, N, 2, generator=g)
    col = torch.rand(B, N, C, generator=g)
    op = torch.rand(B, N, generator=g) * 0.5 + 0.45
    bg = torch.rand(1 if bg1 else B, C, generator=g)
    th = torch.rand(B, N, generator=g) * 6.28 if theta else None
    scene = [None if t is None else t.to(dev) for t in (mu, ls, col, op, bg, th)]
    gout = torch.randn(B, C, H, W, generator=g).to(dev)
    if kind == "cull":
        kw = dict(TILE=TILE, cutoff=cutoff, odds=odds)
        fn = lambda *a, theta=None: RH.render_alpha_full_triton(*a, H, W, theta=theta, cull=True, **kw)
    elif kind == "exact":
        kw = {}
        fn = lambda *a, theta=None: RH.render_alpha_full_triton(*a, H, W, theta=theta, cull=False)
    elif kind == "octave":
        kw = dict(TILE=TILE, odds=odds)
        fn = lambda *a, theta=None: RH.render_alpha_octave(*a, H, W, theta=theta, **kw)
    else:
        kw = dict(TILE=TILE, odds=odds, n_coarse=int(rng.integers(0, N + 1)))
        fn = lambda *a, theta=None: RH.render_alpha_multires(*a, H, W, theta=theta, **kw)
    desc = dict(kind=kind, B=B, C=C, H=H, W=W, N=N, theta=theta, bg1=bg1, ls_mean=round(ls_mean, 2), **kw)
    return desc, fn, kw, scene, gout, bg1


def run_api(fn, scene, gout, bg1=False, b=None):
    """fn on leaves copied from scene (image b alone when given, with the whole bg when bg1); (out, grads)."""
    sl = [None if t is None else (t if b is None or (n == "bg" and bg1) else t[b:b + 1]) for n, t in zip(NAMES, scene)]
    L = [None if t is None else t.detach().clone().requires_grad_(True) for t in sl]
    out = fn(*L[:5], theta=L[5])
    (out * (gout if b is None else gout[b:b + 1])).sum().backward()
    return out.detach(), {n: (None if t is None else t.grad) for n, t in zip(NAMES, L)}


@pytest.mark.parametrize("k", range(N_API_CASES))
def test_random_entry_point_call(dev, k):
    desc, fn, kw, scene, gout, bg1 = draw_api(k, dev)
    print(f"random entry-point case {k}: {desc}", flush=True)
    H, W = desc["H"], desc["W"]
    out, grads = run_api(fn, scene, gout)
    for b in range(desc["B"]):
        ob, gb = run_api(fn, scene, gout, bg1, b)
        assert torch.equal(ob[0], out[b]), f"image {b} differs from its single-image call"
        for n in NAMES:
            if gb[n] is not None and n != "bg":
                assert torch.equal(gb[n][0], grads[n][b]), f"gradient {n} of image {b} differs"
    ref_img, ref_g = oracle_run(desc["kind"], [None if t is None else t[0:1] for t in scene], gout[0:1], H, W, **kw)
    d = np.abs(np_(out[0]) - ref_img.numpy()).max()
    assert d <= IMG_TOL, f"image max-abs {d:.2e}"
    for n in NAMES:
        if ref_g[n] is not None and n != "bg":
            e = rel_err(np_(grads[n][0]), ref_g[n].numpy())
            assert e <= GRAD_REL_TOL, f"gradient {n}: rel {e:.2e}"


def test_elongated_splat_moment_form(dev):
    """Draw 399,016 of the generator above (seed 400,016): a coarse/fine odds render on 4 x 4 tiles whose coarse level
    holds a splat of aspect 139 with pairs at whitened spans 6 to 8. In the moment form, sum q u^2 along such a
    splat's long axis is a small difference of the mapped moments' terms; with those pairs in the moment form the
    scale gradient missed the tensor-wide bar (1.6e-4) and the splat's own per-splat bar (4.6e-4 of its scale). The
    backward gives pairs of splats more elongated than 16:1 the direct form above span 4."""
    test_random_scene(dev, 399_016)
