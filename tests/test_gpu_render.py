"""Kernel-level parity of the per-tile forward and backward against the float64 C oracle over the same
(bit-exact) pair lists: images within 1e-5 max-abs, gradients within 1e-4 relative."""

import contextlib

import numpy as np
import pytest
import torch

from _gpu_util import GRAD_REL_TOL, IMG_TOL, RH, activate_scale, np_, random_scene, rel_err
from _gpu_util import check_per_splat
from gaussian_splat_encoder import synth
from oracle import c_oracle

pytestmark = pytest.mark.gpu


def oracle_pairs(mu, sc, H, W, TILE, cutoff=3.0):
    return c_oracle.build_tiles(np_(mu[0]), np_(sc[0]), H, W, TILE, cutoff)


def run_case(mu, ls, col, op, bg, th, H, W, TILE, odds, fields, seed=0, check_bwd=True, per_splat=True,
             bwd_on_device_fwd=False, rot32=True, fwd_tol=IMG_TOL):
    """Forward (and backward) of one batch against the C oracle over the oracle's pair list. Gradients are held
    to GRAD_REL_TOL of each tensor's largest magnitude and, with per_splat, every component of every splat to
    PER_SPLAT_TOL of that splat's own scale for it (the oracle's 'mag'). bwd_on_device_fwd (composite renders):
    the oracle's backward starts from the device forward's T, asum and fg instead of its own, so that the
    gradients check the backward alone (float32 forward rounding can decide them where 1 - T is below float32
    resolution). rot32 (the default): the oracle holds each splat's cos and sin as the nearest float32 values, as
    the reference and the device do (rot32=False: in float64; for an elongated splat far thinner than a pixel the
    rounding of its rotation alone then moves its theta gradient by up to ~2e-4 of its scale, see
    test_gpu_per_splat.py). fwd_tol: the image and T bar. The fields' bar is fwd_tol (2 (1 + |S|) + K), with K the
    oracle's sensitivity of the field to a relative change of every unclamped alpha: with odds weights a / (1 - a)
    an alpha error grows by 1 / (1 - a)^2 in S_a and S_ac, so a near-opaque pair's float32 falloff rounding (a few
    1e-6 of it, for a splat far thinner than a pixel) reaches 1e-4 of those fields. Returns the device gradients
    by name and the oracle's (None without the backward)."""
    with (c_oracle.rot32() if rot32 else contextlib.nullcontext()):
        return _run_case(mu, ls, col, op, bg, th, H, W, TILE, odds, fields, seed, check_bwd, per_splat,
                         bwd_on_device_fwd, fwd_tol)


def _run_case(mu, ls, col, op, bg, th, H, W, TILE, odds, fields, seed, check_bwd, per_splat, bwd_on_device_fwd,
              fwd_tol):
    dev = mu.device
    sc = activate_scale(ls)
    P, C = H * W, col.shape[-1]
    gid, st = oracle_pairs(mu, sc, H, W, TILE)
    args = [np_(mu[0]), np_(sc[0]), None if th is None else np_(th[0]), np_(op[0]), np_(col[0])]
    g = torch.Generator().manual_seed(seed)
    if fields:
        slog, sa, sac, bins = RH._forward_cull_fields(mu, sc, col, op, th, H, W, TILE, odds=odds)
        *ref, cond = c_oracle.fwd_cull(*args, gid, st, H, W, TILE, odds=odds, fields=True, cond=True)
        for name, got, r, k in zip(("S_log", "S_a", "S_ac"), (slog, sa, sac), ref, cond):
            d = np.abs(np_(got[0]).reshape(r.shape) - r)
            bar = fwd_tol * (2.0 * (1.0 + np.abs(r)) + k)
            assert np.all(d <= bar), f"{name}: max-abs {d.max():.2e}, {np.max(d / bar):.2f} of its bar"
        # the image composited from the fields meets the image bar
        T = np.exp(ref[0]); asum = np.maximum(ref[1], 1e-8)
        img_ref = (1 - T)[:, None] * ref[2] / asum[:, None] + T[:, None] * np_(bg[0])
        img = RH._composite_fields(slog, sa, sac, bg, 1, H, W, C)[0].permute(1, 2, 0).reshape(P, C)
        assert np.abs(np_(img) - img_ref).max() <= fwd_tol
        if not check_bwd:
            return
        ups = [torch.randn(s.shape, generator=g) for s in (slog, sa, sac)]
        grads = RH._backward_cull_fields(*[u.to(dev) for u in ups], mu, sc, col, op, th, bins, H, W, TILE, odds=odds)
        gref = c_oracle.bwd_cull(*args, gid, st, H, W, TILE, odds=odds, fields=True, dslog=ups[0][0].numpy(),
                                 dsa=ups[1][0].numpy(), dsac=ups[2][0].numpy())
        names = ["mu", "scale", "col", "op", "theta"]
    else:
        out, (T, asum, fg), bins = RH._forward_cull(mu, sc, col, op, bg, th, H, W, TILE, odds=odds)
        ref = c_oracle.fwd_cull(*args, gid, st, H, W, TILE, odds=odds, fields=False, bg=np_(bg[0]))
        assert np.abs(np_(out[0]) - ref[0]).max() <= fwd_tol, f"image max-abs {np.abs(np_(out[0]) - ref[0]).max():.2e}"
        assert np.abs(np_(T[0]) - ref[1]).max() <= fwd_tol, f"T max-abs {np.abs(np_(T[0]) - ref[1]).max():.2e}"
        if not check_bwd:
            return
        gout = torch.randn(out.shape, generator=g).to(dev)
        grads = RH._backward_cull(gout, mu, sc, col, op, bg, th, T, asum, fg, bins, H, W, TILE, odds=odds)
        Tq, aq, fq = ((np_(T[0]).astype(np.float64), np_(asum[0]).astype(np.float64), np_(fg[0]).astype(np.float64))
                      if bwd_on_device_fwd else (ref[1], ref[2], ref[3]))
        gref = c_oracle.bwd_cull(*args, gid, st, H, W, TILE, odds=odds, fields=False, bg=np_(bg[0]), T=Tq,
                                 asum=aq, fg=fq, gout=np_(gout[0]))
        names = ["mu", "scale", "col", "op", "bg", "theta"]
    for name, got in zip(names, grads):
        if got is None:
            assert name == "theta" and th is None
            continue
        r = gref[name]
        e = rel_err(np_(got[0]), r)
        assert e <= GRAD_REL_TOL, f"{name}: rel {e:.2e}"
    got = dict(zip(names, grads))
    if per_splat:
        check_per_splat(got, gref)
    return got, gref


@pytest.mark.parametrize("odds", [False, True])
@pytest.mark.parametrize("fields", [False, True])
@pytest.mark.parametrize("has_theta", [True, False])
def test_modes_small(dev, odds, fields, has_theta):
    H = W = 64
    scene = random_scene(1024, H, W, seed=11, dev=dev, op_max=0.99, theta=has_theta)
    run_case(*scene, H, W, 8, odds, fields, seed=1)


@pytest.mark.parametrize("TILE,H,W", [(4, 37, 51), (8, 37, 51), (16, 37, 51), (16, 96, 64)])
def test_tiles_and_ragged_canvas(dev, TILE, H, W):
    scene = random_scene(600, H, W, seed=TILE * 7 + H, dev=dev, margin=0.2)
    run_case(*scene, H, W, TILE, odds=False, fields=False, seed=2)
    run_case(*scene, H, W, TILE, odds=True, fields=True, seed=3)


def test_alpha_clamp_gate(dev):
    """Opacity 1 at pixel centres drives a onto the 1 - 1e-4 clamp, where the gradient is gated off."""
    H = W = 32
    mu, ls, col, op, bg, th = random_scene(200, H, W, seed=5, dev=dev, ls_mean_px=4.0)
    mu = ((torch.floor(mu * H) + 0.5) / H).contiguous()
    op = torch.ones_like(op)
    run_case(mu, ls, col, op, bg, th, H, W, 8, odds=False, fields=False, seed=4)
    run_case(mu, ls, col, op, bg, th, H, W, 8, odds=True, fields=False, seed=5)


def test_c0_config(dev):
    s = synth.config("c0").to(dev)
    run_case(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.theta[:, :], s.H, s.W, 8, False, False, seed=6)


@pytest.mark.parametrize("odds,fields", [(False, False), (True, True)])
def test_c1_full_size(dev, odds, fields):
    """The headline configuration: 768 x 768, 92,160 splats, forward and backward."""
    s = synth.config("c2").to(dev)
    run_case(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.theta, s.H, s.W, 8, odds, fields, seed=7)


def test_heavy_tail_splats(dev):
    """A C4-like heavy tail at small scale: 2 % of the splats at ~40 px (thousands of tile pairs each), whose
    per-pair sums span many reduction waves; gradients against the oracle."""
    H = W = 256
    mu, ls, col, op, bg, th = random_scene(3000, H, W, seed=41, dev=dev, ls_mean_px=3.0, ls_std=0.5, op_max=0.9)
    g = torch.Generator().manual_seed(42)
    heavy = torch.rand(1, 3000, generator=g) < 0.02
    big = float(np.log(40.0 / W)) + 0.3 * torch.randn(1, 3000, 2, generator=g)
    ls = torch.where(heavy[..., None].to(dev), big.to(dev), ls)
    run_case(mu, ls, col, op, bg, th, H, W, 8, odds=False, fields=False, seed=9)
    run_case(mu, ls, col, op, bg, th, H, W, 8, odds=True, fields=True, seed=10)


@pytest.mark.parametrize("odds,fields", [(False, False), (True, True), (True, False)])
def test_long_pair_lists_wide_split(dev, odds, fields):
    """Few tiles with long pair lists (64 tiles of ~1,500 pairs): the forward takes 16 waves per tile
    (FLAG_WIDE); images and gradients against the oracle."""
    H = W = 64
    scene = random_scene(2000, H, W, seed=23, dev=dev, ls_mean_px=8.0, ls_std=0.3, op_max=0.95)
    sc = activate_scale(scene[1])
    gid, st = oracle_pairs(scene[0], sc, H, W, 8)
    assert RH._wide(8, len(st) - 1, int(st[-1])), "the scene must take the 16-wave forward"
    run_case(*scene, H, W, 8, odds, fields, seed=24)
