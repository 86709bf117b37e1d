"""The per-splat magnitude scales of the float64 C oracle's backward ('mag'), on the CPU.

The GPU tests hold every gradient component of every splat to 1e-4 of that splat's own scale: the sum over its
pixel-pairs of the magnitudes of the terms entering the component (render_triton.py:688-710 with every sum's
terms taken apart). Here the scale is pinned:
* it bounds the gradient (|g| <= mag, the triangle inequality) for every component, alpha and odds, composite
  and fields;
* it equals |g| where the gradient has one term: one splat, one pixel, no rotation, one upstream term;
* it scales like the gradient: twice the upstream gives twice the scale; and a splat's scale does not depend
  on the other splats (fields mode, where the upstream is given);
* a planted error of 3e-4 of one small splat's scale, below the tensor-wide bar, is caught per splat.
"""

import numpy as np
import pytest

from _scenes import PER_SPLAT_NAMES, low_opacity_scene, per_splat_err, per_splat_errors
from oracle import c_oracle
from oracle import render_ref as R


def scene(n, H, W, seed):
    (mu, ls, col, op, bg, th), _, _ = low_opacity_scene(n, H, W, seed=seed)
    sc = R.activate_scale(ls[0]).numpy()
    return mu[0].numpy(), sc, th[0].numpy(), op[0].numpy(), col[0].numpy(), bg[0].numpy()


def upstream(H, W, seed, C=3):
    rng = np.random.default_rng(seed)
    return dict(dslog=rng.standard_normal(H * W), dsa=rng.standard_normal(H * W),
                dsac=rng.standard_normal((H * W, C)))


@pytest.mark.parametrize("odds", [False, True])
@pytest.mark.parametrize("fields", [False, True])
def test_mag_bounds_every_gradient(odds, fields):
    H, W = 40, 48
    mu, sc, th, op, col, bg = scene(300, H, W, seed=11)
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    if fields:
        r = c_oracle.bwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, odds=odds, fields=True, **upstream(H, W, 2))
    else:
        out, T, asum, fg = c_oracle.fwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, odds=odds, bg=bg)
        gout = np.random.default_rng(3).standard_normal(out.shape)
        r = c_oracle.bwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, odds=odds, bg=bg, T=T, asum=asum, fg=fg, gout=gout)
    for name in PER_SPLAT_NAMES:
        g, m = r[name], r["mag"][name]
        assert m.shape == g.shape and np.all(m >= 0)
        assert np.all(np.abs(g) <= m * (1 + 1e-12) + 1e-300), name
        assert m.max() > 0, name
    # the scale is not a loose bound everywhere (random upstream signs: a few terms dominate some splats)
    assert max(np.max(np.abs(r[n]) / np.maximum(r["mag"][n], 1e-300)) for n in PER_SPLAT_NAMES) > 0.25


def test_mag_equals_the_single_term():
    """One splat, one pixel (a 1 x 1 canvas), no rotation, upstream dS_log only: every component has one term."""
    H = W = 1
    mu = np.array([[0.3, 0.7]], np.float32)
    sc = np.array([[0.8, 0.5]], np.float32)
    op = np.array([0.6], np.float32)
    col = np.array([[0.2, 0.5, 0.9]], np.float32)
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    for odds in (False, True):
        # da = -dS_log u alone, then the colour term alone (one channel): one term in every component
        for ups in ((np.array([-1.7]), np.zeros((1, 3))), (np.zeros(1), np.array([[0.0, -0.6, 0.0]]))):
            r = c_oracle.bwd_cull(mu, sc, None, op, col, gid, st, H, W, 8, odds=odds, fields=True, dslog=ups[0],
                                  dsa=np.zeros(1), dsac=ups[1])
            for name in ("mu", "scale", "col", "op"):
                np.testing.assert_allclose(r["mag"][name], np.abs(r[name]), rtol=1e-12, err_msg=name)
            assert abs(r["op"][0]) > 0 and np.all(np.abs(r["mu"]) > 0)


def test_mag_is_linear_in_the_upstream_and_per_splat():
    H = W = 32
    mu, sc, th, op, col, _ = scene(150, H, W, seed=21)
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    ups = upstream(H, W, 5)
    r1 = c_oracle.bwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, odds=True, fields=True, **ups)
    r2 = c_oracle.bwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, odds=True, fields=True,
                           **{k: 2 * v for k, v in ups.items()})
    for name in PER_SPLAT_NAMES:
        np.testing.assert_allclose(r2["mag"][name], 2 * r1["mag"][name], rtol=1e-12, atol=1e-300)
    # splat 0 alone on the same pixels: the same scale as in the full scene
    one = c_oracle.build_tiles(mu[:1], sc[:1], H, W, 8)
    r0 = c_oracle.bwd_cull(mu[:1], sc[:1], th[:1], op[:1], col[:1], *one, H, W, 8, odds=True, fields=True, **ups)
    for name in PER_SPLAT_NAMES:
        np.testing.assert_allclose(r0["mag"][name][0], r1["mag"][name][0], rtol=1e-12)


def test_planted_error_is_caught_per_splat():
    H = W = 48
    mu, sc, th, op, col, _ = scene(400, H, W, seed=31)
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    r = c_oracle.bwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, fields=True, **upstream(H, W, 7))
    for name in ("mu", "scale", "theta", "col", "op"):
        g, m = r[name], r["mag"][name]
        flat_m = m.reshape(len(m), -1)
        # the splat of the smallest scale above a hundred times the floor
        top = flat_m.max(axis=1)
        cand = np.where(top > 1e-5 * flat_m.max())[0]
        i = cand[np.argmin(top[cand])]
        bad = g.copy().reshape(len(g), -1)
        k = int(np.argmax(flat_m[i]))
        bad[i, k] += 3e-4 * flat_m[i, k]
        bad = bad.reshape(g.shape)
        tensor_wide = np.abs(bad - g).max() / np.abs(g).max()
        assert tensor_wide < 1e-4, (name, tensor_wide)      # invisible to the tensor-wide bar
        e, at = per_splat_err(bad, g, m)
        assert e > 2e-4 and at // flat_m.shape[1] == i, (name, e, at)
    assert not any(e > 1e-12 for e, _ in per_splat_errors({n: r[n] for n in PER_SPLAT_NAMES}, r).values())
