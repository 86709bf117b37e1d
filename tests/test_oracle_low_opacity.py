"""The backward's negligible-pair rule, on the CPU oracle.

The per-tile backward gives a pair a zero record when the pair's falloff stays below 2^-30 of the splat's falloff
at the pixel centre nearest its centre, at every pixel of the tile. Two alternatives are planted in the float64 C
oracle (the dropped pairs are removed from its pair list) and held to the per-splat checks of the GPU tests:
* near-transparent splats: the opacity gradient g_op = sum da * falloff (render_triton.py:697-698) carries no
  opacity factor, so the rule must look at the falloff alone: a rule on opacity * falloff drops the far tiles of
  near-transparent splats from their opacity gradient;
* splats far smaller than a pixel: their best pixel may reach only 2^-20, and the scale gradient sum q u^2 weighs
  far pixels by u^2, so an absolute cut at 2^-30 drops terms worth 1e-3 of such a splat's scale gradient, where
  the relative cut keeps every splat's gradients within 1e-7 of its own scale.
"""

import numpy as np
import pytest

from _scenes import low_opacity_scene, per_splat_op_err
from oracle import c_oracle
from oracle import render_ref as R

CULL_LOG2 = 30.0   # the backward's bound: falloff below 2^-30 of the splat's nearest-pixel falloff, over the tile
KWHITEN2 = 0.5 / np.log(2.0)   # m = KWHITEN2 * maha: falloff exp(-maha / 2) = 2^-m


def tile_max_falloff(mu, sc, th, gid, st, H, W, TILE):
    """Per pair of the sorted list, the largest float64 falloff exp(-maha / 2) over its tile's pixel centres."""
    ntx = (W + TILE - 1) // TILE
    tile = np.repeat(np.arange(len(st) - 1), np.diff(st))
    ty, tx = tile // ntx, tile % ntx
    ly, lx = np.meshgrid(np.arange(TILE), np.arange(TILE), indexing="ij")
    yp = ty[:, None] * TILE + ly.reshape(-1)[None]
    xp = tx[:, None] * TILE + lx.reshape(-1)[None]
    inside = (yp < H) & (xp < W)
    py = ((yp.astype(np.float32) + 0.5) / H).astype(np.float64)
    px = ((xp.astype(np.float32) + 0.5) / W).astype(np.float64)
    g = gid[:len(tile)]
    dy, dx = py - mu[g, 0:1], px - mu[g, 1:2]
    c, s = np.cos(th[g])[:, None], np.sin(th[g])[:, None]
    ry, rx = c * dy + s * dx, -s * dy + c * dx
    maha = (ry / sc[g, 0:1]) ** 2 + (rx / sc[g, 1:2]) ** 2
    return np.where(inside, np.exp(-0.5 * maha), 0.0).max(axis=1)


def near_pixel_falloff(mu, sc, th, H, W):
    """Per splat, the float64 falloff at the centre of the canvas pixel that holds its centre (clamped to the
    canvas): the reference of the relative cut."""
    iy = np.clip(np.floor(mu[:, 0] * H), 0, H - 1)
    ix = np.clip(np.floor(mu[:, 1] * W), 0, W - 1)
    dy, dx = (iy + 0.5) / H - mu[:, 0], (ix + 0.5) / W - mu[:, 1]
    c, s = np.cos(th), np.sin(th)
    ry, rx = c * dy + s * dx, -s * dy + c * dx
    return np.exp(-0.5 * ((ry / sc[:, 0]) ** 2 + (rx / sc[:, 1]) ** 2))


def drop_pairs(gid, st, drop):
    """The pair list without the dropped pairs (same order), with its tile starts."""
    tile = np.repeat(np.arange(len(st) - 1), np.diff(st))
    keep = ~drop
    cnt = np.bincount(tile[keep], minlength=len(st) - 1)
    st2 = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    gid2 = gid[:len(tile)][keep].astype(np.int32)
    return (gid2 if gid2.size else np.zeros(1, np.int32)), st2


@pytest.mark.parametrize("odds", [False, True])
def test_falloff_rule_keeps_opacity_gradient(odds):
    H = W = 64
    (mu, ls, col, op, bg, th), low, logu = low_opacity_scene(400, H, W, seed=3, frac=0.1)
    mu, col, op, th = mu[0].numpy(), col[0].numpy(), op[0].numpy(), th[0].numpy()
    sc = R.activate_scale(ls[0]).numpy()
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    rng = np.random.default_rng(7)
    ups = dict(dslog=rng.standard_normal(H * W), dsa=rng.standard_normal(H * W),
               dsac=rng.standard_normal((H * W, 3)))
    args = (mu, sc, th, op, col)

    def g_op(gid_, st_):
        return c_oracle.bwd_cull(*args, gid_, st_, H, W, 8, odds=odds, fields=True, **ups)

    full = g_op(gid, st)
    m64 = [x.astype(np.float64) for x in (mu, sc, th)]
    fmax = tile_max_falloff(*m64, gid, st, H, W, 8)
    tile_of = np.repeat(np.arange(len(st) - 1), np.diff(st))
    thr = 2.0 ** -CULL_LOG2 * near_pixel_falloff(*m64, H, W)[gid[:len(tile_of)]]
    opp = op[gid[:len(tile_of)]].astype(np.float64)
    falloff_rule = drop_pairs(gid, st, fmax < thr)
    product_rule = drop_pairs(gid, st, opp * fmax < thr)
    kept = g_op(*falloff_rule)
    lost = g_op(*product_rule)
    e_kept, _ = per_splat_op_err(kept["op"], full["op"], full["op_scale"])
    e_lost, i = per_splat_op_err(lost["op"], full["op"], full["op_scale"])
    assert e_kept <= 1e-6, e_kept
    assert e_lost > 1e-2, e_lost                  # the planted mistake is caught per splat
    assert op[i] < 1e-3                           # on a near-transparent splat
    # the other gradients carry op * falloff: both rules keep them within the bar
    for name in ("mu", "scale", "col", "theta"):
        for got in (kept, lost):
            e = np.abs(got[name] - full[name]).max() / np.abs(full[name]).max()
            assert e <= 1e-6, (name, e)


def test_op_scale_bounds_the_gradient():
    """op_scale is the sum of the magnitudes of the opacity gradient's terms: |g_op| <= op_scale, with
    equality for a splat whose terms share one sign (a single splat under a uniform positive dS_log)."""
    H = W = 32
    (mu, ls, col, op, bg, th), _, _ = low_opacity_scene(120, H, W, seed=5)
    mu, col, op, th = mu[0].numpy(), col[0].numpy(), op[0].numpy(), th[0].numpy()
    sc = R.activate_scale(ls[0]).numpy()
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    rng = np.random.default_rng(1)
    ups = dict(dslog=rng.standard_normal(H * W), dsa=rng.standard_normal(H * W),
               dsac=rng.standard_normal((H * W, 3)))
    r = c_oracle.bwd_cull(mu, sc, th, op, col, gid, st, H, W, 8, fields=True, **ups)
    assert np.all(np.abs(r["op"]) <= r["op_scale"] * (1 + 1e-12))
    one = c_oracle.build_tiles(mu[:1], sc[:1], H, W, 8)
    z = np.zeros(H * W)
    r1 = c_oracle.bwd_cull(mu[:1], sc[:1], th[:1], op[:1] * 0 + 0.3, col[:1], *one, H, W, 8, fields=True,
                           dslog=-np.ones(H * W), dsa=z, dsac=np.zeros((H * W, 3)))
    assert r1["op"][0] > 0 and abs(r1["op"][0] - r1["op_scale"][0]) <= 1e-12 * r1["op_scale"][0]


def test_relative_cut_keeps_subpixel_splats():
    """Splats of 0.05 to 0.35 px among ordinary ones: the absolute cut (falloff below 2^-30 over the tile) fails the
    per-splat check on their scale gradients, the relative cut passes it."""
    from _scenes import per_splat_errors
    from _scenes import span_scene
    H = W = 96
    mu, ls, col, op, bg, th = span_scene(1500, H, W, seed=75, lo=8.5, hi=80.0, frac=0.7)
    mu, col, op, th = mu[0].numpy(), col[0].numpy(), op[0].numpy(), th[0].numpy()
    sc = R.activate_scale(ls[0]).numpy()
    gid, st = c_oracle.build_tiles(mu, sc, H, W, 8)
    rng = np.random.default_rng(7)
    ups = dict(dslog=rng.standard_normal(H * W), dsa=rng.standard_normal(H * W),
               dsac=rng.standard_normal((H * W, 3)))
    args = (mu, sc, th, op, col)
    full = c_oracle.bwd_cull(*args, gid, st, H, W, 8, fields=True, **ups)
    m64 = [x.astype(np.float64) for x in (mu, sc, th)]
    fmax = tile_max_falloff(*m64, gid, st, H, W, 8)
    n = len(fmax)
    rel = drop_pairs(gid, st, fmax < 2.0 ** -CULL_LOG2 * near_pixel_falloff(*m64, H, W)[gid[:n]])
    ab = drop_pairs(gid, st, fmax < 2.0 ** -CULL_LOG2)
    worst = lambda r: max(e for e, _ in per_splat_errors({k: r[k] for k in ("mu", "scale", "col", "op", "theta")},
                                                         full).values())
    assert worst(c_oracle.bwd_cull(*args, *rel, H, W, 8, fields=True, **ups)) <= 1e-7
    assert worst(c_oracle.bwd_cull(*args, *ab, H, W, 8, fields=True, **ups)) > 1e-4
