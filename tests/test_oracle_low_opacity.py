"""The backward's negligible-pair rule against near-transparent splats, on the CPU oracle.

The per-tile backward gives a pair a zero record when the pair's contribution is negligible at every pixel of
the tile. The opacity gradient g_op = sum da * falloff (render_triton.py:697-698) carries no opacity factor, so
the rule must look at the falloff alone: a rule on opacity * falloff drops the far tiles of near-transparent
splats from their opacity gradient. Here both rules are planted in the float64 C oracle (the dropped pairs
are removed from its pair list) and held to the per-splat check of the GPU tests: the falloff rule passes
it, the opacity * falloff rule fails it by orders of magnitude.
"""

import numpy as np
import pytest

from _scenes import low_opacity_scene, per_splat_op_err
from oracle import c_oracle
from oracle import render_ref as R

CULL_LOG2 = 30.0   # the backward's bound: falloff (or op * falloff) below 2^-30 at every pixel of the tile


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
    fmax = tile_max_falloff(mu.astype(np.float64), sc.astype(np.float64), th.astype(np.float64), gid, st, H, W, 8)
    thr = 2.0 ** -CULL_LOG2
    tile_of = np.repeat(np.arange(len(st) - 1), np.diff(st))
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
