"""numpy restatement of the reference's splat->tile binning. TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Follows gaussian_splat_encoder/render_triton.py:351-409 (`_build_tiles`) op by op. Every arithmetic step
is one separately rounded float32 operation, as in the reference's elementwise torch ops:

    cx = fl(mu_x * W)              cy = fl(mu_y * H)                         (:367-368)
    r  = fl(cutoff * max(sy, sx))                                           (:369)
    rx = fl(r * W)                 ry = fl(r * H)                           (:370-371)
    tx0 = int(clamp(floor(fl(fl(cx - rx) / TILE)), 0, ntx - 1))             (:372)
    tx1 = int(clamp(floor(fl(fl(cx + rx) / TILE)), 0, ntx - 1))             (:373)
    ty0, ty1 likewise with cy, ry, nty                                      (:374-375)
    count = (tx1 - tx0 + 1) * (ty1 - ty0 + 1)                               (:376-377)

Pairs are generated splat-major (k = 0..count-1 walks the rect row by row, :396-404) and ordered by
(tile, splat): a stable sort on the tile id of the splat-major list (:405-407). tile_starts[t] is the
number of pairs whose tile is < t (:408). A batch with no pairs gets gid = [0] and all-zero starts (:392-395).
"""

from __future__ import annotations

import numpy as np


def tile_grid(H: int, W: int, TILE: int):
    ntx = (W + TILE - 1) // TILE
    nty = (H + TILE - 1) // TILE
    return ntx, nty, ntx * nty


def rects(mu: np.ndarray, scale: np.ndarray, H: int, W: int, TILE: int, cutoff: float):
    """Per-splat tile rect (tx0, tx1, ty0, ty1) and count, float32 arithmetic. mu, scale: [N, 2] (y, x)."""
    f32 = np.float32
    mu = np.ascontiguousarray(mu, dtype=f32)
    scale = np.ascontiguousarray(scale, dtype=f32)
    ntx, nty, _ = tile_grid(H, W, TILE)
    cx = mu[:, 1] * f32(W)
    cy = mu[:, 0] * f32(H)
    r = f32(cutoff) * np.maximum(scale[:, 0], scale[:, 1])
    rx = r * f32(W)
    ry = r * f32(H)
    T = f32(TILE)

    def edge(v, hi):
        return np.clip(np.floor(v / T), f32(0), f32(hi)).astype(np.int32)

    tx0 = edge(cx - rx, ntx - 1)
    tx1 = edge(cx + rx, ntx - 1)
    ty0 = edge(cy - ry, nty - 1)
    ty1 = edge(cy + ry, nty - 1)
    counts = ((tx1 - tx0 + 1) * (ty1 - ty0 + 1)).astype(np.int32)
    return tx0, tx1, ty0, ty1, counts


def build_tiles(mu: np.ndarray, scale: np.ndarray, H: int, W: int, TILE: int = 8, cutoff: float = 3.0,
                return_keys: bool = False):
    """One batch: (gid_sorted int32 [tot] or [1], tile_starts int32 [nt+1]); optionally the sorted tile ids."""
    ntx, nty, nt = tile_grid(H, W, TILE)
    tx0, tx1, ty0, ty1, counts = rects(mu, scale, H, W, TILE, cutoff)
    tot = int(counts.astype(np.int64).sum())
    if tot == 0:
        gid = np.zeros(1, np.int32)
        starts = np.zeros(nt + 1, np.int32)
        return (gid, starts, np.zeros(0, np.int32)) if return_keys else (gid, starts)
    n = counts.shape[0]
    gid = np.repeat(np.arange(n, dtype=np.int32), counts)
    start = (np.cumsum(counts.astype(np.int64)) - counts).astype(np.int64)
    k = np.arange(tot, dtype=np.int64) - start[gid]
    w = (tx1 - tx0 + 1)[gid].astype(np.int64)
    tile = (ty0[gid] + k // w) * ntx + (tx0[gid] + k % w)
    order = np.argsort(tile, kind="stable")
    tile_s = tile[order].astype(np.int32)
    gid_s = gid[order].astype(np.int32)
    starts = np.searchsorted(tile_s, np.arange(nt + 1), side="left").astype(np.int32)
    if return_keys:
        return gid_s, starts, tile_s
    return gid_s, starts
