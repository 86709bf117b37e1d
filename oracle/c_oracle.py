"""ctypes binding of oracle.c. TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Builds _build/liboracle.so with the Makefile next to this file on first use if it is missing.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_pairs.restype = ctypes.c_int64
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class rot32:
    """Within this context the oracle rounds each splat's cos and sin to the nearest float32 values (the precision
    in which the reference and the HIP decode hold the rotation); outside it they stay float64."""

    def __enter__(self):
        lib().orc_set_rot32(1)
        return self

    def __exit__(self, *exc):
        lib().orc_set_rot32(0)
        return False


class off32:
    """Within this context the oracle rounds each pixel centre's offsets from a splat centre to float32, as the
    reference's float32 arithmetic and the kernels form them; outside it they are exact."""

    def __enter__(self):
        lib().orc_set_off32(1)
        return self

    def __exit__(self, *exc):
        lib().orc_set_off32(0)
        return False


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def rects(mu, scale, H, W, TILE=8, cutoff=3.0):
    mu, scale = _f32(mu), _f32(scale)
    n = mu.shape[0]
    out = [np.empty(n, np.int32) for _ in range(5)]
    lib().orc_rects(_p(mu), _p(scale), ctypes.c_int(n), ctypes.c_int(H), ctypes.c_int(W), ctypes.c_int(TILE),
                    ctypes.c_float(cutoff), *[_p(o) for o in out])
    return tuple(out)   # tx0, tx1, ty0, ty1, counts


def build_tiles(mu, scale, H, W, TILE=8, cutoff=3.0):
    """(gid_sorted, tile_starts) for one batch via rects + counting sort; tot == 0 gives gid = [0]."""
    tx0, tx1, ty0, ty1, counts = rects(mu, scale, H, W, TILE, cutoff)
    ntx = (W + TILE - 1) // TILE
    nt = ntx * ((H + TILE - 1) // TILE)
    tot = int(counts.astype(np.int64).sum())
    gid = np.zeros(max(tot, 1), np.int32)
    starts = np.zeros(nt + 1, np.int32)
    if tot:
        got = lib().orc_pairs(_p(tx0), _p(tx1), _p(ty0), _p(ty1), ctypes.c_int(len(counts)), ctypes.c_int(ntx),
                              ctypes.c_int(nt), _p(gid), _p(starts))
        assert got == tot
    return gid, starts


def fwd_cull(mu, scale, theta, opacity, color, gid, starts, H, W, TILE=8, odds=False, fields=False, bg=None,
             cond=False):
    """float64 cull forward of one batch. Returns (S_log, S_a, S_ac) if fields else (out, T, asum, fg). cond (with
    fields): also return the fields' sensitivities to a relative change of every unclamped alpha, (K_log, K_a,
    K_ac) = (sum a / (1 - a), sum a dw/da, sum |c| a dw/da) per pixel, as a fourth element."""
    mu, scale, theta, opacity, color = map(_f32, (mu, scale, theta, opacity, color))
    C = color.shape[1]
    P = H * W
    gid = np.ascontiguousarray(gid, np.int32)
    starts = np.ascontiguousarray(starts, np.int32)
    bg = _f32(np.zeros(C) if bg is None else bg)
    a = [np.zeros(P * C), np.zeros(P), np.zeros(P), np.zeros(P * C)]
    f = [np.zeros(P), np.zeros(P), np.zeros(P * C)]
    lib().orc_fwd_cull(_p(mu), _p(scale), _p(theta), _p(opacity), _p(color), ctypes.c_int(C), _p(gid), _p(starts),
                       ctypes.c_int(H), ctypes.c_int(W), ctypes.c_int(TILE), ctypes.c_int(int(odds)),
                       ctypes.c_int(int(fields)), _p(bg), *[_p(x) for x in a], *[_p(x) for x in f])
    if fields:
        return (f[0], f[1], f[2].reshape(P, C)) + (((a[1], a[2], a[3].reshape(P, C)),) if cond else ())
    return a[0].reshape(P, C), a[1], a[2], a[3].reshape(P, C)


def bwd_cull(mu, scale, theta, opacity, color, gid, starts, H, W, TILE=8, odds=False, fields=False, bg=None,
             T=None, asum=None, fg=None, gout=None, dslog=None, dsa=None, dsac=None):
    """float64 cull backward of one batch -> dict of per-splat grads (+ 'bg' in composite mode), plus
    'mag': per splat, for every gradient by name (mu, scale, theta, op, col; same shapes as the gradients) the
    summed magnitudes of the terms of that gradient component, the scale of a per-splat relative check (see
    orc_bwd_cull); 'op_scale' is mag['op']."""
    mu, scale, theta, opacity, color = map(_f32, (mu, scale, theta, opacity, color))
    n, C = color.shape
    d64 = lambda x: None if x is None else np.ascontiguousarray(x, np.float64).reshape(-1)
    bg = _f32(np.zeros(C) if bg is None else bg)
    g_mu, g_sc = np.zeros(2 * n), np.zeros(2 * n)
    g_th = np.zeros(n) if theta is not None else None
    g_op, g_col = np.zeros(n), np.zeros(n * C)
    g_bg = None if fields else np.zeros(C)
    KG = 6 + C
    g_mag = np.zeros(n * KG)
    lib().orc_bwd_cull(_p(mu), _p(scale), _p(theta), _p(opacity), _p(color), ctypes.c_int(C), ctypes.c_int(n),
                       _p(np.ascontiguousarray(gid, np.int32)), _p(np.ascontiguousarray(starts, np.int32)),
                       ctypes.c_int(H), ctypes.c_int(W), ctypes.c_int(TILE), ctypes.c_int(int(odds)),
                       ctypes.c_int(int(fields)), _p(bg), _p(d64(T)), _p(d64(asum)), _p(d64(fg)), _p(d64(gout)),
                       _p(d64(dslog)), _p(d64(dsa)), _p(d64(dsac)), _p(g_mu), _p(g_sc), _p(g_th), _p(g_op),
                       _p(g_col), _p(g_bg), _p(g_mag))
    m = g_mag.reshape(n, KG)
    mag = {"mu": m[:, 0:2].copy(), "scale": m[:, 2:4].copy(), "op": m[:, 5].copy(), "col": m[:, 6:].copy()}
    out = {"mu": g_mu.reshape(n, 2), "scale": g_sc.reshape(n, 2), "op": g_op, "col": g_col.reshape(n, C),
           "op_scale": mag["op"], "mag": mag}
    if g_th is not None:
        out["theta"] = g_th
        mag["theta"] = m[:, 4].copy()
    if g_bg is not None:
        out["bg"] = g_bg
    return out


def exact_rows_f32(mu, scale, theta, opacity, color, ys, xs, row0, row1, bg):
    """render.py's exact fp32 math over rows [row0, row1) of the canvas; returns [rows, W, C]."""
    mu, scale, theta, opacity, color, ys, xs, bg = map(_f32, (mu, scale, theta, opacity, color, ys, xs, bg))
    n, C = color.shape
    W = xs.shape[0]
    out = np.zeros((row1 - row0) * W * C, np.float32)
    lib().orc_exact_rows_f32(_p(mu), _p(scale), _p(theta), _p(opacity), _p(color), ctypes.c_int(C), ctypes.c_int(n),
                             _p(ys), _p(xs), ctypes.c_int(row0), ctypes.c_int(row1), ctypes.c_int(W), _p(bg), _p(out))
    return out.reshape(row1 - row0, W, C)
