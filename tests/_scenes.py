"""Scene generators and checks shared by the CPU and GPU tests (pure torch / numpy; no device code)."""

import math

import numpy as np
import torch

# The opacities of near-transparent splats drawn by low_opacity_scene: exact zeros and the decades that the
# released checkpoint's coarse layer emits (median 1e-5, minimum about 4e-11).
LOW_OPACITIES = (0.0, 1e-10, 1e-8, 1e-6, 1e-4)


def inverse_activation(sigma):
    """Raw log-scale x with softplus(x) + 1e-4 = sigma (params.py:18-28), for sigma > 1e-4."""
    y = sigma - 1e-4
    return torch.where(y > 20, y, torch.log(torch.expm1(y)))


def low_opacity_scene(n, H, W, seed, frac=0.05, sigma_px=(5.0, 40.0), ls_mean_px=3.0, ls_std=0.5, op_max=0.95,
                      theta=True):
    """A random scene (log-normal sizes around ls_mean_px, opacities uniform in [0, op_max)) in which a
    fraction `frac` of the splats are near-transparent and large: opacity drawn from LOW_OPACITIES, sizes
    log-uniform in sigma_px per axis; another `frac` get log-uniform opacities in [1e-12, 1].
    Returns CPU float32 (mu, log_scale, color, opacity, bg, theta) with a batch dimension of 1, and the
    indices of the two subsets."""
    g = torch.Generator().manual_seed(seed)
    mu = torch.rand(1, n, 2, generator=g)
    ls = math.log(ls_mean_px / max(H, W)) + ls_std * torch.randn(1, n, 2, generator=g)
    col = torch.rand(1, n, 3, generator=g)
    op = torch.rand(1, n, generator=g) * op_max
    bg = torch.rand(1, 3, generator=g)
    th = torch.rand(1, n, generator=g) * math.pi if theta else None
    perm = torch.randperm(n, generator=g)
    k = max(1, int(round(frac * n)))
    low, logu = perm[:k], perm[k:2 * k]
    op[0, low] = torch.tensor(LOW_OPACITIES, dtype=torch.float32)[torch.randint(0, len(LOW_OPACITIES), (k,),
                                                                                 generator=g)]
    lo, hi = math.log(sigma_px[0]), math.log(sigma_px[1])
    sig = torch.exp(lo + (hi - lo) * torch.rand(k, 2, generator=g)) / max(H, W)
    ls[0, low] = inverse_activation(sig.double()).float()
    op[0, logu] = (10.0 ** (-12.0 * torch.rand(k, generator=g, dtype=torch.float64))).float()
    return (mu, ls, col, op, bg, th), low.numpy(), logu.numpy()


def per_splat_err(got, ref, scale, floor_frac=1e-7):
    """Largest per-splat error of a gradient, component by component, relative to that splat's own scale for the
    component: the summed magnitudes of the terms of its gradient (the oracle's 'mag'), floored at floor_frac of the
    component's largest scale over the splats (splats whose every pixel-pair is negligible). Returns the error
    and the flat index (splat * components + component) where it is largest."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64).reshape(got.shape)
    scale = np.asarray(scale, np.float64).reshape(got.shape)
    if got.size == 0:
        return 0.0, 0
    g2, r2, s2 = (a.reshape(got.shape[0], -1) for a in (got, ref, scale))
    den = np.maximum(s2, floor_frac * np.maximum(s2.max(axis=0, keepdims=True), 1e-300))
    r = (np.abs(g2 - r2) / den).reshape(-1)
    i = int(np.argmax(r))
    return float(r[i]), i


def per_splat_op_err(got, ref, scale, floor_frac=1e-7):
    """per_splat_err of an opacity gradient [N] (the oracle's op_scale as the scale); returns (error, splat)."""
    return per_splat_err(np.asarray(got).reshape(-1), ref, scale, floor_frac)


# gradient names of the per-pair backward and whether the oracle gives a magnitude scale for them
PER_SPLAT_NAMES = ("mu", "scale", "col", "op", "theta")


def per_splat_errors(got, gref, names=PER_SPLAT_NAMES, floor_frac=1e-7):
    """{name: (error, flat index)} of per_splat_err for every gradient the oracle's 'mag' covers; `got` maps names
    to arrays of the oracle's shapes (None for an absent theta)."""
    out = {}
    for name in names:
        if got.get(name) is None or name not in gref["mag"]:
            continue
        out[name] = per_splat_err(got[name], gref[name], gref["mag"][name], floor_frac)
    return out


KWHITEN = math.sqrt(0.5 / math.log(2.0))   # u = KWHITEN * (rotated offset) / sigma: falloff exp2(-(u^2 + v^2))


def spans(mu, sc, th, H, W, TILE=8):
    """Per splat, the whitened half-span over a TILE x TILE tile: max over u and v of the largest change from the
    tile centre to its corner pixel centres (the kernel's moment_span_ok)."""
    sy, sx = sc[:, 0].astype(np.float64), sc[:, 1].astype(np.float64)
    c, s = np.abs(np.cos(th)), np.abs(np.sin(th))
    cy, cx = 0.5 * (TILE - 1) / H, 0.5 * (TILE - 1) / W
    su = KWHITEN * (c * cy + s * cx) / sy
    sv = KWHITEN * (s * cy + c * cx) / sx
    return np.maximum(su, sv)


def span_scene(n, H, W, seed, lo=5.0, hi=11.0, frac=0.6):
    """A scene in which a fraction `frac` of the splats have spans log-uniform in [lo, hi] over an 8 x 8 tile (their
    smaller sigma set from the drawn span and rotation, the other axis 1 to 12 times larger), the rest ordinary
    splats of a few pixels. CPU float32 tensors with a batch dimension of 1."""
    g = torch.Generator().manual_seed(seed)
    mu = torch.rand(1, n, 2, generator=g)
    th = torch.rand(1, n, generator=g) * math.pi
    sig_px = torch.exp(math.log(3.0) + 0.5 * torch.randn(1, n, 2, generator=g))
    k = int(frac * n)
    span = torch.exp(math.log(lo) + (math.log(hi) - math.log(lo)) * torch.rand(k, generator=g, dtype=torch.float64))
    t = th[0, :k].double()
    cs = torch.cos(t).abs() + torch.sin(t).abs()
    small = KWHITEN * cs * 3.5 / span          # sigma in pixels of the narrow axis (square canvas, 8 x 8 tiles)
    ratio = torch.exp(math.log(12.0) * torch.rand(k, generator=g, dtype=torch.float64))
    which = torch.rand(k, generator=g) < 0.5
    sy = torch.where(which, small, small * ratio)
    sx = torch.where(which, small * ratio, small)
    sig_px[0, :k, 0], sig_px[0, :k, 1] = sy.float(), sx.float()
    ls = inverse_activation((sig_px.double() / max(H, W))).float()
    col = torch.rand(1, n, 3, generator=g)
    op = 0.05 + 0.9 * torch.rand(1, n, generator=g)
    bg = torch.rand(1, 3, generator=g)
    return mu, ls, col, op, bg, th
