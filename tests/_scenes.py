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


def per_splat_op_err(got, ref, scale, floor_frac=1e-7):
    """Largest per-splat error of an opacity gradient, relative to that splat's own scale: the summed
    magnitudes of the terms of its gradient (the oracle's op_scale), floored at floor_frac of the largest
    scale (splats whose every pixel-pair is negligible)."""
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    scale = np.asarray(scale, np.float64).reshape(-1)
    den = np.maximum(scale, floor_frac * max(scale.max(), 1e-300))
    r = np.abs(got - ref) / den
    i = int(np.argmax(r))
    return float(r[i]), i
