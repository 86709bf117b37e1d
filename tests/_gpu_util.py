"""Shared helpers of the GPU parity tests (imported by test_gpu_*.py)."""

import numpy as np
import torch

from gaussian_splat_encoder import render_hip as RH
from gaussian_splat_encoder.params import activate_scale

# Tolerances of the parity bar: rendered images max-abs per channel; gradients relative to the largest
# reference magnitude of each tensor (the reference self-tests' definition of "rel").
IMG_TOL = 1e-5
GRAD_REL_TOL = 1e-4
# Per-splat bar: every gradient component of every splat within 1e-4 of that splat's own scale for the component
# (the oracle's 'mag': the summed magnitudes of the terms entering it), floored at 1e-7 of the largest scale.
PER_SPLAT_TOL = 1e-4


def np_(t):
    return t.detach().float().cpu().numpy()


def rel_err(got, ref, floor=1e-9):
    """max |got - ref| / max |ref|. A reference that is identically zero up to float64 rounding (e.g. the
    rotation gradient of isotropic splats) is compared against `floor` instead."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64).reshape(got.shape)
    return np.abs(got - ref).max() / max(np.abs(ref).max(), floor)


def random_scene(n, H, W, seed, dev, ls_mean_px=2.5, ls_std=0.6, op_max=1.0, theta=True, B=1, margin=0.0):
    """Splats (optionally spilling `margin` beyond the canvas) with log-normal pixel sizes."""
    g = torch.Generator().manual_seed(seed)
    mu = torch.rand(B, n, 2, generator=g) * (1 + 2 * margin) - margin
    ls = np.log(ls_mean_px / max(H, W)) + ls_std * torch.randn(B, n, 2, generator=g)
    col = torch.rand(B, n, 3, generator=g)
    op = torch.rand(B, n, generator=g) * op_max
    bg = torch.rand(B, 3, generator=g)
    th = torch.rand(B, n, generator=g) * 3.14159 if theta else None
    mv = lambda t: None if t is None else t.float().to(dev)
    return mv(mu), mv(ls), mv(col), mv(op), mv(bg), mv(th)


def check_per_splat(got, gref, tol=PER_SPLAT_TOL):
    """Every gradient the oracle gives a per-splat scale for (mu, scale, col, op, theta), per splat and component.
    `got` maps names to device tensors with a batch dimension of 1 (None for an absent theta). Returns the
    errors by name."""
    from _scenes import per_splat_errors
    errs = per_splat_errors({k: None if v is None else np_(v[0]) for k, v in got.items()}, gref)
    worst = {k: f"{e:.2e} at splat {i // max(1, np.asarray(gref[k]).reshape(len(gref[k]), -1).shape[1])}"
             for k, (e, i) in errs.items() if e > tol}
    assert not worst, f"per-splat gradient errors above {tol:g} of the splat's scale: {worst}"
    print("per-splat errors (of each splat's scale):", {k: f"{e:.2e}" for k, (e, _) in errs.items()}, flush=True)
    return {k: e for k, (e, _) in errs.items()}


def device_bins(mu, scale, H, W, TILE=8, cutoff=3.0):
    gid_b, st_b, ntx, nt = RH._build_tiles(mu, scale, H, W, TILE, cutoff)
    return [g.cpu().numpy() for g in gid_b], [s.cpu().numpy() for s in st_b]


__all__ = ["IMG_TOL", "GRAD_REL_TOL", "PER_SPLAT_TOL", "np_", "rel_err", "random_scene", "device_bins",
           "check_per_splat", "activate_scale", "RH"]
