"""Parameters in other floating dtypes through render_alpha_full_triton(cull=True). The reference converts every
input to float32 for its kernels, returns a float32 image, and activates the scale in the log-scale's own dtype
(render_triton.py:134-142, :329); autograd hands each gradient back in its parameter's dtype. Here a log-scale that
is not float32 takes the path where torch activates it (the binning gets scales, not log-scales), so:
* float64 parameters: image and gradients against the float64 oracle at the parity bar (1e-5, 1e-4), the oracle
  binning with exactly the float32 scales the device bins with;
* bfloat16 parameters: the image at 1e-5 against the oracle on the same rounded values (the kernels see exactly
  those), the gradients, which autograd rounds to bfloat16, at 2e-2 relative.
Output dtype float32 and each gradient in its parameter's dtype, both cases."""

import numpy as np
import pytest
import torch

from _gpu_util import GRAD_REL_TOL, IMG_TOL, RH, np_, random_scene, rel_err
from oracle import render_ref as R

pytestmark = pytest.mark.gpu
NAMES = ["mu", "ls", "col", "op", "bg", "th"]


def oracle_from(scene_d, gout, H, W):
    """float64 oracle of the device's computation: every parameter's value as the kernels see it (float32 of the
    input), the scale activated in the input dtype as the device does, binned with its float32 value."""
    mu, ls, col, op, bg, th = [t[0] for t in scene_d]
    f64 = torch.float64
    cv = lambda t: t.detach().float().cpu().to(f64).requires_grad_(True)
    L = [cv(t) for t in (mu, ls, col, op, bg, th)]
    sc_dev = R.activate_scale(ls.detach()).float().cpu()          # what the binning and the kernels get
    sc64 = R.activate_scale(L[1]) if ls.dtype == torch.float64 else \
        sc_dev.to(f64) + (R.activate_scale(L[1]) - R.activate_scale(L[1]).detach())   # value as the device, grad of softplus
    gid, st = R._bin(L[0], sc_dev, H, W, 8, 3.0)
    out = R.cull_composite(L[0], sc64, L[2], L[3], L[4], L[5], gid, st, H, W, 8, False)[0]
    g = gout[0].permute(1, 2, 0).reshape(H * W, -1).cpu().to(f64)
    (out * g).sum().backward()
    img = out.detach().reshape(H, W, -1).permute(2, 0, 1)
    return img, {n: t.grad for n, t in zip(NAMES, L)}


@pytest.mark.parametrize("dtype", [torch.float64, torch.bfloat16])
def test_parameter_dtypes(dev, dtype):
    H = W = 48
    scene = random_scene(400, H, W, seed=71, dev=dev, op_max=0.9)
    scene_d = [t.to(dtype) for t in scene]
    leaves = [t.detach().clone().requires_grad_(True) for t in scene_d]
    g = torch.Generator().manual_seed(72)
    gout = torch.randn(1, 3, H, W, generator=g).to(dev)
    out = RH.render_alpha_full_triton(*leaves[:5], H, W, theta=leaves[5], cull=True)
    assert out.dtype == torch.float32 and out.shape == (1, 3, H, W)
    (out * gout).sum().backward()
    for n, t in zip(NAMES, leaves):
        assert t.grad is not None and t.grad.dtype == dtype, f"grad {n}: {None if t.grad is None else t.grad.dtype}"
    ref, rg = oracle_from(scene_d, gout, H, W)
    d = np.abs(np_(out[0]) - ref.numpy()).max()
    assert d <= IMG_TOL, f"image max-abs {d:.2e}"
    tol = GRAD_REL_TOL if dtype == torch.float64 else 2e-2
    for n, t in zip(NAMES, leaves):
        e = rel_err(np_(t.grad[0]), rg[n].numpy())
        assert e <= tol, f"grad {n}: rel {e:.2e}"
