"""Colour channel counts other than 3. The kernels are instantiated for C = 1..4 (render_triton.py sizes its
colour blocks by next_pow2(C) and takes any count; every caller of the reference uses C = 3); the Python entry
points render more channels as chunks of at most 4 (render_hip._channel_chunks). Each count is checked against the
float64 oracle like C = 3 is: the culled render (alpha and odds), the exact render and the multi-level octave
render, image and the six gradients, at the same tolerances (image 1e-5 max-abs, gradients 1e-4 relative), and the
subsampled exact render against the full one. The upstream gradient has C channels."""

import numpy as np
import pytest
import torch

from _gpu_util import RH, random_scene
from test_gpu_api import compare, device_run, oracle_run

pytestmark = pytest.mark.gpu


def scene_c(C, n, H, W, seed, dev, **kw):
    """random_scene's splats with C colour channels and a C-channel background."""
    mu, ls, _, op, _, th = random_scene(n, H, W, seed=seed, dev=dev, **kw)
    g = torch.Generator().manual_seed(seed + 1000)
    col = torch.rand(1, n, C, generator=g).to(dev)
    bg = torch.rand(1, C, generator=g).to(dev)
    return [mu, ls, col, op, bg, th]


def gout_c(C, H, W, dev, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, C, H, W, generator=g).to(dev)


@pytest.mark.parametrize("C", [1, 2, 4, 5, 8])
@pytest.mark.parametrize("odds", [False, True])
def test_cull_channels(dev, C, odds):
    H = W = 48
    scene = scene_c(C, 500, H, W, seed=40 + C, dev=dev, op_max=0.95)
    gout = gout_c(C, H, W, dev, seed=C)
    out, g = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=True, odds=odds)
    assert out.shape == (1, C, H, W)
    ref, rg = oracle_run("cull", scene, gout, H, W, odds=odds)
    compare(out, g, ref, rg)


@pytest.mark.parametrize("C", [1, 4, 6])
def test_exact_channels(dev, C):
    H = W = 24
    scene = scene_c(C, 200, H, W, seed=50 + C, dev=dev, ls_mean_px=2.0)
    gout = gout_c(C, H, W, dev, seed=10 + C)
    out, g = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=False)
    ref, rg = oracle_run("exact", scene, gout, H, W)
    compare(out, g, ref, rg)


@pytest.mark.parametrize("C", [1, 2, 4, 5])
def test_octave_channels(dev, C):
    """Splats spanning several octaves (as test_gpu_api's multi-level test): the split coarse-level launches, the
    upsample inside the composite and its adjoint, for C channels."""
    H = W = 128
    g = torch.Generator().manual_seed(60 + C)
    n = 400
    sig = torch.exp(torch.rand(1, n, generator=g) * (np.log(0.31) - np.log(0.006)) + np.log(0.006))
    ls = torch.log(torch.exp(sig).clamp_min(1 + 1e-6) - 1.0).unsqueeze(-1).expand(1, n, 2).contiguous()
    mu = torch.rand(1, n, 2, generator=g)
    col = torch.rand(1, n, C, generator=g)
    op = torch.rand(1, n, generator=g) * 0.4
    th = torch.rand(1, n, generator=g) * 3.14159
    bg = torch.rand(1, C, generator=g)
    scene = [t.to(dev) for t in (mu, ls, col, op, bg, th)]
    gout = gout_c(C, H, W, dev, seed=20 + C)
    out, gd = device_run(RH.render_alpha_octave, scene, gout, H=H, W=W, odds=True)
    ref, rg = oracle_run("octave", scene, gout, H, W, odds=True)
    compare(out, gd, ref, rg)


def test_subsampled_channels(dev):
    """render_alpha_subsampled with 7 channels (chunks of 4 and 3) at given pixels against the full exact render of
    the same scene at those pixels (pixel centres (i + 0.5) / H there, linspace in the full render: 1 ulp apart),
    image and gradients, with a background of shape [1, C] over a batch of two."""
    from gaussian_splat_encoder import render as RN
    C, H, W = 7, 20, 28
    mu, ls, _, op, _, th = random_scene(150, H, W, seed=71, dev=dev, ls_mean_px=2.0, B=2)
    g = torch.Generator().manual_seed(72)
    scene = [mu, ls, torch.rand(2, 150, C, generator=g).to(dev), op, torch.rand(1, C, generator=g).to(dev), th]
    idx = torch.randint(0, H * W, (2, 300), generator=torch.Generator().manual_seed(5)).to(dev)
    gsub = torch.randn(2, C, 300, generator=torch.Generator().manual_seed(6)).to(dev)
    leaves = [t.detach().clone().requires_grad_(True) for t in scene]
    sub, px = RN.render_alpha_subsampled(*leaves[:5], H, W, theta=leaves[5], pixel_indices=idx)
    assert sub.shape == (2, C, 300) and torch.equal(px, idx)
    (sub * gsub).sum().backward()
    g_sub = [t.grad.clone() for t in leaves]
    leaves2 = [t.detach().clone().requires_grad_(True) for t in scene]
    full = RN.render_alpha_full(*leaves2[:5], H, W, theta=leaves2[5])
    picked = full.reshape(2, C, H * W).gather(2, idx.unsqueeze(1).expand(2, C, 300))
    assert (picked - sub).abs().max().item() <= 1e-5
    (picked * gsub).sum().backward()
    for a, b in zip(g_sub, [t.grad for t in leaves2]):
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 1e-4 * max(scale, 1e-9)
