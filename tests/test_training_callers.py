"""The training-side callers of the renderer (CPU): the edge-weighted pixel sampler
(efficient_encoder.py:122-141) and the 9-channel parameter assembly (params.py:31-41)."""

import numpy as np
import pytest
import torch
from scipy import stats

from gaussian_splat_encoder.efficient_encoder import edge_pixel_indices, sobel_gradmag
from gaussian_splat_encoder.params import SCALE_EPS, activate_scale, assemble_gaussian_params


def sobel_numpy(img):
    """|grad| of the channel mean by the Sobel / 4 stencils with zero padding, + 1e-6 under the root, float64:
    gx[y, x] = sum_ij kx[i, j] gray[y + i - 1, x + j - 1] (cross-correlation, as conv2d computes it)."""
    gray = img.astype(np.float64).mean(axis=0)
    H, W = gray.shape
    p = np.zeros((H + 2, W + 2))
    p[1:-1, 1:-1] = gray
    kx = np.array([[-1.0, 0.0, 1.0], [-2.0, 0.0, 2.0], [-1.0, 0.0, 1.0]]) / 4.0
    gx = sum(kx[i, j] * p[i:i + H, j:j + W] for i in range(3) for j in range(3))
    gy = sum(kx.T[i, j] * p[i:i + H, j:j + W] for i in range(3) for j in range(3))
    return np.sqrt(gx * gx + gy * gy + 1e-6)


def card(H=16, W=16, seed=0):
    """A fixed image with a sharp vertical edge, a bright square and a little noise: a strongly non-uniform
    gradient magnitude."""
    g = torch.Generator().manual_seed(seed)
    img = torch.zeros(3, H, W)
    img[:, :, W // 2:] = 0.8
    img[0, 3:7, 2:6] = 1.0
    img += 0.02 * torch.rand(3, H, W, generator=g)
    return img


def test_sobel_matches_stencil():
    img = card()
    got = sobel_gradmag(img[None])[0, 0].double().numpy()
    assert np.allclose(got, sobel_numpy(img.numpy()), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("lam", [0.0, 0.3])
def test_edge_sampler_distribution(lam):
    """Empirical frequencies of many draws against (1 - lam) |grad I| / sum + lam / (H W), by a chi-square test;
    a plausible mistake in the law (|grad I|^2 for |grad I|) is rejected by the same test."""
    img = card()
    H, W = img.shape[1:]
    g = sobel_numpy(img.numpy()).reshape(-1)
    pmf = (1 - lam) * g / g.sum() + lam / (H * W)
    torch.manual_seed(1)
    B = 800   # H W = 256 draws per image (the cap), 204,800 in all
    idx = edge_pixel_indices(img[None].expand(B, -1, -1, -1).contiguous(), H * W, lam)
    assert idx.shape == (B, H * W) and idx.dtype == torch.int64
    assert int(idx.min()) >= 0 and int(idx.max()) < H * W
    cnt = np.bincount(idx.reshape(-1).numpy(), minlength=H * W)
    assert stats.chisquare(cnt, pmf * cnt.sum()).pvalue > 1e-3
    wrong = (1 - lam) * g ** 2 / (g ** 2).sum() + lam / (H * W)
    assert stats.chisquare(cnt, wrong * cnt.sum()).pvalue < 1e-9


def test_edge_sampler_uniform_limit_and_size_cap():
    """lam = 1 is uniform over the pixels; more draws than pixels are capped at H W per image."""
    img = card(8, 12)
    torch.manual_seed(2)
    idx = edge_pixel_indices(img[None], 10_000, 1.0)
    assert idx.shape == (1, 8 * 12)
    idx = torch.cat([edge_pixel_indices(img[None], 96, 1.0) for _ in range(600)], dim=1)
    cnt = np.bincount(idx.reshape(-1).numpy(), minlength=96)
    assert stats.chisquare(cnt).pvalue > 1e-3


def test_assemble_gaussian_params_layout():
    g = torch.Generator().manual_seed(0)
    B, N = 2, 5
    enc = {"mu": torch.rand(B, N, 2, generator=g), "log_scale": torch.randn(B, N, 2, generator=g),
           "theta": torch.rand(B, N, generator=g), "color": torch.rand(B, N, 3, generator=g),
           "opacity": torch.rand(B, N, generator=g)}
    p = assemble_gaussian_params(enc)
    assert p.shape == (B, N, 9)
    assert torch.equal(p[..., 0:2], enc["mu"]) and torch.equal(p[..., 2:4], enc["log_scale"])
    assert torch.equal(p[..., 4], enc["theta"]) and torch.equal(p[..., 5:8], enc["color"])
    assert torch.equal(p[..., 8], enc["opacity"])
    # defaults: no rotation -> 0, no opacity -> 1
    q = assemble_gaussian_params(dict(enc, theta=None, opacity=None))
    assert torch.equal(q[..., 4], torch.zeros(B, N)) and torch.equal(q[..., 8], torch.ones(B, N))
    assert torch.equal(q[..., :4], p[..., :4]) and torch.equal(q[..., 5:8], p[..., 5:8])


def test_activate_scale_values():
    x = torch.tensor([-30.0, -2.0, 0.0, 3.0, 19.0, 21.0, 40.0])
    sp = np.log1p(np.exp(x.double().numpy()))
    ref = np.where(x.numpy() > 20, x.numpy().astype(np.float64), sp) + SCALE_EPS
    assert np.allclose(activate_scale(x).double().numpy(), ref, rtol=1e-6, atol=1e-9)
    assert float(activate_scale(torch.tensor(-100.0))) == pytest.approx(SCALE_EPS, rel=1e-6)
