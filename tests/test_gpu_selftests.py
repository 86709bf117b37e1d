"""The reference's own self-tests of the render (render_triton.py:983-1042, :1256-1428) on the device
path, with their shapes and tolerances. Their inputs came from the CUDA RNG and cannot be regenerated, so the
scenes are drawn here from seeded CPU generators with the same distributions:
* the culled render converges to the exact one as the cutoff grows (forward within 5e-3 at some cutoff of 3, 4, 5
  at TILE 16), and its gradients at cutoff 5 are within 1e-2 (relative, per tensor) of the exact backward's;
* the coarse/fine and octave renders approximate the exact full-resolution render (mean relative difference
  below 0.03), and their backward agrees with a central finite difference of the loss in one splat's position
  (relative 5e-2): a coarse splat for the split, the largest splat (deepest octave) for the octave render.
* the octave render at 1024, 1536 and 2048 pixels a side with 4 (H/8)^2 splats stays within the pair budget
  (render_triton.py:1405-1428), its pair total within 36 N; the coarse/fine render of the same kind of scene at
  1024 pixels a side stays below 20 GB of device memory (render_triton.py:1301-1331).
The finite differences sum the loss in float64 so that only the float32 render's own rounding enters them; the
octave render's is taken on the float64 oracle's render (its largest splat covers every pixel, so the float32
renders' rounding at every pixel enters the difference), the device render's own difference held to a bar that
allows for that rounding."""

import math

import pytest
import torch

from _gpu_util import RH, activate_scale
from test_gpu_levels import composed_oracle, octave_lv

pytestmark = pytest.mark.gpu
NAMES = ["mu", "ls", "col", "op", "bg", "th"]


def draw(shape_fns, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return [f(g).to(dev) for f in shape_fns]


def cull_scene(seed, ls_shift, dev, B=2, N=1024, C=3):
    return draw([lambda g: torch.rand(B, N, 2, generator=g),
                 lambda g: torch.rand(B, N, 2, generator=g) - ls_shift,
                 lambda g: torch.rand(B, N, C, generator=g),
                 lambda g: torch.rand(B, N, generator=g),
                 lambda g: torch.rand(B, C, generator=g),
                 lambda g: torch.rand(B, N, generator=g) * 3.14159], seed, dev)


def loss64(out, g):
    return (out.double() * g.double()).sum().item()


def test_cull_forward_converges_to_exact(dev):
    """render_triton.py:1020-1042: B 2, N 1,024, 64 x 64, log-scales U(-2.5, -1.5), TILE 16."""
    H = W = 64
    mu, ls, col, op, bg, th = cull_scene(2, 2.5, dev)
    exact = RH.render_alpha_full_triton(mu, ls, col, op, bg, H, W, theta=th, cull=False)
    diffs = []
    for cutoff in (3.0, 4.0, 5.0):
        cull = RH.render_alpha_full_triton(mu, ls, col, op, bg, H, W, theta=th, cull=True, TILE=16, cutoff=cutoff)
        diffs.append((cull - exact).abs().max().item())
    assert min(diffs) < 5e-3, diffs
    assert diffs[0] >= diffs[1] >= diffs[2], diffs   # the truncation shrinks as the cutoff grows


def test_cull_backward_matches_exact(dev):
    """render_triton.py:983-1017: B 2, N 1,024, 64 x 64, log-scales U(-2, -1), cutoff 5."""
    H = W = 64
    scene = cull_scene(3, 2.0, dev)
    g = torch.Generator().manual_seed(4)
    gC = torch.randn(2, 3, H, W, generator=g).to(dev)
    L = [t.clone().requires_grad_(True) for t in scene]
    out_ex = RH.render_alpha_full_triton(*L[:5], H, W, theta=L[5], cull=False)
    (out_ex * gC).sum().backward()
    L2 = [t.clone().requires_grad_(True) for t in scene]
    out_cu = RH.render_alpha_full_triton(*L2[:5], H, W, theta=L2[5], cull=True, cutoff=5.0)
    (out_cu * gC).sum().backward()
    assert (out_cu - out_ex).abs().max().item() < 5e-3
    for n, a, b in zip(NAMES, L2, L):
        rel = (a.grad - b.grad).abs().max().item() / (b.grad.abs().max().item() + 1e-12)
        assert rel < 1e-2, f"{n}: rel {rel:.2e}"


def test_multires_split_approximates_exact(dev):
    """render_triton.py:1256-1298: 64 coarse splats (sigma 0.12, about 15 px) and 512 fine ones (sigma 0.015) at
    128 x 128, coarse factor 8; finite difference on coarse splat 5's x position."""
    H = W = 128
    nc, nf = 64, 512
    n = nc + nf
    mu, col, op, bg, th = draw([lambda g: torch.rand(1, n, 2, generator=g),
                                lambda g: torch.rand(1, n, 3, generator=g),
                                lambda g: torch.rand(1, n, generator=g) * 0.5,
                                lambda g: torch.rand(1, 3, generator=g),
                                lambda g: torch.rand(1, n, generator=g) * 3.14159], 11, dev)
    ls = torch.empty(1, n, 2, device=dev)
    ls[:, :nc] = math.log(math.exp(0.12) - 1.0)
    ls[:, nc:] = math.log(math.exp(0.015) - 1.0)
    exact = RH.render_alpha_full_triton(mu, ls, col, op, bg, H, W, theta=th, cull=False)
    mr = lambda m: RH.render_alpha_multires(m, ls, col, op, bg, H, W, theta=th, n_coarse=nc, coarse_factor=8)
    rel = (mr(mu) - exact).abs().mean().item() / exact.abs().mean().item()
    assert rel < 0.03, rel
    g = torch.randn(1, 3, H, W, generator=torch.Generator().manual_seed(12)).to(dev)
    mu_g = mu.clone().requires_grad_(True)
    (mr(mu_g) * g).sum().backward()
    ana = mu_g.grad[0, 5, 0].item()
    eps = 1e-3
    mp, mm = mu.clone(), mu.clone()
    mp[0, 5, 0] += eps
    mm[0, 5, 0] -= eps
    fd = (loss64(mr(mp), g) - loss64(mr(mm), g)) / (2 * eps)
    assert abs(ana - fd) / (abs(fd) + 1e-6) < 5e-2, (ana, fd)


def test_octave_split_approximates_exact(dev):
    """render_triton.py:1370-1402: 800 splats at 256 x 256 with log-uniform sigma 0.006-0.31 (about 1.5 to 80
    px, six octaves); finite difference on the largest splat's x position."""
    H = W = 256
    n = 800
    g0 = torch.Generator().manual_seed(17)
    mu = torch.rand(1, n, 2, generator=g0)
    sig = torch.exp(torch.rand(1, n, generator=g0) * (math.log(0.31) - math.log(0.006)) + math.log(0.006))
    ls = torch.log(torch.exp(sig).clamp_min(1 + 1e-6) - 1.0).unsqueeze(-1).expand(1, n, 2).contiguous()
    col = torch.rand(1, n, 3, generator=g0)
    op = torch.rand(1, n, generator=g0) * 0.4
    th = torch.rand(1, n, generator=g0) * 3.14159
    bg = torch.rand(1, 3, generator=g0)
    mu, ls, col, op, th, bg = [t.to(dev) for t in (mu, ls, col, op, th, bg)]
    exact = RH.render_alpha_full_triton(mu, ls, col, op, bg, H, W, theta=th, cull=False)
    oc = lambda m: RH.render_alpha_octave(m, ls, col, op, bg, H, W, theta=th, cutoff=3.0)
    rel = (oc(mu) - exact).abs().mean().item() / exact.abs().mean().item()
    assert rel < 0.03, rel
    g = torch.randn(1, 3, H, W, generator=torch.Generator().manual_seed(18)).to(dev)
    mu_g = mu.clone().requires_grad_(True)
    (oc(mu_g) * g).sum().backward()
    j = int(sig[0].argmax())
    ana = mu_g.grad[0, j, 0].item()
    eps = 1e-3
    mp, mm = mu.clone(), mu.clone()
    mp[0, j, 0] += eps
    mm[0, j, 0] -= eps
    # The largest splat (80 px) covers every pixel, so the two float32 renders differ at all 196,608 of them by
    # their own rounding too (about 1e-5 of the loss between them, several % of a difference taken at eps = 1e-3):
    # the difference is taken on the float64 oracle's render of the same octave composition (same routing, same
    # culled pair lists), and the device's float32 one is held to the same bar with the noise allowed for.
    sc = activate_scale(ls)
    img = lambda m: composed_oracle(m[0], sc[0], col[0], op[0], bg[0], th[0], H, W, 8, octave_lv(), False,
                                    g[0].permute(1, 2, 0).reshape(H * W, 3))[0]
    gl = g[0].permute(1, 2, 0).reshape(H * W, 3).double().cpu().numpy()
    fd = float(((img(mp) - img(mm)) * gl).sum()) / (2 * eps)
    assert abs(ana - fd) / (abs(fd) + 1e-6) < 5e-2, (ana, fd)
    fd32 = (loss64(oc(mp), g) - loss64(oc(mm), g)) / (2 * eps)
    assert abs(ana - fd32) / (abs(fd) + 1e-6) < 0.15, (ana, fd32, fd)


@pytest.mark.parametrize("H", [1024, 1536, 2048])
def test_octave_probe_budget(dev, H):
    """render_triton.py:1405-1428: at H x H with 4 (H/8)^2 splats, half large (sigma 0.20) and half small (sigma
    0.018), the octave render's forward and backward stay within the 48M pair budget (no PairBudgetExceeded), its
    pair total within the 36 N the routing bounds it by, and its image and gradients finite."""
    W = H
    grid = (H // 8) * (W // 8)
    n = 4 * grid
    g = torch.Generator().manual_seed(0)
    mu = torch.rand(1, n, 2, generator=g).to(dev)
    ls = torch.empty(1, n, 2, device=dev)
    ls[:, :n // 2] = math.log(math.exp(0.20) - 1.0)
    ls[:, n // 2:] = math.log(math.exp(0.018) - 1.0)
    col = torch.rand(1, n, 3, generator=g).to(dev)
    op = torch.rand(1, n, generator=g).to(dev)
    bg = torch.rand(1, 3, generator=g).to(dev)
    L = [t.clone().requires_grad_(True) for t in (mu, ls, col, op, bg)]
    out = RH.render_alpha_octave(*L, H, W, max_pairs=48_000_000)
    out.float().pow(2).mean().backward()
    assert torch.isfinite(out).all()
    assert all(torch.isfinite(t.grad).all() for t in L)
    lv = RH._octave_levels(H, W, 8.0, 6)
    _, _, bins = RH._forward_levels(mu, ls, col, op, bg, None, H, W, 8, 3.0, 48_000_000, False, lv,
                                    with_maps=False, scale_is_log=True)
    assert 0 < bins.tot_b[0] <= 36 * n, (bins.tot_b[0], 36 * n)


def test_multires_probe_memory(dev):
    """render_triton.py:1301-1331: the coarse/fine render at 1024 x 1024 with 4 (H/8)^2 splats, the coarse half at
    sigma 0.20 (the initial scale whose full-resolution binning would need about 400M pairs), forward and backward
    with a peak of device memory below 20 GB (torch's allocator statistics), image and gradients finite."""
    H = W = 1024
    grid = (H // 8) * (W // 8)
    nc = nf = 2 * grid
    n = nc + nf
    g = torch.Generator().manual_seed(0)
    mu = torch.rand(1, n, 2, generator=g).to(dev)
    ls = torch.empty(1, n, 2, device=dev)
    ls[:, :nc] = math.log(math.exp(0.20) - 1.0)
    ls[:, nc:] = math.log(math.exp(0.018) - 1.0)
    col = torch.rand(1, n, 3, generator=g).to(dev)
    op = torch.rand(1, n, generator=g).to(dev)
    bg = torch.rand(1, 3, generator=g).to(dev)
    L = [t.clone().requires_grad_(True) for t in (mu, ls, col, op, bg)]
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    out = RH.render_alpha_multires(*L, H, W, n_coarse=nc, coarse_factor=8)
    out.float().pow(2).mean().backward()
    torch.cuda.synchronize(dev)
    peak = (torch.cuda.max_memory_allocated(dev) - base) / 1e9
    assert peak < 20.0, peak
    assert torch.isfinite(out).all() and all(torch.isfinite(t.grad).all() for t in L)
