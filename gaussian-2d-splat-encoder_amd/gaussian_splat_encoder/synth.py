"""Seeded synthetic splat sets for the benchmark configurations.

Every draw comes from a CPU ``torch.Generator`` in a fixed order (positions, log-scales, rotation, RGB,
opacity, then the heavy-tail subset, then the upstream gradient), so the same seed gives the same splats
on any machine and any device. Tensors are created on the CPU and moved afterwards.

Configurations:
  c0 : 64x64, 1,024 splats uniform over the canvas, log-scale ~ N(log 1.5 px, 0.4), opacity sigmoid(N(1,1)).
  c1 : 768x768, 92,160 splats, 10 per 8x8-pixel cell of a 96x96 grid with jitter inside the cell,
       log-scale ~ N(log 3 px, 0.5), opacity sigmoid(N(1.5, 1.5)).
  c2 : c1 plus an upstream image gradient ~ N(0, 1).
  c4 : 2048x2048, 655,360 splats (10 per cell on a 256x256 grid) as c1, with 2 % of the splats
       re-drawn at log-scale ~ N(log 40 px, 0.3) (the heavy tail that stresses binning balance).
"Log-scale ~ N(log k px, s)" means the raw log_scale = ln(k / H) + s * z, before softplus.
  procedural_image : the encoder input of config c3, a seeded RGB card (linear gradient, filled circles and
       rectangles) quantised to uint8 and returned as float in [0, 1].
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class SplatSet:
    mu: torch.Tensor          # [1, N, 2] (y, x) in [0, 1]
    log_scale: torch.Tensor   # [1, N, 2] raw (sy, sx)
    theta: torch.Tensor       # [1, N] radians
    color: torch.Tensor       # [1, N, 3]
    opacity: torch.Tensor     # [1, N]
    bg: torch.Tensor          # [1, 3]
    H: int
    W: int
    grad_out: Optional[torch.Tensor] = None   # [1, 3, H, W] upstream dL/dimage

    @property
    def n(self) -> int:
        return self.mu.shape[1]

    def to(self, device) -> "SplatSet":
        mv = lambda t: None if t is None else t.to(device)
        return SplatSet(mv(self.mu), mv(self.log_scale), mv(self.theta), mv(self.color), mv(self.opacity),
                        mv(self.bg), self.H, self.W, mv(self.grad_out))

    def args(self):
        """Positional arguments of the render entry points: (mu, log_scale, color, opacity, bg, H, W)."""
        return self.mu, self.log_scale, self.color, self.opacity, self.bg, self.H, self.W


def uniform_set(n: int, H: int, W: int, seed: int = 0, sigma_px: float = 1.5, ls_std: float = 0.4,
                op_mean: float = 1.0, op_std: float = 1.0) -> SplatSet:
    """Splats uniform over the canvas (config c0 with the defaults)."""
    g = torch.Generator("cpu").manual_seed(seed)
    mu = torch.rand(1, n, 2, generator=g)
    ls = math.log(sigma_px / H) + ls_std * torch.randn(1, n, 2, generator=g)
    th = math.pi * torch.rand(1, n, generator=g)
    rgb = torch.rand(1, n, 3, generator=g)
    op = torch.sigmoid(op_mean + op_std * torch.randn(1, n, generator=g))
    return SplatSet(mu, ls, th, rgb, op, torch.zeros(1, 3), H, W)


def grid_set(H: int, per_cell: int = 10, cell: int = 8, seed: int = 0, sigma_px: float = 3.0,
             ls_std: float = 0.5, op_mean: float = 1.5, op_std: float = 1.5, heavy_frac: float = 0.0,
             heavy_sigma_px: float = 40.0, heavy_std: float = 0.3, with_grad: bool = False) -> SplatSet:
    """`per_cell` splats in every `cell`x`cell` pixel cell of a square canvas (configs c1, c2 and c4).

    Splat index is (cy * G + cx) * per_cell + m, the cell-major order the encoder emits.
    """
    W = H
    G = H // cell
    n = G * G * per_cell
    g = torch.Generator("cpu").manual_seed(seed)
    cy = torch.arange(G).repeat_interleave(G * per_cell)
    cx = torch.arange(G).repeat_interleave(per_cell).repeat(G)
    cell_yx = torch.stack([cy, cx], dim=-1).float().unsqueeze(0)           # [1, N, 2]
    mu = ((cell_yx + torch.rand(1, n, 2, generator=g)) * cell) / H
    ls = math.log(sigma_px / H) + ls_std * torch.randn(1, n, 2, generator=g)
    th = math.pi * torch.rand(1, n, generator=g)
    rgb = torch.rand(1, n, 3, generator=g)
    op = torch.sigmoid(op_mean + op_std * torch.randn(1, n, generator=g))
    if heavy_frac > 0.0:
        k = int(round(heavy_frac * n))
        idx = torch.randperm(n, generator=g)[:k]
        ls[0, idx] = math.log(heavy_sigma_px / H) + heavy_std * torch.randn(k, 2, generator=g)
    gout = torch.randn(1, 3, H, W, generator=g) if with_grad else None
    return SplatSet(mu, ls, th, rgb, op, torch.zeros(1, 3), H, W, gout)


def config(name: str, seed: int = 0) -> SplatSet:
    """The named benchmark configuration ('c0', 'c1', 'c2', 'c4'), generated on the CPU."""
    if name == "c0":
        return uniform_set(1024, 64, 64, seed=seed)
    if name == "c1":
        return grid_set(768, seed=seed)
    if name == "c2":
        return grid_set(768, seed=seed, with_grad=True)
    if name == "c4":
        return grid_set(2048, seed=seed, heavy_frac=0.02, with_grad=True)
    raise ValueError(f"unknown config {name!r}")


def procedural_image(H: int, W: int, seed: int = 0, n_shapes: int = 24) -> torch.Tensor:
    """[1, 3, H, W] float in [0, 1]: a linear colour gradient in a random direction with `n_shapes` filled
    circles and axis-aligned rectangles of random colour on top, quantised to uint8 (config c3's input)."""
    g = torch.Generator().manual_seed(seed)
    yy, xx = torch.meshgrid((torch.arange(H) + 0.5) / H, (torch.arange(W) + 0.5) / W, indexing="ij")
    c0, c1 = torch.rand(3, generator=g), torch.rand(3, generator=g)
    ang = float(torch.rand(1, generator=g)) * 2 * math.pi
    t = math.cos(ang) * xx + math.sin(ang) * yy
    t = (t - t.min()) / (t.max() - t.min())
    img = c0[:, None, None] * (1 - t) + c1[:, None, None] * t
    for _ in range(n_shapes):
        kind = int(torch.randint(0, 2, (1,), generator=g))
        col = torch.rand(3, generator=g)
        cy, cx = torch.rand(2, generator=g).tolist()
        a, b = (0.02 + 0.15 * torch.rand(2, generator=g)).tolist()
        if kind == 0:
            m = (yy - cy) ** 2 + (xx - cx) ** 2 < a * a
        else:
            m = ((yy - cy).abs() < a) & ((xx - cx).abs() < b)
        img[:, m] = col[:, None]
    u8 = (img * 255).round().clamp(0, 255).to(torch.uint8)
    return (u8.float() / 255).unsqueeze(0)
