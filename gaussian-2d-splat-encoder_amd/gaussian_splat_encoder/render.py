"""The reference's render.py entry points (render.py:61-110) on the HIP exact path.

render_alpha_full and render_alpha_subsampled evaluate every splat at every requested pixel with the same
math as the reference's materialised renderer, through the exact-path kernels (O(P) memory; nothing of
size P x N is materialised). Pixel centres follow render.py: torch.linspace for full frames (:61-65),
((index // W) + 0.5) / H for subsampled pixels (:81-82).
"""

from __future__ import annotations

import torch


def _pixels(H, W, device, dtype):
    """render.py:61-65: [H*W, 2] (y, x) pixel centres from linspace."""
    ys = torch.linspace(0.5 / H, 1 - 0.5 / H, H, device=device, dtype=dtype)
    xs = torch.linspace(0.5 / W, 1 - 0.5 / W, W, device=device, dtype=dtype)
    gy, gx = torch.meshgrid(ys, xs, indexing="ij")
    return torch.stack([gy, gx], dim=-1).reshape(H * W, 2)


def render_alpha_full(mu, log_scale, color, opacity, bg, H, W, theta=None, chunk_pixels=4096):
    """render.py:90-110: full-resolution exact render -> [B,C,H,W]. `chunk_pixels` is accepted for signature
    compatibility; the kernels never materialise the [P, N] falloff, so no chunking is needed."""
    from .render_hip import render_alpha_full_triton
    return render_alpha_full_triton(mu, log_scale, color, opacity, bg, H, W, theta=theta, cull=False)


def render_alpha_subsampled(mu, log_scale, color, opacity, bg, H, W, theta=None, n_pixels=10000,
                            pixel_indices=None):
    """render.py:68-87: exact render at a pixel subsample. Returns (rendered [B,C,n_px], px_idx [B,n_px])."""
    from .params import activate_scale
    from .render_hip import MAX_CHANNELS, _AlphaRender
    B, N, C = color.shape
    device = mu.device
    total = H * W
    if pixel_indices is not None:
        px_idx = pixel_indices
    else:
        n_px = min(n_pixels, total)
        px_idx = torch.randint(0, total, (B, n_px), device=device)
    scale = activate_scale(log_scale)
    outs = []
    for b in range(B):
        py = ((px_idx[b] // W).to(torch.float32) + 0.5) / H
        px = ((px_idx[b] % W).to(torch.float32) + 0.5) / W
        th = theta[b:b + 1] if theta is not None else None
        bgb = bg[b:b + 1] if bg.shape[0] > 1 else bg
        # colour channels in chunks of at most MAX_CHANNELS (render_hip._channel_chunks): each chunk's pixels depend
        # on its own channels only, and autograd adds the chunks' gradients of the shared parameters
        outs.append(torch.cat([_AlphaRender.apply(mu[b:b + 1], scale[b:b + 1], color[b:b + 1, :, k:k + MAX_CHANNELS],
                                                  opacity[b:b + 1], bgb[:, k:k + MAX_CHANNELS], th, py.contiguous(),
                                                  px.contiguous())
                               for k in range(0, C, MAX_CHANNELS)], dim=-1))
    rendered = torch.cat(outs, 0)                                      # [B, n_px, C]
    return rendered.permute(0, 2, 1), px_idx
