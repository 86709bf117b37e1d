"""Feed-forward image -> 2D Gaussian splat encoder, the caller of the renderer (efficient_encoder.py of the
reference, :200-378).

The architecture, the parameter names (the checkpoint's state_dict keys) and the order of operations are the
reference's, because checkpoints trained there must load strictly and produce the same splats:

* backbone: three stride-2 conv -> GELU -> norm stages (widths d/4, d/2, d at strides 2, 4, 8; a fourth at
  stride 16 when stride == 16), fed the image plus its Sobel gradient magnitude (:45-73, :116-124);
* per-cell splat heads: 1x1 convs predicting M splats per feature cell, positions on the cell grid plus a
  tanh-bounded offset, splats flattened cell-major then slot (:144-198);
* variant 'free': one head on the stride-8 features (+ pooled gradient);
* variant 'adaptive': a coarse head of large splats, rendered at residual_grid^2 with render_alpha_octave;
  the residual |image - coarse render| and the coarse luminance condition a fine head that runs on a U-Net
  decoder of the backbone skips at fine_stride (:326-378);
* a per-image background from the pooled stride-8 features (:272-273).

All rendering goes through this package's HIP renderer. `stage_marks` (optional callable taking a stage name)
is called at the stage boundaries of `forward` so a harness can time backbone / coarse render / fine head.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .render import render_alpha_full  # noqa: F401  (re-exported like the reference module)
from .render_hip import render_alpha_full_triton, render_alpha_octave  # noqa: F401


# Architecture of the reference's released checkpoint (its cfg['encoder'] without the training-data field
# image_size): adaptive, d = 256, stride 8, fine stride 4, 2 + 2 splats per cell, 384^2 residual render, odds.
# 833,107 parameters.
GOLDEN_D256 = {"d_feature": 256, "stride": 8, "variant": "adaptive", "use_rotation": True, "use_grad_input": True,
               "gaussians_per_cell": 2, "fine_per_cell": 2, "free_offset_cells": 4.0, "coarse_scale_bias": -3.1,
               "coarse_min_scale": 0.04, "fine_scale_bias": -5.0, "free_scale_bias": -3.0, "residual_grid": 384,
               "norm_type": "group", "opacity_bias": 0.0, "fine_stride": 4, "odds": True}


def _norm(channels: int, norm_type: str) -> nn.Module:
    if norm_type == "group":
        return nn.GroupNorm(8, channels)
    if norm_type == "instance":
        return nn.InstanceNorm2d(channels, affine=True)
    if norm_type == "none":
        return nn.Identity()
    raise ValueError(f"Unknown norm_type: {norm_type}")


def _conv_stage(cin: int, cout: int, k: int, norm_type: str) -> nn.Sequential:
    """conv(k, stride 2) -> GELU -> norm; module indices 0 / 1 / 2 as in the checkpoint keys."""
    return nn.Sequential(nn.Conv2d(cin, cout, k, stride=2, padding=k // 2), nn.GELU(), _norm(cout, norm_type))


class _Backbone(nn.Module):
    """Strided CNN returning its deepest map and the intermediate maps by stride (the fine decoder's skips)."""

    def __init__(self, in_ch: int, d: int, norm_type: str, stride: int):
        super().__init__()
        if stride not in (8, 16):
            raise ValueError(f"stride must be 8 or 16, got {stride}")
        self.stride = stride
        self.stage_s2 = _conv_stage(in_ch, d // 4, 7, norm_type)
        self.stage_s4 = _conv_stage(d // 4, d // 2, 3, norm_type)
        self.stage_s8 = _conv_stage(d // 2, d, 3, norm_type)
        if stride == 16:
            self.stage_s16 = _conv_stage(d, d, 3, norm_type)

    def forward(self, x):
        skips = {}
        for s in (2, 4, 8, 16):
            if s > self.stride:
                break
            x = getattr(self, f"stage_s{s}")(x)
            skips[s] = x
        return x, skips


def _skip_channels(d: int) -> dict:
    return {2: d // 4, 4: d // 2, 8: d, 16: d}


class _UpBlock(nn.Module):
    """Bilinear upsample to the skip's size, concatenate the skip, 3x3 conv -> GELU -> norm."""

    def __init__(self, in_ch: int, skip_ch: int, out_ch: int, norm_type: str):
        super().__init__()
        self.fuse = nn.Sequential(nn.Conv2d(in_ch + skip_ch, out_ch, 3, stride=1, padding=1), nn.GELU(),
                                  _norm(out_ch, norm_type))

    def forward(self, x, skip):
        up = F.interpolate(x, size=skip.shape[2:], mode="bilinear", align_corners=False)
        return self.fuse(torch.cat([up, skip], dim=1))


class _FineDecoder(nn.Module):
    """U-Net decoder from the backbone stride down to fine_stride, one _UpBlock per halving."""

    def __init__(self, d: int, base_stride: int, fine_stride: int, norm_type: str):
        super().__init__()
        if fine_stride not in (2, 4, 8) or fine_stride > base_stride:
            raise ValueError(f"fine_stride must be in (2,4,8) and <= stride, got {fine_stride}")
        skip_ch = _skip_channels(d)
        self.blocks = nn.ModuleList()
        self.target_strides = []
        s, ch = base_stride, d
        while s > fine_stride:
            s //= 2
            out = max(d // 2, 32)
            self.blocks.append(_UpBlock(ch, skip_ch[s], out, norm_type))
            self.target_strides.append(s)
            ch = out
        self.out_ch = ch

    def forward(self, feat, skips):
        for blk, s in zip(self.blocks, self.target_strides):
            feat = blk(feat, skips[s])
        return feat


def sobel_gradmag(img: torch.Tensor) -> torch.Tensor:
    """[B,3,H,W] -> gradient magnitude of the channel mean, [B,1,H,W] (Sobel / 4, +1e-6 under the root)."""
    gray = img.mean(1, keepdim=True)
    kx = torch.tensor([[-1.0, 0.0, 1.0], [-2.0, 0.0, 2.0], [-1.0, 0.0, 1.0]], dtype=img.dtype,
                      device=img.device) / 4.0
    gx = F.conv2d(gray, kx.view(1, 1, 3, 3), padding=1)
    gy = F.conv2d(gray, kx.t().contiguous().view(1, 1, 3, 3), padding=1)
    return torch.sqrt(gx * gx + gy * gy + 1e-6)


def edge_pixel_indices(images: torch.Tensor, n_px: int, lam: float) -> torch.Tensor:
    """n_px pixel indices per image drawn with replacement from (1 - lam) * |grad I| / sum + lam / (H W)
    (efficient_encoder.py:133-141): [B,3,H,W] -> [B, min(n_px, H W)] int64."""
    B, _, H, W = images.shape
    g = sobel_gradmag(images).float().reshape(B, -1)
    g = g / g.sum(1, keepdim=True).clamp_min(1e-8)
    pmf = (1 - lam) * g + lam / (H * W)
    return torch.multinomial(pmf, min(n_px, H * W), replacement=True)


class _SplatHead(nn.Module):
    """M splats per feature cell from 1x1 convs: mu (cell centre + tanh offset of +-offset_cells cells),
    raw log_scale, sigmoid colour, sigmoid opacity (optionally floored), tanh * pi/2 rotation. Splats are
    flattened cell-major then slot: index (y * fW + x) * M + m."""

    def __init__(self, in_ch, M, color_dim=3, scale_bias=-3.0, opacity_bias=2.0, offset_cells=1.0,
                 use_rotation=True, min_opacity=0.0):
        super().__init__()
        self.M, self.color_dim, self.use_rotation = M, color_dim, use_rotation
        self.offset_cells = offset_cells
        self.min_opacity = min_opacity
        self.mu_head = nn.Conv2d(in_ch, 2 * M, 1)
        self.scale_head = nn.Conv2d(in_ch, 2 * M, 1)
        self.color_head = nn.Conv2d(in_ch, color_dim * M, 1)
        self.opacity_head = nn.Conv2d(in_ch, M, 1)
        if use_rotation:
            self.theta_head = nn.Conv2d(in_ch, M, 1)
        nn.init.zeros_(self.mu_head.weight)
        nn.init.zeros_(self.mu_head.bias)
        nn.init.constant_(self.scale_head.bias, scale_bias)
        nn.init.constant_(self.opacity_head.bias, opacity_bias)

    @staticmethod
    def _cells(t, B, M, k, fH, fW):
        """[B, M*k, fH, fW] conv output -> [B, fH*fW*M, k] (cell-major, then slot)."""
        return t.reshape(B, M, k, fH, fW).permute(0, 3, 4, 1, 2).reshape(B, fH * fW * M, k)

    def forward(self, feat):
        B, _, fH, fW = feat.shape
        M = self.M
        ys = torch.linspace(0.5 / fH, 1 - 0.5 / fH, fH, device=feat.device, dtype=feat.dtype)
        xs = torch.linspace(0.5 / fW, 1 - 0.5 / fW, fW, device=feat.device, dtype=feat.dtype)
        gy, gx = torch.meshgrid(ys, xs, indexing="ij")
        base = torch.stack([gy, gx], 0).unsqueeze(0).unsqueeze(0)                     # [1,1,2,fH,fW]
        off = self.offset_cells / max(fH, fW)
        mu = base + torch.tanh(self.mu_head(feat).reshape(B, M, 2, fH, fW)) * off
        mu = mu.permute(0, 3, 4, 1, 2).reshape(B, fH * fW * M, 2).clamp(0.005, 0.995)
        ls = self._cells(self.scale_head(feat), B, M, 2, fH, fW)
        col = torch.sigmoid(self._cells(self.color_head(feat), B, M, self.color_dim, fH, fW))
        op = torch.sigmoid(self._cells(self.opacity_head(feat), B, M, 1, fH, fW)[..., 0])
        if self.min_opacity > 0.0:
            op = self.min_opacity + (1.0 - self.min_opacity) * op
        th = None
        if self.use_rotation:
            th = torch.tanh(self._cells(self.theta_head(feat), B, M, 1, fH, fW)[..., 0]) * (math.pi / 2)
        return {"mu": mu, "log_scale": ls, "color": col, "opacity": op, "theta": th}


class EfficientGaussianEncoder(nn.Module):
    """Image [B,3,H,W] in [0,1] -> splats (mu, log_scale, color, opacity, theta, bg) for render_alpha_octave.
    Constructor arguments and defaults are the reference's (efficient_encoder.py:202-248), so a checkpoint's
    saved `cfg['encoder']` builds the same network."""

    def __init__(self, d_feature=128, stride=8, variant="free", norm_type="group", use_rotation=True,
                 use_grad_input=True, gaussians_per_cell=2, fine_per_cell=2, free_offset_cells=4.0,
                 coarse_scale_bias=-1.5, coarse_min_scale=0.04, fine_scale_bias=-4.0, free_scale_bias=-3.0,
                 opacity_bias=2.0, residual_grid=64, fine_stride=None, coarse_min_opacity=0.0,
                 coarse_offset_cells=2.0, fine_offset_cells=2.0, odds=False):
        super().__init__()
        if variant not in ("free", "adaptive"):
            raise ValueError(f"variant must be 'free' or 'adaptive', got {variant!r}")
        if stride not in (8, 16):
            raise ValueError("the encoder supports stride 8 or 16")
        self.variant = variant
        self.stride = stride
        self.fine_stride = fine_stride if fine_stride is not None else stride
        self.odds = odds
        self.use_grad_input = use_grad_input
        self.residual_grid = residual_grid
        # coarse log_scale floor: softplus(floor) == coarse_min_scale
        self.coarse_ls_floor = math.log(math.exp(coarse_min_scale) - 1.0) if coarse_min_scale > 0 else None
        self.M = gaussians_per_cell
        self.Mf = fine_per_cell
        self.stage_marks = None
        g_ch = 1 if use_grad_input else 0
        self.backbone = _Backbone(3 + g_ch, d_feature, norm_type, stride)
        self.bg_head = nn.Linear(d_feature, 3)
        head_in = d_feature + g_ch
        if variant == "free":
            self.head = _SplatHead(head_in, self.M, scale_bias=free_scale_bias, opacity_bias=opacity_bias,
                                   offset_cells=free_offset_cells, use_rotation=use_rotation)
        else:
            self.coarse_head = _SplatHead(head_in, self.M, scale_bias=coarse_scale_bias, opacity_bias=opacity_bias,
                                          offset_cells=coarse_offset_cells, use_rotation=use_rotation,
                                          min_opacity=coarse_min_opacity)
            self.fine_decoder = _FineDecoder(d_feature, stride, self.fine_stride, norm_type)
            # fine head input: decoded features + gradient + residual (3) + coarse luminance (1)
            self.fine_head = _SplatHead(self.fine_decoder.out_ch + g_ch + 4, self.Mf, scale_bias=fine_scale_bias,
                                        opacity_bias=opacity_bias, offset_cells=fine_offset_cells,
                                        use_rotation=use_rotation)

    def _mark(self, name):
        if self.stage_marks is not None:
            self.stage_marks(name)

    def _with_grad(self, feat, image, size=None):
        """Features with the (pooled) gradient map appended, when the encoder uses it."""
        if not self.use_grad_input:
            return feat
        g = F.adaptive_avg_pool2d(sobel_gradmag(image), feat.shape[2:] if size is None else size)
        return torch.cat([feat, g], dim=1)

    def gather_splat_latents(self, output):
        """[B, N, C] feature of the cell each splat was predicted from, aligned with output['mu'] (the fine
        decoder map for 'adaptive', whose coarse splats get zero rows first; the fused map for 'free')."""
        if "splat_features" not in output:
            raise KeyError("no 'splat_features' -- call forward(image, return_latents=True)")
        feat = output["splat_features"]
        B, C, fH, fW = feat.shape
        per_cell = self.Mf if self.variant == "adaptive" else self.M
        lat = feat.permute(0, 2, 3, 1).reshape(B, fH * fW, 1, C).expand(B, fH * fW, per_cell, C)
        lat = lat.reshape(B, fH * fW * per_cell, C)
        n_coarse = int(output.get("n_coarse", 0))
        if n_coarse:
            lat = torch.cat([lat.new_zeros(B, n_coarse, C), lat], dim=1)
        if lat.shape[1] != output["mu"].shape[1]:
            raise RuntimeError(f"latent/splat axis mismatch: {lat.shape[1]} vs {output['mu'].shape[1]}")
        return lat

    def forward(self, image, return_latents: bool = False):
        x = torch.cat([image, sobel_gradmag(image)], dim=1) if self.use_grad_input else image
        feat, skips = self.backbone(x)
        fused = self._with_grad(feat, image)
        bg = torch.sigmoid(self.bg_head(feat.mean(dim=(2, 3))))
        self._mark("backbone")
        if self.variant == "free":
            out = self.head(fused)
            out.update(bg=bg, n_gaussians=out["mu"].shape[1], backbone_features=feat)
            if return_latents:
                out["splat_features"] = fused
            self._mark("heads")
            return out

        coarse = self.coarse_head(fused)
        if self.coarse_ls_floor is not None:
            coarse["log_scale"] = coarse["log_scale"].clamp(min=self.coarse_ls_floor)
        self._mark("coarse_head")
        rg = self.residual_grid
        c_render = render_alpha_octave(coarse["mu"], coarse["log_scale"], coarse["color"], coarse["opacity"], bg,
                                       rg, rg, coarse["theta"], odds=self.odds)
        self._mark("coarse_render")
        target_small = F.interpolate(image, size=(rg, rg), mode="bilinear", align_corners=False)
        cond = torch.cat([(target_small - c_render).abs(), c_render.mean(1, keepdim=True)], dim=1)
        fine_feat = self.fine_decoder(feat, skips)
        fsz = fine_feat.shape[2:]
        cond_fine = F.interpolate(cond, size=fsz, mode="bilinear", align_corners=False)
        fine_in = torch.cat([self._with_grad(fine_feat, image, fsz), cond_fine], dim=1)
        fine = self.fine_head(fine_in)
        out = {k: torch.cat([coarse[k], fine[k]], dim=1) for k in ("mu", "log_scale", "color", "opacity")}
        out["theta"] = torch.cat([coarse["theta"], fine["theta"]], dim=1) if coarse["theta"] is not None else None
        out.update(bg=bg, n_gaussians=out["mu"].shape[1], n_coarse=coarse["mu"].shape[1], backbone_features=feat)
        if return_latents:
            out["splat_features"] = fine_feat
        self._mark("fine_head")
        return out
