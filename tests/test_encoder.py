"""The encoder caller (efficient_encoder.py / examples/encode_and_render.py of the reference) on the CPU:
architecture and checkpoint format, the splat layout the renderer receives, and an end-to-end known answer —
the released checkpoint's reconstructions of samples/targets/*.png, whose PSNR and live-splat counts the
reference recorded (samples/reconstructions/measurements.json) — with every render done by the float64 C
oracle.

The known-answer test reads the reference checkout (checkpoint and target image) and is skipped where it is
absent; the checkpoint is loaded with torch.load(weights_only=True) only."""

import json
import math
import os

import numpy as np
import pytest
import torch

from gaussian_splat_encoder import efficient_encoder as EE
from gaussian_splat_encoder.checkpoint import encoder_kwargs, load_encoder
from gaussian_splat_encoder.params import activate_scale
from oracle import render_ref as R

REF = "/root/reference"
CKPT = os.path.join(REF, "weights", "encoder_golden_d256.pt")
# cfg['encoder'] of the released checkpoint (its architecture; 833,107 parameters, PROVENANCE.md of the reference)
GOLDEN_CFG = {"d_feature": 256, "stride": 8, "variant": "adaptive", "use_rotation": True, "use_grad_input": True,
              "gaussians_per_cell": 2, "fine_per_cell": 2, "free_offset_cells": 4.0, "coarse_scale_bias": -3.1,
              "coarse_min_scale": 0.04, "fine_scale_bias": -5.0, "free_scale_bias": -3.0, "residual_grid": 384,
              "norm_type": "group", "image_size": 1024, "opacity_bias": 0.0, "fine_stride": 4, "odds": True}


def test_golden_architecture_parameter_count():
    enc = EE.EfficientGaussianEncoder(**encoder_kwargs(GOLDEN_CFG))
    assert sum(p.numel() for p in enc.parameters()) == 833_107


def test_unknown_checkpoint_field_raises():
    with pytest.raises(ValueError, match="Unknown checkpoint architecture"):
        encoder_kwargs({**GOLDEN_CFG, "new_field": 1})


def test_free_variant_cell_major_layout():
    """Zero-initialised position heads put splat (y * fW + x) * M + m exactly on cell (y, x)'s centre; the
    latents gathered for a splat are its cell's features."""
    torch.manual_seed(0)
    enc = EE.EfficientGaussianEncoder(d_feature=32, variant="free", gaussians_per_cell=3).eval()
    img = torch.rand(2, 3, 48, 64)
    with torch.no_grad():
        out = enc(img, return_latents=True)
    fH, fW, M = 6, 8, 3
    assert out["mu"].shape == (2, fH * fW * M, 2) and out["n_gaussians"] == fH * fW * M
    y, x = torch.meshgrid(torch.arange(fH), torch.arange(fW), indexing="ij")
    centres = torch.stack([(y + 0.5) / fH, (x + 0.5) / fW], -1).reshape(fH * fW, 1, 2).expand(fH * fW, M, 2)
    assert torch.allclose(out["mu"][0], centres.reshape(-1, 2), atol=1e-6)
    lat = enc.gather_splat_latents(out)
    feat = out["splat_features"]
    k = (2 * fW + 5) * M + 1                       # cell (2, 5), slot 1
    assert torch.equal(lat[1, k], feat[1, :, 2, 5])
    assert out["opacity"].min() > 0 and out["opacity"].max() < 1
    assert out["theta"].abs().max() <= math.pi / 2


def cpu_octave(mu, log_scale, color, opacity, bg, H, W, theta=None, cutoff=3.0, TILE=8, base_texels=8.0,
               max_octaves=6, max_pairs=48_000_000, odds=False):
    """render_alpha_octave on the CPU through the float64 C oracle -> [B,C,H,W] float32."""
    sc = activate_scale(log_scale.float())
    imgs = []
    for b in range(mu.shape[0]):
        th = None if theta is None else theta[b]
        img = R.octave_forward_c(mu[b], sc[b], color[b], opacity[b], bg[b], th, H, W, cutoff, TILE, base_texels,
                                 max_octaves, odds)
        imgs.append(img.float().reshape(H, W, -1).permute(2, 0, 1))
    return torch.stack(imgs)


@pytest.mark.skipif(not os.path.exists(CKPT), reason="reference checkout (checkpoint) not present")
@pytest.mark.parametrize("sample", [0, 1, 2])
def test_released_checkpoint_reconstruction_psnr(monkeypatch, sample):
    """All three reference reconstructions: splat count, live splats (opacity > 0.1) and PSNR of the odds
    octave render, as examples/encode_and_render.py measured them (here: float64 oracle renders)."""
    from PIL import Image
    enc = load_encoder(CKPT, "cpu")
    assert enc.odds and enc.variant == "adaptive"
    monkeypatch.setattr(EE, "render_alpha_octave", cpu_octave)
    rec = json.load(open(os.path.join(REF, "samples", "reconstructions", "measurements.json")))[sample]
    arr = np.asarray(Image.open(os.path.join(REF, rec["input"])).convert("RGB")).copy()
    x = torch.from_numpy(arr).permute(2, 0, 1).unsqueeze(0).float() / 255
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    with torch.inference_mode():
        out = enc(x)
        img = cpu_octave(out["mu"].float(), out["log_scale"].float(), out["color"].float(), out["opacity"].float(),
                         out["bg"].float(), x.shape[-2], x.shape[-1], theta=out["theta"].float(),
                         odds=enc.odds).clamp(0, 1)
    assert out["mu"].shape[1] == rec["splats"] == 92_160
    assert int((out["opacity"] > 0.1).sum()) == rec["live_splats_opacity_gt_0.1"]
    mse = float((x - img).square().mean())
    psnr = -10 * math.log10(max(mse, 1e-12))
    assert abs(psnr - rec["psnr_db"]) <= 0.005, (psnr, rec["psnr_db"])
