"""The encoder caller end to end on the GPU: the released checkpoint's architecture (seeded random init) on a
procedural card, with the HIP renders inside (coarse residual render) and after (full render), against the
same network on the CPU with every render done by the float64 C oracle."""

import pytest
import torch

from gaussian_splat_encoder import efficient_encoder as EE
from gaussian_splat_encoder import render_hip as RH
from gaussian_splat_encoder import synth

pytestmark = pytest.mark.gpu


def test_golden_architecture_gpu_matches_cpu_oracle(dev, monkeypatch):
    import test_encoder as T
    torch.manual_seed(3)
    cfg = dict(EE.GOLDEN_D256, residual_grid=128)
    enc = EE.EfficientGaussianEncoder(**cfg).eval()
    x = synth.procedural_image(256, 256, seed=5)
    with torch.inference_mode():
        enc_d = EE.EfficientGaussianEncoder(**cfg).eval()
        enc_d.load_state_dict(enc.state_dict())
        enc_d = enc_d.to(dev)
        out_d = enc_d(x.to(dev))
        img_d = RH.render_alpha_octave(out_d["mu"], out_d["log_scale"], out_d["color"], out_d["opacity"], out_d["bg"],
                                       256, 256, theta=out_d["theta"], odds=True)
        monkeypatch.setattr(EE, "render_alpha_octave", T.cpu_octave)
        out_c = enc(x)
        img_c = T.cpu_octave(out_c["mu"], out_c["log_scale"], out_c["color"], out_c["opacity"], out_c["bg"], 256, 256,
                             theta=out_c["theta"], odds=True)
    assert out_d["mu"].shape[1] == out_c["mu"].shape[1] == 32 * 32 * 2 + 64 * 64 * 2
    for k in ("mu", "log_scale", "color", "opacity", "theta", "bg"):
        d = (out_d[k].float().cpu() - out_c[k]).abs().max().item()
        assert d <= 2e-4, f"{k}: {d:.2e}"
    d = (img_d.float().cpu() - img_c).abs().max().item()
    assert d <= 5e-4, f"image max-abs {d:.2e}"
