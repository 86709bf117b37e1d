"""Render parity at the configured sizes of the stress and end-to-end configurations.

* 2048 x 2048, 655,360 splats with a 2 % heavy tail (up to ~10k tile pairs per splat, summed by
  whole waves in the per-splat reduction): single-res forward and forward + backward (composite alpha, fields
  odds) and octave forward + backward (alpha, odds), against the float64 C oracle over the full frame.
* the encoder's own splats (released architecture, seeded random init, procedural 768 x 768 card):
  the coarse 384^2 odds octave render of its 18,432 coarse splats and the full 768^2 odds octave render of all
  92,160 splats, as the encoder and examples/encode_and_render.py make them (efficient_encoder.py:346-348,
  encode_and_render.py:31-38), held to the image bar (1e-5) on identical inputs, separately from the network's
  own GPU-vs-CPU tolerance; and both renders' gradients against the composed oracle.
"""

import numpy as np
import pytest
import torch

from _gpu_util import IMG_TOL, np_
from gaussian_splat_encoder import _lib, synth
from oracle import render_ref as R
from test_gpu_levels import run_levels
from test_gpu_render import run_case

pytestmark = pytest.mark.gpu


def octave_lv():
    return _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)


@pytest.fixture(scope="module")
def c4(dev):
    s = synth.config("c4").to(dev)
    yield s
    del s
    torch.cuda.empty_cache()


@pytest.mark.parametrize("odds,fields", [(False, False), (True, True)])
def test_c4_single_res(c4, odds, fields):
    s = c4
    print(f"c4 single-res odds={odds} fields={fields} N={s.n} {s.H}x{s.W}", flush=True)
    run_case(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.theta, s.H, s.W, 8, odds, fields, seed=61)


@pytest.mark.parametrize("odds", [False, True])
def test_c4_octave(c4, odds):
    s = c4
    print(f"c4 octave odds={odds}", flush=True)
    bins = run_levels(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.theta, s.H, s.W, 8, octave_lv(), odds, seed=62)
    assert sum(1 for n in bins.level_tot_b[0] if n) >= 4   # the heavy tail spans several octaves


@pytest.fixture(scope="module")
def c3_renders(dev):
    """The encoder's two odds octave renders on the GPU, with the inputs each one received."""
    import gaussian_splat_encoder.efficient_encoder as EE
    from gaussian_splat_encoder import render_hip as RH
    torch.manual_seed(0)
    enc = EE.EfficientGaussianEncoder(**EE.GOLDEN_D256).to(dev).eval()
    x = synth.procedural_image(768, 768).to(dev)
    calls = []
    inner = EE.render_alpha_octave

    def recording(mu, log_scale, color, opacity, bg, H, W, theta=None, **kw):
        out = inner(mu, log_scale, color, opacity, bg, H, W, theta=theta, **kw)
        calls.append(((mu, log_scale, color, opacity, bg, theta), H, W, kw, out))
        return out

    EE.render_alpha_octave = recording
    try:
        with torch.inference_mode():
            o = enc(x)
            full = RH.render_alpha_octave(o["mu"], o["log_scale"], o["color"], o["opacity"], o["bg"], 768, 768,
                                          theta=o["theta"], odds=enc.odds)
    finally:
        EE.render_alpha_octave = inner
    assert len(calls) == 1, "the encoder makes one coarse render"
    coarse = calls[0]
    full = ((o["mu"], o["log_scale"], o["color"], o["opacity"], o["bg"], o["theta"]), 768, 768,
            {"odds": enc.odds}, full)
    own = lambda t: None if t is None else t.clone()   # plain tensors, outside inference mode
    out = {}
    for name, (args, H, W, kw, img) in (("coarse", coarse), ("full", full)):
        out[name] = ([own(a) for a in args], H, W, kw, own(img))
    del enc, x, o
    return out


@pytest.mark.parametrize("which,H,N", [("coarse", 384, 18_432), ("full", 768, 92_160)])
def test_c3_render_image(c3_renders, which, H, N):
    (mu, ls, col, op, bg, th), Hh, Ww, kw, img = c3_renders[which]
    assert (Hh, Ww) == (H, H) and mu.shape[1] == N and kw.get("odds") is True
    print(f"c3 {which} {H}x{H} N={N}", flush=True)
    sc = torch.nn.functional.softplus(ls.float()) + 1e-4
    ref = R.octave_forward_c(mu[0], sc[0], col[0], op[0], bg[0], None if th is None else th[0], H, H, odds=True)
    got = np_(img[0]).transpose(1, 2, 0).reshape(H * H, -1)
    d = np.abs(got - ref.numpy()).max()
    assert d <= IMG_TOL, f"{which} image max-abs {d:.2e}"


@pytest.mark.parametrize("which", ["coarse", "full"])
def test_c3_render_gradients(c3_renders, which):
    (mu, ls, col, op, bg, th), H, W, kw, _ = c3_renders[which]
    print(f"c3 {which} fwd+bwd", flush=True)
    run_levels(mu.float(), ls.float(), col.float(), op.float(), bg.float(), None if th is None else th.float(), H, W,
               8, octave_lv(), True, seed=63)
