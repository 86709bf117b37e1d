"""Entry-point parity (render_alpha_full_triton, render_alpha_multires, render_alpha_octave and the
render.py entry points) with autograd, against the torch float64 oracle, plus the reference's own
self-test identities (render_triton.py:983-1533) and error behaviour."""

import numpy as np
import pytest
import torch

from _gpu_util import GRAD_REL_TOL, IMG_TOL, RH, activate_scale, np_, random_scene, rel_err
from gaussian_splat_encoder import render as R_api
from oracle import render_ref as R

pytestmark = pytest.mark.gpu
NAMES = ["mu", "ls", "col", "op", "bg", "th"]


def device_run(fn, scene, gout, **kw):
    L = [None if t is None else t.detach().clone().requires_grad_(True) for t in scene]
    out = fn(*L[:5], theta=L[5], **kw)
    (out * gout).sum().backward()
    return out.detach(), {n: (None if t is None else t.grad) for n, t in zip(NAMES, L)}


def oracle_run(kind, scene, gout, H, W, **kw):
    """float64 oracle of one batch; binning/routing use the device's fp32 activated scale."""
    mu, ls, col, op, bg, th = [None if t is None else t[0] for t in scene]
    L = R.leaves(mu, ls, col, op, bg, th)
    sc32 = activate_scale(ls).detach().cpu()
    sc64 = R.activate_scale(L[1])
    if kind == "cull":
        cutoff, odds, TILE = kw.get("cutoff", 3.0), kw.get("odds", False), kw.get("TILE", 8)
        gid, st = R._bin(L[0], sc32, H, W, TILE, cutoff)
        out = R.cull_composite(L[0], sc64, L[2], L[3], L[4], L[5], gid, st, H, W, TILE, odds)[0]
    elif kind == "exact":
        out = R.exact(L[0], sc64, L[2], L[3], L[4], L[5], H, W)
    elif kind == "multires":
        out = R.multires(L[0], sc64, L[2], L[3], L[4], L[5], H, W, scale32=sc32, **kw)
    elif kind == "octave":
        oct_dev = RH._octave_of(activate_scale(ls).detach().amax(-1) * float(min(H, W)),
                                kw.get("base_texels", 8.0), kw.get("max_octaves", 6)).cpu()
        out = R.octave(L[0], sc64, L[2], L[3], L[4], L[5], H, W, oct=oct_dev, scale32=sc32, **kw)
    g = gout[0].permute(1, 2, 0).reshape(H * W, -1).cpu().to(torch.float64)
    (out * g).sum().backward()
    img = out.detach().reshape(H, W, -1).permute(2, 0, 1)
    return img, {n: (None if t is None else t.grad) for n, t in zip(NAMES, L)}


def compare(dev_out, dev_g, ref_out, ref_g, img_tol=IMG_TOL, grad_tol=GRAD_REL_TOL):
    d = np.abs(np_(dev_out[0]) - ref_out.numpy()).max()
    assert d <= img_tol, f"image max-abs {d:.2e}"
    for n in NAMES:
        if ref_g[n] is None:
            assert dev_g[n] is None
            continue
        e = rel_err(np_(dev_g[n][0]), ref_g[n].numpy())
        assert e <= grad_tol, f"grad {n}: rel {e:.2e}"


def gout_for(H, W, dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, 3, H, W, generator=g).to(dev)


@pytest.mark.parametrize("odds", [False, True])
@pytest.mark.parametrize("has_theta", [True, False])
def test_cull_entry_point(dev, odds, has_theta):
    H = W = 48
    scene = random_scene(500, H, W, seed=21, dev=dev, op_max=0.95, theta=has_theta)
    gout = gout_for(H, W, dev, 1)
    out, g = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=True, odds=odds)
    ref, rg = oracle_run("cull", scene, gout, H, W, odds=odds)
    compare(out, g, ref, rg)


def test_exact_entry_point_and_render_py(dev):
    H = W = 24
    scene = random_scene(200, H, W, seed=22, dev=dev, ls_mean_px=2.0)
    gout = gout_for(H, W, dev, 2)
    out, g = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=False)
    ref, rg = oracle_run("exact", scene, gout, H, W)
    compare(out, g, ref, rg)
    out2, g2 = device_run(R_api.render_alpha_full, scene, gout, H=H, W=W)
    assert torch.equal(out2, out)
    # subsampled pixels equal the full render at those pixels
    idx = torch.randperm(H * W, generator=torch.Generator().manual_seed(3))[:100].to(dev)[None]
    sub, got_idx = R_api.render_alpha_subsampled(*scene[:5], H, W, theta=scene[5], pixel_indices=idx)
    full = out.reshape(1, 3, H * W)
    assert torch.equal(got_idx, idx)
    assert (sub - full[:, :, idx[0]]).abs().max().item() <= 2e-6


def test_multires_none_equals_cull(dev):
    """render_triton.py:1214-1253: the fields path with deferred composite equals the in-kernel composite."""
    H = W = 64
    scene = random_scene(1024, H, W, seed=7, dev=dev)
    gout = gout_for(H, W, dev, 3)
    a, ga = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=True)
    b, gb = device_run(RH.render_alpha_multires, scene, gout, H=H, W=W, n_coarse=None)
    assert (a - b).abs().max().item() <= 1e-6
    for n in NAMES:
        assert rel_err(np_(gb[n]), np_(ga[n])) <= 1e-4, n


@pytest.mark.parametrize("odds", [False, True])
def test_octave_zero_equals_cull(dev, odds):
    """render_triton.py:1334-1367 and 1500-1533 (odds)."""
    H = W = 64
    scene = random_scene(1024, H, W, seed=13, dev=dev, op_max=0.9)
    gout = gout_for(H, W, dev, 4)
    a, ga = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=True, odds=odds)
    b, gb = device_run(RH.render_alpha_octave, scene, gout, H=H, W=W, max_octaves=0, odds=odds)
    assert (a - b).abs().max().item() <= 1e-6
    for n in NAMES:
        assert rel_err(np_(gb[n]), np_(ga[n])) <= 1e-4, n


@pytest.mark.parametrize("odds", [False, True])
def test_octave_multi_level(dev, odds):
    """Splats spanning several octaves (render_triton.py:1370-1402's scene shape) against the oracle's
    octave glue over the same routing."""
    H = W = 128
    g = torch.Generator().manual_seed(17)
    n = 400
    sig = torch.exp(torch.rand(1, n, generator=g) * (np.log(0.31) - np.log(0.006)) + np.log(0.006))
    ls = torch.log(torch.exp(sig).clamp_min(1 + 1e-6) - 1.0).unsqueeze(-1).expand(1, n, 2).contiguous()
    mu = torch.rand(1, n, 2, generator=g)
    col = torch.rand(1, n, 3, generator=g)
    op = torch.rand(1, n, generator=g) * 0.4
    th = torch.rand(1, n, generator=g) * 3.14159
    bg = torch.rand(1, 3, generator=g)
    scene = [t.to(dev) for t in (mu, ls, col, op, bg, th)]
    gout = gout_for(H, W, dev, 5)
    out, gd = device_run(RH.render_alpha_octave, scene, gout, H=H, W=W, odds=odds)
    ref, rg = oracle_run("octave", scene, gout, H, W, odds=odds)
    compare(out, gd, ref, rg)


def test_multires_split(dev):
    H = W = 128
    scene = list(random_scene(576, H, W, seed=11, dev=dev))
    ls = scene[1].clone()
    ls[:, :64] = float(np.log(np.exp(0.12) - 1.0))
    ls[:, 64:] = float(np.log(np.exp(0.015) - 1.0))
    scene[1] = ls
    gout = gout_for(H, W, dev, 6)
    out, gd = device_run(RH.render_alpha_multires, scene, gout, H=H, W=W, n_coarse=64, coarse_factor=8)
    ref, rg = oracle_run("multires", scene, gout, H, W, n_coarse=64, coarse_factor=8)
    compare(out, gd, ref, rg)


def test_errors(dev):
    scene = random_scene(64, 32, 32, seed=1, dev=dev)
    with pytest.raises(NotImplementedError):
        RH.render_alpha_full_triton(*scene[:5], 32, 32, theta=scene[5], cull=False, odds=True)
    with pytest.raises(RH.PairBudgetExceeded):
        RH.render_alpha_octave(*scene[:5], 32, 32, theta=scene[5], max_pairs=10)
    with pytest.raises(Exception, match="TILE"):
        RH.render_alpha_full_triton(*scene[:5], 32, 32, theta=scene[5], cull=True, TILE=5)


BATCH_ENTRIES = {
    "cull": (lambda *a, **k: RH.render_alpha_full_triton(*a, cull=True, **k), {}),
    "octave": (RH.render_alpha_octave, {}),
    "multires": (RH.render_alpha_multires, {"n_coarse": 60, "coarse_factor": 4}),
}


@pytest.mark.parametrize("entry", ["cull", "octave", "multires"])
def test_batch_of_three(dev, entry):
    """B = 3 through each entry point: every batch element's image and gradients (background included) equal
    those of the element rendered alone."""
    H = W = 40
    fn, kw = BATCH_ENTRIES[entry]
    scene = random_scene(300, H, W, seed=31, dev=dev, B=3)
    g = torch.Generator().manual_seed(8)
    gout = torch.randn(3, 3, H, W, generator=g).to(dev)
    out, gd = device_run(fn, scene, gout, H=H, W=W, odds=True, **kw)
    for b in range(3):
        one = [None if t is None else t[b:b + 1] for t in scene]
        o1, g1 = device_run(fn, one, gout[b:b + 1], H=H, W=W, odds=True, **kw)
        assert (o1[0] - out[b]).abs().max().item() <= 1e-6
        for n in ["mu", "ls", "col", "op", "bg", "th"]:
            assert rel_err(np_(g1[n][0]), np_(gd[n][b])) <= 1e-5, n


@pytest.mark.parametrize("entry", ["cull", "octave", "multires"])
def test_background_broadcast_over_batch(dev, entry):
    """A [1, C] background with B = 2 is broadcast over the batch, as the reference's torch composite broadcasts
    it (render_triton.py:921, :980): each image equals the image rendered alone with that background, and the
    background's gradient is the sum of the per-image ones. Shapes that do not match the batch are refused."""
    H = W = 40
    fn, kw = BATCH_ENTRIES[entry]
    mu, ls, col, op, bg, th = random_scene(300, H, W, seed=35, dev=dev, B=2)
    bg1 = bg[:1].clone()
    gout = torch.randn(2, 3, H, W, generator=torch.Generator().manual_seed(9)).to(dev)
    leaves = [t.clone().requires_grad_(True) for t in (mu, ls, col, op, bg1, th)]
    out = fn(*leaves[:5], H, W, theta=leaves[5], odds=True, **kw)
    (out * gout).sum().backward()
    g_bg = torch.zeros_like(bg1)
    for b in range(2):
        one = [t[b:b + 1].clone().requires_grad_(True) for t in (mu, ls, col, op)] + [bg1.clone().requires_grad_(True),
                                                                                     th[b:b + 1].clone()]
        o1 = fn(*one[:5], H, W, theta=one[5], odds=True, **kw)
        (o1 * gout[b:b + 1]).sum().backward()
        assert (o1[0] - out[b]).abs().max().item() <= 1e-6
        g_bg += one[4].grad
        assert rel_err(np_(one[2].grad[0]), np_(leaves[2].grad[b])) <= 1e-5
    assert leaves[4].grad.shape == (1, 3)
    assert rel_err(np_(leaves[4].grad), np_(g_bg)) <= 1e-5
    for bad_bg in (bg[:, :2], torch.rand(3, 3, device=dev)):
        with pytest.raises(ValueError, match="bg must be"):
            fn(mu, ls, col, op, bad_bg, H, W, theta=th, **kw)
    with pytest.raises(ValueError, match="opacity must be"):
        fn(mu, ls, col, op[:1], bg, H, W, theta=th, **kw)


@pytest.mark.parametrize("kind", ["cull", "octave", "multires"])
def test_scale_activation_in_decode_matches_torch_bits(dev, monkeypatch, kind):
    """fp32 log-scales are activated inside the binning's decode pass and the log-scale gradient is chained in
    the per-splat reduction. Both must give exactly the bits of activate_scale (torch's softplus + 1e-4) and
    its autograd: same decoded records, pair lists, image and gradients."""
    H = W = 64
    scene = list(random_scene(800, H, W, seed=41, dev=dev))
    ls = scene[1].clone()
    # every regime of softplus: exp underflow, small, around 0, the threshold 20 and past it
    ls[0, :9, :] = torch.tensor([-100., -30., -8., -2., 0., 1.5, 19.9, 20., 20.5], device=dev)[:, None]
    ls[0, 9:12, 0] = torch.tensor([-4., 2., 21.], device=dev)
    scene[1] = ls
    fn = {"cull": RH.render_alpha_full_triton, "octave": RH.render_alpha_octave,
          "multires": RH.render_alpha_multires}[kind]
    kw = {"cull": {"cull": True}, "octave": {}, "multires": {"n_coarse": 100}}[kind]
    gout = gout_for(H, W, dev, 9)
    mu, _, col, op, _, th = scene
    b_fused = RH._bin(mu, ls, col, op, th, H, W, 8, 3.0, scale_is_log=True)
    b_torch = RH._bin(mu, activate_scale(ls), col, op, th, H, W, 8, 3.0)
    rec = lambda b: b.blocks[0].view(0, 16 * 800, torch.float32)
    assert torch.equal(rec(b_fused), rec(b_torch))
    g_f, s_f = b_fused.as_tuple()[:2]
    g_t, s_t = b_torch.as_tuple()[:2]
    assert torch.equal(g_f[0], g_t[0]) and torch.equal(s_f[0], s_t[0])
    out_f, gd_f = device_run(fn, scene, gout, H=H, W=W, **kw)
    monkeypatch.setattr(RH, "_scale_arg", lambda t: (activate_scale(t), False))
    out_t, gd_t = device_run(fn, scene, gout, H=H, W=W, **kw)
    assert torch.equal(out_f, out_t)
    for n in NAMES:
        assert torch.equal(gd_f[n], gd_t[n]), (n, (gd_f[n] - gd_t[n]).abs().max().item())


def test_kernel_timer_brackets(dev):
    """The tile kernels record the timer's events themselves (splat_time_next_launch): every armed pair is taken
    by exactly one launch, the brackets are positive and no pair stays armed; the binning is bracketed on the
    stream."""
    mu, ls, col, op, bg, th = random_scene(600, 64, 48, seed=21, dev=dev)
    leaves = [t.clone().requires_grad_(True) for t in (mu, ls, col, op, bg, th)]
    RH.kernel_timer.enable(True, names=("fwd", "bwd", "bin"))
    try:
        for _ in range(3):
            out = RH.render_alpha_full_triton(*leaves[:5], 64, 48, theta=leaves[5], cull=True)
            out.backward(torch.ones_like(out))
        ms = RH.kernel_timer.elapsed_ms()
    finally:
        RH.kernel_timer.enable(False)
    assert sorted(ms) == ["bin", "bwd", "fwd"]
    for k, v in ms.items():
        assert len(v) == 3 and all(0.0 < x < 1e3 for x in v), (k, v)
    assert RH._lib.load().splat_time_next_launch(None, None) == 0


@pytest.mark.parametrize("TILE,cutoff", [(4, 3.0), (16, 3.0), (8, 2.0), (8, 4.5)])
@pytest.mark.parametrize("odds", [False, True])
def test_cull_entry_point_tiles_and_cutoffs(dev, TILE, cutoff, odds):
    """The culled entry point at the other tile sizes and cull radii the reference's probes use
    (render_triton.py:1037, :1170), through autograd, on a ragged canvas."""
    H, W = 50, 38
    scene = random_scene(400, H, W, seed=90 + TILE, dev=dev, op_max=0.95, margin=0.1)
    gout = gout_for(H, W, dev, 9)
    out, g = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=True, TILE=TILE, cutoff=cutoff,
                        odds=odds)
    ref, rg = oracle_run("cull", scene, gout, H, W, TILE=TILE, cutoff=cutoff, odds=odds)
    compare(out, g, ref, rg)


def octave_scene(n, seed, dev):
    """Splats whose sizes span several octaves (log-uniform sigma 0.006-0.31 of the image), as in
    test_octave_multi_level."""
    g = torch.Generator().manual_seed(seed)
    sig = torch.exp(torch.rand(1, n, generator=g) * (np.log(0.31) - np.log(0.006)) + np.log(0.006))
    ls = torch.log(torch.exp(sig).clamp_min(1 + 1e-6) - 1.0).unsqueeze(-1).expand(1, n, 2).contiguous()
    mu = torch.rand(1, n, 2, generator=g)
    col = torch.rand(1, n, 3, generator=g)
    op = torch.rand(1, n, generator=g) * 0.4
    th = torch.rand(1, n, generator=g) * 3.14159
    bg = torch.rand(1, 3, generator=g)
    return [t.to(dev) for t in (mu, ls, col, op, bg, th)]


@pytest.mark.parametrize("TILE,base,mo", [(4, 8.0, 6), (16, 8.0, 6), (8, 4.0, 3), (8, 16.0, 2)])
def test_octave_entry_point_options(dev, TILE, base, mo):
    """render_alpha_octave's TILE, base_texels and max_octaves (render_triton.py:935-980) through autograd on a
    ragged canvas, against the oracle's octave glue with the same options (routing and per-level binning)."""
    H, W = 96, 80
    scene = octave_scene(300, 70 + TILE + mo, dev)
    gout = gout_for(H, W, dev, 7)
    kw = dict(TILE=TILE, base_texels=base, max_octaves=mo, odds=True)
    out, gd = device_run(RH.render_alpha_octave, scene, gout, H=H, W=W, **kw)
    ref, rg = oracle_run("octave", scene, gout, H, W, **kw)
    compare(out, gd, ref, rg)


@pytest.mark.parametrize("TILE,cf", [(4, 4), (16, 8), (8, 2)])
def test_multires_entry_point_options(dev, TILE, cf):
    """render_alpha_multires's TILE and coarse_factor (render_triton.py:879-922) through autograd, against the
    oracle's coarse/fine glue with the same options."""
    H, W = 96, 80
    scene = list(random_scene(400, H, W, seed=80 + TILE + cf, dev=dev))
    ls = scene[1].clone()
    ls[:, :80] = float(np.log(np.exp(0.1) - 1.0))
    scene[1] = ls
    gout = gout_for(H, W, dev, 8)
    kw = dict(n_coarse=80, coarse_factor=cf, TILE=TILE, odds=True)
    out, gd = device_run(RH.render_alpha_multires, scene, gout, H=H, W=W, **kw)
    ref, rg = oracle_run("multires", scene, gout, H, W, **kw)
    compare(out, gd, ref, rg)


@pytest.mark.parametrize("entry", ["cull", "octave"])
def test_noncontiguous_parameters(dev, entry):
    """Parameters passed as strided views (transposed, every other element) give the image and gradients of the
    same values passed contiguous, bit for bit; each base tensor's gradient is the view's gradient in the viewed
    elements and zero elsewhere."""
    H = W = 48
    fn, kw = BATCH_ENTRIES[entry]
    mu, ls, col, op, bg, th = random_scene(400, H, W, seed=33, dev=dev)
    N = mu.shape[1]
    z = lambda t: torch.zeros_like(t)
    bases = {
        "mu": mu.transpose(1, 2).contiguous(),                              # [1, 2, N]
        "ls": torch.stack([ls, z(ls)], -1).reshape(1, N, 4).contiguous(),    # values at [..., ::2]
        "col": col.transpose(1, 2).contiguous(),                            # [1, 3, N]
        "op": torch.stack([op, z(op)], -1).reshape(1, 2 * N).contiguous(),  # values at [:, ::2]
        "bg": torch.stack([bg, z(bg)], -1).reshape(1, 6).contiguous(),      # values at [:, ::2]
        "th": torch.stack([th, z(th)], -1).contiguous(),                    # values at [..., 0]
    }
    views = {
        "mu": lambda b: b.transpose(1, 2), "ls": lambda b: b[..., ::2], "col": lambda b: b.transpose(1, 2),
        "op": lambda b: b[:, ::2], "bg": lambda b: b[:, ::2], "th": lambda b: b[..., 0],
    }
    names = ["mu", "ls", "col", "op", "bg", "th"]
    leaves = {n: bases[n].clone().requires_grad_(True) for n in names}
    args = [views[n](leaves[n]) for n in names]
    assert not any(a.is_contiguous() for a in args[:4])
    gout = gout_for(H, W, dev, 9)
    out = fn(*args[:5], H, W, theta=args[5], odds=True, **kw)
    (out * gout).sum().backward()
    ref = [views[n](bases[n]).contiguous().requires_grad_(True) for n in names]
    out_c = fn(*ref[:5], H, W, theta=ref[5], odds=True, **kw)
    (out_c * gout).sum().backward()
    assert torch.equal(out, out_c)
    for n, r in zip(names, ref):
        g = leaves[n].grad
        assert torch.equal(views[n](g), r.grad), n
        rest = g.clone()
        views[n](rest).zero_()
        assert not rest.any(), f"{n}: gradient outside the viewed elements"


@pytest.mark.parametrize("entry", ["cull", "octave", "multires"])
def test_grad_modes(dev, entry):
    """The image does not depend on whether autograd records the render (no_grad, inference_mode: the binning
    then builds no backward maps), and a render where only the colours and opacities need gradients returns
    exactly those gradients of the full backward, the others None."""
    H = W = 40
    fn, kw = BATCH_ENTRIES[entry]
    scene = random_scene(300, H, W, seed=41, dev=dev)
    gout = gout_for(H, W, dev, 10)
    out, gd = device_run(fn, scene, gout, H=H, W=W, odds=True, **kw)
    with torch.no_grad():
        o_ng = fn(*scene[:5], H, W, theta=scene[5], odds=True, **kw)
    with torch.inference_mode():
        o_im = fn(*scene[:5], H, W, theta=scene[5], odds=True, **kw)
    assert torch.equal(o_ng, out) and torch.equal(o_im, out)
    L = [t.detach().clone() for t in scene]
    L[2].requires_grad_(True)
    L[3].requires_grad_(True)
    o_p = fn(*L[:5], H, W, theta=L[5], odds=True, **kw)
    (o_p * gout).sum().backward()
    assert torch.equal(o_p.detach(), out)
    assert torch.equal(L[2].grad, gd["col"]) and torch.equal(L[3].grad, gd["op"])
    assert all(L[i].grad is None for i in (0, 1, 4, 5))


@pytest.mark.parametrize("entry", ["cull", "octave"])
def test_threads_on_own_streams(dev, entry):
    """Two threads, each on a stream of its own (default priority), rendering and differentiating different scenes
    at the same time five times over, get the images and gradients of the same renders run one after another (the
    count's landing buffer and the error state are per thread, the workspaces per call)."""
    import threading
    H = W = 48
    fn, kw = BATCH_ENTRIES[entry]
    scenes = [random_scene(300, H, W, seed=50 + i, dev=dev) for i in range(2)]
    gouts = [gout_for(H, W, dev, 20 + i) for i in range(2)]
    seq = [device_run(fn, s, g, H=H, W=W, odds=True, **kw) for s, g in zip(scenes, gouts)]
    results, errors = [[], []], []
    main = torch.cuda.current_stream(dev)

    def work(i):
        try:
            st = torch.cuda.Stream(device=dev)
            st.wait_stream(main)
            with torch.cuda.stream(st):
                for _ in range(5):
                    results[i].append(device_run(fn, scenes[i], gouts[i], H=H, W=W, odds=True, **kw))
            st.synchronize()
        except Exception as e:   # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a render thread did not finish"
    assert not errors, errors
    for i in range(2):
        assert len(results[i]) == 5
        for out, g in results[i]:
            assert torch.equal(out, seq[i][0])
            for n in NAMES:
                assert torch.equal(g[n], seq[i][1][n]), n


@pytest.mark.parametrize("H,W", [(1, 1), (3, 200), (200, 3), (7, 9)])
def test_tiny_and_thin_canvases(dev, H, W):
    """Canvases of a single pixel, a few pixel rows or columns, and less than a tile: the culled and the
    coarse/fine renders over partial tiles against the oracle. The octave render refuses them with a RuntimeError, as the reference's
    fails with one (its octave 0 renders on a max(8, H) x max(8, W) canvas that it adds to the H x W field,
    render_triton.py:958-962; the oracle's restatement fails the same way)."""
    scene = random_scene(150, H, W, seed=H * 1000 + W, dev=dev, ls_mean_px=3.0, margin=0.2)
    gout = gout_for(H, W, dev, 11)
    out, gd = device_run(RH.render_alpha_full_triton, scene, gout, H=H, W=W, cull=True, odds=True)
    assert out.shape == (1, 3, H, W)
    ref, rg = oracle_run("cull", scene, gout, H, W, odds=True)
    compare(out, gd, ref, rg)
    kw = dict(n_coarse=50, coarse_factor=8, odds=True)   # the coarse group at max(1, H // cf), cf from min(H, W)
    out, gd = device_run(RH.render_alpha_multires, scene, gout, H=H, W=W, **kw)
    ref, rg = oracle_run("multires", scene, gout, H, W, **kw)
    compare(out, gd, ref, rg)
    with pytest.raises(RuntimeError, match="H, W >= 8"):
        RH.render_alpha_octave(*scene[:5], H, W, theta=scene[5], odds=True)
    if min(H, W) > 1:   # a splat at octave 0 (the whole scene routed there with a large base)
        with pytest.raises(RuntimeError):
            oracle_run("octave", scene, gout, H, W, odds=True, base_texels=1e6)
