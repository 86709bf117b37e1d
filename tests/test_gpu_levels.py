"""Fused multi-level renders (octave routing and the coarse/fine split, render_triton.py:879-980).

* routing and per-level pair lists bit-exact against the oracle's per-group binning of the same splats;
* the upsample adjoint against torch's bilinear backward (float64, CPU);
* images within 1e-5 max-abs and gradients within 1e-4 relative at the benchmark size, against the float64
  C oracle composed level by level (fields per level, torch float64 upsample + composite + autograd for
  the glue, then the C oracle's fields backward per level).
"""

import contextlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _gpu_util import GRAD_REL_TOL, IMG_TOL, RH, activate_scale, check_per_splat, np_, random_scene, rel_err
from gaussian_splat_encoder import _lib, synth
from oracle import c_oracle
from oracle import render_ref as R

pytestmark = pytest.mark.gpu


def octave_lv(max_octaves=6, base=8.0):
    return _lib.SplatLevels(1, max_octaves, base, 0, 0, 0)


def split_lv(H, W, n_coarse, cf=8):
    cf = min(cf, max(1, min(H, W) // 8))
    return _lib.SplatLevels(2, 0, 0.0, n_coarse, max(1, H // cf), max(1, W // cf))


def device_level_bins(mu, sc, H, W, TILE, lv, cutoff=3.0):
    B, N, _ = mu.shape
    col = torch.zeros(B, N, 1, device=mu.device)
    op = torch.zeros(B, N, device=mu.device)
    return RH._bin(mu, sc, col, op, None, H, W, TILE, cutoff, lv=lv)


def oracle_levels(sc32, H, W, lv, n_levels):
    """Each splat's level as the reference routes it (render_triton.py:925-932, :950-952, :904-913), with
    octaves past the last distinct canvas folded into the last level."""
    N = sc32.shape[0]
    if lv.mode == 1:
        o = R.octave_of(torch.from_numpy(sc32), H, W, lv.base_texels, lv.max_octaves).numpy()
        return np.minimum(o, n_levels - 1)
    if lv.mode == 2:
        return np.where(np.arange(N) < lv.n_coarse, 1, 0)
    return np.zeros(N, np.int64)


def check_level_bins(mu, sc, H, W, TILE, lv, cutoff=3.0):
    bins = device_level_bins(mu, sc, H, W, TILE, lv, cutoff)
    for b in range(mu.shape[0]):
        mu_b, sc_b = np_(mu[b]), np_(sc[b])
        lev_o = oracle_levels(sc_b, H, W, lv, bins.n_levels)
        lev_d = bins.rect_b[b][:, 3].cpu().numpy()
        assert np.array_equal(lev_d, lev_o), f"routing differs at {np.nonzero(lev_d != lev_o)[0][:5]}"
        gid = bins.gid_b[b].cpu().numpy()
        st = bins.starts_b[b].cpu().numpy()
        for l, (Hl, Wl, ntx, tb, pb) in enumerate(bins.geom):
            te = bins.geom[l + 1][3] if l + 1 < bins.n_levels else bins.nt
            idx = np.nonzero(lev_o == l)[0]
            gid_o, st_o = c_oracle.build_tiles(mu_b[idx], sc_b[idx], Hl, Wl, TILE, cutoff)
            st_l = st[tb:te + 1] - st[tb]
            assert np.array_equal(st_l, st_o), f"level {l}: tile starts differ"
            assert np.array_equal(gid[st[tb]:st[te]], idx[gid_o[:st_o[-1]]]), f"level {l}: pair list differs"
            assert bins.level_tot_b[b][l] == st_o[-1]
    return bins


@pytest.mark.parametrize("name,TILE", [("c1", 8), ("c4", 8), ("c1", 16)])
def test_octave_routing_and_pairs_bit_exact(dev, name, TILE):
    s = synth.config(name)
    mu = s.mu.to(dev)
    sc = activate_scale(s.log_scale.to(dev))
    bins = check_level_bins(mu, sc, s.H, s.W, TILE, octave_lv())
    assert sum(1 for n in bins.level_tot_b[0] if n) >= 2   # the scene spans several octaves


@pytest.mark.parametrize("H,W,TILE,mo,n,margin", [
    (100, 60, 8, 6, 3000, 0.2),    # ragged canvas; octaves clamp to 8 on the short side first
    (64, 64, 4, 20, 2000, 0.0),    # octaves past (8, 8) fold into one level
    (768, 768, 8, 0, 5000, 0.1),   # octave 0 only: the single-canvas pair list
])
def test_octave_edge_cases_bit_exact(dev, H, W, TILE, mo, n, margin):
    mu, ls, *_ = random_scene(n, H, W, seed=H + n + mo, dev=dev, ls_mean_px=12.0, ls_std=1.2, margin=margin,
                              B=2)
    check_level_bins(mu, activate_scale(ls), H, W, TILE, octave_lv(mo))


def test_split_bit_exact(dev):
    H, W = 200, 120
    mu, ls, *_ = random_scene(2500, H, W, seed=9, dev=dev, ls_mean_px=6.0)
    check_level_bins(mu, activate_scale(ls), H, W, 8, split_lv(H, W, 700))


@pytest.mark.parametrize("C", [1, 2, 3, 4])
@pytest.mark.parametrize("H,W", [(100, 60), (16, 1536), (8, 3584)])
def test_upsample_adjoint_matches_torch(dev, H, W, C):
    """dS_l = (d upsample_l / d field_l)^T dS_0 for every coarse level, against torch's bilinear backward. The
    widths take each way the column pass reads a level-0 row: staged in LDS as it lies in memory (60), staged as
    de-interleaved planes with rotated 64-word rows (1536, rows of 1024 pixels and more), and from global memory
    (3584 with C >= 3: 2 + C planes of 3584 floats exceed the 64 KiB of LDS a workgroup stages; with C = 1 or
    2 that width is staged rotated). The wide rows' level widths
    are the row's width over powers of two, so the float32 source positions of the kernels carry no rounding
    that the float64 reference would not (at 1500 wide, 187 texels per row put them about 1e-7 x 1500 apart).
    Colour channel counts 1 to 4 (the rotated layout keeps one plane per channel)."""
    lv = octave_lv(6)
    geom, nt, npix = RH.levels_geometry(H, W, 8, lv)
    g = torch.Generator().manual_seed(4)
    d0 = [torch.randn(H * W, generator=g, dtype=torch.float64), torch.randn(H * W, generator=g, dtype=torch.float64),
          torch.randn(H * W, C, generator=g, dtype=torch.float64)]
    dl = torch.zeros(npix, device=dev); da = torch.zeros(npix, device=dev); dc = torch.zeros(npix, C, device=dev)
    dl[:H * W] = d0[0].float().to(dev); da[:H * W] = d0[1].float().to(dev); dc[:H * W] = d0[2].float().to(dev)
    lib = _lib.load()
    mask = (1 << len(geom)) - 1
    lvr = _lib.ctypes.byref(lv)
    ws = torch.empty(lib.splat_upsample_adjoint_workspace_bytes(C, H, W, 8, lvr), dtype=torch.uint8, device=dev)
    _lib.check(lib.splat_upsample_adjoint(C, H, W, 8, lvr, mask, dl.data_ptr(), da.data_ptr(), dc.data_ptr(),
                                          ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev)), "adjoint")
    for l, (Hl, Wl, _, _, pb) in enumerate(geom[1:], start=1):
        for k, (got, up) in enumerate(zip((dl, da, dc), d0)):
            x = torch.zeros((Hl * Wl,) + up.shape[1:], dtype=torch.float64, requires_grad=True)
            (R.upsample_field(x, Hl, Wl, H, W) * up.reshape((H * W,) + up.shape[1:])).sum().backward()
            ref = x.grad.numpy()
            e = np.abs(np_(got[pb:pb + Hl * Wl]) - ref.reshape(-1, *up.shape[1:])).max() / np.abs(ref).max()
            assert e <= 1e-5, f"level {l} term {k}: rel {e:.2e}"


def composite_bwd_on(T, S_a, fg, bg, gout):
    """float64 gradients of the octave/multires composite (render_triton.py:918-921, 976-980: T = exp(S_log),
    asum = S_a.clamp_min(1e-8), fg = S_ac / asum, out = (1 - T) fg + T bg) w.r.t. S_log [P], S_a [P], S_ac [P,C]
    and bg [C], evaluated at given forward quantities T [P], unclamped S_a [P] and fg [P,C] (clamp_min passes the
    gradient where S_a >= 1e-8)."""
    T, S_a, fg, bg, gout = (np.asarray(a, np.float64) for a in (T, S_a, fg, bg, gout))
    asum = np.maximum(S_a, 1e-8)
    omt = 1.0 - T
    d_slog = T * (gout * (bg[None, :] - fg)).sum(-1)
    d_sac = gout * (omt / asum)[:, None]
    d_sa = np.where(S_a >= 1e-8, -(omt / asum) * (gout * fg).sum(-1), 0.0)
    return d_slog, d_sa, d_sac, (gout * T[:, None]).sum(0)


def composed_oracle(mu, sc, col, op, bg, th, H, W, TILE, lv, odds, gout, cutoff=3.0, fwd=None):
    """float64 oracle of one batch: C-oracle fields per level, torch float64 glue, C-oracle fields backward.
    Returns the image [P, C] and the gradients w.r.t. (mu, activated scale, colour, opacity, bg, theta), plus
    each splat's opacity-gradient scale ("op_scale", see c_oracle.bwd_cull). fwd = (T, S_a, fg): the backward
    starts from these forward quantities (the device forward's) instead of the oracle's own, so that it checks the
    backward alone where float32 forward rounding decides the gradients (1 - T below float32 resolution, S_a at
    the clamp)."""
    mu_, sc_, col_, op_, bg_ = np_(mu), np_(sc), np_(col), np_(op), np_(bg)
    th_ = None if th is None else np_(th)
    N, C = col_.shape
    geom, _, _ = RH.levels_geometry(H, W, TILE, lv)
    lev = oracle_levels(sc_, H, W, lv, len(geom))
    sub = lambda a, idx: None if a is None else a[idx]
    per_level, leaves = [], []
    S = None
    for l, (Hl, Wl, *_r) in enumerate(geom):
        idx = np.nonzero(lev == l)[0]
        if idx.size == 0:
            continue
        args = [sub(mu_, idx), sub(sc_, idx), sub(th_, idx), sub(op_, idx), sub(col_, idx)]
        gid, st = c_oracle.build_tiles(args[0], args[1], Hl, Wl, TILE, cutoff)
        f = [torch.from_numpy(np.ascontiguousarray(x)).requires_grad_(True)
             for x in c_oracle.fwd_cull(*args, gid, st, Hl, Wl, TILE, odds=odds, fields=True)]
        up = f if l == 0 else [R.upsample_field(x, Hl, Wl, H, W) for x in f]
        S = up if S is None else [a + b for a, b in zip(S, up)]
        per_level.append((l, idx, args, gid, st, Hl, Wl))
        leaves.append(f)
    if S is None:
        S = [torch.zeros(H * W, dtype=torch.float64), torch.zeros(H * W, dtype=torch.float64),
             torch.zeros(H * W, C, dtype=torch.float64)]
    bg64 = torch.from_numpy(bg_.astype(np.float64)).requires_grad_(True)
    out = R.composite(*S, bg64, straight_through=False)[0]
    if fwd is None:
        (out * torch.from_numpy(np_(gout)).double()).sum().backward()
        g_bg = bg64.grad.numpy()
    else:   # the composite's gradients at the given forward quantities, through the same upsample adjoints
        d_slog, d_sa, d_sac, g_bg = composite_bwd_on(*fwd, bg_, np_(gout))
        if leaves:
            dS = [torch.from_numpy(d_slog), torch.from_numpy(d_sa), torch.from_numpy(d_sac)]
            sum((s_ * d).sum() for s_, d in zip(S, dS)).backward()
    grads = {"mu": np.zeros((N, 2)), "scale": np.zeros((N, 2)), "col": np.zeros((N, C)), "op": np.zeros(N),
             "theta": np.zeros(N) if th is not None else None, "bg": g_bg}
    mag = {k: np.zeros_like(v) for k, v in grads.items() if v is not None and k != "bg"}
    # each splat's scale ('mag') sums the magnitudes of every term along the whole chain: the composite's
    # per-channel terms, the upsample adjoint's per-destination terms (non-negative weights: the adjoint of the
    # magnitudes), then the fields backward's terms on those magnitudes
    if fwd is None:
        T0 = torch.exp(S[0]).detach().numpy()
        Sa0 = S[1].detach().numpy()
        fg0 = (S[2] / S[1].clamp_min(1e-8)[:, None]).detach().numpy()
    else:
        T0, Sa0, fg0 = (np.asarray(a, np.float64) for a in fwd)
    go = np.abs(np_(gout)).astype(np.float64)
    r0 = (1.0 - T0) / np.maximum(Sa0, 1e-8)
    m0 = [T0 * (go * np.abs(bg_[None, :].astype(np.float64) - fg0)).sum(-1),
          np.where(Sa0 >= 1e-8, r0 * (go * np.abs(fg0)).sum(-1), 0.0), go * np.abs(r0)[:, None]]
    for (l, idx, args, gid, st, Hl, Wl), f in zip(per_level, leaves):
        d = [x.grad.numpy() if x.grad is not None else np.zeros(x.shape) for x in f]
        gl = c_oracle.bwd_cull(*args, gid, st, Hl, Wl, TILE, odds=odds, fields=True, dslog=d[0], dsa=d[1], dsac=d[2])
        if l == 0:
            dm = m0
        else:   # adjoint of the upsample applied to the magnitudes
            xs = [torch.zeros(x.shape, dtype=torch.float64, requires_grad=True) for x in f]
            sum((R.upsample_field(x, Hl, Wl, H, W) * torch.from_numpy(m)).sum() for x, m in zip(xs, m0)).backward()
            dm = [x.grad.numpy() for x in xs]
        gm = c_oracle.bwd_cull(*args, gid, st, Hl, Wl, TILE, odds=odds, fields=True, dslog=dm[0], dsa=dm[1],
                               dsac=dm[2])
        for k in ("mu", "scale", "col", "op", "theta"):
            if grads[k] is not None:
                grads[k][idx] = gl[k]
                mag[k][idx] = np.maximum(gl["mag"][k], gm["mag"][k])
    grads["mag"] = mag
    grads["op_scale"] = mag["op"]
    return out.detach().numpy(), grads


def run_levels(mu, ls, col, op, bg, th, H, W, TILE, lv, odds, seed, img_tol=IMG_TOL, grad_tol=GRAD_REL_TOL,
               want_grads=False, per_splat=True, bwd_on_device_fwd=False, rot32=True):
    """Fused level render of one batch against composed_oracle: the image, every gradient tensor and, with
    per_splat, every gradient component of every splat against that splat's own scale (check_per_splat).
    bwd_on_device_fwd: the gradients are held against the oracle's backward from the device forward's T, S_a and
    fg (the image still against the oracle's own forward). rot32: as in test_gpu_render.run_case. Returns the bins,
    and with want_grads also the device gradients by name and the oracle's."""
    with (c_oracle.rot32() if rot32 else contextlib.nullcontext()):
        return _run_levels(mu, ls, col, op, bg, th, H, W, TILE, lv, odds, seed, img_tol, grad_tol, want_grads,
                           per_splat, bwd_on_device_fwd)


def _run_levels(mu, ls, col, op, bg, th, H, W, TILE, lv, odds, seed, img_tol, grad_tol, want_grads, per_splat,
                bwd_on_device_fwd):
    sc = activate_scale(ls)
    P, C = H * W, col.shape[-1]
    out, (T, asum, fg), bins = RH._forward_levels(mu, sc, col, op, bg, th, H, W, TILE, 3.0, None, odds, lv)
    gout = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed)).to(mu.device)
    g_mu, g_sc, g_col, g_op, g_bg, g_th = RH._backward_levels(gout, col, bg, th is not None, T, asum, fg, bins, odds)
    fwd = (np_(T[0]), np_(asum[0]), np_(fg[0])) if bwd_on_device_fwd else None
    img_ref, gref = composed_oracle(mu[0], sc[0], col[0], op[0], bg[0], None if th is None else th[0], H, W, TILE,
                                    lv, odds, gout[0], fwd=fwd)
    d = np.abs(np_(out[0]) - img_ref.reshape(P, C)).max()
    assert d <= img_tol, f"image max-abs {d:.2e}"
    for name, got in (("mu", g_mu), ("scale", g_sc), ("col", g_col), ("op", g_op), ("bg", g_bg), ("theta", g_th)):
        if got is None:
            assert gref[name] is None
            continue
        e = rel_err(np_(got[0]), gref[name])
        assert e <= grad_tol, f"grad {name}: rel {e:.2e}"
    if per_splat:
        check_per_splat({"mu": g_mu, "scale": g_sc, "col": g_col, "op": g_op, "theta": g_th}, gref)
    if want_grads:
        return bins, {"mu": g_mu, "scale": g_sc, "col": g_col, "op": g_op, "bg": g_bg, "theta": g_th}, gref
    return bins


@pytest.mark.parametrize("odds", [False, True])
def test_octave_full_size(dev, odds):
    """The headline scene rendered with octave routing: 768 x 768, 92,160 splats, forward and backward."""
    s = synth.config("c2").to(dev)
    bins = run_levels(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.theta, s.H, s.W, 8, octave_lv(), odds, seed=3)
    assert sum(1 for n in bins.level_tot_b[0] if n) >= 2


@pytest.mark.parametrize("H,W,TILE,mo", [(100, 60, 8, 6), (64, 64, 4, 20), (48, 80, 16, 3)])
def test_octave_ragged_and_folded(dev, H, W, TILE, mo):
    scene = random_scene(1500, H, W, seed=H * W + mo, dev=dev, ls_mean_px=10.0, ls_std=1.2, op_max=0.8)
    run_levels(*scene, H, W, TILE, octave_lv(mo), odds=True, seed=5)


def test_octave_level0_empty(dev):
    """Every splat routed to coarse octaves: the composite sees only upsampled fields."""
    H = W = 64
    scene = random_scene(300, H, W, seed=8, dev=dev, ls_mean_px=30.0, ls_std=0.2, op_max=0.5)
    bins = run_levels(*scene, H, W, 8, octave_lv(), odds=False, seed=6)
    assert bins.level_tot_b[0][0] == 0


def test_split_levels(dev):
    H, W = 120, 96
    scene = list(random_scene(900, H, W, seed=12, dev=dev, ls_mean_px=3.0))
    ls = scene[1].clone()
    ls[:, :150] += float(np.log(6.0))       # the coarse group holds the large splats
    scene[1] = ls
    run_levels(*scene, H, W, 8, split_lv(H, W, 150), odds=False, seed=7)
    run_levels(*scene, H, W, 8, split_lv(H, W, 150, cf=4), odds=True, seed=8)


def test_empty_scene_levels(dev):
    """No splats: the image is the background and g_bg = sum_p gout."""
    H = W = 32
    z = lambda *s: torch.zeros(*s, device=dev)
    mu, ls, col, op = z(1, 0, 2), z(1, 0, 2), z(1, 0, 3), z(1, 0)
    bg = torch.rand(1, 3, device=dev)
    for fn in (RH.render_alpha_octave, RH.render_alpha_multires):
        b = bg.clone().requires_grad_(True)
        out = fn(mu, ls, col, op, b, H, W)
        assert torch.allclose(out, b[:, :, None, None].expand_as(out))
        out.sum().backward()
        assert torch.allclose(b.grad, torch.full_like(bg, float(H * W)))


def test_level_budget(dev):
    """The budget applies per level (each level is one binned group of the reference)."""
    s = synth.config("c1")
    mu, ls = s.mu.to(dev), s.log_scale.to(dev)
    bins = device_level_bins(mu, activate_scale(ls), s.H, s.W, 8, octave_lv())
    worst = max(bins.level_tot_b[0])
    col, op = s.color.to(dev), s.opacity.to(dev)
    RH.render_alpha_octave(mu, ls, col, op, s.bg.to(dev), s.H, s.W, max_pairs=worst)
    with pytest.raises(RH.PairBudgetExceeded):
        RH.render_alpha_octave(mu, ls, col, op, s.bg.to(dev), s.H, s.W, max_pairs=worst - 1)


@pytest.mark.parametrize("odds", [False, True])
def test_octave_dense_coarse_level(dev, odds):
    """Many large splats on one coarse octave (a few dozen tiles of thousands of pairs): its tiles are split over
    many workgroups in the FIELDS forward and backward; images and gradients against the composed oracle."""
    H = W = 256
    scene = random_scene(2500, H, W, seed=31, dev=dev, ls_mean_px=24.0, ls_std=0.15, op_max=0.6)
    bins = run_levels(*scene, H, W, 8, octave_lv(), odds=odds, seed=11)
    lt = bins.level_tot_b[0]
    assert max(RH._level_splits(bins, lt, bins.level_mask(0) & ~1)) >= 4, "the scene must split a coarse level"
