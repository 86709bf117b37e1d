"""Pins the float64 render oracle (oracle/render_ref.py, oracle/oracle.c) with closed forms, central
finite differences, the cull->exact limit, and cross-checks between the autograd and analytic backwards."""

import contextlib
import math

import numpy as np
import pytest
import torch

from oracle import binning, c_oracle
from oracle import render_ref as R

f64 = torch.float64


def scene(n, H, W, seed, ls_shift=-2.5, op_hi=1.0, theta=True):
    g = torch.Generator().manual_seed(seed)
    mu = torch.rand(n, 2, generator=g)
    ls = torch.rand(n, 2, generator=g) + ls_shift
    col = torch.rand(n, 3, generator=g)
    op = torch.rand(n, generator=g) * op_hi
    bg = torch.rand(3, generator=g)
    th = torch.rand(n, generator=g) * 3.14 if theta else None
    return mu, ls, col, op, bg, th


def bins(mu, scale, H, W, T=8, cutoff=3.0):
    return binning.build_tiles(mu.detach().float().numpy(), scale.detach().float().numpy(), H, W, T, cutoff)


# ---------------------------------------------------------------- closed forms
def test_single_splat_closed_form():
    H = W = 16
    mu = torch.tensor([[0.5, 0.5]], dtype=f64)
    scale = torch.tensor([[0.1, 0.05]], dtype=f64)
    col = torch.tensor([[0.2, 0.4, 0.8]], dtype=f64)
    op = torch.tensor([0.5], dtype=f64)
    bg = torch.tensor([0.1, 0.0, 1.0], dtype=f64)
    gid, st = bins(mu, scale, H, W)
    out, T, asum, fg = R.cull_composite(mu, scale, col, op, bg, None, gid, st, H, W)
    # pixel (row 9, col 8): centre (9.5/16, 8.5/16); offsets dy = 1.5/16, dx = 0.5/16
    dy, dx = 1.5 / 16, 0.5 / 16
    a = 0.5 * math.exp(-0.5 * ((dy / 0.1) ** 2 + (dx / 0.05) ** 2))
    p = 9 * W + 8
    exp_out = [a * c + (1 - a) * b for c, b in zip([0.2, 0.4, 0.8], [0.1, 0.0, 1.0])]
    assert torch.allclose(out[p], torch.tensor(exp_out, dtype=f64), atol=1e-12)
    assert abs(T[p].item() - (1 - a)) < 1e-12 and abs(asum[p].item() - a) < 1e-12
    # the C oracle agrees
    o2, T2, _, _ = c_oracle.fwd_cull(mu.numpy(), scale.numpy(), None, op.numpy(), col.numpy(), gid, st, H, W, bg=bg.numpy())
    assert np.allclose(o2[p], exp_out, atol=1e-7)


def test_zero_opacity_gives_background_and_clamp():
    H = W = 16
    mu, ls, col, op, bg, th = scene(40, H, W, 1, ls_shift=-2.0)
    scale = R.activate_scale(ls).to(f64)
    gid, st = bins(mu, scale, H, W)
    out, T, _, _ = R.cull_composite(mu.to(f64), scale, col.to(f64), torch.zeros(40, dtype=f64), bg.to(f64),
                                    th.to(f64), gid, st, H, W)
    assert torch.equal(out, bg.to(f64).expand_as(out)) and torch.all(T == 1)
    # opacity 1 at the splat centre hits the clamp: a = float32(1 - 1e-4), T = 1 - a = 1.00017e-4
    mu1 = ((torch.tensor([[8.0, 8.0]]) + 0.5) / 16).to(f64)
    s1 = torch.tensor([[0.05, 0.05]], dtype=f64)
    g1, st1 = bins(mu1, s1, H, W)
    _, T1, _, _ = R.cull_composite(mu1, s1, torch.ones(1, 3, dtype=f64), torch.ones(1, dtype=f64),
                                   torch.zeros(3, dtype=f64), None, g1, st1, H, W)
    assert abs(T1[8 * W + 8].item() - (1.0 - R.CLAMP)) < 1e-12 and abs(1.0 - R.CLAMP - 1.0001659e-4) < 1e-11


def test_theta_none_equals_theta_zero():
    H = W = 24
    mu, ls, col, op, bg, _ = scene(50, H, W, 2)
    sc = R.activate_scale(ls).to(f64)
    gid, st = bins(mu, sc, H, W)
    a = R.cull_composite(mu.to(f64), sc, col.to(f64), op.to(f64), bg.to(f64), None, gid, st, H, W)[0]
    b = R.cull_composite(mu.to(f64), sc, col.to(f64), op.to(f64), bg.to(f64), torch.zeros(50, dtype=f64), gid, st,
                         H, W)[0]
    assert torch.allclose(a, b, atol=1e-14)


def test_odds_two_splat_closed_form():
    H = W = 8
    mu = torch.tensor([[4.5 / 8, 4.5 / 8], [4.5 / 8, 4.5 / 8]], dtype=f64)
    scale = torch.tensor([[0.2, 0.2], [0.3, 0.1]], dtype=f64)
    col = torch.tensor([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]], dtype=f64)
    op = torch.tensor([0.9, 0.3], dtype=f64)
    gid, st = bins(mu, scale, H, W)
    S = R.cull_fields(mu, scale, col, op, None, gid, st, H, W, odds=True)
    p = 4 * W + 4                                                         # the shared centre pixel
    w1, w2 = 0.9 / 0.1, 0.3 / 0.7
    assert abs(S[1][p].item() - (w1 + w2)) < 1e-12
    assert torch.allclose(S[2][p], torch.tensor([w1, 0.0, w2], dtype=f64), atol=1e-12)
    assert abs(S[0][p].item() - (math.log(0.1) + math.log(0.7))) < 1e-12


# ---------------------------------------------------------------- gradients
def test_autograd_matches_central_differences():
    H = W = 16
    mu, ls, col, op, bg, th = scene(12, H, W, 3, ls_shift=-2.0, op_hi=0.8)
    L = R.leaves(mu, ls, col, op, bg, th)
    g = torch.Generator().manual_seed(9)
    gout = torch.randn(H * W, 3, generator=g, dtype=f64)
    sc0 = R.activate_scale(L[1]).detach()
    gid, st = bins(L[0], sc0, H, W, cutoff=3.0)

    def loss(mu_, ls_, col_, op_, bg_, th_):
        out = R.cull_composite(mu_, R.activate_scale(ls_), col_, op_, bg_, th_, gid, st, H, W)[0]
        return (out * gout).sum()

    loss(*L).backward()
    eps = 1e-6
    for i, t in enumerate(L):
        for j in range(min(4, t.numel())):
            idx = np.unravel_index(j * 3 % t.numel(), t.shape)
            args = [x.detach().clone() for x in L]
            args[i][idx] += eps
            lp = loss(*args).item()
            args[i][idx] -= 2 * eps
            lm = loss(*args).item()
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - t.grad[idx].item()) <= 1e-6 * max(1.0, abs(fd)), (i, idx, fd, t.grad[idx].item())


@pytest.mark.parametrize("odds", [False, True])
@pytest.mark.parametrize("fields", [False, True])
@pytest.mark.parametrize("has_theta", [True, False])
def test_c_analytic_backward_matches_autograd(odds, fields, has_theta):
    H, W = 24, 32
    mu, ls, col, op, bg, th = scene(80, H, W, 4, op_hi=0.99, theta=has_theta)
    sc = R.activate_scale(ls)                                             # fp32 activated scale, as kernels get
    m64, s64, c64, o64, b64 = (x.to(f64).requires_grad_(True) for x in (mu, sc, col, op, bg))
    t64 = th.to(f64).requires_grad_(True) if has_theta else None
    gid, st = bins(mu, sc, H, W)
    g = torch.Generator().manual_seed(5)
    if fields:
        S = R.cull_fields(m64, s64, c64, o64, t64, gid, st, H, W, odds=odds)
        ups = [torch.randn(s.shape, generator=g, dtype=f64) for s in S]
        sum((s * u).sum() for s, u in zip(S, ups)).backward()
        ref = c_oracle.bwd_cull(mu.numpy(), sc.numpy(), None if th is None else th.numpy(), op.numpy(), col.numpy(),
                                gid, st, H, W, odds=odds, fields=True, dslog=ups[0].numpy(), dsa=ups[1].numpy(),
                                dsac=ups[2].numpy())
    else:
        out, T, asum, fg = R.cull_composite(m64, s64, c64, o64, b64, t64, gid, st, H, W, odds=odds)
        gout = torch.randn(out.shape, generator=g, dtype=f64)
        (out * gout).sum().backward()
        ref = c_oracle.bwd_cull(mu.numpy(), sc.numpy(), None if th is None else th.numpy(), op.numpy(), col.numpy(),
                                gid, st, H, W, odds=odds, fields=False, bg=bg.numpy(), T=T.detach().numpy(),
                                asum=asum.detach().numpy(), fg=fg.detach().numpy(), gout=gout.numpy())
        assert np.allclose(ref["bg"], b64.grad.numpy(), rtol=1e-9, atol=1e-12)
    pairs = [("mu", m64), ("scale", s64), ("col", c64), ("op", o64)] + ([("theta", t64)] if has_theta else [])
    for name, t in pairs:
        a = t.grad.numpy().reshape(ref[name].shape)
        assert np.allclose(ref[name], a, rtol=1e-9, atol=1e-12 * max(1.0, np.abs(a).max())), name


def test_c_forward_matches_torch_forward():
    H, W = 40, 24
    mu, ls, col, op, bg, th = scene(200, H, W, 6, op_hi=0.99)
    sc = R.activate_scale(ls)
    gid, st = bins(mu, sc, H, W)
    for odds in (False, True):
        S = R.cull_fields(mu.to(f64), sc.to(f64), col.to(f64), op.to(f64), th.to(f64), gid, st, H, W, odds=odds)
        C = c_oracle.fwd_cull(mu.numpy(), sc.numpy(), th.numpy(), op.numpy(), col.numpy(), gid, st, H, W, odds=odds,
                              fields=True)
        for a, b in zip(S, C):
            assert np.allclose(a.numpy(), b, rtol=1e-12, atol=1e-12)
        out = R.cull_composite(mu.to(f64), sc.to(f64), col.to(f64), op.to(f64), bg.to(f64), th.to(f64), gid, st, H, W,
                               odds=odds)
        Co = c_oracle.fwd_cull(mu.numpy(), sc.numpy(), th.numpy(), op.numpy(), col.numpy(), gid, st, H, W, odds=odds,
                               fields=False, bg=bg.numpy())
        for a, b in zip(out, Co):
            assert np.allclose(a.numpy(), b, rtol=1e-12, atol=1e-12)


def test_float32_rotation_and_offset_options_single_splat():
    """`c_oracle.rot32` (cos and sin rounded to float32) and `c_oracle.off32` (pixel-centre offsets from the splat
    centre rounded to float32) on one elongated rotated splat whose centre lies near the canvas' left edge, so that
    the float32 offsets of the pixels along its long axis are not exact (pixel and splat centre more than a factor of
    two apart): in each of the four combinations S_log equals the single-splat closed form evaluated in numpy with the
    same roundings, and each option changes the result; at theta = 0 (cos and sin exact in float32) rot32 changes
    nothing."""
    H, W = 24, 40
    mu = np.array([[0.4137, 0.0213]], np.float32)
    sc = np.array([[0.006, 0.3]], np.float32)
    op = np.array([0.8], np.float32)
    col = np.ones((1, 3), np.float32)
    gid, st = binning.build_tiles(mu, sc, H, W, 8, 3.0)
    ntx = (W + 7) // 8
    tiles = np.repeat(np.arange(len(st) - 1), np.diff(st))
    yy, xx = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    covered = np.isin((yy // 8) * ntx + xx // 8, tiles).reshape(-1)
    py32 = ((yy + np.float32(0.5)) / np.float32(H)).astype(np.float32).reshape(-1)
    px32 = ((xx + np.float32(0.5)) / np.float32(W)).astype(np.float32).reshape(-1)

    def closed_form(theta, r32, o32):
        th = np.float64(np.float32(theta))
        c, s = np.cos(th), np.sin(th)
        if r32:
            c, s = float(np.float32(c)), float(np.float32(s))
        if o32:
            dy = (py32 - mu[0, 0]).astype(np.float64)       # float32 subtraction, rounded once
            dx = (px32 - mu[0, 1]).astype(np.float64)
        else:
            dy = py32.astype(np.float64) - np.float64(mu[0, 0])
            dx = px32.astype(np.float64) - np.float64(mu[0, 1])
        ry, rx = c * dy + s * dx, -s * dy + c * dx
        m = ry ** 2 / np.float64(sc[0, 0]) ** 2 + rx ** 2 / np.float64(sc[0, 1]) ** 2
        a = np.minimum(np.exp(-0.5 * m) * np.float64(op[0]), R.CLAMP)
        return np.where(covered, np.log(1.0 - a), 0.0)

    def oracle(theta, r32, o32):
        th = np.array([theta], np.float32)
        with contextlib.ExitStack() as es:
            if r32:
                es.enter_context(c_oracle.rot32())
            if o32:
                es.enter_context(c_oracle.off32())
            return c_oracle.fwd_cull(mu, sc, th, op, col, gid, st, H, W, fields=True)[0]

    got = {}
    for r32 in (False, True):
        for o32 in (False, True):
            got[r32, o32] = oracle(0.37, r32, o32)
            want = closed_form(0.37, r32, o32)
            assert np.allclose(got[r32, o32], want, rtol=1e-12, atol=0.0), (r32, o32)
    assert np.abs(got[True, False] - got[False, False]).max() > 1e-9
    assert np.abs(got[False, True] - got[False, False]).max() > 1e-9
    assert np.array_equal(oracle(0.0, True, False), oracle(0.0, False, False))


@pytest.mark.parametrize("odds", [False, True])
def test_fields_alpha_sensitivity_matches_central_differences(odds):
    """The C oracle's sensitivities of the fields to a relative change of every unclamped alpha (the condition
    behind the GPU tests' fields bar) equal central differences of the float64 torch fields over opacity (1 +- e),
    which scales every alpha below the clamp by the same factor; a splat of opacity 1 centred on a pixel puts pairs
    on the clamp, whose share is zero. The colour term takes |c|: negating the colours leaves it unchanged."""
    H, W = 24, 24
    mu, ls, col, op, bg, th = scene(60, H, W, 11, ls_shift=-2.0, op_hi=0.95)
    mu[0] = torch.tensor([12.5 / 24, 12.5 / 24])
    op[0] = 1.0
    sc = R.activate_scale(ls)
    gid, st = bins(mu, sc, H, W)
    args = [mu.numpy(), sc.numpy(), th.numpy(), op.numpy()]
    _, _, _, K = c_oracle.fwd_cull(*args, col.numpy(), gid, st, H, W, odds=odds, fields=True, cond=True)
    _, _, _, Kn = c_oracle.fwd_cull(*args, -col.numpy(), gid, st, H, W, odds=odds, fields=True, cond=True)
    e = 1e-6
    Sp, Sm = (R.cull_fields(mu.to(f64), sc.to(f64), col.to(f64), op.to(f64) * (1 + s * e), th.to(f64), gid, st, H, W,
                            odds=odds) for s in (1, -1))
    fd = [(p - m).numpy() / (2 * e) for p, m in zip(Sp, Sm)]
    assert K[0].max() > 1.0
    for k, d, sign in zip(K, fd, (-1.0, 1.0, 1.0)):
        assert np.allclose(k, sign * d, rtol=1e-6, atol=1e-9 * np.abs(k).max())
    assert np.array_equal(K[2], Kn[2])
    # at the splat centre the clamped pair adds nothing: the clamp holds a, and a (1 + e) stays on it
    p = 12 * W + 12
    base = c_oracle.fwd_cull(*[a[1:] for a in args], col.numpy()[1:], *bins(mu[1:], sc[1:], H, W), H, W, odds=odds,
                             fields=True, cond=True)[3]
    assert abs(K[0][p] - base[0][p]) <= 1e-12 * max(1.0, K[0][p])


# ---------------------------------------------------------------- limits and identities
def test_cull_converges_to_exact():
    H = W = 32
    mu, ls, col, op, bg, th = scene(150, H, W, 7, ls_shift=-2.5)
    sc = R.activate_scale(ls).to(f64)
    ex = R.exact(mu.to(f64), sc, col.to(f64), op.to(f64), bg.to(f64), th.to(f64), H, W)
    errs = []
    for cutoff in (3.0, 5.0, 9.0):
        gid, st = bins(mu, sc, H, W, cutoff=cutoff)
        cu = R.cull_composite(mu.to(f64), sc, col.to(f64), op.to(f64), bg.to(f64), th.to(f64), gid, st, H, W)[0]
        errs.append((cu - ex).abs().max().item())
    assert errs[0] > errs[1] > errs[2] and errs[2] < 1e-6
    assert errs[0] < 5e-2


def test_exact_f32_restatement_close_to_f64():
    H = W = 16
    mu, ls, col, op, bg, th = scene(64, H, W, 8, ls_shift=-2.0)
    sc = R.activate_scale(ls)
    ex = R.exact(mu.to(f64), sc.to(f64), col.to(f64), op.to(f64), bg.to(f64), th.to(f64), H, W)
    f32 = R.render_alpha_full_f32(mu[None], ls[None], col[None], op[None], bg[None], H, W, theta=th[None])[0]
    assert (f32.to(f64) - ex).abs().max().item() < 1e-5
    ys, xs = R.linspace_centres(H, W)[:, 0].reshape(H, W)[:, 0], R.linspace_centres(H, W)[:W, 1]
    rows = c_oracle.exact_rows_f32(mu.numpy(), sc.numpy(), th.numpy(), op.numpy(), col.numpy(), ys.float().numpy(),
                                   xs.float().numpy(), 0, H, bg.numpy())
    assert np.abs(rows.reshape(-1, 3) - ex.numpy()).max() < 1e-5


def test_multires_and_octave_identities():
    H = W = 32
    mu, ls, col, op, bg, th = scene(120, H, W, 9)
    sc = R.activate_scale(ls)
    m, s, c, o, b, t = (x.to(f64) for x in (mu, sc, col, op, bg, th))
    gid, st = bins(mu, sc, H, W)
    cull = R.composite(*R.cull_fields(m, s, c, o, t, gid, st, H, W), b, straight_through=False)[0]
    assert torch.allclose(R.multires(m, s, c, o, b, t, H, W, n_coarse=None), cull, atol=1e-14)
    assert torch.allclose(R.octave(m, s, c, o, b, t, H, W, max_octaves=0), cull, atol=1e-14)
    # splitting a group is exact at one resolution (the monoid): two halves at full res sum to the whole
    half = 60
    S1 = R.fields_group(m[:half], s[:half], c[:half], o[:half], t[:half], H, W, 8, 3.0, False)
    S2 = R.fields_group(m[half:], s[half:], c[half:], o[half:], t[half:], H, W, 8, 3.0, False)
    S = R.cull_fields(m, s, c, o, t, gid, st, H, W)
    for a1, a2, a in zip(S1, S2, S):
        assert torch.allclose(a1 + a2, a, atol=1e-12)
