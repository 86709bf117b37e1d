"""torch float64 (CPU) restatement of the reference renderer. TEST INFRASTRUCTURE ONLY (see oracle/__init__).

All functions take one batch unless noted, with fp32 inputs promoted to float64 leaves; gradients come
from autograd. Pixel centres are computed in fp32 first, exactly as the reference does, then promoted.

Reference map:
  cull_fields / cull_composite   render_triton.py:423-517 (S_log, S_a, S_ac; composite :509-517)
  composite backward convention  render_triton.py:650-654: dS_a = -sum(dfg*fg)/asum even where asum is
                                 clamped, reproduced with a straight-through clamp
  exact                          render.py:34-58, 61-65, 90-110 (materialised, linspace pixel centres)
  odds_exact                     render_triton.py:1431-1457 (`_torch_odds_ref`)
  multires / octave              render_triton.py:864-922, 925-980
  octave_forward_c               render_triton.py:935-980 forward with the C oracle's fields (full-size frames)
  render_alpha_full_f32          render.py:90-110 in float32: the CPU baseline (reference's own CPU path)
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import binning

CLAMP = float(np.float32(1.0 - 1e-4))   # the clamp as the reference applies it to float32 alphas (render_triton.py:106)
f64 = torch.float64


def activate_scale(log_scale: torch.Tensor) -> torch.Tensor:
    """params.py:28, in the dtype of the input."""
    return F.softplus(log_scale) + 1e-4


def cull_centres(H: int, W: int):
    """fp32 (i + 0.5) / size, promoted (render_triton.py:455-456)."""
    ys = ((torch.arange(H, dtype=torch.float32) + 0.5) / H).to(f64)
    xs = ((torch.arange(W, dtype=torch.float32) + 0.5) / W).to(f64)
    return ys, xs


def linspace_centres(H: int, W: int):
    """render.py:61-65 pixel centres in fp32, promoted; returns [P, 2] (y, x)."""
    ys = torch.linspace(0.5 / H, 1 - 0.5 / H, H, dtype=torch.float32)
    xs = torch.linspace(0.5 / W, 1 - 0.5 / W, W, dtype=torch.float32)
    gy, gx = torch.meshgrid(ys, xs, indexing="ij")
    return torch.stack([gy, gx], dim=-1).reshape(H * W, 2).to(f64)


def _alpha(py, px, mu, scale, opacity, theta):
    """Per-(pixel, splat) alpha with broadcasting; also returns fo = opacity * falloff (pre-clamp)."""
    dy = py - mu[..., 0]
    dx = px - mu[..., 1]
    if theta is not None:
        c, s = torch.cos(theta), torch.sin(theta)
        ry = c * dy + s * dx
        rx = -s * dy + c * dx
    else:
        ry, rx = dy, dx
    maha = ry * ry / (scale[..., 0] ** 2) + rx * rx / (scale[..., 1] ** 2)
    fo = torch.exp(-0.5 * maha) * opacity
    return fo.clamp(max=CLAMP), fo


def cull_fields(mu, scale, color, opacity, theta, gid, starts, H, W, TILE=8, odds=False, chunk=1 << 15):
    """Partial-sum fields of one splat group over its fixed pair list. mu [N,2], scale [N,2], color [N,C],
    opacity [N], theta [N] or None (float64, may require grad); gid/starts from the binning.
    Returns S_log [P], S_a [P] (unclamped), S_ac [P, C]."""
    P = H * W
    C = color.shape[-1]
    gid = torch.as_tensor(np.asarray(gid), dtype=torch.long)
    starts = torch.as_tensor(np.asarray(starts), dtype=torch.long)
    ntx = (W + TILE - 1) // TILE
    nt = starts.numel() - 1
    tot = int(starts[-1])
    ys, xs = cull_centres(H, W)
    ly = torch.arange(TILE * TILE) // TILE
    lx = torch.arange(TILE * TILE) % TILE
    S_log = torch.zeros(P + 1, dtype=f64)
    S_a = torch.zeros(P + 1, dtype=f64)
    S_ac = torch.zeros(P + 1, C, dtype=f64)
    if tot == 0:
        return S_log[:P], S_a[:P], S_ac[:P]
    tile = torch.repeat_interleave(torch.arange(nt), starts[1:] - starts[:-1])
    for s0 in range(0, tot, chunk):
        s1 = min(tot, s0 + chunk)
        t = tile[s0:s1]
        g = gid[s0:s1]
        yp = (t // ntx)[:, None] * TILE + ly[None, :]
        xp = (t % ntx)[:, None] * TILE + lx[None, :]
        valid = (yp < H) & (xp < W)
        pix = torch.where(valid, yp * W + xp, torch.full_like(yp, P))          # masked -> dummy slot P
        py = ys[yp.clamp(max=H - 1)]
        px = xs[xp.clamp(max=W - 1)]
        a, _ = _alpha(py, px, mu[g][:, None, :], scale[g][:, None, :], opacity[g][:, None],
                      None if theta is None else theta[g][:, None])
        w = a / (1.0 - a) if odds else a
        flat = pix.reshape(-1)
        S_log = S_log.index_add(0, flat, torch.log(1.0 - a).reshape(-1))
        S_a = S_a.index_add(0, flat, w.reshape(-1))
        S_ac = S_ac.index_add(0, flat, (w[..., None] * color[g][:, None, :]).reshape(-1, C))
    return S_log[:P], S_a[:P], S_ac[:P]


def composite(S_log, S_a, S_ac, bg, straight_through=True):
    """T = exp(S_log), asum = max(S_a, 1e-8), fg = S_ac/asum, out = (1-T) fg + T bg.

    straight_through=True reproduces the in-kernel composite's gradient (render_triton.py:650-654), which
    ignores the clamp; False is torch's clamp_min gradient, used by the multires/octave glue (:918, :976)."""
    if straight_through:
        asum = S_a + (S_a.clamp_min(1e-8) - S_a).detach()
    else:
        asum = S_a.clamp_min(1e-8)
    T = torch.exp(S_log)
    fg = S_ac / asum[..., None]
    out = (1.0 - T)[..., None] * fg + T[..., None] * bg
    return out, T, asum, fg


def cull_composite(mu, scale, color, opacity, bg, theta, gid, starts, H, W, TILE=8, odds=False):
    """render_alpha_full_triton(cull=True) for one batch over a fixed pair list; returns out [P, C] etc."""
    S = cull_fields(mu, scale, color, opacity, theta, gid, starts, H, W, TILE, odds)
    return composite(*S, bg, straight_through=True)


def exact(mu, scale, color, opacity, bg, theta, H, W, odds=False, chunk=4096):
    """Every pixel sums every splat (render.py:34-58 with render.py:61-65 centres); [P, C]."""
    pyx = linspace_centres(H, W)
    outs = []
    for s0 in range(0, H * W, chunk):
        p = pyx[s0:s0 + chunk]
        a, _ = _alpha(p[:, 0:1], p[:, 1:2], mu[None], scale[None], opacity[None],
                      None if theta is None else theta[None])
        w = a / (1.0 - a) if odds else a
        S_log = torch.log1p(-a).sum(-1)
        S_a = w.sum(-1)
        S_ac = w @ color
        outs.append(composite(S_log, S_a, S_ac, bg, straight_through=False)[0])
    return torch.cat(outs, 0)


def upsample_field(x, Hc, Wc, H, W):
    """render_triton.py:864-876: bilinear, align_corners=False; x [Pc] or [Pc, C] -> [P] or [P, C]."""
    if x.dim() == 1:
        return F.interpolate(x.view(1, 1, Hc, Wc), size=(H, W), mode="bilinear", align_corners=False).reshape(H * W)
    C = x.shape[-1]
    g = x.view(1, Hc, Wc, C).permute(0, 3, 1, 2)
    y = F.interpolate(g, size=(H, W), mode="bilinear", align_corners=False)
    return y.permute(0, 2, 3, 1).reshape(H * W, C)


def _bin(mu, scale, H, W, TILE, cutoff):
    return binning.build_tiles(mu.detach().float().numpy(), scale.detach().float().numpy(), H, W, TILE, cutoff)


def fields_group(mu, scale, color, opacity, theta, H, W, TILE, cutoff, odds, scale32=None):
    """Bin (fp32: `scale32` when given, the exact bits a device run binned with) then evaluate the fields."""
    gid, starts = _bin(mu, scale if scale32 is None else scale32, H, W, TILE, cutoff)
    return cull_fields(mu, scale, color, opacity, theta, gid, starts, H, W, TILE, odds)


def multires(mu, scale, color, opacity, bg, theta, H, W, n_coarse=None, coarse_factor=8, cutoff=3.0, TILE=8,
             odds=False, scale32=None):
    """render_triton.py:879-922 for one batch; `scale32` (fp32) bins when given."""
    N = mu.shape[0]
    th = lambda lo, hi: None if theta is None else theta[lo:hi]
    s32 = lambda lo, hi: None if scale32 is None else scale32[lo:hi]
    if n_coarse is None or n_coarse <= 0 or n_coarse >= N:
        S = fields_group(mu, scale, color, opacity, theta, H, W, TILE, cutoff, odds, scale32)
    else:
        cf = min(coarse_factor, max(1, min(H, W) // 8))
        Hc, Wc = max(1, H // cf), max(1, W // cf)
        Sc = fields_group(mu[:n_coarse], scale[:n_coarse], color[:n_coarse], opacity[:n_coarse], th(0, n_coarse),
                          Hc, Wc, TILE, cutoff, odds, s32(0, n_coarse))
        Sf = fields_group(mu[n_coarse:], scale[n_coarse:], color[n_coarse:], opacity[n_coarse:], th(n_coarse, N),
                          H, W, TILE, cutoff, odds, s32(n_coarse, N))
        S = tuple(f + upsample_field(c, Hc, Wc, H, W) for f, c in zip(Sf, Sc))
    return composite(*S, bg, straight_through=False)[0]


def octave_of(scale_f32: torch.Tensor, H: int, W: int, base_texels=8.0, max_octaves=6):
    """render_triton.py:925-932, 950-952 in fp32: the routing the reference computes (non-differentiable)."""
    scale_px = scale_f32.detach().float().amax(-1) * float(min(H, W))
    o = torch.ceil(torch.log2((scale_px / base_texels).clamp_min(1e-6)))
    return o.clamp(0, max_octaves).to(torch.int64)


def octave(mu, scale, color, opacity, bg, theta, H, W, cutoff=3.0, TILE=8, base_texels=8.0, max_octaves=6,
           odds=False, oct=None, scale32=None):
    """render_triton.py:935-980 for one batch. `oct` overrides the routing and `scale32` the binning scale
    (to share both with a device run)."""
    if oct is None:
        oct = octave_of(scale if scale32 is None else scale32, H, W, base_texels, max_octaves)
    P = H * W
    C = color.shape[-1]
    S = [torch.zeros(P, dtype=f64), torch.zeros(P, dtype=f64), torch.zeros(P, C, dtype=f64)]
    for o in range(max_octaves + 1):
        idx = (oct == o).nonzero(as_tuple=True)[0]
        if idx.numel() == 0:
            continue
        Ho, Wo = max(8, H >> o), max(8, W >> o)
        Fo = fields_group(mu[idx], scale[idx], color[idx], opacity[idx], None if theta is None else theta[idx],
                          Ho, Wo, TILE, cutoff, odds, None if scale32 is None else scale32[idx])
        if o == 0:
            S = [a + b for a, b in zip(S, Fo)]
        else:
            S = [a + upsample_field(b, Ho, Wo, H, W) for a, b in zip(S, Fo)]
    return composite(*S, bg, straight_through=False)[0]


def leaves(mu, log_scale, color, opacity, bg, theta):
    """float64 CPU leaves requiring grad from fp32 tensors (any device)."""
    cv = lambda t: None if t is None else t.detach().cpu().to(f64).requires_grad_(True)
    return cv(mu), cv(log_scale), cv(color), cv(opacity), cv(bg), cv(theta)


def render_alpha_full_f32(mu, log_scale, color, opacity, bg, H, W, theta=None, chunk_pixels=4096, rows=None):
    """render.py:90-110 restated in fp32 torch (materialised [B, P, N] falloff, chunked): the reference's
    own CPU renderer, used as the CPU baseline. `rows=(r0, r1)` renders only that band of rows.
    Returns [B, P_band, C]."""
    B, N, C = color.shape
    scale = activate_scale(log_scale)
    pix = linspace_centres(H, W).float()
    if rows is not None:
        pix = pix[rows[0] * W: rows[1] * W]
    out = []
    for s in range(0, pix.shape[0], chunk_pixels):
        p = pix[s:s + chunk_pixels]
        diff = p[None, :, None, :] - mu[:, None, :, :]                       # [B, P, N, 2]
        if theta is not None:
            c, sn = torch.cos(theta), torch.sin(theta)
            dy, dx = diff[..., 0], diff[..., 1]
            diff = torch.stack([c[:, None] * dy + sn[:, None] * dx, -sn[:, None] * dy + c[:, None] * dx], dim=-1)
        maha = (diff.pow(2) / scale[:, None].pow(2)).sum(-1)
        alpha = (torch.exp(-0.5 * maha) * opacity[:, None]).clamp(max=CLAMP)
        T = torch.log1p(-alpha).sum(-1).exp()
        asum = alpha.sum(-1).clamp_min(1e-8)
        fg = torch.bmm(alpha, color) / asum[..., None]
        out.append((1.0 - T)[..., None] * fg + T[..., None] * bg[:, None])
    return torch.cat(out, 1)


def octave_forward_c(mu, scale, color, opacity, bg, theta, H, W, cutoff=3.0, TILE=8, base_texels=8.0,
                     max_octaves=6, odds=False):
    """render_triton.py:935-980 forward for one batch with the fields from the float64 C oracle (fast enough
    for full-size frames): octave routing on the fp32 activated `scale`, per-octave binning and fields, then
    float64 upsample + sum + composite. Inputs are fp32 CPU tensors; returns the image [P, C] float64."""
    from . import c_oracle
    sc = scale.detach().float().cpu()
    np32 = lambda t: None if t is None else t.detach().float().cpu().numpy()
    mu_, sc_, col_, op_, th_ = np32(mu), sc.numpy(), np32(color), np32(opacity), np32(theta)
    oct_ = octave_of(sc, H, W, base_texels, max_octaves).numpy()
    P, C = H * W, col_.shape[-1]
    S = [torch.zeros(P, dtype=f64), torch.zeros(P, dtype=f64), torch.zeros(P, C, dtype=f64)]
    for o in range(max_octaves + 1):
        idx = np.nonzero(oct_ == o)[0]
        if idx.size == 0:
            continue
        Ho, Wo = max(8, H >> o), max(8, W >> o)
        sub = lambda a: None if a is None else np.ascontiguousarray(a[idx])
        gid, st = c_oracle.build_tiles(sub(mu_), sub(sc_), Ho, Wo, TILE, cutoff)
        f = [torch.from_numpy(np.ascontiguousarray(x)) for x in
             c_oracle.fwd_cull(sub(mu_), sub(sc_), sub(th_), sub(op_), sub(col_), gid, st, Ho, Wo, TILE, odds=odds,
                               fields=True)]
        S = [a + (b if o == 0 else upsample_field(b, Ho, Wo, H, W)) for a, b in zip(S, f)]
    return composite(*S, torch.as_tensor(np32(bg), dtype=f64), straight_through=False)[0]
