"""Tile-binned differentiable alpha-compositing renderer on hand-written HIP kernels (gfx950).

Drop-in for gaussian_splat_encoder/render_triton.py of the reference: the same entry points, arguments,
tensor layouts, autograd contracts and exceptions. Compositing is the reference's order-independent
alpha monoid (render_triton.py:10-14):

    a_n   = min(opacity_n * exp(-maha_n / 2), 1 - 1e-4)
    T     = exp(sum_n log(1 - a_n))
    fg[c] = sum_n w_n color_n[c] / max(sum_n w_n, 1e-8)       w = a, or the odds a/(1-a) with odds=True
    C[c]  = (1 - T) fg[c] + T bg[c]

Layouts: mu [B,N,2] (y, x) in [0,1]; log_scale [B,N,2] raw; color [B,N,C]; opacity [B,N]; bg [B,C];
theta [B,N] radians or None. Images come back as [B,C,H,W] (a permuted view of [B,H,W,C]).

Device work goes through libsplat_hip.so (include/splat_render.h); this module only allocates outputs,
drives the per-batch calls on the current stream and does the octave / multires glue.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import FLAG_FIELDS, FLAG_ODDS, check, ptr
from .params import activate_scale
from .render import _pixels


class PairBudgetExceeded(RuntimeError):
    """Raised before any pair allocation when a render would bin more (tile, splat) pairs than max_pairs
    (render_triton.py:51-55, raised at :378-385)."""


def _dev_check(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the HIP splat renderer needs device tensors (got a CPU tensor)")


def _f32(t):
    return None if t is None else t.detach().contiguous().float()


def _empty(shape, dev, dtype=torch.float32):
    return torch.empty(shape, device=dev, dtype=dtype)


def _ws(nbytes, dev):
    return torch.empty(max(int(nbytes), 1), device=dev, dtype=torch.uint8)


class KernelTimer:
    """Optional HIP-event brackets around the per-tile forward and backward calls, recorded on the stream
    the kernels run on. Enabled by `kernel_timer.enable()`; `elapsed_ms()` syncs and returns per-name lists."""

    def __init__(self):
        self.enabled = False
        self.events = {}

    def enable(self, on=True):
        self.enabled = on
        self.events = {}

    def record(self, name):
        if not self.enabled:
            return None
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def close(self, name, start):
        if start is not None:
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            self.events.setdefault(name, []).append((start, end))

    def elapsed_ms(self):
        torch.cuda.synchronize()
        return {k: [a.elapsed_time(b) for a, b in v] for k, v in self.events.items()}


kernel_timer = KernelTimer()


class TileBins:
    """Per-batch binning result: decoded splat records, pair list ordered by (tile, splat) and CSR tile
    starts (`gid_b`/`starts_b`/`ntx`/`nt` carry the meaning of the reference's `tiles` tuple), plus the
    splat-major pair maps the backward's per-splat reduction uses (offsets, pair -> splat, pair -> sorted
    position)."""

    def __init__(self, rec_b, gid_b, starts_b, tot_b, H, W, TILE, ntx, nt, off_b=None, psplat_b=None, pinv_b=None):
        self.rec_b, self.gid_b, self.starts_b, self.tot_b = rec_b, gid_b, starts_b, tot_b
        self.H, self.W, self.TILE, self.ntx, self.nt = H, W, TILE, ntx, nt
        self.off_b, self.psplat_b, self.pinv_b = off_b, psplat_b, pinv_b

    def as_tuple(self):
        return self.gid_b, self.starts_b, self.ntx, self.nt


def _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs=None, with_maps=True) -> TileBins:
    """Decode + bin every batch (render_triton.py:351-409). One host read of the per-batch pair totals.
    with_maps=False skips the pair maps only the backward needs (forward-only renders)."""
    _dev_check(mu, scale, color, opacity, theta)
    ev = kernel_timer.record("bin")
    bins = _bin_impl(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps)
    kernel_timer.close("bin", ev)
    return bins


def _bin_impl(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps):
    B, N, C = color.shape
    dev = mu.device
    lib = _lib.load()
    mu_, sc_, col_, op_, th_ = _f32(mu), _f32(scale), _f32(color), _f32(opacity), _f32(theta)
    ntx = (W + TILE - 1) // TILE
    nt = ntx * ((H + TILE - 1) // TILE)
    stream = _lib.stream_ptr(dev)
    if N == 0:
        return TileBins([_empty((0, 16), dev)] * B, [torch.zeros(1, dtype=torch.int32, device=dev)] * B,
                        [torch.zeros(nt + 1, dtype=torch.int32, device=dev)] * B, [0] * B, H, W, TILE, ntx, nt)
    info = torch.empty((B, 2), dtype=torch.int64, device=dev)
    rec_b, rect_b, off_b = [], [], []
    ws1 = _ws(lib.splat_bin_count_workspace_bytes(N), dev)
    for b in range(B):
        rec = _empty((N, 16), dev)
        rect = torch.empty((N, 4), dtype=torch.int32, device=dev)
        off = torch.empty(N + 1, dtype=torch.int32, device=dev)
        check(lib.splat_bin_count(ptr(mu_[b]), ptr(sc_[b]), None if th_ is None else ptr(th_[b]), ptr(op_[b]),
                                  ptr(col_[b]), C, N, H, W, TILE, float(cutoff), ptr(rec), ptr(rect), ptr(off),
                                  ptr(info[b]), ptr(ws1), ws1.numel(), stream), "splat_bin_count")
        rec_b.append(rec); rect_b.append(rect); off_b.append(off)
    info_h = info.cpu()                                                   # the one host sync of binning
    if bool((info_h[:, 1] & 1).any()):
        raise ValueError("binning: a splat has an empty tile rect (negative cutoff or scale)")
    if bool((info_h[:, 1] & 2).any()):
        raise PairBudgetExceeded(f"binning: {int(info_h[:, 0].max())} pairs exceed the int32 pair index range")
    tots = [int(x) for x in info_h[:, 0]]
    if max_pairs is not None:
        worst = max(tots)
        if worst > max_pairs:
            raise PairBudgetExceeded(
                f"_build_tiles: {worst} (tile,gaussian) pairs exceeds the {max_pairs} budget @ {H}x{W} "
                f"TILE={TILE} cutoff={cutoff} N={N}. Route large splats through the low-res (octave) pass "
                f"instead of culling at full res. Refusing to allocate.")
    gid_b, starts_b, psplat_b, pinv_b = [], [], [], []
    for b in range(B):
        tot = tots[b]
        gid = torch.empty(max(tot, 1), dtype=torch.int32, device=dev)
        starts = torch.empty(nt + 1, dtype=torch.int32, device=dev)
        psplat = torch.empty(max(tot, 1), dtype=torch.int32, device=dev) if with_maps else None
        pinv = torch.empty(max(tot, 1), dtype=torch.int32, device=dev) if with_maps else None
        ws2 = _ws(lib.splat_bin_pairs_workspace_bytes(N, nt, tot), dev)
        check(lib.splat_bin_pairs(ptr(rect_b[b]), ptr(off_b[b]), N, H, W, TILE, tot, ptr(gid), ptr(starts),
                                  ptr(psplat), ptr(pinv), ptr(ws2), ws2.numel(), stream), "splat_bin_pairs")
        gid_b.append(gid); starts_b.append(starts); psplat_b.append(psplat); pinv_b.append(pinv)
    return TileBins(rec_b, gid_b, starts_b, tots, H, W, TILE, ntx, nt, off_b, psplat_b, pinv_b)


def _build_tiles(mu, scale, H, W, TILE, cutoff, max_pairs=None):
    """(gid_b, starts_b, ntx, nt) exactly as render_triton.py:351-409 returns them."""
    B, N, _ = mu.shape
    dummy_col = torch.zeros((B, N, 1), device=mu.device)
    dummy_op = torch.zeros((B, N), device=mu.device)
    return _bin(mu, scale, dummy_col, dummy_op, None, H, W, TILE, cutoff, max_pairs, with_maps=False).as_tuple()


# ----------------------------------------------------------------------------------------------- cull path
def _forward_cull(mu, scale, color, opacity, bg, theta, H, W, TILE=8, cutoff=3.0, max_pairs=None, odds=False):
    """Composite forward (render_triton.py:538-567): out [B,P,C], (T, asum, fg), bins."""
    B, N, C = color.shape
    P = H * W
    dev = mu.device
    bins = _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs)
    out, T, asum, fg = _empty((B, P, C), dev), _empty((B, P), dev), _empty((B, P), dev), _empty((B, P, C), dev)
    bgf = _f32(bg)
    flags = FLAG_ODDS if odds else 0
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    for b in range(B):
        ev = kernel_timer.record("fwd")
        check(lib.splat_render_fwd(ptr(bins.rec_b[b]), ptr(bins.gid_b[b]), ptr(bins.starts_b[b]), C, H, W, TILE,
                                   flags, ptr(bgf[b]), ptr(out[b]), ptr(T[b]), ptr(asum[b]), ptr(fg[b]), None, None,
                                   None, stream), "splat_render_fwd")
        kernel_timer.close("fwd", ev)
    return out, (T, asum, fg), bins


def _forward_cull_fields(mu, scale, color, opacity, theta, H, W, TILE=8, cutoff=3.0, max_pairs=None, odds=False):
    """FIELDS forward (render_triton.py:570-599): S_log [B,P], S_a [B,P] (unclamped), S_ac [B,P,C], bins."""
    B, N, C = color.shape
    P = H * W
    dev = mu.device
    bins = _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs)
    slog, sa, sac = _empty((B, P), dev), _empty((B, P), dev), _empty((B, P, C), dev)
    flags = FLAG_FIELDS | (FLAG_ODDS if odds else 0)
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    for b in range(B):
        if N == 0:
            slog[b].zero_(); sa[b].zero_(); sac[b].zero_()
            continue
        check(lib.splat_render_fwd(ptr(bins.rec_b[b]), ptr(bins.gid_b[b]), ptr(bins.starts_b[b]), C, H, W, TILE,
                                   flags, None, None, None, None, None, ptr(slog[b]), ptr(sa[b]), ptr(sac[b]), stream),
              "splat_render_fwd")
    return slog, sa, sac, bins


def _grads_out(B, N, C, dev, has_th):
    return (_empty((B, N, 2), dev), _empty((B, N, 2), dev), _empty((B, N, C), dev), _empty((B, N), dev),
            _empty((B, N), dev) if has_th else None)


def _backward_pairs(bins, b, flags, C, H, W, TILE, upstream, grads, g_bg, lib, stream):
    """Both backward steps for batch b: per-tile pair sums, then the per-splat reduction into `grads`."""
    dev = bins.rec_b[b].device
    tot = bins.tot_b[b]
    N = bins.off_b[b].numel() - 1
    sums = _empty((lib.splat_pair_sums_bytes(tot) // 4,), dev)
    bg_part = _empty((C * bins.nt,), dev) if g_bg is not None else None
    ev = kernel_timer.record("bwd")
    check(lib.splat_render_bwd(ptr(bins.rec_b[b]), ptr(bins.gid_b[b]), ptr(bins.starts_b[b]), tot, C, H, W, TILE,
                               flags, *[ptr(u) for u in upstream], ptr(sums), ptr(bg_part), stream),
          "splat_render_bwd")
    kernel_timer.close("bwd", ev)
    ev = kernel_timer.record("reduce")
    ws = _ws(lib.splat_reduce_workspace_bytes(tot), dev)
    g_mu, g_scale, g_col, g_op, g_th = grads
    check(lib.splat_reduce_pairs(ptr(bins.rec_b[b]), ptr(bins.off_b[b]), ptr(bins.psplat_b[b]), ptr(bins.pinv_b[b]),
                                 tot, N, C, ptr(sums), ptr(bg_part), bins.nt, ptr(g_mu[b]), ptr(g_scale[b]),
                                 None if g_th is None else ptr(g_th[b]), ptr(g_op[b]), ptr(g_col[b]), ptr(g_bg),
                                 ptr(ws), ws.numel(), stream), "splat_reduce_pairs")
    kernel_timer.close("reduce", ev)


def _backward_cull(grad_out, mu, scale, color, opacity, bg, theta, T, asum, fg, bins, H, W, TILE=8, odds=False):
    """render_triton.py:723-765: grads for mu, scale, color, opacity, bg, theta (None without theta)."""
    B, N, C = color.shape
    dev = mu.device
    grads = _grads_out(B, N, C, dev, theta is not None)
    g_bg = _empty((B, C), dev)
    go, bgf = _f32(grad_out), _f32(bg)
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    flags = FLAG_ODDS if odds else 0
    for b in range(B):
        up = (bgf[b], T[b], asum[b], fg[b], go[b], None, None, None)
        _backward_pairs(bins, b, flags, C, H, W, TILE, up, grads, g_bg[b], lib, stream)
    g_mu, g_scale, g_col, g_op, g_th = grads
    return g_mu, g_scale, g_col, g_op, g_bg, g_th


def _backward_cull_fields(dS_log, dS_a, dS_ac, mu, scale, color, opacity, theta, bins, H, W, TILE=8, odds=False):
    """render_triton.py:768-810: grads for mu, scale, color, opacity, theta from the fields' upstream grads."""
    B, N, C = color.shape
    dev = mu.device
    grads = _grads_out(B, N, C, dev, theta is not None)
    if N == 0:
        return grads
    dl, da, dc = _f32(dS_log), _f32(dS_a), _f32(dS_ac)
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    flags = FLAG_FIELDS | (FLAG_ODDS if odds else 0)
    for b in range(B):
        up = (None, None, None, None, None, dl[b], da[b], dc[b])
        _backward_pairs(bins, b, flags, C, H, W, TILE, up, grads, None, lib, stream)
    return grads


class _AlphaRenderCull(torch.autograd.Function):
    """render_triton.py:813-833. Inputs (mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds)."""

    @staticmethod
    def forward(ctx, mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds=False):
        out, (T, asum, fg), bins = _forward_cull(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds=odds)
        ctx.has_theta = theta is not None
        ctx.HW = (H, W, TILE)
        ctx.odds = odds
        ctx.tiles = bins
        ctx.save_for_backward(mu, scale, color, opacity, bg, theta if theta is not None else mu.new_zeros(1),
                              T, asum, fg)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        mu, scale, color, opacity, bg, theta, T, asum, fg = ctx.saved_tensors
        H, W, TILE = ctx.HW
        th = theta if ctx.has_theta else None
        g_mu, g_scale, g_col, g_op, g_bg, g_th = _backward_cull(grad_out, mu, scale, color, opacity, bg, th, T, asum,
                                                                fg, ctx.tiles, H, W, TILE, odds=ctx.odds)
        return g_mu, g_scale, g_col, g_op, g_bg, g_th, None, None, None, None, None


class _AlphaRenderCullFields(torch.autograd.Function):
    """render_triton.py:836-861: raw partial-sum fields of one splat group; no bg, no composite."""

    @staticmethod
    def forward(ctx, mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, odds=False):
        slog, sa, sac, bins = _forward_cull_fields(mu, scale, color, opacity, theta, H, W, TILE=TILE, cutoff=cutoff,
                                                   max_pairs=max_pairs, odds=odds)
        ctx.has_theta = theta is not None
        ctx.HW = (H, W, TILE)
        ctx.odds = odds
        ctx.tiles = bins
        ctx.save_for_backward(mu, scale, color, opacity, theta if theta is not None else mu.new_zeros(1))
        return slog, sa, sac

    @staticmethod
    def backward(ctx, dS_log, dS_a, dS_ac):
        mu, scale, color, opacity, theta = ctx.saved_tensors
        H, W, TILE = ctx.HW
        th = theta if ctx.has_theta else None
        dev = mu.device
        B, N, C = color.shape
        P = H * W
        z = lambda t, shape: torch.zeros(shape, device=dev) if t is None else t
        dS_log, dS_a, dS_ac = z(dS_log, (B, P)), z(dS_a, (B, P)), z(dS_ac, (B, P, C))
        g_mu, g_scale, g_col, g_op, g_th = _backward_cull_fields(dS_log, dS_a, dS_ac, mu, scale, color, opacity, th,
                                                                 ctx.tiles, H, W, TILE, odds=ctx.odds)
        return g_mu, g_scale, g_col, g_op, g_th, None, None, None, None, None, None


# ----------------------------------------------------------------------------------------------- exact path
def _forward(mu, scale, color, opacity, bg, py, px, theta):
    """render_triton.py:128-157: every pixel sums every splat. Returns out [B,P,C], T, asum, fg."""
    _dev_check(mu, scale, color, opacity, bg, theta)
    B, N, C = color.shape
    P = py.shape[0]
    dev = mu.device
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    mu_, sc_, col_, op_, th_, bgf = _f32(mu), _f32(scale), _f32(color), _f32(opacity), _f32(theta), _f32(bg)
    pyf, pxf = _f32(py), _f32(px)
    out, T, asum, fg = _empty((B, P, C), dev), _empty((B, P), dev), _empty((B, P), dev), _empty((B, P, C), dev)
    recs = []
    for b in range(B):
        rec = _empty((max(N, 1), 16), dev)
        if N:
            check(lib.splat_decode(ptr(mu_[b]), ptr(sc_[b]), None if th_ is None else ptr(th_[b]), ptr(op_[b]),
                                   ptr(col_[b]), C, N, ptr(rec), stream), "splat_decode")
        check(lib.splat_exact_fwd(ptr(rec), N, C, ptr(pyf), ptr(pxf), P, ptr(bgf[b]), ptr(out[b]), ptr(T[b]),
                                  ptr(asum[b]), ptr(fg[b]), stream), "splat_exact_fwd")
        recs.append(rec)
    return out, T, asum, fg, recs


def _backward(grad_out, mu, scale, color, opacity, bg, py, px, theta, T, asum, fg, recs=None):
    """render_triton.py:269-303: grads for mu, scale, color, opacity, bg, theta."""
    B, N, C = color.shape
    P = py.shape[0]
    dev = mu.device
    has_th = theta is not None
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    g_mu, g_scale, g_col, g_op, g_th = _grads_out(B, N, C, dev, has_th)
    g_bg = _empty((B, C), dev)
    if N == 0:
        g_bg.copy_((_f32(grad_out) * T.unsqueeze(-1)).sum(dim=1))
        return g_mu, g_scale, g_col, g_op, g_bg, g_th
    if recs is None:
        recs = _forward(mu, scale, color, opacity, bg, py, px, theta)[4]
    go, bgf, pyf, pxf = _f32(grad_out), _f32(bg), _f32(py), _f32(px)
    ws = _ws(lib.splat_exact_bwd_workspace_bytes(N, C, P), dev)
    for b in range(B):
        check(lib.splat_exact_bwd(ptr(recs[b]), N, C, ptr(pyf), ptr(pxf), P, ptr(bgf[b]), ptr(T[b]), ptr(asum[b]),
                                  ptr(fg[b]), ptr(go[b]), ptr(g_mu[b]), ptr(g_scale[b]),
                                  None if g_th is None else ptr(g_th[b]), ptr(g_op[b]), ptr(g_col[b]), ptr(g_bg[b]),
                                  ptr(ws), ws.numel(), stream), "splat_exact_bwd")
    return g_mu, g_scale, g_col, g_op, g_bg, g_th


class _AlphaRender(torch.autograd.Function):
    """render_triton.py:307-323 (exact path)."""

    @staticmethod
    def forward(ctx, mu, scale, color, opacity, bg, theta, py, px):
        out, T, asum, fg, recs = _forward(mu, scale, color, opacity, bg, py, px, theta)
        ctx.has_theta = theta is not None
        ctx.recs = recs
        ctx.save_for_backward(mu, scale, color, opacity, bg, theta if theta is not None else mu.new_zeros(1),
                              py, px, T, asum, fg)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        mu, scale, color, opacity, bg, theta, py, px, T, asum, fg = ctx.saved_tensors
        th = theta if ctx.has_theta else None
        g_mu, g_scale, g_col, g_op, g_bg, g_th = _backward(grad_out, mu, scale, color, opacity, bg, py, px, th, T,
                                                           asum, fg, ctx.recs)
        return g_mu, g_scale, g_col, g_op, g_bg, g_th, None, None


# ----------------------------------------------------------------------------------------------- public API
def render_alpha_full_triton(mu, log_scale, color, opacity, bg, H, W, theta=None, cull=False, TILE=8, cutoff=3.0,
                             odds=False):
    """render_triton.py:326-347. cull=False: exact (every pixel sums every splat); cull=True: tile-binned
    at `cutoff` sigma. Returns [B,C,H,W]. The name is kept for drop-in compatibility; no Triton is used."""
    B, N, C = color.shape
    scale = activate_scale(log_scale)
    if cull:
        out = _AlphaRenderCull.apply(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds)
    else:
        if odds:
            raise NotImplementedError("odds compositing is only wired through the cull/octave path; "
                                      "use cull=True or render_alpha_octave")
        pyx = _pixels(H, W, mu.device, torch.float32)
        out = _AlphaRender.apply(mu, scale, color, opacity, bg, theta, pyx[:, 0].contiguous(),
                                 pyx[:, 1].contiguous())
    return out.reshape(B, H, W, C).permute(0, 3, 1, 2)


def _upsample_field(x, Hc, Wc, H, W):
    """render_triton.py:864-876: bilinear (align_corners=False) upsample of [B,Pc] / [B,Pc,C] to (H, W)."""
    B = x.shape[0]
    if x.dim() == 2:
        y = F.interpolate(x.view(B, 1, Hc, Wc), size=(H, W), mode="bilinear", align_corners=False)
        return y.reshape(B, H * W)
    C = x.shape[-1]
    g = x.view(B, Hc, Wc, C).permute(0, 3, 1, 2)
    y = F.interpolate(g, size=(H, W), mode="bilinear", align_corners=False)
    return y.permute(0, 2, 3, 1).reshape(B, H * W, C)


def _composite_fields(slog, sa, sac, bg, B, H, W, C):
    """render_triton.py:918-922 / 976-980: clamp, exp, divide, blend with bg -> [B,C,H,W] view."""
    asum = sa.clamp_min(1e-8)
    T = slog.exp()
    fg = sac / asum.unsqueeze(-1)
    img = (1.0 - T).unsqueeze(-1) * fg + T.unsqueeze(-1) * bg.float().unsqueeze(1)
    return img.reshape(B, H, W, C).permute(0, 3, 1, 2)


def render_alpha_multires(mu, log_scale, color, opacity, bg, H, W, theta=None, n_coarse=None, coarse_factor=8,
                          cutoff=3.0, TILE=8, max_pairs=48_000_000, odds=False):
    """render_triton.py:879-922: coarse group [0, n_coarse) at H/cf, fine group at native resolution; the
    fields are summed (bilinear upsample of the coarse ones) and composited once."""
    B, N, C = color.shape
    scale = activate_scale(log_scale)
    has_th = theta is not None

    def fields(lo, hi, H_, W_):
        th = theta[:, lo:hi] if has_th else None
        return _AlphaRenderCullFields.apply(mu[:, lo:hi], scale[:, lo:hi], color[:, lo:hi], opacity[:, lo:hi], th,
                                            H_, W_, TILE, cutoff, max_pairs, odds)

    if n_coarse is None or n_coarse <= 0 or n_coarse >= N:
        slog, sa, sac = fields(0, N, H, W)
    else:
        cf = min(coarse_factor, max(1, min(H, W) // 8))
        Hc = max(1, H // cf); Wc = max(1, W // cf)
        slc, sac_a, sac_c = fields(0, n_coarse, Hc, Wc)
        slf, saf, sacf = fields(n_coarse, N, H, W)
        slog = slf + _upsample_field(slc, Hc, Wc, H, W)
        sa = saf + _upsample_field(sac_a, Hc, Wc, H, W)
        sac = sacf + _upsample_field(sac_c, Hc, Wc, H, W)
    return _composite_fields(slog, sa, sac, bg, B, H, W, C)


def _octave_of(scale_px, base_texels=8.0, max_octaves=6):
    """render_triton.py:925-932: o = clamp(ceil(log2(sigma_px / base_texels)), 0, max_octaves)."""
    o = torch.ceil(torch.log2((scale_px / base_texels).clamp_min(1e-6)))
    return o.clamp(0, max_octaves).to(torch.int64)


def render_alpha_octave(mu, log_scale, color, opacity, bg, H, W, theta=None, cutoff=3.0, TILE=8, base_texels=8.0,
                        max_octaves=6, max_pairs=48_000_000, odds=False):
    """render_triton.py:935-980: each splat renders at the octave H/2^o where its footprint spans a bounded
    number of tiles; octave fields are upsampled to (H, W), summed and composited once."""
    B, N, C = color.shape
    scale = activate_scale(log_scale)
    has_th = theta is not None
    rep = float(min(H, W))
    scale_px = scale.detach().amax(-1) * rep
    oct = _octave_of(scale_px, base_texels, max_octaves)
    P = H * W
    slog_l, sa_l, sac_l = [], [], []
    for b in range(B):
        slog_b = mu.new_zeros(P); sa_b = mu.new_zeros(P); sac_b = mu.new_zeros(P, C)
        ob = oct[b]
        for o in range(max_octaves + 1):
            idx = (ob == o).nonzero(as_tuple=True)[0]
            if idx.numel() == 0:
                continue
            Ho = max(8, H >> o); Wo = max(8, W >> o)
            m = mu[b:b + 1, idx]; s = scale[b:b + 1, idx]; cl = color[b:b + 1, idx]
            op_ = opacity[b:b + 1, idx]; th = theta[b:b + 1, idx] if has_th else None
            sl, saa, sc = _AlphaRenderCullFields.apply(m, s, cl, op_, th, Ho, Wo, TILE, cutoff, max_pairs, odds)
            if o == 0:
                slog_b = slog_b + sl[0]; sa_b = sa_b + saa[0]; sac_b = sac_b + sc[0]
            else:
                slog_b = slog_b + _upsample_field(sl, Ho, Wo, H, W)[0]
                sa_b = sa_b + _upsample_field(saa, Ho, Wo, H, W)[0]
                sac_b = sac_b + _upsample_field(sc, Ho, Wo, H, W)[0]
        slog_l.append(slog_b); sa_l.append(sa_b); sac_l.append(sac_b)
    slog = torch.stack(slog_l); sa = torch.stack(sa_l); sac = torch.stack(sac_l)
    return _composite_fields(slog, sa, sac, bg, B, H, W, C)
