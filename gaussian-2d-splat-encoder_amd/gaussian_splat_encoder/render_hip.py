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

import threading

import torch
import torch.nn.functional as F

from . import _lib
from ._lib import FLAG_DEFER, FLAG_FIELDS, FLAG_LOG_SCALE, FLAG_ODDS, FLAG_UPS, FLAG_WIDE, SplatLevels, check, ptr
from .params import activate_scale
from .render import _pixels


class PairBudgetExceeded(RuntimeError):
    """Raised before any pair allocation when a render would bin more (tile, splat) pairs than max_pairs
    (render_triton.py:51-55, raised at :378-385)."""


def _dev_check(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the HIP splat renderer needs device tensors (got a CPU tensor)")


def _batch_args(mu, log_scale, color, opacity, bg, theta):
    """Checks the parameter shapes against color [B,N,C] and returns bg as [B,C]. The per-image launches take
    image b's data at b times each tensor's batch stride, so every tensor must hold B images. A bg of shape
    [1,C] is broadcast over the batch (the composite of render_triton.py:921, :980 broadcasts it; autograd sums
    its gradient back to [1,C])."""
    cs = color.shape
    if len(cs) != 3:
        raise ValueError(f"color must be [B,N,C], got {tuple(cs)}")
    B, N, C = cs
    bn2, bn = (B, N, 2), (B, N)
    if mu.shape != bn2 or log_scale.shape != bn2 or opacity.shape != bn or (theta is not None and theta.shape != bn):
        for name, t, shape in (("mu", mu, bn2), ("log_scale", log_scale, bn2), ("opacity", opacity, bn),
                               ("theta", theta, bn)):
            if t is not None and t.shape != shape:
                raise ValueError(f"{name} must be {list(shape)} for color {list(cs)}, got {list(t.shape)}")
    bs = bg.shape
    if bs == (B, C):
        return bg
    if bs == (1, C):
        return bg.expand(B, C)
    raise ValueError(f"bg must be [{B},{C}] or [1,{C}] for color {list(cs)}, got {list(bs)}")


def _f32(t):
    """t as contiguous fp32 (itself when it already is: the kernels only take its data pointer)."""
    if t is None or (t.dtype is torch.float32 and t.is_contiguous()):
        return t
    return t.detach().contiguous().float()


def _bptr(t, b):
    """Device pointer of image b of a contiguous [B, ...] tensor (None stays NULL)."""
    if t is None:
        return None
    p = t.data_ptr()
    return p if b == 0 else p + b * t.stride(0) * t.element_size()


def _empty(shape, dev, dtype=torch.float32):
    return torch.empty(shape, device=dev, dtype=dtype)


def _ws(nbytes, dev):
    return torch.empty(max(int(nbytes), 1), device=dev, dtype=torch.uint8)


class KernelTimer:
    """Optional HIP-event brackets of the render's stages, recorded on the stream the kernels run on. Enabled by
    `kernel_timer.enable()`; `elapsed_ms()` syncs and returns per-name lists. The tile kernels ("fwd", "bwd")
    record their events themselves at their own start and end (splat_time_next_launch), so a bracket holds the
    kernel alone even when the GPU waits for the host's launch; other stages are bracketed on the stream."""

    KERNEL_STAGES = ("fwd", "bwd")

    def __init__(self):
        self.enabled = False
        self.names = None
        self.events = {}
        self._pool = []   # events of earlier brackets, reused (creating one costs more host time than recording)

    def enable(self, on=True, names=None):
        """names: the stages to bracket (all when None)."""
        self.enabled = on
        self.names = None if names is None else set(names)
        self._recycle()

    def _take(self):
        if self._pool:
            return self._pool.pop()
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()   # creates the HIP event (torch creates it lazily)
        return ev

    def _event(self):
        ev = self._take()
        ev.record()
        return ev

    def _recycle(self):
        for v in self.events.values():
            for a, b in v:
                self._pool += [a, b]
        self.events = {}

    def record(self, name):
        if not self.enabled or (self.names is not None and name not in self.names):
            return None
        if name in self.KERNEL_STAGES:
            a, b = self._take(), self._take()
            _lib.load().splat_time_next_launch(a.cuda_event, b.cuda_event)
            return (a, b)
        return self._event()

    def close(self, name, start):
        """Ends a bracket opened by record(). Called in a `finally:` after the stage, so that events armed for a
        launch that never happened (the stage raised first) are disarmed: the library then holds no handle of
        events that could be destroyed before its next launch. Unused events go back to the pool."""
        if start is None:
            return
        if isinstance(start, tuple):
            if _lib.load().splat_time_next_launch(None, None):   # no launch took the events
                self._pool += list(start)
            else:
                self.events.setdefault(name, []).append(start)
        else:
            self.events.setdefault(name, []).append((start, self._event()))

    def elapsed_ms(self):
        torch.cuda.synchronize()
        return {k: [a.elapsed_time(b) for a, b in v] for k, v in self.events.items()}


kernel_timer = KernelTimer()


class TileBins:
    """Per-batch binning result: decoded splat records, pair list ordered by (tile, splat) and CSR tile
    starts (`gid_b`/`starts_b`/`ntx`/`nt` carry the meaning of the reference's `tiles` tuple), plus the
    map the backward uses from sorted to splat-major pair order (`pq`: sorted pair -> splat-major index; the
    splat of splat-major pair q is the g with offsets[g] <= q < offsets[g + 1]).

    Each image's buffers live in two allocations (`blocks[b]`: rec, rect, offsets; `pairs[b]`: gid, starts,
    pair_q); kernels take raw pointers (`p(b, name)`), tensor views are built on first use.

    With levels (`lv` set) the tile ids are global over the levels: `geom[l] = (H_l, W_l, ntx_l, tbase_l,
    pbase_l)`, `nt` / `npix` are the totals, `level_tot_b[b][l]` the pairs of level l and `rect_b[b][:, 3]`
    each splat's level."""

    _SLOT = {"rec": (0, 0), "rect": (0, 1), "off": (0, 2), "gid": (1, 0), "starts": (1, 1), "pq": (1, 2)}

    def __init__(self, N, tot_b, H, W, TILE, ntx, nt, blocks, pairs, with_maps, lv=None, geom=None, npix=None,
                 level_tot_b=None):
        self.N, self.tot_b = N, tot_b
        self.H, self.W, self.TILE, self.ntx, self.nt = H, W, TILE, ntx, nt
        self.blocks, self.pairs, self.with_maps = blocks, pairs, with_maps
        self.lv, self.geom, self.npix, self.level_tot_b = lv, geom, npix, level_tot_b
        self.pending = None   # a _Pending while the pair count of a deferred binning is unread
        self._views = {}
        self._ptrs = {}

    def p(self, b, name):
        """Device pointer of buffer `name` of image b (None for maps that were not built)."""
        key = (b, name)
        v = self._ptrs.get(key, 0)
        if v == 0:
            which, i = self._SLOT[name]
            v = None if (which == 1 and i >= 2 and not self.with_maps) else \
                (self.blocks if which == 0 else self.pairs)[b].ptr(i)
            self._ptrs[key] = v
        return v

    def _list(self, name):
        v = self._views.get(name)
        if v is None:
            N, out = self.N, []
            for b in range(len(self.tot_b)):
                n = max(self.tot_b[b], 1)
                blk, pb = self.blocks[b], self.pairs[b]
                if name == "rec":
                    out.append(blk.view(0, 16 * max(N, 1), torch.float32, (max(N, 1), 16)))
                elif name == "rect":
                    out.append(blk.view(1, 4 * N, torch.int32, (N, 4)))
                elif name == "off":
                    out.append(blk.view(2, N + 1, torch.int32))
                elif name == "gid":
                    out.append(pb.view(0, n, torch.int32))
                elif name == "starts":
                    out.append(pb.view(1, self.nt + 1, torch.int32))
                else:
                    out.append(pb.view(2, n, torch.int32) if self.with_maps else None)
            v = self._views[name] = out
        return v

    rec_b = property(lambda self: self._list("rec"))
    rect_b = property(lambda self: self._list("rect"))
    off_b = property(lambda self: self._list("off"))
    gid_b = property(lambda self: self._list("gid"))
    starts_b = property(lambda self: self._list("starts"))
    pq_b = property(lambda self: self._list("pq"))

    def as_tuple(self):
        return self.gid_b, self.starts_b, self.ntx, self.nt

    @property
    def n_levels(self):
        return 1 if self.geom is None else len(self.geom)

    @property
    def ntiles0(self):
        """Tiles of level 0 (the composite's canvas)."""
        return self.nt if self.geom is None else self.geom[1][3] if len(self.geom) > 1 else self.nt

    def level_mask(self, b):
        """Levels of batch b holding pairs, with level 0 always set (the composite covers every pixel)."""
        return 1 if self.level_tot_b is None else _mask_of(self.level_tot_b[b])


def _mask_of(lt):
    """Level mask of per-level pair totals lt: the levels holding pairs, and level 0."""
    m = 1
    for l, n in enumerate(lt):
        if n > 0:
            m |= 1 << l
    return m


def levels_geometry(H, W, TILE, lv):
    """[(H_l, W_l, ntx_l, tbase_l, pbase_l)] per level, total tiles, total packed pixel slots."""
    key = (H, W, TILE, _lv_key(lv))
    hit = _GEOM.get(key)
    if hit is not None:
        return hit
    lib = _lib.load()
    ref = None if lv is None else _lib.ctypes.byref(lv)
    n = lib.splat_levels_geometry(H, W, TILE, ref, None, 0)
    if n < 0:
        check(-n, "splat_levels_geometry")
    buf = (_lib.ctypes.c_int * (5 * n + 2))()
    check(0 if lib.splat_levels_geometry(H, W, TILE, ref, buf, 5 * n + 2) == n else 1, "splat_levels_geometry")
    geom = [tuple(buf[5 * l:5 * l + 5]) for l in range(n)]
    _GEOM[key] = hit = (geom, buf[5 * n], buf[5 * n + 1])
    return hit


def _lv_key(lv):
    return None if lv is None else (lv.mode, lv.max_octaves, lv.base_texels, lv.n_coarse, lv.coarse_H, lv.coarse_W)


_GEOM = {}          # (H, W, TILE, levels) -> levels_geometry result
_PAIRS_HW = {}      # binning configuration -> most pairs one image needed so far (sizes the next capacity)
_LEVELS_SEEN = {}   # binning configuration -> per-level pair totals of its last binning (plans deferred launches)
_WS1 = {}           # binning configuration -> count-phase workspace bytes
_tls = threading.local()


def _info_host():
    """Pinned int64 landing buffer of the binning's one read-back (per thread, reused)."""
    buf = getattr(_tls, "info", None)
    if buf is None:
        t = torch.empty(2 + _lib.MAX_LEVELS, dtype=torch.int64, pin_memory=True)
        buf = _tls.info = (t, t.numpy())
    return buf


def _align(n):
    return (n + 255) & ~255


_CARVE_OFF = {}   # tuple of sizes -> sub-buffer offsets (the renders of one configuration repeat their sizes)
_PAIRS_WS = {}    # (binning configuration, capacity) -> pair-phase workspace bytes
_SUMS_FLOATS = {}   # capacity -> floats of one image's per-pair sums (16-byte aligned)


class _Carve:
    """Sub-buffers of one uint8 device allocation (256-byte aligned)."""

    def __init__(self, sizes, dev, zero=False):
        key = tuple(sizes)
        off = _CARVE_OFF.get(key)
        if off is None:
            off, o = [], 0
            for n in sizes:
                off.append(o)
                o += _align(max(int(n), 1))
            off.append(o)
            if len(_CARVE_OFF) > 4096:
                _CARVE_OFF.clear()
            _CARVE_OFF[key] = off
        self.off = off
        self.buf = (torch.zeros if zero else torch.empty)(off[-1], dtype=torch.uint8, device=dev)
        self.base = self.buf.data_ptr()

    def ptr(self, i):
        return self.base + self.off[i]

    def nbytes(self, i):
        return self.off[i + 1] - self.off[i]

    def view(self, i, n, dtype, shape=None):
        t = self.buf[self.off[i]:self.off[i] + 4 * n].view(dtype)     # 4-byte element types only
        return t if shape is None else t.view(shape)


def _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs=None, with_maps=True, lv=None,
         scale_is_log=False, defer=False) -> TileBins:
    """Decode + bin every batch (render_triton.py:351-409). One host read of the pair totals per image.
    with_maps=False skips the pair maps only the backward needs (forward-only renders). `lv` (a
    _lib.SplatLevels) routes splats to levels (octave / coarse-fine renders, render_triton.py:879-980).
    scale_is_log: `scale` holds fp32 raw log-scales, activated in the decode pass (params.py:18-28).
    defer: for one image whose configuration has been binned before, return with the read of the pair count
    still pending (bins.pending): the caller queues its launches on the speculative pair list first, then calls
    _finish (which redoes the pair phase when the count exceeded the capacity)."""
    _dev_check(mu, scale, color, opacity, theta)
    ev = kernel_timer.record("bin")
    try:
        return _bin_impl(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps, lv,
                         FLAG_LOG_SCALE if scale_is_log else 0, defer)
    finally:
        kernel_timer.close("bin", ev)


def _budget_error(n, max_pairs, H, W, TILE, cutoff, N):
    return PairBudgetExceeded(
        f"_build_tiles: {n} (tile,gaussian) pairs exceeds the {max_pairs} budget @ {H}x{W} "
        f"TILE={TILE} cutoff={cutoff} N={N}. Route large splats through the low-res (octave) pass "
        f"instead of culling at full res. Refusing to allocate.")


def _pair_buffers(lib, N, nt, cap, with_maps, dev, geo, key=None):
    """gid, starts, pair_q and the pair-phase workspace for up to `cap` pairs, one allocation.
    geo = (H, W, TILE, levels byref or None); key: the binning configuration (caches the workspace size)."""
    c = max(cap, 1)
    m = c if with_maps else 0
    wk = None if key is None else (key, cap)
    wsb = _PAIRS_WS.get(wk) if wk is not None else None
    if wsb is None:
        wsb = lib.splat_bin_pairs_workspace_bytes(N, *geo, cap)
        if wk is not None:
            if len(_PAIRS_WS) > 4096:
                _PAIRS_WS.clear()
            _PAIRS_WS[wk] = wsb
    return _Carve([4 * c, 4 * (nt + 1), 4 * m, wsb], dev)


class _Pending:
    """A binning whose pair count has not been read yet (FLAG_DEFER): what settling it needs."""

    __slots__ = ("lib", "info_p", "info_np", "blk", "cap", "budget", "key", "geo", "N", "L", "nt", "geom", "cutoff",
                 "max_pairs", "with_maps", "stream", "dev")

    def __init__(self, lib, info_p, info_np, blk, cap, budget, key, geo, N, L, nt, geom, cutoff, max_pairs, with_maps,
                 stream, dev):
        self.lib, self.info_p, self.info_np, self.blk, self.cap, self.budget = lib, info_p, info_np, blk, cap, budget
        self.key, self.geo, self.N, self.L, self.nt, self.geom = key, geo, N, L, nt, geom
        self.cutoff, self.max_pairs, self.with_maps, self.stream, self.dev = cutoff, max_pairs, with_maps, stream, dev


def _settle(p, rc, pb):
    """The checks after the read of one image's totals (p: a _Pending): raises for the budget and bad rects,
    redoes the pair phase with exact buffers when the count exceeded the capacity. Returns (pair buffers, tot,
    level totals, redone)."""
    lib, info_np, L, geom = p.lib, p.info_np, p.L, p.geom
    H, W, TILE, lvr = p.geo
    tot = int(info_np[0])
    lt = info_np[2:2 + L].tolist()
    if rc == _lib.STATUS_BUDGET:
        l = max(range(L), key=lambda i: lt[i])
        Hl, Wl = (H, W) if geom is None else geom[l][:2]
        raise _budget_error(lt[l], p.max_pairs, Hl, Wl, TILE, p.cutoff, p.N)
    if rc == 1 and info_np[1] & 1:
        raise ValueError("binning: a splat has an empty tile rect (negative cutoff or scale)")
    if rc == 4:
        raise PairBudgetExceeded(f"binning: {tot} pairs exceed the int32 pair index range")
    redone = rc == _lib.STATUS_CAPACITY
    if redone:
        pb = _pair_buffers(lib, p.N, p.nt, tot, p.with_maps, p.dev, p.geo)
        blk = p.blk
        check(lib.splat_bin_pairs(blk.ptr(1), blk.ptr(2), blk.ptr(4), p.N, H, W, TILE, lvr, tot, pb.ptr(0), pb.ptr(1),
                                  None, pb.ptr(2) if p.with_maps else None, pb.ptr(3), pb.nbytes(3), p.stream),
              "splat_bin_pairs")
    else:
        check(rc, "splat_bin")
    if tot > _PAIRS_HW.get(p.key, 0):
        _PAIRS_HW[p.key] = tot
    _LEVELS_SEEN[p.key] = lt
    return pb, tot, lt, redone


def _bin_impl(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps, lv, sflags, defer=False):
    B, N, C = color.shape
    dev = mu.device
    lib = _lib.load()
    lvr = None if lv is None else _lib.ctypes.byref(lv)
    mu_, sc_, col_, op_, th_ = _f32(mu), _f32(scale), _f32(color), _f32(opacity), _f32(theta)
    geom, nt, npix = levels_geometry(H, W, TILE, lv)
    L = len(geom)
    ntx = geom[0][2]
    if lv is None:
        geom = None
    if N == 0:
        blk = _Carve([64, 0, 4], dev, zero=True)
        pb = _Carve([4, 4 * (nt + 1), 0, 0], dev, zero=True)
        return TileBins(0, [0] * B, H, W, TILE, ntx, nt, [blk] * B, [pb] * B, False, lv, geom, npix, [[0] * L] * B)
    stream = _lib.stream_ptr(dev)
    key = (N, H, W, TILE, float(cutoff), _lv_key(lv))
    hw = _PAIRS_HW.get(key, 0)
    cap = hw + (hw >> 4) + 1024 if hw else 0
    info_t, info_np = _info_host()
    info_p = info_t.data_ptr()
    geo = (H, W, TILE, lvr)
    ws1_bytes = _WS1.get(key)
    if ws1_bytes is None:
        ws1_bytes = _WS1[key] = lib.splat_bin_count_workspace_bytes(N, *geo)
    budget = -1 if max_pairs is None else int(max_pairs)
    defer = defer and B == 1 and cap > 0
    blocks, pairs, tots, level_tots = [], [], [], []
    for b in range(B):
        blk = _Carve([64 * N, 16 * N, 4 * (N + 1), 8 * (2 + L), ws1_bytes], dev)
        pb = _pair_buffers(lib, N, nt, cap, with_maps, dev, geo, key) if cap else None
        pp = (lambda i: None) if pb is None else pb.ptr
        info_np[0] = info_np[1] = 0
        rc = lib.splat_bin(_bptr(mu_, b), _bptr(sc_, b), _bptr(th_, b), _bptr(op_, b), _bptr(col_, b),
                           C, N, H, W, TILE, float(cutoff), lvr, sflags | (FLAG_DEFER if defer else 0), budget,
                           blk.ptr(0), blk.ptr(1), blk.ptr(2), blk.ptr(3), info_p, blk.ptr(4), ws1_bytes, cap, pp(0),
                           pp(1), None, pp(2) if with_maps else None, pp(3), 0 if pb is None else pb.nbytes(3), stream)
        pend = _Pending(lib, info_p, info_np, blk, cap, budget, key, geo, N, L, nt, geom, cutoff, max_pairs, with_maps,
                        stream, dev)
        if defer:
            check(rc, "splat_bin")
            bins = TileBins(N, [None], H, W, TILE, ntx, nt, [blk], [pb], with_maps, lv, geom, npix, [None])
            bins.pending = pend
            return bins
        pb, tot, lt, _ = _settle(pend, rc, pb)
        blocks.append(blk)
        pairs.append(pb)
        tots.append(tot)
        level_tots.append(lt)
    return TileBins(N, tots, H, W, TILE, ntx, nt, blocks, pairs, with_maps, lv, geom, npix, level_tots)


def _finish(bins):
    """Reads the totals of a deferred binning (one image) and settles it; True when its pair phase had to be
    redone (the count exceeded the speculated capacity), so that launches queued on the speculative pair list
    must be repeated."""
    p = bins.pending
    if p is None:
        return False
    bins.pending = None
    rc = p.lib.splat_bin_finish(p.info_p, p.blk.ptr(3), p.L, p.budget, p.cap, p.stream)
    pb, tot, lt, redone = _settle(p, rc, bins.pairs[0])
    bins.pairs[0] = pb
    bins.tot_b[0] = tot
    bins.level_tot_b[0] = lt
    bins._views = {}
    bins._ptrs = {}
    return redone


def _speculated_levels(bins):
    """Per-level pair totals to plan the launches of a deferred binning by: the last totals of this configuration."""
    if bins.pending is None:
        return bins.level_tot_b[0]
    return _LEVELS_SEEN.get(bins.pending.key)


def _build_tiles(mu, scale, H, W, TILE, cutoff, max_pairs=None):
    """(gid_b, starts_b, ntx, nt) exactly as render_triton.py:351-409 returns them."""
    B, N, _ = mu.shape
    dummy_col = torch.zeros((B, N, 1), device=mu.device)
    dummy_op = torch.zeros((B, N), device=mu.device)
    return _bin(mu, scale, dummy_col, dummy_op, None, H, W, TILE, cutoff, max_pairs, with_maps=False).as_tuple()


# ----------------------------------------------------------------------------------------------- cull path
def _wide(TILE, ntiles, pairs):
    """FLAG_WIDE (16 waves per 8x8 tile instead of 4 in the forward, instead of 1 in the backward) for a launch over
    few tiles with long pair lists, where fewer waves per tile would leave most of the GPU idle."""
    return FLAG_WIDE if TILE == 8 and 0 < ntiles < 2048 and pairs >= 128 * ntiles else 0


_SPLIT_PAIRS = 128   # pairs per workgroup the split launches of the coarse levels aim at
_SPLIT_MAX = 64


def _level_splits(bins, lt, mask):
    """Chunks per tile of every level for the split FIELDS launches over the coarse levels (ctypes int array):
    a level in `mask` gets about _SPLIT_PAIRS pairs per chunk on average over its tiles (1 to _SPLIT_MAX chunks),
    so a dense coarse level's few tiles with long pair lists are spread over many workgroups; level 0 and levels
    outside `mask` get 1 (unused)."""
    geom, L = bins.geom, bins.n_levels
    sp = (_lib.ctypes.c_int * L)()
    for l in range(L):
        sp[l] = 1
        if l and (mask >> l) & 1:
            tiles = (geom[l + 1][3] if l + 1 < L else bins.nt) - geom[l][3]
            if tiles:
                sp[l] = max(1, min(_SPLIT_MAX, -(-int(lt[l]) // (_SPLIT_PAIRS * tiles))))
    return sp


def _fwd_order(bins, lt, mask, held):
    """What the summation order of a levels forward launched for per-level totals lt over the levels in `mask`
    depends on, over the levels in `held`: each coarse level's chunks per tile (their partial sums are added in
    chunk order) and the level-0 composite's waves per tile."""
    sp = _level_splits(bins, lt, mask & ~1)
    return (tuple(sp[l] for l in range(1, bins.n_levels) if (held >> l) & 1),
            _wide(bins.TILE, bins.ntiles0, lt[0]))


def _fields_buffers(npix, C, dev):
    """Packed level fields S_log [Pt], S_a [Pt], S_ac [Pt,C], views of one allocation."""
    slog, sa, sac = torch.empty(npix * (2 + C), device=dev).split_with_sizes((npix, npix, npix * C))
    return slog, sa, sac.view(npix, C)


_SPLIT_WS = {}   # (C, H, W, TILE, levels, mask, splits) -> split-launch workspace bytes
_ADJ_WS = {}     # (C, H, W, TILE, levels) -> upsample-adjoint workspace bytes


def _fields_split_fwd(lib, bins, b, C, odd, lt, mask, fl, stream):
    """FIELDS forward of the coarse levels in `mask` of image b into the packed fields fl, one split launch."""
    L = bins.n_levels
    lvr = _lib.ctypes.byref(bins.lv)
    sp = _level_splits(bins, lt, mask)
    key = (C, bins.H, bins.W, bins.TILE, _lv_key(bins.lv), mask, tuple(sp))
    nb = _SPLIT_WS.get(key)
    if nb is None:
        nb = _SPLIT_WS[key] = lib.splat_fields_split_workspace_bytes(C, bins.H, bins.W, bins.TILE, lvr, 1, L, mask, sp)
    ws = _ws(nb, fl[0].device) if nb else None
    check(lib.splat_render_fields_split(bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"), C, bins.H, bins.W,
                                        bins.TILE, odd, lvr, 1, L, mask, sp, *[ptr(t) for t in fl], ptr(ws), nb,
                                        stream), "splat_render_fields_split")


def _render_fwd(lib, bins, b, C, flags, lev, mask, comp, fields, stream):
    """splat_render_fwd for batch b over levels lev = (begin, end); comp = (bg, out, T, asum, fg) or Nones,
    fields = (slog, sa, sac) or Nones."""
    lvr = None if bins.lv is None else _lib.ctypes.byref(bins.lv)
    check(lib.splat_render_fwd(bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"), C, bins.H, bins.W,
                               bins.TILE, flags, lvr, lev[0], lev[1], mask, *[ptr(t) for t in comp],
                               *[ptr(t) for t in fields], stream), "splat_render_fwd")


def _composite_buffers(B, P, C, dev):
    """out [B,P,C], T [B,P], asum [B,P], fg [B,P,C] as contiguous views of one allocation (strided views: one
    operation each)."""
    n = B * P
    t = torch.empty(n * (2 * C + 2), device=dev)
    return (t.as_strided((B, P, C), (P * C, C, 1), 0), t.as_strided((B, P), (P, 1), n * C),
            t.as_strided((B, P), (P, 1), n * (C + 1)), t.as_strided((B, P, C), (P * C, C, 1), n * (C + 2)))


def _forward_cull(mu, scale, color, opacity, bg, theta, H, W, TILE=8, cutoff=3.0, max_pairs=None, odds=False,
                  with_maps=True, scale_is_log=False, plan=None):
    """Composite forward (render_triton.py:538-567): out [B,P,C], (T, asum, fg), bins. plan: a _BwdPlan to
    prepare for the backward (its buffers are allocated while the pair count is read back)."""
    B, N, C = color.shape
    P = H * W
    dev = mu.device
    bins = _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps, scale_is_log=scale_is_log,
                defer=True)
    out, T, asum, fg = _composite_buffers(B, P, C, dev)
    bgf = _f32(bg)
    flags = FLAG_ODDS if odds else 0
    lib, stream = _lib.load(), _lib.stream_ptr(dev)

    def launch(tots):
        for b in range(B):
            comp = (_bptr(bgf, b), _bptr(out, b), _bptr(T, b), _bptr(asum, b), _bptr(fg, b))
            if not kernel_timer.enabled:
                _render_fwd(lib, bins, b, C, flags | _wide(TILE, bins.nt, tots[b]), (0, 1), 1, comp, (None,) * 3,
                            stream)
                continue
            ev = kernel_timer.record("fwd")
            try:
                _render_fwd(lib, bins, b, C, flags | _wide(TILE, bins.nt, tots[b]), (0, 1), 1, comp, (None,) * 3,
                            stream)
            finally:
                kernel_timer.close("fwd", ev)

    if bins.pending is not None:   # queued on the speculative pair list before the count is read
        spec = _speculated_levels(bins)[0]
        launch([spec])
        if plan is not None:         # the backward's buffers, allocated while the GPU works towards the count
            plan.allocate(bins, B, N, C, dev, lib, bins.pending.cap)
        # launched again when the pair phase was redone, or when the count asks for another number of waves per
        # tile than the speculated one (they group the per-pixel sums: the image depends on the inputs alone)
        if _finish(bins) or _wide(TILE, bins.nt, bins.tot_b[0]) != _wide(TILE, bins.nt, spec):
            launch(bins.tot_b)
    else:
        launch(bins.tot_b)
    if plan is not None:
        plan.bind(bins, B, N, C, dev, lib, stream, flags, (bgf, T, asum, fg))
    return out, (T, asum, fg), bins


class _BwdPlan:
    """The backward of a culled composite render prepared by its forward: the gradient outputs, the per-pair sums
    and per-tile background partials (allocated while the forward waits for the pair count), and the argument lists
    of the two backward launches per image, complete but for the upstream gradient's pointer. The backward then runs
    two C-ABI calls per image (render_triton.py:723-765 in two kernels)."""

    __slots__ = ("grads", "sums", "ns", "cap", "bwd_head", "bwd_tail", "red_args", "lsc", "has_th", "keep")

    def __init__(self, has_th, lsc=None):
        self.has_th = has_th
        self.lsc = _f32(lsc)   # the raw log-scales as the reduction reads them (kept alive here)
        self.cap = -1
        self.sums = None

    def allocate(self, bins, B, N, C, dev, lib, cap):
        """Gradient outputs and one buffer for the per-pair sums of every image (ns floats each, 16-byte aligned)
        followed by the per-tile background partials (the kernels take both by pointer)."""
        self.grads = _grads_bg_out(B, N, C, dev, self.has_th)
        ns = _SUMS_FLOATS.get(cap)
        if ns is None:
            if len(_SUMS_FLOATS) > 1024:
                _SUMS_FLOATS.clear()
            ns = _SUMS_FLOATS[cap] = (lib.splat_pair_sums_bytes(max(cap, 1)) // 4 + 3) & ~3
        self.sums = torch.empty(B * ns + C * bins.ntiles0, device=dev)
        self.ns = ns
        self.cap = cap

    def bind(self, bins, B, N, C, dev, lib, stream, flags, comp):
        tots = bins.tot_b
        if self.sums is None or max(tots) > self.cap:
            self.allocate(bins, B, N, C, dev, lib, max(tots))
        ns = self.ns
        g_mu, g_scale, g_col, g_op, g_th, g_bg = self.grads
        bgf, T, asum, fg = comp
        self.keep = bgf   # the kernels read the background through its pointer
        lvr = None if bins.lv is None else _lib.ctypes.byref(bins.lv)
        sums0 = self.sums.data_ptr()
        bgp = sums0 + 4 * B * ns
        self.bwd_head, self.bwd_tail, self.red_args = [], [], []
        for b in range(B):
            sb = sums0 + 4 * ns * b
            self.bwd_head.append((bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"), bins.p(b, "pq"), tots[b], C,
                                  bins.H, bins.W, bins.TILE, flags | _wide(bins.TILE, bins.nt, tots[b]), lvr, 0, 1, 1,
                                  _bptr(bgf, b), _bptr(T, b), _bptr(asum, b), _bptr(fg, b)))
            self.bwd_tail.append((None, None, None, sb, bgp, stream))
            sl = lambda t: None if N == 0 else _bptr(t, b)
            self.red_args.append((bins.p(b, "rec") if N else None, bins.p(b, "off") if N else None, None, tots[b], N, C,
                                  sb, bgp, bins.ntiles0, sl(self.lsc), sl(g_mu), sl(g_scale), sl(g_th), sl(g_op),
                                  sl(g_col), _bptr(g_bg, b), stream))

    def run(self, lib, grad_out, H, W, C):
        """The two launches per image with grad_out [B,C,H,W]; returns the gradients (the plan then holds none)."""
        B = grad_out.shape[0]
        img = H * W * C
        if grad_out.dtype is torch.float32 and grad_out.stride() == (img, 1, W * C, C):
            g0 = grad_out.data_ptr()     # the image's own [B,H,W,C] layout: no copy
        else:
            go = grad_out.permute(0, 2, 3, 1).contiguous().float()
            g0 = go.data_ptr()
        timed = kernel_timer.enabled
        for b in range(B):
            if not timed:
                check(lib.splat_render_bwd(*self.bwd_head[b], g0 + 4 * img * b, *self.bwd_tail[b]), "splat_render_bwd")
                check(lib.splat_reduce_pairs(*self.red_args[b]), "splat_reduce_pairs")
                continue
            ev = kernel_timer.record("bwd")
            try:
                check(lib.splat_render_bwd(*self.bwd_head[b], g0 + 4 * img * b, *self.bwd_tail[b]), "splat_render_bwd")
            finally:
                kernel_timer.close("bwd", ev)
            ev = kernel_timer.record("reduce")
            try:
                check(lib.splat_reduce_pairs(*self.red_args[b]), "splat_reduce_pairs")
            finally:
                kernel_timer.close("reduce", ev)
        g_mu, g_scale, g_col, g_op, g_th, g_bg = self.grads
        self.grads = self.sums = self.keep = None
        return g_mu, g_scale, g_col, g_op, g_bg, g_th


def _forward_cull_fields(mu, scale, color, opacity, theta, H, W, TILE=8, cutoff=3.0, max_pairs=None, odds=False,
                         with_maps=True):
    """FIELDS forward (render_triton.py:570-599): S_log [B,P], S_a [B,P] (unclamped), S_ac [B,P,C], bins."""
    B, N, C = color.shape
    P = H * W
    dev = mu.device
    bins = _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps)
    slog, sa, sac = _empty((B, P), dev), _empty((B, P), dev), _empty((B, P, C), dev)
    flags = FLAG_FIELDS | (FLAG_ODDS if odds else 0)
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    for b in range(B):
        _render_fwd(lib, bins, b, C, flags | _wide(TILE, bins.nt, bins.tot_b[b]), (0, 1), 1, (None,) * 5,
                    (slog[b], sa[b], sac[b]), stream)
    return slog, sa, sac, bins


def _forward_levels(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv, with_maps=True,
                    scale_is_log=False, plan=None):
    """Fused multi-level forward (render_triton.py:879-980 without the per-group torch glue): one binning
    over every level, FIELDS renders of the coarse levels into packed fields, then the level-0 composite
    adds their bilinear upsamples. Returns out [B,P,C], (T, asum unclamped, fg), bins. plan: a _LevelsBwdPlan to
    prepare for the backward (its buffers are allocated while the pair count is read back)."""
    B, N, C = color.shape
    P = H * W
    dev = mu.device
    bins = _bin(mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, with_maps, lv=lv,
                scale_is_log=scale_is_log, defer=True)
    out, T, asum, fg = _composite_buffers(B, P, C, dev)
    L = bins.n_levels
    # packed fields, reused across the batch (stream order); slots [0, P) belong to level 0 and stay unused
    fl = _fields_buffers(bins.npix, C, dev) if L > 1 else (None, None, None)
    bgf = _f32(bg)
    odd = FLAG_ODDS if odds else 0
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    nt0 = bins.ntiles0

    def launch(b, lt, mask):
        """The launches of image b for per-level pair totals lt (they size the coarse levels' split and pick the
        16-wave composite) over the levels in mask (a level in mask that holds no pair renders zeros)."""
        ev = kernel_timer.record("fwd")
        try:
            if mask & ~1:
                _fields_split_fwd(lib, bins, b, C, odd, lt, mask & ~1, fl, stream)
            _render_fwd(lib, bins, b, C, FLAG_UPS | odd | _wide(TILE, nt0, lt[0]), (0, 1), mask,
                        (_bptr(bgf, b), _bptr(out, b), _bptr(T, b), _bptr(asum, b), _bptr(fg, b)), fl, stream)
        finally:
            kernel_timer.close("fwd", ev)

    if bins.pending is not None:   # queued on the speculative pair list and levels before the count is read
        lt_spec = _speculated_levels(bins)
        mask_spec = _mask_of(lt_spec)
        launch(0, lt_spec, mask_spec)
        if plan is not None:         # the backward's buffers, allocated while the GPU works towards the count
            plan.allocate(bins, B, N, C, dev, lib, bins.pending.cap)
        redone = _finish(bins)
        lt, held = bins.level_tot_b[0], bins.level_mask(0)
        # launched again when the pair phase was redone, when a level holding pairs was left out, or when the
        # count asks for another summation order than the speculated totals gave
        if redone or held & ~mask_spec or _fwd_order(bins, lt_spec, mask_spec, held) != _fwd_order(bins, lt, held,
                                                                                                     held):
            launch(0, lt, held)
    else:
        for b in range(B):
            launch(b, bins.level_tot_b[b], bins.level_mask(b))
    if plan is not None:
        plan.bind(bins, B, N, C, dev, lib, stream, odd, (bgf, T, asum, fg))
    return out, (T, asum, fg), bins


def _grads_out(B, N, C, dev, has_th):
    return (_empty((B, N, 2), dev), _empty((B, N, 2), dev), _empty((B, N, C), dev), _empty((B, N), dev),
            _empty((B, N), dev) if has_th else None)


def _grads_bg_out(B, N, C, dev, has_th):
    """g_mu [B,N,2], g_scale [B,N,2], g_col [B,N,C], g_op [B,N], g_th [B,N] (or None) and g_bg [B,C]: views of one
    allocation (each a contiguous tensor of its own shape)."""
    n2, nc, n1 = B * N * 2, B * N * C, B * N
    t = torch.empty(2 * n2 + nc + (2 if has_th else 1) * n1 + B * C, device=dev)
    o = 2 * n2 + nc + n1
    return (t.as_strided((B, N, 2), (2 * N, 2, 1), 0), t.as_strided((B, N, 2), (2 * N, 2, 1), n2),
            t.as_strided((B, N, C), (N * C, C, 1), 2 * n2), t.as_strided((B, N), (N, 1), 2 * n2 + nc),
            t.as_strided((B, N), (N, 1), o) if has_th else None,
            t.as_strided((B, C), (C, 1), o + (n1 if has_th else 0)))


def _render_bwd(lib, bins, b, C, flags, lev, mask, upstream, sums, bg_part, stream):
    """splat_render_bwd for batch b over levels lev = (begin, end); upstream = (bg, T, asum, fg, gout, dslog,
    dsa, dsac) with Nones where unused."""
    lvr = None if bins.lv is None else _lib.ctypes.byref(bins.lv)
    check(lib.splat_render_bwd(bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"), bins.p(b, "pq"),
                               bins.tot_b[b], C,
                               bins.H, bins.W, bins.TILE, flags, lvr, lev[0], lev[1], mask,
                               *[ptr(u) for u in upstream], ptr(sums), ptr(bg_part), stream), "splat_render_bwd")


def _reduce(lib, bins, b, C, sums, bg_part, grads, g_bg, stream, lsc=None):
    """Per-splat reduction of batch b's pair sums into `grads` (and g_bg from the level-0 tile partials).
    lsc: the fp32 raw log-scales [B,N,2] of a scale_is_log binning; g_scale is then w.r.t. them."""
    tot = bins.tot_b[b]
    N = bins.N
    g_mu, g_scale, g_col, g_op, g_th = grads
    sl = lambda t: None if N == 0 else _bptr(t, b)
    ev = kernel_timer.record("reduce")
    try:
        check(lib.splat_reduce_pairs(bins.p(b, "rec") if N else None, bins.p(b, "off") if N else None,
                                     None, tot, N, C, ptr(sums), ptr(bg_part),
                                     bins.ntiles0, sl(lsc), sl(g_mu), sl(g_scale), sl(g_th), sl(g_op), sl(g_col),
                                     ptr(g_bg), stream), "splat_reduce_pairs")
    finally:
        kernel_timer.close("reduce", ev)


def _bwd_buffers(lib, bins, b, C, with_bg, dev):
    """Per-pair sums and (optionally) the level-0 per-tile background partials, one allocation."""
    ns = (lib.splat_pair_sums_bytes(bins.tot_b[b]) // 4 + 3) & ~3   # partials start 16-byte aligned
    if not with_bg:
        return torch.empty(ns, device=dev), None
    return torch.empty(ns + C * bins.ntiles0, device=dev).split_with_sizes((ns, C * bins.ntiles0))


def _backward_pairs(bins, b, flags, C, upstream, grads, g_bg, lib, stream, lsc=None):
    """Both backward steps for batch b of a single-level render: per-tile pair sums, then the per-splat
    reduction into `grads`."""
    dev = bins.blocks[b].buf.device
    sums, bg_part = _bwd_buffers(lib, bins, b, C, g_bg is not None, dev)
    flags |= _wide(bins.TILE, bins.nt, bins.tot_b[b])
    ev = kernel_timer.record("bwd")
    try:
        _render_bwd(lib, bins, b, C, flags, (0, 1), 1, upstream, sums, bg_part, stream)
    finally:
        kernel_timer.close("bwd", ev)
    _reduce(lib, bins, b, C, sums, bg_part, grads, g_bg, stream, lsc)


def _backward_cull(grad_out, mu, scale, color, opacity, bg, theta, T, asum, fg, bins, H, W, TILE=8, odds=False,
                   scale_is_log=False):
    """render_triton.py:723-765: grads for mu, scale, color, opacity, bg, theta (None without theta) from
    grad_out [B,P,C]. scale_is_log: `scale` holds the raw log-scales the binning activated; g_scale is w.r.t.
    them."""
    B, N, C = color.shape
    return _backward_cull_raw(grad_out, bg, scale if scale_is_log else None, B, N, C, mu.device, theta is not None,
                              T, asum, fg, bins, odds)


def _backward_cull_raw(grad_out, bg, lsc, B, N, C, dev, has_th, T, asum, fg, bins, odds):
    """_backward_cull on what it reads: grad_out [B,P,C], bg, the raw log-scales lsc (or None) and shapes."""
    g_mu, g_scale, g_col, g_op, g_th, g_bg = _grads_bg_out(B, N, C, dev, has_th)
    grads = (g_mu, g_scale, g_col, g_op, g_th)
    go, bgf = _f32(grad_out), _f32(bg)
    lsc = _f32(lsc)
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    flags = FLAG_ODDS if odds else 0
    for b in range(B):
        up = (_bptr(bgf, b), _bptr(T, b), _bptr(asum, b), _bptr(fg, b), _bptr(go, b), None, None, None)
        _backward_pairs(bins, b, flags, C, up, grads, _bptr(g_bg, b), lib, stream, lsc)
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
        _backward_pairs(bins, b, flags, C, up, grads, None, lib, stream)
    return grads


def _backward_levels(grad_out, color, bg, has_theta, T, asum, fg, bins, odds, log_scale=None):
    """Backward of _forward_levels: level-0 composite backward (clamp_min gradient of S_a, render_triton.py
    :918 / :976) writing the pixel upstream, its exact adjoint through the upsample onto the coarse levels,
    their FIELDS backward, then one per-splat reduction over the pairs of every level. log_scale: the raw
    log-scales of a scale_is_log binning (g_scale is then w.r.t. them)."""
    B, N, C = color.shape
    dev = color.device
    g_mu, g_scale, g_col, g_op, g_th, g_bg = _grads_bg_out(B, N, C, dev, has_theta)
    grads = (g_mu, g_scale, g_col, g_op, g_th)
    go, bgf = _f32(grad_out), _f32(bg)
    lib, stream = _lib.load(), _lib.stream_ptr(dev)
    odd = FLAG_ODDS if odds else 0
    L = bins.n_levels
    npix = bins.npix if L > 1 else bins.H * bins.W
    dS = _fields_buffers(npix, C, dev)   # the pixel upstream dS_log, dS_a, dS_ac, reused across the batch
    lvr = None if bins.lv is None else _lib.ctypes.byref(bins.lv)
    adj_ws = None
    if L > 1:
        key = (C, bins.H, bins.W, bins.TILE, _lv_key(bins.lv))
        nb = _ADJ_WS.get(key)
        if nb is None:
            nb = _ADJ_WS[key] = lib.splat_upsample_adjoint_workspace_bytes(C, bins.H, bins.W, bins.TILE, lvr)
        adj_ws = _ws(nb, dev)
    lsc = None if log_scale is None else _f32(log_scale)
    nt0 = bins.ntiles0
    for b in range(B):
        mask = bins.level_mask(b)
        lt = bins.level_tot_b[b]
        sums, bg_part = _bwd_buffers(lib, bins, b, C, True, dev)
        ev = kernel_timer.record("bwd")
        try:
            _render_bwd(lib, bins, b, C, FLAG_UPS | odd | _wide(bins.TILE, nt0, lt[0]), (0, 1), mask,
                        (_bptr(bgf, b), _bptr(T, b), _bptr(asum, b), _bptr(fg, b), _bptr(go, b), *dS), sums,
                        bg_part, stream)
            if mask & ~1:
                check(lib.splat_upsample_adjoint(C, bins.H, bins.W, bins.TILE, lvr, mask, *[ptr(t) for t in dS],
                                                 ptr(adj_ws), adj_ws.numel(), stream), "splat_upsample_adjoint")
                check(lib.splat_render_fields_split_bwd(bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"),
                                                        bins.p(b, "pq"), bins.tot_b[b], C, bins.H, bins.W, bins.TILE,
                                                        odd, lvr, 1, L, mask & ~1, _level_splits(bins, lt, mask & ~1),
                                                        *[ptr(t) for t in dS], ptr(sums), stream),
                      "splat_render_fields_split_bwd")
        finally:
            kernel_timer.close("bwd", ev)
        _reduce(lib, bins, b, C, sums, bg_part, grads, _bptr(g_bg, b), stream, lsc)
    return g_mu, g_scale, g_col, g_op, g_bg, g_th


class _LevelsBwdPlan:
    """_backward_levels prepared by its forward: the gradient outputs, the pixel upstream fields, the upsample
    adjoint's workspace, the per-pair sums and the level-0 background partials (allocated while the forward waits
    for the pair count), and the argument lists of the backward's launches per image, complete but for the
    upstream gradient's pointer. The backward then runs its C-ABI calls only (the same launches, in the same order,
    as _backward_levels)."""

    __slots__ = ("grads", "dS", "adj", "adj_n", "sums", "ns", "cap", "calls", "lsc", "has_th", "keep")

    def __init__(self, has_th, lsc=None):
        self.has_th = has_th
        self.lsc = _f32(lsc)   # the raw log-scales as the reduction reads them (kept alive here)
        self.cap = -1
        self.sums = None

    def allocate(self, bins, B, N, C, dev, lib, cap):
        self.grads = _grads_bg_out(B, N, C, dev, self.has_th)
        L = bins.n_levels
        self.dS = _fields_buffers(bins.npix if L > 1 else bins.H * bins.W, C, dev)   # reused across the batch
        self.adj, self.adj_n = None, 0
        if L > 1:
            key = (C, bins.H, bins.W, bins.TILE, _lv_key(bins.lv))
            nb = _ADJ_WS.get(key)
            if nb is None:
                lvr = _lib.ctypes.byref(bins.lv)
                nb = _ADJ_WS[key] = lib.splat_upsample_adjoint_workspace_bytes(C, bins.H, bins.W, bins.TILE, lvr)
            self.adj = _ws(nb, dev)
            self.adj_n = self.adj.numel()
        ns = _SUMS_FLOATS.get(cap)
        if ns is None:
            if len(_SUMS_FLOATS) > 1024:
                _SUMS_FLOATS.clear()
            ns = _SUMS_FLOATS[cap] = (lib.splat_pair_sums_bytes(max(cap, 1)) // 4 + 3) & ~3
        self.sums = torch.empty(B * ns + C * bins.ntiles0, device=dev)   # per-image sums, then the partials
        self.ns = ns
        self.cap = cap

    def bind(self, bins, B, N, C, dev, lib, stream, odd, comp):
        tots = bins.tot_b
        if self.sums is None or max(tots) > self.cap:
            self.allocate(bins, B, N, C, dev, lib, max(tots))
        g_mu, g_scale, g_col, g_op, g_th, g_bg = self.grads
        bgf, T, asum, fg = comp
        self.keep = bgf   # the kernels read the background through its pointer
        L = bins.n_levels
        lvr = None if bins.lv is None else _lib.ctypes.byref(bins.lv)
        ds = tuple(t.data_ptr() for t in self.dS)
        sums0 = self.sums.data_ptr()
        bgp = sums0 + 4 * B * self.ns
        nt0 = bins.ntiles0
        self.calls = []
        for b in range(B):
            mask, lt = bins.level_mask(b), bins.level_tot_b[b]
            sb = sums0 + 4 * self.ns * b
            head = (bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"), bins.p(b, "pq"), tots[b], C, bins.H,
                    bins.W, bins.TILE, FLAG_UPS | odd | _wide(bins.TILE, nt0, lt[0]), lvr, 0, 1, mask, _bptr(bgf, b),
                    _bptr(T, b), _bptr(asum, b), _bptr(fg, b))
            tail = (*ds, sb, bgp, stream)
            adj = split = None
            if mask & ~1:
                adj = (C, bins.H, bins.W, bins.TILE, lvr, mask, *ds, ptr(self.adj), self.adj_n, stream)
                split = (bins.p(b, "rec"), bins.p(b, "gid"), bins.p(b, "starts"), bins.p(b, "pq"), tots[b], C, bins.H,
                         bins.W, bins.TILE, odd, lvr, 1, L, mask & ~1, _level_splits(bins, lt, mask & ~1), *ds, sb,
                         stream)
            sl = lambda t: None if N == 0 else _bptr(t, b)
            red = (bins.p(b, "rec") if N else None, bins.p(b, "off") if N else None, None, tots[b], N, C, sb, bgp, nt0,
                   sl(self.lsc), sl(g_mu), sl(g_scale), sl(g_th), sl(g_op), sl(g_col), _bptr(g_bg, b), stream)
            self.calls.append((head, tail, adj, split, red))

    def run(self, lib, go):
        """The launches per image with the upstream gradient go [B,P,C] (float32, contiguous per image); returns the
        gradients (the plan then holds none)."""
        img = go.shape[1] * go.shape[2]
        g0 = go.data_ptr()
        for b, (head, tail, adj, split, red) in enumerate(self.calls):
            ev = kernel_timer.record("bwd")
            try:
                check(lib.splat_render_bwd(*head, g0 + 4 * img * b, *tail), "splat_render_bwd")
                if adj is not None:
                    check(lib.splat_upsample_adjoint(*adj), "splat_upsample_adjoint")
                    check(lib.splat_render_fields_split_bwd(*split), "splat_render_fields_split_bwd")
            finally:
                kernel_timer.close("bwd", ev)
            ev = kernel_timer.record("reduce")
            try:
                check(lib.splat_reduce_pairs(*red), "splat_reduce_pairs")
            finally:
                kernel_timer.close("reduce", ev)
        g_mu, g_scale, g_col, g_op, g_th, g_bg = self.grads
        self.grads = self.sums = self.keep = self.dS = self.adj = None
        return g_mu, g_scale, g_col, g_op, g_bg, g_th


class _AlphaRenderCull(torch.autograd.Function):
    """render_triton.py:813-833. Inputs (mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds).
    scale_is_log=True: `scale` is the fp32 raw log-scale, activated inside the binning's decode pass, and its
    gradient is w.r.t. the log-scale (what activate_scale + this Function would give, in one node).

    The output is the [B,C,H,W] view of the [B,H*W,C] composite that render_alpha_full_triton returns (:347), made
    here so that no view nodes follow the Function; the backward reads bg (and the raw log-scales) only, the
    forward's composite buffers (T, asum, fg) are kept on ctx."""

    @staticmethod
    def forward(ctx, mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds=False, scale_is_log=False):
        B, N, C = color.shape
        grad = any(ctx.needs_input_grad[:6])
        plan = _BwdPlan(theta is not None, scale if scale_is_log else None) if grad and N > 0 else None
        out, (T, asum, fg), bins = _forward_cull(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds=odds,
                                                 with_maps=grad, scale_is_log=scale_is_log, plan=plan)
        ctx.meta = (B, N, C, mu.device, theta is not None, H, W, TILE, odds, scale_is_log)
        ctx.tiles = bins
        ctx.fwd = (T, asum, fg)
        ctx.plan = plan
        # the backward reads bg and the raw log-scales through the plan's pointers: keep them alive
        if scale_is_log:
            ctx.save_for_backward(bg, scale)
        else:
            ctx.save_for_backward(bg)
        return out.view(B, H, W, C).permute(0, 3, 1, 2)

    @staticmethod
    def backward(ctx, grad_out):
        B, N, C, dev, has_th, H, W, TILE, odds, scale_is_log = ctx.meta
        plan, ctx.plan = ctx.plan, None
        if plan is not None and plan.grads is not None:
            g_mu, g_scale, g_col, g_op, g_bg, g_th = plan.run(_lib.load(), grad_out, H, W, C)
            return g_mu, g_scale, g_col, g_op, g_bg, g_th, None, None, None, None, None, None
        saved = ctx.saved_tensors
        bg = saved[0]
        lsc = saved[1] if scale_is_log else None
        T, asum, fg = ctx.fwd
        go = grad_out.permute(0, 2, 3, 1).reshape(B, H * W, C)   # a view when the gradient has the image's layout
        g_mu, g_scale, g_col, g_op, g_bg, g_th = _backward_cull_raw(go, bg, lsc, B, N, C, dev, has_th, T, asum, fg,
                                                                    ctx.tiles, odds)
        return g_mu, g_scale, g_col, g_op, g_bg, g_th, None, None, None, None, None, None


class _AlphaRenderCullFields(torch.autograd.Function):
    """render_triton.py:836-861: raw partial-sum fields of one splat group; no bg, no composite."""

    @staticmethod
    def forward(ctx, mu, scale, color, opacity, theta, H, W, TILE, cutoff, max_pairs, odds=False):
        slog, sa, sac, bins = _forward_cull_fields(mu, scale, color, opacity, theta, H, W, TILE=TILE, cutoff=cutoff,
                                                   max_pairs=max_pairs, odds=odds,
                                                   with_maps=any(ctx.needs_input_grad[:5]))
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


class _AlphaRenderLevels(torch.autograd.Function):
    """Fused octave / coarse-fine render (render_triton.py:879-980) with the levels described by `lv`:
    inputs (mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv, scale_is_log)
    -> the [B,C,H,W] view of the [B,H*W,C] composite (made here, so that no view nodes follow the Function).
    scale_is_log as in _AlphaRenderCull."""

    @staticmethod
    def forward(ctx, mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv,
                scale_is_log=False):
        grad = any(ctx.needs_input_grad[:6])
        N = color.shape[1]
        plan = _LevelsBwdPlan(theta is not None, scale if scale_is_log else None) if grad and N > 0 else None
        out, (T, asum, fg), bins = _forward_levels(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff,
                                                   max_pairs, odds, lv, grad, scale_is_log=scale_is_log, plan=plan)
        ctx.plan = plan
        ctx.has_theta = theta is not None
        ctx.odds = odds
        ctx.tiles = bins
        ctx.scale_is_log = scale_is_log
        ctx.fwd = (T, asum, fg)   # internal buffers, kept on ctx like the cull Function's
        ctx.save_for_backward(color, bg, scale if scale_is_log else None)
        B, P, C = out.shape
        return out.view(B, H, W, C).permute(0, 3, 1, 2)

    @staticmethod
    def backward(ctx, grad_out):
        color, bg, log_scale = ctx.saved_tensors
        T, asum, fg = ctx.fwd
        B, C, H, W = grad_out.shape
        go = grad_out.permute(0, 2, 3, 1).reshape(B, H * W, C)   # a view when the gradient has the image's layout
        plan, ctx.plan = ctx.plan, None
        if plan is not None:
            g_mu, g_scale, g_col, g_op, g_bg, g_th = plan.run(_lib.load(), _f32(go))
        else:
            g_mu, g_scale, g_col, g_op, g_bg, g_th = _backward_levels(go, color, bg, ctx.has_theta, T, asum, fg,
                                                                      ctx.tiles, ctx.odds, log_scale)
        return (g_mu, g_scale, g_col, g_op, g_bg, g_th) + (None,) * 8


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
def _scale_arg(log_scale):
    """(scale, scale_is_log) for the binned autograd Functions: fp32 raw log-scales go in as they are and are
    activated in the decode pass (the bits of activate_scale in fp32); other dtypes are activated by torch
    first, in their own dtype, as the reference does."""
    if log_scale.dtype == torch.float32:
        return log_scale, True
    return activate_scale(log_scale), False


MAX_CHANNELS = 4   # colour channels per launch: the kernels are instantiated for C = 1..4


def _channel_chunks(render, color, bg):
    """A render of C > MAX_CHANNELS colour channels (render_triton.py pads C to the next power of two and takes any
    count) as renders of at most MAX_CHANNELS channels each, concatenated along the channel dimension of the image
    (dim 1 of [B,C,H,W], or of [B,C,n] for pixel subsamples). Everything but the colour sums is independent of the
    colour (pair lists, S_log, S_a), each channel's image depends on its own colour and background only, and the
    backward is linear in the upstream gradient, so the chunks' images are the image's channels and autograd's sum of
    the chunks' gradients of the shared parameters is their gradient. render(color_chunk, bg_chunk) renders one
    chunk; `bg` is [B,C] or [1,C]. Each chunk bins the splats again (the pair lists are the same)."""
    C = color.shape[-1]
    return torch.cat([render(color[..., k:k + MAX_CHANNELS], bg[..., k:k + MAX_CHANNELS])
                      for k in range(0, C, MAX_CHANNELS)], dim=1)


def _apply_levels(mu, log_scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv):
    bg = _batch_args(mu, log_scale, color, opacity, bg, theta)
    if color.shape[-1] > MAX_CHANNELS:
        return _channel_chunks(lambda c, b: _apply_levels(mu, log_scale, c, opacity, b, theta, H, W, TILE, cutoff,
                                                          max_pairs, odds, lv), color, bg)
    scale, is_log = _scale_arg(log_scale)
    return _AlphaRenderLevels.apply(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv,
                                    is_log)


def render_alpha_full_triton(mu, log_scale, color, opacity, bg, H, W, theta=None, cull=False, TILE=8, cutoff=3.0,
                             odds=False):
    """render_triton.py:326-347. cull=False: exact (every pixel sums every splat); cull=True: tile-binned
    at `cutoff` sigma. Returns [B,C,H,W]. The name is kept for drop-in compatibility; no Triton is used."""
    B, N, C = color.shape
    bg = _batch_args(mu, log_scale, color, opacity, bg, theta)
    if C > MAX_CHANNELS:
        return _channel_chunks(lambda c, b: render_alpha_full_triton(mu, log_scale, c, opacity, b, H, W, theta=theta,
                                                                     cull=cull, TILE=TILE, cutoff=cutoff, odds=odds),
                               color, bg)
    if cull:
        scale, is_log = _scale_arg(log_scale)
        return _AlphaRenderCull.apply(mu, scale, color, opacity, bg, theta, H, W, TILE, cutoff, odds, is_log)
    else:
        scale = activate_scale(log_scale)
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


def _multires_levels(H, W, N, n_coarse, coarse_factor):
    """render_triton.py:896-913: the coarse group [0, n_coarse) renders on (H // cf, W // cf) with
    cf = min(coarse_factor, max(1, min(H, W) // 8)); without a split every splat renders at (H, W)."""
    if n_coarse is None or n_coarse <= 0 or n_coarse >= N:
        return SplatLevels(0, 0, 0.0, 0, 0, 0)
    cf = min(coarse_factor, max(1, min(H, W) // 8))
    return SplatLevels(2, 0, 0.0, int(n_coarse), max(1, H // cf), max(1, W // cf))


def render_alpha_multires(mu, log_scale, color, opacity, bg, H, W, theta=None, n_coarse=None, coarse_factor=8,
                          cutoff=3.0, TILE=8, max_pairs=48_000_000, odds=False):
    """render_triton.py:879-922: coarse group [0, n_coarse) at H/cf, fine group at native resolution; the
    fields are summed (bilinear upsample of the coarse ones) and composited once. Fused: one binning over
    both canvases and one composite kernel that upsamples the coarse fields in its epilogue."""
    B, N, C = color.shape
    lv = _multires_levels(H, W, N, n_coarse, coarse_factor)
    return _apply_levels(mu, log_scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv)


def _octave_of(scale_px, base_texels=8.0, max_octaves=6):
    """render_triton.py:925-932: o = clamp(ceil(log2(sigma_px / base_texels)), 0, max_octaves)."""
    o = torch.ceil(torch.log2((scale_px / base_texels).clamp_min(1e-6)))
    return o.clamp(0, max_octaves).to(torch.int64)


def _octave_levels(H, W, base_texels, max_octaves):
    if min(H, W) < 8:
        raise ValueError(f"render_alpha_octave: octave 0 renders on (max(8, H), max(8, W)), which needs H, W >= 8 "
                         f"(got {H}x{W})")
    if max_octaves < 0:
        raise ValueError(f"render_alpha_octave: max_octaves={max_octaves} < 0")
    return SplatLevels(1, int(max_octaves), float(base_texels), 0, 0, 0)


def render_alpha_octave(mu, log_scale, color, opacity, bg, H, W, theta=None, cutoff=3.0, TILE=8, base_texels=8.0,
                        max_octaves=6, max_pairs=48_000_000, odds=False):
    """render_triton.py:935-980: each splat renders at the octave H/2^o where its footprint spans a bounded
    number of tiles; octave fields are upsampled to (H, W), summed and composited once. Fused: the routing
    happens in the binning pass, every octave shares one pair list, and the level-0 composite kernel
    upsamples the coarse octaves' fields in its epilogue (octaves whose canvas is clamped to 8x8 share one
    level, which sums the same fields).

    H and W must be at least 8: the reference renders octave 0 on a max(8, H) x max(8, W) canvas and adds it to
    the H x W field (render_triton.py:958-962), a shape error as soon as a splat routes to octave 0 on a
    smaller canvas; here such a canvas is refused up front (RuntimeError) whatever the routing."""
    B, N, C = color.shape
    if H < 8 or W < 8:
        raise RuntimeError(f"render_alpha_octave: H={H} W={W}; the octave render needs H, W >= 8 (its octave 0 "
                           f"renders on a max(8, H) x max(8, W) canvas)")
    lv = _octave_levels(H, W, base_texels, max_octaves)
    return _apply_levels(mu, log_scale, color, opacity, bg, theta, H, W, TILE, cutoff, max_pairs, odds, lv)
