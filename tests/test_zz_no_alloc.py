"""splat_bin_noalloc, the binning entry point that allocates nothing (its count and pair-phase workspaces live
in the library's own device scratch), called through the C-ABI and checked bit for bit against splat_bin
(the same binning with caller-provided workspaces): the decoded records, rects, offsets, totals, the pair list
and tile starts, and both pair maps. Two calls in a row, the second with a smaller input, so a stale scratch
from the first call cannot go unseen; calls from two threads on two streams at once (the library orders them on
the device); then the limits (a pair capacity beyond the scratch, a count beyond the caller's buffers)."""

import threading

import numpy as np
import pytest
import torch

from _gpu_util import RH, random_scene
from gaussian_splat_encoder import _lib, synth

pytestmark = pytest.mark.gpu


def reference_bins(mu, ls, col, op, th, H, W, lv):
    return RH._bin(mu, ls, col, op, th, H, W, 8, 3.0, lv=lv, scale_is_log=True)


def noalloc_bins(mu, ls, col, op, th, H, W, lv, cap, max_pairs=-1):
    """splat_bin_noalloc with outputs sized for `cap` pairs; returns (status, outputs by name, info_host)."""
    dev = mu.device
    lib = _lib.load()
    N, C = col.shape[1], col.shape[2]
    geom, nt, _ = RH.levels_geometry(H, W, 8, lv)
    L = len(geom)
    i32 = lambda *s: torch.full(s, -7, dtype=torch.int32, device=dev)
    out = {"rec": torch.full((N, 16), float("nan"), device=dev), "rect": i32(N, 4), "off": i32(N + 1),
           "info": torch.full((2 + L,), -7, dtype=torch.int64, device=dev), "gid": i32(max(cap, 1)),
           "starts": i32(nt + 1), "psplat": i32(max(cap, 1)), "pq": i32(max(cap, 1))}
    info_host = torch.zeros(2 + _lib.MAX_LEVELS, dtype=torch.int64, pin_memory=True)
    p = _lib.ptr
    lvr = None if lv is None else _lib.ctypes.byref(lv)
    rc = lib.splat_bin_noalloc(p(mu[0]), p(ls[0]), None if th is None else p(th[0]), p(op[0]), p(col[0]), C, N, H, W, 8,
                               3.0, lvr, _lib.FLAG_LOG_SCALE, max_pairs, p(out["rec"]), p(out["rect"]), p(out["off"]),
                               p(out["info"]), info_host.data_ptr(), cap, p(out["gid"]), p(out["starts"]),
                               p(out["psplat"]), p(out["pq"]), _lib.stream_ptr(dev))
    torch.cuda.current_stream(dev).synchronize()
    return rc, out, info_host.numpy()[:2 + L].copy()


def assert_same(ref, got, info):
    tot = ref.tot_b[0]
    L = ref.n_levels
    assert info[0] == tot and info[1] == 0
    if ref.level_tot_b is not None:
        assert list(info[2:2 + L]) == list(ref.level_tot_b[0])
    assert torch.equal(got["rec"].view(torch.int32), ref.rec_b[0].view(torch.int32)), "decoded records"
    assert torch.equal(got["rect"], ref.rect_b[0]), "rects"
    assert torch.equal(got["off"], ref.off_b[0]), "offsets"
    assert torch.equal(got["starts"], ref.starts_b[0]), "tile starts"
    for k, r in (("gid", ref.gid_b[0]), ("pq", ref.pq_b[0])):
        assert torch.equal(got[k][:tot], r[:tot]), k
    # pair_splat (not requested by the renderer): the splat of every splat-major pair
    off = ref.off_b[0].long()
    want = torch.repeat_interleave(torch.arange(off.numel() - 1, device=off.device), off[1:] - off[:-1])
    assert torch.equal(got["psplat"][:tot].long(), want), "pair_splat"


def test_noalloc_matches_splat_bin_twice(dev):
    # call 1: the benchmark frame (768 x 768, 92,160 splats, 1.84M pairs), single canvas
    s = synth.config("c1").to(dev)
    args = (s.mu, s.log_scale, s.color, s.opacity, s.theta, s.H, s.W)
    ref = reference_bins(*args, None)
    print(f"noalloc call 1: c1 N={s.n} pairs={ref.tot_b[0]}", flush=True)
    rc, got, info = noalloc_bins(*args, None, ref.tot_b[0] + 100)
    _lib.check(rc, "splat_bin_noalloc")
    assert_same(ref, got, info)
    # call 2: a smaller frame with octave levels (ragged canvas, 3,000 splats)
    mu, ls, col, op, _, th = random_scene(3000, 100, 60, seed=77, dev=dev, ls_mean_px=10.0, ls_std=1.2, margin=0.2)
    lv = _lib.SplatLevels(1, 6, 8.0, 0, 0, 0)
    args = (mu, ls, col, op, th, 100, 60)
    ref = reference_bins(*args, lv)
    print(f"noalloc call 2: 100x60 octaves N=3000 pairs={ref.tot_b[0]}", flush=True)
    rc, got, info = noalloc_bins(*args, lv, ref.tot_b[0])
    _lib.check(rc, "splat_bin_noalloc")
    assert_same(ref, got, info)
    assert sum(1 for n in info[2:] if n) >= 2


def test_noalloc_limits(dev):
    s = synth.config("c0").to(dev)
    args = (s.mu, s.log_scale, s.color, s.opacity, s.theta, s.H, s.W)
    ref = reference_bins(*args, None)
    tot = ref.tot_b[0]
    # a pair capacity whose workspace exceeds the scratch: refused before any launch
    rc, _, _ = noalloc_bins(*args, None, 60_000_000)
    assert rc == _lib.STATUS_WORKSPACE and b"scratch" in _lib.load().splat_last_error()
    # a count above the caller's buffers: status 6 with the count in info_host, the pair list left empty
    rc, got, info = noalloc_bins(*args, None, tot - 1)
    assert rc == _lib.STATUS_CAPACITY and info[0] == tot
    # and the budget, per level
    rc, _, info = noalloc_bins(*args, None, tot, max_pairs=tot - 1)
    assert rc == _lib.STATUS_BUDGET and info[0] == tot
    rc, got, info = noalloc_bins(*args, None, tot, max_pairs=tot)
    _lib.check(rc, "splat_bin_noalloc")
    assert_same(ref, got, info)


def test_noalloc_two_threads_two_streams(dev):
    """Two threads, each on a stream of its own, bin different scenes through the one scratch at the same time, six
    times each: every call bit for bit equal to splat_bin's result (the library serialises the calls' kernels on
    the device, so neither sees the other's workspace)."""
    s = synth.config("c1").to(dev)
    a = (s.mu, s.log_scale, s.color, s.opacity, s.theta, s.H, s.W)
    mu, ls, col, op, _, th = random_scene(20000, 300, 200, seed=78, dev=dev, ls_mean_px=6.0, ls_std=1.0, margin=0.1)
    b = (mu, ls, col, op, th, 300, 200)
    refs = [(a, None, reference_bins(*a, None)), (b, _lib.SplatLevels(1, 6, 8.0, 0, 0, 0), None)]
    refs[1] = (b, refs[1][1], reference_bins(*b, refs[1][1]))
    torch.cuda.synchronize()
    errors = []

    def worker(k):
        args, lv, ref = refs[k]
        try:
            with torch.cuda.stream(torch.cuda.Stream(dev)):
                for it in range(6):
                    rc, got, info = noalloc_bins(*args, lv, ref.tot_b[0] + 10)
                    _lib.check(rc, "splat_bin_noalloc")
                    assert_same(ref, got, info)
        except Exception as e:   # reported by the main thread
            errors.append(f"thread {k}: {e!r}")

    print("noalloc: two threads on two streams", flush=True)
    ts = [threading.Thread(target=worker, args=(k,)) for k in (0, 1)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
