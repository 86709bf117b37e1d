"""Benchmark of the tile-binned splat renderer on one MI355X.

Workload (BASELINE.json configs[1]/[2]): one 768x768 RGB fp32 frame from 92,160 seeded synthetic splats
(10 per 8x8 cell of a 96x96 grid), upstream gradient ~ N(0, 1). A step is one forward + backward render
through render_alpha_full_triton(cull=True): binning (decode with the scale activation, count, scan, pair
expansion, the sort on the tile id, tile starts), per-tile compositing, and the backward to every splat
parameter. Inputs are resident in HBM before the timed region. `value` is frames/s x 0.589824 Mpix of the
fwd+bwd step.

Also reported: forward-only, the render_alpha_octave entry point, the 2048x2048 stress set
(configs[4]: fwd and fwd+bwd, single-res and octave), the encoder end-to-end frame (configs[3]: per-stage
ms), per-stage event times (back-to-back launches), the device time of the step's kernel chain, per-step
median / p10 / p90, the roofline of the dominant kernel from HIP events that its launches record at their own
start and end in fwd+bwd steps, and the reference's CPU renderer (render.py math) on the host cores: a bounded
band of the same frame, and configs[0] (64x64, 1,024 splats, seed 0: 3 warm-ups and 20 timed runs, median, p10
and p90).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gaussian-2d-splat-encoder_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from gaussian_splat_encoder import render_hip as RH  # noqa: E402
from gaussian_splat_encoder import synth  # noqa: E402

# AMD's published MI355X peaks: fp32 vector 157.3 TFLOP/s, HBM3E 8.0 TB/s.
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
# Algorithmic flops per pixel-pair evaluation, counting each operation of the reference's expressions once
# (render_triton.py:476-499 forward, :668-710 backward incl. the 9 pixel-reduction adds), per-splat terms
# hoisted.
FLOPS_FWD = {False: 27, True: 28}
FLOPS_BWD = {False: 71, True: 74}


def algorithmic_bytes_fwd(N, tot, P):
    """Composite forward: splat params 36 B/splat, pair list 8 B/pair (id + gathered record index), out+T+
    asum+fg 32 B/pixel."""
    return 36 * N + 8 * tot + 32 * P


def algorithmic_bytes_bwd(N, tot, P):
    """Backward: params in + grads out 72 B/splat, pair ids 4 B/pair, T+asum+fg+gout 32 B/pixel."""
    return 72 * N + 4 * tot + 32 * P


def ppe_levels(bins, TILE=8):
    """Pixel-pair evaluations of a binning over every level (octave / coarse-fine renders): per level, the sum over
    its tiles of pairs x the tile's pixels on that level's canvas."""
    if bins.geom is None:
        return ppe_of(bins, bins.H, bins.W, TILE)
    st = bins.starts_b[0].long()
    cnt = (st[1:] - st[:-1]).double()
    total = 0.0
    for l, (Hl, Wl, ntx, tb, _) in enumerate(bins.geom):
        te = bins.geom[l + 1][3] if l + 1 < len(bins.geom) else bins.nt
        t = torch.arange(te - tb, device=cnt.device)
        ty, tx = t // ntx, t % ntx
        ph = torch.clamp(Hl - ty * TILE, max=TILE).double()
        pw = torch.clamp(Wl - tx * TILE, max=TILE).double()
        total += float((cnt[tb:te] * ph * pw).sum().item())
    return total


def stage_rate(ppe, flops_per_ppe, ms):
    """A render stage's algorithmic rate: flops of its pixel-pair evaluations over the stage's whole time (binning
    and every launch included), and that as a fraction of the fp32 vector peak."""
    tf = flops_per_ppe * ppe / (ms * 1e-3) / 1e12
    return {"ppe": int(ppe), "alg_tflops": round(tf, 2), "frac_of_peak": round(tf / PEAK_FP32_TFLOPS, 4)}


def ppe_of(bins, H, W, TILE=8):
    """Pixel-pair evaluations: sum over tiles of pairs x in-canvas pixels of the tile."""
    st = bins.starts_b[0].long()
    cnt = (st[1:] - st[:-1]).double()
    ntx = bins.ntx
    t = torch.arange(cnt.numel(), device=cnt.device)
    ty, tx = t // ntx, t % ntx
    ph = torch.clamp(H - ty * TILE, max=TILE).double()
    pw = torch.clamp(W - tx * TILE, max=TILE).double()
    return float((cnt * ph * pw).sum().item())


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary
    (profiles/<kernel>_c2_traffic.md: a line `traffic_bytes_per_launch: <int>`), else None."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_c2_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.strip().startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def copy_calibration(mib):
    """A plain elementwise copy of `mib` MiB (reads and writes mib MiB), five launches: the known-size
    kernel that scales FETCH_SIZE / WRITE_SIZE."""
    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    for _ in range(5):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_mib": mib, "kernel": "vectorized_elementwise_kernel (mul)",
                      "read_bytes": n * 4, "write_bytes": n * 4}), flush=True)


def time_loop(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


def kernel_times(leaves, H, W, odds, reps):
    """Average device time (ms) of each stage of the fwd+bwd step, from HIP events on the stream the kernels
    run on. The forward tile kernel, the backward tile kernel and the per-splat reduction are each launched
    `reps` times back to back between two events (same inputs, outputs overwritten), so the GPU never waits
    on the host inside the bracket; the binning (which reads its pair count back to the host once per call)
    is bracketed call by call. Also returns the binning of the frame (pair count, pixel-pairs)."""
    dev = leaves[0].device
    mu, ls, col, op, bg, th = [t.detach() for t in leaves]
    sc = torch.nn.functional.softplus(ls) + 1e-4
    out, (T, asum, fg), bins = RH._forward_cull(mu, sc, col, op, bg, th, H, W, 8, 3.0, odds=odds)
    C = col.shape[-1]
    gout = torch.randn(out.shape, device=dev, generator=torch.Generator(device=dev).manual_seed(1))
    lib, stream = RH._lib.load(), RH._lib.stream_ptr(dev)
    flags = RH.FLAG_ODDS if odds else 0
    bgf = bg.contiguous()
    comp = (bgf[0], out[0], T[0], asum[0], fg[0])
    sums, bg_part = RH._bwd_buffers(lib, bins, 0, C, True, dev)
    up = (bgf[0], T[0], asum[0], fg[0], gout[0], None, None, None)
    grads = RH._grads_out(1, mu.shape[1], C, dev, th is not None)
    g_bg = torch.empty(1, C, device=dev)
    fwd_flags = flags | RH._wide(8, bins.nt, bins.tot_b[0])

    def span(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    ms = {
        "fwd": span(lambda: RH._render_fwd(lib, bins, 0, C, fwd_flags, (0, 1), 1, comp, (None,) * 3, stream)),
        "bwd": span(lambda: RH._render_bwd(lib, bins, 0, C, flags, (0, 1), 1, up, sums, bg_part, stream)),
        "reduce": span(lambda: RH._reduce(lib, bins, 0, C, sums, bg_part, grads, g_bg[0], stream)),
    }
    # the binning's kernels alone, as a render queues them: splat_bin with pair buffers for the known pair count
    # (the count phase, then the pair phase queued before the count is read) and a deferred read, so the calls
    # queue back to back with no host read between them; each call gets its own pinned totals, read afterwards
    lsf = ls.contiguous()
    N, tot = mu.shape[1], bins.tot_b[0]
    blk, pb = bins.blocks[0], bins.pairs[0]
    thp = None if th is None else th.data_ptr()
    infos = [torch.zeros(2 + RH._lib.MAX_LEVELS, dtype=torch.int64, pin_memory=True) for _ in range(reps + 3)]
    queued = []

    def bin_kernels():
        info = infos[len(queued)]
        RH._lib.check(lib.splat_bin(mu.data_ptr(), lsf.data_ptr(), thp, op.data_ptr(), col.data_ptr(), C, N, H, W, 8,
                                    3.0, None, RH.FLAG_LOG_SCALE | RH._lib.FLAG_DEFER, -1, blk.ptr(0), blk.ptr(1),
                                    blk.ptr(2), blk.ptr(3), info.data_ptr(), blk.ptr(4), blk.nbytes(4), tot, pb.ptr(0),
                                    pb.ptr(1), None, pb.ptr(2) if bins.with_maps else None, pb.ptr(3), pb.nbytes(3),
                                    stream), "splat_bin")
        queued.append(info)

    ms["bin_kernels"] = span(bin_kernels)
    for info in queued:
        RH._lib.check(lib.splat_bin_finish(info.data_ptr(), blk.ptr(3), 1, -1, tot, stream), "splat_bin_finish")
        assert int(info[0]) == tot
    RH.kernel_timer.enable(True)
    for _ in range(reps):
        RH._bin(mu, lsf, col, op, th, H, W, 8, 3.0, scale_is_log=True)
    ev = RH.kernel_timer.elapsed_ms()
    RH.kernel_timer.enable(False)
    ms["bin_call"] = sum(ev["bin"]) / len(ev["bin"])
    return ms, bins


def step_times(fn, steps, warmup):
    """Per-step wall times (ms) of `steps` steps, each ended by a device synchronisation: median, p10, p90."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    out = []
    for _ in range(steps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        out.append((time.perf_counter() - t0) * 1e3)
    return percentiles(out)


def percentiles(v):
    """(median, p10, p90) of a list of times."""
    a = np.asarray(v, np.float64)
    return tuple(float(x) for x in np.percentile(a, [50, 10, 90]))


def cpu_share():
    """(CPU model, cores in this process's affinity mask, threads used): the threads are the affinity mask's
    cores, capped by OMP_NUM_THREADS where the host sets it (the GPU boxes give a process a 16-core share and
    say so there)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    aff = len(os.sched_getaffinity(0))
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", aff))
    except ValueError:
        share = aff
    return model, aff, max(1, min(aff, share))


def cpu_runs(fn, warmup, runs):
    for _ in range(warmup):
        fn()
    out = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        out.append(time.perf_counter() - t0)
    return out


def cpu_baseline(s_c1, band_rows=(368, 372), band_runs=10):
    """The reference's CPU renderer (render.py:34-110 math: exact, every pixel x every splat, fp32 torch with the
    falloff materialised in pixel chunks), restated in oracle/render_ref.render_alpha_full_f32, forward only, on
    the host cores of this box:
    * the headline workload's frame (768 x 768, 92,160 splats): a band of rows rendered 1 + band_runs times,
      median scaled to a frame (`value`);
    * configs[0], the CPU-runnable case (64 x 64, 1,024 splats, seed 0, black background): 3 warm-ups and 20
      timed runs (`c0`).
    Times are perf_counter medians with p10 / p90."""
    sys.path.insert(0, ROOT)
    from oracle import render_ref
    model, aff, n = cpu_share()
    torch.set_num_threads(n)
    c0 = synth.config("c0")
    P0 = c0.H * c0.W

    def run_c0():
        render_ref.render_alpha_full_f32(c0.mu, c0.log_scale, c0.color, c0.opacity, c0.bg, c0.H, c0.W,
                                         theta=c0.theta, chunk_pixels=4096)

    t0s = percentiles(cpu_runs(run_c0, 3, 20))
    s = s_c1
    rows = band_rows[1] - band_rows[0]

    def run_band():
        render_ref.render_alpha_full_f32(s.mu, s.log_scale, s.color, s.opacity, s.bg, s.H, s.W, theta=s.theta,
                                         chunk_pixels=256, rows=band_rows)

    tb = percentiles(cpu_runs(run_band, 1, band_runs))
    scale = s.H / rows
    frame_s = tb[0] * scale
    ppe_band = rows * s.W * s.n
    return {"value": round(s.H * s.W / 1e6 / frame_s, 6), "unit": "Mpix/s", "cores": n, "kind": "port",
            "ms_per_frame": round(frame_s * 1e3, 1),
            "ms_per_frame_p10_p90": [round(tb[1] * scale * 1e3, 1), round(tb[2] * scale * 1e3, 1)],
            "ppe_per_s": round(ppe_band / tb[0], 1),
            "cpu_model": model, "affinity_cores": aff, "threads": n,
            "sample": f"render.py exact fp32 forward (oracle/render_ref.render_alpha_full_f32, torch CPU, {n} threads "
                      f"of {aff} in the affinity mask, {model}) over rows {band_rows[0]}-{band_rows[1] - 1} of the "
                      f"768x768 / 92,160-splat frame ({ppe_band / 1e9:.3f} G pixel-pairs per run, 1 warm-up + "
                      f"{band_runs} runs, median scaled to a frame); forward only",
            "c0": {"workload": "configs[0]: 64x64 RGB, 1,024 splats, seed 0, black background, forward only",
                   "ms_per_frame": round(t0s[0] * 1e3, 3), "ms_p10": round(t0s[1] * 1e3, 3),
                   "ms_p90": round(t0s[2] * 1e3, 3), "mpix_s": round(P0 / 1e6 / t0s[0], 4),
                   "ppe_per_s": round(P0 * c0.n / t0s[0], 1), "runs": "3 warm-ups + 20 timed"}}


def stress_c4(steps, warmup, odds):
    """2048x2048, 655,360 splats with a 2 % heavy tail; fwd and fwd+bwd, single-res cull and the
    octave entry point. Reported next to the headline, not as `value`."""
    s = synth.config("c4").to("cuda")
    H, W = s.H, s.W
    gout = s.grad_out.permute(0, 2, 3, 1).contiguous().permute(0, 3, 1, 2)
    leaves = [t.detach().clone().requires_grad_(True) for t in (s.mu, s.log_scale, s.color, s.opacity, s.bg,
                                                                  s.theta)]

    def run(octave, bwd):
        def fn():
            for t in leaves:
                t.grad = None
            with torch.set_grad_enabled(bwd):
                if octave:
                    out = RH.render_alpha_octave(*leaves[:5], H, W, theta=leaves[5], odds=odds)
                else:
                    out = RH.render_alpha_full_triton(*leaves[:5], H, W, theta=leaves[5], cull=True, odds=odds)
                if bwd:
                    out.backward(gout)
        return fn

    res = {"workload": "2048x2048 RGB, 655,360 splats (2 % heavy tail at ~40 px); configs[4]"}
    for name, octave, bwd in (("fwd", False, False), ("fwd_bwd", False, True), ("octave_fwd", True, False),
                              ("octave_fwd_bwd", True, True)):
        ms, _ = time_loop(run(octave, bwd), steps, warmup)
        res[name + "_ms"] = round(ms, 4)
        res[name + "_mpix_s"] = round(H * W / 1e6 / (ms * 1e-3), 2)
    with torch.no_grad():
        sc = torch.nn.functional.softplus(s.log_scale) + 1e-4
        bins = RH._bin(s.mu, sc, s.color, s.opacity, s.theta, H, W, 8, 3.0, with_maps=False)
        obins = RH._bin(s.mu, sc, s.color, s.opacity, s.theta, H, W, 8, 3.0, with_maps=False,
                        lv=RH._octave_levels(H, W, 8.0, 6))
    res["pairs"] = bins.tot_b[0]
    ppe, oppe = ppe_of(bins, H, W), ppe_levels(obins)
    ff, fb = FLOPS_FWD[odds], FLOPS_FWD[odds] + FLOPS_BWD[odds]
    res["stage_roofline"] = {"fwd": stage_rate(ppe, ff, res["fwd_ms"]), "fwd_bwd": stage_rate(ppe, fb, res["fwd_bwd_ms"]),
                             "octave_fwd": stage_rate(oppe, ff, res["octave_fwd_ms"]),
                             "octave_fwd_bwd": stage_rate(oppe, fb, res["octave_fwd_bwd_ms"])}
    del bins, obins, leaves, s
    torch.cuda.empty_cache()
    return res


def e2e_c3(steps, warmup):
    """the released checkpoint's encoder architecture with seeded random-init weights (the
    checkpoint file is not shipped) on a seeded procedural 768x768 card, forward in inference mode as
    examples/encode_and_render.py runs it: backbone, coarse 384^2 odds octave render, fine decoder + head, then
    the full 768^2 odds octave render of all 92,160 splats. Per-stage ms are medians of HIP-event spans."""
    from gaussian_splat_encoder.efficient_encoder import GOLDEN_D256, EfficientGaussianEncoder
    torch.manual_seed(0)
    enc = EfficientGaussianEncoder(**GOLDEN_D256).to("cuda").eval()
    x = synth.procedural_image(768, 768).to("cuda")
    marks = []

    def mark(name):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        marks.append((name, ev))

    enc.stage_marks = mark
    spans = {}
    with torch.inference_mode():
        for it in range(warmup + steps):
            marks.clear()
            mark("start")
            out = enc(x)
            RH.render_alpha_octave(out["mu"], out["log_scale"], out["color"], out["opacity"], out["bg"], 768, 768,
                                   theta=out["theta"], odds=enc.odds)
            mark("full_render")
            torch.cuda.synchronize()
            if it >= warmup:
                for (_, a), (name, b) in zip(marks[:-1], marks[1:]):
                    spans.setdefault(name, []).append(a.elapsed_time(b))
                spans.setdefault("total", []).append(marks[0][1].elapsed_time(marks[-1][1]))
    med = lambda v: sorted(v)[len(v) // 2]
    res = {"workload": "768x768 procedural card -> random-init 833,107-parameter adaptive encoder (d=256) -> "
                       "odds octave renders (384^2 coarse, 768^2 full); configs[3]",
           "splats": int(out["mu"].shape[1]), "stages_ms": {k: round(med(v), 4) for k, v in spans.items()}}
    # the two renders' pixel-pair evaluations: one more frame with the renders' arguments captured
    from gaussian_splat_encoder import efficient_encoder as EE
    calls = []
    orig = EE.render_alpha_octave

    def capture(mu, log_scale, color, opacity, bg, H, W, theta=None, **kw):
        calls.append((mu, log_scale, color, opacity, H, W, theta))
        return orig(mu, log_scale, color, opacity, bg, H, W, theta, **kw)

    EE.render_alpha_octave = capture
    try:
        with torch.inference_mode():
            out = enc(x)
            capture(out["mu"], out["log_scale"], out["color"], out["opacity"], out["bg"], 768, 768, out["theta"],
                    odds=enc.odds)
    finally:
        EE.render_alpha_octave = orig
    rates = {}
    with torch.inference_mode():
        for name, (mu, ls, col, op, H, W, th) in zip(("coarse_render", "full_render"), calls[-2:]):
            sc = torch.nn.functional.softplus(ls.float()) + 1e-4
            bins = RH._bin(mu.float(), sc, col.float(), op.float(), None if th is None else th.float(), H, W, 8, 3.0,
                           with_maps=False, lv=RH._octave_levels(H, W, 8.0, 6))
            rates[name] = stage_rate(ppe_levels(bins), FLOPS_FWD[bool(enc.odds)], res["stages_ms"][name])
    res["stage_roofline"] = rates
    del enc, out, x
    torch.cuda.empty_cache()
    return res


def pair_classes(name, TILE=8, cutoff=3.0):
    """How the backward's per-tile kernel (k_bwd_cull) classes the pairs of a configuration's single-res render, and
    the passes its lanes run: the kernel's tests restated in float64 numpy on the device's own pair lists.
    negligible: falloff below 2^-30 of the splat's falloff at the 3 x 3 pixel centres around the one nearest its
    centre (an upper bound of m over them), at every pixel centre of the tile (a zero record); near-opaque:
    op * falloff may exceed 0.99 in the tile (one careful pass per pair, lane = pixel); direct: whitened half-span
    over the tile above 8, or above 4 for a splat whose scales differ by more than a factor of 16 (the direct form);
    moment: the rest.
    Passes: per tile, the moment pairs and the direct pairs each run in passes of up to 64 (lane = pair); a last
    pass of r < 64 pairs gives each pair Lp lanes (the largest power of two with r Lp <= 64)."""
    s = synth.config(name)
    dev = torch.device("cuda:0")
    mu, ls = s.mu.to(dev), s.log_scale.to(dev)
    sc = torch.nn.functional.softplus(ls) + 1e-4
    gid_b, st_b, ntx, nt = RH._build_tiles(mu, sc, s.H, s.W, TILE, cutoff)
    gid = gid_b[0].cpu().numpy().astype(np.int64)
    st = st_b[0].cpu().numpy().astype(np.int64)
    H, W = s.H, s.W
    m64 = mu[0].cpu().double().numpy()
    s64 = sc[0].cpu().double().numpy()
    th = s.theta[0].double().numpy()
    op = s.opacity[0].double().numpy()
    tot = int(st[-1])
    tile = np.repeat(np.arange(nt), np.diff(st))
    g = gid[:tot]
    ty, tx = tile // ntx, tile % ntx
    c32 = lambda i, n: ((i.astype(np.float32) + np.float32(0.5)) / np.float32(n)).astype(np.float64)
    py0, py1 = c32(ty * TILE, H), c32(ty * TILE + TILE - 1, H)
    px0, px1 = c32(tx * TILE, W), c32(tx * TILE + TILE - 1, W)
    k = np.sqrt(0.5 / np.log(2.0))
    cs, sn = np.cos(th)[g], np.sin(th)[g]
    sy, sx = s64[g, 0], s64[g, 1]
    A, B, Cc, D = k * cs / sy, k * sn / sy, -k * sn / sx, k * cs / sx
    gy, gx = m64[g, 0], m64[g, 1]
    cy, cx = 0.5 * (py1 - py0), 0.5 * (px1 - px0)
    uc = A * (py0 + cy - gy) + B * (px0 + cx - gx)   # u, v at the middle of the tile's pixel centres
    vc = Cc * (py0 + cy - gy) + D * (px0 + cx - gx)
    su, sv = np.abs(A) * cy + np.abs(B) * cx, np.abs(Cc) * cy + np.abs(D) * cx   # their half-spans over the box
    du, dv = np.maximum(np.abs(uc) - su, 0), np.maximum(np.abs(vc) - sv, 0)
    box_m = du * du + dv * dv
    ny = (np.clip(np.floor(gy * H), 0, H - 1) + 0.5) / H - gy
    nx = (np.clip(np.floor(gx * W), 0, W - 1) + 0.5) / W - gx
    un = np.abs(A * ny + B * nx) + np.abs(A) / H + np.abs(B) / W   # |u|, |v| at the nearest centre + one pixel step
    vn = np.abs(Cc * ny + D * nx) + np.abs(Cc) / H + np.abs(D) / W
    negl = box_m > 30.0 + (un * un + vn * vn)
    dy = np.maximum(np.maximum(py0 - gy, gy - py1), 0)
    dx = np.maximum(np.maximum(px0 - gx, gx - px1), 0)
    lop = np.log2(np.maximum(op[g], 1e-45))
    near = ~negl & (op[g] > 0.99) & ((dy * dy + dx * dx) * k * k <
                                     np.maximum(sy, sx) ** 2 * (lop - np.log2(0.99) + 1e-3))
    span = np.maximum(su, sv)
    elong = np.maximum(sy, sx) > 16.0 * np.minimum(sy, sx)
    direct = ~negl & ~near & ((span > 8.0) | (elong & (span > 4.0)))
    moment = ~negl & ~near & ~direct
    out = {"pairs": tot, "share": {c: round(float(m.mean()), 5) for c, m in
                                   (("negligible", negl), ("near_opaque", near), ("direct", direct), ("moment", moment))}}
    # passes per tile (the kernel's queues: whole passes of 64, then the rest)
    lane_pairs = 0
    pass_time = 0.0
    for m in (moment, direct):
        n = np.bincount(tile[m], minlength=nt)
        full, r = n // 64, n % 64
        lp = np.ones_like(r)
        for _ in range(6):
            lp = np.where((r * lp * 2 <= 64) & (lp * 2 <= TILE * TILE), lp * 2, lp)
        pass_time += float(full.sum() + np.where(r > 0, 1.0 / np.where(r > 0, lp, 1), 0).sum())
        lane_pairs += int(n.sum())
    out["row_loop_passes"] = round(pass_time, 1)
    out["lane_use_in_passes"] = round(lane_pairs / max(64 * pass_time, 1), 4)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--odds", action="store_true", help="odds compositing instead of alpha")
    ap.add_argument("--no-c4", action="store_true", help="skip the 2048x2048 stress configuration")
    ap.add_argument("--no-c3", action="store_true", help="skip the encoder end-to-end configuration")
    ap.add_argument("--only", choices=("c3", "c4"), default=None,
                    help="run only the encoder end-to-end frame (c3) or the 2048x2048 stress set (c4) and print its "
                         "JSON object (for profiling one configuration)")
    ap.add_argument("--pair-classes", action="store_true",
                    help="only print how the backward classes the pairs of C2 and C4 (shares, passes) and exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a MIB-MiB copy kernel (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              f"the multi-GPU sharding of this path is a design only, not built", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.pair_classes:
        print(json.dumps({"pair_classes": {c: pair_classes(c) for c in ("c2", "c4")}}), flush=True)
        return
    if args.only == "c3":
        print(json.dumps({"c3": e2e_c3(max(10, args.steps // 2), max(3, args.warmup // 2))}), flush=True)
        return
    if args.only == "c4":
        print(json.dumps({"c4": stress_c4(max(5, args.steps // 5), max(2, args.warmup // 5), args.odds)}), flush=True)
        return
    dev = torch.device("cuda:0")
    s_cpu = synth.config("c2")
    s = s_cpu.to(dev)
    H, W, N = s.H, s.W, s.n
    P = H * W
    odds = args.odds
    # dL/dimage stored in the image's own memory layout ([B,H,W,C] behind the [B,C,H,W] view)
    gout = s.grad_out.permute(0, 2, 3, 1).contiguous().permute(0, 3, 1, 2)
    leaves = [t.detach().clone().requires_grad_(True) for t in (s.mu, s.log_scale, s.color, s.opacity, s.bg,
                                                                  s.theta)]

    def fwd():
        with torch.no_grad():
            return RH.render_alpha_full_triton(*leaves[:5], H, W, theta=leaves[5], cull=True, odds=odds)

    def fwd_bwd():
        for t in leaves:
            t.grad = None
        out = RH.render_alpha_full_triton(*leaves[:5], H, W, theta=leaves[5], cull=True, odds=odds)
        out.backward(gout)

    def oct_fwd():
        with torch.no_grad():
            return RH.render_alpha_octave(*leaves[:5], H, W, theta=leaves[5], odds=odds)

    def oct_fwd_bwd():
        for t in leaves:
            t.grad = None
        RH.render_alpha_octave(*leaves[:5], H, W, theta=leaves[5], odds=odds).backward(gout)

    # the headline: fwd + bwd, then the other measurements
    ms, wall_ms = time_loop(fwd_bwd, args.steps, args.warmup)
    # the roofline's launch durations: the forward and backward tile kernels record HIP events (reused from a
    # pool) at their own start and end (hipExtLaunchKernel), over K more steps of the same loop (kept out of the
    # timed steps: on a host-bound box the timer's host time would lower `value`)
    RH.kernel_timer.enable(True, names=("fwd", "bwd"))
    time_loop(fwd_bwd, args.steps, 2)                     # creates the events
    RH.kernel_timer.enable(True, names=("fwd", "bwd"))    # and returns them to the pool for the measured steps
    time_loop(fwd_bwd, args.steps, 0)
    in_step = {k: sum(v[-args.steps:]) / len(v[-args.steps:]) for k, v in RH.kernel_timer.elapsed_ms().items()}
    RH.kernel_timer.enable(False)
    # per-step statistics of the same steps (each step ended by a synchronisation)
    st_fb = step_times(fwd_bwd, args.steps, 2)
    st_f = step_times(fwd, args.steps, args.warmup)
    ms_fwd, _ = time_loop(fwd, args.steps, args.warmup)
    ms_oct_fwd, _ = time_loop(oct_fwd, args.steps, args.warmup)
    ms_oct, _ = time_loop(oct_fwd_bwd, args.steps, args.warmup)

    # stage device times: HIP events around K back-to-back launches of each stage on the stream it runs on
    avg, bins = kernel_times(leaves, H, W, odds, args.steps)
    tot = bins.tot_b[0]
    ppe = ppe_of(bins, H, W)
    fl_f, fl_b = FLOPS_FWD[odds] * ppe, FLOPS_BWD[odds] * ppe
    kern = {
        "fwd": {"ms": in_step["fwd"], "tflops": fl_f / (in_step["fwd"] * 1e-3) / 1e12,
                "gbs": algorithmic_bytes_fwd(N, tot, P) / (in_step["fwd"] * 1e-3) / 1e9},
        "bwd": {"ms": in_step["bwd"], "tflops": fl_b / (in_step["bwd"] * 1e-3) / 1e12,
                "gbs": algorithmic_bytes_bwd(N, tot, P) / (in_step["bwd"] * 1e-3) / 1e9},
    }
    chain = avg["bin_kernels"] + in_step["fwd"] + in_step["bwd"] + avg["reduce"]
    dom = "bwd" if in_step["bwd"] >= in_step["fwd"] else "fwd"
    dk = kern[dom]
    traffic = measured_traffic(f"k_{dom}_cull")
    mpix = P / 1e6
    line = {
        "metric": "render ms/frame + Mpix/s at 768x768, 92,160 splats (fwd, fwd+bwd); % roofline",
        "value": round(mpix / (ms * 1e-3), 2),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splat set of BASELINE configs[2]; CPU torch.Generator, seed 0)",
        "config": {"workload": "768x768 RGB, 92,160 splats, fwd+bwd, render_alpha_full_triton(cull=True, TILE=8, "
                               f"cutoff=3, odds={odds}); configs[2]",
                   "H": H, "W": W, "splats": N, "pairs": tot, "pixel_pairs": int(ppe)},
        "roofline": {"bound": "valu", "kernel": f"k_{dom}_cull",
                     "achieved": round(dk["tflops"], 3), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(dk["tflops"] / PEAK_FP32_TFLOPS, 4), "traffic": traffic,
                     "flops_per_launch": fl_b if dom == "bwd" else fl_f, "avg_launch_ms": round(dk["ms"], 4),
                     "hbm_achieved_gbs": round(dk["gbs"], 1),
                     "hbm_frac": round(dk["gbs"] / PEAK_HBM_GBS, 4)},
        "kernels": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in kern.items()},
        "stages_ms": {k: round(v, 4) for k, v in avg.items()},
        "fwd_ms": round(ms_fwd, 4),
        "fwd_mpix_s": round(mpix / (ms_fwd * 1e-3), 2),
        "octave_fwd_ms": round(ms_oct_fwd, 4),
        "octave_fwd_bwd_ms": round(ms_oct, 4),
        "wall_ms_per_step": round(wall_ms, 4),
        "step_ms_median_p10_p90": [round(x, 4) for x in st_fb],
        "fwd_step_ms_median_p10_p90": [round(x, 4) for x in st_f],
        # device time of the step's kernels alone: the binning's kernels back to back, the two tile kernels as
        # they ran inside the fwd+bwd steps, the reduction back to back
        "gpu_chain_ms": round(chain, 4),
        "gpu_chain_mpix_s": round(mpix / (chain * 1e-3), 2),
    }
    if not args.no_c4:
        line["c4"] = stress_c4(max(5, args.steps // 5), max(2, args.warmup // 5), odds)
    if not args.no_c3:
        line["c3"] = e2e_c3(max(10, args.steps // 2), max(3, args.warmup // 2))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(s_cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
