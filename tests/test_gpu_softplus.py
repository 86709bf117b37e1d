"""The scale activation of the binning's decode pass against torch's, densely, bit for bit.

The render entry points hand fp32 raw log-scales to the binning (SPLAT_FLAG_LOG_SCALE), whose decode pass
evaluates softplus(x) + 1e-4 (params.py:18-28; render_triton.py:948 activates before binning) and whose per-splat
reduction chains the scale gradient through softplus' derivative. The pair lists are bit-exact only if every
activated scale has the bits of torch's F.softplus(x) + 1e-4 on the device, so this sweeps:
* 2^24 evenly spaced float32 log-scales over [-88, 30] (the exp underflow end to past the threshold of 20);
* every float32 in [19.5, 20.5] (the threshold where torch passes x through);
* 2^24 random float32 bit patterns, kept where they lie in [-88, 30] (every exponent, so every scale of x).
Forward: splat_bin_count's records (sy, sx) against F.softplus(x) + 1e-4. Backward: splat_reduce_pairs with the
log-scales given against torch's softplus_backward of the same pass's scale gradient without them.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gaussian_splat_encoder import _lib

pytestmark = pytest.mark.gpu

R_SY = 12   # record slots of the activated scale (sy, sx)


def sweeps():
    lin = torch.linspace(-88.0, 30.0, 1 << 24, dtype=torch.float32)
    lo = np.float32(19.5).view(np.int32)
    hi = np.float32(20.5).view(np.int32)
    thr = torch.from_numpy(np.arange(lo, hi + 1, dtype=np.int32).view(np.float32).copy())
    bits = torch.randint(-(1 << 31), (1 << 31) - 1, (1 << 24,), generator=torch.Generator().manual_seed(5),
                         dtype=torch.int64).to(torch.int32)
    rnd = bits.view(torch.float32)
    rnd = rnd[torch.isfinite(rnd) & (rnd >= -88.0) & (rnd <= 30.0)]
    return {"linspace": lin, "threshold": thr, "bit patterns": rnd}


def decode(x, dev, lib, stream):
    """splat_bin_count on one 8 x 8 tile with the pairs of log-scales x as (sy, sx): the records."""
    N = x.numel() // 2
    g = torch.Generator().manual_seed(N)
    mu = torch.rand(N, 2, generator=g).to(dev)
    theta = (torch.rand(N, generator=g) * 3.0).to(dev)
    op = torch.rand(N, generator=g).to(dev)
    col = torch.rand(N, 3, generator=g).to(dev)
    ls = x.view(N, 2).to(dev)
    rec = torch.empty(N, 16, device=dev)
    rect = torch.empty(N, 4, dtype=torch.int32, device=dev)
    off = torch.empty(N + 1, dtype=torch.int32, device=dev)
    info = torch.empty(2 + _lib.MAX_LEVELS, dtype=torch.int64, device=dev)
    ws = torch.empty(max(1, lib.splat_bin_count_workspace_bytes(N, 8, 8, 8, None)), dtype=torch.uint8, device=dev)
    p = _lib.ptr
    _lib.check(lib.splat_bin_count(p(mu), p(ls), p(theta), p(op), p(col), 3, N, 8, 8, 8, 3.0, None,
                                   _lib.FLAG_LOG_SCALE, p(rec), p(rect), p(off), p(info), p(ws), ws.numel(), stream),
               "splat_bin_count")
    torch.cuda.synchronize()
    assert int(info[0]) == N and int(info[1]) == 0
    return ls, rec


def scale_grads(ls, rec, dev, lib, stream):
    """splat_reduce_pairs over one random pair record per splat, without and with the log-scales."""
    N = ls.shape[0]
    sums = torch.randn(N, 9, generator=torch.Generator().manual_seed(3)).to(dev)
    off = torch.arange(N + 1, dtype=torch.int32, device=dev)
    outs = []
    for lsc in (None, ls):
        g = [torch.empty(N, 2, device=dev), torch.empty(N, 2, device=dev), torch.empty(N, device=dev),
             torch.empty(N, device=dev), torch.empty(N, 3, device=dev)]
        p = _lib.ptr
        _lib.check(lib.splat_reduce_pairs(p(rec), p(off), None, N, N, 3, p(sums), None, 0, p(lsc), *[p(t) for t in g],
                                          None, stream), "splat_reduce_pairs")
        outs.append(g[1])
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("name", ["linspace", "threshold", "bit patterns"])
def test_softplus_bits(dev, name):
    x = sweeps()[name]
    x = x[: x.numel() // 2 * 2]
    lib = _lib.load()
    stream = _lib.stream_ptr(dev)
    print(f"softplus sweep {name}: {x.numel()} values", flush=True)
    ls, rec = decode(x, dev, lib, stream)
    want = F.softplus(ls) + 1e-4
    got = rec[:, R_SY:R_SY + 2].contiguous()
    diff = got.view(torch.int32) != want.view(torch.int32)
    n_bad = int(diff.sum())
    assert n_bad == 0, f"{n_bad} activated scales differ, first at x={ls[diff][:4].tolist()}"
    g_sc, g_ls = scale_grads(ls, rec, dev, lib, stream)
    want_g = torch.ops.aten.softplus_backward(g_sc, ls, 1.0, 20.0)
    diff = g_ls.view(torch.int32) != want_g.view(torch.int32)
    n_bad = int(diff.sum())
    assert n_bad == 0, f"{n_bad} log-scale gradients differ, first at x={ls[diff][:4].tolist()}"
