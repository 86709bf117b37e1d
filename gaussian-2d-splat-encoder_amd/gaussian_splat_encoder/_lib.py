"""ctypes binding of libsplat_hip.so (the C-ABI declared in include/splat_render.h).

torch is imported first so that its HIP runtime is the one the library binds to (both carry the soname
libamdhip64.so.7; the dynamic loader reuses the copy torch already loaded). A missing library is an error:
there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os

import torch

from ._build import LIB_PATH

_VP = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_LL = ctypes.c_longlong



class SplatLevels(ctypes.Structure):
    """struct splat_levels: mode 0 single canvas, 1 octave routing, 2 coarse/fine split by index."""
    _fields_ = [("mode", _I), ("max_octaves", _I), ("base_texels", _F), ("n_coarse", _I),
                ("coarse_H", _I), ("coarse_W", _I)]


_LV = ctypes.POINTER(SplatLevels)
_U = ctypes.c_uint

# name -> (restype, argtypes)
_SIGS = {
    "splat_last_error": (ctypes.c_char_p, []),
    "splat_abi_version": (_I, []),
    "splat_decode": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _VP, _VP]),
    "splat_bin_count_workspace_bytes": (_SZ, [_I, _I, _I, _I, _LV]),
    "splat_levels_geometry": (_I, [_I, _I, _I, _LV, _VP, _I]),
    "splat_bin_count": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _F, _LV, _I, _VP, _VP, _VP, _VP, _VP, _SZ,
                             _VP]),
    "splat_bin_pairs_workspace_bytes": (_SZ, [_I, _I, _I, _I, _LV, _LL]),
    "splat_bin": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _F, _LV, _I, _LL, _VP, _VP, _VP, _VP, _VP, _VP, _SZ,
                       _LL, _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "splat_bin_pairs": (_I, [_VP, _VP, _VP, _I, _I, _I, _I, _LV, _LL, _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "splat_bin_finish": (_I, [_VP, _VP, _I, _LL, _LL, _VP]),
    "splat_bin_noalloc": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _F, _LV, _I, _LL, _VP, _VP, _VP, _VP, _VP,
                               _LL, _VP, _VP, _VP, _VP, _VP]),
    "splat_time_next_launch": (_I, [_VP, _VP]),
    "splat_render_fwd": (_I, [_VP, _VP, _VP, _I, _I, _I, _I, _I, _LV, _I, _I, _U, _VP, _VP, _VP, _VP, _VP, _VP,
                              _VP, _VP, _VP]),
    "splat_pair_sums_bytes": (_SZ, [_LL]),
    "splat_render_bwd": (_I, [_VP, _VP, _VP, _VP, _LL, _I, _I, _I, _I, _I, _LV, _I, _I, _U, _VP, _VP, _VP, _VP,
                              _VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "splat_fields_split_workspace_bytes": (_SZ, [_I, _I, _I, _I, _LV, _I, _I, _U, _VP]),
    "splat_render_fields_split": (_I, [_VP, _VP, _VP, _I, _I, _I, _I, _I, _LV, _I, _I, _U, _VP, _VP, _VP, _VP, _VP,
                                       _SZ, _VP]),
    "splat_render_fields_split_bwd": (_I, [_VP, _VP, _VP, _VP, _LL, _I, _I, _I, _I, _I, _LV, _I, _I, _U, _VP, _VP,
                                           _VP, _VP, _VP, _VP]),
    "splat_upsample_adjoint_workspace_bytes": (_SZ, [_I, _I, _I, _I, _LV]),
    "splat_upsample_adjoint": (_I, [_I, _I, _I, _I, _LV, _U, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "splat_reduce_pairs": (_I, [_VP, _VP, _VP, _LL, _I, _I, _VP, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "splat_exact_fwd": (_I, [_VP, _I, _I, _VP, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP]),
    "splat_exact_bwd_workspace_bytes": (_SZ, [_I, _I, _I]),
    "splat_exact_bwd": (_I, [_VP, _I, _I, _VP, _VP, _I, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                             _VP, _SZ, _VP]),
}

EXPORTED = tuple(_SIGS)

FLAG_FIELDS = 1
FLAG_ODDS = 2
FLAG_UPS = 4
FLAG_WIDE = 8
FLAG_LOG_SCALE = 16
FLAG_DEFER = 32
MAX_LEVELS = 12   # kMaxLevels of the library

STATUS_WORKSPACE = 5
STATUS_CAPACITY = 6
STATUS_BUDGET = 7
_STATUS = {1: "invalid argument", 2: "HIP error", 3: "unsupported configuration", 4: "overflow",
           5: "workspace too small", 6: "pair capacity too small", 7: "pair budget exceeded"}

_lib = None


class SplatError(RuntimeError):
    """A non-zero status from the C-ABI."""


def load(path: str = LIB_PATH):
    """Load (once) and return the library with its signatures set."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"HIP extension {path} is not built: run __graft_entry__.build() "
                           f"(or python -m gaussian_splat_encoder._build)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().splat_last_error().decode(errors="replace")
        raise SplatError(f"{what} failed ({_STATUS.get(status, status)}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None stays NULL; an int is taken as a pointer already)."""
    return t if t is None or type(t) is int else t.data_ptr()


def stream_ptr(device=None) -> int:
    """Raw hipStream_t of the current stream of `device` (torch's cheap accessor, no Stream object)."""
    idx = device.index if isinstance(device, torch.device) else device
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
