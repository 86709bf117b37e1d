"""Encoder checkpoints: the torch zip archive {step, model, cfg} with `cfg['encoder']` holding the
EfficientGaussianEncoder constructor arguments (the format examples/encode_and_render.py:19-28 of the
reference reads). Loaded with torch.load(weights_only=True): tensors, dicts and plain values only, nothing in
the file is executed."""

from __future__ import annotations

import inspect

import torch

from .efficient_encoder import EfficientGaussianEncoder

# keys of cfg['encoder'] that describe training data, not the network
_IGNORED = {"image_size"}


def encoder_kwargs(cfg_encoder: dict) -> dict:
    """Constructor arguments from a checkpoint's cfg['encoder']; unknown architecture fields raise
    ValueError (a checkpoint from a newer architecture must not load silently)."""
    accepted = set(inspect.signature(EfficientGaussianEncoder.__init__).parameters) - {"self"}
    unknown = set(cfg_encoder) - accepted - _IGNORED
    if unknown:
        raise ValueError(f"Unknown checkpoint architecture fields: {sorted(unknown)}")
    return {k: v for k, v in cfg_encoder.items() if k in accepted}


def load_encoder(checkpoint_path, device="cpu") -> EfficientGaussianEncoder:
    """Build the encoder a checkpoint describes, load its weights strictly, move it to `device`, eval mode."""
    ck = torch.load(checkpoint_path, map_location="cpu", weights_only=True)
    if not isinstance(ck, dict) or "model" not in ck or "cfg" not in ck:
        raise ValueError(f"{checkpoint_path}: not an encoder checkpoint (expected keys step, model, cfg)")
    enc = EfficientGaussianEncoder(**encoder_kwargs(dict(ck["cfg"]["encoder"])))
    enc.load_state_dict(ck["model"], strict=True)
    return enc.to(device).eval()
