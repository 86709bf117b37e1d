"""Splat parameter contract: scale activation and the 9-channel token layout.

Follows gaussian_splat_encoder/params.py:15-41 of the reference. The activation stays a torch op so that
the scale the HIP kernels receive has exactly the bits the reference computes, and the log-scale gradient
chains through autograd.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

# Width floor of the smallest splat in normalised units (params.py:15). Every renderer entry point adds it.
SCALE_EPS = 1e-4


def activate_scale(log_scale: torch.Tensor) -> torch.Tensor:
    """Raw log-scale -> the sigma the renderers draw with: softplus(log_scale) + SCALE_EPS (params.py:18-28)."""
    return F.softplus(log_scale) + SCALE_EPS


def assemble_gaussian_params(enc_out: dict) -> torch.Tensor:
    """Encoder output dict -> [B, N, 9] = [mu(2), log_scale(2), theta(1), color(3), opacity(1)] (params.py:31-41).

    A missing theta becomes zeros and a missing opacity becomes ones, as in the reference.
    """
    mu = enc_out["mu"]
    ls = enc_out["log_scale"]
    th = enc_out["theta"]
    th = th.unsqueeze(-1) if th is not None else torch.zeros_like(mu[..., :1])
    col = enc_out["color"]
    op = enc_out["opacity"]
    op = op.unsqueeze(-1) if op is not None else torch.ones_like(mu[..., :1])
    return torch.cat([mu, ls, th, col, op], dim=-1)
