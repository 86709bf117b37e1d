"""Host-side argument checks of the render entry points (CPU; no kernel runs): parameter shapes against
color [B,N,C], and the background broadcast of a [1,C] bg over the batch."""

import pytest
import torch

from gaussian_splat_encoder import render_hip as RH


def scene(B=2, N=5, C=3):
    return (torch.rand(B, N, 2), torch.rand(B, N, 2), torch.rand(B, N, C), torch.rand(B, N), torch.rand(B, C),
            torch.rand(B, N))


def test_batch_args_accepts_and_broadcasts():
    mu, ls, col, op, bg, th = scene()
    assert RH._batch_args(mu, ls, col, op, bg, th) is bg
    b1 = RH._batch_args(mu, ls, col, op, bg[:1], None)
    assert b1.shape == (2, 3) and torch.equal(b1[1], bg[0])


@pytest.mark.parametrize("which,bad", [(0, torch.rand(2, 5, 3)), (1, torch.rand(1, 5, 2)), (3, torch.rand(2, 4)),
                                       (4, torch.rand(2, 2)), (4, torch.rand(3, 3)), (4, torch.rand(3)),
                                       (5, torch.rand(2, 6))])
def test_batch_args_refuses_mismatched_shapes(which, bad):
    args = list(scene())
    args[which] = bad
    with pytest.raises(ValueError, match="must be"):
        RH._batch_args(*args)


def test_entry_points_check_shapes_before_the_device():
    mu, ls, col, op, bg, th = scene()
    for fn in (lambda *a, **k: RH.render_alpha_full_triton(*a, cull=True, **k), RH.render_alpha_octave,
               RH.render_alpha_multires):
        with pytest.raises(ValueError, match="bg must be"):
            fn(mu, ls, col, op, torch.rand(3, 3), 16, 16, theta=th)
