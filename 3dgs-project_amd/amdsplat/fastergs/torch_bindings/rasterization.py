"""Faster-GS's differentiable rasterizer entry (`torch_bindings/rasterization.py`) over the
MI355X path: `RasterizerSettings`, `_Rasterize` and `diff_rasterize(means, scales, rotations,
opacities, sh_coefficients_0, sh_coefficients_rest, densification_info, rasterizer_settings)
-> image`, called as at cluster/tests/test_lean_adam.py:107-124 (fields of the settings at
:119-121; the class-attribute visibility hand-off of cluster/patches/fastergs_lean_adam.patch:
329-343).
"""
from __future__ import annotations

from typing import Any, NamedTuple

import torch

from ... import raster3d as R
from .. import _C


class RasterizerSettings(NamedTuple):
    w2c: torch.Tensor
    cam_position: torch.Tensor
    bg_color: torch.Tensor
    active_sh_bases: int
    width: int
    height: int
    focal_x: float
    focal_y: float
    center_x: float
    center_y: float
    near_plane: float
    far_plane: float
    proper_antialiasing: bool

    def as_tuple(self) -> tuple:
        return tuple(self)


class _Rasterize(torch.autograd.Function):
    # The reference patch's visibility hand-off: with track_visibility set, each differentiable
    # forward leaves its n_touched_tiles (int32 [N], > 0 = visible) in last_visibility (and in the
    # same alias of amdsplat.rasterize, which FusedAdam(sparse=True) reads when step() is not
    # handed a mask).
    track_visibility: bool = False
    last_visibility: "torch.Tensor | None" = None

    @staticmethod
    def forward(ctx: Any, means, scales, rotations, opacities, sh_coefficients_0, sh_coefficients_rest,
                densification_info, rasterizer_settings: RasterizerSettings):
        image, pb, tb, ib, bb, n_inst, n_buckets, sel = _C.forward(means, scales, rotations, opacities,
                                                                   sh_coefficients_0, sh_coefficients_rest,
                                                                   *rasterizer_settings.as_tuple())
        if _Rasterize.track_visibility or R._Rasterize3D.track_visibility:
            vis = pb.state.touched
            _Rasterize.last_visibility = vis
            R._Rasterize3D.last_visibility = vis
        ctx.rasterizer_settings = rasterizer_settings
        ctx.densification_info = densification_info
        ctx.buffers = (pb, tb, ib, bb)
        ctx.buffer_state = (n_inst, n_buckets, sel)
        ctx.save_for_backward(image, means, scales, rotations, opacities, sh_coefficients_rest)
        # a new tensor object over the image's storage: the primitive buffers on ctx hold the
        # forward state and its image, and returning that same object would make a reference cycle
        # (output -> grad_fn -> ctx -> buffers -> output) that only the cyclic collector frees
        return image.detach()

    @staticmethod
    def backward(ctx: Any, grad_image):
        image, means, scales, rotations, opacities, sh_rest = ctx.saved_tensors
        grads = _C.backward(ctx.densification_info, grad_image.contiguous(), image, means, scales, rotations,
                            opacities, sh_rest, *ctx.buffers, *ctx.rasterizer_settings.as_tuple(), *ctx.buffer_state)
        return (*grads, None, None)


def diff_rasterize(means, scales, rotations, opacities, sh_coefficients_0, sh_coefficients_rest,
                   densification_info, rasterizer_settings: RasterizerSettings) -> torch.Tensor:
    """Renders the image [3, H, W]; densification_info ([2 or 3, N] float32, or empty) receives
    the view's densification statistics in the backward."""
    return _Rasterize.apply(means, scales, rotations, opacities, sh_coefficients_0, sh_coefficients_rest,
                            densification_info, rasterizer_settings)
