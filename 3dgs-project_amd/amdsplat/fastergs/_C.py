"""The extension functions of Faster-GS's rasterizer (`FasterGSCudaBackend._C`) over the MI355X
path, with the call shapes of the reference's 3D tests:

    image, pb, tb, ib, bb, n_inst, n_buckets, sel = _C.forward(means, scales, rotations, opacities, sh0,
        sh_rest, w2c, cam_position, bg, active_sh_bases, W, H, fx, fy, cx, cy, near, far, proper_antialiasing)
    grads = _C.backward(densification_info, grad_image, image, means, scales, rotations, opacities, sh_rest,
        pb, tb, ib, bb, *settings, n_inst, n_buckets, sel[, mode])
    _C.n_touched_tiles(pb, n), _C.adam_step(...), _C.adam_step_sparse(...)

(phase1/tests/test_parity.py:82-98, cluster/tests/test_lean_adam.py:46-47,123,
cluster/patches/fastergs_lean_adam.patch:206-220,308-317). Parameters are Faster-GS's raw ones:
log-scales, unnormalised (w, x, y, z) rotations, opacity logits [N, 1], SH DC [N, 1, 3] and
rest [N, K - 1, 3]; w2c is the row-major world-to-camera matrix (x right, y down, z forward).

Where Faster-GS returns opaque byte blobs, forward returns the forward's device state as the
primitive buffers (tile, instance and bucket blobs are None) and backward takes it back; the
counts are Python ints (one device read, as Faster-GS's own count readbacks,
phase2/fastergs_readback.patch:46-85). `mode` selects among Faster-GS's blend-backward kernels
(phase1/fastergs_macro.patch:493-509); every mode runs the one bucketed backward here.
"""
from __future__ import annotations

import math

import torch

from .. import raster3d as R
from ..adam import adam_step, adam_step_sparse  # noqa: F401  (the patch's _C.adam_step / adam_step_sparse)

__all__ = ["forward", "backward", "n_touched_tiles", "adam_step", "adam_step_sparse"]


class PrimitiveBuffers:
    """What forward returns in place of Faster-GS's primitive byte blob: the forward's device
    state, and the SH DC coefficients (backward is handed only the rest)."""

    __slots__ = ("state", "sh0")

    def __init__(self, state: R.ForwardState, sh0: torch.Tensor):
        self.state = state
        self.sh0 = sh0


def camera(w2c, cam_position, width, height, focal_x, focal_y, center_x, center_y, near_plane, far_plane,
           proper_antialiasing) -> R.Camera:
    """Camera of Faster-GS's settings. The SH view directions are taken from the camera centre of
    w2c; a cam_position that is not that centre is an error (not silently replaced)."""
    vm = torch.as_tensor(w2c).detach().to("cpu", torch.float64).reshape(4, 4)
    centre = -(vm[:3, :3].T @ vm[:3, 3])
    cp = torch.as_tensor(cam_position).detach().to("cpu", torch.float64).reshape(3)
    if float((cp - centre).abs().max()) > 1e-4 * max(1.0, float(centre.abs().max())):
        raise ValueError(f"cam_position {cp.tolist()} is not the camera centre {centre.tolist()} of w2c")
    return R.Camera(vm.float(), float(focal_x), float(focal_y), float(center_x), float(center_y), int(width),
                    int(height), float(near_plane), float(far_plane), bool(proper_antialiasing))


def sh_degree_of(active_sh_bases: int, sh_rest: torch.Tensor) -> int:
    deg = math.isqrt(int(active_sh_bases)) - 1
    if deg < 0 or (deg + 1) ** 2 != int(active_sh_bases) or active_sh_bases > 1 + sh_rest.shape[1]:
        raise ValueError(f"active_sh_bases must be 1, 4, 9 or 16 and at most {1 + sh_rest.shape[1]}, "
                         f"got {active_sh_bases}")
    return deg


def _opacity_logits(opacities: torch.Tensor) -> torch.Tensor:
    if opacities.dim() == 2 and opacities.shape[1] == 1:
        return opacities.reshape(-1)
    if opacities.dim() != 1:
        raise ValueError(f"opacities must be [N, 1] (or [N]), got {tuple(opacities.shape)}")
    return opacities


def _bg(bg) -> tuple:
    return tuple(float(x) for x in torch.as_tensor(bg).detach().cpu().reshape(3).tolist())


def forward(means, scales, rotations, opacities, sh_coefficients_0, sh_coefficients_rest, w2c, cam_position, bg,
            active_sh_bases, width, height, focal_x, focal_y, center_x, center_y, near_plane, far_plane,
            proper_antialiasing):
    cam = camera(w2c, cam_position, width, height, focal_x, focal_y, center_x, center_y, near_plane, far_plane,
                 proper_antialiasing)
    deg = sh_degree_of(active_sh_bases, sh_coefficients_rest)
    sh0 = sh_coefficients_0.detach().contiguous()
    fs = R.forward_pass(means.detach(), scales.detach(), rotations.detach(), _opacity_logits(opacities.detach()),
                        (sh0, sh_coefficients_rest.detach()), cam, sh_degree=deg, bg=_bg(bg))
    return fs.image, PrimitiveBuffers(fs, sh0), None, None, None, fs.m, fs.n_buckets, 0


def backward(densification_info, grad_image, image, means, scales, rotations, opacities, sh_coefficients_rest,
             primitive_buffers, tile_buffers, instance_buffers, bucket_buffers, w2c, cam_position, bg,
             active_sh_bases, width, height, focal_x, focal_y, center_x, center_y, near_plane, far_plane,
             proper_antialiasing, n_instances, n_buckets, instance_primitive_indices_selector, mode=None):
    """Returns (grad means, grad scales, grad rotations, grad opacities [N, 1], grad SH DC, grad SH
    rest); densification_info ([2 or 3, N] float32, or empty) gets this view's statistics added."""
    if not isinstance(primitive_buffers, PrimitiveBuffers):
        raise TypeError("primitive_buffers must be what forward returned")
    fs = primitive_buffers.state
    di = densification_info if densification_info is not None and densification_info.numel() > 0 else None
    if di is not None and (di.dim() != 2 or di.shape[0] not in (2, 3)):
        raise ValueError(f"densification_info must be [2 or 3, N] or empty, got {tuple(di.shape)}")
    g = R.backward_pass(fs, means.detach().contiguous(), scales.detach().contiguous(),
                        rotations.detach().contiguous(), _opacity_logits(opacities.detach()).contiguous(),
                        (primitive_buffers.sh0, sh_coefficients_rest.detach().contiguous()), grad_image,
                        abs_grad=di is not None and di.shape[0] == 3)
    g_means, g_scales, g_rot, g_op, (g_sh0, g_rest), grad2d, _ = g
    if di is not None:
        R.densification_stats(grad2d, fs.touched, fs.cam.width, fs.cam.height, di)
    return g_means, g_scales, g_rot, g_op.reshape(opacities.shape), g_sh0, g_rest


def n_touched_tiles(primitive_buffers, n_primitives: int) -> torch.Tensor:
    """int32 [n_primitives]: tiles each primitive reaches in the forward (0 = culled)."""
    t = primitive_buffers.state.touched
    if t.numel() != int(n_primitives):
        raise ValueError(f"the buffers hold {t.numel()} primitives, not {n_primitives}")
    return t.clone()
