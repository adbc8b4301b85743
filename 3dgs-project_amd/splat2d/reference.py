"""Dense differentiable renderer with the phase0 model (the reference's `ref_state` /
`ref_render`, phase0/splat2d/ops.py:350-398, exported at phase0/splat2d/__init__.py:7): every
splat against every pixel in PyTorch ops on the tensors' own device, gradients by autograd. It
is the ground truth the reference's gradient checks compare both custom backwards with
(phase0/tests/gradcheck/test_gradcheck.py:40-47, :96-100) and the source of its counting checks
(phase0/tests/gradcheck/test_opcount.py:73-143); the tiled HIP kernels behind `render` are the
product path. Cost O(N * H * W): small scenes only.

Model (phase0/csrc/macrotile/splat2d_common.h:90-254):
  * pixel (x, y) samples at (x + 0.5, y + 0.5); with d = pixel - mean and the Cholesky factor
    (l0, l1, l2): a = l0 dx + l1 dy, b = l2 dy, q = a^2 + b^2;
  * raw alpha = sigmoid(opacity_logit) exp(-q / 2), alpha = min(raw, 0.99);
  * splats in index order; splat i is composited where alpha_i >= 1/255 and the pixel's T
    before it is >= 1e-4 (no tile restriction: the whole image);
  * image = sum_i colour_i alpha_i T_i, no background.

The splat axis is evaluated at once for a block of pixels. T before splat i is the product of
(1 - alpha) over the earlier splats that pass the alpha test, as long as that product stays at or
above 1e-4; once it falls below, it stays below (T only falls), so "alpha passes and that
product >= 1e-4" is exactly the set of composited splats.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

ALPHA_MIN = 1.0 / 255.0
ALPHA_MAX = 0.99
T_STOP = 1e-4


@dataclass(frozen=True)
class RefState:
    image: Tensor        # [H, W, 3]
    t_final: Tensor      # [H, W]
    raw_alpha: Tensor    # [H, W, N] sigmoid(logit) exp(-q / 2), before the 0.99 clamp (detached)
    contributes: Tensor  # [H, W, N] bool: the splat is composited into the pixel


def _exclusive(t_incl: Tensor) -> Tensor:
    return torch.cat([torch.ones_like(t_incl[:, :1]), t_incl[:, :-1]], dim=1)


def ref_state(means: Tensor, chol: Tensor, opacity_logit: Tensor, colors: Tensor, height: int, width: int,
              max_block_elems: int = 1 << 22) -> RefState:
    """Front-to-back compositing of the whole image in PyTorch ops (differentiable image and
    t_final). max_block_elems bounds the pixel-by-splat block evaluated at once."""
    dtype, device = means.dtype, means.device
    n = means.shape[0]
    H, W = int(height), int(width)
    if n == 0:
        return RefState(image=torch.zeros(H, W, 3, dtype=dtype, device=device),
                        t_final=torch.ones(H, W, dtype=dtype, device=device),
                        raw_alpha=torch.zeros(H, W, 0, dtype=dtype, device=device),
                        contributes=torch.zeros(H, W, 0, dtype=torch.bool, device=device))
    ys, xs = torch.meshgrid(torch.arange(H, dtype=dtype, device=device) + 0.5,
                            torch.arange(W, dtype=dtype, device=device) + 0.5, indexing="ij")
    xs, ys = xs.reshape(-1, 1), ys.reshape(-1, 1)
    o = torch.sigmoid(opacity_logit).reshape(1, n)
    mx, my = means[:, 0].reshape(1, n), means[:, 1].reshape(1, n)
    l0, l1, l2 = chol[:, 0].reshape(1, n), chol[:, 1].reshape(1, n), chol[:, 2].reshape(1, n)
    block = max(1, max_block_elems // n)
    images, t_finals, raws, used = [], [], [], []
    for p0 in range(0, H * W, block):
        dx = xs[p0:p0 + block] - mx  # [pixels, N]
        dy = ys[p0:p0 + block] - my
        a = l0 * dx + l1 * dy
        b = l2 * dy
        raw = o * torch.exp(-0.5 * (a * a + b * b))
        alpha = torch.clamp(raw, max=ALPHA_MAX)
        with torch.no_grad():
            passes = alpha >= ALPHA_MIN
            t_before = _exclusive(torch.cumprod(1.0 - torch.where(passes, alpha, torch.zeros_like(alpha)), dim=1))
            comp = passes & (t_before >= T_STOP)
        a_c = torch.where(comp, alpha, torch.zeros_like(alpha))
        t_incl = torch.cumprod(1.0 - a_c, dim=1)
        images.append((a_c * _exclusive(t_incl)) @ colors)
        t_finals.append(t_incl[:, -1])
        raws.append(raw.detach())
        used.append(comp)
    return RefState(image=torch.cat(images, 0).reshape(H, W, 3),
                    t_final=torch.cat(t_finals, 0).reshape(H, W),
                    raw_alpha=torch.cat(raws, 0).reshape(H, W, n),
                    contributes=torch.cat(used, 0).reshape(H, W, n))


def ref_render(means: Tensor, chol: Tensor, opacity_logit: Tensor, colors: Tensor, height: int,
               width: int) -> Tensor:
    """Differentiable dense reference image [H, W, 3]."""
    return ref_state(means, chol, opacity_logit, colors, height, width).image
