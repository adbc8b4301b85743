"""Dense differentiable renderer with the toy2d rules (the reference's `render_reference`,
toy2d/gs2d/reference.py:22-58, exported at toy2d/gs2d/__init__.py:3): every Gaussian against
every pixel in PyTorch ops on the tensors' own device, gradients by autograd. It is the
`backend='ref'` of `rasterize` and the ground truth the reference's callers compare with
(toy2d/tests/test_cuda.py:5, toy2d/gradcheck_report.py:11); the tiled HIP kernels are the
product path. Cost O(N * H * W): small scenes only.

Rules (toy2d/gs2d/reference.py:3-8, toy2d/csrc/rasterize.cu:37-101):
  * a Gaussian reaches only the pixels of the tiles inside its tile rectangle (Bins.rect);
  * pixel (x, y) sits at integer coordinates; power = -0.5 (A dx^2 + C dy^2) - B dx dy, and the
    splat is skipped where power > 0;
  * alpha = min(0.99, opacity exp(power)), skipped where alpha < 1/255;
  * front to back in Bins.order; a pixel stops before the splat that would take T below 1e-4;
  * out = sum_i c_i alpha_i T_i + T_final bg.

The depth axis is evaluated at once for a block of pixels: with a_i the alpha of the splats a
pixel may blend (zero elsewhere), T after splat i is the cumulative product of (1 - a); T only
falls, so the splats whose product falls below 1e-4 are exactly the terminating one and all
after it, which the pixel does not blend.
"""
from __future__ import annotations

import torch

from .binning import TILE, Bins

ALPHA_MIN = 1.0 / 255.0
ALPHA_MAX = 0.99
T_MIN = 1e-4


def render_reference(means, conic, color, opacity, bins: Bins, bg=None, pixels_per_block: int = 2048):
    """(3, H, W) image of the Gaussians in bins.order, differentiable in means, conic, color and
    opacity. bg: (3,) background (default black)."""
    H, W = bins.H, bins.W
    dtype, device = means.dtype, means.device
    if bg is None:
        bg = torch.zeros(3, dtype=dtype, device=device)
    order = bins.order.to(device).long()
    if order.numel() == 0:
        return bg.reshape(3, 1, 1).expand(3, H, W).clone()
    m, cn, col, op = means[order], conic[order], color[order], opacity[order]
    rect = bins.rect.to(device).long()[order]
    ys, xs = torch.meshgrid(torch.arange(H, device=device), torch.arange(W, device=device), indexing="ij")
    xs, ys = xs.reshape(-1), ys.reshape(-1)
    blocks = []
    for p0 in range(0, H * W, pixels_per_block):
        x, y = xs[p0:p0 + pixels_per_block], ys[p0:p0 + pixels_per_block]
        tx, ty = (x // TILE)[None, :], (y // TILE)[None, :]
        inrect = (tx >= rect[:, 0:1]) & (tx < rect[:, 2:3]) & (ty >= rect[:, 1:2]) & (ty < rect[:, 3:4])
        dx = m[:, 0:1] - x.to(dtype)[None, :]
        dy = m[:, 1:2] - y.to(dtype)[None, :]
        power = -0.5 * (cn[:, 0:1] * dx * dx + cn[:, 2:3] * dy * dy) - cn[:, 1:2] * dx * dy
        alpha = torch.clamp(op[:, None] * torch.exp(power), max=ALPHA_MAX)  # [N, pixels]
        with torch.no_grad():
            ok = inrect & (power <= 0) & (alpha >= ALPHA_MIN)
            t_after = torch.cumprod(1.0 - torch.where(ok, alpha, torch.zeros_like(alpha)), dim=0)
            blended = ok & (t_after >= T_MIN)
        a = torch.where(blended, alpha, torch.zeros_like(alpha))
        t_incl = torch.cumprod(1.0 - a, dim=0)
        t_before = torch.cat([torch.ones_like(t_incl[:1]), t_incl[:-1]], 0)
        c = (a * t_before).T @ col  # [pixels, 3]
        blocks.append(c + t_incl[-1][:, None] * bg[None, :])
    return torch.cat(blocks, 0).T.reshape(3, H, W)
