"""Learnable 2D Gaussians and their activation (caller side of the rasterizer; the same
parametrisation and seeded initialisation as toy2d/gs2d/params.py:16-59, so a seed gives
the same Gaussians as the reference).

The rasterizer sees four tensors per Gaussian: means [N,2] (pixels), conic [N,3] = (A, B, C)
of the inverse covariance [[A, B], [B, C]], color [N,3] in [0,1], opacity [N] in [0,1].
"""
import math

import torch


class Gaussians2D(torch.nn.Module):
    def __init__(self, n: int, H: int, W: int, seed: int = 0, dtype=torch.float32):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        spacing = math.sqrt(H * W / n) * 0.5
        # draw order: positions, scales, angles, colours, opacities, depths
        self.xy = torch.nn.Parameter(torch.rand(n, 2, generator=gen, dtype=dtype) * torch.tensor([W, H], dtype=dtype))
        self.log_scale = torch.nn.Parameter(torch.log(spacing * (0.5 + torch.rand(n, 2, generator=gen, dtype=dtype))))
        self.theta = torch.nn.Parameter(torch.rand(n, generator=gen, dtype=dtype) * math.pi)
        self.rgb_logit = torch.nn.Parameter(0.5 * torch.randn(n, 3, generator=gen, dtype=dtype))
        self.opacity_logit = torch.nn.Parameter(0.5 * torch.randn(n, generator=gen, dtype=dtype))
        # fixed draw order: smaller depth is in front
        self.register_buffer("depth", torch.rand(n, generator=gen, dtype=dtype))

    def activated(self):
        return activate(self.xy, self.log_scale, self.theta, self.rgb_logit, self.opacity_logit)

    def activated_fused(self):
        """(means, conic, color, opacity, cov, radii) of activate_fused: the activation and the
        3-sigma radii in one launch (CUDA parameters)."""
        return activate_fused(self.xy, self.log_scale, self.theta, self.rgb_logit, self.opacity_logit)


def activate(xy, log_scale, theta, rgb_logit, opacity_logit):
    """(means, conic, color, opacity, cov): cov = (xx, xy, yy) of R diag(s^2) R^T."""
    var = torch.exp(2.0 * log_scale)
    c, s = torch.cos(theta), torch.sin(theta)
    vx, vy = var[:, 0], var[:, 1]
    cxx = c * c * vx + s * s * vy
    cxy = c * s * (vx - vy)
    cyy = s * s * vx + c * c * vy
    det = cxx * cyy - cxy * cxy
    conic = torch.stack([cyy / det, -cxy / det, cxx / det], dim=-1)
    return xy, conic, torch.sigmoid(rgb_logit), torch.sigmoid(opacity_logit), torch.stack([cxx, cxy, cyy], dim=-1)


class _ActivateFused(torch.autograd.Function):
    @staticmethod
    def forward(ctx, xy, log_scale, theta, rgb_logit, opacity_logit):
        from amdsplat._lib import call, ptr, stream_handle

        ls, th, rl, ol = (t.detach().contiguous() for t in (log_scale, theta, rgb_logit, opacity_logit))
        n = xy.shape[0]
        dev = xy.device
        radii = torch.empty(n, dtype=torch.int32, device=dev)
        conic, color, cov = (torch.empty(n, 3, dtype=torch.float32, device=dev) for _ in range(3))
        opacity = torch.empty(n, dtype=torch.float32, device=dev)
        call("gs2d_activate_fwd", ptr(ls), ptr(th), ptr(rl), ptr(ol), n, ptr(conic), ptr(color), ptr(opacity),
             ptr(cov), ptr(radii), stream_handle(dev))
        ctx.save_for_backward(ls, th, rl, ol)
        ctx.mark_non_differentiable(cov, radii)
        return xy.view_as(xy), conic, color, opacity, cov, radii

    @staticmethod
    def backward(ctx, g_means, g_conic, g_color, g_opacity, _g_cov, _g_radii):
        from amdsplat._lib import call, ptr, stream_handle

        ls, th, rl, ol = ctx.saved_tensors
        n = ls.shape[0]
        dev = ls.device
        g_ls, g_rl = torch.empty_like(ls), torch.empty_like(rl)
        g_th, g_ol = torch.empty_like(th), torch.empty_like(ol)
        gc, gcol, gop = (None if g is None else g.contiguous().float() for g in (g_conic, g_color, g_opacity))
        call("gs2d_activate_bwd", ptr(ls), ptr(th), ptr(rl), ptr(ol), n, ptr(gc), ptr(gcol), ptr(gop), ptr(g_ls),
             ptr(g_th), ptr(g_rl), ptr(g_ol), stream_handle(dev))
        return g_means, g_ls, g_th, g_rl, g_ol


def activate_fused(xy, log_scale, theta, rgb_logit, opacity_logit):
    """activate and radii_from_cov in one HIP launch (and one for the backward), for fit loops on
    the GPU: (means, conic, color, opacity, cov, radii). The same operations in the same order on
    float32 CUDA tensors, with exp / cos / sin from the device math library (which may round
    differently from the tensor library's in the last place); cov and radii take no gradient."""
    if not xy.is_cuda or any(t.dtype != torch.float32 for t in (xy, log_scale, theta, rgb_logit, opacity_logit)):
        raise ValueError("activate_fused takes float32 CUDA tensors")
    return _ActivateFused.apply(xy, log_scale, theta, rgb_logit, opacity_logit)


@torch.no_grad()
def radii_from_cov(cov: torch.Tensor) -> torch.Tensor:
    """Integer 3-sigma radius of the larger eigenvalue (0 for a degenerate covariance)."""
    cxx, cxy, cyy = cov.unbind(-1)
    det = cxx * cyy - cxy * cxy
    mid = 0.5 * (cxx + cyy)
    lam = mid + torch.sqrt(torch.clamp(mid * mid - det, min=0.1))
    r = torch.ceil(3.0 * torch.sqrt(lam))
    return torch.where(det > 0, r, torch.zeros_like(r)).to(torch.int32)


def fit_scene_4k(n: int = 4096, size: int = 256, seed: int = 0):
    """The 2D image-fit workload: n Gaussians on a size x size image with means U(0, size)^2,
    log-scales N(ln 2, 0.3) per axis, angle U(0, pi), opacity sigmoid(N(0, 1)), colour U(0, 1),
    a fixed U(0, 1) depth and a U(0, 1) target image [3, size, size], drawn in that order from
    one seeded CPU generator. Returns the rasterizer inputs (means, conic, color, opacity), the
    covariance, the depth and the target (float32, CPU)."""
    g = torch.Generator().manual_seed(seed)
    xy = torch.rand(n, 2, generator=g) * float(size)
    log_scale = math.log(2.0) + 0.3 * torch.randn(n, 2, generator=g)
    theta = torch.rand(n, generator=g) * math.pi
    opacity = torch.sigmoid(torch.randn(n, generator=g))
    color = torch.rand(n, 3, generator=g)
    depth = torch.rand(n, generator=g)
    target = torch.rand(3, size, size, generator=g)
    means, conic, _, _, cov = activate(xy, log_scale, theta, torch.zeros(n, 3), torch.zeros(n))
    return means, conic, color, opacity, cov, depth, target


def fit_model_4k(n: int = 4096, size: int = 256, seed: int = 0):
    """The 2D image-fit workload as a trainable model: the draws of fit_scene_4k (same generator
    and order) as the raw parameters of a Gaussians2D (colour and opacity through their logits),
    and the target image. Returns (model, target), float32 on the CPU."""
    g = torch.Generator().manual_seed(seed)
    xy = torch.rand(n, 2, generator=g) * float(size)
    log_scale = math.log(2.0) + 0.3 * torch.randn(n, 2, generator=g)
    theta = torch.rand(n, generator=g) * math.pi
    opacity_logit = torch.randn(n, generator=g)
    color = torch.rand(n, 3, generator=g)
    depth = torch.rand(n, generator=g)
    target = torch.rand(3, size, size, generator=g)
    model = Gaussians2D(n, size, size, seed=seed)
    with torch.no_grad():
        model.xy.copy_(xy)
        model.log_scale.copy_(log_scale)
        model.theta.copy_(theta)
        model.rgb_logit.copy_(torch.logit(color))
        model.opacity_logit.copy_(opacity_logit)
        model.depth.copy_(depth)
    return model, target
