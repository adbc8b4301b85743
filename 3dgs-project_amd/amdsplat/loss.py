"""Fused L1 + D-SSIM training loss on the GPU (gs_l1_ssim_fwd / gs_l1_ssim_bwd).

`l1_ssim_loss(image, target, lambda_dssim=0.2)` = (1 - lambda) mean|image - target| +
lambda (1 - mean SSIM(image, target)), differentiable with respect to image; `fused_ssim(img1,
img2)` mirrors the fused-ssim extension's call (mean SSIM, 11x11 Gaussian window, sigma 1.5,
"same" padding), differentiable with respect to img1. Images are [C, H, W] or [1, C, H, W]
float32 CUDA tensors. The loss value stays on the device (no host synchronisation).
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr


def _as_chw(t: torch.Tensor) -> torch.Tensor:
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise ValueError("batched images are not supported: pass [C, H, W] or [1, C, H, W]")
        t = t[0]
    if t.dim() != 3:
        raise ValueError(f"expected [C, H, W], got {tuple(t.shape)}")
    if not (t.is_cuda and t.dtype == torch.float32):
        raise ValueError("images must be float32 CUDA tensors")
    return t.contiguous()


class _L1Ssim(torch.autograd.Function):
    @staticmethod
    def forward(ctx, image, target, lambda_dssim: float):
        x, y = _as_chw(image), _as_chw(target.detach())
        if x.shape != y.shape:
            raise ValueError(f"shape mismatch {tuple(x.shape)} vs {tuple(y.shape)}")
        C, H, W = x.shape
        dev = x.device
        dmap = torch.empty(C, 3, H, W, dtype=torch.float32, device=dev) if ctx.needs_input_grad[0] else None
        loss = torch.empty(3, dtype=torch.float32, device=dev)
        ws = torch.empty(max(_lib.size_call("gs_l1_ssim_workspace_size", C, H, W), 1), dtype=torch.uint8, device=dev)
        call("gs_l1_ssim_fwd", ptr(x), ptr(y), C, H, W, float(lambda_dssim), ptr(dmap), ptr(loss), ptr(ws),
             ws.numel(), _lib.stream_handle(dev))
        ctx.save_for_backward(x, y, dmap)
        ctx.lam = float(lambda_dssim)
        ctx.in_shape = image.shape
        ctx.mark_non_differentiable(loss)
        return loss[0].clone(), loss

    @staticmethod
    def backward(ctx, grad_out, _grad_parts):
        x, y, dmap = ctx.saved_tensors
        if dmap is None:
            return None, None, None
        C, H, W = x.shape
        g = torch.empty_like(x)
        go = grad_out.detach().to(torch.float32).contiguous().reshape(1)
        call("gs_l1_ssim_bwd", ptr(x), ptr(y), ptr(dmap), C, H, W, ctx.lam, ptr(go), ptr(g),
             _lib.stream_handle(x.device))
        return g.reshape(ctx.in_shape), None, None


def l1_ssim_loss(image: torch.Tensor, target: torch.Tensor, lambda_dssim: float = 0.2,
                 return_parts: bool = False):
    """Returns the loss (0-dim device tensor); with return_parts also (L, mean L1, mean SSIM) [3]."""
    loss, parts = _L1Ssim.apply(image, target, lambda_dssim)
    return (loss, parts) if return_parts else loss


def fused_ssim(img1: torch.Tensor, img2: torch.Tensor, padding: str = "same", train: bool = True) -> torch.Tensor:
    """Mean SSIM of img1 against img2 (differentiable with respect to img1)."""
    if padding != "same":
        raise ValueError("only padding='same' (zero padding, the trainers' setting) is provided")
    return 1.0 - l1_ssim_loss(img1, img2, 1.0)
