"""Float64 restatement of the L1 + D-SSIM loss (TEST INFRASTRUCTURE: used by tests/ only).

SSIM (Wang et al. 2004) as the 3DGS trainers compute it: an 11x11 Gaussian window (sigma 1.5,
normalised), zero padding of 5 ("same"), C1 = 0.01^2, C2 = 0.03^2, mean over pixels and
channels; the fused-ssim extension the reference trains with (results/phase1/README.md:46-47)
computes the same map. L = (1 - lambda) mean|x - y| + lambda (1 - mean SSIM), lambda = 0.2 in the
reference's configs (phase2/logs/run_4559238/runs/b_room_up_s10/training_config.yaml:100).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

C1, C2 = 0.01 ** 2, 0.03 ** 2


def gaussian_1d(size: int = 11, sigma: float = 1.5) -> torch.Tensor:
    x = torch.arange(size, dtype=torch.float64) - size // 2
    g = torch.exp(-(x * x) / (2.0 * sigma * sigma))
    return g / g.sum()


def ssim_map(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """x, y: [C, H, W] float64. Returns the per-pixel SSIM [C, H, W]."""
    C = x.shape[0]
    g = gaussian_1d()
    win = (g[:, None] * g[None, :]).expand(C, 1, 11, 11).contiguous()
    f = lambda t: F.conv2d(t[None], win, padding=5, groups=C)[0]
    mu1, mu2 = f(x), f(y)
    s11 = f(x * x) - mu1 * mu1
    s22 = f(y * y) - mu2 * mu2
    s12 = f(x * y) - mu1 * mu2
    return ((2 * mu1 * mu2 + C1) * (2 * s12 + C2)) / ((mu1 * mu1 + mu2 * mu2 + C1) * (s11 + s22 + C2))


def l1_ssim(x: torch.Tensor, y: torch.Tensor, lam: float = 0.2) -> torch.Tensor:
    return (1.0 - lam) * (x - y).abs().mean() + lam * (1.0 - ssim_map(x, y).mean())


def loss_and_grad(x: np.ndarray, y: np.ndarray, lam: float = 0.2):
    """Float64 loss parts (L, mean L1, mean SSIM) and dL/dx for float32 numpy images."""
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    yt = torch.from_numpy(y.astype(np.float64))
    smap = ssim_map(xt, yt)
    l1 = (xt - yt).abs().mean()
    L = (1.0 - lam) * l1 + lam * (1.0 - smap.mean())
    L.backward()
    return (float(L.detach()), float(l1.detach()), float(smap.detach().mean())), xt.grad.numpy()


def ssim_brute(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """Direct summation of the definition with explicit zero padding (tiny images only)."""
    g = gaussian_1d().numpy()
    w = np.outer(g, g)
    C, H, W = x.shape
    out = np.zeros((C, H, W))
    for c in range(C):
        for i in range(H):
            for j in range(W):
                m = np.zeros(5)
                for a in range(11):
                    for b in range(11):
                        ii, jj = i + a - 5, j + b - 5
                        if 0 <= ii < H and 0 <= jj < W:
                            u, v = float(x[c, ii, jj]), float(y[c, ii, jj])
                            m += w[a, b] * np.array([u, v, u * u, v * v, u * v])
                s11, s22, s12 = m[2] - m[0] ** 2, m[3] - m[1] ** 2, m[4] - m[0] * m[1]
                out[c, i, j] = ((2 * m[0] * m[1] + C1) * (2 * s12 + C2)) / ((m[0] ** 2 + m[1] ** 2 + C1) * (s11 + s22 + C2))
    return out
