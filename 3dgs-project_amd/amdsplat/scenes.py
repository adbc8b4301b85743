"""Seeded synthetic 3D scenes and cameras for the benchmark workloads.

Everything is drawn on the CPU with a torch.Generator in a fixed call order, so a scene is
the same on every machine; tensors are moved to the target device afterwards.

  sh_rgb_100k   100k Gaussians, SH degree 0, 800x800, fx=fy=1111, camera at radius 4
  sh3_1m        1M Gaussians, SH degree 3, 1297x840, fx=fy=1160, 8 orbit poses radius U(3,5)
  sh3_3m        3M Gaussians, SH degree 3, 1957x1091, fx=fy=1450, 8 orbit poses
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .raster3d import Camera

SH_C0 = 0.28209479177387814


@dataclass
class Scene:
    name: str
    means: torch.Tensor
    log_scales: torch.Tensor
    quats: torch.Tensor
    opacity_logits: torch.Tensor
    sh: torch.Tensor
    cameras: list
    bg: tuple = (0.0, 0.0, 0.0)

    @property
    def n(self) -> int:
        return self.means.shape[0]

    def to(self, device) -> "Scene":
        return Scene(self.name, *(t.to(device).contiguous() for t in (self.means, self.log_scales, self.quats,
                                                                       self.opacity_logits, self.sh)),
                     self.cameras, self.bg)

    def params(self):
        return self.means, self.log_scales, self.quats, self.opacity_logits, self.sh


def look_at(eye, target=(0.0, 0.0, 0.0), up=(0.0, 0.0, 1.0)) -> torch.Tensor:
    """World-to-camera 4x4 with OpenCV axes (x right, y down, z toward the target)."""
    e = torch.tensor(eye, dtype=torch.float64)
    f = torch.tensor(target, dtype=torch.float64) - e
    f = f / f.norm()
    u = torch.tensor(up, dtype=torch.float64)
    r = torch.linalg.cross(f, u)
    if r.norm() < 1e-9:
        r = torch.linalg.cross(f, torch.tensor([0.0, 1.0, 0.0], dtype=torch.float64))
    r = r / r.norm()
    d = torch.linalg.cross(f, r)
    R = torch.stack([r, d, f])
    vm = torch.eye(4, dtype=torch.float64)
    vm[:3, :3] = R
    vm[:3, 3] = -R @ e
    return vm.float()


def orbit_cameras(n_poses: int, seed: int, radius: tuple, width: int, height: int, f: float,
                  near: float = 0.01, far: float = 100.0) -> list:
    g = torch.Generator().manual_seed(seed)
    cams = []
    for _ in range(n_poses):
        r = radius[0] + (radius[1] - radius[0]) * torch.rand(1, generator=g, dtype=torch.float64).item()
        az = 2.0 * math.pi * torch.rand(1, generator=g, dtype=torch.float64).item()
        el = (torch.rand(1, generator=g, dtype=torch.float64).item() - 0.5) * 1.0
        eye = (r * math.cos(el) * math.cos(az), r * math.cos(el) * math.sin(az), r * math.sin(el))
        cams.append(Camera(look_at(eye), f, f, width / 2.0, height / 2.0, width, height, near, far))
    return cams


def random_quats(n: int, g: torch.Generator) -> torch.Tensor:
    q = torch.randn(n, 4, generator=g)
    return q / q.norm(dim=1, keepdim=True)


def sh_rgb_100k(n: int = 100_000, seed: int = 0) -> Scene:
    g = torch.Generator().manual_seed(seed)
    means = 0.5 * torch.randn(n, 3, generator=g)
    log_scales = -5.0 + 3.0 * torch.rand(n, 3, generator=g)
    quats = random_quats(n, g)
    opacity_logits = torch.randn(n, generator=g)
    colors = torch.rand(n, 3, generator=g)
    sh = ((colors - 0.5) / SH_C0).reshape(n, 1, 3)
    cam = Camera(look_at((4.0, 0.0, 0.0)), 1111.0, 1111.0, 400.0, 400.0, 800, 800, 0.01, 100.0)
    return Scene("sh_rgb_100k", means, log_scales, quats, opacity_logits, sh.contiguous(), [cam])


def _mixture_means(n: int, g: torch.Generator) -> torch.Tensor:
    n_ball = int(round(0.8 * n))
    ball = torch.randn(n_ball, 3, generator=g)
    d = torch.randn(n - n_ball, 3, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    r = 8.0 + 4.0 * torch.rand(n - n_ball, 1, generator=g)
    return torch.cat([ball, d * r], 0)


def sh3_scene(n: int, log_scale_mu: float, log_scale_sigma: float, width: int, height: int, f: float,
              seed: int = 0, name: str = "sh3") -> Scene:
    g = torch.Generator().manual_seed(seed)
    means = _mixture_means(n, g)
    log_scales = log_scale_mu + log_scale_sigma * torch.randn(n, 3, generator=g)
    quats = random_quats(n, g)
    opacity_logits = -1.0 + 1.5 * torch.randn(n, generator=g)
    sh = torch.empty(n, 16, 3)
    sh[:, 0, :] = 0.5 * torch.randn(n, 3, generator=g)
    sh[:, 1:, :] = 0.05 * torch.randn(n, 15, 3, generator=g)
    cams = orbit_cameras(8, seed, (3.0, 5.0), width, height, f)
    return Scene(name, means, log_scales, quats, opacity_logits, sh, cams)


def sh3_1m(n: int = 1_000_000, seed: int = 0) -> Scene:
    return sh3_scene(n, -4.5, 1.0, 1297, 840, 1160.0, seed, "sh3_1m")


def sh3_3m(n: int = 3_000_000, seed: int = 0) -> Scene:
    return sh3_scene(n, -4.0, 1.2, 1957, 1091, 1450.0, seed, "sh3_3m")


def small_scene(n: int, width: int, height: int, seed: int = 0, sh_coeffs: int = 16,
                scale: tuple = (0.01, 0.1), opacity: tuple = (0.05, 0.95), depth: tuple = (2.0, 8.0),
                spread: float = 0.6) -> Scene:
    """Test scene in camera space (identity view), after phase1/tests/test_parity.py:59-84:
    depths U(depth), x/y spread slightly beyond the frustum, log-uniform scales, raw quats,
    opacities U(opacity), DC ~ 0.8 N(0,1) (some colours clamp), rest ~ 0.1 N(0,1)."""
    g = torch.Generator().manual_seed(seed)

    def u(lo, hi, *shape):
        return lo + (hi - lo) * torch.rand(*shape, generator=g)

    focal = 0.9 * width
    z = u(*depth, n)
    x = u(-spread, spread, n) * width / focal * z
    y = u(-spread, spread, n) * height / focal * z
    means = torch.stack([x, y, z], -1)
    log_scales = torch.log(u(*scale, n, 3))
    quats = torch.randn(n, 4, generator=g)
    o = u(*opacity, n)
    opacity_logits = torch.log(o / (1 - o))
    sh = torch.empty(n, sh_coeffs, 3)
    sh[:, 0, :] = 0.8 * torch.randn(n, 3, generator=g)
    if sh_coeffs > 1:
        sh[:, 1:, :] = 0.1 * torch.randn(n, sh_coeffs - 1, 3, generator=g)
    cam = Camera(torch.eye(4), focal, focal, width / 2 + 0.3, height / 2 - 0.2, width, height, 0.2, 1000.0)
    return Scene(f"small_{n}_{width}x{height}", means, log_scales, quats, opacity_logits, sh, [cam])
