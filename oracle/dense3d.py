"""Differentiable float64 PyTorch reference of the 3D path (for autograd gradients).

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker).

`preprocess64` restates the projection with plain torch ops (autograd differentiates it, so
it pins the hand-derived preprocess backward). `blend64` composites front to back given the
forward's discrete structure -- which list entries were blended into which pixel, taken
from the float32 oracle (oracle.contrib_mask) -- so the function it differentiates is the
same piecewise-smooth branch the kernels take, without float64 re-deciding thresholds.
Rules: phase1/fastergs_macro.patch:125-211, phase1/PLAN.md:51-54 (alpha = o G, no clamp,
colour clamped at 0, background added as T_final * bg).
"""
from __future__ import annotations

import math

import numpy as np
import torch

SH0 = 0.28209479177387814
SH1 = 0.4886025119029199
SH2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792, 0.5462742152960396)
SH3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154, -0.4570457994644658,
       1.445305721320277, -0.5900435899266435)


def sh_basis64(d: torch.Tensor, n: int) -> torch.Tensor:
    """[N, n] real SH basis (3DGS convention) of unit directions d [N, 3]."""
    x, y, z = d[:, 0], d[:, 1], d[:, 2]
    b = [torch.full_like(x, SH0)]
    if n > 1:
        b += [-SH1 * y, SH1 * z, -SH1 * x]
    if n > 4:
        xx, yy, zz = x * x, y * y, z * z
        b += [SH2[0] * x * y, SH2[1] * y * z, SH2[2] * (2 * zz - xx - yy), SH2[3] * x * z, SH2[4] * (xx - yy)]
    if n > 9:
        b += [SH3[0] * y * (3 * xx - yy), SH3[1] * x * y * z, SH3[2] * y * (4 * zz - xx - yy),
              SH3[3] * z * (2 * zz - 3 * xx - 3 * yy), SH3[4] * x * (4 * zz - xx - yy), SH3[5] * z * (xx - yy),
              SH3[6] * x * (xx - 3 * yy)]
    return torch.stack(b, -1)


def cam_derived(cam):
    """Camera centre and Jacobian clamp limits, rounded to float32 exactly like the kernels."""
    vm = cam.viewmat.detach().cpu().double().reshape(4, 4)
    R = vm[:3, :3].float().double()
    t = vm[:3, 3].float().double()
    campos = torch.tensor([float(np.float32(-sum(float(vm[i, j]) * float(vm[i, 3]) for i in range(3))))
                           for j in range(3)], dtype=torch.float64)
    lim = [float(np.float32(v)) for v in (-1.3 * cam.cx / cam.fx, 1.3 * (cam.width - cam.cx) / cam.fx,
                                          -1.3 * cam.cy / cam.fy, 1.3 * (cam.height - cam.cy) / cam.fy)]
    return R, t, campos, lim


def quat_to_rot(q: torch.Tensor) -> torch.Tensor:
    q = q / q.norm(dim=1, keepdim=True)
    w, x, y, z = q.unbind(1)
    return torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1).reshape(-1, 3, 3)


def preprocess64(means, log_scales, quats, opacity_logits, sh, cam, sh_degree):
    """Returns dict(mean2d [N,2], conic [N,3] (A,B,C), opacity [N] (blended: compensated when
    cam.proper_antialiasing), color [N,3] (clamped), depth [N], cov2d [N,3] (a,b,c)) as
    differentiable float64 tensors."""
    R, t, campos, (lxlo, lxhi, lylo, lyhi) = cam_derived(cam)
    v = means @ R.T + t
    vx, vy, vz = v.unbind(1)
    o = torch.sigmoid(opacity_logits)
    Rq = quat_to_rot(quats)
    s = torch.exp(log_scales)
    M = Rq * s[:, None, :]
    Sig = M @ M.transpose(1, 2)
    tx, ty = vx / vz, vy / vz
    txc, tyc = tx.clamp(lxlo, lxhi), ty.clamp(lylo, lyhi)
    zeros = torch.zeros_like(vz)
    J = torch.stack([cam.fx / vz, zeros, -cam.fx * txc / vz, zeros, cam.fy / vz, -cam.fy * tyc / vz], -1).reshape(-1, 2, 3)
    Tm = J @ R
    cov = Tm @ Sig @ Tm.transpose(1, 2)
    a = cov[:, 0, 0] + 0.3
    b = cov[:, 0, 1]
    c = cov[:, 1, 1] + 0.3
    det = a * c - b * b
    if getattr(cam, "proper_antialiasing", False):
        # Mip-Splatting's 2D filter: the dilated splat keeps the undilated splat's integral
        o = o * torch.sqrt(torch.clamp((cov[:, 0, 0] * cov[:, 1, 1] - b * b) / det, min=0.0))
    conic = torch.stack([c / det, -b / det, a / det], -1)
    mean2d = torch.stack([cam.fx * tx + cam.cx, cam.fy * ty + cam.cy], -1)
    d = means - campos
    d = d / d.norm(dim=1, keepdim=True)
    nb = (sh_degree + 1) ** 2
    basis = sh_basis64(d, nb)
    color = (basis[:, :, None] * sh[:, :nb, :]).sum(1) + 0.5
    color = torch.clamp(color, min=0.0)
    return dict(mean2d=mean2d, conic=conic, opacity=o, color=color, depth=vz, cov2d=torch.stack([a, b, c], -1))


def blend64(mean2d, conic, opacity, color, point_list, ranges, mask, width, height, bg=(0.0, 0.0, 0.0),
            scores=None):
    """Front-to-back compositing per 16x16 tile given the blended-entry mask [M, 256].
    Returns (image [3,H,W], final_T [H,W]) as differentiable float64 tensors. scores (optional
    float64 [N] tensor) receives each Gaussian's blending weights summed over the image."""
    dev = mean2d.device
    tiles_x = (width + 15) // 16
    img = torch.zeros(3, height, width, dtype=torch.float64, device=dev)
    fT = torch.ones(height, width, dtype=torch.float64, device=dev)
    bg = torch.tensor(bg, dtype=torch.float64, device=dev)
    t_idx = torch.arange(256, device=dev)
    lx, ly = t_idx % 16, t_idx // 16
    mask_t = torch.as_tensor(mask.astype(np.bool_), device=dev)
    pl = torch.as_tensor(point_list.astype(np.int64), device=dev)
    out_img = []
    for tile in range(ranges.shape[0]):
        s, e = int(ranges[tile, 0]), int(ranges[tile, 1])
        tx, ty = tile % tiles_x, tile // tiles_x
        px, py = tx * 16 + lx, ty * 16 + ly
        inside = (px < width) & (py < height)
        if not bool(inside.any()):
            continue
        pxf, pyf = px.double() + 0.5, py.double() + 0.5
        if e > s:
            ids = pl[s:e]
            m2 = mean2d[ids]
            cn = conic[ids]
            dx = m2[:, 0:1] - pxf[None, :]
            dy = m2[:, 1:2] - pyf[None, :]
            power = -0.5 * (cn[:, 0:1] * dx * dx + 2 * cn[:, 1:2] * dx * dy + cn[:, 2:3] * dy * dy)
            alpha = opacity[ids][:, None] * torch.exp(torch.clamp(power, max=0.0))
            a = torch.where(mask_t[s:e], alpha, torch.zeros_like(alpha))  # [L, 256]
            one_minus = 1.0 - a
            Tb = torch.cumprod(torch.cat([torch.ones_like(one_minus[:1]), one_minus[:-1]], 0), 0)
            w = a * Tb
            if scores is not None:
                scores.index_add_(0, ids, (w * inside[None, :]).sum(1).detach())
            C = w.T @ color[ids]  # [256, 3]
            T_fin = Tb[-1] * one_minus[-1]
        else:
            C = torch.zeros(256, 3, dtype=torch.float64, device=dev)
            T_fin = torch.ones(256, dtype=torch.float64, device=dev)
        out_img.append((px[inside], py[inside], C[inside], T_fin[inside]))
    for px, py, C, T_fin in out_img:
        img = img.index_put((torch.zeros_like(px), py, px), C[:, 0] + T_fin * bg[0])
        img = img.index_put((torch.ones_like(px), py, px), C[:, 1] + T_fin * bg[1])
        img = img.index_put((torch.full_like(px, 2), py, px), C[:, 2] + T_fin * bg[2])
        fT = fT.index_put((py, px), T_fin)
    return img, fT


def rel_err(a, b) -> float:
    a = torch.as_tensor(np.asarray(a) if not torch.is_tensor(a) else a).double().cpu().flatten()
    b = torch.as_tensor(np.asarray(b) if not torch.is_tensor(b) else b).double().cpu().flatten()
    nb = float(b.norm())
    nd = float((a - b).norm())
    return nd / nb if nb > 0 else nd


def sh_norm_constant(l: int, m: int) -> float:
    """Orthonormal real-SH normalisation sqrt((2l+1)/(4 pi) (l-|m|)!/(l+|m|)!) (times sqrt(2) for m != 0)."""
    k = math.sqrt((2 * l + 1) / (4 * math.pi) * math.factorial(l - abs(m)) / math.factorial(l + abs(m)))
    return k * (math.sqrt(2.0) if m != 0 else 1.0)
