"""Writes the golden fixtures of the 2D surfaces by running the reference's own Python code
in this container (toy2d/gs2d and phase0/splat2d, read from the reference tree; nothing of it
is copied or shipped -- only the input/output arrays are saved).

What the fixtures pin, and why an import was needed: the reference's binning
(toy2d/gs2d/binning.py:34-88, phase0/splat2d/ops.py:206-255) defines the tile lists bit for
bit, and its dense float64 renderers (toy2d/gs2d/reference.py:22-58,
phase0/splat2d/ops.py:350-398) with autograd give the images and gradients the references'
own GPU tests compare against (toy2d/tests/test_cuda.py, phase0/tests/gradcheck). The scenes
are the references' test scenes (toy2d/tests/scenes.py:8-43,
phase0/tests/gradcheck/conftest.py:23-163), rebuilt here with the same seeds.

    python tests/golden/make_golden.py            # needs /root/reference and torch (CPU)
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent


def toy2d_fixtures():
    sys.path.insert(0, str(REF / "toy2d"))
    from gs2d import Gaussians2D, bin_gaussians, render_reference  # reference code, read in place
    from gs2d.params import radii_from_cov

    scenes = {"tiny": (12, 18, 20, 1.5, 0.0, 4), "sparse_odd": (60, 37, 41, 1.0, 0.0, 1),
              "dense": (300, 20, 20, 6.0, 0.0, 2), "opaque": (80, 32, 48, 1.5, 6.0, 3)}
    bg = (0.2, 0.5, 0.8)
    for name, (n, H, W, scale_mult, op_shift, seed) in scenes.items():
        g = Gaussians2D(n, H, W, seed=seed, dtype=torch.float64)
        with torch.no_grad():
            g.log_scale += torch.log(torch.tensor(scale_mult, dtype=torch.float64))
            g.opacity_logit += op_shift
        means, conic, color, opacity, cov = (t.detach() for t in g.activated())
        radii = radii_from_cov(cov)
        bins = bin_gaussians(means, radii, g.depth, H, W)
        leaves = [t.clone().requires_grad_(True) for t in (means, conic, color, opacity)]
        bgt = torch.tensor(bg, dtype=torch.float64)
        img = render_reference(*leaves, bins, bgt)
        dout = torch.randn(3, H, W, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
        grads = torch.autograd.grad(img, leaves, dout)
        np.savez_compressed(
            OUT / f"toy2d_{name}.npz", H=H, W=W, bg=np.array(bg), means=means.numpy(), conic=conic.numpy(),
            color=color.numpy(), opacity=opacity.numpy(), depth=g.depth.numpy(), radii=radii.numpy(),
            rect=bins.rect.numpy(), order=bins.order.numpy(), point_list=bins.point_list.numpy(),
            ranges=bins.ranges.numpy(), bucket_offsets=bins.bucket_offsets.numpy(),
            bucket_to_tile=bins.bucket_to_tile.numpy(), num_buckets=bins.num_buckets, image=img.detach().numpy(),
            dout=dout.numpy(), g_means=grads[0].numpy(), g_conic=grads[1].numpy(), g_color=grads[2].numpy(),
            g_opacity=grads[3].numpy())
        print(f"toy2d {name}: n={n} pairs={bins.point_list.numel()} buckets={bins.num_buckets}")
    sys.path.pop(0)


def phase0_fixtures():
    sys.path.insert(0, str(REF / "phase0"))
    from splat2d.ops import bin_tiles, ref_render, ref_state  # reference code, read in place

    def uniform(g, lo, hi, *shape):
        return lo + (hi - lo) * torch.rand(*shape, generator=g, dtype=torch.float64)

    def make(name, seed, n, H, W, sigma, opacity, box=(0.3, 0.7)):
        g = torch.Generator().manual_seed(seed)
        means = torch.stack([uniform(g, box[0] * W, box[1] * W, n), uniform(g, box[0] * H, box[1] * H, n)], -1)
        l0 = 1.0 / uniform(g, sigma[0], sigma[1], n)
        l2 = 1.0 / uniform(g, sigma[0], sigma[1], n)
        l1 = uniform(g, -0.3, 0.3, n) * torch.minimum(l0, l2)
        o = uniform(g, opacity[0], opacity[1], n)
        colors = uniform(g, 0.05, 0.95, n, 3)
        return name, means, torch.stack([l0, l1, l2], -1), torch.log(o / (1 - o)), colors, H, W

    scenes = [make(f"seed{s}_n{n}", s, n, 32, 32, (22.0, 40.0), (0.05, 0.2)) for s in (0, 1, 2) for n in (8, 32)]
    scenes.append(make("dense_n96", 7, 96, 32, 32, (30.0, 45.0), (0.02, 0.06)))
    base = make("sparse_n150", 11, 144, 40, 56, (1.5, 6.0), (0.2, 0.9), box=(-0.05, 1.05))
    k = 6
    scenes.append(("sparse_n150",
                   torch.cat([torch.tensor([[20.3, 17.7]], dtype=torch.float64).repeat(k, 1), base[1]]),
                   torch.cat([torch.tensor([[1 / 4.0, 0.01, 1 / 5.0]], dtype=torch.float64).repeat(k, 1), base[2]]),
                   torch.cat([torch.full((k,), math.log(0.999 / 0.001), dtype=torch.float64), base[3]]),
                   torch.cat([torch.linspace(0.1, 0.9, 3 * k, dtype=torch.float64).reshape(k, 3), base[4]]),
                   base[5], base[6]))
    for name, means, chol, logit, colors, H, W in scenes:
        bins = bin_tiles(means, chol, logit, H, W)
        st = ref_state(means, chol, logit, colors, H, W)
        gi = torch.randn(H, W, 3, generator=torch.Generator().manual_seed(sum(map(ord, name)) + 12345),
                         dtype=torch.float64)
        leaves = [t.clone().requires_grad_(True) for t in (means, chol, logit, colors)]
        grads = torch.autograd.grad(ref_render(*leaves, H, W), leaves, gi)
        np.savez_compressed(
            OUT / f"phase0_{name}.npz", H=H, W=W, means=means.numpy(), chol=chol.numpy(), opacity_logit=logit.numpy(),
            colors=colors.numpy(), tile_offsets=bins.tile_offsets.numpy(), tile_ids=bins.tile_ids.numpy(),
            bucket_offsets=bins.bucket_offsets.numpy(), bucket_tile=bins.bucket_tile.numpy(),
            image=st.image.detach().numpy(), t_final=st.t_final.detach().numpy(),
            n_contrib=st.contributes.sum(-1).numpy().astype(np.int32), grad_image=gi.numpy(),
            g_means=grads[0].numpy(), g_chol=grads[1].numpy(), g_opacity_logit=grads[2].numpy(),
            g_colors=grads[3].numpy())
        print(f"phase0 {name}: n={means.shape[0]} ids={bins.tile_ids.numel()} buckets={bins.num_buckets}")
    sys.path.pop(0)


if __name__ == "__main__":
    toy2d_fixtures()
    phase0_fixtures()
