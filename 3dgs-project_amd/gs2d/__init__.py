"""Drop-in for the toy2d `gs2d` package (toy2d/gs2d/__init__.py): 2D Gaussians, tile binning
and the differentiable tile rasterizer, running on the MI355X through libamdsplat.so.

    from gs2d import Gaussians2D, bin_gaussians, rasterize
    from gs2d.params import radii_from_cov
    means, conic, color, opacity, cov = model.activated()
    bins = bin_gaussians(means, radii_from_cov(cov.detach()), model.depth, H, W)
    img = rasterize(means, conic, color, opacity, bins, backend="splat")   # [3, H, W]

Binning runs on the GPU (the reference's runs as PyTorch ops); backends "splat" (bucketed
backward) and "pixel" (per-pixel backward) are HIP kernels. `render_reference` (backend "ref")
is the dense PyTorch ground truth of the same rules, on whatever device its inputs are.
"""
from .binning import BUCKET, TILE, Bins, bin_gaussians
from .params import Gaussians2D
from .raster import rasterize
from .reference import render_reference

__all__ = ["Gaussians2D", "Bins", "bin_gaussians", "TILE", "BUCKET", "render_reference", "rasterize"]
