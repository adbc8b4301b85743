"""Tile binning for the toy2d rules, on the GPU: which Gaussians touch which 16x16 tile,
front to back (replaces toy2d/gs2d/binning.py:34-88, same `Bins` fields and meaning).

Rectangles follow getRect of the 3-sigma radius (float32, truncated, clamped to the grid);
each tile's list is in stable depth order (ties by index), which is the order the reference
obtains from argsort(tile * n + depth_rank). Lists, ranges and buckets are produced by
gs2d_rects_toy + gs_bin_fill_rect (a stable depth sort of the Gaussians, instance emission in
that order, and a stable sort by tile).
"""
from dataclasses import dataclass, field

import torch

from amdsplat import raster2d as R2
from amdsplat._lib import call, ptr

TILE = R2.TILE      # tile side in pixels; one workgroup per tile
BUCKET = R2.BUCKET  # list entries per bucket of the bucketed backward


@dataclass
class Bins:
    H: int
    W: int
    tiles_x: int
    tiles_y: int
    rect: torch.Tensor            # (N, 4) int32 xmin, ymin, xmax, ymax in tiles (max exclusive)
    order: torch.Tensor           # (N,) int64 Gaussian ids, front to back
    point_list: torch.Tensor      # (M,) int32 Gaussian id per (tile, Gaussian) pair, tile-major, front to back
    ranges: torch.Tensor          # (T, 2) int32 [start, end) into point_list per tile
    bucket_offsets: torch.Tensor  # (T,) int32 first bucket of each tile
    bucket_to_tile: torch.Tensor  # (B,) int32 tile of each bucket
    num_buckets: int
    bucket_offsets_ext: torch.Tensor = field(default=None, repr=False)  # (T + 1,) with the total

    def to(self, device):
        kw = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in self.__dict__.items()}
        return Bins(**kw)

    def offsets_ext(self) -> torch.Tensor:
        """bucket_offsets with the bucket count appended ([T + 1], as the kernels take it)."""
        if self.bucket_offsets_ext is None:
            tail = torch.tensor([self.num_buckets], dtype=torch.int32, device=self.bucket_offsets.device)
            self.bucket_offsets_ext = torch.cat([self.bucket_offsets.to(torch.int32), tail]).contiguous()
        return self.bucket_offsets_ext


@torch.no_grad()
def bin_gaussians(means: torch.Tensor, radii: torch.Tensor, depth: torch.Tensor, H: int, W: int) -> Bins:
    R2.require_cuda(means, radii, depth, names=("means", "radii", "depth"))
    dev = means.device
    n = means.shape[0]
    tiles_x, tiles_y = R2.tiles_of(W, H)
    m32 = means.detach().float().contiguous()
    r32 = radii.to(torch.int32).contiguous()
    rect = torch.empty(n, 4, dtype=torch.int32, device=dev)
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    call("gs2d_rects_toy", ptr(m32), ptr(r32), n, W, H, ptr(rect), ptr(counts), R2.stream(dev))
    rb = R2.bin_rects(rect, counts, depth, W, H, want_order=True)
    T = tiles_x * tiles_y
    return Bins(H, W, tiles_x, tiles_y, rect, rb.order.long(), rb.point_list, rb.ranges,
                rb.bucket_offsets[:T], rb.bucket_to_tile, rb.num_buckets, rb.bucket_offsets)
