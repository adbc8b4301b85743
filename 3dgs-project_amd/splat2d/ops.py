"""phase0 operator surface on the MI355X (replaces phase0/splat2d/ops.py:155-347 and the
extension functions of phase0/csrc/macrotile/bindings.cpp:156-239).

``render(means, chol, opacity_logit, colors, height, width, mode, depths)`` -> [H, W, 3].
``load_extension()`` returns an object with the extension's functions and return values:
    forward(means, chol, opacity_logit, colors, tile_offsets, tile_ids, bucket_offsets,
            bucket_tile, height, width) -> [image, t_final, n_contrib, last_contrib, ckpt]
    backward_pixel(grad_image, means, chol, opacity_logit, colors, tile_offsets, tile_ids,
                   bucket_offsets, bucket_tile, t_final, last_contrib, height, width)
    backward_splat(grad_image, means, chol, opacity_logit, colors, tile_offsets, tile_ids,
                   bucket_offsets, bucket_tile, image, ckpt, height, width)
        -> [d_means, d_chol, d_opacity_logit, d_colors]
    get_counters() / reset_counters(): atomic adds, checkpoint bytes and splat-pixel
        evaluations, counted by the GPU kernels (the reference counts them in its CPU twin,
        phase0/csrc/macrotile/splat2d_common.h:260-266).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch
from torch import Tensor

from amdsplat import raster2d as R2
from amdsplat._lib import call, ptr
from splat2d.reference import RefState, ref_render, ref_state  # noqa: F401  (the dense reference model)

Mode = Literal["pixel", "splat"]
MODES: tuple = ("pixel", "splat")

TILE = 16
TILE_PIXELS = TILE * TILE
BUCKET = 32
NUM_PARAMS = 9
CKPT_STRIDE = 4
ALPHA_MIN = 1.0 / 255.0
ALPHA_MAX = 0.99
T_STOP = 1e-4


@dataclass(frozen=True)
class TileBins:
    """CSR tile lists (splat ids in index order) and the 32-splat bucket tables."""

    tile_offsets: Tensor    # int32 [num_tiles + 1]
    tile_ids: Tensor        # int32 [tile_offsets[-1]]
    bucket_offsets: Tensor  # int32 [num_tiles + 1]
    bucket_tile: Tensor     # int32 [num_buckets]
    tiles_x: int
    tiles_y: int

    @property
    def num_buckets(self) -> int:
        return int(self.bucket_tile.numel())


def bin_tiles(means: Tensor, chol: Tensor, opacity_logit: Tensor, height: int, width: int) -> TileBins:
    """Tiles of each splat's alpha >= 1/255 ellipse bounding box (one pixel of slack), evaluated
    in float64 on the GPU; per-tile lists in index order."""
    R2.require_cuda(means, chol, opacity_logit, names=("means", "chol", "opacity_logit"))
    dev = means.device
    n = means.shape[0]
    dt = means.dtype if means.dtype in (torch.float32, torch.float64) else torch.float64
    m, c, o = (t.detach().to(dt).contiguous() for t in (means, chol, opacity_logit))
    rect = torch.empty(n, 4, dtype=torch.int32, device=dev)
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    call("gs2d_rects_phase0", R2.dtype_code(m), ptr(m), ptr(c), ptr(o), n, width, height, ptr(rect), ptr(counts),
         R2.stream(dev))
    rb = R2.bin_rects(rect, counts, None, width, height)
    tx, ty = R2.tiles_of(width, height)
    return TileBins(rb.tile_offsets, rb.point_list, rb.bucket_offsets, rb.bucket_to_tile, tx, ty)


class _Extension:
    def __init__(self):
        self._counters = None
        self._ckpt_bytes = 0
        # the GPU kernels count their atomic adds and splat-pixel evaluations (get_counters)
        # unless this is off; the reference's CUDA kernels count nothing, so timings of them
        # compare with this off
        self.counting = True

    def _ctr(self, device) -> Tensor | None:
        if not self.counting:
            return None
        if self._counters is None or self._counters.device != device:
            self._counters = torch.zeros(3, dtype=torch.int64, device=device)
        return self._counters

    @staticmethod
    def _scene(means, chol, opacity_logit, colors, tile_offsets, tile_ids, bucket_offsets, bucket_tile, height,
               width):
        R2.require_cuda(means, chol, opacity_logit, colors, tile_offsets, tile_ids, bucket_offsets, bucket_tile,
                        names=("means", "chol", "opacity_logit", "colors", "tile_offsets", "tile_ids",
                               "bucket_offsets", "bucket_tile"))
        if means.dim() != 2 or means.shape[1] != 2:
            raise RuntimeError("means must be [N, 2]")
        n = means.shape[0]
        if tuple(chol.shape) != (n, 3) or tuple(opacity_logit.shape) != (n,) or tuple(colors.shape) != (n, 3):
            raise RuntimeError("chol must be [N, 3], opacity_logit [N] and colors [N, 3]")
        if not (chol.dtype == opacity_logit.dtype == colors.dtype == means.dtype):
            raise RuntimeError("all splat parameters must share one floating dtype")
        for t in (tile_offsets, tile_ids, bucket_offsets, bucket_tile):
            if t.dtype != torch.int32:
                raise RuntimeError("tile/bucket tables must be int32")
        if height <= 0 or width <= 0:
            raise RuntimeError("image must be non-empty")
        tx, ty = R2.tiles_of(width, height)
        if tile_offsets.numel() != tx * ty + 1 or bucket_offsets.numel() != tx * ty + 1:
            raise RuntimeError("tile_offsets / bucket_offsets have the wrong length")
        rec = R2.pack(R2.PHASE0, means.contiguous(), chol.contiguous(), colors.contiguous(),
                      opacity_logit.contiguous())
        return rec, tile_offsets.contiguous(), tile_ids.contiguous(), bucket_offsets.contiguous(), \
            bucket_tile.contiguous()

    def forward(self, means, chol, opacity_logit, colors, tile_offsets, tile_ids, bucket_offsets, bucket_tile,
                height, width):
        rec, toff, tids, boff, btile = self._scene(means, chol, opacity_logit, colors, tile_offsets, tile_ids,
                                                   bucket_offsets, bucket_tile, height, width)
        nb = int(btile.numel())
        ctr = self._ctr(rec.device)
        image, t_final, n_contrib, last_contrib, _, ckpt = R2.blend_fwd(
            R2.PHASE0, rec, toff, 1, tids, boff, nb, int(width), int(height), save_ckpt=True, counters=ctr)
        self._ckpt_bytes += nb * TILE_PIXELS * CKPT_STRIDE * rec.element_size()
        return [image, t_final, n_contrib, last_contrib, ckpt]

    def backward_pixel(self, grad_image, means, chol, opacity_logit, colors, tile_offsets, tile_ids,
                       bucket_offsets, bucket_tile, t_final, last_contrib, height, width):
        rec, toff, tids, _, _ = self._scene(means, chol, opacity_logit, colors, tile_offsets, tile_ids,
                                            bucket_offsets, bucket_tile, height, width)
        g_img = grad_image.contiguous().to(rec.dtype)
        if tuple(g_img.shape) != (height, width, 3):
            raise RuntimeError("grad_image must be [H, W, 3]")
        g = R2.blend_bwd_pixel(R2.PHASE0, rec, toff, 1, tids, int(width), int(height), None,
                               t_final.contiguous(), last_contrib.contiguous().to(torch.int32), g_img,
                               counters=self._ctr(rec.device))
        dm, dc, dl, dcol = R2.split_grads(g)
        return [dm, dc, dl, dcol]

    def backward_splat(self, grad_image, means, chol, opacity_logit, colors, tile_offsets, tile_ids, bucket_offsets,
                       bucket_tile, image, ckpt, height, width, last_contrib=None, tile_max=None):
        rec, toff, tids, boff, btile = self._scene(means, chol, opacity_logit, colors, tile_offsets, tile_ids,
                                                   bucket_offsets, bucket_tile, height, width)
        g_img = grad_image.contiguous().to(rec.dtype)
        if tuple(g_img.shape) != (height, width, 3):
            raise RuntimeError("grad_image must be [H, W, 3]")
        nb = int(btile.numel())
        if ckpt.shape[0] != nb:
            raise RuntimeError("ckpt must have one slot per bucket")
        # without last_contrib (the reference's signature has none) each pixel replays its
        # buckets and stops by the T < 1e-4 rule; with it, buckets past the pixel are skipped
        lim = None if last_contrib is None else last_contrib.contiguous().to(torch.int32)
        g = R2.blend_bwd_bucket(R2.PHASE0, rec, toff, 1, tids, boff, btile, nb, int(width), int(height),
                                image.contiguous(), g_img, lim, tile_max, ckpt.contiguous(),
                                counters=self._ctr(rec.device))
        dm, dc, dl, dcol = R2.split_grads(g)
        return [dm, dc, dl, dcol]

    def get_counters(self) -> dict:
        c = [0, 0, 0] if self._counters is None else [int(x) for x in self._counters.cpu().tolist()]
        return {"atomic_adds": c[0], "checkpoint_bytes": self._ckpt_bytes, "splat_pixel_evals": c[2]}

    def reset_counters(self) -> None:
        if self._counters is not None:
            self._counters.zero_()
        self._ckpt_bytes = 0


_EXT: _Extension | None = None


def load_extension(with_cuda: bool | None = None, verbose: bool = False) -> _Extension:
    """The compiled extension (libamdsplat.so, loaded on first use). There is no CPU build:
    `with_cuda=False` raises."""
    global _EXT
    if with_cuda is False:
        raise RuntimeError("splat2d runs on the GPU only (there is no CPU extension)")
    if _EXT is None:
        from amdsplat import _lib

        _lib.lib()
        _EXT = _Extension()
    return _EXT


class _Splat2dFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, chol, opacity_logit, colors, bins: TileBins, height: int, width: int, mode: str):
        ext = load_extension()
        image, t_final, _n_contrib, last_contrib, ckpt = ext.forward(
            means, chol, opacity_logit, colors, bins.tile_offsets, bins.tile_ids, bins.bucket_offsets,
            bins.bucket_tile, height, width)
        ctx.save_for_backward(means, chol, opacity_logit, colors, image, t_final, last_contrib, ckpt)
        ctx.bins, ctx.height, ctx.width, ctx.mode = bins, height, width, mode
        return image

    @staticmethod
    def backward(ctx, grad_image):
        means, chol, opacity_logit, colors, image, t_final, last_contrib, ckpt = ctx.saved_tensors
        b: TileBins = ctx.bins
        ext = load_extension()
        tables = (b.tile_offsets, b.tile_ids, b.bucket_offsets, b.bucket_tile)
        if ctx.mode == "pixel":
            g = ext.backward_pixel(grad_image, means, chol, opacity_logit, colors, *tables, t_final, last_contrib,
                                   ctx.height, ctx.width)
        else:
            g = ext.backward_splat(grad_image, means, chol, opacity_logit, colors, *tables, image, ckpt, ctx.height,
                                   ctx.width, last_contrib=last_contrib)
        return g[0], g[1], g[2], g[3], None, None, None, None


def render(means: Tensor, chol: Tensor, opacity_logit: Tensor, colors: Tensor, height: int, width: int,
           mode: Mode = "splat", depths: Tensor | None = None) -> Tensor:
    """Render an [H, W, 3] image. Splats are taken in index order unless ``depths`` is given."""
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
    if depths is not None:
        order = torch.argsort(depths, stable=True)
        means, chol = means[order], chol[order]
        opacity_logit, colors = opacity_logit[order], colors[order]
    bins = bin_tiles(means, chol, opacity_logit, height, width)
    return _Splat2dFunction.apply(means, chol, opacity_logit, colors, bins, height, width, mode)
