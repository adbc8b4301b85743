"""Host side of the 2D surfaces: thin wrappers over the C ABI shared by `gs2d` (toy2d rules)
and `splat2d` (phase0 rules). Every function enqueues HIP kernels on the current torch
stream; PyTorch owns all device memory. Nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call, ptr

TILE = 16
BUCKET = 32
TILE_PIXELS = TILE * TILE
REC_FLOATS = 16
GRAD_FLOATS = 12
TOY2D, PHASE0 = 1, 2
F32, F64 = 0, 1


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float64:
        return F64
    raise TypeError(f"expected a float32 or float64 tensor, got {t.dtype}")


def require_cuda(*tensors, names=None):
    for k, t in enumerate(tensors):
        if t is not None and t.device.type != "cuda":
            name = names[k] if names else f"argument {k}"
            raise RuntimeError(f"{name} must be a CUDA (ROCm) tensor: this rasterizer runs on the GPU only")


def _u8(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def tiles_of(width: int, height: int) -> tuple[int, int]:
    return (width + TILE - 1) // TILE, (height + TILE - 1) // TILE


def stream(device) -> int | None:
    return _lib.stream_handle(device)


def bg_array(bg):
    if bg is None:
        return None
    vals = bg.detach().cpu().double().reshape(-1).tolist() if torch.is_tensor(bg) else [float(x) for x in bg]
    if len(vals) != 3:
        raise ValueError("bg must have 3 values")
    return (C.c_double * 3)(*vals)


@dataclass
class RectBins:
    """Output of rectangle binning (all int32 CUDA tensors)."""

    point_list: torch.Tensor      # [m]
    ranges: torch.Tensor          # [T, 2] CSR [start, end)
    tile_offsets: torch.Tensor    # [T + 1]
    bucket_offsets: torch.Tensor  # [T + 1]
    bucket_to_tile: torch.Tensor  # [B]
    order: torch.Tensor | None    # [n] stable argsort of depth (if asked for)
    num_buckets: int


# Tile binning of the 2D surfaces: "auto" (the library's choice by size), "spans" or "radix".
BINNING = "auto"


def bin_rects(rects: torch.Tensor, counts: torch.Tensor, depth: torch.Tensor | None, width: int, height: int,
              want_order: bool = False, binning: str | None = None) -> RectBins:
    """Per-tile lists of the Gaussians whose tile rectangle covers the tile, in stable depth
    order (depth given) or index order. Two host reads: the instance and bucket counts.
    binning: "auto", "spans" or "radix" (default: the module's BINNING); the lists are the same."""
    flags = _lib.BIN_FLAGS[binning or BINNING]
    dev = rects.device
    n = rects.shape[0]
    tx, ty = tiles_of(width, height)
    T = tx * ty
    st = stream(dev)
    if n > 0:
        # the instance count, summed on the library's side stream and read without draining st
        call("gs_count_begin", ptr(counts), n, 0, st)
        mv = C.c_uint64()
        call("gs_count_end", C.byref(mv))
        m = int(mv.value)
    else:
        m = 0
    point_list = torch.empty(m, dtype=torch.int32, device=dev)
    ranges = torch.empty(T, 2, dtype=torch.int32, device=dev)
    tile_offsets = torch.empty(T + 1, dtype=torch.int32, device=dev)
    boff = torch.empty(T + 1, dtype=torch.int32, device=dev)
    order = torch.empty(n, dtype=torch.int32, device=dev) if want_order else None
    d = None
    dcode = F32
    if depth is not None:
        d = depth.detach().contiguous()
        if d.dtype not in (torch.float32, torch.float64):
            d = d.float()
        dcode = dtype_code(d)
    ws = _u8(_lib.size_call("gs_bin_workspace_size", n, m, tx, ty, flags), dev)
    call("gs_bin_fill_rect", ptr(rects), ptr(d), dcode, ptr(counts), n, tx, ty, m, None, ptr(point_list), ptr(ranges),
         ptr(tile_offsets), ptr(boff), ptr(order), flags, ptr(ws), ws.numel(), st)
    nb = int(boff[T].item())
    b2t = torch.empty(max(nb, 1), dtype=torch.int32, device=dev)
    call("gs_bucket_fill", ptr(boff), T, ptr(b2t), nb, st)
    return RectBins(point_list, ranges, tile_offsets, boff, b2t[:nb], order, nb)


def pack(rules: int, means, shape, color, opacity) -> torch.Tensor:
    """Splat records [n, 16] (dtype of means) for the blend kernels."""
    n = means.shape[0]
    rec = torch.empty(n, REC_FLOATS, dtype=means.dtype, device=means.device)
    call("gs2d_pack", rules, dtype_code(means), ptr(means), ptr(shape), ptr(color), ptr(opacity), n, ptr(rec),
         stream(means.device))
    return rec


def blend_fwd(rules: int, rec: torch.Tensor, ranges: torch.Tensor, range_stride: int, point_list: torch.Tensor,
              bucket_offsets: torch.Tensor | None, num_buckets: int, width: int, height: int, bg=None,
              save_ckpt: bool = True, counters: torch.Tensor | None = None):
    """Returns (image, final_T, n_contrib, last_contrib, tile_max, ckpt)."""
    dev = rec.device
    dt = rec.dtype
    tx, ty = tiles_of(width, height)
    shape = (3, height, width) if rules == TOY2D else (height, width, 3)
    # every output is written whole by the kernel (each pixel, each tile, each bucket slot)
    image = torch.empty(shape, dtype=dt, device=dev)
    final_T = torch.empty(height, width, dtype=dt, device=dev)
    n_contrib = torch.empty(height, width, dtype=torch.int32, device=dev)
    last_contrib = torch.empty(height, width, dtype=torch.int32, device=dev)
    tile_max = torch.empty(tx * ty, dtype=torch.int32, device=dev)
    if save_ckpt:
        ckpt = torch.empty(num_buckets, TILE_PIXELS, 4, dtype=dt, device=dev)
    else:
        ckpt = torch.empty(0, dtype=dt, device=dev)
    call("gs2d_blend_fwd", rules, dtype_code(rec), ptr(rec), ptr(ranges), range_stride, ptr(point_list),
         ptr(bucket_offsets) if save_ckpt else None, width, height, bg_array(bg), ptr(image), ptr(final_T),
         ptr(n_contrib), ptr(last_contrib), ptr(tile_max), ptr(ckpt) if save_ckpt else None, ptr(counters),
         stream(dev))
    return image, final_T, n_contrib, last_contrib, tile_max, ckpt


def blend_bwd_bucket(rules: int, rec, ranges, range_stride, point_list, bucket_offsets, bucket_to_tile,
                     num_buckets: int, width: int, height: int, image, grad_image, limit, tile_max, ckpt,
                     counters=None) -> torch.Tensor:
    """Bucketed backward; returns grad_rec [n, 12] (dtype of rec)."""
    dev = rec.device
    n = rec.shape[0]
    g = torch.empty(n, GRAD_FLOATS, dtype=rec.dtype, device=dev)
    call("gs2d_blend_bwd_bucket", rules, dtype_code(rec), ptr(rec), ptr(ranges), range_stride, ptr(point_list),
         ptr(bucket_offsets), ptr(bucket_to_tile), num_buckets, n, width, height, ptr(image), ptr(grad_image),
         ptr(limit), ptr(tile_max), ptr(ckpt), ptr(g), ptr(counters), stream(dev))
    return g


def blend_bwd_pixel(rules: int, rec, ranges, range_stride, point_list, width: int, height: int, bg, final_T, limit,
                    grad_image, counters=None) -> torch.Tensor:
    dev = rec.device
    n = rec.shape[0]
    g = torch.empty(n, GRAD_FLOATS, dtype=rec.dtype, device=dev)
    call("gs2d_blend_bwd_pixel", rules, dtype_code(rec), ptr(rec), ptr(ranges), range_stride, ptr(point_list), n,
         width, height, bg_array(bg), ptr(final_T), ptr(limit), ptr(grad_image), ptr(g), ptr(counters), stream(dev))
    return g


def split_grads(g: torch.Tensor):
    """(dmeans [n,2], dshape [n,3], dopacity [n], dcolor [n,3]) from a grad record [n,12]
    (one launch)."""
    n = g.shape[0]
    dm = torch.empty(n, 2, dtype=g.dtype, device=g.device)
    ds = torch.empty(n, 3, dtype=g.dtype, device=g.device)
    dop = torch.empty(n, dtype=g.dtype, device=g.device)
    dc = torch.empty(n, 3, dtype=g.dtype, device=g.device)
    if n:
        call("gs2d_unpack_grads", dtype_code(g), ptr(g), n, ptr(dm), ptr(ds), ptr(dop), ptr(dc), stream(g.device))
    return dm, ds, dop, dc
