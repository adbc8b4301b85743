"""Differentiable toy2d-rule rasterizer on the MI355X (replaces toy2d/gs2d/raster.py:14-64 and
the extension functions of toy2d/csrc/rasterize.cu:366-454).

`ext()` returns an object with the reference extension's three functions and return values:
    forward(means, conic, color, opacity, bg, ranges, point_list, bucket_offsets, num_buckets,
            H, W, save_buckets) -> [out (3,H,W), final_T (H,W), n_contrib (H,W), bucket_state (B,256,4)]
    backward_pixel(means, conic, color, opacity, bg, ranges, point_list, final_T, n_contrib, dL_dout)
    backward_splat(means, conic, color, opacity, bg, ranges, point_list, bucket_offsets,
                   bucket_to_tile, out, final_T, n_contrib, bucket_state, dL_dout)
        -> [dmeans, dconic, dcolor, dopacity]
Inputs are CUDA tensors; float32 as in the reference, float64 also accepted.
"""
import torch

from amdsplat import raster2d as R2

from .binning import Bins
from .reference import render_reference


def _check(means, conic, color, opacity):
    R2.require_cuda(means, conic, color, opacity, names=("means", "conic", "color", "opacity"))
    n = means.shape[0]
    for name, t, shape in (("means", means, (n, 2)), ("conic", conic, (n, 3)), ("color", color, (n, 3)),
                           ("opacity", opacity, (n,))):
        if tuple(t.shape) != shape:
            raise RuntimeError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
        if t.dtype != means.dtype:
            raise RuntimeError(f"{name} must have dtype {means.dtype}")
    R2.dtype_code(means)


def _pack(means, conic, color, opacity):
    _check(means, conic, color, opacity)
    return R2.pack(R2.TOY2D, means.contiguous(), conic.contiguous(), color.contiguous(), opacity.contiguous())


class _Ext:
    """The reference extension's functions (rasterize_forward / _backward_pixel / _backward_splat)."""

    @staticmethod
    def forward(means, conic, color, opacity, bg, ranges, point_list, bucket_offsets, num_buckets, H, W,
                save_buckets):
        rec = _pack(means, conic, color, opacity)
        # (the kernels read each tile's first bucket only: no appended total is needed)
        boff = bucket_offsets.to(torch.int32).contiguous() if save_buckets else None
        out, final_T, n_contrib, _, _, ckpt = R2.blend_fwd(
            R2.TOY2D, rec, ranges.contiguous(), 2, point_list.contiguous(), boff, int(num_buckets), int(W), int(H),
            bg=bg, save_ckpt=bool(save_buckets))
        return [out, final_T, n_contrib, ckpt]

    @staticmethod
    def backward_pixel(means, conic, color, opacity, bg, ranges, point_list, final_T, n_contrib, dL_dout):
        rec = _pack(means, conic, color, opacity)
        H, W = final_T.shape
        g = R2.blend_bwd_pixel(R2.TOY2D, rec, ranges.contiguous(), 2, point_list.contiguous(), W, H, bg,
                               final_T.contiguous(), n_contrib.contiguous(), dL_dout.contiguous().to(rec.dtype))
        dm, dc, dop, dcol = R2.split_grads(g)
        return [dm, dc, dcol, dop]

    @staticmethod
    def backward_splat(means, conic, color, opacity, bg, ranges, point_list, bucket_offsets, bucket_to_tile, out,
                       final_T, n_contrib, bucket_state, dL_dout, tile_max=None, offsets_ext=None):
        rec = _pack(means, conic, color, opacity)
        H, W = final_T.shape
        nb = int(bucket_to_tile.shape[0])
        boff = offsets_ext if offsets_ext is not None else bucket_offsets.to(torch.int32).contiguous()
        g = R2.blend_bwd_bucket(R2.TOY2D, rec, ranges.contiguous(), 2, point_list.contiguous(), boff,
                                bucket_to_tile.contiguous(), nb, W, H, out.contiguous(),
                                dL_dout.contiguous().to(rec.dtype), n_contrib.contiguous(), tile_max,
                                bucket_state.contiguous())
        dm, dc, dop, dcol = R2.split_grads(g)
        return [dm, dc, dcol, dop]


_EXT = _Ext()


def ext() -> _Ext:
    """The compiled rasterizer (libamdsplat.so is loaded on first use; raises if not built)."""
    from amdsplat import _lib

    _lib.lib()
    return _EXT


class _Rasterize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, conic, color, opacity, bg, bins: Bins, mode: str):
        rec = _pack(means, conic, color, opacity)
        save = mode == "splat"
        boff = bins.offsets_ext() if save else None
        out, final_T, n_contrib, _, tile_max, bstate = R2.blend_fwd(
            R2.TOY2D, rec, bins.ranges, 2, bins.point_list, boff, bins.num_buckets, bins.W, bins.H, bg=bg,
            save_ckpt=save)
        ctx.bins, ctx.mode = bins, mode
        ctx.save_for_backward(rec, bg, out, final_T, n_contrib, tile_max, bstate)
        return out

    @staticmethod
    def backward(ctx, dout):
        rec, bg, out, final_T, n_contrib, tile_max, bstate = ctx.saved_tensors
        b = ctx.bins
        dout = dout.contiguous().to(rec.dtype)
        if ctx.mode == "pixel":
            g = R2.blend_bwd_pixel(R2.TOY2D, rec, b.ranges, 2, b.point_list, b.W, b.H, bg, final_T, n_contrib, dout)
        else:
            g = R2.blend_bwd_bucket(R2.TOY2D, rec, b.ranges, 2, b.point_list, b.offsets_ext(), b.bucket_to_tile,
                                    b.num_buckets, b.W, b.H, out, dout, n_contrib, tile_max, bstate)
        dmeans, dconic, dopacity, dcolor = R2.split_grads(g)
        return dmeans, dconic, dcolor, dopacity, None, None, None


def rasterize(means, conic, color, opacity, bins: Bins, bg=None, backend: str = "splat"):
    """Render a (3, H, W) image. backend: 'splat' (HIP, bucketed backward), 'pixel' (HIP,
    per-pixel backward) or 'ref' (render_reference: dense PyTorch ops on the tensors' device,
    autograd gradients; only when asked for by name)."""
    if bg is None:
        bg = torch.zeros(3, dtype=means.dtype, device=means.device)
    if backend == "ref":
        return render_reference(means, conic, color, opacity, bins, bg)
    if backend not in ("pixel", "splat"):
        raise ValueError(f"unknown backend {backend!r}")
    return _Rasterize.apply(means, conic, color, opacity, bg, bins, backend)
