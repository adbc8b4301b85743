"""ctypes wrappers of the 2D oracle (oracle2d.c in liboracle.so) and of the reference's own
phase0 CPU twin (oracle/_ref/libsplat2d_ref.so, built by ref.mk when the reference tree is
present).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product packages. All arrays are numpy, on the host.

Layouts follow the GPU entry points: rules 1 = toy2d (image [3,H,W], background, checkpoint
(T, C), n_contrib = last position + 1), rules 2 = phase0 (image [H,W,3], checkpoint (C, T),
n_contrib = count, last_contrib = last position + 1).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

import oracle as O

HERE = Path(__file__).resolve().parent
REF_LIB = HERE / "_ref" / "libsplat2d_ref.so"
TOY2D, PHASE0 = 1, 2


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _sfx(dtype):
    return "f64" if np.dtype(dtype) == np.float64 else "f32"


def _lib():
    L = O.lib()
    if not getattr(L, "_or2d_ready", False):
        for s in ("f32", "f64"):
            getattr(L, f"or2d_forward_{s}").restype = C.c_int64
            getattr(L, f"or2d_backward_bucket_{s}").restype = C.c_int64
            getattr(L, f"or2d_backward_pixel_{s}").restype = C.c_int64
        L.or2d_bin.restype = C.c_int64
        L.or_exp_f32.restype = C.c_float
        L.or_exp_f32.argtypes = [C.c_float]
        L.or_exp_f64.restype = C.c_double
        L.or_exp_f64.argtypes = [C.c_double]
        L.or_log_f64.restype = C.c_double
        L.or_log_f64.argtypes = [C.c_double]
        L._or2d_ready = True
    return L


def exp_f32(x: float) -> float:
    return float(_lib().or_exp_f32(C.c_float(x)))


def exp_f64(x: float) -> float:
    return float(_lib().or_exp_f64(C.c_double(x)))


def log_f64(x: float) -> float:
    return float(_lib().or_log_f64(C.c_double(x)))


def tiles(W, H):
    return (W + 15) // 16, (H + 15) // 16


def rects_toy(means, radii, W, H):
    means = np.ascontiguousarray(means, np.float32)
    radii = np.ascontiguousarray(radii, np.int32)
    n = len(radii)
    rects = np.zeros((n, 4), np.int32)
    counts = np.zeros(n, np.uint32)
    _lib().or2d_rects_toy(_p(means), _p(radii), C.c_int64(n), C.c_int(W), C.c_int(H), _p(rects), _p(counts))
    return rects, counts


def rects_phase0(means, chol, logit, W, H):
    dt = np.asarray(means).dtype if np.asarray(means).dtype == np.float64 else np.float32
    means, chol, logit = (np.ascontiguousarray(a, dt) for a in (means, chol, logit))
    n = len(logit)
    rects = np.zeros((n, 4), np.int32)
    counts = np.zeros(n, np.uint32)
    getattr(_lib(), f"or2d_rects_phase0_{_sfx(dt)}")(_p(means), _p(chol), _p(logit), C.c_int64(n), C.c_int(W),
                                                      C.c_int(H), _p(rects), _p(counts))
    return rects, counts


def bin_rects(rects, depth, W, H):
    """Per-tile lists. depth: None (index order), float32 or float64 array.
    Returns (order, point_list, ranges [T,2], bucket_offsets [T+1])."""
    tx, ty = tiles(W, H)
    rects = np.ascontiguousarray(rects, np.int32)
    n = len(rects)
    d32 = d64 = None
    if depth is not None:
        depth = np.asarray(depth)
        if depth.dtype == np.float64:
            d64 = np.ascontiguousarray(depth)
        else:
            d32 = np.ascontiguousarray(depth, np.float32)
    m_est = int(np.maximum(rects[:, 2] - rects[:, 0], 0).astype(np.int64) @ np.maximum(rects[:, 3] - rects[:, 1], 0))
    order = np.zeros(max(n, 1), np.uint32)
    pl = np.zeros(max(m_est, 1), np.uint32)
    ranges = np.zeros((tx * ty, 2), np.uint32)
    boff = np.zeros(tx * ty + 1, np.uint32)
    m = _lib().or2d_bin(_p(rects), _p(d32), _p(d64), C.c_int64(n), C.c_int(tx), C.c_int(ty), _p(order), _p(pl),
                        _p(ranges), _p(boff))
    assert m == m_est
    return order[:n], pl[:m], ranges, boff


def forward(rules, means, shape, color, opac, point_list, ranges, boff, W, H, bg=None, with_ckpt=True):
    dt = np.asarray(means).dtype
    dt = np.float64 if dt == np.float64 else np.float32
    means, shape, color, opac = (np.ascontiguousarray(a, dt) for a in (means, shape, color, opac))
    image = np.zeros((3, H, W) if rules == TOY2D else (H, W, 3), dt)
    final_T = np.zeros((H, W), dt)
    n_contrib = np.zeros((H, W), np.int32)
    last_contrib = np.zeros((H, W), np.int32)
    nb = int(boff[-1])
    ckpt = np.zeros((max(nb, 1), 256, 4), dt) if with_ckpt else None
    bgd = None if bg is None else np.ascontiguousarray(bg, np.float64)
    evals = getattr(_lib(), f"or2d_forward_{_sfx(dt)}")(
        C.c_int(rules), _p(means), _p(shape), _p(color), _p(opac), _p(np.ascontiguousarray(ranges, np.uint32)),
        _p(np.ascontiguousarray(point_list, np.uint32)), _p(np.ascontiguousarray(boff, np.uint32)), C.c_int(W),
        C.c_int(H), _p(bgd), _p(image), _p(final_T), _p(n_contrib), _p(last_contrib), _p(ckpt))
    return dict(image=image, final_T=final_T, n_contrib=n_contrib, last_contrib=last_contrib, ckpt=ckpt,
                evals=int(evals))


def backward_bucket(rules, means, shape, color, opac, point_list, ranges, boff, W, H, image, grad_image, limit,
                    ckpt):
    """Returns (grad_rec [n,12] float64, number of atomics)."""
    dt = np.float64 if np.asarray(means).dtype == np.float64 else np.float32
    means, shape, color, opac, image, grad_image, ckpt = (np.ascontiguousarray(a, dt) for a in
                                                          (means, shape, color, opac, image, grad_image, ckpt))
    n = len(opac)
    g = np.zeros((max(n, 1), 12), np.float64)
    at = getattr(_lib(), f"or2d_backward_bucket_{_sfx(dt)}")(
        C.c_int(rules), _p(means), _p(shape), _p(color), _p(opac), C.c_int64(n),
        _p(np.ascontiguousarray(ranges, np.uint32)), _p(np.ascontiguousarray(point_list, np.uint32)),
        _p(np.ascontiguousarray(boff, np.uint32)), C.c_int(W), C.c_int(H), _p(image), _p(grad_image),
        _p(np.ascontiguousarray(limit, np.int32)), _p(ckpt), _p(g))
    return g[:n], int(at)


def backward_pixel(rules, means, shape, color, opac, point_list, ranges, W, H, final_T, limit, grad_image, bg=None):
    dt = np.float64 if np.asarray(means).dtype == np.float64 else np.float32
    means, shape, color, opac, final_T, grad_image = (np.ascontiguousarray(a, dt) for a in
                                                      (means, shape, color, opac, final_T, grad_image))
    n = len(opac)
    g = np.zeros((max(n, 1), 12), np.float64)
    bgd = None if bg is None else np.ascontiguousarray(bg, np.float64)
    at = getattr(_lib(), f"or2d_backward_pixel_{_sfx(dt)}")(
        C.c_int(rules), _p(means), _p(shape), _p(color), _p(opac), C.c_int64(n),
        _p(np.ascontiguousarray(ranges, np.uint32)), _p(np.ascontiguousarray(point_list, np.uint32)), C.c_int(W),
        C.c_int(H), _p(bgd), _p(final_T), _p(np.ascontiguousarray(limit, np.int32)), _p(grad_image), _p(g))
    return g[:n], int(at)


# ---------------------------------------------------------------------------------------
# The reference's own phase0 CPU twin (oracle/_ref)
# ---------------------------------------------------------------------------------------
_ref = None


def ref_available() -> bool:
    return REF_LIB.exists()


def _reflib():
    global _ref
    if _ref is None:
        _ref = C.CDLL(str(REF_LIB))
    return _ref


def ref_forward(means, chol, logit, colors, tile_offsets, tile_ids, bucket_offsets, bucket_tile, H, W):
    dt = np.float64 if np.asarray(means).dtype == np.float64 else np.float32
    means, chol, logit, colors = (np.ascontiguousarray(a, dt) for a in (means, chol, logit, colors))
    T = len(tile_offsets) - 1
    nb = len(bucket_tile)
    image = np.zeros((H, W, 3), dt)
    t_final = np.zeros((H, W), dt)
    n_contrib = np.zeros((H, W), np.int32)
    last = np.zeros((H, W), np.int32)
    ckpt = np.zeros((max(nb, 1), 256, 4), dt)
    i32 = lambda a: np.ascontiguousarray(a, np.int32)  # noqa: E731
    tabs = [i32(tile_offsets), i32(tile_ids) if len(tile_ids) else np.zeros(1, np.int32), i32(bucket_offsets),
            i32(bucket_tile) if nb else np.zeros(1, np.int32)]
    getattr(_reflib(), f"ref2d_forward_{_sfx(dt)}")(
        _p(means), _p(chol), _p(logit), _p(colors), *map(_p, tabs), C.c_int(T), C.c_int(nb), C.c_int(H), C.c_int(W),
        _p(image), _p(t_final), _p(n_contrib), _p(last), _p(ckpt))
    return dict(image=image, t_final=t_final, n_contrib=n_contrib, last_contrib=last, ckpt=ckpt)


def ref_backward(mode, means, chol, logit, colors, tile_offsets, tile_ids, bucket_offsets, bucket_tile, H, W,
                 grad_image, fwd):
    dt = np.float64 if np.asarray(means).dtype == np.float64 else np.float32
    means, chol, logit, colors, grad_image = (np.ascontiguousarray(a, dt) for a in
                                              (means, chol, logit, colors, grad_image))
    n = len(logit)
    T = len(tile_offsets) - 1
    nb = len(bucket_tile)
    gm, gc, gl, gcol = (np.zeros(s, dt) for s in ((n, 2), (n, 3), (n,), (n, 3)))
    i32 = lambda a: np.ascontiguousarray(a, np.int32)  # noqa: E731
    tabs = [i32(tile_offsets), i32(tile_ids) if len(tile_ids) else np.zeros(1, np.int32), i32(bucket_offsets),
            i32(bucket_tile) if nb else np.zeros(1, np.int32)]
    getattr(_reflib(), f"ref2d_backward_{_sfx(dt)}")(
        C.c_int(1 if mode == "splat" else 0), _p(means), _p(chol), _p(logit), _p(colors), *map(_p, tabs), C.c_int(T),
        C.c_int(nb), C.c_int(H), C.c_int(W), _p(grad_image), _p(fwd["image"]), _p(fwd["t_final"]),
        _p(fwd["last_contrib"]), _p(fwd["ckpt"]), _p(gm), _p(gc), _p(gl), _p(gcol))
    return gm, gc, gl, gcol


def ref_counters():
    out = np.zeros(3, np.int64)
    _reflib().ref2d_counters(_p(out))
    return dict(atomic_adds=int(out[0]), checkpoint_bytes=int(out[1]), splat_pixel_evals=int(out[2]))


def ref_reset_counters():
    _reflib().ref2d_reset_counters()
