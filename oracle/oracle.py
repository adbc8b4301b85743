"""ctypes wrapper of liboracle.so (the C restatement in this folder).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package. All arrays are numpy, on the host.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


class OrCamera(C.Structure):
    _fields_ = [("viewmat", C.c_float * 16), ("fx", C.c_float), ("fy", C.c_float), ("cx", C.c_float),
                ("cy", C.c_float), ("width", C.c_int32), ("height", C.c_int32), ("near_plane", C.c_float),
                ("far_plane", C.c_float), ("flags", C.c_int32)]


def build(force: bool = False) -> Path:
    srcs = list(HERE.glob("*.c"))
    if force or not LIB.exists() or any(s.stat().st_mtime > LIB.stat().st_mtime for s in srcs):
        subprocess.run(["make", "-C", str(HERE), "-B" if force else "all"], check=True, capture_output=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = C.CDLL(str(LIB))
        _lib.or_bin.restype = C.c_int64
        for name in ("or_exp2_neg", "or_exp2_any", "or_sigmoid", "or_log_pos"):
            getattr(_lib, name).restype = C.c_float
            getattr(_lib, name).argtypes = [C.c_float]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def camera(cam) -> OrCamera:
    """OrCamera from an amdsplat.rasterize.Camera (or any object with the same fields)."""
    oc = OrCamera()
    vm = np.asarray(cam.viewmat.detach().cpu().float().numpy() if hasattr(cam.viewmat, "detach")
                    else cam.viewmat, dtype=np.float32).reshape(-1)
    for i in range(16):
        oc.viewmat[i] = float(vm[i])
    oc.fx, oc.fy, oc.cx, oc.cy = cam.fx, cam.fy, cam.cx, cam.cy
    oc.width, oc.height = cam.width, cam.height
    oc.near_plane, oc.far_plane = cam.near, cam.far
    oc.flags = 1 if getattr(cam, "proper_antialiasing", False) else 0
    return oc


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def preprocess_fwd(means, log_scales, quats, opacity_logits, sh, cam, sh_degree):
    means, log_scales, quats, opacity_logits, sh = map(f32, (means, log_scales, quats, opacity_logits, sh))
    n, K = means.shape[0], sh.shape[1]
    rec = np.zeros((n, 16), np.float32)
    touched = np.zeros(n, np.uint32)
    lib().or_preprocess_fwd(_p(means), _p(log_scales), _p(quats), _p(opacity_logits), _p(sh), C.c_int64(n),
                            C.c_int(K), C.c_int(sh_degree), C.byref(camera(cam)), _p(rec), _p(touched))
    return rec, touched


def bin_instances(rec, touched, cam):
    n = rec.shape[0]
    T = ((cam.width + 15) // 16) * ((cam.height + 15) // 16)
    m = int(touched.astype(np.int64).sum())
    keys = np.zeros(max(m, 1), np.uint64)
    pl = np.zeros(max(m, 1), np.uint32)
    ranges = np.zeros((T, 2), np.uint32)
    boff = np.zeros(T + 1, np.uint32)
    got = lib().or_bin(_p(f32(rec)), _p(np.ascontiguousarray(touched, np.uint32)), C.c_int64(n),
                       C.byref(camera(cam)), _p(keys), _p(pl), _p(ranges), _p(boff))
    assert got == m, (got, m)
    return keys[:m], pl[:m], ranges, boff


def blend_fwd(rec, point_list, ranges, boff, width, height, bg=(0.0, 0.0, 0.0), with_ckpt=True, scores=None):
    """scores: None, or a float64 [n] array that receives each splat's summed blending weights."""
    T = ranges.shape[0]
    nb = int(boff[-1])
    image = np.zeros((3, height, width), np.float32)
    final_T = np.zeros((height, width), np.float32)
    n_contrib = np.zeros((height, width), np.int32)
    tile_max = np.zeros(T, np.uint32)
    ckpt = np.zeros((max(nb, 1), 256, 4), np.float32) if with_ckpt else None
    amb = np.zeros((height, width), np.uint8)
    bgc = np.asarray(bg, np.float32)
    lib().or_blend_fwd(_p(f32(rec)), _p(np.ascontiguousarray(ranges, np.uint32)),
                       _p(np.ascontiguousarray(point_list, np.uint32)), _p(np.ascontiguousarray(boff, np.uint32)),
                       C.c_int(width), C.c_int(height), _p(bgc), _p(image), _p(final_T), _p(n_contrib),
                       _p(tile_max), _p(ckpt), _p(amb), _p(scores))
    return image, final_T, n_contrib, tile_max, ckpt, amb.astype(bool)


def blend_bwd(rec, point_list, ranges, boff, width, height, image, grad_image, final_T, n_contrib, tile_max,
              ckpt, n, grad_alpha=None, conic64=False):
    """grad2d [n, 12] float32; with conic64=True also the conic-gradient sums (columns 2-4)
    unrounded, float64 [n, 4]: returns (grad2d, conic64)."""
    grad2d = np.zeros((n, 12), np.float32)
    c64 = np.zeros((n, 4), np.float64) if conic64 else None
    lib().or_blend_bwd(_p(f32(rec)), _p(np.ascontiguousarray(ranges, np.uint32)),
                       _p(np.ascontiguousarray(point_list, np.uint32)), _p(np.ascontiguousarray(boff, np.uint32)),
                       C.c_int(width), C.c_int(height), _p(f32(image)), _p(f32(grad_image)), _p(f32(final_T)),
                       _p(None if grad_alpha is None else f32(grad_alpha)),
                       _p(np.ascontiguousarray(n_contrib, np.int32)), _p(np.ascontiguousarray(tile_max, np.uint32)),
                       _p(f32(ckpt)), C.c_int64(n), _p(grad2d), _p(c64))
    return (grad2d, c64) if conic64 else grad2d


def preprocess_bwd(means, log_scales, quats, opacity_logits, sh, cam, sh_degree, rec, touched, grad2d, conic64=None):
    """conic64: None, or float64 [n, 4] conic-gradient sums that replace grad2d's columns 2-4."""
    means, log_scales, quats, opacity_logits, sh = map(f32, (means, log_scales, quats, opacity_logits, sh))
    n, K = means.shape[0], sh.shape[1]
    gm = np.zeros((n, 3), np.float32)
    gls = np.zeros((n, 3), np.float32)
    gq = np.zeros((n, 4), np.float32)
    gop = np.zeros(n, np.float32)
    gsh = np.zeros((n, K, 3), np.float32)
    lib().or_preprocess_bwd(_p(means), _p(log_scales), _p(quats), _p(opacity_logits), _p(sh), C.c_int64(n),
                            C.c_int(K), C.c_int(sh_degree), C.byref(camera(cam)), _p(f32(rec)),
                            _p(np.ascontiguousarray(touched, np.uint32)), _p(f32(grad2d)),
                            _p(None if conic64 is None else np.ascontiguousarray(conic64, np.float64)), _p(gm), _p(gls),
                            _p(gq), _p(gop), _p(gsh))
    return gm, gls, gq, gop, gsh


def render(means, log_scales, quats, opacity_logits, sh, cam, sh_degree, bg=(0.0, 0.0, 0.0)):
    """Full forward. Returns a dict of every intermediate, with the pruning scores (float64 [n])."""
    rec, touched = preprocess_fwd(means, log_scales, quats, opacity_logits, sh, cam, sh_degree)
    keys, pl, ranges, boff = bin_instances(rec, touched, cam)
    scores = np.zeros(rec.shape[0], np.float64)
    image, final_T, n_contrib, tile_max, ckpt, amb = blend_fwd(rec, pl, ranges, boff, cam.width, cam.height, bg,
                                                               scores=scores)
    return dict(rec=rec, touched=touched, keys=keys, point_list=pl, ranges=ranges, bucket_offsets=boff,
                image=image, final_T=final_T, n_contrib=n_contrib, tile_max=tile_max, ckpt=ckpt, amb=amb,
                scores=scores)


def exp2_neg(x: float) -> float:
    return float(lib().or_exp2_neg(C.c_float(x)))


def exp2_any(x: float) -> float:
    return float(lib().or_exp2_any(C.c_float(x)))


def log_pos(x: float) -> float:
    return float(lib().or_log_pos(C.c_float(x)))


def sigmoid(x: float) -> float:
    return float(lib().or_sigmoid(C.c_float(x)))


def contrib_mask(rec, point_list, ranges, width, height, n_contrib):
    m = point_list.shape[0]
    mask = np.zeros((max(m, 1), 256), np.uint8)
    lib().or_contrib_mask(_p(f32(rec)), _p(np.ascontiguousarray(ranges, np.uint32)),
                          _p(np.ascontiguousarray(point_list, np.uint32)), C.c_int(width), C.c_int(height),
                          _p(np.ascontiguousarray(n_contrib, np.int32)), _p(mask))
    return mask[:m]


def sh_basis(dirs, n):
    """Real SH basis values [len(dirs), n] of unit directions (float32 oracle routine)."""
    d = f32(dirs).reshape(-1, 3)
    out = np.zeros((d.shape[0], 16), np.float32)
    fn = lib().or_sh_basis
    buf = (C.c_float * 16)()
    for i, (x, y, z) in enumerate(d):
        fn(C.c_float(x), C.c_float(y), C.c_float(z), C.c_int(n), buf)
        out[i, :n] = np.frombuffer(buf, np.float32, n)
    return out[:, :n]
