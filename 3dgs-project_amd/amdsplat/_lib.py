"""ctypes binding of the C ABI in include/amdsplat.h (libamdsplat.so, built for gfx950).

The library is the only compute path: if it is missing or a call fails, the functions here
raise; nothing falls back to a CPU implementation.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libamdsplat.so"

c_float_p = C.c_void_p  # device pointers are passed as integers
_vp = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int
_sz = C.c_size_t


class GsCamera(C.Structure):
    _fields_ = [
        ("viewmat", C.c_float * 16),
        ("fx", C.c_float),
        ("fy", C.c_float),
        ("cx", C.c_float),
        ("cy", C.c_float),
        ("width", C.c_int32),
        ("height", C.c_int32),
        ("near_plane", C.c_float),
        ("far_plane", C.c_float),
        ("flags", C.c_int32),
    ]


GS_ACCUMULATE = 1  # gs_blend_bwd_3d flag: add to grad2d instead of zeroing it first
GS_ABS_GRAD = 2  # gs_blend_bwd_3d flag: also accumulate |dL/dmean2d| into grad2d[:, 9:11]
GS_BLEND_LIST_CLEARED = 1  # gs_blend_fwd_3d flag: gs_bin_fill_3d cleared the bucket list's header
GS_FLOAT32, GS_FLOAT64, GS_BFLOAT16 = 0, 1, 2
GS_CAM_PROPER_ANTIALIASING = 1  # gs_camera.flags bit
GS_BIN_SPANS, GS_BIN_RADIX = 2, 4  # binning path forced (gs_camera.flags, rect flags)
BIN_FLAGS = {"auto": 0, "spans": GS_BIN_SPANS, "radix": GS_BIN_RADIX}
GS_BIN_PATH_RADIX, GS_BIN_PATH_SPANS = 0, 1  # gs_bin_path
GS_ADAM_MAX_GROUPS = 8


class GsAdamGroup(C.Structure):
    _fields_ = [
        ("grad", C.c_void_p),
        ("param", C.c_void_p),
        ("exp_avg", C.c_void_p),
        ("exp_avg_sq", C.c_void_p),
        ("n_elements", C.c_int64),
        ("moment_dtype", C.c_int32),
        ("step", C.c_int32),
        ("lr", C.c_double),
        ("beta1", C.c_double),
        ("beta2", C.c_double),
        ("eps", C.c_double),
    ]


class AmdSplatError(RuntimeError):
    pass


_SIGS = {
    "gs_last_error": (C.c_char_p, []),
    "gs_version": (_i32, []),
    "gs_splat_record_floats": (_i32, []),
    "gs_grad2d_floats": (_i32, []),
    "gs_scan_workspace_size": (_sz, [_i64]),
    "gs_scan_u32": (_i32, [_vp, _vp, _i64, _vp, _sz, _vp]),
    "gs_sum_u32": (_i32, [_vp, _i64, _vp, _vp]),
    "gs_count_begin": (_i32, [_vp, _i64, _i32, _vp]),
    "gs_count_end": (_i32, [C.POINTER(C.c_uint64)]),
    "gs_preprocess_fwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, C.POINTER(GsCamera), _vp, _vp,
                                 _vp, _vp, _vp]),
    "gs_bin_prepare_workspace_size": (_sz, [_i64]),
    "gs_bin_prepare_3d": (_i32, [_vp, _vp, _vp, _i64, C.POINTER(GsCamera), _vp, _vp, _vp, _sz, _vp]),
    "gs_bin_workspace_size": (_sz, [_i64, _i64, _i32, _i32, _i32]),
    "gs_bin_fill_3d_workspace_size": (_sz, [_i64, _i64, C.POINTER(GsCamera)]),
    "gs_bin_path": (_i32, [_i64, C.POINTER(GsCamera)]),
    "gs_bin_fill_3d": (_i32, [_vp, _vp, _vp, _vp, _i64, C.POINTER(GsCamera), _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                              _sz, _vp]),
    "gs_rect_counts": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp]),
    "gs_bin_fill_rect": (_i32, [_vp, _vp, _i32, _vp, _i64, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp,
                                _sz, _vp]),
    "gs_bucket_fill": (_i32, [_vp, _i32, _vp, _i64, _vp]),
    "gs_blend_fwd_3d": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, C.POINTER(C.c_float), _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                               _vp, _vp, _i64, _i32, _vp]),
    "gs_blend_scores_3d": (_i32, [_vp, _vp, _vp, _i32, _i32, _i64, _vp, _vp]),
    "gs_blend_bwd_3d": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                               _vp, _vp, _vp, _i32, _vp, _vp]),
    "gs_preprocess_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, C.POINTER(GsCamera), _vp, _vp,
                                 _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gs_adam_step": (_i32, [C.POINTER(GsAdamGroup), _i32, _i64, _vp, _vp]),
    "gs_densification_stats": (_i32, [_vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp]),
    "gs_l1_ssim_workspace_size": (_sz, [_i32, _i32, _i32]),
    "gs_l1_ssim_fwd": (_i32, [_vp, _vp, _i32, _i32, _i32, C.c_float, _vp, _vp, _vp, _sz, _vp]),
    "gs_l1_ssim_bwd": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, C.c_float, _vp, _vp, _vp]),
    "gs_l1_ssim_fwd_noalloc": (_i32, [_vp, _vp, _i32, _i32, _i32, C.c_float, _vp, _vp, _vp]),
    "gs_stage_marks": (_i32, [_i32]),
    "gs_stage_marks_read": (_i32, [C.POINTER(C.c_float), C.POINTER(C.c_char_p), _i32]),
    "gs_probe_copy": (_i32, [_vp, _vp, _i64, _vp]),
    "gs_probe_read_sums": (_i64, [_i64]),
    "gs_probe_read": (_i32, [_vp, _i64, _vp, _vp]),
    "gs_probe_fma": (_i32, [_vp, _i64, _i32, _vp]),
    # 2D rule sets
    "gs2d_activate_fwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gs2d_activate_bwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gs2d_rects_toy": (_i32, [_vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp]),
    "gs2d_rects_phase0": (_i32, [_i32, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp]),
    "gs2d_pack": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "gs2d_unpack_grads": (_i32, [_i32, _vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "gs2d_blend_fwd": (_i32, [_i32, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _i32, C.POINTER(C.c_double), _vp, _vp, _vp,
                              _vp, _vp, _vp, _vp, _vp]),
    "gs2d_blend_bwd_bucket": (_i32, [_i32, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _vp, _vp]),
    "gs2d_blend_bwd_pixel": (_i32, [_i32, _i32, _vp, _vp, _i32, _vp, _i64, _i32, _i32, C.POINTER(C.c_double), _vp,
                                    _vp, _vp, _vp, _vp, _vp]),
}

_lib = None
_missing: set[str] = set()


def lib() -> C.CDLL:
    """Loads libamdsplat.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise AmdSplatError(
                f"{LIB_PATH} not found: build it with `python 3dgs-project_amd/build.py` "
                "(or __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            try:
                fn = getattr(L, name)
            except AttributeError:
                _missing.add(name)
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> set[str]:
    lib()
    return set(_SIGS) - _missing


def call(name: str, *args) -> None:
    L = lib()
    if name in _missing:
        raise AmdSplatError(f"{name} is not exported by {LIB_PATH}")
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.gs_last_error().decode(errors="replace")
        raise AmdSplatError(f"{name} failed (code {rc}): {msg}")


def size_call(name: str, *args) -> int:
    return int(getattr(lib(), name)(*args))


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None or empty tensors)."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def stream_handle(device=None) -> int | None:
    """The current HIP stream of `device` (a torch.device, an index or None for the current
    device) as an integer, None for the null stream."""
    import torch

    if isinstance(device, torch.device):
        idx = device.index if device.index is not None else torch.cuda.current_device()
    elif isinstance(device, int):
        idx = device
    else:
        idx = torch.cuda.current_device()
    # the raw handle straight from the stream registry (torch.cuda.current_stream builds a Stream
    # object and parses the device on every call: ~10 us a call on the host)
    return torch._C._cuda_getCurrentRawStream(idx) or None


def float3(v) -> C.Array:
    arr = (C.c_float * 3)(*[float(x) for x in v])
    return arr


def make_camera(viewmat, fx: float, fy: float, cx: float, cy: float, width: int, height: int,
                near: float, far: float, flags: int = 0) -> GsCamera:
    cam = GsCamera()
    if hasattr(viewmat, "reshape"):
        flat = viewmat.reshape(-1).tolist()
    else:
        flat = [x for row in viewmat for x in row] if viewmat and isinstance(viewmat[0], (list, tuple)) else viewmat
    if len(flat) != 16:
        raise ValueError("viewmat must be 4x4")
    cam.viewmat[:] = [float(x) for x in flat]
    cam.fx, cam.fy, cam.cx, cam.cy = float(fx), float(fy), float(cx), float(cy)
    cam.width, cam.height = int(width), int(height)
    cam.near_plane, cam.far_plane = float(near), float(far)
    cam.flags = int(flags)
    return cam


def env_debug() -> bool:
    return os.environ.get("AMDSPLAT_DEBUG", "0") == "1"
