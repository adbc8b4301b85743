"""3D Gaussian-splat rasterizer: `rasterize(means, scales, quats, opacities, sh, viewmat, K, W, H)`.

Host side of the MI355X path. Every stage is a C-ABI call into libamdsplat.so on the current
torch stream; this module only allocates the buffers (PyTorch owns all device memory) and
wires the stages:

    preprocess -> scan(tiles touched) -> [read M] -> emit keys + radix sort + ranges + buckets
    -> bucket->tile table -> forward blend                       (forward)
    bucketed blend backward -> preprocess backward                (backward)

The operator surface follows the reference's 3D call sites: gsplat's
`rasterization(means, quats, scales, opac, colors, viewmats, K, W, H) -> (img, alpha, meta)`
(cluster/build_env.sbatch:47-55) and Faster-GS's raw-parameter convention for
`_C.forward` / `_C.backward` (phase1/tests/test_parity.py:59-98: log-scales, unnormalised
quaternions, opacity logits, SH coefficients).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import call, ptr

TILE = 16
BUCKET = 32
REC_FLOATS = 16
GRAD2D_FLOATS = 12
# gs_count_begin on the library's side stream (True) or on the forward's own stream (False: the
# depth sort then waits for the 3-5 us sum, but the host saves an event record and a stream wait,
# about 20 us of host time per view; 100k SH0 step 0.281 -> 0.278 ms, 1M SH3 unchanged)
COUNT_ON_SIDE_STREAM = False
# the tile binning of the views rasterize(...), rasterize_inference and pruning_scores build:
# "auto", "spans" or "radix" (forward_pass takes its Camera's own field)
BINNING = "auto"


def _u8(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _layout(parts: dict):
    """Byte offsets (256-byte aligned) of named regions of one allocation, and its size."""
    offs, total = {}, 0
    for name, nbytes in parts.items():
        offs[name] = total
        total += (int(nbytes) + 255) & ~255
    return offs, max(total, 1)


@dataclass
class Camera:
    """Pinhole camera: row-major world-to-camera `viewmat` (4x4, OpenCV axes) and intrinsics."""

    viewmat: torch.Tensor
    fx: float
    fy: float
    cx: float
    cy: float
    width: int
    height: int
    near: float = 0.01
    far: float = 100.0
    proper_antialiasing: bool = False
    binning: str = "auto"  # "auto", "spans" or "radix": which tile binning the forward takes

    @staticmethod
    def from_K(viewmat, K, width: int, height: int, near: float = 0.01, far: float = 100.0,
               proper_antialiasing: bool = False, binning: str = "auto") -> "Camera":
        k = (K.detach().cpu().double() if torch.is_tensor(K) else torch.as_tensor(K, dtype=torch.float64)).tolist()
        vm = torch.as_tensor(viewmat, dtype=torch.float32).detach().cpu().reshape(4, 4)
        return Camera(vm, float(k[0][0]), float(k[1][1]), float(k[0][2]), float(k[1][2]), int(width),
                      int(height), float(near), float(far), bool(proper_antialiasing), binning)

    @property
    def tiles_x(self) -> int:
        return (self.width + TILE - 1) // TILE

    @property
    def tiles_y(self) -> int:
        return (self.height + TILE - 1) // TILE

    @property
    def n_tiles(self) -> int:
        return self.tiles_x * self.tiles_y

    def c_struct(self) -> _lib.GsCamera:
        flags = (_lib.GS_CAM_PROPER_ANTIALIASING if self.proper_antialiasing else 0) | _lib.BIN_FLAGS[self.binning]
        return _lib.make_camera(self.viewmat.detach().cpu().float().reshape(-1).tolist(), self.fx, self.fy, self.cx,
                                self.cy, self.width, self.height, self.near, self.far, flags)


@dataclass
class ForwardState:
    """Device buffers of one forward pass (kept for the backward)."""

    cam: Camera
    n: int
    sh_coeffs: int
    sh_degree: int
    rec: torch.Tensor            # [n, 16] splat records
    touched: torch.Tensor        # [n] int32 tiles touched (0 = culled)
    order: torch.Tensor          # [n] int32 Gaussians by depth (culled last)
    offsets: torch.Tensor | None  # [n + 1] int32 instance offsets over `order`; None on the span path
    path: int  # the tile binning's path (GS_BIN_PATH_*)
    m: int                       # instances
    keys: torch.Tensor           # [m] int64 sorted keys (empty unless keep_keys)
    point_list: torch.Tensor     # [m] int32
    ranges: torch.Tensor         # [T, 2] int32
    bucket_offsets: torch.Tensor  # [T + 1] int32
    n_buckets_max: int
    bucket_to_tile: torch.Tensor | None  # [n_buckets_max] int32 (None: inference)
    image: torch.Tensor | None   # [3, H, W]
    final_T: torch.Tensor | None  # [H, W]
    n_contrib: torch.Tensor | None  # [H, W] int32 (None: inference)
    tile_max: torch.Tensor | None  # [T] int32 (None: inference)
    ckpt: torch.Tensor | None    # [n_buckets_max, 256, 4] (None: inference)
    bucket_list: torch.Tensor | None = None  # [4 + n_buckets_max] int32: buckets the backward reads
    bg: tuple = (0.0, 0.0, 0.0)
    timings: dict = field(default_factory=dict)
    grad2d: torch.Tensor | None = None  # [n, 12] zeroed by the forward blend, for the first backward
    # [n, 4] float64, zeroed with grad2d: the elongated splats' conic-gradient sums (gs_blend_bwd_3d)
    grad_conic64: torch.Tensor | None = None
    ccam: "_lib.GsCamera | None" = None  # the camera as the C calls take it (built once per forward)
    last_conic64: torch.Tensor | None = None  # the float64 conic sums of the last backward
    alpha: torch.Tensor | None = None  # [H, W] 1 - final_T, written by the forward blend

    @property
    def n_buckets(self) -> int:
        return int(self.bucket_offsets[-1].item())


class StageTimer:
    """Records torch.cuda events on the current stream between stages (no-op if disabled)."""

    def __init__(self, enabled: bool):
        self.enabled = enabled
        self.marks: list[tuple[str, torch.cuda.Event]] = []

    def mark(self, name: str) -> None:
        if self.enabled:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            self.marks.append((name, e))

    def result(self, sync: bool = True) -> dict:
        """Per-stage milliseconds (a stage is the interval that ends at its mark; the interval
        ending at a "start" mark, e.g. between a forward and its backward, is not a stage); with
        sync=False the caller must have synchronised."""
        if not self.enabled or len(self.marks) < 2:
            return {}
        if sync:
            torch.cuda.synchronize()
        out = {}
        for (_, a), (name, b) in zip(self.marks[:-1], self.marks[1:]):
            if name != "start":
                out[name] = out.get(name, 0.0) + a.elapsed_time(b)
        return out


def _count_end() -> int:
    """The instance count of the pending gs_count_begin on this thread and device."""
    m = ctypes.c_uint64()
    call("gs_count_end", ctypes.byref(m))
    return int(m.value)


def _check_inputs(means, log_scales, quats, opacity_logits, sh):
    n = means.shape[0]
    dev = means.device
    if dev.type != "cuda":
        raise ValueError("amdsplat.rasterize runs on the GPU: inputs must be CUDA tensors")
    for name, t, shape in (("means", means, (n, 3)), ("scales", log_scales, (n, 3)), ("quats", quats, (n, 4)),
                           ("opacities", opacity_logits, (n,))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
        if t.dtype != torch.float32 or t.device != dev:
            raise ValueError(f"{name} must be float32 on {dev}")
    sh_a, sh_b = sh if isinstance(sh, (tuple, list)) else (sh, None)
    if sh_b is None:
        if sh_a.dim() != 3 or sh_a.shape[0] != n or sh_a.shape[2] != 3 or sh_a.shape[1] not in (1, 4, 9, 16):
            raise ValueError(f"sh must have shape [N, K, 3] with K in (1, 4, 9, 16), got {tuple(sh_a.shape)}")
    else:
        if tuple(sh_a.shape) != (n, 1, 3) or sh_b.dim() != 3 or sh_b.shape[0] != n or sh_b.shape[2] != 3 \
                or sh_b.shape[1] + 1 not in (4, 9, 16):
            raise ValueError(f"split SH must be ([N, 1, 3], [N, K - 1, 3]) with K in (4, 9, 16), got "
                             f"{tuple(sh_a.shape)}, {tuple(sh_b.shape)}")
    for t in (sh_a, sh_b):
        if t is not None and (t.dtype != torch.float32 or t.device != dev):
            raise ValueError(f"sh must be float32 on {dev}")


def _sh_parts(sh):
    """(coefficients or DC, rest or None, K) of an [N, K, 3] tensor or a (DC, rest) pair. A pair
    whose rest holds no coefficients ([N, 0, 3]: Faster-GS's degree-0 model) is the DC alone."""
    if isinstance(sh, (tuple, list)):
        a, b = sh[0].contiguous(), sh[1].contiguous()
        if b.dim() == 3 and b.shape[1] == 0:
            return a, None, 1
        return a, b, 1 + b.shape[1]
    sh = sh.contiguous()
    return sh, None, sh.shape[1]


def forward_pass(means, log_scales, quats, opacity_logits, sh, cam: Camera, sh_degree: int | None = None,
                 bg=(0.0, 0.0, 0.0), timing: bool = False, keep_keys: bool = False,
                 for_backward: bool = True, _scores: torch.Tensor | None = None) -> ForwardState:
    """Runs the forward stages; inputs are contiguous float32 CUDA tensors (raw parameters). sh is
    [N, K, 3] or the (DC [N, 1, 3], rest [N, K - 1, 3]) pair. for_backward=False is the inference
    blend: no bucket table, checkpoints or n_contrib (those fields are None), same image bits."""
    means, log_scales, quats = means.contiguous(), log_scales.contiguous(), quats.contiguous()
    opacity_logits = opacity_logits.contiguous()
    sh_a, sh_b, K = _sh_parts(sh)
    _check_inputs(means, log_scales, quats, opacity_logits, (sh_a, sh_b))
    n = means.shape[0]
    dev = means.device
    if sh_degree is None:
        sh_degree = int(round(math.sqrt(K))) - 1
    ccam = cam.c_struct()
    st = _lib.stream_handle(dev)
    tm = timing if isinstance(timing, StageTimer) else StageTimer(bool(timing))
    tm.mark("start")

    rec = torch.empty(n, REC_FLOATS, dtype=torch.float32, device=dev)
    touched = torch.empty(n, dtype=torch.int32, device=dev)
    dkeys = torch.empty(n, dtype=torch.int32, device=dev)
    n_waves = (n + 63) // 64
    wave_counts = torch.empty(n_waves, dtype=torch.int32, device=dev)
    call("gs_preprocess_fwd", ptr(means), ptr(log_scales), ptr(quats), ptr(opacity_logits), ptr(sh_a), ptr(sh_b),
         n, K, sh_degree, ccam, ptr(rec), ptr(touched), ptr(dkeys), ptr(wave_counts), st)
    tm.mark("preprocess")
    # The instance count m (the total of the per-wavefront tile counts) needs only the
    # preprocess: the library's side stream sums the counts and copies the total to host memory
    # while the depth sort runs on this stream, so the host sizes the fill's buffers without the
    # stream draining first.
    counting = n > 0
    if counting:
        call("gs_count_begin", ptr(wave_counts), n_waves, int(COUNT_ON_SIDE_STREAM), st)
    try:
        return _forward_rest(means, sh_a, sh_b, K, n, dev, sh_degree, cam, ccam, st, tm, rec, touched, dkeys, bg,
                             timing, keep_keys, for_backward, _scores, counting)
    except BaseException:
        if counting:
            try:
                _count_end()  # the side stream's copy is done before any buffer it reads is freed
            except _lib.AmdSplatError:
                pass
        raise


def _forward_rest(means, sh_a, sh_b, K, n, dev, sh_degree, cam, ccam, st, tm, rec, touched, dkeys, bg, timing,
                  keep_keys, for_backward, _scores, counting):
    """forward_pass after the preprocess: the depth ordering, the count, the fill and the blend."""
    T = cam.n_tiles
    H, W = cam.height, cam.width
    # The tile binning's path: the radix path takes the depth order and the instance offsets in
    # that order; the span binning the depth order alone.
    path = _lib.lib().gs_bin_path(n, ccam)
    order = torch.empty(n, dtype=torch.int32, device=dev)
    offsets = torch.empty(n + 1, dtype=torch.int32, device=dev) if path != _lib.GS_BIN_PATH_SPANS else None
    ws = _u8(_lib.size_call("gs_bin_prepare_workspace_size", n), dev)
    call("gs_bin_prepare_3d", ptr(rec), ptr(touched), ptr(dkeys), n, ccam, ptr(order), ptr(offsets), ptr(ws),
         ws.numel(), st)
    tm.mark("depth_order")
    # Everything whose size does not depend on the instance count is allocated while the copy
    # and the depth sort run; after the count arrives the host only carves the count-sized
    # buffers out of one allocation and launches the fill, before the depth sort ends.
    ranges = torch.empty(T, 2, dtype=torch.int32, device=dev)
    bucket_offsets = torch.empty(T + 1, dtype=torch.int32, device=dev)
    backward_state = for_backward and _scores is None
    n_contrib = tile_max = grad2d = conic64 = gbuf = image = final_T = alpha = None
    if backward_state:
        n_contrib = torch.empty(H, W, dtype=torch.int32, device=dev)
        tile_max = torch.empty(T, dtype=torch.int32, device=dev)
        # the backward's screen gradients [n, 12] float32 and the elongated splats' float64 conic
        # sums [n, 4], one buffer that the forward blend's workgroups zero
        gbuf = torch.empty(n * (GRAD2D_FLOATS + 8), dtype=torch.float32, device=dev)
        grad2d = gbuf[:n * GRAD2D_FLOATS].view(n, GRAD2D_FLOATS)
        conic64 = gbuf[n * GRAD2D_FLOATS:].view(torch.float64).view(n, 4)
    if _scores is None:
        image = torch.empty(3, H, W, dtype=torch.float32, device=dev)
        final_T = torch.empty(H, W, dtype=torch.float32, device=dev)
        alpha = torch.empty(H, W, dtype=torch.float32, device=dev)
    # addresses the calls after the readback take (ctypes conversions done before the wait)
    p_rec, p_dkeys, p_order, p_offsets = ptr(rec), ptr(dkeys), ptr(order), ptr(offsets)
    p_ranges, p_boff, bg3 = ptr(ranges), ptr(bucket_offsets), _lib.float3(bg)
    m = 0
    if counting:
        m = _count_end()
        if m >= 1 << 32:
            raise _lib.AmdSplatError(f"{m} tile instances exceed the 32-bit instance index")
    nb_max = (m + (BUCKET - 1) * T) // BUCKET if backward_state else 0  # >= sum over tiles of ceil(len / 32)
    # the fill's scratch is its own allocation, released when this function returns: nothing the
    # blends or the backward read lives in it (the caching allocator reuses it in stream order)
    ws_fill = _u8(_lib.lib().gs_bin_fill_3d_workspace_size(n, m, ccam), dev)
    parts = {"point_list": 4 * m, "keys": 8 * m if keep_keys else 0}
    if backward_state:
        parts.update(bucket_to_tile=4 * max(nb_max, 1), blist=4 * (4 + nb_max), ckpt=4096 * max(nb_max, 1))
    offs, total = _layout(parts)
    arena = torch.empty(total, dtype=torch.uint8, device=dev)
    # the kernels are launched from raw addresses; the tensor views are made after the launches,
    # so that the host reaches the fill while the depth sort still runs
    base = arena.data_ptr()
    adr = {k: (base + o if parts[k] > 0 else None) for k, o in offs.items()}
    # the fill also clears the bucket list's header for the forward blend
    call("gs_bin_fill_3d", p_rec, p_dkeys, p_order, p_offsets, n, ccam, m, adr["keys"], adr["point_list"], p_ranges,
         p_boff, adr.get("blist"), ptr(ws_fill), ws_fill.numel(), st)
    tm.mark("binning")
    if _scores is None:
        call("gs_blend_fwd_3d", p_rec, p_ranges, adr["point_list"], p_boff, W, H, bg3, ptr(image), ptr(final_T),
             ptr(alpha), ptr(n_contrib), ptr(tile_max), adr.get("ckpt"), adr.get("blist"), adr.get("bucket_to_tile"),
             ptr(gbuf), gbuf.numel() if gbuf is not None else 0,
             _lib.GS_BLEND_LIST_CLEARED if backward_state else 0, st)
    else:  # pruning scores: the blend's weights, no image
        call("gs_blend_scores_3d", p_rec, p_ranges, adr["point_list"], W, H, n, ptr(_scores), st)

    def view(name, dtype):
        o = offs[name]
        return arena[o:o + parts[name]].view(dtype)

    point_list = view("point_list", torch.int32)
    keys = view("keys", torch.int64) if keep_keys else torch.empty(0, dtype=torch.int64, device=dev)
    if _scores is not None:
        tm.mark("scores")
        return ForwardState(cam, n, K, sh_degree, rec, touched, order, offsets, path, m, keys, point_list, ranges,
                            bucket_offsets, 0, None, None, None, None, None, None, None, tuple(bg),
                            {} if isinstance(timing, StageTimer) else tm.result())
    bucket_to_tile = ckpt = blist = None
    if backward_state:
        bucket_to_tile = view("bucket_to_tile", torch.int32)
        blist = view("blist", torch.int32)
        ckpt = view("ckpt", torch.float32).view(max(nb_max, 1), 256, 4)
    tm.mark("blend_fwd")
    return ForwardState(cam, n, K, sh_degree, rec, touched, order, offsets, path, m, keys, point_list, ranges,
                        bucket_offsets, nb_max, bucket_to_tile, image, final_T, n_contrib, tile_max, ckpt, blist,
                        tuple(bg),
                        {} if isinstance(timing, StageTimer) else tm.result(), grad2d, conic64, ccam, None, alpha)


def backward_pass(fs: ForwardState, means, log_scales, quats, opacity_logits, sh, grad_image,
                  grad_alpha=None, timing: bool = False, counters: torch.Tensor | None = None,
                  abs_grad: bool = True):
    """Returns (grad_means, grad_log_scales, grad_quats, grad_opacity_logits, grad_sh, grad2d, timings);
    grad_sh is a (DC, rest) pair when sh is. abs_grad: also sum |dL/dmean2d| into grad2d[:, 9:11]
    (densification by absolute gradient); otherwise those columns stay zero. The conic columns
    (2-4) of the elongated splats (2D condition number >= 256) are summed in float64 into
    fs.last_conic64 [n, 4] instead, their rows marked in column 11 (only those rows of it hold
    sums); combined_grad2d(grad2d, fs.last_conic64) gives all screen-space gradients.
    counters: optional int64 [3] CUDA tensor that the blend backward adds its atomic count and
    pair-evaluation count to (slots 0 and 2)."""
    dev = means.device
    n = fs.n
    cam = fs.cam
    st = _lib.stream_handle(dev)
    grad_image = grad_image.contiguous().float()
    if grad_alpha is not None:
        grad_alpha = grad_alpha.contiguous().float()
    tm = timing if isinstance(timing, StageTimer) else StageTimer(bool(timing))
    tm.mark("start")
    if fs.grad2d is not None:
        # zeroed by the forward blend; a second backward of the same forward starts from zeros
        grad2d, fs.grad2d = fs.grad2d, None
        conic64, fs.grad_conic64 = fs.grad_conic64, None
    else:
        grad2d = torch.zeros(n, GRAD2D_FLOATS, dtype=torch.float32, device=dev)
        conic64 = torch.zeros(n, 4, dtype=torch.float64, device=dev)
    fs.last_conic64 = conic64
    call("gs_blend_bwd_3d", ptr(fs.rec), ptr(fs.ranges), ptr(fs.point_list), ptr(fs.bucket_offsets),
         ptr(fs.bucket_to_tile), fs.n_buckets_max, n, cam.width, cam.height, ptr(fs.image), ptr(grad_image),
         ptr(fs.final_T), ptr(grad_alpha), ptr(fs.n_contrib), ptr(fs.tile_max), ptr(fs.ckpt), ptr(fs.bucket_list),
         ptr(grad2d), ptr(conic64),
         _lib.GS_ACCUMULATE | (_lib.GS_ABS_GRAD if abs_grad else 0), ptr(counters), st)
    tm.mark("blend_bwd")
    g_means = torch.empty(n, 3, dtype=torch.float32, device=dev)
    g_ls = torch.empty(n, 3, dtype=torch.float32, device=dev)
    g_q = torch.empty(n, 4, dtype=torch.float32, device=dev)
    g_op = torch.empty(n, dtype=torch.float32, device=dev)
    sh_a, sh_b, _ = _sh_parts(sh)
    if sh_b is None:
        g_sh = torch.empty(n, fs.sh_coeffs, 3, dtype=torch.float32, device=dev)
        g_a, g_b = g_sh, None
        if isinstance(sh, (tuple, list)):  # (DC, empty rest): the pair back, the rest's gradient empty
            g_sh = (g_sh, torch.empty(n, 0, 3, dtype=torch.float32, device=dev))
    else:
        g_a = torch.empty(n, 1, 3, dtype=torch.float32, device=dev)
        g_b = torch.empty(n, fs.sh_coeffs - 1, 3, dtype=torch.float32, device=dev)
        g_sh = (g_a, g_b)
    call("gs_preprocess_bwd", ptr(means), ptr(log_scales), ptr(quats), ptr(opacity_logits), ptr(sh_a), ptr(sh_b),
         n, fs.sh_coeffs, fs.sh_degree, fs.ccam if fs.ccam is not None else cam.c_struct(), ptr(fs.touched),
         ptr(grad2d), ptr(conic64), ptr(g_means),
         ptr(g_ls), ptr(g_q), ptr(g_op), ptr(g_a), ptr(g_b), st)
    tm.mark("preprocess_bwd")
    return g_means, g_ls, g_q, g_op, g_sh, grad2d, {} if isinstance(timing, StageTimer) else tm.result()


def combined_grad2d(grad2d: torch.Tensor, conic64: torch.Tensor | None) -> torch.Tensor:
    """The screen-space gradients of a backward as float64 [n, 12]: grad2d with the elongated
    splats' float64 conic sums (the rows marked in column 11) added to columns 2-4, and the mark
    cleared."""
    g = grad2d.double()
    if conic64 is not None:
        marked = grad2d[:, 11] != 0  # the rows that hold float64 sums
        g[marked, 2:5] += conic64[marked, :3]
    g[:, 11] = 0.0
    return g


def densification_stats(grad2d: torch.Tensor, touched: torch.Tensor, width: int, height: int,
                        info: torch.Tensor) -> None:
    """Adds one view's densification statistics to info [2 or 3, N] (float32, in place): a visible
    count, the NDC norm of the mean2d gradient and (3 rows) the NDC norm of the summed |dL/dmean2d|."""
    n = touched.shape[0]
    if info.dim() != 2 or info.shape[1] != n or info.shape[0] not in (2, 3) or info.dtype != torch.float32 \
            or not info.is_contiguous():
        raise ValueError(f"densification_info must be contiguous float32 [2 or 3, {n}]")
    call("gs_densification_stats", ptr(grad2d), ptr(touched), n, int(width), int(height), int(info.shape[0]),
         ptr(info), _lib.stream_handle(info.device))


class _Rasterize3D(torch.autograd.Function):
    # Compatibility alias of the visibility hand-off of Faster-GS's lean Adam patch
    # (cluster/patches/fastergs_lean_adam.patch:329-343): with track_visibility set, each
    # differentiable forward also leaves its tiles_touched (int32 [n], > 0 = visible in that view)
    # in last_visibility, where FusedAdam(sparse=True).step() looks when it is not handed a mask.
    # The per-call hand-off is aux["visibility"] (FusedAdam.step(visibility=...)): two forwards in
    # flight each keep their own.
    track_visibility: bool = False
    last_visibility: "torch.Tensor | None" = None

    @staticmethod
    def forward(ctx, means, log_scales, quats, opacity_logits, sh, sh_rest, cam, sh_degree, bg, dinfo=None,
                timer=None):
        shp = sh if sh_rest is None else (sh, sh_rest)
        fs = forward_pass(means, log_scales, quats, opacity_logits, shp, cam, sh_degree, bg,
                          timing=timer if timer is not None else False)
        # an output the loss does not use gets None, not a zero tensor: an alpha nobody
        # differentiates costs the backward nothing
        ctx.set_materialize_grads(False)
        ctx.fs = fs
        ctx.timer = timer
        ctx.dinfo = dinfo
        ctx.split = sh_rest is not None
        ctx.save_for_backward(means, log_scales, quats, opacity_logits, sh, sh_rest)
        alpha = fs.alpha.detach()  # 1 - final_T, written by the blend
        n_buckets = fs.bucket_offsets[-1]
        m = torch.tensor(fs.m, dtype=torch.int64)  # host tensor: the count is already on the host
        # The outputs are new tensor objects over the forward state's storage: were they the
        # state's own objects, output -> grad_fn -> ctx -> state -> output would be a reference
        # cycle, and each view's buffers (about 1 GB at 1M Gaussians) would wait for Python's
        # cyclic garbage collector instead of being freed when the output is.
        image, touched = fs.image.detach(), fs.touched.detach()
        if _Rasterize3D.track_visibility:
            _Rasterize3D.last_visibility = touched
        ctx.mark_non_differentiable(touched, n_buckets, m)
        return image, alpha, touched, n_buckets, m

    @staticmethod
    def backward(ctx, grad_image, grad_alpha, _grad_touched, _grad_nb, _grad_m):
        means, log_scales, quats, opacity_logits, sh, sh_rest = ctx.saved_tensors
        fs = ctx.fs
        if grad_image is None:
            grad_image = torch.zeros_like(fs.image)
        shp = (sh, sh_rest) if ctx.split else sh
        # |dL/dmean2d| only when the caller's densification_info has its third row
        abs_grad = ctx.dinfo is not None and ctx.dinfo.shape[0] == 3
        gm, gls, gq, gop, gsh, grad2d, _ = backward_pass(fs, means.contiguous(), log_scales.contiguous(),
                                                         quats.contiguous(), opacity_logits.contiguous(),
                                                         shp, grad_image, grad_alpha,
                                                         timing=ctx.timer if ctx.timer is not None else False,
                                                         abs_grad=abs_grad)
        ctx.grad2d = grad2d
        if ctx.dinfo is not None:
            densification_stats(grad2d, fs.touched, fs.cam.width, fs.cam.height, ctx.dinfo)
        g_a, g_b = gsh if ctx.split else (gsh, None)
        return gm, gls, gq, gop, g_a, g_b, None, None, None, None, None


class _Aux(dict):
    """rasterize's aux dict; "n_visible" is counted on the device when first read (two small
    kernels that a caller who does not read it does not pay for)."""

    def __missing__(self, key):
        if key == "n_visible":
            v = self[key] = (self["tiles_touched"] > 0).sum()
            return v
        raise KeyError(key)


def rasterize(means, scales, quats, opacities, sh, viewmat, K, W: int, H: int, bg=None, near: float = 0.01,
              far: float = 100.0, sh_degree: int | None = None, activated: bool = False,
              densification_info: torch.Tensor | None = None, proper_antialiasing: bool = False,
              timing: bool = False):
    """Renders one view. Returns (image [3, H, W], alpha [H, W], aux).

    Parameters follow Faster-GS's raw convention unless `activated=True`:
      means [N,3]; scales [N,3] log-scales (activated: positive scales); quats [N,4] (w, x, y, z),
      any norm; opacities [N] or [N,1] logits (activated: opacities in (0,1)); sh [N,K,3] SH
      coefficients, K in {1,4,9,16}, or the pair (DC [N,1,3], rest [N,K-1,3]) that trainers keep
      as two parameters; viewmat [4,4] world-to-camera (OpenCV axes); K [3,3] intrinsics.
    aux (gsplat's `meta`, cluster/build_env.sbatch:54; nothing in it makes the host wait):
      "tiles_touched"  [N] int32, tiles each Gaussian reaches (0 = culled)
      "visibility"     the same tensor: the mask FusedAdam(sparse=True).step(visibility=...) takes
      "n_instances"    int, the (tile, Gaussian) instances sorted (Faster-GS's n_instances)
      "n_buckets"      0-dim int32 device tensor, 32-entry buckets of the tile lists (n_buckets)
      "n_visible"      0-dim int64 device tensor, Gaussians with tiles_touched > 0
      "timings"        (timing=True only) a StageTimer: aux["timings"].result() gives the ms of
                       each forward stage and, once the backward has run, of the backward stages
    Gradients flow to means, scales, quats, opacities and sh. densification_info [2 or 3, N]
    float32 (optional, as the first argument of Faster-GS's backward): the backward adds this view's
    statistics to it (see densification_stats). proper_antialiasing: Faster-GS's setting of that
    name -- each splat's opacity is scaled by sqrt(det S / det(S + 0.3 I)) so that the 0.3 px^2
    low-pass does not add energy (S the projected 2D covariance); gradients include the factor.
    """
    means, scales, quats, opacities, _ = _prepare(means, scales, quats, opacities, sh, activated)
    cam = Camera.from_K(viewmat, K, W, H, near, far, proper_antialiasing, BINNING)
    if bg is None:
        bg = (0.0, 0.0, 0.0)
    bg = tuple(float(x) for x in (bg.tolist() if torch.is_tensor(bg) else bg))
    sh_a, sh_b = sh if isinstance(sh, (tuple, list)) else (sh, None)
    timer = StageTimer(True) if timing else None
    image, alpha, touched, n_buckets, m = _Rasterize3D.apply(means, scales, quats, opacities, sh_a, sh_b, cam,
                                                             sh_degree, bg, densification_info, timer)
    aux = _Aux(tiles_touched=touched, visibility=touched, n_instances=int(m.item()), n_buckets=n_buckets)
    if timer is not None:
        aux["timings"] = timer
    return image, alpha, aux


def _prepare(means, scales, quats, opacities, sh, activated):
    if opacities.dim() == 2:
        opacities = opacities.reshape(-1)
    if activated:
        scales = torch.log(scales)
        opacities = torch.logit(opacities)
    return means, scales, quats, opacities, tuple(sh) if isinstance(sh, (tuple, list)) else sh


@torch.no_grad()
def rasterize_inference(means, scales, quats, opacities, sh, viewmat, K, W: int, H: int, bg=None,
                        near: float = 0.01, far: float = 100.0, sh_degree: int | None = None,
                        activated: bool = False, proper_antialiasing: bool = False):
    """Forward only, for evaluation and viewers (Faster-GS's inference blend,
    upstream/upstream_main_kernels.patch:131-150): returns (image [3, H, W], alpha [H, W]), the
    same bits as rasterize, without the backward's bucket table, checkpoints or autograd state."""
    means, scales, quats, opacities, sh = _prepare(means, scales, quats, opacities, sh, activated)
    cam = Camera.from_K(viewmat, K, W, H, near, far, proper_antialiasing, BINNING)
    bg = (0.0, 0.0, 0.0) if bg is None else tuple(float(x) for x in (bg.tolist() if torch.is_tensor(bg) else bg))
    fs = forward_pass(means.detach(), scales.detach(), quats.detach(), opacities.detach(),
                      tuple(t.detach() for t in sh) if isinstance(sh, tuple) else sh.detach(), cam,
                      sh_degree=sh_degree, bg=bg, for_backward=False)
    return fs.image, fs.alpha


@torch.no_grad()
def pruning_scores(means, scales, quats, opacities, sh, viewmat, K, W: int, H: int, near: float = 0.01,
                   far: float = 100.0, sh_degree: int | None = None, activated: bool = False,
                   proper_antialiasing: bool = False, scores: torch.Tensor | None = None) -> torch.Tensor:
    """Per-Gaussian contribution of one view (the role of Faster-GS's pruning-score blend,
    upstream/upstream_main_kernels.patch:152-198): scores[g] += sum over the pixels g is blended
    into of its blending weight alpha * T, under the forward's rules. Pass the same `scores`
    ([N] float32 CUDA) for every view to accumulate over a set of views; returns it."""
    means, scales, quats, opacities, sh = _prepare(means, scales, quats, opacities, sh, activated)
    cam = Camera.from_K(viewmat, K, W, H, near, far, proper_antialiasing, BINNING)
    n = means.shape[0]
    if scores is None:
        scores = torch.zeros(n, dtype=torch.float32, device=means.device)
    if tuple(scores.shape) != (n,) or scores.dtype != torch.float32 or not scores.is_contiguous() \
            or scores.device != means.device:
        raise ValueError(f"scores must be a contiguous float32 [{n}] tensor on {means.device}")
    forward_pass(means.detach(), scales.detach(), quats.detach(), opacities.detach(),
                 tuple(t.detach() for t in sh) if isinstance(sh, tuple) else sh.detach(), cam,
                 sh_degree=sh_degree, _scores=scores)
    return scores
