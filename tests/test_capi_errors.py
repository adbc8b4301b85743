"""Error paths of the C ABI and of the Python operator surfaces.

The reference's extensions reject bad input before any work: toy2d's CHECK_INPUT (a CUDA tensor,
contiguous, the right dtype; toy2d/csrc/rasterize.cu:355-358) and phase0's argument checks
(shapes, one floating dtype, int32 tables, a non-empty image; phase0/csrc/macrotile/
bindings.cpp:54-78). Here every entry point of include/amdsplat.h returns a GS_ERR_* code with a
message (gs_last_error) and enqueues nothing; the Python surfaces raise.

  - Without a GPU (argument checks that come before anything touches the device): NULL
    pointers, negative or out-of-range sizes, unknown enums, invalid cameras, missing
    workspaces. Only NULL pointers are passed, so nothing could be dereferenced.
  - With a GPU (marked `gpu`): a workspace one byte short and a misaligned pointer, each with
    real device buffers of the full size, checking that the outputs were not touched and that
    the next, valid call succeeds and is right; bad tensors at the Python surfaces.
"""
import ctypes

import numpy as np
import pytest
import torch

from amdsplat import _lib
from amdsplat._lib import ptr

GS_ERR_ARG, GS_ERR_WORKSPACE, GS_ERR_ALIGN = 1, 2, 4


def cam(W=64, H=48, near=0.01, far=100.0, fx=50.0, flags=0):
    return _lib.make_camera(np.eye(4, dtype=np.float32), fx, fx, W / 2, H / 2, W, H, near, far, flags)


def expect(rc, code, text):
    msg = _lib.lib().gs_last_error().decode()
    assert rc == code, (rc, msg)
    assert text in msg, msg


# ---------------------------------------------------------------------------------------
# Host-side argument checks (no GPU needed)
# ---------------------------------------------------------------------------------------
def test_negative_sizes_and_nulls_are_refused():
    L = _lib.lib()
    expect(L.gs_scan_u32(None, None, -1, None, 0, None), GS_ERR_ARG, "invalid scan arguments")
    expect(L.gs_sum_u32(None, 5, None, None), GS_ERR_ARG, "invalid sum arguments")
    expect(L.gs_preprocess_fwd(None, None, None, None, None, None, 10, 16, 3, cam(), None, None, None, None, None),
           GS_ERR_ARG, "null")
    expect(L.gs_preprocess_fwd(None, None, None, None, None, None, -1, 16, 3, cam(), None, None, None, None, None),
           GS_ERR_ARG, "n must be >= 0")
    expect(L.gs_count_begin(None, -1, 0, None), GS_ERR_ARG, "invalid count arguments")
    expect(L.gs_count_end(None), GS_ERR_ARG, "null pointer")
    expect(L.gs_bin_fill_3d(None, None, None, None, -5, cam(), 0, None, None, None, None, None, None, 0, None),
           GS_ERR_ARG, "invalid sizes")
    expect(L.gs_bin_fill_3d(None, None, None, None, 10, cam(), 5, None, None, None, None, None, None, 0, None),
           GS_ERR_ARG, "null output")
    expect(L.gs_densification_stats(None, None, 10, 64, 48, 4, None, None), GS_ERR_ARG, "")  # rows must be 2 or 3
    expect(L.gs_l1_ssim_fwd(None, None, 3, 0, 16, ctypes.c_float(0.2), None, None, None, 0, None), GS_ERR_ARG,
           "invalid image size")
    expect(L.gs_l1_ssim_bwd(None, None, None, 3, 16, 16, ctypes.c_float(0.2), None, None, None), GS_ERR_ARG,
           "null pointer")


def test_unknown_enums_are_refused():
    L = _lib.lib()
    expect(L.gs2d_pack(7, _lib.GS_FLOAT32, None, None, None, None, 4, None, None), GS_ERR_ARG, "invalid rules 7")
    expect(L.gs2d_pack(1, 5, None, None, None, None, 4, None, None), GS_ERR_ARG, "invalid dtype 5")  # toy2d rules
    expect(L.gs2d_rects_phase0(9, None, None, None, 4, 16, 16, None, None, None), GS_ERR_ARG, "invalid dtype 9")
    expect(L.gs_bin_fill_rect(None, None, 9, None, 4, 2, 2, 0, None, None, None, None, None, None, 0, None, 0,
                              None), GS_ERR_ARG, "invalid depth dtype")
    expect(L.gs_l1_ssim_fwd(None, None, 3, 16, 16, ctypes.c_float(1.5), None, None, None, 0, None), GS_ERR_ARG,
           "null pointer")


def test_invalid_cameras_are_refused():
    L = _lib.lib()
    for c, text in ((cam(near=0.0), "near"), (cam(near=5.0, far=1.0), "near"), (cam(W=0), "image size"),
                    (cam(fx=-1.0), "focal")):
        expect(L.gs_bin_prepare_3d(None, None, None, 10, c, None, None, None, 0, None), GS_ERR_ARG, text)
        expect(L.gs_preprocess_fwd(None, None, None, None, None, None, 10, 16, 3, c, None, None, None, None, None),
               GS_ERR_ARG, text)
    expect(L.gs_bin_prepare_3d(None, None, None, 10, None, None, None, None, 0, None), GS_ERR_ARG, "camera is NULL")


def test_sh_layout_checks():
    L = _lib.lib()
    expect(L.gs_preprocess_fwd(None, None, None, None, None, None, 10, 5, 1, cam(), None, None, None, None, None),
           GS_ERR_ARG, "sh_coeffs must be 1, 4, 9 or 16")
    expect(L.gs_preprocess_fwd(None, None, None, None, None, None, 10, 4, 2, cam(), None, None, None, None, None),
           GS_ERR_ARG, "sh_degree 2 needs more than 4")


def test_adam_group_checks():
    L = _lib.lib()
    groups = (_lib.GsAdamGroup * (_lib.GS_ADAM_MAX_GROUPS + 1))()
    expect(L.gs_adam_step(groups, _lib.GS_ADAM_MAX_GROUPS + 1, 4, None, None), GS_ERR_ARG, "parameter groups")
    g = (_lib.GsAdamGroup * 1)()
    g[0].n_elements, g[0].moment_dtype, g[0].step = 12, _lib.GS_FLOAT32, 1
    expect(L.gs_adam_step(g, 1, 4, None, None), GS_ERR_ARG, "group 0")  # null arrays
    g[0].n_elements = 0
    g[0].step = 0
    expect(L.gs_adam_step(g, 1, 4, None, None), GS_ERR_ARG, "group 0: step must be >= 1")
    g[0].step, g[0].moment_dtype = 1, _lib.GS_FLOAT64
    expect(L.gs_adam_step(g, 1, 4, None, None), GS_ERR_ARG, "group 0: moments")


def test_missing_workspace_is_refused():
    L = _lib.lib()
    n = 1 << 20
    assert L.gs_scan_workspace_size(n) > 0
    expect(L.gs_scan_u32(None, None, 0, None, 0, None), GS_ERR_ARG, "")  # out NULL
    c = cam(640, 480)
    need = L.gs_bin_prepare_workspace_size(n)
    assert need > 0
    # a size query never asks for less than the call checks for
    assert L.gs_bin_fill_3d_workspace_size(n, 5 * n, c) <= L.gs_bin_workspace_size(n, 5 * n, 40, 30, 0)


# ---------------------------------------------------------------------------------------
# Device-side failures (real buffers of the full size; nothing may be written)
# ---------------------------------------------------------------------------------------
@pytest.mark.gpu
def test_scan_workspace_one_byte_short_then_a_good_call():
    L = _lib.lib()
    n = 100_003
    x = torch.randint(0, 50, (n,), dtype=torch.int32, device="cuda")
    out = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
    need = L.gs_scan_workspace_size(n)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    expect(L.gs_scan_u32(ptr(x), ptr(out), n, ptr(ws), need - 1, None), GS_ERR_WORKSPACE, "scan workspace too small")
    torch.cuda.synchronize()
    assert bool((out == -7).all())
    assert L.gs_scan_u32(ptr(x), ptr(out), n, ptr(ws), need, None) == 0
    want = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(x.cpu().long(), 0)])
    assert torch.equal(out.cpu().long(), want)


@pytest.mark.gpu
def test_fill_workspace_short_then_a_good_call():
    """gs_bin_fill_3d with a workspace one byte short: GS_ERR_WORKSPACE, outputs untouched, then the
    same call with the full workspace gives the forward's own lists."""
    from amdsplat import raster3d as R
    from amdsplat import scenes

    sc = scenes.small_scene(3000, 160, 120, seed=3, sh_coeffs=16)
    p = [t.cuda().contiguous() for t in sc.params()]
    fs = R.forward_pass(*p, sc.cameras[0], sh_degree=3)
    torch.cuda.synchronize()
    L = _lib.lib()
    cc = fs.ccam
    n, m, T = fs.n, fs.m, fs.cam.n_tiles
    dkeys = torch.empty(n, dtype=torch.int32, device="cuda")
    wc = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
    rec = torch.empty_like(fs.rec)
    touched = torch.empty_like(fs.touched)
    sh = p[4]
    assert L.gs_preprocess_fwd(ptr(p[0]), ptr(p[1]), ptr(p[2]), ptr(p[3]), ptr(sh), None, n, 16, 3, cc, ptr(rec),
                               ptr(touched), ptr(dkeys), ptr(wc), None) == 0
    order = torch.empty(n, dtype=torch.int32, device="cuda")
    offs = torch.empty(n + 1, dtype=torch.int32, device="cuda")
    pws = torch.empty(L.gs_bin_prepare_workspace_size(n), dtype=torch.uint8, device="cuda")
    assert L.gs_bin_prepare_3d(ptr(rec), ptr(touched), ptr(dkeys), n, cc, ptr(order), ptr(offs), ptr(pws),
                               pws.numel(), None) == 0
    need = L.gs_bin_fill_3d_workspace_size(n, m, cc)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    pl = torch.full((m,), -3, dtype=torch.int32, device="cuda")
    ranges = torch.full((T, 2), -3, dtype=torch.int32, device="cuda")
    boff = torch.full((T + 1,), -3, dtype=torch.int32, device="cuda")
    expect(L.gs_bin_fill_3d(ptr(rec), ptr(dkeys), ptr(order), ptr(offs), n, cc, m, None, ptr(pl), ptr(ranges),
                            ptr(boff), None, ptr(ws), need - 1, None), GS_ERR_WORKSPACE, "binning workspace too small")
    torch.cuda.synchronize()
    assert bool((pl == -3).all()) and bool((ranges == -3).all()) and bool((boff == -3).all())
    assert L.gs_bin_fill_3d(ptr(rec), ptr(dkeys), ptr(order), ptr(offs), n, cc, m, None, ptr(pl), ptr(ranges),
                            ptr(boff), None, ptr(ws), need, None) == 0
    torch.cuda.synchronize()
    assert torch.equal(pl, fs.point_list) and torch.equal(ranges, fs.ranges) and torch.equal(boff, fs.bucket_offsets)


@pytest.mark.gpu
@pytest.mark.parametrize("side", [0, 1])
def test_count_readback_pairs_and_sums(side):
    """gs_count_begin / gs_count_end: the sum of the counts on either stream; an end without a
    begin and a second begin before the end are refused, and the next pair works."""
    L = _lib.lib()
    m = ctypes.c_uint64()
    expect(L.gs_count_end(ctypes.byref(m)), GS_ERR_ARG, "without gs_count_begin")
    for n in (0, 1, 63, 64, 1000, 300_001):
        c = torch.randint(0, 1 << 20, (n,), dtype=torch.int32, device="cuda")
        assert L.gs_count_begin(ptr(c), n, side, None) == 0
        if n == 1000:
            expect(L.gs_count_begin(ptr(c), n, side, None), GS_ERR_ARG, "was not ended")
        assert L.gs_count_end(ctypes.byref(m)) == 0
        assert m.value == int(c.long().sum()), n
    expect(L.gs_count_end(ctypes.byref(m)), GS_ERR_ARG, "without gs_count_begin")


@pytest.mark.gpu
def test_loss_workspace_short_then_a_good_call():
    L = _lib.lib()
    C, H, W = 3, 64, 80
    g = torch.Generator().manual_seed(3)
    x = torch.rand(C, H, W, generator=g).cuda()
    y = torch.rand(C, H, W, generator=g).cuda()
    loss = torch.full((3,), -1.0, device="cuda")
    need = L.gs_l1_ssim_workspace_size(C, H, W)
    ws = torch.empty(need + 16, dtype=torch.uint8, device="cuda")
    expect(L.gs_l1_ssim_fwd(ptr(x), ptr(y), C, H, W, ctypes.c_float(0.2), None, ptr(loss), ptr(ws), need - 1, None),
           GS_ERR_WORKSPACE, "workspace too small")
    torch.cuda.synchronize()
    assert bool((loss == -1.0).all())
    assert L.gs_l1_ssim_fwd(ptr(x), ptr(y), C, H, W, ctypes.c_float(0.2), None, ptr(loss), ptr(ws), need, None) == 0
    torch.cuda.synchronize()
    from amdsplat import l1_ssim_loss
    ref = l1_ssim_loss(x, y, 0.2)
    assert torch.allclose(loss[0], ref, rtol=1e-6, atol=0)


@pytest.mark.gpu
def test_misaligned_records_are_refused_then_a_good_call():
    L = _lib.lib()
    n = 1000
    c = cam(160, 120)
    g = torch.Generator().manual_seed(5)
    means = (torch.rand(n, 3, generator=g) - 0.5).cuda()
    means[:, 2] += 4.0
    ls = torch.full((n, 3), -3.0).cuda()
    q = torch.randn(n, 4, generator=g).cuda()
    op = torch.zeros(n).cuda()
    sh = torch.rand(n, 16, 3, generator=g).cuda()
    big = torch.full((n * 16 + 4,), -9.0, device="cuda")
    touched = torch.full((n,), -9, dtype=torch.int32, device="cuda")
    expect(L.gs_preprocess_fwd(ptr(means), ptr(ls), ptr(q), ptr(op), ptr(sh), None, n, 16, 3, c, ptr(big) + 4,
                               ptr(touched), None, None, None), GS_ERR_ALIGN, "16-byte")
    torch.cuda.synchronize()
    assert bool((big == -9.0).all()) and bool((touched == -9).all())
    assert L.gs_preprocess_fwd(ptr(means), ptr(ls), ptr(q), ptr(op), ptr(sh), None, n, 16, 3, c, ptr(big),
                               ptr(touched), None, None, None) == 0
    torch.cuda.synchronize()
    assert int((touched > 0).sum()) > 0


# ---------------------------------------------------------------------------------------
# The Python surfaces
# ---------------------------------------------------------------------------------------
@pytest.mark.gpu
def test_rasterize_rejects_bad_tensors_and_accepts_strided_views():
    """Wrong device, dtype and shape raise before any launch; a non-contiguous (strided) view is
    taken as its contiguous copy (the reference's extensions raise there instead): same image."""
    from amdsplat import rasterize, scenes

    sc = scenes.small_scene(2000, 96, 64, seed=9, sh_coeffs=16)
    c = sc.cameras[0]
    K = torch.tensor([[c.fx, 0.0, c.cx], [0.0, c.fy, c.cy], [0.0, 0.0, 1.0]])
    p = [t.cuda().contiguous() for t in sc.params()]
    args = dict(viewmat=c.viewmat, K=K, W=c.width, H=c.height)
    with pytest.raises(ValueError, match="CUDA"):
        rasterize(*[t.cpu() for t in p], **args)
    with pytest.raises(ValueError, match="float32"):
        rasterize(p[0].double(), *p[1:], **args)
    with pytest.raises(ValueError, match="shape"):
        rasterize(p[0][:, :2].contiguous(), *p[1:], **args)
    with pytest.raises(ValueError, match="sh must"):
        rasterize(*p[:4], p[4][:, :5].contiguous(), **args)
    img, _, _ = rasterize(*p, **args)
    strided = [torch.cat([t, t], 1)[:, :t.shape[1]] if t.dim() > 1 else torch.stack([t, t], 1)[:, 0] for t in p[:4]]
    assert not strided[0].is_contiguous()
    img2, _, _ = rasterize(*strided, p[4], **args)
    torch.cuda.synchronize()
    assert torch.equal(img, img2)


@pytest.mark.gpu
def test_2d_surfaces_reject_mixed_dtypes_and_cpu_tensors():
    from gs2d import raster as gr
    from splat2d import ops as so

    n = 16
    means = torch.rand(n, 2, device="cuda") * 32
    with pytest.raises(RuntimeError, match="dtype"):
        gr._check(means, torch.rand(n, 3, device="cuda").double(), torch.rand(n, 3, device="cuda"),
                  torch.rand(n, device="cuda"))
    with pytest.raises((RuntimeError, ValueError)):
        so.render(means.cpu(), torch.rand(n, 3), torch.zeros(n), torch.rand(n, 3), 32, 32)
