"""GPU check of the allocation-free L1 + D-SSIM forward (gs_l1_ssim_fwd_noalloc) against the
workspace entry point gs_l1_ssim_fwd, both called through the C ABI: the same kernels, so the
loss parts and the per-pixel SSIM derivative maps must be the same bits. Two calls in a row,
the second on a smaller image (the static buffer keeps the first call's partial sums), then a
third at the first size again; an image larger than the static buffer is refused on the host
before anything is launched."""
import ctypes

import numpy as np
import pytest
import torch

from amdsplat import _lib
from amdsplat._lib import ptr

pytestmark = pytest.mark.gpu


def _images(c, h, w, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(c, h, w, generator=g)
    y = (x + 0.2 * torch.randn(c, h, w, generator=g)).clamp(0, 1)
    return x.cuda(), y.cuda()


def _with_workspace(x, y, lam):
    c, h, w = x.shape
    dmap = torch.empty(c, 3, h, w, device="cuda")
    loss = torch.empty(3, device="cuda")
    ws = torch.empty(max(_lib.size_call("gs_l1_ssim_workspace_size", c, h, w), 1), dtype=torch.uint8, device="cuda")
    _lib.call("gs_l1_ssim_fwd", ptr(x), ptr(y), c, h, w, lam, ptr(dmap), ptr(loss), ptr(ws), ws.numel(),
              _lib.stream_handle())
    return loss, dmap


def _no_alloc(x, y, lam):
    c, h, w = x.shape
    dmap = torch.empty(c, 3, h, w, device="cuda")
    loss = torch.empty(3, device="cuda")
    _lib.call("gs_l1_ssim_fwd_noalloc", ptr(x), ptr(y), c, h, w, lam, ptr(dmap), ptr(loss), _lib.stream_handle())
    return loss, dmap


@pytest.mark.parametrize("lam", [0.2, 1.0])
def test_no_alloc_forward_equals_workspace_forward(lam):
    # 1297x840 (the training workload's frame), then a smaller ragged image, then the first again
    for (c, h, w), seed in (((3, 840, 1297), 1), ((3, 37, 53), 2), ((3, 840, 1297), 3)):
        print(f"[no-alloc] shape {(c, h, w)} seed {seed} lambda {lam}", flush=True)
        x, y = _images(c, h, w, seed)
        l_ws, d_ws = _with_workspace(x, y, lam)
        l_na, d_na = _no_alloc(x, y, lam)
        torch.cuda.synchronize()
        assert torch.equal(l_ws, l_na), (l_ws.tolist(), l_na.tolist())
        assert torch.equal(d_ws, d_na)
        assert np.isfinite(l_na.cpu().numpy()).all()


def test_no_alloc_forward_without_dmap_and_on_a_side_stream():
    x, y = _images(3, 64, 80, 5)
    l_ws, _ = _with_workspace(x, y, 0.2)
    loss = torch.empty(3, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _lib.call("gs_l1_ssim_fwd_noalloc", ptr(x), ptr(y), 3, 64, 80, 0.2, None, ptr(loss), _lib.stream_handle())
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(l_ws, loss)


def test_no_alloc_refuses_images_beyond_its_buffer():
    L = _lib.lib()
    max_tiles = 131072
    # 3 channels x 256 x 256 tiles of 16 px = 196608 tile-channels: refused on the host
    h = w = 256 * 16
    # real buffers of the full size (about 200 MB each): should the size check ever regress, the
    # call reads and writes inside them and the assertions below fail, instead of a fault
    img = torch.zeros(3, h, w, device="cuda")
    tgt = torch.zeros(3, h, w, device="cuda")
    loss = torch.zeros(3, device="cuda")
    rc = L.gs_l1_ssim_fwd_noalloc(ptr(img), ptr(tgt), 3, h, w, ctypes.c_float(0.2), None, ptr(loss), None)
    torch.cuda.synchronize()
    del img, tgt
    assert rc == 1  # GS_ERR_ARG
    assert torch.equal(loss, torch.zeros(3, device="cuda"))  # nothing was launched
    assert b"static" in L.gs_last_error()
    assert 3 * (h // 16) * (w // 16) > max_tiles
    # the next call succeeds (no pending error is left behind)
    x, y = _images(1, 16, 16, 7)
    l_ws, _ = _with_workspace(x, y, 0.2)
    l_na, _ = _no_alloc(x, y, 0.2)
    torch.cuda.synchronize()
    assert torch.equal(l_ws, l_na)
