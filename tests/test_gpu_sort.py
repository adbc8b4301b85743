"""GPU checks of the radix sorts behind the binning, against what the definition of a stable
sort fixes: numpy's stable argsort of the same keys, and the exclusive scan of the counts in
that order. No oracle is involved; the inputs are chosen to reach every sort configuration
(1 to 4 passes, 4 / 8 / 16 rounds per tile, one tile up to thousands of tiles, keys that are
all equal or all distinct) and the tile sort's ranges on canvases with up to 16384 tiles (the
14-bit tile sort, whose scratch the workspace size must cover).
"""
import numpy as np
import pytest
import torch

from amdsplat import _lib
from amdsplat import raster2d as R2
from amdsplat._lib import call, ptr

pytestmark = pytest.mark.gpu

NEAR, FAR = 0.01, 100.0


def host_order_key(v: float) -> int:
    u = int(np.float32(v).view(np.uint32))
    return (~u & 0xFFFFFFFF) if u & 0x80000000 else (u | 0x80000000)


DKEY_CULL = host_order_key(FAR) - host_order_key(NEAR)  # 27 bits for near/far = 0.01 / 100


def camera(W=640, H=480, near=NEAR, far=FAR):
    return _lib.make_camera(np.eye(4, dtype=np.float32), 500.0, 500.0, W / 2, H / 2, W, H, near, far)


def depth_keys(n, kind, rng, cull=DKEY_CULL):
    if kind == "distinct":
        k = rng.integers(1, cull, n, dtype=np.int64)
    elif kind == "few_values":
        k = rng.choice(rng.integers(1, cull, 37, dtype=np.int64), n)
    elif kind == "culled_mix":  # a third culled (the largest key), the rest spread
        k = rng.integers(1, cull, n, dtype=np.int64)
        k[rng.random(n) < 0.33] = cull
    else:  # "equal"
        k = np.full(n, min(12345, cull - 1), np.int64)
    return k.astype(np.uint32)


# tiles of 1024, 2048 and 4096 keys (by size): one partial tile, exact multiples, one key more
@pytest.mark.parametrize("n", [1, 63, 1024, 1025, 4097, 100_003, 524_288, 524_289, 1_000_000, 8_388_608,
                               9_000_001])
@pytest.mark.parametrize("kind", ["distinct", "few_values", "culled_mix", "equal"])
def test_depth_order_is_the_stable_argsort(n, kind):
    check_depth_order(n, kind, 9)


@pytest.mark.parametrize("n", [100_003, 1_000_000])
def test_depth_order_offsets_beyond_31_bits(n):
    """Instance counts whose total passes 2^31 (the offsets are unsigned 32-bit)."""
    check_depth_order(n, "distinct", (1 << 32) // n - 1)


# near / far planes whose depth keys take 1 and 2 passes of 9 bits (and 3 for the default)
@pytest.mark.parametrize("far", [1.0 + 400 * 2.0 ** -23, 1.03, 60.0])
@pytest.mark.parametrize("n", [1025, 1_000_000])
def test_depth_order_few_key_bits(n, far):
    check_depth_order(n, "culled_mix", 9, near=1.0, far=far)


def check_depth_order(n, kind, max_count, near=NEAR, far=FAR):
    rng = np.random.default_rng(n + len(kind))
    cull = host_order_key(far) - host_order_key(near)
    keys = depth_keys(n, kind, rng, cull)
    counts = rng.integers(0, max_count, n).astype(np.uint32)
    dev = torch.device("cuda")
    kd = torch.from_numpy(keys.view(np.int32)).to(dev)
    cd = torch.from_numpy(counts.view(np.int32)).to(dev)
    order = torch.empty(n, dtype=torch.int32, device=dev)
    offsets = torch.empty(n + 1, dtype=torch.int32, device=dev)
    ws = torch.empty(max(_lib.size_call("gs_bin_prepare_workspace_size", n), 1), dtype=torch.uint8, device=dev)
    cam = camera(near=near, far=far)
    call("gs_bin_prepare_3d", None, ptr(cd), ptr(kd), n, cam, ptr(order), ptr(offsets), ptr(ws), ws.numel(),
         _lib.stream_handle(dev))
    want = np.argsort(keys, kind="stable")
    assert np.array_equal(order.cpu().numpy(), want)
    scan = np.zeros(n + 1, np.int64)
    np.cumsum(counts[want], out=scan[1:])
    assert scan[-1] < 1 << 32
    assert np.array_equal(offsets.cpu().numpy().view(np.uint32).astype(np.int64), scan)
    if n == 100_003:  # without the offsets (nor the counts): the same order
        order2 = torch.empty_like(order)
        call("gs_bin_prepare_3d", None, None, ptr(kd), n, cam, ptr(order2), None, ptr(ws), ws.numel(),
             _lib.stream_handle(dev))
        assert torch.equal(order2, order)


def numpy_rect_binning(rects, depth, tiles_x, T):
    """Lists of a stable depth order, instances emitted row-major per rectangle, then stably
    sorted by tile; ranges and 32-entry bucket offsets."""
    order = np.argsort(depth, kind="stable")
    r = rects[order].astype(np.int64)
    w, h = r[:, 2] - r[:, 0], r[:, 3] - r[:, 1]
    cnt = np.where((w > 0) & (h > 0), w * h, 0)
    m = int(cnt.sum())
    g = np.repeat(np.arange(len(order)), cnt)
    start = np.zeros(len(order), np.int64)
    np.cumsum(cnt[:-1], out=start[1:])
    local = np.arange(m) - start[g]
    tile = (r[g, 1] + local // w[g]) * tiles_x + r[g, 0] + local % w[g]
    srt = np.argsort(tile, kind="stable")
    point_list = order[g[srt]].astype(np.int32)
    per_tile = np.bincount(tile, minlength=T)
    begin = np.zeros(T + 1, np.int64)
    np.cumsum(per_tile, out=begin[1:])
    ranges = np.stack([begin[:-1], begin[1:]], 1)
    boff = np.zeros(T + 1, np.int64)
    np.cumsum((per_tile + 31) // 32, out=boff[1:])
    return point_list, ranges, boff


@pytest.mark.parametrize("W,H,n,rmax", [
    (333, 250, 5_000, 5),           # 336 tiles
    (1297, 840, 400_000, 5),        # 4346 tiles
    (2048, 2048, 200_000, 16),      # 16384 tiles, ~10M instances
    (8192, 40, 60_000, 40),         # 512 x 3 tiles: the widest canvas of the span binning
    (40, 8192, 60_000, 40),         # 3 x 512 tiles: the tallest
    (8208, 40, 60_000, 40),         # 513 tiles wide: instances emitted and radix-sorted by tile
    (40, 8208, 60_000, 40),         # 513 tiles tall: the same
    (2000, 1200, 30_000, 200),      # wide rectangles: spans of up to 125 tiles
    (17, 17, 3_000, 3),             # 2 x 2 tiles
    (16, 16, 1_000, 2),             # one tile
])
@pytest.mark.parametrize("binning", ["spans", "radix"])
def test_rect_binning_matches_the_stable_sort(W, H, n, rmax, binning):
    rng = np.random.default_rng(W * H + n)
    tiles_x, tiles_y = (W + 15) // 16, (H + 15) // 16
    T = tiles_x * tiles_y
    x0 = rng.integers(-2, tiles_x, n)
    y0 = rng.integers(-2, tiles_y, n)
    rects = np.stack([x0, y0, x0 + rng.integers(0, rmax, n), y0 + rng.integers(0, rmax, n)], 1).astype(np.int32)
    rects[:, 2:] = np.minimum(rects[:, 2:], [tiles_x, tiles_y])
    rects[:, :2] = np.maximum(rects[:, :2], 0)
    depth = rng.choice(rng.random(n // 3 + 1).astype(np.float32), n)  # ties in depth
    dev = torch.device("cuda")
    rd = torch.from_numpy(rects).to(dev).contiguous()
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    call("gs_rect_counts", ptr(rd), n, tiles_x, tiles_y, ptr(counts), _lib.stream_handle(dev))
    rb = R2.bin_rects(rd, counts, torch.from_numpy(depth).to(dev), W, H, binning=binning)
    pl, ranges, boff = numpy_rect_binning(rects, depth, tiles_x, T)
    assert len(pl) == rb.point_list.numel()
    assert np.array_equal(rb.point_list.cpu().numpy(), pl)
    assert np.array_equal(rb.ranges.cpu().numpy().astype(np.int64), ranges)
    assert np.array_equal(rb.bucket_offsets.cpu().numpy().astype(np.int64), boff)


@pytest.mark.parametrize("n,offset", [(0, 0), (1, 0), (3, 1), (4097, 0), (1_000_003, 1), (15_625, 0)])
def test_sum_u32(n, offset):
    """gs_sum_u32 (the instance count of the 3D forward) against numpy's uint64 sum, over values up to
    2^31 (the total exceeds 32 bits) and at an input that is not 16-byte aligned."""
    rng = np.random.default_rng(n)
    vals = rng.integers(0, 1 << 31, n + offset, dtype=np.int64).astype(np.uint32)
    dev = torch.device("cuda")
    d = torch.from_numpy(vals.view(np.int32)).to(dev)
    out = torch.full((1,), -1, dtype=torch.int64, device=dev)
    call("gs_sum_u32", d.data_ptr() + 4 * offset, n, ptr(out), _lib.stream_handle(dev))
    assert int(out.item()) == int(vals[offset:].astype(np.uint64).sum())
