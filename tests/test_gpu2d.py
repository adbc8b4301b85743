"""GPU parity of the 2D surfaces (gs2d with toy2d rules, splat2d with phase0 rules): the HIP
kernels, called through the C ABI by the drop-in packages, against the golden fixtures of the
reference's own Python code and against the CPU oracle.

Bars: binning (rectangles, depth order, lists, ranges, buckets) bit-exact; per-pixel counts
bit-exact against the oracle; float32 images and gradients within the reference's 1e-5 gate
(toy2d/tests/test_cuda.py:8-31, phase0/tests/gradcheck/test_gradcheck.py:62-70); float64
within 1e-12 (forward) / 1e-10 (gradients) (test_gradcheck.py:73-100).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle2d as O2
import gs2d
import splat2d
from gs2d.params import Gaussians2D, radii_from_cov
from splat2d import ops as P0
from amdsplat import raster2d as R2

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
TOY = ["tiny", "sparse_odd", "dense", "opaque"]
PH0 = [f"seed{s}_n{n}" for s in (0, 1, 2) for n in (8, 32)] + ["dense_n96", "sparse_n150"]


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel(a, b):
    a = a.detach().double().cpu().numpy() if torch.is_tensor(a) else np.asarray(a, np.float64)
    b = b.detach().double().cpu().numpy() if torch.is_tensor(b) else np.asarray(b, np.float64)
    nb = np.linalg.norm(b.ravel())
    d = np.linalg.norm((a - b).ravel())
    return float(d / nb) if nb > 0 else float(d)


def cuda(a, dtype=None):
    t = torch.as_tensor(a).cuda()
    return t.to(dtype) if dtype is not None else t


# ---------------------------------------------------------------------------------------
# toy2d / gs2d
# ---------------------------------------------------------------------------------------
def toy_bins(f):
    return gs2d.bin_gaussians(cuda(f["means"]), cuda(f["radii"]), cuda(f["depth"]), int(f["H"]), int(f["W"]))


@pytest.mark.parametrize("name", TOY)
def test_gs2d_binning_bit_exact(name):
    f = load(f"toy2d_{name}")
    b = toy_bins(f)
    torch.cuda.synchronize()
    assert np.array_equal(b.rect.cpu().numpy(), f["rect"])
    assert np.array_equal(b.order.cpu().numpy(), f["order"])
    assert np.array_equal(b.point_list.cpu().numpy(), f["point_list"])
    assert np.array_equal(b.ranges.cpu().numpy(), f["ranges"])
    assert np.array_equal(b.bucket_offsets.cpu().numpy(), f["bucket_offsets"])
    assert np.array_equal(b.bucket_to_tile.cpu().numpy(), f["bucket_to_tile"])
    assert b.num_buckets == int(f["num_buckets"])


@pytest.mark.parametrize("backend", ["splat", "pixel"])
@pytest.mark.parametrize("name", TOY)
def test_gs2d_float32_matches_reference(name, backend):
    """toy2d/tests/test_cuda.py:17-31: fp32 GPU vs the fp64 reference, rel err < 1e-5."""
    f = load(f"toy2d_{name}")
    bins = toy_bins(f)
    x = [cuda(f[k], torch.float32).requires_grad_(True) for k in ("means", "conic", "color", "opacity")]
    out = gs2d.rasterize(*x, bins, cuda(f["bg"], torch.float32), backend=backend)
    assert rel(out, f["image"]) < 1e-5
    grads = torch.autograd.grad(out, x, cuda(f["dout"], torch.float32))
    for key, g in zip(("g_means", "g_conic", "g_color", "g_opacity"), grads):
        assert rel(g, f[key]) < 1e-5, f"{backend}/{name}/{key}: {rel(g, f[key]):.2e}"


@pytest.mark.parametrize("backend", ["splat", "pixel"])
@pytest.mark.parametrize("name", TOY)
def test_gs2d_float64(name, backend):
    f = load(f"toy2d_{name}")
    bins = toy_bins(f)
    x = [cuda(f[k]).requires_grad_(True) for k in ("means", "conic", "color", "opacity")]
    out = gs2d.rasterize(*x, bins, cuda(f["bg"]), backend=backend)
    assert rel(out, f["image"]) < 1e-12
    grads = torch.autograd.grad(out, x, cuda(f["dout"]))
    for key, g in zip(("g_means", "g_conic", "g_color", "g_opacity"), grads):
        assert rel(g, f[key]) < 1e-9, f"{backend}/{name}/{key}: {rel(g, f[key]):.2e}"


@pytest.mark.parametrize("name", TOY)
def test_gs2d_forward_matches_oracle_bit_for_bit(name):
    f = load(f"toy2d_{name}")
    bins = toy_bins(f)
    W, H = int(f["W"]), int(f["H"])
    p32 = [f[k].astype(np.float32) for k in ("means", "conic", "color", "opacity")]
    e = gs2d.raster.ext()
    out, fT, nc, bstate = e.forward(*[cuda(a) for a in p32], cuda(f["bg"], torch.float32), bins.ranges,
                                    bins.point_list, bins.bucket_offsets, bins.num_buckets, H, W, True)
    rects, _ = O2.rects_toy(f["means"].astype(np.float32), f["radii"], W, H)
    order, pl, ranges, boff = O2.bin_rects(rects, f["depth"], W, H)
    ref = O2.forward(O2.TOY2D, *p32, pl, ranges, boff, W, H, bg=f["bg"])
    assert np.array_equal(nc.cpu().numpy(), ref["n_contrib"])
    assert np.abs(out.cpu().numpy() - ref["image"]).max() <= 1e-6
    assert np.abs(fT.cpu().numpy() - ref["final_T"]).max() <= 1e-6
    # checkpoints the backward reads (bucket start < the pixel's n_contrib)
    ck, rck = bstate.cpu().numpy(), ref["ckpt"]
    for tile in range(len(ranges)):
        for b in range(int(boff[tile]), int(boff[tile + 1])):
            bstart = (b - int(boff[tile])) * 32
            tx, ty = tile % ((W + 15) // 16), tile // ((W + 15) // 16)
            for t in range(256):
                px, py = tx * 16 + t % 16, ty * 16 + t // 16
                if px < W and py < H and ref["n_contrib"][py, px] > bstart:
                    assert np.abs(ck[b, t] - rck[b, t]).max() <= 1e-6


def test_gs2d_bucket_states_after_a_tile_stops_are_zero():
    """600 nearly opaque splats over one 16x16 tile: every pixel stops within the first bucket, so the
    workgroup stops at its second 256-entry round. The reference leaves the states of the buckets
    it did not reach zero (toy2d/csrc/rasterize.cu:131-133, 383); here the output is allocated
    without clearing (poisoned first with NaN through the caching allocator) and the kernel zeroes
    those slots itself."""
    n, H, W = 600, 16, 16
    means = torch.full((n, 2), 8.0, device="cuda")
    conic = torch.tensor([[0.01, 0.0, 0.01]], device="cuda").repeat(n, 1)
    color = torch.rand(n, 3, generator=torch.Generator().manual_seed(3)).cuda()
    opacity = torch.full((n,), 0.99, device="cuda")
    radii = torch.full((n,), 30, dtype=torch.int32, device="cuda")
    depth = torch.arange(n, dtype=torch.float32, device="cuda")
    bins = gs2d.bin_gaussians(means, radii, depth, H, W)
    assert bins.num_buckets == 19
    poison = torch.full((bins.num_buckets, 256, 4), float("nan"), device="cuda")
    del poison
    e = gs2d.raster.ext()
    bg = torch.zeros(3, device="cuda")
    out, fT, nc, bstate = e.forward(means, conic, color, opacity, bg, bins.ranges, bins.point_list,
                                    bins.bucket_offsets, bins.num_buckets, H, W, True)
    torch.cuda.synchronize()
    # every pixel stopped within the first bucket (all 600 splats cover every pixel with alpha > 1/255)
    assert int(nc.max()) < 32
    b = bstate.cpu()
    assert torch.equal(b[8:], torch.zeros_like(b[8:]))  # rounds the workgroup never started
    assert torch.equal(b[0, :, 0], torch.ones(256))  # the first state: T = 1 (toy2d: T first)
    assert not torch.isnan(b).any()


@pytest.mark.parametrize("binning,backend", [("spans", "splat"), ("radix", "splat"), ("radix", "pixel")])
def test_gs2d_bench_scene_against_oracle(binning, backend, monkeypatch):
    """512x512, 50k Gaussians of the reference benchmark: pair / bucket counts of its results
    file, bit-exact lists and counts, forward within 1e-5, gradients within 1e-4 (atomic order);
    with either tile binning, and the per-pixel backward (a wavefront's pixels' gradients of each
    splat summed before its atomics) as well as the bucketed one."""
    monkeypatch.setattr(R2, "BINNING", binning)
    rows = json.loads((GOLD / "toy2d_bench_counts.json").read_text())["rows"]
    row = rows[1]
    S, n = row["size"], row["n"]
    g = Gaussians2D(n, S, S, seed=0)
    with torch.no_grad():
        means, conic, color, opacity, cov = (t.detach() for t in g.activated())
        radii = radii_from_cov(cov)
    bins = gs2d.bin_gaussians(means.cuda(), radii.cuda(), g.depth.cuda(), S, S)
    assert bins.point_list.numel() == row["pairs"] and bins.num_buckets == row["buckets"]
    rects, _ = O2.rects_toy(means.numpy(), radii.numpy(), S, S)
    order, pl, ranges, boff = O2.bin_rects(rects, g.depth.numpy(), S, S)
    assert np.array_equal(bins.point_list.cpu().numpy(), pl)
    x = [t.cuda().requires_grad_(True) for t in (means, conic, color, opacity)]
    bg = torch.tensor([0.2, 0.5, 0.8])
    out = gs2d.rasterize(*x, bins, bg.cuda(), backend=backend)
    dout = torch.randn(3, S, S, generator=torch.Generator().manual_seed(1))
    grads = torch.autograd.grad(out, x, dout.cuda())
    p = [t.numpy() for t in (means, conic, color, opacity)]
    ref = O2.forward(O2.TOY2D, *p, pl, ranges, boff, S, S, bg=bg.double().numpy())
    assert np.abs(out.detach().cpu().numpy() - ref["image"]).max() <= 1e-5
    gr, _ = O2.backward_bucket(O2.TOY2D, *p, pl, ranges, boff, S, S, ref["image"], dout.numpy(), ref["n_contrib"],
                               ref["ckpt"])
    for cols, gg in (((0, 1), grads[0]), ((2, 3, 4), grads[1]), ((6, 7, 8), grads[2]), ((5,), grads[3])):
        assert rel(gg.reshape(-1, len(cols)), gr[:, list(cols)]) < 1e-4


@pytest.mark.parametrize("binning", ["spans", "radix"])
def test_gs2d_sparse_wide_canvas_ranges(binning, monkeypatch):
    """A 2048x1280 canvas (10240 tiles: more than one 8192-tile chunk of the bucket-offset scan)
    with two clusters of small Gaussians, so most tiles (the first and last ones included) hold
    no instance: the ranges (from the tile sort's last pass by atomic min / max, or from the span
    binning's tile counts), the empty tiles' positions, the bucket offsets and the lists equal the
    oracle's bit for bit."""
    monkeypatch.setattr(R2, "BINNING", binning)
    W, H = 2048, 1280
    gen = torch.Generator().manual_seed(7)
    n = 3000
    centre = torch.tensor([[700.0, 300.0], [1500.0, 1000.0]])
    means = centre[torch.randint(0, 2, (n,), generator=gen)] + 120.0 * torch.randn(n, 2, generator=gen)
    radii = torch.randint(0, 40, (n,), generator=gen, dtype=torch.int32)
    depth = torch.rand(n, generator=gen)
    bins = gs2d.bin_gaussians(means.cuda(), radii.cuda(), depth.cuda(), H, W)
    rects, _ = O2.rects_toy(means.numpy(), radii.numpy(), W, H)
    order, pl, ranges, boff = O2.bin_rects(rects, depth.numpy(), W, H)
    assert bins.tiles_x * bins.tiles_y == 10240
    rg = bins.ranges.cpu().numpy()
    assert (rg[:, 1] == rg[:, 0]).sum() > 5000 and rg[0, 0] == rg[0, 1] and rg[-1, 0] == rg[-1, 1]
    assert np.array_equal(rg.astype(np.int64), ranges.astype(np.int64))
    assert np.array_equal(bins.point_list.cpu().numpy(), pl)
    assert np.array_equal(bins.offsets_ext().cpu().numpy().astype(np.int64), boff.astype(np.int64))


@pytest.mark.parametrize("binning", ["spans", "radix"])
@pytest.mark.parametrize("size", [(16, 16), (12, 9)])
def test_gs2d_single_tile_canvas(size, binning, monkeypatch):
    """A canvas of one tile (on the radix path the tile sort has no pass, so the ranges come from
    the key-change kernel); lists and ranges equal the oracle's."""
    monkeypatch.setattr(R2, "BINNING", binning)
    W, H = size
    gen = torch.Generator().manual_seed(3)
    n = 40
    means = torch.rand(n, 2, generator=gen) * torch.tensor([W, H], dtype=torch.float32)
    radii = torch.randint(0, 6, (n,), generator=gen, dtype=torch.int32)
    depth = torch.rand(n, generator=gen)
    bins = gs2d.bin_gaussians(means.cuda(), radii.cuda(), depth.cuda(), H, W)
    rects, _ = O2.rects_toy(means.numpy(), radii.numpy(), W, H)
    order, pl, ranges, boff = O2.bin_rects(rects, depth.numpy(), W, H)
    assert len(ranges) == 1 and len(pl) > 0
    assert np.array_equal(bins.ranges.cpu().numpy().astype(np.int64), ranges.astype(np.int64))
    assert np.array_equal(bins.point_list.cpu().numpy(), pl)
    assert np.array_equal(bins.offsets_ext().cpu().numpy().astype(np.int64), boff.astype(np.int64))


def test_gs2d_empty_scene():
    means = torch.rand(50, 2, dtype=torch.float32) * 40
    radii = torch.zeros(50, dtype=torch.int32)
    bins = gs2d.bin_gaussians(means.cuda(), radii.cuda(), torch.rand(50).cuda(), 40, 40)
    assert bins.point_list.numel() == 0 and bins.num_buckets == 0
    x = [means.cuda().requires_grad_(True), torch.ones(50, 3).cuda().requires_grad_(True),
         torch.rand(50, 3).cuda().requires_grad_(True), torch.rand(50).cuda().requires_grad_(True)]
    bg = torch.tensor([0.2, 0.5, 0.8]).cuda()
    out = gs2d.rasterize(*x, bins, bg)
    assert torch.allclose(out, bg[:, None, None].expand_as(out))
    grads = torch.autograd.grad(out.sum(), x)
    assert all(float(g.abs().sum()) == 0.0 for g in grads)


def test_gs2d_rejects_cpu_tensors():
    with pytest.raises(RuntimeError, match="GPU"):
        gs2d.bin_gaussians(torch.rand(4, 2), torch.ones(4, dtype=torch.int32), torch.rand(4), 16, 16)


# ---------------------------------------------------------------------------------------
# phase0 / splat2d
# ---------------------------------------------------------------------------------------
def ph0_params(f, dtype, grad=True):
    return [cuda(f[k], dtype).requires_grad_(grad) for k in ("means", "chol", "opacity_logit", "colors")]


@pytest.mark.parametrize("name", PH0)
def test_splat2d_binning_bit_exact(name):
    f = load(f"phase0_{name}")
    m, c, l, _ = ph0_params(f, torch.float64, grad=False)
    b = splat2d.bin_tiles(m, c, l, int(f["H"]), int(f["W"]))
    torch.cuda.synchronize()
    for key in ("tile_offsets", "tile_ids", "bucket_offsets", "bucket_tile"):
        assert np.array_equal(getattr(b, key).cpu().numpy(), f[key]), key


@pytest.mark.parametrize("mode", ["splat", "pixel"])
@pytest.mark.parametrize("name", PH0)
def test_splat2d_float32_and_float64(name, mode):
    f = load(f"phase0_{name}")
    H, W = int(f["H"]), int(f["W"])
    for dtype, ftol, gtol in ((torch.float32, 1e-5, 1e-5), (torch.float64, 1e-12, 1e-10)):
        params = ph0_params(f, dtype)
        image = splat2d.render(*params, H, W, mode=mode)
        assert rel(image, f["image"]) < ftol
        grads = torch.autograd.grad(image, params, cuda(f["grad_image"], dtype))
        for key, g in zip(("g_means", "g_chol", "g_opacity_logit", "g_colors"), grads):
            assert rel(g, f[key]) < gtol, f"{name}/{mode}/{dtype}/{key}: {rel(g, f[key]):.2e}"


@pytest.mark.parametrize("name", ["seed0_n8", "seed1_n32", "dense_n96"])
def test_splat2d_modes_agree_and_counts(name):
    """phase0/tests/gradcheck/test_gradcheck.py:84-92 (modes agree) and test_opcount.py:63-123
    (n_contrib, atomic-count formulas, checkpoint bytes)."""
    f = load(f"phase0_{name}")
    H, W = int(f["H"]), int(f["W"])
    ext = P0.load_extension()
    for dtype, tol in ((torch.float32, 3e-6), (torch.float64, 1e-12)):
        res = {}
        for mode in ("pixel", "splat"):
            params = ph0_params(f, dtype)
            ext.reset_counters()
            image = splat2d.render(*params, H, W, mode=mode)
            res[mode] = torch.autograd.grad(image, params, cuda(f["grad_image"], dtype))
            res[mode + "_ctr"] = ext.get_counters()
        for a, b in zip(res["splat"], res["pixel"]):
            assert rel(a, b) < tol
        # counts from the oracle's emulation of the same thread mappings
        b = splat2d.bin_tiles(*ph0_params(f, dtype, grad=False)[:3], H, W)
        pl = b.tile_ids.cpu().numpy().astype(np.uint32)
        toff = b.tile_offsets.cpu().numpy()
        ranges = np.stack([toff[:-1], toff[1:]], 1).astype(np.uint32)
        boff = b.bucket_offsets.cpu().numpy().astype(np.uint32)
        npd = np.float64 if dtype == torch.float64 else np.float32
        p = [f[k].astype(npd) for k in ("means", "chol", "colors", "opacity_logit")]
        out = O2.forward(O2.PHASE0, *p, pl, ranges, boff, W, H)
        _, at_b = O2.backward_bucket(O2.PHASE0, *p, pl, ranges, boff, W, H, out["image"],
                                     f["grad_image"].astype(npd), out["last_contrib"], out["ckpt"])
        _, at_p = O2.backward_pixel(O2.PHASE0, *p, pl, ranges, W, H, out["final_T"], out["last_contrib"],
                                    f["grad_image"].astype(npd))
        assert res["splat_ctr"]["atomic_adds"] == at_b
        assert res["pixel_ctr"]["atomic_adds"] == at_p == int(out["n_contrib"].sum()) * 9
        assert res["splat_ctr"]["checkpoint_bytes"] == b.num_buckets * 256 * 4 * (8 if dtype == torch.float64 else 4)


@pytest.mark.parametrize("name", ["seed0_n8", "seed2_n8"])
@pytest.mark.parametrize("mode", ["splat", "pixel"])
def test_splat2d_gradcheck_float64(name, mode):
    """phase0/tests/gradcheck/test_gradcheck.py:51-59 on the GPU."""
    f = load(f"phase0_{name}")
    H, W = int(f["H"]), int(f["W"])

    def fn(means, chol, opacity_logit, colors):
        return splat2d.render(means, chol, opacity_logit, colors, H, W, mode=mode)

    assert torch.autograd.gradcheck(fn, tuple(ph0_params(f, torch.float64)), eps=1e-6, atol=1e-8, rtol=1e-6)


@pytest.mark.parametrize("mode", ["splat", "pixel"])
@pytest.mark.parametrize("name", ["seed1_n32", "dense_n96", "sparse_n150"])
def test_splat2d_render_against_ref_render(name, mode):
    """phase0/tests/gradcheck/test_gradcheck.py:62-81 and :95-100 with the package's own
    ref_render (float64 autograd, on the GPU) as the reference: float32 grads within 1e-5,
    float64 grads within 1e-10, the float64 image within 1e-12."""
    f = load(f"phase0_{name}")
    H, W = int(f["H"]), int(f["W"])
    gi = cuda(f["grad_image"], torch.float64)
    ref = ph0_params(f, torch.float64)
    want_img = splat2d.ref_render(*ref, H, W)
    want = torch.autograd.grad(want_img, ref, gi)
    for dtype, gtol in ((torch.float32, 1e-5), (torch.float64, 1e-10)):
        params = ph0_params(f, dtype)
        image = splat2d.render(*params, H, W, mode=mode)
        if dtype == torch.float64:
            assert rel(image, want_img) < 1e-12
        got = torch.autograd.grad(image, params, gi.to(dtype))
        for key, g, w in zip(("means", "chol", "opacity_logit", "colors"), got, want):
            assert rel(g, w) < gtol, f"{name}/{mode}/{dtype}/{key}: {rel(g, w):.2e}"


def test_splat2d_extension_surface_and_limitless_backward():
    """The extension functions of phase0/csrc/macrotile/bindings.cpp:156-239 with their return
    values; backward_splat without a per-pixel limit (the reference's signature) equals the
    autograd path's."""
    f = load("phase0_sparse_n150")
    H, W = int(f["H"]), int(f["W"])
    m, c, l, col = ph0_params(f, torch.float32, grad=False)
    b = splat2d.bin_tiles(m, c, l, H, W)
    ext = P0.load_extension()
    image, t_final, n_contrib, last_contrib, ckpt = ext.forward(m, c, l, col, b.tile_offsets, b.tile_ids,
                                                                b.bucket_offsets, b.bucket_tile, H, W)
    assert image.shape == (H, W, 3) and ckpt.shape == (b.num_buckets, 256, 4)
    # float32 decisions against the float32 oracle (the float64 reference may flip a threshold)
    toff = b.tile_offsets.cpu().numpy()
    ranges = np.stack([toff[:-1], toff[1:]], 1).astype(np.uint32)
    p32 = [f[k].astype(np.float32) for k in ("means", "chol", "colors", "opacity_logit")]
    ref = O2.forward(O2.PHASE0, *p32, b.tile_ids.cpu().numpy().astype(np.uint32), ranges,
                     b.bucket_offsets.cpu().numpy().astype(np.uint32), W, H)
    assert np.array_equal(n_contrib.cpu().numpy(), ref["n_contrib"])
    assert np.array_equal(last_contrib.cpu().numpy(), ref["last_contrib"])
    assert np.abs(ckpt.cpu().numpy() - ref["ckpt"]).max() <= 1e-6
    m64 = ph0_params(f, torch.float64, grad=False)
    n64 = ext.forward(*m64, b.tile_offsets, b.tile_ids, b.bucket_offsets, b.bucket_tile, H, W)[2]
    assert np.array_equal(n64.cpu().numpy(), f["n_contrib"])  # test_opcount.py:89-92
    gi = cuda(f["grad_image"], torch.float32)
    tabs = (b.tile_offsets, b.tile_ids, b.bucket_offsets, b.bucket_tile)
    g_ref = ext.backward_splat(gi, m, c, l, col, *tabs, image, ckpt, H, W)
    g_lim = ext.backward_splat(gi, m, c, l, col, *tabs, image, ckpt, H, W, last_contrib=last_contrib)
    g_pix = ext.backward_pixel(gi, m, c, l, col, *tabs, t_final, last_contrib, H, W)
    for a, bb, p in zip(g_ref, g_lim, g_pix):
        assert rel(a, bb) < 1e-6 and rel(a, p) < 1e-5
    with pytest.raises(RuntimeError):
        P0.load_extension(with_cuda=False)


def test_splat2d_depth_order():
    f = load("phase0_dense_n96")
    H, W = int(f["H"]), int(f["W"])
    params = ph0_params(f, torch.float64, grad=False)
    depths = torch.rand(params[0].shape[0], generator=torch.Generator().manual_seed(3), dtype=torch.float64).cuda()
    order = torch.argsort(depths, stable=True)
    a = splat2d.render(*params, H, W, depths=depths)
    b = splat2d.render(*[p[order] for p in params], H, W)
    assert torch.equal(a, b)


@pytest.mark.parametrize("backend", ["splat", "pixel"])
def test_gs2d_fit_workload_4k_256(backend):
    """The 2D image-fit workload at its own size (4096 Gaussians, 256x256, L1 against a U(0,1)
    target): binning bit-exact, forward within 1e-5 and the gradients of the L1 step within
    1e-4 of the CPU oracle (same upstream gradient for both)."""
    from gs2d.params import fit_scene_4k

    means, conic, color, opacity, cov, depth, target = fit_scene_4k()
    S = 256
    radii = radii_from_cov(cov)
    bins = gs2d.bin_gaussians(means.cuda(), radii.cuda(), depth.cuda(), S, S)
    rects, _ = O2.rects_toy(means.numpy(), radii.numpy(), S, S)
    order, pl, ranges, boff = O2.bin_rects(rects, depth.numpy(), S, S)
    assert np.array_equal(bins.point_list.cpu().numpy(), pl)
    assert np.array_equal(bins.ranges.cpu().numpy().astype(np.uint32).ravel(), ranges.ravel())
    x = [t.cuda().requires_grad_(True) for t in (means, conic, color, opacity)]
    out = gs2d.rasterize(*x, bins, backend=backend)
    loss = (out - target.cuda()).abs().mean()
    grads = torch.autograd.grad(loss, x)
    dout = (torch.sign(out.detach() - target.cuda()) / out.numel()).cpu()
    p = [t.numpy() for t in (means, conic, color, opacity)]
    ref = O2.forward(O2.TOY2D, *p, pl, ranges, boff, S, S)
    assert np.abs(out.detach().cpu().numpy() - ref["image"]).max() <= 1e-5
    gr, _ = O2.backward_bucket(O2.TOY2D, *p, pl, ranges, boff, S, S, ref["image"], dout.numpy(), ref["n_contrib"],
                               ref["ckpt"])
    for cols, gg in (((0, 1), grads[0]), ((2, 3, 4), grads[1]), ((6, 7, 8), grads[2]), ((5,), grads[3])):
        assert rel(gg.reshape(-1, len(cols)), gr[:, list(cols)]) < 1e-4


@pytest.mark.parametrize("spread", [False, True])
def test_fused_activation_matches_the_reference_activation(spread):
    """gs2d.params.activate_fused against activate / radii_from_cov (the reference's operations as
    tensor ops on the same GPU): outputs within a few float32 ulps (exp, cos and sin may round
    differently in the last place), radii equal except where 3 sqrt(lambda) lies within 1e-5 of an
    integer. Gradients: on the fit's own initial Gaussians (anisotropy <= 3) within 1e-5 relative
    L2 of float64 autograd of activate; with scales spread over e^(+-3) (condition numbers up to
    ~1e5, where float32 cancels in the conic's det terms) no further from float64 than 1.5x the
    float32 autograd of activate itself."""
    from gs2d.params import Gaussians2D, activate, activate_fused, radii_from_cov

    g = Gaussians2D(20_000, 512, 512, seed=3).cuda()
    if spread:
        with torch.no_grad():
            g.log_scale.add_(torch.randn(g.log_scale.shape, generator=torch.Generator().manual_seed(1)).cuda())
            g.theta.mul_(3.0)
    ref = activate(g.xy, g.log_scale, g.theta, g.rgb_logit, g.opacity_logit)
    out = activate_fused(g.xy, g.log_scale, g.theta, g.rgb_logit, g.opacity_logit)
    for k, name in enumerate(["means", "conic", "color", "opacity", "cov"]):
        a, b = out[k].detach(), ref[k].detach()
        err = ((a - b).abs() / b.abs().clamp_min(1e-30)).max().item()
        assert err < 4e-6, f"{name}: {err:.2e}"
    r_ref = radii_from_cov(ref[4].detach())
    c64 = ref[4].detach().double()
    mid = 0.5 * (c64[:, 0] + c64[:, 2])
    det = c64[:, 0] * c64[:, 2] - c64[:, 1] ** 2
    t = 3.0 * torch.sqrt(mid + torch.sqrt((mid * mid - det).clamp_min(0.1)))
    near_int = (t - t.round()).abs() < 1e-5
    assert int(((out[5] != r_ref) & ~near_int).sum()) == 0
    # gradients: a random linear loss of means, conic, colour and opacity
    gen = torch.Generator().manual_seed(5)
    w = [torch.randn(t.shape, generator=gen).cuda() for t in out[:4]]
    params = (g.xy, g.log_scale, g.theta, g.rgb_logit, g.opacity_logit)

    def grads(fn, dtype):
        leaves = [p.detach().to(dtype).clone().requires_grad_(True) for p in params]
        o = fn(*leaves)
        sum(((r * wi.to(dtype)).sum() for r, wi in zip(o[:4], w))).backward()
        return [x.grad.double() for x in leaves]

    g64, g32, gf = grads(activate, torch.float64), grads(activate, torch.float32), grads(activate_fused, torch.float32)
    for a, t32, b, name in zip(gf, g32, g64, ["xy", "log_scale", "theta", "rgb_logit", "opacity_logit"]):
        e = ((a - b).norm() / b.norm()).item()
        e32 = ((t32 - b).norm() / b.norm()).item()
        bound = 1.5 * e32 + 1e-7 if spread else 1e-5
        assert e < bound, f"grad {name}: {e:.2e} (float32 autograd of activate: {e32:.2e})"
