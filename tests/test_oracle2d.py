"""CPU checks that pin the 2D oracle (oracle2d.c) for both 2D rule sets:

  - against the golden fixtures written from the reference's own Python code
    (tests/golden/make_golden.py): tile rectangles, depth order, per-tile lists, ranges and
    bucket tables bit for bit; float64 image and gradients of the dense reference renderers;
  - against the known-answer pair / bucket counts of the reference's benchmark
    (toy2d/results/bench-cfda5b4-4473561.json:11-76);
  - against the reference's own phase0 CPU twin, compiled from its sources into oracle/_ref
    (forward, both backwards and the atomic-count formulas of
    phase0/tests/gradcheck/test_opcount.py:63-86);
  - elementary functions against float64 math.
Tolerances are those of the references' own tests (toy2d/tests/test_cpu.py:43-66,
phase0/tests/gradcheck/test_gradcheck.py:62-100).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle2d as O2

GOLD = Path(__file__).resolve().parent / "golden"
TOY = ["tiny", "sparse_odd", "dense", "opaque"]
PH0 = [f"seed{s}_n{n}" for s in (0, 1, 2) for n in (8, 32)] + ["dense_n96", "sparse_n150"]


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a - b))


# ---------------------------------------------------------------------------------------
def test_exp_and_log_accuracy():
    xs = np.linspace(-100.0, 80.0, 40001)
    got = np.array([O2.exp_f64(x) for x in xs])
    ref = np.exp(xs)
    assert np.max(np.abs(got - ref) / ref) < 4e-16
    got32 = np.array([O2.exp_f32(float(np.float32(x))) for x in xs[xs > -87]])
    ref32 = np.exp(np.float32(xs[xs > -87]).astype(np.float64))
    assert np.max(np.abs(got32 - ref32) / ref32) < 2.4e-7  # 2 ulp
    ys = np.exp(np.linspace(-700, 700, 20001))
    got = np.array([O2.log_f64(y) for y in ys])
    assert np.max(np.abs(got - np.log(ys)) / np.maximum(1.0, np.abs(np.log(ys)))) < 5e-16


# ---------------------------------------------------------------------------------------
# toy2d
# ---------------------------------------------------------------------------------------
def toy_bins(f):
    rects, counts = O2.rects_toy(f["means"].astype(np.float32), f["radii"], int(f["W"]), int(f["H"]))
    order, pl, ranges, boff = O2.bin_rects(rects, f["depth"], int(f["W"]), int(f["H"]))
    return rects, order, pl, ranges, boff


@pytest.mark.parametrize("name", TOY)
def test_toy2d_binning_matches_reference_bit_for_bit(name):
    f = load(f"toy2d_{name}")
    rects, order, pl, ranges, boff = toy_bins(f)
    assert np.array_equal(rects, f["rect"])
    assert np.array_equal(order, f["order"])
    assert np.array_equal(pl, f["point_list"].astype(np.uint32))
    assert np.array_equal(ranges, f["ranges"].astype(np.uint32))
    assert np.array_equal(boff[:-1], f["bucket_offsets"].astype(np.uint32))
    assert int(boff[-1]) == int(f["num_buckets"])


@pytest.mark.parametrize("name", TOY)
def test_toy2d_forward_and_gradients_float64(name):
    f = load(f"toy2d_{name}")
    W, H = int(f["W"]), int(f["H"])
    rects, order, pl, ranges, boff = toy_bins(f)
    p = [f[k] for k in ("means", "conic", "color", "opacity")]
    out = O2.forward(O2.TOY2D, p[0], p[1], p[2], p[3], pl, ranges, boff, W, H, bg=f["bg"])
    assert rel(out["image"], f["image"]) < 1e-12  # toy2d/tests/test_cpu.py:43-48
    for mode in ("bucket", "pixel"):
        if mode == "bucket":
            g, _ = O2.backward_bucket(O2.TOY2D, p[0], p[1], p[2], p[3], pl, ranges, boff, W, H, out["image"],
                                      f["dout"], out["n_contrib"], out["ckpt"])
        else:
            g, _ = O2.backward_pixel(O2.TOY2D, p[0], p[1], p[2], p[3], pl, ranges, W, H, out["final_T"],
                                     out["n_contrib"], f["dout"], bg=f["bg"])
        for cols, key in (((0, 1), "g_means"), ((2, 3, 4), "g_conic"), ((6, 7, 8), "g_color"), ((5,), "g_opacity")):
            e = rel(g[:, list(cols)].reshape(f[key].shape), f[key])
            assert e < 1e-9, f"{name}/{mode}/{key}: {e:.2e}"  # toy2d/tests/test_cpu.py:51-66


@pytest.mark.parametrize("name", TOY)
def test_toy2d_float32_within_gate(name):
    f = load(f"toy2d_{name}")
    W, H = int(f["W"]), int(f["H"])
    rects, order, pl, ranges, boff = toy_bins(f)
    p = [f[k].astype(np.float32) for k in ("means", "conic", "color", "opacity")]
    out = O2.forward(O2.TOY2D, *p, pl, ranges, boff, W, H, bg=f["bg"])
    assert rel(out["image"], f["image"]) < 1e-5  # toy2d/tests/test_cuda.py:8-31 gate
    g, _ = O2.backward_bucket(O2.TOY2D, *p, pl, ranges, boff, W, H, out["image"], f["dout"].astype(np.float32),
                              out["n_contrib"], out["ckpt"])
    assert rel(g[:, 0:2], f["g_means"]) < 1e-5 and rel(g[:, 6:9], f["g_color"]) < 1e-5


def test_toy2d_bench_pair_and_bucket_counts():
    """Known answer: pairs and buckets of Gaussians2D(n, S, S, seed=0) at the six benchmark sizes."""
    from gs2d.params import Gaussians2D, radii_from_cov

    rows = json.loads((GOLD / "toy2d_bench_counts.json").read_text())["rows"]
    for r in rows[:4]:
        S, n = r["size"], r["n"]
        g = Gaussians2D(n, S, S, seed=0)
        with torch.no_grad():
            means, conic, color, opacity, cov = g.activated()
            radii = radii_from_cov(cov)
        rects, _ = O2.rects_toy(means.detach().numpy(), radii.numpy(), S, S)
        order, pl, ranges, boff = O2.bin_rects(rects, g.depth.numpy(), S, S)
        assert len(pl) == r["pairs"] and int(boff[-1]) == r["buckets"], (S, n)


# ---------------------------------------------------------------------------------------
# phase0
# ---------------------------------------------------------------------------------------
def ph0_bins(f, dtype=np.float64):
    m, c, l = (f[k].astype(dtype) for k in ("means", "chol", "opacity_logit"))
    rects, counts = O2.rects_phase0(m, c, l, int(f["W"]), int(f["H"]))
    order, pl, ranges, boff = O2.bin_rects(rects, None, int(f["W"]), int(f["H"]))
    return pl, ranges, boff


@pytest.mark.parametrize("name", PH0)
def test_phase0_binning_matches_reference_bit_for_bit(name):
    f = load(f"phase0_{name}")
    pl, ranges, boff = ph0_bins(f)
    toff = np.concatenate([ranges[:, 0], ranges[-1:, 1]])
    assert np.array_equal(toff, f["tile_offsets"].astype(np.uint32))
    assert np.array_equal(pl, f["tile_ids"].astype(np.uint32))
    assert np.array_equal(boff, f["bucket_offsets"].astype(np.uint32))


@pytest.mark.parametrize("name", PH0)
def test_phase0_forward_and_gradients_float64(name):
    f = load(f"phase0_{name}")
    W, H = int(f["W"]), int(f["H"])
    pl, ranges, boff = ph0_bins(f)
    p = [f[k] for k in ("means", "chol", "colors", "opacity_logit")]
    out = O2.forward(O2.PHASE0, *p, pl, ranges, boff, W, H)
    assert rel(out["image"], f["image"]) < 1e-12  # test_gradcheck.py:95-100
    assert np.array_equal(out["n_contrib"], f["n_contrib"])  # test_opcount.py:89-92
    gb, _ = O2.backward_bucket(O2.PHASE0, *p, pl, ranges, boff, W, H, out["image"], f["grad_image"],
                               out["last_contrib"], out["ckpt"])
    gp, _ = O2.backward_pixel(O2.PHASE0, *p, pl, ranges, W, H, out["final_T"], out["last_contrib"], f["grad_image"])
    for g in (gb, gp):
        for cols, key in (((0, 1), "g_means"), ((2, 3, 4), "g_chol"), ((5,), "g_opacity_logit"),
                          ((6, 7, 8), "g_colors")):
            e = rel(g[:, list(cols)].reshape(f[key].shape), f[key])
            assert e < 1e-10, f"{name}/{key}: {e:.2e}"  # test_gradcheck.py:73-81


needs_ref = pytest.mark.skipif(not O2.ref_available(), reason="oracle/_ref not built (needs the reference tree)")


@needs_ref
@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("name", ["seed0_n32", "dense_n96", "sparse_n150"])
def test_phase0_oracle_matches_reference_cpu_twin(name, dtype):
    f = load(f"phase0_{name}")
    W, H = int(f["W"]), int(f["H"])
    m, c, l, col = (f[k].astype(dtype) for k in ("means", "chol", "opacity_logit", "colors"))
    pl, ranges, boff = ph0_bins(f)
    out = O2.forward(O2.PHASE0, m, c, col, l, pl, ranges, boff, W, H)
    toff = f["tile_offsets"]
    btile = f["bucket_tile"]
    ref = O2.ref_forward(m, c, l, col, toff, f["tile_ids"], f["bucket_offsets"], btile, H, W)
    assert np.array_equal(out["n_contrib"], ref["n_contrib"])
    assert np.array_equal(out["last_contrib"], ref["last_contrib"])
    tol = 1e-14 if dtype == np.float64 else 1e-6
    assert np.abs(out["image"] - ref["image"]).max() < tol
    assert np.abs(out["ckpt"] - ref["ckpt"]).max() < tol
    gi = f["grad_image"].astype(dtype)
    for mode in ("splat", "pixel"):
        if mode == "splat":
            g, at = O2.backward_bucket(O2.PHASE0, m, c, col, l, pl, ranges, boff, W, H, out["image"], gi,
                                       out["last_contrib"], out["ckpt"])
        else:
            g, at = O2.backward_pixel(O2.PHASE0, m, c, col, l, pl, ranges, W, H, out["final_T"], out["last_contrib"],
                                      gi)
        O2.ref_reset_counters()
        rg = O2.ref_backward(mode, m, c, l, col, toff, f["tile_ids"], f["bucket_offsets"], btile, H, W, gi, ref)
        assert at == O2.ref_counters()["atomic_adds"]  # same atomic-count formula
        gtol = 1e-12 if dtype == np.float64 else 2e-6
        for cols, r in (((0, 1), rg[0]), ((2, 3, 4), rg[1]), ((5,), rg[2]), ((6, 7, 8), rg[3])):
            assert rel(g[:, list(cols)].reshape(r.shape), r) < gtol, (mode, cols)


# ---------------------------------------------------------------------------------------
# gs2d.render_reference (the dense backend 'ref') against the reference's own dense renderer
# ---------------------------------------------------------------------------------------
def fixture_bins(f):
    import gs2d

    H, W = int(f["H"]), int(f["W"])
    tx, ty = (W + 15) // 16, (H + 15) // 16
    z = torch.zeros(0, dtype=torch.int32)
    return gs2d.Bins(H, W, tx, ty, torch.from_numpy(f["rect"]), torch.from_numpy(f["order"]), z, z, z, z, 0)


@pytest.mark.parametrize("name", TOY)
def test_render_reference_matches_reference_renderer(name):
    """Image and autograd gradients (upstream dout) of gs2d.render_reference in float64 against
    the values the reference's render_reference gave for the same scene (the golden fixture):
    1e-12 (toy2d/tests/test_cpu.py:43-48)."""
    import gs2d

    f = load(f"toy2d_{name}")
    x = [torch.tensor(f[k], dtype=torch.float64, requires_grad=True) for k in ("means", "conic", "color", "opacity")]
    img = gs2d.render_reference(*x, fixture_bins(f), torch.tensor(f["bg"]))
    assert rel(img.detach().numpy(), f["image"]) < 1e-12
    (img * torch.tensor(f["dout"])).sum().backward()
    for t, key in zip(x, ("g_means", "g_conic", "g_color", "g_opacity")):
        assert rel(t.grad.numpy(), f[key]) < 1e-12, key
    # the same through rasterize(backend='ref'), in blocks of another size
    img2 = gs2d.rasterize(*[t.detach() for t in x], fixture_bins(f), torch.tensor(f["bg"]), backend="ref")
    assert rel(img2.numpy(), f["image"]) < 1e-12
    img3 = gs2d.render_reference(*[t.detach() for t in x], fixture_bins(f), torch.tensor(f["bg"]), pixels_per_block=7)
    assert rel(img3.numpy(), f["image"]) < 1e-12


# ---------------------------------------------------------------------------------------
# splat2d.ref_state / ref_render (the dense phase0 model) against the reference's own
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", PH0)
def test_splat2d_ref_render_matches_reference_model(name):
    """Image, T, composited-splat counts and autograd gradients (upstream grad_image) of
    splat2d.ref_state / ref_render in float64 against what the reference's ref_state /
    ref_render gave for the same scene (the golden fixture): 1e-12, counts exact
    (phase0/tests/gradcheck/test_gradcheck.py:96-100, test_opcount.py:89-92)."""
    from splat2d.ops import ref_render, ref_state

    f = load(f"phase0_{name}")
    H, W = int(f["H"]), int(f["W"])
    x = [torch.tensor(f[k], dtype=torch.float64, requires_grad=True)
         for k in ("means", "chol", "opacity_logit", "colors")]
    st = ref_state(*x, H, W)
    assert rel(st.image.detach().numpy(), f["image"]) < 1e-12
    assert rel(st.t_final.detach().numpy(), f["t_final"]) < 1e-12
    assert np.array_equal(st.contributes.sum(-1).numpy(), f["n_contrib"])
    # a composited splat passed the alpha test (raw alpha, clamped at 0.99, >= 1/255)
    assert bool((torch.clamp(st.raw_alpha, max=0.99)[st.contributes] >= 1.0 / 255.0).all())
    grads = torch.autograd.grad(ref_render(*x, H, W), x, torch.tensor(f["grad_image"]))
    for g, key in zip(grads, ("g_means", "g_chol", "g_opacity_logit", "g_colors")):
        assert rel(g.numpy(), f[key]) < 1e-12, key
    # blocks of another size (31 pixels) give the same image
    small = ref_state(*[t.detach() for t in x], H, W, max_block_elems=31 * x[0].shape[0])
    assert rel(small.image.numpy(), f["image"]) < 1e-12
    assert torch.equal(small.contributes, st.contributes)


def test_splat2d_ref_state_empty_and_opaque_stop():
    """No splats: a black image with T = 1. A stack of opaque splats (alpha 0.99 each): T falls
    by 100x per splat, so the third splat is the last composited one (T before it 1e-4, T
    before the fourth 1e-6 < 1e-4)."""
    from splat2d.ops import ref_state

    z = torch.zeros(0, 2, dtype=torch.float64)
    st = ref_state(z, torch.zeros(0, 3, dtype=torch.float64), torch.zeros(0, dtype=torch.float64),
                   torch.zeros(0, 3, dtype=torch.float64), 5, 7)
    assert st.image.shape == (5, 7, 3) and float(st.image.abs().max()) == 0.0
    assert float((st.t_final - 1).abs().max()) == 0.0 and st.contributes.shape == (5, 7, 0)
    k = 5
    means = torch.tensor([[2.5, 2.5]], dtype=torch.float64).repeat(k, 1)
    chol = torch.tensor([[1e-3, 0.0, 1e-3]], dtype=torch.float64).repeat(k, 1)  # flat over the image
    logit = torch.full((k,), 50.0, dtype=torch.float64)  # sigmoid -> 1, clamped to 0.99
    colors = torch.eye(3, dtype=torch.float64).repeat(2, 1)[:k]
    st = ref_state(means, chol, logit, colors, 4, 4)
    assert st.contributes.sum(-1).unique().tolist() == [3]
    a = 0.99
    want = torch.tensor([a, a * (1 - a), a * (1 - a) ** 2], dtype=torch.float64)  # weights of splats 0, 1, 2
    assert torch.allclose(st.image[0, 0], want, rtol=1e-9, atol=0)
    assert abs(float(st.t_final[0, 0]) - (1 - a) ** 3) < 1e-15
