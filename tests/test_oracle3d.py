"""CPU checks that pin the 3D oracle (no GPU): the C restatement against closed forms,
quadrature identities, a float64 autograd restatement and brute force on tiny inputs, plus
the C ABI library's exported symbols.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a wrong sign
or index, a transposed operand) fails it:
  - elementary functions against float64 math at a dense grid of points;
  - the SH basis against orthonormality on the sphere (constants, polynomial forms) and
    against the unit-sphere forms of the reference's SH backward
    (phase2/sh_coalesce.patch:102-149, signs and band layout);
  - the projection against closed forms (on-axis isotropic Gaussian, off-axis mean);
  - the hand-derived backwards (blend replay, preprocess chain rule) against float64
    autograd of dense3d, whose forward is itself checked against the oracle;
  - the tiled forward against a brute-force dense render over all Gaussians (binning
    completeness + blend rules), and the binning against its invariants
    (toy2d/tests/test_cpu.py:10-21: complete lists, depth order, bucket count).
"""
import dataclasses
import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import dense3d as D
import oracle as O
from amdsplat import scenes

ROOT = Path(__file__).resolve().parent.parent
BG = (0.2, 0.5, 0.8)


def small(n=400, W=96, H=72, seed=0, **kw):
    return scenes.small_scene(n, W, H, seed=seed, **kw)


def np_params(sc):
    return [t.numpy() for t in sc.params()]


# ---------------------------------------------------------------------------------------
# C ABI library
# ---------------------------------------------------------------------------------------
def header_functions():
    text = (ROOT / "include" / "amdsplat.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gs\w*)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import ctypes

    from amdsplat import _lib

    L = ctypes.CDLL(str(_lib.LIB_PATH))
    names = header_functions()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in include/amdsplat.h but not exported: {missing}"
    # every declared entry point has a ctypes signature in the binding
    assert not [n for n in names if n not in _lib._SIGS]


def test_binning_path_choice():
    """gs_bin_path (host only): the radix path by default, the span binning from 2M Gaussians
    on canvases of at most 512 tiles a side, each forced by its flag where it applies."""
    from amdsplat import _lib

    def path(n, flags=0, W=640, H=480):
        cam = _lib.make_camera(np.eye(4, dtype=np.float32), 500.0, 500.0, W / 2, H / 2, W, H, 0.01, 100.0,
                               flags=flags)
        return _lib.lib().gs_bin_path(n, cam)

    assert path(1_000_000) == _lib.GS_BIN_PATH_RADIX
    assert path(2_000_000) == _lib.GS_BIN_PATH_SPANS
    assert path(2_000_000, W=16 * 513) == _lib.GS_BIN_PATH_RADIX
    assert path(1000, _lib.GS_BIN_SPANS) == _lib.GS_BIN_PATH_SPANS
    assert path(3_000_000, _lib.GS_BIN_RADIX) == _lib.GS_BIN_PATH_RADIX


# ---------------------------------------------------------------------------------------
# Elementary functions
# ---------------------------------------------------------------------------------------
def test_exp2_polynomial_within_one_ulp():
    xs = np.linspace(-64.0, 0.0, 20001, dtype=np.float32)
    got = np.array([O.exp2_neg(float(x)) for x in xs], np.float64)
    ref = np.exp2(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 1.0
    assert O.exp2_neg(0.0) == 1.0 and O.exp2_neg(-1.0) == 0.5


def test_log_and_sigmoid_accuracy():
    xs = np.exp(np.linspace(-20, 20, 4001)).astype(np.float32)
    got = np.array([O.log_pos(float(x)) for x in xs], np.float64)
    ref = np.log(xs.astype(np.float64))
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) < 4e-7
    zs = np.linspace(-30, 30, 2001, dtype=np.float32)
    got = np.array([O.sigmoid(float(z)) for z in zs], np.float64)
    ref = 1.0 / (1.0 + np.exp(-zs.astype(np.float64)))
    # exp(z) is evaluated as 2^(z log2 e): the rounding of the product costs ~|z| 2^-24 relative
    assert np.max(np.abs(got - ref) / ref / np.maximum(1.0, np.abs(zs))) < 1e-7


# ---------------------------------------------------------------------------------------
# Spherical harmonics
# ---------------------------------------------------------------------------------------
def sphere_quadrature(n_theta=12, n_phi=24):
    """Gauss-Legendre in cos(theta) x uniform phi: exact for polynomials of degree < 2*n_theta."""
    zt, wt = np.polynomial.legendre.leggauss(n_theta)
    phi = 2 * np.pi * np.arange(n_phi) / n_phi
    Z, P = np.meshgrid(zt, phi, indexing="ij")
    r = np.sqrt(1 - Z * Z)
    dirs = np.stack([r * np.cos(P), r * np.sin(P), Z], -1).reshape(-1, 3)
    w = (wt[:, None] * np.full(n_phi, 2 * np.pi / n_phi)[None, :]).reshape(-1)
    return dirs, w


def test_sh_basis_is_orthonormal():
    dirs, w = sphere_quadrature()
    B = O.sh_basis(dirs, 16).astype(np.float64)
    gram = (B * w[:, None]).T @ B
    assert np.abs(gram - np.eye(16)).max() < 2e-6


def test_sh_basis_matches_reference_unit_sphere_forms():
    """phase2/sh_coalesce.patch:105-149 writes bands 2-3 in forms reduced with x^2+y^2+z^2=1
    (e.g. C2b zz - C2c, y (C3d - C3e zz)); the constants follow from the normalisation."""
    K = D.sh_norm_constant
    c1 = K(1, 0)
    rng = np.random.default_rng(0)
    d = rng.standard_normal((500, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    x, y, z = d.T
    xx, yy, zz = x * x, y * y, z * z
    # constant names of the reference: C2a = 6 K22, C2b = 1.5 K20, C2c = 0.5 K20, C2d = 3 K22,
    # C3a = 15 K33, C3b = 45 K33, C3c = 30 K32, C3d = 1.5 K31, C3e = 7.5 K31, C3f = 2.5 K30,
    # C3g = 1.5 K30, C3h = 15 K32 (associated-Legendre factors times the normalisation)
    ref = np.stack([
        np.full_like(x, K(0, 0)), -c1 * y, c1 * z, -c1 * x,
        6 * K(2, 2) * x * y, -3 * K(2, 1) * y * z, 1.5 * K(2, 0) * zz - 0.5 * K(2, 0),
        -3 * K(2, 1) * x * z, 3 * K(2, 2) * (xx - yy),
        y * (15 * K(3, 3) * yy - 45 * K(3, 3) * xx),
        30 * K(3, 2) * x * y * z,
        y * (1.5 * K(3, 1) - 7.5 * K(3, 1) * zz),
        z * (2.5 * K(3, 0) * zz - 1.5 * K(3, 0)),
        x * (1.5 * K(3, 1) - 7.5 * K(3, 1) * zz),
        15 * K(3, 2) * z * (xx - yy),
        x * (45 * K(3, 3) * yy - 15 * K(3, 3) * xx),
    ], -1)
    got = O.sh_basis(d, 16).astype(np.float64)
    assert np.abs(got - ref).max() < 3e-6


# ---------------------------------------------------------------------------------------
# Projection
# ---------------------------------------------------------------------------------------
def one_gaussian(p, log_s, q=(1.0, 0.0, 0.0, 0.0), logit=2.0, sh0=(0.3, -0.2, 0.1)):
    means = np.array([p], np.float32)
    ls = np.full((1, 3), log_s, np.float32)
    quats = np.array([q], np.float32)
    op = np.array([logit], np.float32)
    sh = np.zeros((1, 16, 3), np.float32)
    sh[0, 0] = sh0
    return means, ls, quats, op, sh


def test_preprocess_on_axis_isotropic_closed_form():
    cam = scenes.Camera(torch.eye(4), 500.0, 500.0, 64.3, 47.8, 128, 96, 0.2, 100.0)
    z, s = 4.0, 0.05
    rec, touched = O.preprocess_fwd(*one_gaussian((0.0, 0.0, z), math.log(s)), cam, 0)
    assert touched[0] > 0
    r = rec[0]
    assert r[0] == np.float32(64.3) and r[1] == np.float32(47.8)  # mean2d = principal point
    a = (500.0 * s / z) ** 2 + 0.3  # cov2d = (f s / z)^2 I + dilation
    np.testing.assert_allclose(r[2], 1.0 / a, rtol=2e-6)
    assert abs(r[3]) < 1e-9
    np.testing.assert_allclose(r[4], 1.0 / a, rtol=2e-6)
    np.testing.assert_allclose(r[5], 1.0 / (1.0 + math.exp(-2.0)), rtol=1e-6)
    assert r[6] == np.float32(z)
    np.testing.assert_allclose(r[7], math.log(255.0 / (1.0 + math.exp(-2.0))), rtol=1e-6)
    # SH degree 0: colour = C0 sh0 + 0.5, clamped at 0 with the mask bit set
    np.testing.assert_allclose(r[8:11], np.maximum(D.SH0 * np.array([0.3, -0.2, 0.1]) + 0.5, 0), rtol=1e-6)
    # the pixel bounds are the alpha >= 1/255 extent: sqrt(2 ln(255 o) a)
    ext = math.sqrt(2 * r[7] * a)
    b = r[12:16].view(np.int32)
    assert b[0] == math.ceil(64.3 - ext - 0.5) and b[1] == math.floor(64.3 + ext - 0.5)


def aa_camera(cam):
    return dataclasses.replace(cam, proper_antialiasing=True)


def test_proper_antialiasing_on_axis_closed_form():
    """Isotropic on-axis Gaussian: S = sigma^2 I, S' = (sigma^2 + 0.3) I, so the blended
    opacity is o sigma^2 / (sigma^2 + 0.3) and the conic is unchanged."""
    cam = scenes.Camera(torch.eye(4), 500.0, 500.0, 64.3, 47.8, 128, 96, 0.2, 100.0)
    z, s = 4.0, 0.01
    g = one_gaussian((0.0, 0.0, z), math.log(s))
    plain, _ = O.preprocess_fwd(*g, cam, 0)
    rec, touched = O.preprocess_fwd(*g, aa_camera(cam), 0)
    assert touched[0] > 0
    sig2 = (500.0 * s / z) ** 2
    o = 1.0 / (1.0 + math.exp(-2.0))
    np.testing.assert_allclose(rec[0, 5], o * sig2 / (sig2 + 0.3), rtol=2e-6)
    np.testing.assert_allclose(rec[0, 7], math.log(255.0 * o * sig2 / (sig2 + 0.3)), rtol=2e-6)
    assert np.array_equal(rec[0, 2:5], plain[0, 2:5]) and rec[0, 6] == plain[0, 6]


@pytest.mark.parametrize("s", [0.003, 0.006, 0.012])
def test_proper_antialiasing_keeps_the_splat_integral(s):
    """Summed over the pixels, one Gaussian's alpha is 2 pi sqrt(det S') (o' - 1/255) (the
    integral of o' G' over o' G' >= 1/255). With the compensation o' sqrt(det S') = o sqrt(det S):
    the dilated splat carries the undilated one's mass, without it (sigma^2 + 0.3) / sigma^2 more."""
    cam = scenes.Camera(torch.eye(4), 500.0, 500.0, 64.0, 48.0, 128, 96, 0.2, 100.0)
    z, logit = 4.0, 3.0
    g = list(one_gaussian((0.0, 0.0, z), math.log(s), logit=logit, sh0=(0.5 / D.SH0, 0.0, 0.0)))
    o = 1.0 / (1.0 + math.exp(-logit))
    sig2 = (500.0 * s / z) ** 2
    for c, expect in ((cam, 2 * math.pi * (sig2 + 0.3) * (o - 1 / 255)),
                      (aa_camera(cam), 2 * math.pi * (o * sig2 - (sig2 + 0.3) / 255))):
        ref = O.render(*g, c, 0, bg=(0.0, 0.0, 0.0))
        total = float(ref["image"][0].astype(np.float64).sum())  # colour 1: image = alpha
        np.testing.assert_allclose(total, expect, rtol=0.01)
    assert (sig2 + 0.3) / sig2 > 1.1  # the two cases differ by far more than the tolerance


def test_preprocess_off_axis_mean_and_rotation_invariance():
    cam = scenes.Camera(torch.eye(4), 400.0, 300.0, 50.0, 40.0, 100, 80, 0.2, 100.0)
    p = (0.3, -0.2, 5.0)
    q = np.array([0.3, -0.5, 0.7, 0.1])
    r1, _ = O.preprocess_fwd(*one_gaussian(p, math.log(0.02), tuple(q)), cam, 3)
    np.testing.assert_allclose(r1[0, :2], [400.0 * 0.3 / 5.0 + 50.0, 300.0 * -0.2 / 5.0 + 40.0], rtol=1e-6)
    # an isotropic Gaussian's covariance does not depend on its rotation, nor on |q|
    r2, _ = O.preprocess_fwd(*one_gaussian(p, math.log(0.02), tuple(3.7 * q)), cam, 3)
    r3, _ = O.preprocess_fwd(*one_gaussian(p, math.log(0.02)), cam, 3)
    np.testing.assert_allclose(r1[0, 2:5], r3[0, 2:5], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(r1[0, 2:5], r2[0, 2:5], rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------------------
# Projection pinned independently of the oracle's formulas: rotations from scipy (a library
# routine), the covariance from a closed form or a float64 central-difference Jacobian of the
# pinhole map, and the SH view direction from the camera centre of the inverted view matrix.
# A transposed rotation, one wrong sign in a Jacobian cross term or a reversed view direction
# fails these.
# ---------------------------------------------------------------------------------------
def wxyz_quat(rot) -> np.ndarray:
    """(w, x, y, z) quaternion of a scipy Rotation (scipy's own order is (x, y, z, w))."""
    x, y, z, w = rot.as_quat()
    return np.array([w, x, y, z])


def conic_of(cov) -> np.ndarray:
    """(A, B, C) of the inverse of the symmetric 2x2 [[a, b], [b, c]]: (c, -b, a) / det."""
    a, b, c = cov[0, 0], cov[0, 1], cov[1, 1]
    det = a * c - b * b
    return np.array([c / det, -b / det, a / det])


def viewmat_np(rot, t) -> np.ndarray:
    vm = np.eye(4)
    vm[:3, :3] = rot.as_matrix()
    vm[:3, 3] = t
    return vm


def pinhole_jacobian_fd(vm, p_world, fx, fy, cx, cy, h=1e-6):
    """float64 central differences of p -> (fx X/Z + cx, fy Y/Z + cy), (X, Y, Z) = R p + t."""
    def proj(p):
        X, Y, Z = vm[:3, :3] @ p + vm[:3, 3]
        return np.array([fx * X / Z + cx, fy * Y / Z + cy])

    J = np.zeros((2, 3))
    for k in range(3):
        e = np.zeros(3)
        e[k] = h
        J[:, k] = (proj(p_world + e) - proj(p_world - e)) / (2 * h)
    return J


def assert_conic_close(got, cov_expect, rtol=2e-5):
    want = conic_of(cov_expect)
    scale = np.abs(want).max()
    assert np.abs(np.asarray(got, np.float64) - want).max() <= rtol * scale, (got, want)


@pytest.mark.parametrize("theta", [0.4, -0.4, 1.1, -1.1])
def test_preprocess_anisotropic_on_axis_closed_form(theta):
    """A Gaussian on the optical axis with scales (s1, s2, s3), turned by theta about the axis:
    cov2d = (f/z)^2 R(theta) diag(s1^2, s2^2) R(theta)^T + 0.3 I, R(theta) the 2D rotation
    (image x right, y down, as the camera's x and y). The off-diagonal term
    (f/z)^2 (s1^2 - s2^2) sin(theta) cos(theta) changes sign with theta, so a transposed
    rotation fails."""
    from scipy.spatial.transform import Rotation

    f, z = 500.0, 4.0
    s = np.array([0.06, 0.02, 0.04])
    cam = scenes.Camera(torch.eye(4), f, f, 64.3, 47.8, 128, 96, 0.2, 100.0)
    q = wxyz_quat(Rotation.from_euler("z", theta))
    g = one_gaussian((0.0, 0.0, z), 0.0, tuple(q))
    g[1][0] = np.log(s).astype(np.float32)
    rec, touched = O.preprocess_fwd(*g, cam, 0)
    assert touched[0] > 0
    c, sn = math.cos(theta), math.sin(theta)
    s1, s2 = float(np.float32(s[0])) ** 2, float(np.float32(s[1])) ** 2
    k = (f / z) ** 2
    cov = np.array([[k * (s1 * c * c + s2 * sn * sn) + 0.3, k * (s1 - s2) * sn * c],
                    [k * (s1 - s2) * sn * c, k * (s1 * sn * sn + s2 * c * c) + 0.3]])
    assert abs(cov[0, 1]) > 0.5  # the cross term is far from zero: its sign is tested
    assert_conic_close(rec[0, 2:5], cov)
    assert r_sign(rec[0, 3]) == -r_sign(cov[0, 1])  # B = -b / det


def r_sign(v) -> int:
    return 1 if v > 0 else (-1 if v < 0 else 0)


@pytest.mark.parametrize("case", range(6))
def test_preprocess_covariance_against_finite_difference_jacobian(case):
    """General camera pose and Gaussian orientation, off the optical axis: cov2d - 0.3 I equals
    J Sigma J^T with J the float64 central-difference Jacobian of the pinhole map at the mean
    (through the world-to-camera transform) and Sigma = R diag(s^2) R^T, R from scipy. The last
    case sits outside the 1.3x frustum (to the right and above the image): the covariance is
    then the one at the clamped direction, i.e. J is the Jacobian at the point of the same
    depth on the clamp boundary."""
    from scipy.spatial.transform import Rotation

    rng = np.random.default_rng(100 + case)
    W, H, fx, fy, cx, cy = 160, 120, 150.0, 170.0, 83.0, 55.0
    rview = Rotation.from_rotvec(rng.normal(size=3) * 0.4)
    t = rng.normal(size=3) * 0.5
    vm = viewmat_np(rview, t)
    cam = scenes.Camera(torch.tensor(vm, dtype=torch.float32), fx, fy, cx, cy, W, H, 0.2, 100.0)
    vm32 = cam.viewmat.double().numpy()  # the float32 matrix the oracle sees
    z = 3.0 + case * 0.5
    if case < 5:
        u, v = rng.uniform(0.15, 0.85) * W, rng.uniform(0.15, 0.85) * H  # target pixel
        s = np.exp(rng.uniform(np.log(0.01), np.log(0.08), size=3))
    else:
        u, v = W + 0.5 * W * 1.3, -0.6 * H  # beyond both clamp limits; a wide Gaussian reaches the image
        s = np.array([1.2, 0.9, 1.0])
    p_cam = np.array([(u - cx) / fx * z, (v - cy) / fy * z, z])
    Rv, tv = vm32[:3, :3], vm32[:3, 3]
    p_world = np.linalg.solve(Rv, p_cam - tv).astype(np.float32).astype(np.float64)
    rq = Rotation.from_quat(rng.normal(size=4))
    q = wxyz_quat(rq) * rng.uniform(0.5, 2.0)  # any norm
    g = one_gaussian(tuple(p_world), 0.0, tuple(q))
    g[1][0] = np.log(s).astype(np.float32)
    rec, touched = O.preprocess_fwd(*g, cam, 0)
    assert touched[0] > 0, "the test Gaussian must be visible"
    Rg = rq.as_matrix()
    s32 = g[1][0].astype(np.float64)
    Sigma = Rg @ np.diag(np.exp(s32) ** 2) @ Rg.T
    if case < 5:
        J = pinhole_jacobian_fd(vm32, p_world, fx, fy, cx, cy)
    else:
        X, Y, Z = Rv @ p_world + tv
        txc = min(max(X / Z, -1.3 * cx / fx), 1.3 * (W - cx) / fx)
        tyc = min(max(Y / Z, -1.3 * cy / fy), 1.3 * (H - cy) / fy)
        assert txc != X / Z and tyc != Y / Z  # both clamps active
        p_clamp = np.linalg.solve(Rv, np.array([txc * Z, tyc * Z, Z]) - tv)
        J = pinhole_jacobian_fd(vm32, p_clamp, fx, fy, cx, cy)
    cov = J @ Sigma @ J.T + 0.3 * np.eye(2)
    assert abs(cov[0, 1]) > 1e-3 * np.sqrt(cov[0, 0] * cov[1, 1])  # a real cross term
    assert_conic_close(rec[0, 2:5], cov, rtol=5e-5)
    # the mean projects to the pixel it was placed at (unclamped), the depth is Z
    np.testing.assert_allclose(rec[0, 0:2], [u, v], rtol=1e-5, atol=2e-3)
    np.testing.assert_allclose(rec[0, 6], z, rtol=1e-6)


@pytest.mark.parametrize("band,axis", [(1, 1), (2, 2), (3, 0)], ids=["y", "z", "x"])
def test_sh_degree1_colour_follows_the_view_direction(band, axis):
    """Degree 1 with one band coefficient c only: colour = 0.5 + c b(d), with the 3DGS basis
    (-C1 y, C1 z, -C1 x) at d = (mean - camera centre) / |mean - camera centre|, the camera
    centre taken from the inverted view matrix. A reversed direction flips the sign of the
    band's contribution."""
    from scipy.spatial.transform import Rotation

    W, H, f = 128, 96, 120.0
    vm = viewmat_np(Rotation.from_rotvec([0.3, -0.5, 0.2]), [0.4, -0.3, 2.5])
    cam = scenes.Camera(torch.tensor(vm, dtype=torch.float32), f, f, 64.0, 48.0, W, H, 0.2, 100.0)
    vm32 = cam.viewmat.double().numpy()
    campos = np.linalg.inv(vm32)[:3, 3]
    p_cam = np.array([0.5, 0.7, 2.5])  # in view, off axis: every direction component well away from 0
    p_world = np.linalg.solve(vm32[:3, :3], p_cam - vm32[:3, 3]).astype(np.float32).astype(np.float64)
    g = list(one_gaussian(tuple(p_world), math.log(0.05), sh0=(0.0, 0.0, 0.0)))
    cvals = np.array([0.3, -0.4, 0.5])
    g[4][0, band] = cvals
    rec, touched = O.preprocess_fwd(*g, cam, 1)
    assert touched[0] > 0
    d = p_world - campos
    d /= np.linalg.norm(d)
    assert abs(d[axis]) > 0.1
    c1 = D.sh_norm_constant(1, 0)
    sign = -1.0 if band in (1, 3) else 1.0
    want = 0.5 + sign * c1 * d[axis] * cvals
    np.testing.assert_allclose(rec[0, 8:11], want, rtol=0, atol=2e-6)
    # the reversed direction would give a colour that differs by far more than the tolerance
    assert np.abs((0.5 - sign * c1 * d[axis] * cvals) - want).min() > 1e-2


def test_preprocess_culls_behind_and_far():
    cam = scenes.Camera(torch.eye(4), 400.0, 400.0, 50.0, 40.0, 100, 80, 0.2, 10.0)
    for z in (-1.0, 0.1, 12.0):
        _, touched = O.preprocess_fwd(*one_gaussian((0.0, 0.0, z), math.log(0.05)), cam, 0)
        assert touched[0] == 0


@pytest.mark.parametrize("aa", [False, True], ids=["plain", "proper_antialiasing"])
def test_preprocess_matches_float64_restatement(aa):
    sc = small(seed=3)
    cam = aa_camera(sc.cameras[0]) if aa else sc.cameras[0]
    rec, touched = O.preprocess_fwd(*np_params(sc), cam, 3)
    vis = touched > 0
    assert vis.sum() > 50
    P = [t.double() for t in sc.params()]
    pre = D.preprocess64(*P, cam, 3)
    np.testing.assert_allclose(rec[vis, 0:2], pre["mean2d"][vis].numpy(), rtol=1e-5, atol=1e-4)
    conic = pre["conic"][vis].numpy()
    scale = np.abs(conic).max(1, keepdims=True)
    assert np.abs(rec[vis, 2:5] - conic).max() / 1 <= 1e-4 * scale.max()
    np.testing.assert_allclose(rec[vis, 8:11], pre["color"][vis].numpy(), atol=2e-6)
    np.testing.assert_allclose(rec[vis, 5], pre["opacity"][vis].numpy(), rtol=2e-6)


# ---------------------------------------------------------------------------------------
# Binning
# ---------------------------------------------------------------------------------------
def band_touch_f64(r, tx, ty, tiles_x, margin):
    """Whether the alpha >= 1/255 ellipse of record r reaches a pixel centre column of tile
    (tx, ty) at some y of the tile's rows (both clipped to r's pixel bounds), in float64.
    Returns True / False, or None within `margin` px of the boundary."""
    mx, my, A, B, C, thr = (float(v) for v in (r[0], r[1], r[2], r[3], r[4], r[7]))
    x0, x1, y0, y1 = (int(v) for v in r[12:16].view(np.int32))
    cx0, cx1 = max(tx * 16, x0), min(tx * 16 + 15, x1)
    Y0, Y1 = max(ty * 16, y0) + 0.5, min(ty * 16 + 15, y1) + 0.5
    if cx0 > cx1 or Y0 > Y1:
        return False
    best = -np.inf
    for c in range(cx0, cx1 + 1):
        u = c + 0.5 - mx
        # max over y in [Y0, Y1] of thr - 0.5 (A u^2 + 2 B u v + C v^2), v = y - my
        v_star = np.clip(-B * u / C, Y0 - my, Y1 - my)
        val = thr - 0.5 * (A * u * u + 2 * B * u * v_star + C * v_star * v_star)
        best = max(best, val)
    if abs(best) < margin:
        return None
    return best >= 0


def test_binning_lists_complete_sorted_and_bucketed():
    sc = small(n=600, seed=5)
    cam = sc.cameras[0]
    rec, touched = O.preprocess_fwd(*np_params(sc), cam, 3)
    keys, pl, ranges, boff = O.bin_instances(rec, touched, cam)
    tiles_x, T = cam.tiles_x, cam.n_tiles
    assert int((ranges[:, 1] - ranges[:, 0]).sum()) == len(pl) == int(touched.sum())
    assert np.all(keys[1:] >= keys[:-1])
    assert np.array_equal(np.diff(boff), (ranges[:, 1] - ranges[:, 0] + 31) // 32)
    depth = rec[:, 6]
    undecided = 0
    for t in range(T):
        s, e = ranges[t]
        lst = pl[s:e].astype(np.int64)
        assert np.all(keys[s:e] >> np.uint64(32) == t)
        # front to back, ties in index order
        dl = depth[lst]
        assert np.all((dl[1:] > dl[:-1]) | ((dl[1:] == dl[:-1]) & (lst[1:] > lst[:-1])))
        members = set(lst.tolist())
        tx, ty = t % tiles_x, t // tiles_x
        for g in np.nonzero(touched)[0]:
            want = band_touch_f64(rec[g], tx, ty, tiles_x, 1e-3)
            if want is None:
                undecided += 1
                continue
            assert want == (g in members), f"tile {t}, Gaussian {g}: expected {want}"
    assert undecided < 20


def test_binning_counts_match_emitted_tiles():
    sc = small(n=300, seed=6, scale=(0.02, 0.3))
    cam = sc.cameras[0]
    rec, touched = O.preprocess_fwd(*np_params(sc), cam, 3)
    keys, pl, ranges, boff = O.bin_instances(rec, touched, cam)
    per_g = np.bincount(pl, minlength=sc.n)
    assert np.array_equal(per_g, touched.astype(np.int64))


# ---------------------------------------------------------------------------------------
# Blending
# ---------------------------------------------------------------------------------------
def brute_force_render(rec, touched, W, H, bg):
    """All visible Gaussians at every pixel, depth order (ties by index), float64, with the
    forward's rules (G = exp(min(power, 0)), alpha = o G >= 1/255, stop once T < 1e-4)."""
    vis = np.nonzero(touched)[0]
    order = vis[np.lexsort((vis, rec[vis, 6]))]
    ys, xs = np.mgrid[0:H, 0:W]
    px, py = xs.reshape(-1) + 0.5, ys.reshape(-1) + 0.5
    T = np.ones(px.shape)
    C = np.zeros((px.size, 3))
    done = np.zeros(px.shape, bool)
    for g in order:
        r = rec[g].astype(np.float64)
        b = rec[g, 12:16].view(np.int32)
        dx, dy = r[0] - px, r[1] - py
        power = np.minimum(-0.5 * (r[2] * dx * dx + 2 * r[3] * dx * dy + r[4] * dy * dy), 0.0)
        alpha = r[5] * np.exp(power)
        inb = (xs.reshape(-1) >= b[0]) & (xs.reshape(-1) <= b[1]) & (ys.reshape(-1) >= b[2]) & (ys.reshape(-1) <= b[3])
        ok = inb & (alpha >= 1 / 255) & ~done
        a = np.where(ok, alpha, 0.0)
        C += (a * T)[:, None] * r[8:11][None, :]
        T = T * (1 - a)
        done |= T < 1e-4
    img = C + T[:, None] * np.asarray(bg)[None, :]
    return img.T.reshape(3, H, W), T.reshape(H, W)


def test_tiled_forward_equals_brute_force_over_all_gaussians():
    sc = small(n=500, seed=7)
    cam = sc.cameras[0]
    ref = O.render(*np_params(sc), cam, 3, bg=BG)
    img, fT = brute_force_render(ref["rec"], ref["touched"], cam.width, cam.height, BG)
    diff = np.abs(ref["image"] - img).max(0)
    # decisions at the alpha / T thresholds may differ between float32 and float64 on a
    # handful of pixels; everywhere else the images agree to float32 rounding
    assert (diff > 1e-5).mean() < 2e-3
    assert np.median(diff) < 1e-6


def test_termination_rule_and_checkpoints():
    sc = small(n=800, seed=8, opacity=(0.6, 0.99), scale=(0.05, 0.3))
    cam = sc.cameras[0]
    ref = O.render(*np_params(sc), cam, 3, bg=BG)
    fT, nc = ref["final_T"], ref["n_contrib"]
    assert (fT < 1e-4).any(), "scene must reach early termination"
    # a terminated pixel stops right after the splat that took T below 1e-4
    assert np.all(fT[fT < 1e-4] > 0)
    # checkpoints: T is non-increasing over a pixel's buckets and starts at 1
    ck = ref["ckpt"]
    boff = ref["bucket_offsets"]
    for tile in range(len(boff) - 1):
        b0, b1 = int(boff[tile]), int(boff[tile + 1])
        if b1 > b0:
            assert np.all(ck[b0, :, 3] == 1.0)
            assert np.all(np.diff(ck[b0:b1, :, 3], axis=0) <= 0)


def test_blend_forward_matches_dense_float64():
    sc = small(n=400, seed=9)
    cam = sc.cameras[0]
    ref = O.render(*np_params(sc), cam, 3, bg=BG)
    mask = O.contrib_mask(ref["rec"], ref["point_list"], ref["ranges"], cam.width, cam.height, ref["n_contrib"])
    P = [t.double() for t in sc.params()]
    pre = D.preprocess64(*P, cam, 3)
    img, fT = D.blend64(pre["mean2d"], pre["conic"], pre["opacity"], pre["color"], ref["point_list"],
                        ref["ranges"], mask, cam.width, cam.height, BG)
    assert np.abs(img.numpy() - ref["image"]).max() <= 1e-5
    assert np.abs(fT.numpy() - ref["final_T"]).max() <= 1e-5


def test_pruning_scores_sum_to_the_image_coverage_and_match_dense_weights():
    """Per pixel the blending weights sum to 1 - T_final, so the scores of all splats sum to the
    image's total alpha; per splat they equal the float64 dense weights of the same blend."""
    sc = small(n=500, seed=21)
    cam = sc.cameras[0]
    ref = O.render(*np_params(sc), cam, 3, bg=BG)
    np.testing.assert_allclose(ref["scores"].sum(), (1.0 - ref["final_T"].astype(np.float64)).sum(), rtol=1e-5)
    assert np.all(ref["scores"][ref["touched"] == 0] == 0)
    mask = O.contrib_mask(ref["rec"], ref["point_list"], ref["ranges"], cam.width, cam.height, ref["n_contrib"])
    r = torch.tensor(ref["rec"], dtype=torch.float64)
    conic = r[:, 2:5]
    s64 = torch.zeros(sc.n, dtype=torch.float64)
    D.blend64(r[:, 0:2], conic, r[:, 5], r[:, 8:11], ref["point_list"], ref["ranges"], mask, cam.width,
              cam.height, BG, scores=s64)
    assert (ref["scores"] > 0).sum() > 100
    np.testing.assert_allclose(ref["scores"], s64.numpy(), rtol=2e-5, atol=1e-6)


def test_blend_backward_replay_matches_autograd():
    sc = small(n=400, seed=10)
    cam = sc.cameras[0]
    ref = O.render(*np_params(sc), cam, 3, bg=BG)
    mask = O.contrib_mask(ref["rec"], ref["point_list"], ref["ranges"], cam.width, cam.height, ref["n_contrib"])
    rec = ref["rec"].astype(np.float64)
    m2 = torch.tensor(rec[:, 0:2], requires_grad=True)
    con = torch.tensor(rec[:, 2:5], requires_grad=True)
    op = torch.tensor(rec[:, 5], requires_grad=True)
    col = torch.tensor(rec[:, 8:11], requires_grad=True)
    img, fT = D.blend64(m2, con, op, col, ref["point_list"], ref["ranges"], mask, cam.width, cam.height, BG)
    g = torch.Generator().manual_seed(1)
    gi = torch.randn(3, cam.height, cam.width, generator=g, dtype=torch.float64)
    ga = torch.randn(cam.height, cam.width, generator=g, dtype=torch.float64)
    ((img * gi).sum() + ((1 - fT) * ga).sum()).backward()
    g2 = O.blend_bwd(ref["rec"], ref["point_list"], ref["ranges"], ref["bucket_offsets"], cam.width, cam.height,
                     ref["image"], gi.float().numpy(), ref["final_T"], ref["n_contrib"], ref["tile_max"],
                     ref["ckpt"], sc.n, grad_alpha=ga.float().numpy())
    vis = ref["touched"] > 0
    # (the opacity column holds opacity times dL/dopacity)
    for cols, t in (((0, 1), m2.grad), ((2, 3, 4), con.grad), ((5,), (op.grad * op.detach())[:, None]),
                    ((6, 7, 8), col.grad)):
        a = g2[vis][:, list(cols)]
        b = t.numpy()[vis]
        assert D.rel_err(a, b) < 2e-5, (cols, D.rel_err(a, b))


@pytest.mark.parametrize("aa", [False, True], ids=["plain", "proper_antialiasing"])
def test_preprocess_backward_matches_autograd(aa):
    sc = small(n=300, seed=11)
    cam = aa_camera(sc.cameras[0]) if aa else sc.cameras[0]
    rec, touched = O.preprocess_fwd(*np_params(sc), cam, 3)
    vis = touched > 0
    rng = np.random.default_rng(2)
    g2 = rng.standard_normal((sc.n, 12)).astype(np.float32)
    g2[:, 9:] = 0
    gm, gls, gq, gop, gsh = O.preprocess_bwd(*np_params(sc), cam, 3, rec, touched, g2)
    P = [t.double().requires_grad_(True) for t in sc.params()]
    pre = D.preprocess64(*P, cam, 3)
    g2t = torch.tensor(g2, dtype=torch.float64) * torch.tensor(vis, dtype=torch.float64)[:, None]
    # clamped colour channels carry no gradient: preprocess64 clamps with torch.clamp as well
    # (g2's opacity column is opacity times dL/dopacity)
    o_det = pre["opacity"].detach()
    loss = ((pre["mean2d"] * g2t[:, 0:2]).sum() + (pre["conic"] * g2t[:, 2:5]).sum()
            + (pre["opacity"] * g2t[:, 5] / torch.where(o_det > 0, o_det, 1.0)).sum()
            + (pre["color"] * g2t[:, 6:9]).sum())
    loss.backward()
    for name, a, t in (("means", gm, P[0]), ("log_scales", gls, P[1]), ("quats", gq, P[2]),
                       ("opacity", gop, P[3]), ("sh", gsh, P[4])):
        e = D.rel_err(a[vis], t.grad.numpy()[vis])
        assert e < 1e-4, f"{name}: {e:.2e}"
        assert np.all(a[~vis] == 0)


def test_degree0_rest_gradients_are_zero():
    sc = small(n=200, seed=12)
    cam = sc.cameras[0]
    rec, touched = O.preprocess_fwd(*np_params(sc), cam, 0)
    g2 = np.ones((sc.n, 12), np.float32)
    gsh = O.preprocess_bwd(*np_params(sc), cam, 0, rec, touched, g2)[4]
    assert np.all(gsh[:, 1:, :] == 0)
    assert np.any(gsh[:, 0, :] != 0)


# ---------------------------------------------------------------------------------------
# Screen-space mean gradient of one splat against the continuous closed form
# ---------------------------------------------------------------------------------------
def single_splat_scene(sigma_px=10.0, logit=1.5, W=160, H=120, mx=81.3, my=58.7):
    """One isotropic Gaussian on the optical axis whose projected (dilated) std-dev is sigma_px,
    colour (1, 0, 0) (SH degree 0), at pixel position (mx, my)."""
    f, z = 500.0, 4.0
    s = math.sqrt(sigma_px ** 2 - 0.3) * z / f
    cam = scenes.Camera(torch.eye(4), f, f, mx, my, W, H, 0.2, 100.0)
    g = one_gaussian((0.0, 0.0, z), math.log(s), logit=logit, sh0=(0.5 / D.SH0, -0.5 / D.SH0, -0.5 / D.SH0))
    return cam, g


def test_mean2d_gradient_of_one_splat_matches_closed_form():
    """C_p = c alpha_p with alpha_p = o exp(-|p - mu|^2 / (2 sigma^2)) where o G >= 1/255 (radius R,
    U = R^2 / (2 sigma^2) = ln(255 o)). With the red upstream gradient a (px - mux) + b (py - muy),
    dL/dmu = (a, b) 2 pi c o sigma^2 (1 - (1 + U) / (255 o)); with the constant upstream gradient 1,
    sum_p |dL/dmux at p| = (c o / sigma^2) 4 sigma^3 (sqrt(pi/2) erf(R / (sigma sqrt 2)) - (R/sigma) e^-U).
    The pixel sums approximate the integrals to about 3e-4 at sigma = 10 px. The NDC norm of
    the densification statistic, |(W/2 g_x, H/2 g_y)|, follows with W != H."""
    sigma, logit = 10.0, 1.5
    cam, g = single_splat_scene(sigma, logit)
    o = 1.0 / (1.0 + math.exp(-logit))
    ref = O.render(*g, cam, 0)
    assert ref["touched"][0] > 0 and np.allclose(ref["rec"][0, 8:11], [1.0, 0.0, 0.0], atol=1e-6)
    mx, my = float(ref["rec"][0, 0]), float(ref["rec"][0, 1])
    U = math.log(255.0 * o)
    R_ = sigma * math.sqrt(2.0 * U)
    ys, xs = np.mgrid[0:cam.height, 0:cam.width]
    a, b = 0.7, -1.3
    gi = np.zeros((3, cam.height, cam.width), np.float32)
    gi[0] = a * (xs + 0.5 - mx) + b * (ys + 0.5 - my)

    def bwd(upstream):
        return O.blend_bwd(ref["rec"], ref["point_list"], ref["ranges"], ref["bucket_offsets"], cam.width,
                           cam.height, ref["image"], upstream, ref["final_T"], ref["n_contrib"], ref["tile_max"],
                           ref["ckpt"], 1)[0]

    g2 = bwd(gi)
    K = 2.0 * math.pi * o * sigma ** 2 * (1.0 - (1.0 + U) / (255.0 * o))
    np.testing.assert_allclose(g2[0:2], [a * K, b * K], rtol=2e-3)
    ndc = math.hypot(cam.width / 2 * g2[0], cam.height / 2 * g2[1])
    np.testing.assert_allclose(ndc, K * math.hypot(cam.width / 2 * a, cam.height / 2 * b), rtol=2e-3)
    assert abs(math.hypot(cam.height / 2 * a, cam.width / 2 * b) * K - ndc) > 0.05 * ndc  # W, H not swapped
    ones = np.zeros_like(gi)
    ones[0] = 1.0
    g1 = bwd(ones)
    absx = (o / sigma ** 2) * 4.0 * sigma ** 3 * (math.sqrt(math.pi / 2) * math.erf(R_ / (sigma * math.sqrt(2)))
                                                 - (R_ / sigma) * math.exp(-U))
    np.testing.assert_allclose(g1[9:11], [absx, absx], rtol=2e-3)
    assert abs(g1[0]) < 1e-3 * absx  # the signed sum cancels by symmetry
