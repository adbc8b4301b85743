"""CPU checks pinning the L1 + D-SSIM restatement (oracle/loss_ref.py): the closed forms of
SSIM, the zero-padded convolution against direct summation of the definition, and its gradient
against finite differences."""
import numpy as np
import torch

import loss_ref as L


def test_identical_images_have_ssim_one():
    x = torch.rand(3, 20, 24, dtype=torch.float64)
    assert torch.allclose(L.ssim_map(x, x), torch.ones_like(x), atol=1e-12)


def test_constant_images_interior_closed_form():
    a, b = 0.3, 0.7
    x = torch.full((1, 30, 30), a, dtype=torch.float64)
    y = torch.full((1, 30, 30), b, dtype=torch.float64)
    s = L.ssim_map(x, y)[0, 5:25, 5:25]  # window fully inside: mu = value, sigma = 0
    expect = (2 * a * b + L.C1) / (a * a + b * b + L.C1)
    assert torch.allclose(s, torch.full_like(s, expect), atol=1e-12)


def test_window_is_the_normalised_gaussian():
    g = L.gaussian_1d().numpy()
    assert abs(g.sum() - 1.0) < 1e-15 and np.argmax(g) == 5
    assert abs(g[4] / g[5] - np.exp(-1.0 / (2 * 1.5 ** 2))) < 1e-14


def test_convolution_equals_direct_summation():
    rng = np.random.default_rng(0)
    x, y = rng.random((2, 7, 9)), rng.random((2, 7, 9))
    conv = L.ssim_map(torch.from_numpy(x), torch.from_numpy(y)).numpy()
    assert np.abs(conv - L.ssim_brute(x, y)).max() < 1e-12


def test_gradient_matches_finite_differences():
    x = torch.rand(2, 9, 13, dtype=torch.float64, requires_grad=True)
    y = torch.rand(2, 9, 13, dtype=torch.float64)
    assert torch.autograd.gradcheck(lambda t: L.l1_ssim(t, y, 0.2), (x,), eps=1e-6, atol=1e-8)
